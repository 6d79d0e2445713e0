// vs_internal.h -- launch parameters and launcher declarations shared between
// the kernel translation units and the C-ABI layer (api.hip).
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>
#include "../../include/vsplat.h"

namespace vs {

constexpr uint32_t TILE_W_HOST_ = 16;   // tile edge in pixels (kernels/helpers.rs:15)

// Device counters written by the projection stage and read back once.
enum : uint32_t {
    CNT_VISIBLE = 0,      // splats surviving every cull
    CNT_DEPTH_MIN = 1,    // min / max raw f32 bits of visible depths
    CNT_DEPTH_MAX = 2,
    CNT_EMITTERS = 3,     // splats that hit at least one tile
    CNT_ISECT64 = 4,      // words 4..5: total intersections as a u64
    CNT_BOUNDED = 6,      // min(total intersections, the arena's capacity): the pairs emitted
    CNT_KEPT = 7,         // depth cutoff: splats keeping at least one pair (the emitters)
    CNT_COUNT = 8,
};

// Rows of the projection's per-block statistics, [BS_ROWS][ceil(N/256)].
enum : uint32_t {
    BS_HITS = 0,          // tiles hit
    BS_VISIBLE = 1,       // splats surviving the culls
    BS_DMIN = 2,          // min / max raw depth bits of the visible splats
    BS_DMAX = 3,
    BS_EMIT = 4,          // splats with at least one hit; exclusive offsets after finalize
    BS_ROWS = 5,
};

// Per-context device flags (read back with the projection counters).
enum : uint32_t {
    FLAG_SORT_STALL = 0,  // a one-sweep look-back gave up waiting
    CTX_FLAGS = 4,
};

// A projected splat's row: four float4, one aligned 64-byte segment, so the
// emission and raster gathers touch one segment per splat (three planes of
// 16 + 16 + 4 bytes touched three):
//   q0 = x, y, c00, c01    q1 = c11, opacity, r, g    q2 = b, power, 0, 0    q3 unused
// power = logf(255 opacity), the exponent bound of the tile footprint.
constexpr uint32_t PROJ_Q = 4;

struct ProjectArgs {
    vs_camera cam;
    uint32_t img_w, img_h, tile_bw, tile_bh;
    uint32_t num_splats, sh_degree;
    float log_scale_offset;
    const float* transforms;
    const void* sh;                  // [N,K,3] f32, or f16 bits when sh_half
    uint32_t sh_half;
    const float* min_scale;          // [N] scale floor (apply_scale_floor) or null
    uint32_t mip;                    // SplatRenderMode::Mip
    const float* decoder;            // [816] neural appearance (rows of 12, sh_degree = direction band) or null
    const float* raw_opac;
    // outputs, indexed by global splat id
    float* opacities;           // [N]
    float* max_radius;          // [N]
    uint32_t* counts;           // [N] tiles hit
    uint32_t* depth_bits;       // [N] raw f32 bits of view z
    float4* proj;               // [N][PROJ_Q] projected rows (layout above)
    float4* proj_aux;           // [N] z, nx, ny, nz (geometry) or null
    float4* proj_surf;          // [N][4] surfels: M rows, low-pass centre, normal (vs_surfel.h layout), or null
    uint32_t* compact;          // [N] g + 1 for splats past every cull, else 0 (compact_from_global)
    uint32_t* block_stats;      // [BS_ROWS][ceil(N/256)]
    float* visible;             // [N] cleared to 0 (the forward marks the splats it blends), or null
    uint32_t* ranges;           // [num_tiles, 2] set to (0xFFFFFFFF, 0) for the tile sort's range pass
    uint32_t num_tiles;
};

struct CompactArgs {
    uint32_t num_splats;
    const uint32_t* counts;          // [N]
    const uint32_t* depth_bits;      // [N]
    const uint32_t* block_offsets;   // row BS_EMIT of the block stats after finalize
    const uint32_t* counters;        // device counters (CNT_DEPTH_MIN)
    uint32_t* keys;                  // [M] depth bits - min
    uint32_t* vals;                  // [M] global ids
    uint32_t* zero;                  // [zero_words] cleared (the depth sort's one-sweep state), or null
    uint64_t zero_words;
    uint32_t* zero2;                 // [zero2_words] cleared (the slot scan's look-back status), or null
    uint64_t zero2_words;
};

// Emission splits the emitters by slot count: up to EMIT_SMALL_LIST slots
// in depth order, more in global-id order (their slot bases scattered by id).
constexpr uint32_t EMIT_SMALL_LIST = 64;

struct EmitArgs {
    uint32_t num_splats, tile_bw, tile_bh;
    uint32_t num_emitters;           // M: length of `order` (a capacity when m_dev is set)
    const uint32_t* m_dev;           // device count of emitters (lagged renders), or null
    const uint32_t* order;           // [M] global ids of the emitters, nearest first
    const uint32_t* counts;          // [N]
    const uint32_t* slot_base;       // [M + 1] first slot of the j-th nearest emitter (exclusive scan), then the total
    const uint32_t* slot_base_g;     // [N] the same, at the global id (emitters of more than EMIT_SMALL_LIST slots only)
    const float4* proj;              // [N][PROJ_Q] projected rows
    uint32_t* tiles;                 // [capacity] tile id (T = sentinel)
    uint32_t* vals;                  // [capacity] global id
    uint32_t capacity;               // slots at or past it are dropped (the farthest splats' pairs)
    uint32_t* zero;                  // [zero_words] cleared (the tile sort's one-sweep state), or null
    uint64_t zero_words;
    // depth cutoff (null cut: every tile keeps every splat)
    const uint8_t* cut;              // [T] last depth bin each tile keeps
    const uint16_t* allow;           // [bh][CUT_BINS][bw + 1] tiles before x in row ty keeping bin b
    const uint32_t* depth_bits;      // [N] raw depth bits (the splat's bin)
    const uint32_t* counters;        // the projection's counters (depth range)
    uint32_t* counts_out;            // count pass: [N] tiles kept per splat
    const uint32_t* sat;             // count pass: [bh][CUT_BINS][bw + 1] allow summed over rows 0..ty
    uint32_t* kept_blocks;           // count pass: [ceil(N / PROJ_BLOCK)] splats per block keeping a pair
    uint32_t* listed;                // emission: the list's length (slots the scan handed out), or null
};

// Depth cutoff: a lower bound on the opacity that splats of each depth bin
// lay over the whole of a tile gives the bin by which every pixel of the tile
// has reached the raster's stopping transmittance; later bins never reach
// the tile's pixels and are not listed for it.
constexpr uint32_t CUT_BINS = 64;         // depth bins, equal spans of the raw depth bits
constexpr float CUT_SCALE = 4096.0f;      // fixed-point units per nat of -ln(1 - alpha)
constexpr uint32_t CUT_FRONT = 16;        // front bins, whose masses every splat adds
constexpr uint32_t CUT_MAX_BW = 4096;     // tile columns the row kernel holds in LDS
constexpr uint32_t CUT_AUTO_PER_TILE = 2048;   // VS_CUTOFF_AUTO: listed pairs per tile that turn it on
struct CutArgs {
    uint32_t num_splats, tile_bw, tile_bh;
    const uint32_t* counts;          // [N] tiles per splat (0: not listed anywhere)
    const uint32_t* depth_bits;      // [N]
    const uint32_t* counters;        // depth range
    const float4* proj;              // [N][PROJ_Q] projected rows
    uint32_t* mass;                  // [bh][CUT_BINS][bw + 1] fixed-point mass differences along each row
    uint8_t* cut;                    // [T]
    uint16_t* allow;                 // [bh][CUT_BINS][bw + 1]
    uint32_t* sat;                   // [bh][CUT_BINS][bw + 1] allow summed over rows 0..ty (may alias mass)
    uint32_t* pend;                  // [bh][bw + 1] per row, the tiles left of x whose front bins' masses
                                     // stay below the stopping mass
    uint32_t* pend_total;            // the tiles still short of it after the front bins (all rows)
};

struct RasterArgs {
    uint32_t img_w, img_h, tile_bw, tile_bh, num_tiles;
    uint32_t num_splats;             // ids at or past it (only a corrupt list holds them) are skipped
    const uint32_t* order;           // [8 ceil(T/8)] tile of each workgroup (launch_tile_order), or null
    float bg_r, bg_g, bg_b;
    const uint32_t* gids;            // sorted intersections -> global splat id
    const uint32_t* ranges;          // [T,2]
    uint32_t* ranges_shrunk;         // [T,2] written by bwd-info passes (may alias nothing else)
    uint32_t* aux_ranges;            // [T,2] the caller's copy of the shrunk ranges (bwd-info passes), or null
    const float4* proj;              // [N][PROJ_Q] projected rows
    const float4* proj_aux;
    const float4* proj_surf;         // [N][4] surfels (vs_surfel.h layout) or null
    uint32_t surf_crit;              // surfels outside training: median by the surface criterion
    void* out;                       // f32 [H,W,C] or u32 [H,W]
    float* visible;                  // [N] or null
    uint8_t* qpass;                  // [I][4] bwd-info passes: byte q = 1 << q when a pixel of quadrant q
                                     // passed (blended or stopped) at that list entry, or null
    // The L1 term's cotangent of the RGBA image written with it (null l1_v: none):
    // target [H,W] packed RGBA8, circle mask (l1_mr <= 0: none), 1 / (3 masked pixels)
    const uint32_t* l1_gt;
    float* l1_v;                     // [H,W,4]
    float l1_mcx, l1_mcy, l1_mr, l1_inv;
};

struct RasterBwdArgs {
    uint32_t img_w, img_h, tile_bw, tile_bh, num_tiles;
    uint32_t num_splats;             // ids at or past it are skipped
    const uint32_t* order;           // [8 ceil(T/8)] tile of each workgroup, or null
    float bg_r, bg_g, bg_b;
    const uint32_t* gids;
    const uint32_t* ranges;          // shrunk ranges
    const float4* proj;              // [N][PROJ_Q] projected rows
    const float4* proj_surf;         // [N][4] surfels, or null
    const float* out_img;            // [H,W,C]
    const float* v_out;              // [H,W,C]
    uint32_t channels;
    float* v_combined;               // [N,10], surfels [N,17]
    const uint32_t* qpass;           // [I] the forward's quadrant pass bytes (RasterArgs::qpass), or null
};

struct ProjectBwdArgs {
    vs_camera cam;
    uint32_t num_splats, sh_degree;
    float log_scale_offset;
    const float* transforms;
    const void* sh;                  // [N,K,3] f32, or f16 bits when sh_half
    uint32_t sh_half;
    const float* min_scale;          // [N] scale floor (apply_scale_floor) or null
    uint32_t mip;                    // SplatRenderMode::Mip
    const float* decoder;            // neural appearance: no SH term here (the neural backward adds it)
    uint32_t surfel;                 // surfels: v_combined rows of 17 (surfel_backwards)
    const float* raw_opac;
    const uint32_t* counts;          // visible <=> counts defined; culled rows get zeros
    const float* v_combined;         // [N,10]
    float* v_transforms;
    float* v_sh;
    float* v_raw_opac;
    float* v_refine;
};

struct NeuralBwdArgs {
    vs_camera cam;
    uint32_t num_splats, degree;     // degree: the decoder's direction band
    const float* transforms;
    const void* rows;                // [N,12] f32, or f16 bits when half
    uint32_t half;
    const float* decoder;            // [816]
    const float* v_combined;         // [N,10]
    float* v_transforms;             // [N,10] mean += view-direction term, or null
    float* v_rows;                   // [N,12] or null
    float* v_rows_sq;                // [N] or null
    float* partials;                 // [gridDim, 816]
    float* v_decoder;                // [816] or null
};

struct PoseBwdArgs {
    vs_camera cam;
    uint32_t num_splats, sh_degree;
    float log_scale_offset;
    const float* transforms;
    const void* sh;                  // [N,K,3] f32, or f16 bits when sh_half
    uint32_t sh_half;
    const float* min_scale;          // [N] scale floor or null
    uint32_t mip;
    const float* raw_opac;
    const float* v_combined;         // [N,10]
    float* partials;                 // [ceil(N/256), 12] block sums
    float* v_pose;                   // [12]
};

struct ProjectUpdateArgs {
    vs_camera cam;
    uint32_t num_splats, sh_degree;
    float log_scale_offset;
    float* transforms;               // [N,10] stepped in place
    const void* sh;                  // [N,K,3] f32, or f16 bits when sh_half
    uint32_t sh_half;
    const float* min_scale;          // [N] scale floor (apply_scale_floor) or null
    uint32_t mip;                    // SplatRenderMode::Mip
    float* raw_opac;                 // [N] stepped in place
    const uint32_t* compact;         // [N] g + 1 if visible, else 0
    const float* v_combined;         // [N,10]
    uint32_t* w_t;                   // [N,10] packed moments
    const float* lr_scale;           // [10] device
    uint32_t* w_o;                   // [N] packed moments
    float beta1, beta2, inv1, inv2, epsilon, lr_opac, opac_reg;
    uint32_t round_seed;
    float* color_dir;                // [N+1,6] or null
    float* v_refine;                 // [N] or null
    float* grad_sq;                  // [N] or null
};

struct LossArgs {
    uint32_t img_w, img_h, channels;     // channels 3 or 4
    const float* pred;                   // [H,W,C]
    const uint32_t* gt;                  // [H,W] RGBA8 packed
    float l1_weight, ssim_weight, alpha_weight_cfg;
    int32_t composite, mask;
    float bg[3];
    float rgb_weight, alpha_weight;      // 1 / (3 H W), alpha_weight_cfg / (H W)
    float* partials;                     // [planes, tiles] or null
    float* coeffs;                       // [3][3][H,W] or null
    float* loss_map;                     // [H,W,C] or null
    float* total;                        // [1] or null (needs partials)
};

struct LossBwdArgs {
    LossArgs fwd;                        // configuration
    uint32_t img_w, img_h, channels;
    const float* pred;
    const uint32_t* gt;
    const float* dl;                     // [1] or [planes, tiles]
    const float* coeffs;                 // [3][3][H,W] from the forward
    float* dl_dpred;                     // [H,W,C]
    float rgb_weight, alpha_weight;
};

struct ShStepArgs {
    uint32_t num_splats, sh_degree;
    uint32_t num_values, num_blocks;     // N*K*3 and ceil(num_values / 128)
    uint16_t* sh;                        // [N,K,3] f16 bits, stepped in place
    const float* color_dir;              // [rows,6] colour gradient + view direction, row 0 zero
    const uint32_t* grad_rows;           // [N] row of color_dir per splat, 0 = culled
    const float* grad_sq;                // [N]
    float* variance;                     // [N] second moment, updated in place
    uint32_t* codes;                     // [num_blocks*32] biased 8-bit first-moment codes
    float* scales;                       // [num_blocks]
    const float* lr_scale;               // [K*3]
    float beta1, beta2, inv1, inv2, epsilon, lr;
    uint32_t round_seed, first;
};

// ---- launchers (return hipError_t of the launch) -------------------------------
hipError_t launch_project(const ProjectArgs& a, hipStream_t s);
// Reduces the projection's block stats into `counters` (and a copy at
// `host_copy`, a pinned readback slot, if given) and turns the block emitter
// counts (row BS_EMIT) into exclusive offsets in place.
hipError_t launch_finalize_counts(uint32_t* block_stats, uint32_t nblocks, uint32_t* counters, uint32_t isect_capacity,
                                  hipStream_t s, uint32_t* host_copy = nullptr);
hipError_t launch_compact(const CompactArgs& a, hipStream_t s);
hipError_t launch_emit(const EmitArgs& a, hipStream_t s);
// Depth cutoff: the opacity mass of every splat's core (mass zeroed by the
// caller), each tile's cutoff bin and the rows' kept-tile prefix counts, their
// sums over rows (sat, which may reuse the masses' memory), then each splat's
// kept tiles (EmitArgs: counts = the projection's, counts_out, sat).
// back: the splats of bins >= CUT_FRONT whose box holds a pending tile
// (a.pend from launch_cut_pending); otherwise the splats of the front bins
hipError_t launch_cut_mass(const CutArgs& a, bool back, hipStream_t s);
hipError_t launch_cut_pending(const CutArgs& a, hipStream_t s);
// Exclusive scan of v[0, n) in place (one workgroup); *total = the sum.
hipError_t launch_scan_blocks(uint32_t* v, uint32_t n, uint32_t* total, hipStream_t s);
hipError_t launch_cut_rows(const CutArgs& a, hipStream_t s);
hipError_t launch_cut_sat(const CutArgs& a, hipStream_t s);
hipError_t launch_count_kept(const EmitArgs& a, hipStream_t s);
hipError_t launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, hipStream_t s);
hipError_t launch_fill_f32(float* p, float value, uint64_t n, hipStream_t s);

// Validation scan (the reference's validate_tensor_val, validation.rs:60-140):
// over the elements of an [n / row, row] array whose column lies in
// [col0, col1), count NaN, Inf, finite values below `lo` and above `hi`, and
// keep the first NaN and first Inf element index.  `stats` holds
// VALIDATE_WORDS u32: counts, then the two indices (start at 0xFFFFFFFF).
enum { VAL_NAN = 0, VAL_INF = 1, VAL_BELOW = 2, VAL_ABOVE = 3, VAL_FIRST_NAN = 4, VAL_FIRST_INF = 5, VALIDATE_WORDS = 8 };
hipError_t launch_validate(const void* p, bool half, uint64_t n, uint32_t row, uint32_t col0, uint32_t col1, float lo,
                           float hi, uint32_t* stats, hipStream_t s);
// Ranges of the first min(*n_dev, n) sorted tile ids (all n when n_dev is null).
hipError_t launch_tile_ranges(const uint32_t* tiles, uint32_t n, uint32_t num_tiles, uint32_t* ranges, hipStream_t s,
                              const uint32_t* n_dev = nullptr);
// Dispatch order of the raster kernels from tile ranges [T,2]: XCD bands,
// longest list first within each (order holds 8 ceil(T/8) entries).  With
// `shrunk_init`, every tile's entry there is set to (start, start): the
// forward's shrunk ranges, whose ends it raises.
// `fix_empty`: ranges left at (0xFFFFFFFF, 0) by the sort become (0, 0).
// `flags_to` (optional): copies nflags words of flags_from there (the
// lagged render's pinned readback slot).
// `aux_out` (optional): the caller's tile offsets, set like `shrunk_init`
// when that is given (the forward raises their ends too), else to the
// (fixed) ranges.
hipError_t launch_tile_order(uint32_t* ranges, uint32_t num_tiles, uint32_t* order, hipStream_t s,
                             uint32_t* shrunk_init = nullptr, bool fix_empty = false,
                             const uint32_t* flags_from = nullptr, uint32_t* flags_to = nullptr, uint32_t nflags = 0,
                             uint32_t* aux_out = nullptr, float* zero = nullptr, uint64_t zero_floats = 0);
hipError_t launch_ranges_init(uint32_t* ranges, uint32_t num_tiles, hipStream_t s);
hipError_t launch_tiles_from_ranges(const uint32_t* ranges, uint32_t num_tiles, uint32_t n, uint32_t* tiles,
                                    hipStream_t s);
hipError_t launch_raster_fwd(const RasterArgs& a, bool bwd_info, bool geometry, bool smooth, hipStream_t s);
// With `start` and `stop` set, the kernel is launched by hipExtLaunchKernelGGL,
// which records the two events around the kernel's own execution.
hipError_t launch_raster_bwd(const RasterBwdArgs& a, bool smooth, hipStream_t s, hipEvent_t start = nullptr,
                             hipEvent_t stop = nullptr);
hipError_t launch_project_bwd(const ProjectBwdArgs& a, hipStream_t s);
hipError_t launch_project_update(const ProjectUpdateArgs& a, hipStream_t s);
// Camera gradient: per-splat rows summed per 256-splat block, then the blocks (in order).
hipError_t launch_pose_bwd(const PoseBwdArgs& a, hipStream_t s);
// Neural appearance backward: rows, mean term, per-block decoder partials, then their sum.
hipError_t launch_neural_bwd(const NeuralBwdArgs& a, hipStream_t s);
uint32_t neural_bwd_blocks(uint32_t num_splats);
uint32_t pose_bwd_blocks(uint32_t num_splats);
hipError_t launch_geo_encode(const float* m, const float* v, uint32_t n, float epsilon, uint32_t* words, hipStream_t s);
hipError_t launch_geo_decode(const uint32_t* words, uint32_t n, float epsilon, float* m, float* v, hipStream_t s);
hipError_t launch_geo_zero_rows(uint32_t* words, const uint32_t* rows, uint32_t num_rows, uint32_t row_width,
                                uint64_t num_words, hipStream_t s);
// Streaming kernels of known traffic for memory-counter calibration
// (k_calib.hip): mode bit 0 = write (else read), bit 1 = 4-byte words (else
// 16-byte); `sink` holds calib_sink_words() u32 for the read kernels.
hipError_t launch_stream_probe(void* buf, uint64_t bytes, int mode, uint32_t* sink, hipStream_t s);
uint32_t calib_sink_words();
hipError_t launch_exp2_range(uint32_t first_bits, uint64_t count, float* out, hipStream_t s);
// div_cr's quotients for given divisor bit patterns, and its mismatches with
// the division over all 2^32 divisors (mismatches zeroed by the caller).
hipError_t launch_division_values(float a, const uint32_t* bits, uint64_t count, float* out, hipStream_t s);
hipError_t launch_division_check(float a, unsigned long long* mismatches, hipStream_t s);
hipError_t launch_l1_cotangent(const float* pred, uint32_t channels, const void* gt, bool packed, uint32_t w, uint32_t h,
                               float mcx, float mcy, float mr, float inv_count, float* v_out, hipStream_t s);
hipError_t launch_loss_forward(const LossArgs& a, hipStream_t s);
hipError_t launch_loss_backward(const LossBwdArgs& a, bool scalar, hipStream_t s);
hipError_t launch_sh_step(const ShStepArgs& a, hipStream_t s);
hipError_t launch_b8_encode(const float* values, uint32_t n, uint32_t* codes, float* scales, hipStream_t s);
hipError_t launch_b8_decode(const uint32_t* codes, const float* scales, uint32_t n, float* values, hipStream_t s);
hipError_t launch_b8_zero_rows(uint32_t* codes, uint32_t n, const uint32_t* rows, uint32_t num_rows,
                               uint32_t row_width, hipStream_t s);
hipError_t launch_count_mask(uint32_t w, uint32_t h, float mcx, float mcy, float mr, uint32_t* out, hipStream_t s);

// Scans.  `tmp` needs scan_tmp_words(n) u32 words.  With a permutation `perm`
// (n distinct indices below `perm_bound`, the length of `in`) the scan runs
// along it: element i of the sequence is in[perm[i]] and its result goes to
// out[perm[i]], or to out[i] when `out_in_order` is set, in which case
// `out_scattered` (if given) also receives it at [perm[i]]; an index at or
// past perm_bound reads 0 (and is not scattered).
size_t scan_tmp_words(uint64_t n);
// `n_dev` (device, may be null): only the first min(*n_dev, n) elements are
// scanned, read and written.
hipError_t scan_u32(const uint32_t* in, uint32_t* out, uint64_t n, bool inclusive, uint32_t* tmp,
                    uint32_t* total_out, hipStream_t s, const uint32_t* perm = nullptr,
                    const uint32_t* n_dev = nullptr, uint32_t perm_bound = 0xFFFFFFFFu, bool out_in_order = false,
                    uint32_t* out_scattered = nullptr);
hipError_t scan_single_block(uint32_t* data, uint32_t n, bool inclusive, uint32_t* total_out, hipStream_t s);
// The same exclusive scan in one kernel by decoupled look-back, written in
// sequence order (out[i]; with both `perm` and `out_scattered`, also
// out_scattered[perm[i]] for the elements whose input exceeds
// `scatter_above`).  `status` needs scan_lookback_status_words(n) words, zero
// on entry; a look-back that waits past `spin_limit` polls sets *err.  With
// `write_end`, out[n] (out holds n + 1 words) receives the total.
uint64_t scan_lookback_status_words(uint64_t n);
hipError_t scan_u32_lookback(const uint32_t* in, uint32_t* out, uint64_t n, uint32_t* status, uint32_t* err,
                             hipStream_t s, uint32_t spin_limit, const uint32_t* perm = nullptr,
                             const uint32_t* n_dev = nullptr, uint32_t perm_bound = 0xFFFFFFFFu,
                             uint32_t* out_scattered = nullptr, bool write_end = false, uint32_t scatter_above = 0u);

// Radix sort.  `tmp` needs sort_tmp_bytes(n, key64, radix_bits) bytes.
size_t sort_tmp_bytes(uint64_t n, bool key64, uint32_t radix_bits = 8);
// `err` (device word, may be null: then the one-sweep schedule is not used)
// is or-ed with 1 if a one-sweep look-back gave up waiting: after
// `spin_limit` polls of a predecessor that has not published its counts.
constexpr uint32_t SORT_SPIN_LIMIT_DEFAULT = 1u << 18;
// A u32 sort of tile ids may produce the tiles' [start, end) ranges itself:
// `ranges` [num_tiles, 2] must hold (0xFFFFFFFF, 0) beforehand (tiles left so
// are empty; launch_tile_order turns them into (0, 0)).  When the sort does
// so (its last pass is a one-sweep pass) it sets `done` and does not write
// the sorted keys; otherwise the caller finds the ranges (launch_tile_ranges).
struct TileRangesOut {
    uint32_t* ranges;
    uint32_t num_tiles;
    bool done;
};
hipError_t radix_sort_pairs(const void* keys_in, const uint32_t* vals_in, void* keys_out, uint32_t* vals_out,
                            uint32_t n, const uint32_t* n_dev, bool key64, uint32_t first_bit, uint32_t end_bit,
                            void* tmp, uint32_t* err, hipStream_t s,
                            uint32_t spin_limit = SORT_SPIN_LIMIT_DEFAULT, TileRangesOut* tr = nullptr,
                            bool state_zeroed = false, uint32_t radix_bits = 8,
                            const uint32_t* key_span = nullptr);
// radix_bits = 7 or 9: digits of that width (u32 keys of the one-sweep
// schedule; 8 elsewhere).  key_span (device [min, max], or null): the keys are values
// minus min, so no key has a bit at or above bitlen(max - min), and a pass
// whose digit lies there copies its input (not with a range pass).
// The words of `tmp` that a u32-key sort of n keys over [first_bit, end_bit)
// needs cleared before it runs (its one-sweep histograms and tile status):
// a caller that clears them in a kernel of its own passes state_zeroed and
// the sort skips its fill.  {nullptr, 0} when the sort would not use them.
struct SortZeroSpan { uint32_t* ptr; uint64_t words; };
SortZeroSpan sort_zero_span(uint32_t n, uint32_t first_bit, uint32_t end_bit, void* tmp, uint32_t radix_bits = 8);

} // namespace vs
