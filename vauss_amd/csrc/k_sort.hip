// k_sort.hip -- stable LSD radix sort of (key, u32 value) pairs, 8-bit digits
// (7 or 9 bits for the render's sorts, see sort_impl), u32 or u64 keys.
//
// Replaces crates/splat-train-sort (radix_argsort*, lib.rs:15-189;
// kernels.rs:35-341).  Two schedules share one block-level ranking step, in
// which each wavefront ranks its keys in input order with ballot-based digit
// matching (8 ballots per step, no atomics) and the block reorders its tile by
// digit in LDS so that equal digits leave in consecutive addresses:
//
//  * one-sweep (n >= ONESWEEP_MIN): one histogram kernel counts the digits of
//    every pass in a single read of the keys; each pass is then a single
//    kernel in which each block publishes its tile's per-digit counts and sums
//    its predecessors' counts by decoupled look-back (a block only waits on
//    lower-indexed blocks, which are dispatched first and publish before they
//    wait, so the chain drains; a bounded spin turns anything else into a
//    reported error, not a hang);
//  * three kernels per pass for small or device-counted inputs: upsweep
//    (per-tile digit histograms into a [256 x blocks] table), an exclusive
//    scan of that table (k_scan.hip), and the scatter.
//
// Ranking in (wave, step, lane) order with waves owning consecutive key
// ranges keeps every pass stable, so the sort is stable.
#include "vs_internal.h"

namespace vs {

#ifndef VS_SORT_ITEMS
#define VS_SORT_ITEMS 8
#endif
#ifndef VS_ONESWEEP_MIN
#define VS_ONESWEEP_MIN (1u << 12)   // below it the input is one block of the three-kernel schedule
#endif
constexpr int SORT_BLOCK = 256;
constexpr int SORT_ITEMS = VS_SORT_ITEMS;
constexpr uint32_t SORT_TILE = SORT_BLOCK * SORT_ITEMS;   // keys per block of the three-kernel schedule
constexpr int SORT_WAVES = SORT_BLOCK / 64;

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K k, uint32_t shift) { return (uint32_t)(k >> shift) & 0xFFu; }
// A digit of RB bits (RB = 8 or 9).
template <int RB, typename K>
__device__ __forceinline__ uint32_t digit_rb(K k, uint32_t shift) { return (uint32_t)(k >> shift) & ((1u << RB) - 1u); }

// Adds the digits of 64 consecutive keys (one per lane, the first `nvalid`
// valid) to a wavefront's LDS histogram: only the first lane of each run of
// equal digits adds, with the run's length, so runs (a splat's tiles along a
// row share the high digit of the tile id) cost one LDS atomic, not one per
// key on the same address.
__device__ __forceinline__ void hist_add_runs(uint32_t* hist, uint32_t d, uint32_t lane, uint32_t nvalid) {
    const uint64_t above_me = ~((2ull << lane) - 1ull);   // lanes above this one (none for lane 63)
    const uint32_t prev = __shfl_up(d, 1);
    const bool head = lane < nvalid && (lane == 0 || prev != d);
    const uint64_t nxt = __ballot(head) & above_me;
    const uint32_t end = nxt ? (uint32_t)__builtin_ctzll(nxt) : nvalid;
    if (head) atomicAdd(&hist[d], end - lane);
}

template <typename K>
__global__ void __launch_bounds__(SORT_BLOCK) sort_upsweep_kernel(const K* __restrict__ keys, uint32_t n_cap,
                                                                  const uint32_t* __restrict__ n_dev, uint32_t shift,
                                                                  uint32_t* __restrict__ table, uint32_t nblocks) {
    __shared__ uint32_t hist[SORT_WAVES][256];
    const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    // Wavefront w counts keys [base + w*64*ITEMS, ...), the same keys its
    // wavefront ranks in the scatter kernel.
    const uint32_t wbase = blockIdx.x * SORT_TILE + wave * (64 * SORT_ITEMS);
    K k[SORT_ITEMS];
#pragma unroll
    for (int i = 0; i < SORT_ITEMS; ++i) {
        const uint32_t idx = wbase + i * 64 + lane;
        k[i] = idx < n ? keys[idx] : (K)0;
    }
    for (uint32_t i = threadIdx.x; i < SORT_WAVES * 256; i += SORT_BLOCK) (&hist[0][0])[i] = 0;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < SORT_ITEMS; ++i) {
        const uint32_t b = wbase + i * 64;
        const uint32_t nvalid = b < n ? min(64u, n - b) : 0u;
        if (nvalid) hist_add_runs(hist[wave], digit_of(k[i], shift), lane, nvalid);
    }
    __syncthreads();
    const uint32_t d = threadIdx.x;
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < SORT_WAVES; ++w) c += hist[w][d];
    table[(size_t)d * nblocks + blockIdx.x] = c;
}

// Block-level ranking of one tile of up to BLOCK * ITEMS keys, in two
// phases so that a one-sweep pass can publish its digit counts (and look back)
// between them:
//  * count(): loads the tile, ranks every key among the equal digits of its
//    wavefront (ballot matching), and turns the per-wave digit histograms into
//    each wave's exclusive offset within its digit; returns, in thread
//    d < 2^RB, the tile's count of digit d;
//  * place(): from those counts, digit_start[d] (the first LDS slot of digit d)
//    and the digit-ordered (stable) tile in s_keys / s_vals.
template <typename K, int BLOCK, int ITEMS, int RB = 8>
struct TileRanker {
    static constexpr uint32_t R = 1u << RB;   // digits
    static_assert(BLOCK >= (int)R && BLOCK % 64 == 0, "one thread per digit");
    static constexpr int WAVES = BLOCK / 64;
    K key[ITEMS];
    uint32_t val[ITEMS], dig[ITEMS], rank[ITEMS];
    uint32_t run = 0;

    __device__ __forceinline__ uint32_t count(const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
                                              uint32_t base, uint32_t n, uint32_t shift, uint32_t (*wave_hist)[R]) {
        const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        // Issue every load of the tile before any ranking step, so a wavefront
        // waits for memory once rather than once per step.
        const uint32_t wbase = base + wave * (64 * ITEMS);
#pragma unroll
        for (int s = 0; s < ITEMS; ++s) {
            const uint32_t idx = wbase + s * 64 + lane;
            key[s] = idx < n ? keys_in[idx] : (K)0;
        }
#pragma unroll
        for (int s = 0; s < ITEMS; ++s) {
            const uint32_t idx = wbase + s * 64 + lane;
            val[s] = idx < n ? vals_in[idx] : 0u;
        }
        for (uint32_t i = threadIdx.x; i < WAVES * R; i += BLOCK) (&wave_hist[0][0])[i] = 0;
        __syncthreads();

        const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
#pragma unroll
        for (int s = 0; s < ITEMS; ++s) {
            const uint32_t idx = wbase + s * 64 + lane;
            const bool valid = idx < n;
            const uint32_t d = digit_rb<RB>(key[s], shift);
            dig[s] = valid ? d : R;
            uint64_t peers = __ballot(valid);
#pragma unroll
            for (int b = 0; b < RB; ++b) {
                const uint64_t bal = __ballot((d >> b) & 1u);
                peers &= ((d >> b) & 1u) ? bal : ~bal;
            }
            uint32_t r = 0;
            if (valid) {
                const uint32_t before = wave_hist[wave][d];
                r = before + (uint32_t)__popcll(peers & lt_mask);
                if ((peers & lt_mask) == 0) wave_hist[wave][d] = before + (uint32_t)__popcll(peers);
            }
            rank[s] = r;
            __builtin_amdgcn_wave_barrier();
        }
        __syncthreads();
        // per-digit totals; each wave's count becomes its exclusive offset within the digit
        run = 0;
        const uint32_t d = threadIdx.x;
        if (d < R) {
#pragma unroll
            for (int w = 0; w < WAVES; ++w) {
                const uint32_t c = wave_hist[w][d];
                wave_hist[w][d] = run;
                run += c;
            }
        }
        return run;
    }

    __device__ __forceinline__ void place(uint32_t (*wave_hist)[R], uint32_t* digit_start, uint32_t* s_tot,
                                          K* s_keys, uint32_t* s_vals) {
        const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        const uint32_t d = threadIdx.x;
        // exclusive scan of the digit counts over the R digits
        uint32_t incl = run;
        if (d < R) {
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(incl, o);
                if ((int)lane >= o) incl += t;
            }
            if (lane == 63) s_tot[wave] = incl;
        }
        __syncthreads();
        if (d < R) {
            uint32_t wo = 0;
            for (uint32_t w = 0; w < wave; ++w) wo += s_tot[w];
            digit_start[d] = wo + incl - run;
        }
        __syncthreads();
#pragma unroll
        for (int s = 0; s < ITEMS; ++s) {
            if (dig[s] < R) {
                const uint32_t pos = digit_start[dig[s]] + wave_hist[wave][dig[s]] + rank[s];
                s_keys[pos] = key[s];
                s_vals[pos] = val[s];
            }
        }
        __syncthreads();
    }
};

template <typename K>
__global__ void __launch_bounds__(SORT_BLOCK) sort_scatter_kernel(const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
                                                                  K* __restrict__ keys_out, uint32_t* __restrict__ vals_out,
                                                                  uint32_t n_cap, const uint32_t* __restrict__ n_dev, uint32_t shift,
                                                                  const uint32_t* __restrict__ offsets, uint32_t nblocks) {
    __shared__ uint32_t wave_hist[SORT_WAVES][256];
    __shared__ uint32_t digit_start[256];
    __shared__ uint32_t s_tot[SORT_WAVES];
    __shared__ K s_keys[SORT_TILE];
    __shared__ uint32_t s_vals[SORT_TILE];

    __shared__ uint32_t s_gstart[256];

    const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
    const uint32_t base = blockIdx.x * SORT_TILE;
    if (base >= n) return;   // uniform per block
    {
        TileRanker<K, SORT_BLOCK, SORT_ITEMS> rk;
        rk.count(keys_in, vals_in, base, n, shift, wave_hist);
        rk.place(wave_hist, digit_start, s_tot, s_keys, s_vals);
    }
    if (threadIdx.x < 256) s_gstart[threadIdx.x] = offsets[(size_t)threadIdx.x * nblocks + blockIdx.x];
    __syncthreads();
    const uint32_t count = min(SORT_TILE, n - base);
    for (uint32_t i = threadIdx.x; i < count; i += SORT_BLOCK) {
        const K k = s_keys[i];
        const uint32_t d = digit_of(k, shift);
        const uint32_t gpos = s_gstart[d] + (i - digit_start[d]);
        if (gpos < n) {   // always true for a consistent table; keeps a bad rank from writing out of bounds
            keys_out[gpos] = k;
            vals_out[gpos] = s_vals[i];
        }
    }
}

// ---- one-sweep schedule ---------------------------------------------------------
// Tile shapes: inputs of OS_SMALL_N keys or more use OS_BLOCK x OS_ITEMS
// (8192) keys per block, which halves the look-back chain, the bound of a
// pass over a long array; shorter inputs use OS_SMALL_BLOCK x OS_SMALL_ITEMS
// (4096), which spreads them over more blocks (a pass there costs about the
// latency of one block).  Measured on MI355X (u32 pairs, 4 passes over 30M
// random keys): 8192-key tiles 0.86 ms, 4096 1.16 ms; a look-back window of
// 8 predecessors per step beat 16 and 32.
#ifndef VS_OS_BLOCK
#define VS_OS_BLOCK 512
#endif
#ifndef VS_OS_ITEMS
#define VS_OS_ITEMS 16
#endif
#ifndef VS_OS_SMALL_BLOCK
#define VS_OS_SMALL_BLOCK 512
#endif
#ifndef VS_OS_SMALL_ITEMS
#define VS_OS_SMALL_ITEMS 8
#endif
#ifndef VS_OS_SMALL_N
#define VS_OS_SMALL_N (2u << 20)
#endif
#ifndef VS_LOOKBACK
#define VS_LOOKBACK 8
#endif
#ifndef VS_HIST_BLOCKS
#define VS_HIST_BLOCKS 1024
#endif
constexpr uint32_t ONESWEEP_MIN = VS_ONESWEEP_MIN;
constexpr int OS_BLOCK = VS_OS_BLOCK;
constexpr int OS_ITEMS = VS_OS_ITEMS;
constexpr uint32_t OS_TILE = OS_BLOCK * OS_ITEMS;
constexpr int OS_SMALL_BLOCK = VS_OS_SMALL_BLOCK;
constexpr int OS_SMALL_ITEMS = VS_OS_SMALL_ITEMS;
constexpr uint32_t OS_SMALL_TILE = OS_SMALL_BLOCK * OS_SMALL_ITEMS;
constexpr uint32_t OS_SMALL_N = VS_OS_SMALL_N;
constexpr uint32_t OS_MIN_TILE = OS_TILE < OS_SMALL_TILE ? OS_TILE : OS_SMALL_TILE;
constexpr uint32_t ONESWEEP_MAX_KEYS = 1u << 30;       // counts fit the 30-bit status payload
constexpr uint32_t OS_AGGREGATE = 1u << 30;            // status: this tile's own count
constexpr uint32_t OS_PREFIX = 2u << 30;               // status: count of this tile and all before it
constexpr uint32_t OS_VALUE = (1u << 30) - 1u;
constexpr int LOOKBACK = VS_LOOKBACK;                  // predecessor statuses read per look-back step
constexpr uint32_t HIST_BLOCKS = VS_HIST_BLOCKS;
constexpr int HIST_ITEMS = 16;       // keys per lane in flight per chunk (the kernel is latency-bound below that)

// Digit histograms of every pass in one read: ghist[x][p][d] (zeroed by the
// caller), one copy per XCD x = block index mod 8 (the XCD the block runs on),
// so the blocks' closing atomics spread over eight sets of addresses; a pass
// sums the eight copies of a digit.  Each wavefront takes chunks of
// HIST_ITEMS x 64 consecutive keys.  Digits of RB bits.
constexpr uint32_t HIST_COPIES = 8;
// NT threads per block, ITEMS keys per lane and chunk.  256-thread blocks
// keep one LDS histogram per wavefront; wider blocks share one (the same
// keys per block in a quarter of the chunks per wavefront: a shorter chain
// of dependent LDS adds, and the same closing global atomics).
constexpr int HIST_NT = 1024;
constexpr int HIST_NT_ITEMS = 4;
static_assert(HIST_NT * HIST_NT_ITEMS == 4096, "a block's first chunks cover the 4096 keys per block of its grid");
template <typename K, int RB = 8, int NT = SORT_BLOCK, int ITEMS = HIST_ITEMS>
__global__ void __launch_bounds__(NT) sort_histogram_kernel(const K* __restrict__ keys, uint32_t n_cap,
                                                            const uint32_t* __restrict__ n_dev, uint32_t first_bit,
                                                            uint32_t passes, uint32_t* __restrict__ ghist) {
    constexpr uint32_t R = 1u << RB;
    constexpr int HP = (8 * (int)sizeof(K) + RB - 1) / RB;   // passes a key can need
    constexpr int W = NT / 64;
    constexpr int COPIES = (NT == SORT_BLOCK) ? W : 1;
    __shared__ uint32_t h[COPIES][HP][R];
    const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < COPIES * HP * R; i += NT) (&h[0][0][0])[i] = 0;
    __syncthreads();
    const uint64_t stride = (uint64_t)gridDim.x * W * 64 * ITEMS;
    for (uint64_t c = ((uint64_t)blockIdx.x * W + wave) * 64 * ITEMS; c < n; c += stride) {
        K k[ITEMS];
#pragma unroll
        for (int s = 0; s < ITEMS; ++s) {
            const uint64_t idx = c + (uint64_t)s * 64 + lane;
            k[s] = idx < n ? keys[idx] : (K)0;
        }
#pragma unroll
        for (int s = 0; s < ITEMS; ++s) {
            const uint64_t b = c + (uint64_t)s * 64;
            if (b >= n) break;                                   // uniform across the wavefront
            const uint32_t nvalid = (uint32_t)min((uint64_t)64, (uint64_t)n - b);
            for (uint32_t p = 0; p < passes; ++p)
                hist_add_runs(h[COPIES == 1 ? 0 : wave][p], digit_rb<RB>(k[s], first_bit + RB * p), lane, nvalid);
        }
    }
    __syncthreads();
    uint32_t* mine = ghist + (size_t)(blockIdx.x % HIST_COPIES) * passes * R;
    for (uint32_t i = threadIdx.x; i < passes * R; i += NT) {
        uint32_t c = 0;
#pragma unroll
        for (int w = 0; w < COPIES; ++w) c += (&h[w][0][0])[i];
        if (c) atomicAdd(&mine[i], c);
    }
}

__device__ __forceinline__ uint32_t status_load(uint32_t* p) {
    return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ void status_store(uint32_t* p, uint32_t v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// One pass over digits of RB bits: rank a tile, find its digits' global
// offsets by look-back, scatter.  `status` is [nblocks][2^RB], zeroed before
// the pass.  key_span (null: unused) is the [min, max] of values whose
// differences the keys are: a pass whose digit lies above every key's
// highest set bit is the identity, and copies its tile.
template <typename K, int BLOCK, int ITEMS, int RB = 8>
__global__ void __launch_bounds__(BLOCK) sort_onesweep_kernel(const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
                                                                   K* __restrict__ keys_out, uint32_t* __restrict__ vals_out,
                                                                   uint32_t n_cap, const uint32_t* __restrict__ n_dev, uint32_t shift,
                                                                   const uint32_t* __restrict__ ghist, uint32_t ghist_copy_stride,
                                                                   uint32_t* status,
                                                                   uint32_t* err, uint32_t spin_limit,
                                                                   uint32_t* __restrict__ ranges, uint32_t num_tiles,
                                                                   const uint32_t* __restrict__ key_span) {
    constexpr uint32_t TILE = BLOCK * ITEMS;
    constexpr uint32_t R = 1u << RB;
    __shared__ uint32_t wave_hist[BLOCK / 64][R];
    __shared__ uint32_t digit_start[R];
    __shared__ uint32_t s_tot[BLOCK / 64];
    __shared__ uint32_t s_gstart[R];        // where this tile's digit d starts in the output
    __shared__ K s_keys[TILE];
    __shared__ uint32_t s_vals[TILE];

    // Tile = block index.  Workgroups are dispatched in index order on each
    // XCD, so every block this one waits on (lower indices) is already
    // running or finished and never waits on a higher one: the chain drains.
    // (A global ticket counter would serialise ~2k same-address atomics per
    // pass across the XCDs.)
    const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
    const uint32_t tile = blockIdx.x;
    const uint32_t base = tile * TILE;
    // A tile past the end has no successor with keys.
    if (base >= n) return;
    if (key_span) {
        // every key is below 2^bits: a digit above that is 0 for all (uniform)
        const uint32_t span = key_span[1] - key_span[0];
        const uint32_t bits = span ? 32u - (uint32_t)__builtin_clz(span) : 0u;
        if (shift >= bits) {
            const uint32_t count = min(TILE, n - base);
            for (uint32_t i = threadIdx.x; i < count; i += BLOCK) {
                keys_out[base + i] = keys_in[base + i];
                vals_out[base + i] = vals_in[base + i];
            }
            return;
        }
    }
    const uint32_t d = threadIdx.x;
    // The pass's global digit counts (the sum of the eight histogram copies)
    // are loaded first, so their latency overlaps the tile's.
    uint32_t gh[HIST_COPIES];
#pragma unroll
    for (uint32_t x = 0; x < HIST_COPIES; ++x) gh[x] = d < R ? ghist[(size_t)x * ghist_copy_stride + d] : 0u;
    TileRanker<K, BLOCK, ITEMS, RB> rk;
    const uint32_t cnt = rk.count(keys_in, vals_in, base, n, shift, wave_hist);

    // The tile's digit counts are published as soon as they are known, and
    // the look-back runs before the tile is reordered in LDS, so the tile's
    // prefix reaches its successors as early as it can.
    uint32_t excl = 0;
    if (d < R) {
        uint32_t* my = status + (size_t)tile * R + d;
        status_store(my, (tile == 0 ? OS_PREFIX : OS_AGGREGATE) | cnt);
        if (tile > 0) {
            // Look back over predecessors LOOKBACK at a time (independent loads),
            // newest first, summing aggregates until a prefix; a not-yet-published
            // tile is polled again.
            int j = (int)tile - 1;
            uint32_t spins = 0;
            while (true) {
                uint32_t st[LOOKBACK];
    #pragma unroll
                for (int i = 0; i < LOOKBACK; ++i)
                    st[i] = (j - i >= 0) ? status_load(status + (size_t)(j - i) * R + d) : OS_PREFIX;
                int used = 0;
                bool found = false, stalled = false;
    #pragma unroll
                for (int i = 0; i < LOOKBACK; ++i) {
                    if (found || stalled) continue;
                    const uint32_t flag = st[i] & ~OS_VALUE;
                    if (flag == 0u) { stalled = true; continue; }
                    excl += st[i] & OS_VALUE;
                    ++used;
                    found = flag == OS_PREFIX;
                }
                if (found) break;
                j -= used;
                if (stalled) {
                    if (++spins > spin_limit) { atomicOr(err, 1u); break; }
                    __builtin_amdgcn_s_sleep(1);
                }
            }
            status_store(my, OS_PREFIX | (excl + cnt));
        }
    }
    rk.place(wave_hist, digit_start, s_tot, s_keys, s_vals);
    // global exclusive start of digit d: sum of ghist[0..d) (block scan over R)
    {
        const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        uint32_t c = 0u;
#pragma unroll
        for (uint32_t x = 0; x < HIST_COPIES; ++x) c += gh[x];
        uint32_t incl = c;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o);
            if ((int)lane >= o) incl += t;
        }
        if (lane == 63 && d < R) s_tot[wave] = incl;   // place() has finished with s_tot
        __syncthreads();
        if (d < R) {
            uint32_t wo = 0;
            for (uint32_t w = 0; w < wave; ++w) wo += s_tot[w];
            s_gstart[d] = excl + wo + incl - c;
        }
    }
    __syncthreads();
    const uint32_t count = min(TILE, n - base);
    for (uint32_t i = threadIdx.x; i < count; i += BLOCK) {
        const K k = s_keys[i];
        const uint32_t dd = digit_rb<RB>(k, shift);
        const uint32_t gpos = s_gstart[dd] + (i - digit_start[dd]);
        if (gpos < n) {   // always true for consistent counts; keeps a bad count from writing out of bounds
            if (!ranges) keys_out[gpos] = k;
            vals_out[gpos] = s_vals[i];
            if (ranges && (uint64_t)k < num_tiles) {
                // The last pass: within a digit's run of this tile the keys are
                // sorted (earlier passes sorted the lower bits), so a key change
                // inside the run is a range bound; a run's first and last keys
                // may continue in another tile's run and meet there by min / max.
                const uint32_t t = (uint32_t)k;
                const uint32_t run_lo = digit_start[dd], run_hi = dd < R - 1 ? digit_start[dd + 1] : count;
                if (i == run_lo || s_keys[i - 1] != k) atomicMin(&ranges[2 * t], gpos);
                if (i + 1 == run_hi || s_keys[i + 1] != k) atomicMax(&ranges[2 * t + 1], gpos + 1);
            }
        }
    }
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t sort_tmp_bytes(uint64_t n, bool key64, uint32_t radix_bits) {
    const uint64_t nblocks = (n + SORT_TILE - 1) / SORT_TILE;
    const size_t ks = key64 ? 8 : 4;
    const uint32_t rb = (radix_bits == 7 || radix_bits == 9) ? radix_bits : 8u;
    const uint64_t max_passes = (8 * ks + rb - 1) / rb, R = 1ull << rb;
    size_t b = 0;
    b += align_up(n * ks, 256);                 // ping-pong keys
    b += align_up(n * 4, 256);                  // ping-pong values
    b += align_up(nblocks * 256 * 4, 256);      // digit table
    b += align_up(scan_tmp_words(nblocks * 256) * 4, 256);
    // one-sweep: histograms and per-pass tile status
    const uint64_t os_tiles = (n + OS_MIN_TILE - 1) / OS_MIN_TILE;
    b += align_up((size_t)(HIST_COPIES * max_passes * R * 4 + 64 + max_passes * os_tiles * R * 4), 256);
    return b + 256;
}

template <typename K, int RB>
static void launch_onesweep_pass(bool small, uint32_t os_tiles, const K* src_k, const uint32_t* src_v, K* dk,
                                 uint32_t* dv, uint32_t n, const uint32_t* n_dev, uint32_t shift, const uint32_t* gh,
                                 uint32_t gh_stride, uint32_t* status, uint32_t* err, uint32_t spin_limit,
                                 uint32_t* rng, uint32_t nt, const uint32_t* key_span, hipStream_t s) {
    if (small)
        sort_onesweep_kernel<K, OS_SMALL_BLOCK, OS_SMALL_ITEMS, RB><<<os_tiles, OS_SMALL_BLOCK, 0, s>>>(
            src_k, src_v, dk, dv, n, n_dev, shift, gh, gh_stride, status, err, spin_limit, rng, nt, key_span);
    else
        sort_onesweep_kernel<K, OS_BLOCK, OS_ITEMS, RB><<<os_tiles, OS_BLOCK, 0, s>>>(
            src_k, src_v, dk, dv, n, n_dev, shift, gh, gh_stride, status, err, spin_limit, rng, nt, key_span);
}

// Digits of 8 bits, or of 7 or 9 (radix_bits, u32 keys, one-sweep schedule
// only): 9-bit digits cover a view's depth span (27 bits) in three passes,
// 7-bit ones a tile id of up to 14 bits in two, with a quarter of the
// look-back and one ballot fewer per key than 8-bit ones.
template <typename K>
static hipError_t sort_impl(const K* keys_in, const uint32_t* vals_in, K* keys_out, uint32_t* vals_out, uint32_t n,
                            const uint32_t* n_dev, uint32_t first_bit, uint32_t end_bit, void* tmp, uint32_t* err,
                            hipStream_t s, uint32_t spin_limit, TileRangesOut* tr, bool state_zeroed,
                            uint32_t radix_bits, const uint32_t* key_span) {
    if (n == 0) return hipSuccess;
    const uint32_t bits = end_bit > first_bit ? end_bit - first_bit : 0;
    if (bits == 0) {
        hipError_t e = hipMemcpyAsync(keys_out, keys_in, (size_t)n * sizeof(K), hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return e;
        return hipMemcpyAsync(vals_out, vals_in, (size_t)n * 4, hipMemcpyDeviceToDevice, s);
    }
    const bool onesweep = n >= ONESWEEP_MIN && n < ONESWEEP_MAX_KEYS && err != nullptr;
    const uint32_t rb = (onesweep && sizeof(K) == 4 && (radix_bits == 7 || radix_bits == 9)) ? radix_bits : 8u;
    const uint32_t R = 1u << rb;
    const uint32_t passes = (bits + rb - 1) / rb;
    const uint32_t nblocks = (n + SORT_TILE - 1) / SORT_TILE;
    char* p = reinterpret_cast<char*>(align_up(reinterpret_cast<uintptr_t>(tmp), 256));
    K* tk = reinterpret_cast<K*>(p); p += align_up((size_t)n * sizeof(K), 256);
    uint32_t* tv = reinterpret_cast<uint32_t*>(p); p += align_up((size_t)n * 4, 256);
    uint32_t* table = reinterpret_cast<uint32_t*>(p); p += align_up((size_t)nblocks * 256 * 4, 256);
    uint32_t* stmp = reinterpret_cast<uint32_t*>(p); p += align_up(scan_tmp_words((uint64_t)nblocks * 256) * 4, 256);
    const bool small = n < OS_SMALL_N;
    const uint32_t os_tile = small ? OS_SMALL_TILE : OS_TILE;
    const uint32_t os_tiles = (n + os_tile - 1) / os_tile;
    uint32_t* ghist = reinterpret_cast<uint32_t*>(p);          // [HIST_COPIES][passes][R]
    uint32_t* status = ghist + HIST_COPIES * passes * R + 16; // [passes][os_tiles][R]
    if (onesweep) {
        hipError_t e = hipSuccess;
        if (!state_zeroed)
            e = launch_fill_u32(ghist, 0u, (uint64_t)HIST_COPIES * passes * R + 16 + (uint64_t)passes * os_tiles * R, s);
        if (e != hipSuccess) return e;
        // ~4k keys per block up to HIST_BLOCKS blocks: each block ends with
        // passes x R global atomics, so a grid much wider than the data
        // only adds atomics (16k keys per block starves short inputs).
        const uint32_t hist_blocks = (uint32_t)max((uint64_t)1, min((uint64_t)HIST_BLOCKS, ((uint64_t)n + 4095) / 4096));
        if constexpr (sizeof(K) == 4) {
            if (rb == 9)
                sort_histogram_kernel<K, 9, HIST_NT, HIST_NT_ITEMS><<<hist_blocks, HIST_NT, 0, s>>>(keys_in, n, n_dev, first_bit, passes, ghist);
            else if (rb == 7)
                sort_histogram_kernel<K, 7, HIST_NT, HIST_NT_ITEMS><<<hist_blocks, HIST_NT, 0, s>>>(keys_in, n, n_dev, first_bit, passes, ghist);
            else
                sort_histogram_kernel<K, 8, HIST_NT, HIST_NT_ITEMS><<<hist_blocks, HIST_NT, 0, s>>>(keys_in, n, n_dev, first_bit, passes, ghist);
        } else {
            sort_histogram_kernel<K, 8><<<hist_blocks, SORT_BLOCK, 0, s>>>(keys_in, n, n_dev, first_bit, passes, ghist);
        }
        e = hipGetLastError();
        if (e != hipSuccess) return e;
    }
    const K* src_k = keys_in;
    const uint32_t* src_v = vals_in;
    for (uint32_t pass = 0; pass < passes; ++pass) {
        const bool to_out = ((passes - 1 - pass) % 2) == 0;
        K* dk = to_out ? keys_out : tk;
        uint32_t* dv = to_out ? vals_out : tv;
        const uint32_t shift = first_bit + rb * pass;
        // the last pass of a tile sort derives the tile ranges instead of writing the keys
        uint32_t* rng = (tr && pass + 1 == passes) ? tr->ranges : nullptr;
        const uint32_t nt = tr ? tr->num_tiles : 0u;
        hipError_t e;
        if (onesweep) {
            const uint32_t* gh = ghist + pass * R;
            uint32_t* st = status + (size_t)pass * os_tiles * R;
            if constexpr (sizeof(K) == 4) {
                if (rb == 7)
                    launch_onesweep_pass<K, 7>(small, os_tiles, src_k, src_v, dk, dv, n, n_dev, shift, gh, passes * R, st,
                                               err, spin_limit, rng, nt, key_span, s);
                else if (rb == 9)
                    launch_onesweep_pass<K, 9>(small, os_tiles, src_k, src_v, dk, dv, n, n_dev, shift, gh, passes * R, st,
                                               err, spin_limit, rng, nt, key_span, s);
                else
                    launch_onesweep_pass<K, 8>(small, os_tiles, src_k, src_v, dk, dv, n, n_dev, shift, gh, passes * R, st,
                                               err, spin_limit, rng, nt, key_span, s);
            } else {
                launch_onesweep_pass<K, 8>(small, os_tiles, src_k, src_v, dk, dv, n, n_dev, shift, gh, passes * R, st, err,
                                           spin_limit, rng, nt, nullptr, s);
            }
            if (rng) tr->done = true;
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        } else {
            sort_upsweep_kernel<K><<<nblocks, SORT_BLOCK, 0, s>>>(src_k, n, n_dev, shift, table, nblocks);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
            e = scan_u32(table, table, (uint64_t)nblocks * 256, false, stmp, nullptr, s);
            if (e != hipSuccess) return e;
            sort_scatter_kernel<K><<<nblocks, SORT_BLOCK, 0, s>>>(src_k, src_v, dk, dv, n, n_dev, shift, table, nblocks);
            e = hipGetLastError();
            if (e != hipSuccess) return e;
        }
        src_k = dk;
        src_v = dv;
    }
    return hipSuccess;
}

hipError_t radix_sort_pairs(const void* keys_in, const uint32_t* vals_in, void* keys_out, uint32_t* vals_out,
                            uint32_t n, const uint32_t* n_dev, bool key64, uint32_t first_bit, uint32_t end_bit,
                            void* tmp, uint32_t* err, hipStream_t s, uint32_t spin_limit, TileRangesOut* tr,
                            bool state_zeroed, uint32_t radix_bits, const uint32_t* key_span) {
    if (tr) tr->done = false;
    if (tr && key_span) return hipErrorInvalidValue;   // a range pass never skips
    if (key64)
        return sort_impl<uint64_t>(static_cast<const uint64_t*>(keys_in), vals_in, static_cast<uint64_t*>(keys_out),
                                   vals_out, n, n_dev, first_bit, end_bit, tmp, err, s, spin_limit, nullptr, false, 8u,
                                   nullptr);
    return sort_impl<uint32_t>(static_cast<const uint32_t*>(keys_in), vals_in, static_cast<uint32_t*>(keys_out),
                               vals_out, n, n_dev, first_bit, end_bit, tmp, err, s, spin_limit, tr, state_zeroed,
                               radix_bits, key_span);
}

SortZeroSpan sort_zero_span(uint32_t n, uint32_t first_bit, uint32_t end_bit, void* tmp, uint32_t radix_bits) {
    // the layout of sort_impl<uint32_t>: ping-pong keys, values, digit table, scan scratch, then the
    // one-sweep histograms and status
    const uint32_t bits = end_bit > first_bit ? end_bit - first_bit : 0;
    if (n == 0 || bits == 0 || !(n >= ONESWEEP_MIN && n < ONESWEEP_MAX_KEYS)) return SortZeroSpan{nullptr, 0};
    const uint32_t rb = (radix_bits == 7 || radix_bits == 9) ? radix_bits : 8u;
    const uint64_t R = 1ull << rb;
    const uint32_t passes = (bits + rb - 1) / rb;
    const uint32_t nblocks = (n + SORT_TILE - 1) / SORT_TILE;
    char* p = reinterpret_cast<char*>(align_up(reinterpret_cast<uintptr_t>(tmp), 256));
    p += align_up((size_t)n * 4, 256);
    p += align_up((size_t)n * 4, 256);
    p += align_up((size_t)nblocks * 256 * 4, 256);
    p += align_up(scan_tmp_words((uint64_t)nblocks * 256) * 4, 256);
    const uint32_t os_tile = n < OS_SMALL_N ? OS_SMALL_TILE : OS_TILE;
    const uint64_t os_tiles = (n + os_tile - 1) / os_tile;
    return SortZeroSpan{reinterpret_cast<uint32_t*>(p), (uint64_t)HIST_COPIES * passes * R + 16 + (uint64_t)passes * os_tiles * R};
}

} // namespace vs
