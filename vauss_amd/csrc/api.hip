// api.hip -- the C ABI of include/vsplat.h: argument checks, buffer planning,
// the stage sequence of a render, and the sort / scan / loss entry points.
#include <hip/hip_runtime.h>
#include <algorithm>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <new>
#include <string>
#include <vector>
#include "vs_internal.h"
#include "vs_capacity.h"

using namespace vs;

namespace {

thread_local std::string g_last_error;

vs_status fail(vs_status st, const std::string& msg) {
    g_last_error = msg;
    return st;
}
vs_status hip_fail(hipError_t e, const char* what) {
    return fail(e == hipErrorOutOfMemory ? VS_ERR_OOM : VS_ERR_HIP,
                std::string(what) + ": " + hipGetErrorString(e));
}

#define VS_HIP(call, what)                                  \
    do {                                                    \
        hipError_t e_ = (call);                             \
        if (e_ != hipSuccess) return hip_fail(e_, what);    \
    } while (0)

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

uint32_t bit_length(uint64_t v) {
    uint32_t b = 0;
    while (v) { ++b; v >>= 1; }
    return b;
}

enum Stage { ST_PROJECT, ST_EMIT, ST_SORT, ST_RANGES, ST_RASTER_FWD, ST_RASTER_BWD, ST_PROJECT_BWD, ST_OTHER, ST_N };

} // namespace

struct vs_ctx {
    int device = 0;
    hipStream_t stream = nullptr;
    uint32_t* host_counters = nullptr;    // pinned readback of the projection counters (+ CTX_FLAGS words)
    uint32_t* dev_flags = nullptr;        // device: [0] set when a sort or scan look-back gave up waiting
    uint32_t timing = 0;                  // bitmask of timed stages (VS_TIME_*)
    uint32_t spin_limit = SORT_SPIN_LIMIT_DEFAULT;   // look-back polls before a one-sweep pass gives up
    // the unmasked pixel count of the last circular L1 mask (vs_l1_cotangent)
    struct MaskKey { uint32_t w, h; float cx, cy, r; } l1_mask{0, 0, 0.0f, 0.0f, 0.0f};
    uint64_t l1_mask_count = 0;
    vs_cutoff_mode depth_cutoff = VS_CUTOFF_OFF;    // vs_ctx_set_depth_cutoff (opt-in)
    bool validate = false;                // scan inputs and gradients for NaN / Inf (vs_ctx_set_validation)
    bool poison = false;                  // fill every library allocation with POISON_WORD first
    uint32_t* dev_val = nullptr;          // device: validation counters, VALIDATE_WORDS per check
    uint32_t* host_val = nullptr;         // pinned mirror of dev_val
    // Stage event pairs recorded since the last vs_ctx_stage_times(); the
    // pool is reused, so timing many renders needs no extra synchronisation.
    struct Rec { int stage; hipEvent_t b, e; };
    std::vector<Rec> recs;
    std::vector<hipEvent_t> pool;
    // Lagged training renders (render.rs:57-304): capacity hints per
    // (image size, count slot) and the not-yet-read counts of the last lagged
    // render at each key, copied to pinned memory behind an event.
    bool lagged = false;
    CapacityTable caps;
    struct Pending { uint32_t* host = nullptr; hipEvent_t ev = nullptr; size_t capacity = 0; uint32_t splats = 0;
                     size_t limit = 0; bool live = false; };
    std::map<CapacityKey, Pending> pending;
    uint64_t lagged_renders = 0, lagged_overflows = 0;
    uint64_t surfel_lens_dropped = 0;   // surfel renders whose camera had lens distortion (rendered as pinhole)
    hipEvent_t take() {
        if (!pool.empty()) { hipEvent_t e = pool.back(); pool.pop_back(); return e; }
        hipEvent_t e = nullptr;
        hipEventCreate(&e);
        return e;
    }
    // Stage-timing events: recorded without the system-scope fence (a cache
    // write-back and invalidate that stalls the stream for several
    // microseconds); they are only read by vs_ctx_stage_times after a stream
    // synchronisation.
    std::vector<hipEvent_t> tpool;
    hipEvent_t take_timing() {
        if (!tpool.empty()) { hipEvent_t e = tpool.back(); tpool.pop_back(); return e; }
        hipEvent_t e = nullptr;
        hipEventCreateWithFlags(&e, hipEventDisableSystemFence);
        return e;
    }
    // Library allocations freed by the last renders, reused in stream order:
    // every library buffer lives on `stream`, so a block freed behind earlier
    // work is free for any later work on it, and a render that takes one
    // leaves no allocator packet in the stream.
    struct Block { void* p; size_t bytes; };
    std::vector<Block> cache;
    std::map<void*, size_t> live;      // size of each library allocation in use
    size_t cached_bytes = 0;
};

struct vs_fwd_state {
    vs_ctx* ctx = nullptr;
    vs_camera cam{};
    uint32_t W = 0, H = 0, N = 0, degree = 0, K = 0, sh_half = 0, mip = 0, neural = 0, surfel = 0;
    const float* min_scale = nullptr;   // the forward's scale floor (borrowed), or null
    float lso = 0.0f;
    float bg[3] = {0, 0, 0};
    vs_pass pass = VS_PASS_FORWARD;
    uint32_t tbw = 0, tbh = 0, T = 0, V = 0, I = 0, M = 0;
    void* arena = nullptr;        // per-splat buffers
    void* isect_arena = nullptr;  // per-intersection buffers
    uint32_t* counts = nullptr;
    uint32_t* depth_bits = nullptr;
    uint32_t* compact = nullptr;  // [N] g + 1 past every cull, else 0
    float4* proj = nullptr;          // [N][PROJ_Q] projected rows
    float4* proj_aux = nullptr;
    float4* proj_surf = nullptr;  // [N][4] surfels: M rows, low-pass centre, normal
    float* opacities = nullptr;
    float* max_radius = nullptr;
    float* visible = nullptr;
    uint32_t* block_stats = nullptr;
    uint32_t* counters = nullptr;
    uint32_t* ranges = nullptr;
    uint32_t* ranges_shrunk = nullptr;
    uint32_t* tile_order = nullptr;   // [8 ceil(T/8)] raster dispatch order
    float* v_combined = nullptr;
    uint32_t* tiles = nullptr;    // [I] sorted tile ids (written on demand, see tiles_pending)
    uint32_t* gids = nullptr;     // [I] sorted global ids
    uint32_t* qpass = nullptr;    // [I] bwd-info passes: the forward's quadrant pass bytes (the emission's
                                  // tile-id buffer, free once the tile sort has read it)
    // the tile sort produced the ranges and skipped the sorted ids: the state
    // view rebuilds them from the ranges
    mutable bool tiles_pending = false;
    // depth cutoff: the lists' length (device) and each splat's listed pairs
    bool cutoff = false;
    uint32_t* listed = nullptr;
    uint32_t* kept_counts = nullptr;
};

namespace {

struct StageTimer {
    vs_ctx* c;
    Stage s;
    hipEvent_t b = nullptr;
    StageTimer(vs_ctx* ctx, Stage st) : c(ctx), s(st) {
        if (c->timing & (1u << s)) { b = c->take_timing(); hipEventRecord(b, c->stream); }
    }
    ~StageTimer() {
        if (b) {
            hipEvent_t e = c->take_timing();
            hipEventRecord(e, c->stream);
            c->recs.push_back(vs_ctx::Rec{(int)s, b, e});
        }
    }
};

// RasterPass predicates, gaussian_splats.rs:60-107 (on the pass kind, the
// value's low byte).
bool pass_bwd_info(vs_pass p) { return p != VS_PASS_FORWARD; }
bool pass_training(vs_pass p) {
    return p == VS_PASS_BACKWARD || p == VS_PASS_BACKWARD_DENSE || p == VS_PASS_EXPOSURE ||
           p == VS_PASS_BACKWARD_FUSED_UPDATE;
}
bool pass_has_slot(vs_pass p) { return p == VS_PASS_BACKWARD_DENSE || p == VS_PASS_EXPOSURE; }
bool pass_geometry(vs_pass p) { return p == VS_PASS_GEOMETRY || p == VS_PASS_GEOMETRY_TRAIN_DEPTH; }
// Surfel depth by the surface criterion: every inference pass but GEOMETRY_TRAIN_DEPTH.
bool pass_surface_criterion(vs_pass p) { return !pass_training(p) && p != VS_PASS_GEOMETRY_TRAIN_DEPTH; }

const char* const SORT_STALL_MSG =
    "a one-sweep look-back (radix sort or slot scan) gave up waiting for a predecessor's counts; its output is wrong";

// The sort-stall flag as copied to ctx->host_counters[CNT_COUNT + ...] behind
// the last readback: report it (and clear the device word) if set.
vs_status take_sort_flag(vs_ctx* c) {
    if (c->host_counters[CNT_COUNT + FLAG_SORT_STALL] == 0u) return VS_OK;
    c->host_counters[CNT_COUNT + FLAG_SORT_STALL] = 0u;
    VS_HIP(launch_fill_u32(c->dev_flags, 0u, CTX_FLAGS, c->stream), "flag reset");
    return fail(VS_ERR_HIP, SORT_STALL_MSG);
}

// Copy the device flags behind everything enqueued so far and wait for them:
// a sort that gave up is reported by the call that ran it.
vs_status sync_sort_flag(vs_ctx* c) {
    VS_HIP(hipMemcpyAsync(c->host_counters + CNT_COUNT, c->dev_flags, CTX_FLAGS * 4, hipMemcpyDeviceToHost, c->stream),
           "flag readback");
    VS_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    return take_sort_flag(c);
}

// The f32 bit pattern of -12345.0, the value the reference's test builds add to
// every fresh tensor (crates/splat-train-cube/src/host.rs:23-36): a kernel that
// reads a slot it never wrote then sees a value far from any real one.
constexpr uint32_t POISON_WORD = 0xC640E400u;
// The depth sort's digits: 9 bits, so three passes cover the 25-27 bits a
// view's depth keys (depth bits - minimum) span.
constexpr uint32_t DEPTH_RADIX_BITS = 9;
static_assert(CNT_DEPTH_MAX == CNT_DEPTH_MIN + 1, "the depth sort reads [min, max] as a pair");
// The tile sort's digits: the narrowest of 7, 8 and 9 bits that sorts `bits`
// in as few passes as 9-bit digits would (7 for the 13-14 bits of tile ids
// up to 2560 x 1440 images: two passes of 128-digit look-back).
static uint32_t tile_radix_bits(uint32_t bits) {
    const uint32_t passes = (bits + 8) / 9;
    for (uint32_t rb = 7; rb < 9; ++rb)
        if ((bits + rb - 1) / rb <= passes) return rb;
    return 9;
}

// Every buffer the library allocates for itself: stream-ordered, and filled
// with POISON_WORD first when the context asks for it.
constexpr size_t CACHE_MAX_BLOCKS = 8;
constexpr size_t CACHE_MAX_BYTES = size_t(4) << 30;

// A library buffer of at least `bytes` on the context's stream: the smallest
// cached block that fits (and is at most twice the request), else a new
// stream-ordered allocation.
hipError_t lib_alloc(vs_ctx* c, void** p, size_t bytes, hipStream_t s) {
    bytes = std::max<size_t>(align256(bytes), 256);
    size_t best = c->cache.size();
    for (size_t i = 0; i < c->cache.size(); ++i) {
        const size_t b = c->cache[i].bytes;
        if (b >= bytes && b <= 2 * bytes && (best == c->cache.size() || b < c->cache[best].bytes)) best = i;
    }
    hipError_t e = hipSuccess;
    if (best < c->cache.size()) {
        *p = c->cache[best].p;
        c->cached_bytes -= c->cache[best].bytes;
        bytes = c->cache[best].bytes;
        c->cache.erase(c->cache.begin() + (ptrdiff_t)best);
    } else {
        e = hipMallocAsync(p, bytes, s);
        if (e != hipSuccess) return e;
    }
    c->live[*p] = bytes;
    if (!c->poison || bytes < 4) return hipSuccess;
    return launch_fill_u32(static_cast<uint32_t*>(*p), POISON_WORD, bytes / 4, s);
}

// Returns a lib_alloc buffer to the cache behind the work already enqueued on
// the context's stream; the oldest cached blocks beyond the cache's bounds
// go back to the stream-ordered allocator.
void lib_free(vs_ctx* c, void* p) {
    if (!p) return;
    auto it = c->live.find(p);
    if (it == c->live.end()) { hipFreeAsync(p, c->stream); return; }
    c->cache.push_back(vs_ctx::Block{p, it->second});
    c->cached_bytes += it->second;
    c->live.erase(it);
    while (!c->cache.empty() && (c->cache.size() > CACHE_MAX_BLOCKS || c->cached_bytes > CACHE_MAX_BYTES)) {
        hipFreeAsync(c->cache.front().p, c->stream);
        c->cached_bytes -= c->cache.front().bytes;
        c->cache.erase(c->cache.begin());
    }
}

// Hands every cached block back to the allocator (on a stream change, where
// stream order no longer covers reuse, and at context destruction).
void drain_cache(vs_ctx* c) {
    for (auto& b : c->cache) hipFreeAsync(b.p, c->stream);
    c->cache.clear();
    c->cached_bytes = 0;
}

// validate_tensor_val (validation.rs:60-140): NaN and Inf are errors, values
// outside [lo, hi] are logged.
struct Check {
    const char* name;
    const void* p;
    bool half;
    uint64_t n;
    uint32_t row, col0, col1;
    float lo, hi;
};
constexpr int MAX_CHECKS = 8;

vs_status run_checks(vs_ctx* c, const Check* checks, int count) {
    hipStream_t s = c->stream;
    for (int i = 0; i < count; ++i) {
        uint32_t* h = c->host_val + i * VALIDATE_WORDS;
        for (int w = 0; w < VALIDATE_WORDS; ++w) h[w] = 0u;
        h[VAL_FIRST_NAN] = h[VAL_FIRST_INF] = 0xFFFFFFFFu;
    }
    VS_HIP(hipMemcpyAsync(c->dev_val, c->host_val, (size_t)count * VALIDATE_WORDS * 4, hipMemcpyHostToDevice, s),
           "validation reset");
    for (int i = 0; i < count; ++i) {
        const Check& k = checks[i];
        VS_HIP(launch_validate(k.p, k.half, k.n, k.row, k.col0, k.col1, k.lo, k.hi, c->dev_val + i * VALIDATE_WORDS, s),
               "validation scan");
    }
    VS_HIP(hipMemcpyAsync(c->host_val, c->dev_val, (size_t)count * VALIDATE_WORDS * 4, hipMemcpyDeviceToHost, s),
           "validation readback");
    VS_HIP(hipStreamSynchronize(s), "hipStreamSynchronize(validation)");
    std::string bad;
    for (int i = 0; i < count; ++i) {
        const Check& k = checks[i];
        const uint32_t* h = c->host_val + i * VALIDATE_WORDS;
        const uint64_t total = k.n / k.row * (k.col1 - k.col0);
        if (h[VAL_BELOW])
            std::fprintf(stderr, "vsplat: tensor '%s': %u values < %g of %llu\n", k.name, h[VAL_BELOW], (double)k.lo,
                         (unsigned long long)total);
        if (h[VAL_ABOVE])
            std::fprintf(stderr, "vsplat: tensor '%s': %u values > %g of %llu\n", k.name, h[VAL_ABOVE], (double)k.hi,
                         (unsigned long long)total);
        if (h[VAL_NAN] || h[VAL_INF]) {
            char msg[256];
            std::snprintf(msg, sizeof msg, "%stensor '%s' has %u NaN (first @ element %lld), %u Inf (first @ element %lld)",
                          bad.empty() ? "" : "; ", k.name, h[VAL_NAN],
                          h[VAL_NAN] ? (long long)h[VAL_FIRST_NAN] : -1LL, h[VAL_INF],
                          h[VAL_INF] ? (long long)h[VAL_FIRST_INF] : -1LL);
            bad += msg;
        }
    }
    if (!bad.empty()) return fail(VS_ERR_NONFINITE, bad);
    return VS_OK;
}

// Splats::validate_values (gaussian_splats.rs:417-470) on the inputs of a render.
vs_status validate_splats(vs_ctx* c, const vs_splats* sp) {
    const uint64_t N = sp->num_splats;
    if (N == 0) return VS_OK;
    const uint64_t K = sp->decoder ? 4u : (uint64_t)(sp->sh_degree + 1) * (sp->sh_degree + 1);
    const float inf = __builtin_inff();
    Check ch[MAX_CHECKS];
    int n = 0;
    ch[n++] = Check{"means", sp->transforms, false, N * 10, 10, 0, 3, -inf, inf};
    ch[n++] = Check{"rotations", sp->transforms, false, N * 10, 10, 3, 7, -inf, inf};
    ch[n++] = Check{"log_scales", sp->transforms, false, N * 10, 10, 7, 10, -10.0f, 10.0f};
    ch[n++] = Check{"sh_coeffs", sp->sh_coeffs, sp->sh_dtype == VS_SH_F16, N * K * 3, 1, 0, 1, -5.0f, 5.0f};
    ch[n++] = Check{"raw_opacity", sp->raw_opacities, false, N, 1, 0, 1, -20.0f, 20.0f};
    if (sp->min_scale) ch[n++] = Check{"min_scale", sp->min_scale, false, N, 1, 0, 1, -inf, inf};
    if (sp->decoder) ch[n++] = Check{"decoder", sp->decoder, false, 816, 1, 0, 1, -inf, inf};
    return run_checks(c, ch, n);
}

vs_status check_splats(const vs_splats* sp) {
    if (!sp) return fail(VS_ERR_INVALID, "splats is null");
    if (sp->sh_degree > 4) return fail(VS_ERR_INVALID, "SH degree must be 0..4 (1, 4, 9, 16 or 25 coefficients)");
    if (sp->sh_dtype != VS_SH_F32 && sp->sh_dtype != VS_SH_F16)
        return fail(VS_ERR_INVALID, "SH coefficients must use f16 or f32");
    if (sp->num_splats > 0 && (!sp->transforms || !sp->sh_coeffs || !sp->raw_opacities))
        return fail(VS_ERR_INVALID, "splat parameter pointer is null");
    if (((uintptr_t)sp->transforms & 7u) != 0) return fail(VS_ERR_INVALID, "transforms must be 8-byte aligned");
    if (((uintptr_t)sp->sh_coeffs & 15u) != 0) return fail(VS_ERR_INVALID, "sh_coeffs must be 16-byte aligned");
    if (((uintptr_t)sp->raw_opacities & 3u) != 0) return fail(VS_ERR_INVALID, "raw_opacities must be 4-byte aligned");
    if (((uintptr_t)sp->min_scale & 3u) != 0) return fail(VS_ERR_INVALID, "min_scale must be 4-byte aligned");
    if (sp->decoder && sp->sh_degree > 3)
        return fail(VS_ERR_INVALID, "neural appearance: sh_degree is the decoder's direction band, 0..3");
    if (((uintptr_t)sp->decoder & 3u) != 0) return fail(VS_ERR_INVALID, "decoder must be 4-byte aligned");
    return VS_OK;
}

} // namespace

// ---- allocation-free sort scratch --------------------------------------------
// One array per GPU, used by vs_radix_argsort_u32_noalloc in place of the
// per-call allocation of vs_radix_argsort_u32.  In host code `scratch` names
// a host-side stand-in, not device memory: the device address of each GPU's
// copy comes from hipGetSymbolAddress, taken once per device (with that device
// current) when the first context on it is created, and only that address is
// ever handed to kernels.  A failed lookup leaves the context usable; only the
// allocation-free sort then reports it.
//
// Calls on one stream are ordered by the stream.  A call on another stream
// than the array's last user first waits (hipStreamWaitEvent, no allocation)
// on an event recorded after that user's sort, so sorts from different
// contexts or streams never overlap in the array.
constexpr uint32_t NOALLOC_SORT_MAX_KEYS = 1u << 22;
constexpr size_t SCRATCH_BYTES = (size_t)40 << 20;
static __device__ __align__(256) uint8_t scratch[SCRATCH_BYTES];

namespace {
constexpr int MAX_DEVICES = 64;
struct ScratchSlot {
    bool tried = false;
    void* ptr = nullptr;             // the array's device address on this GPU
    hipEvent_t done = nullptr;       // recorded after the last sort that used it
    bool used = false;
    hipStream_t last = nullptr;      // that sort's stream
    std::string error;               // why `ptr` is missing
};
std::mutex g_scratch_mutex;
ScratchSlot g_scratch[MAX_DEVICES];

// Set-up, called with `device` current.  Never fails the caller: a missing
// address is recorded and reported by the allocation-free sort.
void init_scratch(int device) {
    if (device < 0 || device >= MAX_DEVICES) return;
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ScratchSlot& sl = g_scratch[device];
    if (sl.tried) return;
    sl.tried = true;
    if (sort_tmp_bytes(NOALLOC_SORT_MAX_KEYS, false) + 256 > SCRATCH_BYTES) {
        sl.error = "the scratch array is smaller than its maximum sort needs";
        return;
    }
    void* ptr = nullptr;
    hipError_t e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr) {
        sl.error = std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e != hipSuccess ? e : hipErrorInvalidSymbol);
        return;
    }
    e = hipEventCreateWithFlags(&sl.done, hipEventDisableTiming);
    if (e != hipSuccess) {
        sl.done = nullptr;
        sl.error = std::string("hipEventCreateWithFlags: ") + hipGetErrorString(e);
        return;
    }
    sl.ptr = ptr;
}
} // namespace

extern "C" const char* vs_last_error(void) { return g_last_error.c_str(); }
extern "C" const char* vs_version(void) { return "vsplat-gfx950 0.1"; }

extern "C" vs_status vs_ctx_create(int device, void* hip_stream, vs_ctx** out) {
    if (!out) return fail(VS_ERR_INVALID, "out is null");
    *out = nullptr;
    int count = 0;
    VS_HIP(hipGetDeviceCount(&count), "hipGetDeviceCount");
    if (device < 0 || device >= count) return fail(VS_ERR_INVALID, "device index out of range");
    VS_HIP(hipSetDevice(device), "hipSetDevice");
    vs_ctx* c = new (std::nothrow) vs_ctx();
    if (!c) return fail(VS_ERR_OOM, "context allocation");
    c->device = device;
    c->stream = static_cast<hipStream_t>(hip_stream);
    hipError_t e = hipHostMalloc(reinterpret_cast<void**>(&c->host_counters), (CNT_COUNT + CTX_FLAGS) * sizeof(uint32_t),
                                 hipHostMallocDefault);
    if (e != hipSuccess) { delete c; return hip_fail(e, "hipHostMalloc"); }
    e = hipMalloc(reinterpret_cast<void**>(&c->dev_flags), CTX_FLAGS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMemset(c->dev_flags, 0, CTX_FLAGS * sizeof(uint32_t));
    if (e == hipSuccess) e = hipMalloc(reinterpret_cast<void**>(&c->dev_val), MAX_CHECKS * VALIDATE_WORDS * sizeof(uint32_t));
    if (e == hipSuccess)
        e = hipHostMalloc(reinterpret_cast<void**>(&c->host_val), MAX_CHECKS * VALIDATE_WORDS * sizeof(uint32_t),
                          hipHostMallocDefault);
    if (e != hipSuccess) {
        hipHostFree(c->host_counters);
        if (c->dev_flags) hipFree(c->dev_flags);
        if (c->dev_val) hipFree(c->dev_val);
        delete c;
        return hip_fail(e, "context buffers");
    }
    init_scratch(device);
    // VSPLAT_POISON=1 poisons every allocation of this context (a debug aid for test runs).
    const char* poison_env = std::getenv("VSPLAT_POISON");
    c->poison = poison_env && poison_env[0] == '1';
    // Keep freed stream-ordered allocations in the pool between renders.
    hipMemPool_t pool;
    if (hipDeviceGetDefaultMemPool(&pool, device) == hipSuccess) {
        uint64_t thr = ~0ull;
        hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &thr);
    }
    *out = c;
    return VS_OK;
}

extern "C" void vs_ctx_destroy(vs_ctx* c) {
    if (!c) return;
    hipSetDevice(c->device);
    drain_cache(c);
    hipStreamSynchronize(c->stream);
    for (auto& r : c->recs) { hipEventDestroy(r.b); hipEventDestroy(r.e); }
    for (auto e : c->pool) hipEventDestroy(e);
    for (auto e : c->tpool) hipEventDestroy(e);
    for (auto& kv : c->pending) {
        if (kv.second.ev) hipEventDestroy(kv.second.ev);
        if (kv.second.host) hipHostFree(kv.second.host);
    }
    hipHostFree(c->host_counters);
    hipHostFree(c->host_val);
    hipFree(c->dev_flags);
    hipFree(c->dev_val);
    delete c;
}

extern "C" vs_status vs_ctx_set_stream(vs_ctx* c, void* hip_stream) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    hipStream_t ns = static_cast<hipStream_t>(hip_stream);
    if (ns != c->stream) {
        // cached blocks were freed in the old stream's order: return them there
        drain_cache(c);
        VS_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize(old stream)");
    }
    c->stream = ns;
    return VS_OK;
}

extern "C" vs_status vs_ctx_set_depth_cutoff(vs_ctx* c, vs_cutoff_mode mode) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    if (mode != VS_CUTOFF_AUTO && mode != VS_CUTOFF_OFF && mode != VS_CUTOFF_ON)
        return fail(VS_ERR_INVALID, "unknown depth cutoff mode");
    c->depth_cutoff = mode;
    return VS_OK;
}

extern "C" vs_status vs_ctx_set_validation(vs_ctx* c, int enable) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    c->validate = enable != 0;
    return VS_OK;
}

extern "C" vs_status vs_ctx_set_poison(vs_ctx* c, int enable) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    c->poison = enable != 0;
    return VS_OK;
}

extern "C" vs_status vs_ctx_set_sort_spin_limit(vs_ctx* c, uint32_t polls) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    c->spin_limit = polls == 0xFFFFFFFFu ? SORT_SPIN_LIMIT_DEFAULT : polls;
    return VS_OK;
}

extern "C" vs_status vs_ctx_enable_timing(vs_ctx* c, uint32_t stages) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    if (stages & ~(uint32_t)VS_TIME_ALL) return fail(VS_ERR_INVALID, "unknown stage bit in the timing mask");
    c->timing = stages;
    return VS_OK;
}

extern "C" vs_status vs_ctx_stage_times(vs_ctx* c, vs_stage_times* out) {
    if (!c || !out) return fail(VS_ERR_INVALID, "null argument");
    VS_HIP(hipStreamSynchronize(c->stream), "hipStreamSynchronize");
    float ms[ST_N] = {};
    for (auto& r : c->recs) {
        float v = 0.0f;
        if (hipEventElapsedTime(&v, r.b, r.e) == hipSuccess) ms[r.stage] += v;
        c->tpool.push_back(r.b);
        c->tpool.push_back(r.e);
    }
    c->recs.clear();
    out->project_ms = ms[ST_PROJECT];
    out->emit_ms = ms[ST_EMIT];
    out->sort_ms = ms[ST_SORT];
    out->ranges_ms = ms[ST_RANGES];
    out->raster_fwd_ms = ms[ST_RASTER_FWD];
    out->raster_bwd_ms = ms[ST_RASTER_BWD];
    out->project_bwd_ms = ms[ST_PROJECT_BWD];
    out->other_ms = ms[ST_OTHER];
    return VS_OK;
}

extern "C" void vs_fwd_state_free(vs_fwd_state* st) {
    if (!st) return;
    hipSetDevice(st->ctx->device);
    lib_free(st->ctx, st->isect_arena);
    lib_free(st->ctx, st->arena);
    delete st;
}

namespace {

// settle_pending (render.rs:254-282): wait for the last lagged render at `k`
// (long finished by now), fold its count into the hint and report it.
vs_status settle(vs_ctx* ctx, const CapacityKey& k, bool& have, uint32_t& vis, uint32_t& isects) {
    have = false;
    auto it = ctx->pending.find(k);
    if (it == ctx->pending.end() || !it->second.live) return VS_OK;
    vs_ctx::Pending& p = it->second;
    VS_HIP(hipEventSynchronize(p.ev), "hipEventSynchronize(lagged counts)");
    p.live = false;
    const uint32_t* hc = p.host;
    if (hc[CNT_COUNT + FLAG_SORT_STALL] != 0u) {
        // the lagged render's own sorts: reported by the next call at its key
        VS_HIP(launch_fill_u32(ctx->dev_flags, 0u, CTX_FLAGS, ctx->stream), "flag reset");
        return fail(VS_ERR_HIP, std::string("the previous lagged render at this size: ") + SORT_STALL_MSG);
    }
    uint64_t I64 = 0;
    std::memcpy(&I64, hc + CNT_ISECT64, 8);
    ctx->lagged_renders += 1;
    if (I64 > p.capacity) {
        ctx->lagged_overflows += 1;
        std::fprintf(stderr, "vsplat: intersection capacity overflow: required=%llu, capacity=%zu, dropped=%.3f%% "
                     "(farthest splats), overflows=%llu/%llu renders\n", (unsigned long long)I64, p.capacity,
                     100.0 * (1.0 - (double)p.capacity / (double)I64), (unsigned long long)ctx->lagged_overflows,
                     (unsigned long long)ctx->lagged_renders);
    }
    ctx->caps.record(k, (size_t)I64, p.splats, p.limit);
    have = true;
    vis = hc[CNT_VISIBLE];
    isects = (uint32_t)std::min<uint64_t>(I64, 0xFFFFFFFFull);
    return VS_OK;
}

// intersection_ceiling (render.rs:197-216): the most intersections one render
// may allocate, consulting free device memory only for arenas big enough to
// matter (24 bytes per intersection at the arena's peak).
size_t isect_ceiling(size_t wanted, size_t limit) {
    size_t cap = limit;
    size_t free_b = 0, total_b = 0;
    if (wanted * 24 > (size_t)1 << 30 && hipMemGetInfo(&free_b, &total_b) == hipSuccess && wanted * 24 > free_b / 4)
        cap = std::min(cap, free_b / 24);
    return std::min(std::max<size_t>(cap, (size_t)1 << 16), limit);
}

} // namespace

extern "C" vs_status vs_ctx_set_lagged_counts(vs_ctx* c, int enable) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    c->lagged = enable != 0;
    return VS_OK;
}

extern "C" vs_status vs_ctx_settle_lagged_counts(vs_ctx* c, uint64_t* renders, uint64_t* overflows) {
    if (!c) return fail(VS_ERR_INVALID, "ctx is null");
    VS_HIP(hipSetDevice(c->device), "hipSetDevice");
    std::vector<CapacityKey> keys;
    for (auto& kv : c->pending) keys.push_back(kv.first);
    for (auto& k : keys) {
        bool have = false;
        uint32_t v = 0, i = 0;
        vs_status st = settle(c, k, have, v, i);
        if (st != VS_OK) return st;
    }
    // One line per settle so a clamped render shows in any log.
    std::fprintf(stderr, "vsplat: lagged render counts: %llu overflows / %llu renders\n",
                 (unsigned long long)c->lagged_overflows, (unsigned long long)c->lagged_renders);
    if (renders) *renders = c->lagged_renders;
    if (overflows) *overflows = c->lagged_overflows;
    return VS_OK;
}

// The L1 cotangent a forward may write with its image (vs_render_forward_l1).
struct L1Fuse {
    const uint32_t* gt;
    float mcx, mcy, mr;
    float* v_out;
};
static float l1_inv_count(vs_ctx* ctx, uint32_t w, uint32_t h, float mcx, float mcy, float mr);

static vs_status render_forward(vs_ctx* ctx, const vs_camera* cam, const vs_splats* sp, uint32_t W, uint32_t H,
                                const float background[3], vs_pass pass, vs_render_mode mode, vs_fwd_out* out,
                                vs_fwd_state** state_out, const L1Fuse* l1) {
    if (state_out) *state_out = nullptr;
    if (!ctx || !cam || !out || !background) return fail(VS_ERR_INVALID, "null argument");
    if (W == 0 || H == 0) return fail(VS_ERR_INVALID, "Can't render images with 0 size.");
    if (mode != VS_MODE_DEFAULT && mode != VS_MODE_MIP && mode != VS_MODE_SURFEL)
        return fail(VS_ERR_INVALID, "unknown render mode");
    const uint32_t pass_value = (uint32_t)pass;
    if (pass_value > 0xFFFFu || (pass_value & 0xFFu) > (uint32_t)VS_PASS_GEOMETRY_TRAIN_DEPTH)
        return fail(VS_ERR_INVALID, "unknown pass");
    const uint32_t count_slot = pass_value >> 8;
    pass = static_cast<vs_pass>(pass_value & 0xFFu);
    if (count_slot != 0 && !pass_has_slot(pass))
        return fail(VS_ERR_INVALID, "only VS_PASS_BACKWARD_DENSE and VS_PASS_EXPOSURE take a count slot");
    if (cam->model < VS_CAMERA_PINHOLE || cam->model > VS_CAMERA_TPF)
        return fail(VS_ERR_INVALID, "unknown camera model");
    vs_status vst = check_splats(sp);
    if (vst != VS_OK) return vst;
    if (mode == VS_MODE_SURFEL && sp->decoder)
        return fail(VS_ERR_UNSUPPORTED, "surfels take SH colour (no neural appearance)");
    if (!out->out_img) return fail(VS_ERR_INVALID, "out_img is null");
    if (pass_bwd_info(pass) && ((uintptr_t)out->out_img & 15u)) return fail(VS_ERR_INVALID, "out_img must be 16-byte aligned");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = ctx->stream;
    if (ctx->validate) {
        vs_status ve = validate_splats(ctx, sp);
        if (ve != VS_OK) return ve;
    }

    vs_fwd_state* st = new (std::nothrow) vs_fwd_state();
    if (!st) return fail(VS_ERR_OOM, "state allocation");
    struct Guard { vs_fwd_state*& p; ~Guard() { if (p) vs_fwd_state_free(p); } } guard{st};
    st->ctx = ctx;
    st->cam = *cam;
    st->W = W; st->H = H; st->N = sp->num_splats; st->degree = sp->sh_degree;
    st->neural = sp->decoder ? 1u : 0u;
    st->K = sp->decoder ? 4u : (sp->sh_degree + 1) * (sp->sh_degree + 1);
    st->sh_half = sp->sh_dtype == VS_SH_F16 ? 1u : 0u;
    st->mip = mode == VS_MODE_MIP ? 1u : 0u;
    st->surfel = mode == VS_MODE_SURFEL ? 1u : 0u;
    if (st->surfel && st->cam.model != VS_CAMERA_PINHOLE) {
        // render.rs:451-469: surfel ray-plane coverage is pinhole-only; a lens
        // camera renders as the pinhole with its focal length and principal point.
        if (ctx->surfel_lens_dropped++ == 0)
            std::fprintf(stderr, "vsplat: surfel (2DGS) rendering is pinhole-only: lens distortion ignored\n");
        st->cam.model = VS_CAMERA_PINHOLE;
    }
    st->min_scale = sp->min_scale;
    st->lso = sp->log_scale_offset;
    st->bg[0] = background[0]; st->bg[1] = background[1]; st->bg[2] = background[2];
    st->pass = pass;
    st->tbw = (W + TILE_W_HOST_ - 1) / TILE_W_HOST_;
    st->tbh = (H + TILE_W_HOST_ - 1) / TILE_W_HOST_;
    const uint64_t T64 = (uint64_t)st->tbw * st->tbh;
    // 2^24 tiles (a 65536 x 65536 image): a wavefront's 64 bounding boxes hold
    // under 2^30 tiles, and tile rows and offsets stay exact in f32.
    if (T64 > (1ull << 24)) return fail(VS_ERR_INVALID, "image too large (more than 2^24 tiles)");
    st->T = (uint32_t)T64;
    const uint32_t N = st->N, T = st->T;
    const bool bwd_info = pass_bwd_info(pass);
    const bool surfel = st->surfel != 0u;
    // Surfel renders with backward state always carry the geometry channels (render.rs:471-473).
    const bool geometry = pass_geometry(pass) || (surfel && bwd_info);
    const bool smooth = pass == VS_PASS_BACKWARD_SMOOTH_CUTOFF;
    const uint32_t nblocks = (N + 255) / 256;

    // ---- lagged training renders (render.rs:741-768) ------------------------------
    // A training render at a size with a capacity hint sizes its intersection
    // arena from it and does not wait for its own counts; it reports the
    // previous training render's at this size.  Other renders stay exact.
    const CapacityKey key{W, H, count_slot};
    const size_t limit = (size_t)std::max<uint64_t>(std::min<uint64_t>((uint64_t)N * T, 0xFFFFFFFFull), 1);
    const bool training = pass_training(pass);
    bool have_lag = false;
    uint32_t lag_vis = 0, lag_isects = 0;
    if (ctx->lagged && training) {
        vs_status se = settle(ctx, key, have_lag, lag_vis, lag_isects);
        if (se != VS_OK) return se;
    }
    size_t hint = 0;
    const bool lagged = ctx->lagged && training && N > 0 && ctx->caps.hint(key, N, limit, hint);
    const uint32_t isect_cap = lagged ? (uint32_t)std::min(hint, isect_ceiling(hint, limit)) : 0xFFFFFFFFu;
    // A lagged render's counts and flags go straight to the key's pinned slot
    // (the projection's counter kernel and the forward's tile-order kernel
    // write them there), read by the next training render at this key.
    vs_ctx::Pending* lag_slot = nullptr;
    if (lagged) {
        lag_slot = &ctx->pending[key];
        if (!lag_slot->host) {
            VS_HIP(hipHostMalloc(reinterpret_cast<void**>(&lag_slot->host), (CNT_COUNT + CTX_FLAGS) * sizeof(uint32_t),
                                 hipHostMallocDefault), "hipHostMalloc(lagged counts)");
            VS_HIP(hipEventCreateWithFlags(&lag_slot->ev, hipEventDisableTiming), "hipEventCreate(lagged counts)");
        }
    }

    // ---- per-splat arena -----------------------------------------------------
    size_t off = 0;
    auto take = [&](size_t bytes) { const size_t o = off; off += align256(bytes); return o; };
    const size_t o_counts = take((size_t)N * 4), o_depth = take((size_t)N * 4), o_compact = take((size_t)N * 4);
    const size_t o_proj = take((size_t)N * PROJ_Q * 16);
    const size_t o_aux = (geometry && !surfel) ? take((size_t)N * 16) : 0;
    const size_t o_surf = surfel ? take((size_t)N * 64) : 0;
    const size_t o_opac = out->opacities ? 0 : take((size_t)N * 4);
    const size_t o_rad = out->max_radius ? 0 : take((size_t)N * 4);
    const size_t o_vis = (bwd_info && !out->visible) ? take((size_t)N * 4) : 0;
    const size_t o_bs = take((size_t)std::max(nblocks, 1u) * 4 * BS_ROWS);
    const size_t o_cnt = take(CNT_COUNT * 4);
    const size_t o_rng = take((size_t)T * 8), o_rngs = take((size_t)T * 8);
    const size_t o_ord = take((size_t)8 * ((T + 7) / 8) * 4);
    VS_HIP(lib_alloc(ctx, &st->arena, off, s), "hipMallocAsync(splat arena)");
    char* base = static_cast<char*>(st->arena);
    st->counts = reinterpret_cast<uint32_t*>(base + o_counts);
    st->depth_bits = reinterpret_cast<uint32_t*>(base + o_depth);
    st->compact = reinterpret_cast<uint32_t*>(base + o_compact);
    st->proj = reinterpret_cast<float4*>(base + o_proj);
    st->proj_aux = (geometry && !surfel) ? reinterpret_cast<float4*>(base + o_aux) : nullptr;
    st->proj_surf = surfel ? reinterpret_cast<float4*>(base + o_surf) : nullptr;
    st->opacities = out->opacities ? out->opacities : reinterpret_cast<float*>(base + o_opac);
    st->max_radius = out->max_radius ? out->max_radius : reinterpret_cast<float*>(base + o_rad);
    st->visible = bwd_info ? (out->visible ? out->visible : reinterpret_cast<float*>(base + o_vis)) : nullptr;
    st->block_stats = reinterpret_cast<uint32_t*>(base + o_bs);
    st->counters = reinterpret_cast<uint32_t*>(base + o_cnt);
    st->ranges = reinterpret_cast<uint32_t*>(base + o_rng);
    st->ranges_shrunk = reinterpret_cast<uint32_t*>(base + o_rngs);
    st->tile_order = reinterpret_cast<uint32_t*>(base + o_ord);

    // ---- projection --------------------------------------------------------------
    {
        StageTimer tm(ctx, ST_PROJECT);
        ProjectArgs pa{};
        pa.cam = *cam;
        pa.img_w = W; pa.img_h = H; pa.tile_bw = st->tbw; pa.tile_bh = st->tbh;
        pa.num_splats = N; pa.sh_degree = sp->sh_degree; pa.log_scale_offset = sp->log_scale_offset;
        pa.transforms = sp->transforms; pa.sh = sp->sh_coeffs; pa.sh_half = st->sh_half; pa.min_scale = st->min_scale; pa.mip = st->mip; pa.decoder = sp->decoder; pa.raw_opac = sp->raw_opacities;
        pa.opacities = st->opacities; pa.max_radius = st->max_radius; pa.counts = st->counts;
        pa.depth_bits = st->depth_bits; pa.proj = st->proj;
        pa.proj_aux = st->proj_aux; pa.proj_surf = st->proj_surf; pa.compact = st->compact; pa.block_stats = st->block_stats;
        pa.visible = bwd_info ? st->visible : nullptr;   // cleared by the projection
        pa.ranges = st->ranges; pa.num_tiles = T;         // initialised by the projection
        VS_HIP(launch_project(pa, s), "project kernel");
        VS_HIP(launch_finalize_counts(st->block_stats, nblocks, st->counters, isect_cap, s,
                                      lag_slot ? lag_slot->host : nullptr), "projection counts");
        if (N == 0) VS_HIP(launch_ranges_init(st->ranges, T, s), "range init");
    }
    const uint32_t tile_bits = bit_length(T);     // the sentinel tile id T must fit too
    uint32_t depth_bits = 32;
    // Device-resident counts for the lagged path (null: the exact host counts).
    const uint32_t* m_dev = nullptr;
    const uint32_t* i_dev = nullptr;
    if (!lagged) {
        VS_HIP(hipMemcpyAsync(ctx->host_counters, st->counters, CNT_COUNT * 4, hipMemcpyDeviceToHost, s), "counter readback");
        VS_HIP(hipMemcpyAsync(ctx->host_counters + CNT_COUNT, ctx->dev_flags, CTX_FLAGS * 4, hipMemcpyDeviceToHost, s),
               "flag readback");
        VS_HIP(hipStreamSynchronize(s), "hipStreamSynchronize");
        const uint32_t* hc = ctx->host_counters;
        vs_status fe = take_sort_flag(ctx);   // a lagged render's sorts, enqueued earlier on this context
        if (fe != VS_OK) return fe;
        st->V = hc[CNT_VISIBLE];
        st->M = hc[CNT_EMITTERS];
        uint64_t I64 = 0;
        std::memcpy(&I64, hc + CNT_ISECT64, 8);
        if (I64 > 0xFFFFFFFFull) return fail(VS_ERR_CAPACITY, "intersection count exceeds u32");
        st->I = (uint32_t)I64;
        const uint32_t dmin = (st->V > 0) ? hc[CNT_DEPTH_MIN] : 0u;
        const uint32_t dmax = (st->V > 0) ? hc[CNT_DEPTH_MAX] : 0u;
        depth_bits = bit_length((uint64_t)(dmax - dmin));
        ctx->caps.record(key, (size_t)I64, N, limit);   // every exact render refines the hint
    } else {
        // Capacities: every splat may emit; the arena holds isect_cap pairs.
        st->V = N;
        st->M = N;
        st->I = isect_cap;
        m_dev = st->counters + CNT_EMITTERS;
        i_dev = st->counters + CNT_BOUNDED;
    }
    const uint32_t I = st->I, M = st->M;
    // Depth cutoff (gaussian modes): per-tile tables of (bh x CUT_BINS x (bw + 1))
    // u32 masses (then their sums over rows) and u16 prefix counts, at most 256 MiB.
    const uint64_t cut_words = (uint64_t)st->tbh * CUT_BINS * ((uint64_t)st->tbw + 1u);
    bool cutoff = false;
    if (!surfel && N > 0 && I > 0 && st->tbw <= CUT_MAX_BW && cut_words * 6u <= (256ull << 20) &&
        ctx->depth_cutoff != VS_CUTOFF_OFF)
        cutoff = ctx->depth_cutoff == VS_CUTOFF_ON || (uint64_t)I >= (uint64_t)CUT_AUTO_PER_TILE * T;
    st->cutoff = cutoff;
    hipEvent_t sort_done = nullptr;   // exact renders: the sorts' flag readback
    struct EventBack { vs_ctx* c; hipEvent_t& e; ~EventBack() { if (e) c->pool.push_back(e); } } sort_done_back{ctx, sort_done};

    // ---- binning: compaction, depth sort, slot scan, emission, tile sort ------------
    if (I > 0) {
        size_t ioff = 0;
        auto itake = [&](size_t bytes) { const size_t o = ioff; ioff += align256(bytes); return o; };
        const size_t o_tu = itake((size_t)I * 4), o_vu = itake((size_t)I * 4);
        const size_t o_t = itake((size_t)I * 4), o_v = itake((size_t)I * 4);
        const size_t o_dk = itake((size_t)M * 4), o_dv = itake((size_t)M * 4);
        const size_t o_dks = itake((size_t)M * 4), o_ord = itake((size_t)M * 4), o_base = itake((size_t)(M + 1) * 4);
        const size_t o_base_g = itake((size_t)N * 4);
        const size_t o_scan = itake(scan_lookback_status_words(M) * 4);
        const size_t o_mass = cutoff ? itake(cut_words * 4) : 0, o_allow = cutoff ? itake(cut_words * 2) : 0;
        const size_t o_cut = cutoff ? itake(T) : 0, o_kept = cutoff ? itake((size_t)N * 4) : 0;
        const size_t o_listed = cutoff ? itake(4) : 0;
        const size_t o_pend = cutoff ? itake((size_t)st->tbh * ((size_t)st->tbw + 1u) * 4) : 0;
        const size_t o_kblk = cutoff ? itake((size_t)nblocks * 4) : 0;
        const size_t o_ptot = cutoff ? itake(4) : 0;
        // serves both sorts (the depth sort on 9-bit digits, the tile sort on tile_rb-bit ones)
        const uint32_t tile_rb = tile_radix_bits(tile_bits);
        const size_t o_tmp = itake(std::max(sort_tmp_bytes(I, false, tile_rb), sort_tmp_bytes(M, false, DEPTH_RADIX_BITS)));
        VS_HIP(lib_alloc(ctx, &st->isect_arena, ioff, s), "hipMallocAsync(intersection arena)");
        char* ib = static_cast<char*>(st->isect_arena);
        uint32_t* tiles_u = reinterpret_cast<uint32_t*>(ib + o_tu);
        uint32_t* vals_u = reinterpret_cast<uint32_t*>(ib + o_vu);
        st->tiles = reinterpret_cast<uint32_t*>(ib + o_t);
        st->gids = reinterpret_cast<uint32_t*>(ib + o_v);
        uint32_t* dkeys = reinterpret_cast<uint32_t*>(ib + o_dk);
        uint32_t* dvals = reinterpret_cast<uint32_t*>(ib + o_dv);
        uint32_t* dkeys_sorted = reinterpret_cast<uint32_t*>(ib + o_dks);
        uint32_t* order = reinterpret_cast<uint32_t*>(ib + o_ord);
        uint32_t* slot_base = reinterpret_cast<uint32_t*>(ib + o_base);   // [M + 1], nearest emitter first, then the total
        uint32_t* slot_base_g = reinterpret_cast<uint32_t*>(ib + o_base_g);   // [N], written for emitters only
        uint32_t* scan_tmp = reinterpret_cast<uint32_t*>(ib + o_scan);
        uint32_t* err = ctx->dev_flags + FLAG_SORT_STALL;
        // the sorts' one-sweep state (shared scratch) is cleared by the kernel
        // before each sort: compaction for the depth sort, emission for the tile sort
        const SortZeroSpan depth_zero = sort_zero_span(M, 0, depth_bits, ib + o_tmp, DEPTH_RADIX_BITS);
        const SortZeroSpan tile_zero = (M > 0 && N > 0) ? sort_zero_span(I, 0, tile_bits, ib + o_tmp, tile_rb)
                                                         : SortZeroSpan{nullptr, 0};
        uint32_t* cut_mass = cutoff ? reinterpret_cast<uint32_t*>(ib + o_mass) : nullptr;
        uint16_t* cut_allow = cutoff ? reinterpret_cast<uint16_t*>(ib + o_allow) : nullptr;
        uint8_t* cut_tile = cutoff ? reinterpret_cast<uint8_t*>(ib + o_cut) : nullptr;
        st->kept_counts = cutoff ? reinterpret_cast<uint32_t*>(ib + o_kept) : nullptr;
        st->listed = cutoff ? reinterpret_cast<uint32_t*>(ib + o_listed) : nullptr;
        if (cutoff) {
            // each tile's cutoff bin, then each splat's pairs under it
            StageTimer tm(ctx, ST_EMIT);
            CutArgs ka{};
            ka.num_splats = N; ka.tile_bw = st->tbw; ka.tile_bh = st->tbh;
            ka.counts = st->counts; ka.depth_bits = st->depth_bits; ka.counters = st->counters;
            ka.proj = st->proj;
            ka.mass = cut_mass; ka.cut = cut_tile; ka.allow = cut_allow;
            ka.sat = cut_mass;   // the masses are spent once the bins are known
            ka.pend = reinterpret_cast<uint32_t*>(ib + o_pend);
            ka.pend_total = reinterpret_cast<uint32_t*>(ib + o_ptot);
            VS_HIP(launch_fill_u32(cut_mass, 0u, cut_words, s), "zero cutoff masses");
            VS_HIP(launch_cut_mass(ka, false, s), "cutoff masses (front bins)");
            VS_HIP(launch_cut_pending(ka, s), "cutoff pending tiles");
            VS_HIP(launch_cut_mass(ka, true, s), "cutoff masses (back bins)");
            VS_HIP(launch_cut_rows(ka, s), "cutoff bins");
            VS_HIP(launch_cut_sat(ka, s), "cutoff box counts");
            EmitArgs ca{};
            ca.num_splats = N; ca.tile_bw = st->tbw; ca.tile_bh = st->tbh;
            ca.counts = st->counts; ca.proj = st->proj;
            ca.cut = cut_tile; ca.allow = cut_allow; ca.depth_bits = st->depth_bits; ca.counters = st->counters;
            ca.counts_out = st->kept_counts; ca.sat = ka.sat;
            ca.kept_blocks = reinterpret_cast<uint32_t*>(ib + o_kblk);
            VS_HIP(launch_count_kept(ca, s), "cutoff counts");
            // the emitters are the splats that keep a pair: their count stays on the device
            VS_HIP(launch_scan_blocks(ca.kept_blocks, nblocks, st->counters + CNT_KEPT, s), "cutoff emitter offsets");
            m_dev = st->counters + CNT_KEPT;
        }
        const uint32_t* slot_counts = cutoff ? st->kept_counts : st->counts;
        {
            StageTimer tm(ctx, ST_EMIT);
            CompactArgs ca{};
            ca.num_splats = N; ca.counts = slot_counts; ca.depth_bits = st->depth_bits;
            ca.block_offsets = cutoff ? reinterpret_cast<const uint32_t*>(ib + o_kblk)
                                      : st->block_stats + (size_t)BS_EMIT * nblocks;
            ca.counters = st->counters;
            ca.keys = dkeys; ca.vals = dvals;
            ca.zero = depth_zero.ptr; ca.zero_words = depth_zero.words;   // the depth sort's one-sweep state
            ca.zero2 = scan_tmp; ca.zero2_words = scan_lookback_status_words(M);   // the slot scan's status
            VS_HIP(launch_compact(ca, s), "compaction");
        }
        {
            StageTimer tm(ctx, ST_SORT);
            // lagged counts sort over 32 bits: a pass above the view's depth
            // span (max - min of the visible depth bits) copies its input
            VS_HIP(radix_sort_pairs(dkeys, dvals, dkeys_sorted, order, M, m_dev, false, 0, depth_bits, ib + o_tmp,
                                    err, s, ctx->spin_limit, nullptr, depth_zero.ptr != nullptr, DEPTH_RADIX_BITS,
                                    lagged ? st->counters + CNT_DEPTH_MIN : nullptr),
                   "depth sort");
        }
        {
            StageTimer tm(ctx, ST_EMIT);
            VS_HIP(scan_u32_lookback(slot_counts, slot_base, M, scan_tmp, err, s, ctx->spin_limit, order, m_dev, N,
                                     slot_base_g, true, EMIT_SMALL_LIST),
                   "slot scan");
            EmitArgs ea{};
            ea.num_splats = N; ea.tile_bw = st->tbw; ea.tile_bh = st->tbh;
            ea.num_emitters = M; ea.m_dev = m_dev; ea.order = order;
            ea.counts = slot_counts; ea.slot_base = slot_base; ea.slot_base_g = slot_base_g;
            ea.zero = tile_zero.ptr; ea.zero_words = tile_zero.words;      // the tile sort's one-sweep state
            ea.proj = st->proj; ea.tiles = tiles_u; ea.vals = vals_u; ea.capacity = I;
            if (cutoff) {
                ea.cut = cut_tile; ea.allow = cut_allow; ea.depth_bits = st->depth_bits; ea.counters = st->counters;
                ea.listed = st->listed;
            }
            VS_HIP(launch_emit(ea, s), "emit kernel");
        }
        TileRangesOut tro{st->ranges, T, false};   // the tile sort's last pass finds the ranges
        {
            StageTimer tm(ctx, ST_SORT);
            VS_HIP(radix_sort_pairs(tiles_u, vals_u, st->tiles, st->gids, I, cutoff ? st->listed : i_dev, false, 0,
                                    tile_bits, ib + o_tmp, err, s, ctx->spin_limit, &tro, tile_zero.ptr != nullptr,
                                    tile_rb),
                   "tile sort");
            st->tiles_pending = tro.done;
        }
        if (bwd_info) st->qpass = tiles_u;
        if (!lagged) {
            // An exact render reports a sort that gave up before it returns: the
            // flag follows the sorts, and the host waits for it after the raster
            // is enqueued (the raster still runs behind the wait).
            VS_HIP(hipMemcpyAsync(ctx->host_counters + CNT_COUNT, ctx->dev_flags, CTX_FLAGS * 4, hipMemcpyDeviceToHost, s),
                   "flag readback");
            sort_done = ctx->take();
            VS_HIP(hipEventRecord(sort_done, s), "hipEventRecord(sorts)");
        }
        if (!tro.done) {
            StageTimer tm(ctx, ST_RANGES);
            VS_HIP(launch_tile_ranges(st->tiles, I, T, st->ranges, s, cutoff ? st->listed : i_dev), "tile ranges");
        }
    }

    // ---- rasterize ---------------------------------------------------------------
    {
        StageTimer tm(ctx, ST_RASTER_FWD);
        RasterArgs ra{};
        ra.img_w = W; ra.img_h = H; ra.tile_bw = st->tbw; ra.tile_bh = st->tbh; ra.num_tiles = T; ra.num_splats = N;
        // longest lists first within each XCD's band (the forward's cost grows with its list)
        // the caller's tile offsets are written by this pass and the forward
        // (no copy behind the forward)
        VS_HIP(launch_tile_order(st->ranges, T, st->tile_order, s, bwd_info ? st->ranges_shrunk : nullptr, true,
                                 ctx->dev_flags, lag_slot ? lag_slot->host + CNT_COUNT : nullptr, CTX_FLAGS,
                                 out->tile_offsets),
               "tile order");
        ra.order = st->tile_order;
        ra.bg_r = background[0]; ra.bg_g = background[1]; ra.bg_b = background[2];
        ra.gids = st->gids; ra.ranges = st->ranges; ra.ranges_shrunk = st->ranges_shrunk;
        ra.aux_ranges = bwd_info ? out->tile_offsets : nullptr;
        ra.proj = st->proj; ra.proj_aux = st->proj_aux;
        // surfels outside training take the median by the surface criterion (gaussian_splats.rs:100-106)
        ra.proj_surf = st->proj_surf; ra.surf_crit = (surfel && pass_surface_criterion(pass)) ? 1u : 0u;
        ra.out = out->out_img; ra.visible = st->visible;
        ra.qpass = reinterpret_cast<uint8_t*>(st->qpass);
        if (l1) {
            ra.l1_gt = l1->gt; ra.l1_v = l1->v_out;
            ra.l1_mcx = l1->mcx; ra.l1_mcy = l1->mcy; ra.l1_mr = l1->mr;
            ra.l1_inv = l1_inv_count(ctx, W, H, l1->mcx, l1->mcy, l1->mr);
        }
        VS_HIP(launch_raster_fwd(ra, bwd_info, geometry, smooth, s), "raster forward");
    }
    if (sort_done) {
        VS_HIP(hipEventSynchronize(sort_done), "hipEventSynchronize(sorts)");
        vs_status fe = take_sort_flag(ctx);
        if (fe != VS_OK) return fe;
    }
    if (lagged) {
        // Counts leave behind an event; the next training render at this size
        // (or vs_ctx_settle_lagged_counts) reads them.
        vs_ctx::Pending& p = *lag_slot;
        VS_HIP(hipEventRecord(p.ev, s), "hipEventRecord(lagged counts)");
        p.capacity = isect_cap; p.splats = N; p.limit = limit; p.live = true;
        out->num_visible = have_lag ? std::min(lag_vis, N) : 0u;
        out->num_intersections = have_lag ? lag_isects : 0u;
    } else {
        out->num_visible = st->V;
        out->num_intersections = I;
    }
    if (bwd_info && state_out) {
        *state_out = st;
        st = nullptr;   // ownership passes to the caller
    }
    return VS_OK;
}

extern "C" vs_status vs_render_forward(vs_ctx* ctx, const vs_camera* cam, const vs_splats* sp, uint32_t W, uint32_t H,
                                       const float background[3], vs_pass pass, vs_render_mode mode, vs_fwd_out* out,
                                       vs_fwd_state** state_out) {
    return render_forward(ctx, cam, sp, W, H, background, pass, mode, out, state_out, nullptr);
}

extern "C" vs_status vs_render_forward_l1(vs_ctx* ctx, const vs_camera* cam, const vs_splats* sp, uint32_t W,
                                          uint32_t H, const float background[3], vs_pass pass, vs_render_mode mode,
                                          const uint32_t* gt_packed, float mask_cx, float mask_cy, float mask_radius,
                                          float* v_out, vs_fwd_out* out, vs_fwd_state** state_out) {
    if (state_out) *state_out = nullptr;
    const vs_pass base = static_cast<vs_pass>((uint32_t)pass & 0xFFu);
    if (!pass_bwd_info(base) || pass_geometry(base) || mode == VS_MODE_SURFEL)
        return fail(VS_ERR_INVALID, "the fused L1 cotangent takes an RGBA training pass (no geometry channels, no surfels)");
    if (!gt_packed || !v_out) return fail(VS_ERR_INVALID, "null argument");
    if ((uintptr_t)v_out & 15u) return fail(VS_ERR_INVALID, "v_out must be 16-byte aligned");
    const L1Fuse l1{gt_packed, mask_cx, mask_cy, mask_radius, v_out};
    return render_forward(ctx, cam, sp, W, H, background, pass, mode, out, state_out, &l1);
}

extern "C" vs_status vs_render_backward(vs_ctx* ctx, vs_fwd_state* st, const vs_splats* sp, const float* out_img,
                                        const float* v_out, vs_grads* grads) {
    if (!ctx || !st || !out_img || !v_out || !grads) return fail(VS_ERR_INVALID, "null argument");
    if (!pass_bwd_info(st->pass)) return fail(VS_ERR_INVALID, "the forward pass kept no backward state");
    vs_status vst = check_splats(sp);
    if (vst != VS_OK) return vst;
    if (sp->num_splats != st->N || sp->sh_degree != st->degree || (sp->sh_dtype == VS_SH_F16) != (st->sh_half != 0))
        return fail(VS_ERR_INVALID, "splats differ from the forward's");
    if ((sp->min_scale != nullptr) != (st->min_scale != nullptr))
        return fail(VS_ERR_INVALID, "the backward's scale floor must match the forward's (both set or both null)");
    if ((sp->decoder != nullptr) != (st->neural != 0u))
        return fail(VS_ERR_INVALID, "the backward's decoder must match the forward's (both set or both null)");
    if (st->neural && grads->v_sh_coeffs && ((uintptr_t)grads->v_sh_coeffs & 15u))
        return fail(VS_ERR_INVALID, "neural row gradients must be 16-byte aligned");
    if (((uintptr_t)out_img & 15u) || ((uintptr_t)v_out & 15u)) return fail(VS_ERR_INVALID, "images must be 16-byte aligned");
    if (grads->v_transforms && ((uintptr_t)grads->v_transforms & 7u)) return fail(VS_ERR_INVALID, "v_transforms must be 8-byte aligned");
    const bool dense = grads->v_transforms || grads->v_sh_coeffs || grads->v_raw_opacities || grads->v_refine_weight ||
                       grads->v_decoder || grads->v_coeffs_sq;
    if (st->pass == VS_PASS_BACKWARD_FUSED_UPDATE && (dense || !grads->v_combined))
        return fail(VS_ERR_INVALID, "a BACKWARD_FUSED_UPDATE render's backward stops at v_combined: pass only "
                                    "v_combined (gaussian_splats.rs:83-86)");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = ctx->stream;
    const uint32_t N = st->N;
    float* vc = grads->v_combined;
    void* vc_alloc = nullptr;
    const uint32_t n_grads = st->surfel ? 17u : 10u;      // raster gradient components per splat
    if (!vc && N > 0) {
        VS_HIP(lib_alloc(ctx, &vc_alloc, (size_t)N * n_grads * 4, s), "hipMallocAsync(v_combined)");
        vc = static_cast<float*>(vc_alloc);
    }
    if (vc && ((uintptr_t)vc & 7u)) return fail(VS_ERR_INVALID, "v_combined must be 8-byte aligned");
    {
        // The raster backward's stage time is its kernel's own execution: the
        // launch records the two events around the dispatch.
        if (st->I > 0) {
            RasterBwdArgs rb{};
            rb.img_w = st->W; rb.img_h = st->H; rb.tile_bw = st->tbw; rb.tile_bh = st->tbh; rb.num_tiles = st->T;
            rb.num_splats = N;
            // the backward walks the shrunk ranges: order by their lengths; the
            // same launch clears v_combined
            VS_HIP(launch_tile_order(st->ranges_shrunk, st->T, st->tile_order, s, nullptr, false, nullptr, nullptr, 0,
                                     nullptr, vc, (uint64_t)N * n_grads),
                   "tile order and v_combined clear");
            rb.order = st->tile_order;
            rb.bg_r = st->bg[0]; rb.bg_g = st->bg[1]; rb.bg_b = st->bg[2];
            rb.gids = st->gids; rb.ranges = st->ranges_shrunk;
            rb.proj = st->proj;
            rb.out_img = out_img; rb.v_out = v_out;
            rb.channels = (pass_geometry(st->pass) || st->surfel) ? 12u : 4u;
            rb.proj_surf = st->proj_surf;
            rb.v_combined = vc;
            rb.qpass = st->qpass;
            hipEvent_t eb = nullptr, ee = nullptr;
            if (ctx->timing & (1u << ST_RASTER_BWD)) { eb = ctx->take_timing(); ee = ctx->take_timing(); }
            VS_HIP(launch_raster_bwd(rb, st->pass == VS_PASS_BACKWARD_SMOOTH_CUTOFF, s, eb, ee), "raster backward");
            if (eb) ctx->recs.push_back(vs_ctx::Rec{(int)ST_RASTER_BWD, eb, ee});
        } else {
            VS_HIP(launch_fill_f32(vc, 0.0f, (uint64_t)N * n_grads, s), "zero v_combined");
        }
    }
    // With no dense gradient requested the backward stops at the raster
    // gradients (the reference's BackwardFusedUpdate pass: vs_project_update
    // then takes v_combined).
    if (dense) {
        StageTimer tm(ctx, ST_PROJECT_BWD);
        ProjectBwdArgs pb{};
        pb.cam = st->cam; pb.num_splats = N; pb.sh_degree = st->degree; pb.log_scale_offset = st->lso;
        pb.transforms = sp->transforms; pb.sh = sp->sh_coeffs; pb.sh_half = st->sh_half; pb.min_scale = sp->min_scale; pb.mip = st->mip; pb.raw_opac = sp->raw_opacities;
        pb.decoder = sp->decoder; pb.surfel = st->surfel;
        pb.counts = st->counts; pb.v_combined = vc;
        pb.v_transforms = grads->v_transforms; pb.v_sh = grads->v_sh_coeffs;
        pb.v_raw_opac = grads->v_raw_opacities; pb.v_refine = grads->v_refine_weight;
        VS_HIP(launch_project_bwd(pb, s), "projection backward");
        if (st->neural) {
            // project_bwd_neural's second half (bwd/render_bwd.rs:390-435)
            NeuralBwdArgs nb{};
            nb.cam = st->cam; nb.num_splats = N; nb.degree = st->degree; nb.transforms = sp->transforms;
            nb.rows = sp->sh_coeffs; nb.half = st->sh_half; nb.decoder = sp->decoder; nb.v_combined = vc;
            nb.v_transforms = grads->v_transforms; nb.v_rows = grads->v_sh_coeffs; nb.v_rows_sq = grads->v_coeffs_sq;
            nb.v_decoder = grads->v_decoder;
            void* part = nullptr;
            VS_HIP(lib_alloc(ctx, &part, (size_t)neural_bwd_blocks(N) * 816 * sizeof(float), s),
                   "hipMallocAsync(decoder partials)");
            nb.partials = static_cast<float*>(part);
            const hipError_t e = launch_neural_bwd(nb, s);
            lib_free(ctx, part);
            VS_HIP(e, "neural backward");
        }
    }
    vs_status ve = VS_OK;
    if (ctx->validate && N > 0) {
        // bwd_validate (gaussian_splats.rs:475-509): the parameter gradients, or
        // the raster gradients when the backward stops there
        const uint32_t K = st->neural ? 4u : (st->degree + 1) * (st->degree + 1);
        const float inf = __builtin_inff();
        Check ch[MAX_CHECKS];
        int n = 0;
        if (grads->v_transforms) ch[n++] = Check{"gradient_transforms", grads->v_transforms, false, (uint64_t)N * 10, 1, 0, 1, -inf, inf};
        if (grads->v_sh_coeffs) ch[n++] = Check{"gradient_sh_coeffs", grads->v_sh_coeffs, false, (uint64_t)N * K * 3, 1, 0, 1, -inf, inf};
        if (grads->v_raw_opacities) ch[n++] = Check{"gradient_raw_opacities", grads->v_raw_opacities, false, N, 1, 0, 1, -inf, inf};
        if (!dense) ch[n++] = Check{"gradient_v_combined", vc, false, (uint64_t)N * n_grads, 1, 0, 1, -inf, inf};
        ve = run_checks(ctx, ch, n);
    }
    if (vc_alloc) lib_free(ctx, vc_alloc);
    return ve;
}

extern "C" vs_status vs_pose_backward(vs_ctx* ctx, vs_fwd_state* st, const vs_splats* sp, const float* v_combined,
                                      float* v_pose) {
    if (!ctx || !st || !v_combined || !v_pose) return fail(VS_ERR_INVALID, "null argument");
    if (!pass_bwd_info(st->pass)) return fail(VS_ERR_INVALID, "the forward pass kept no backward state");
    if (st->neural) return fail(VS_ERR_UNSUPPORTED, "the camera gradient follows the SH colour path (no neural appearance)");
    if (st->surfel) return fail(VS_ERR_UNSUPPORTED, "the camera gradient is built for gaussians (not surfels)");
    vs_status vst = check_splats(sp);
    if (vst != VS_OK) return vst;
    if (sp->num_splats != st->N || sp->sh_degree != st->degree || (sp->sh_dtype == VS_SH_F16) != (st->sh_half != 0))
        return fail(VS_ERR_INVALID, "splats differ from the forward's");
    if ((sp->min_scale != nullptr) != (st->min_scale != nullptr))
        return fail(VS_ERR_INVALID, "the scale floor must match the forward's (both set or both null)");
    if ((uintptr_t)v_combined & 7u) return fail(VS_ERR_INVALID, "v_combined must be 8-byte aligned");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = ctx->stream;
    StageTimer tm(ctx, ST_PROJECT_BWD);
    PoseBwdArgs pa{};
    pa.cam = st->cam; pa.num_splats = st->N; pa.sh_degree = st->degree; pa.log_scale_offset = st->lso;
    pa.transforms = sp->transforms; pa.sh = sp->sh_coeffs; pa.sh_half = st->sh_half; pa.min_scale = sp->min_scale;
    pa.mip = st->mip; pa.raw_opac = sp->raw_opacities; pa.v_combined = v_combined; pa.v_pose = v_pose;
    void* part = nullptr;
    const uint32_t nb = pose_bwd_blocks(st->N);
    if (nb > 0) VS_HIP(lib_alloc(ctx, &part, (size_t)nb * 12 * sizeof(float), s), "hipMallocAsync(pose partials)");
    pa.partials = static_cast<float*>(part);
    const hipError_t e = launch_pose_bwd(pa, s);
    if (part) lib_free(ctx, part);
    VS_HIP(e, "pose backward");
    return VS_OK;
}

extern "C" vs_status vs_project_update(vs_ctx* ctx, vs_fwd_state* st, float* transforms, const void* sh_coeffs,
                                       float* raw_opacities, const float* v_combined, uint32_t* w_t,
                                       const float* lr_scale, uint32_t* w_o, const vs_adam_step* adam,
                                       vs_update_out* out) {
    if (!ctx || !st || !adam || !out) return fail(VS_ERR_INVALID, "null argument");
    if (!pass_bwd_info(st->pass)) return fail(VS_ERR_INVALID, "the forward pass kept no backward state");
    if (st->neural) return fail(VS_ERR_UNSUPPORTED, "the fused update takes SH colour (neural appearance trains unfused)");
    if (st->surfel) return fail(VS_ERR_UNSUPPORTED, "the fused update is built for gaussians (surfels train unfused)");
    const uint32_t N = st->N;
    if (N > 0 && (!transforms || !sh_coeffs || !raw_opacities || !v_combined || !w_t || !lr_scale || !w_o))
        return fail(VS_ERR_INVALID, "parameter, gradient or moment pointer is null");
    if (((uintptr_t)transforms & 7u) || ((uintptr_t)v_combined & 7u))
        return fail(VS_ERR_INVALID, "transforms and v_combined must be 8-byte aligned");
    if (((uintptr_t)sh_coeffs & 15u)) return fail(VS_ERR_INVALID, "sh_coeffs must be 16-byte aligned");
    if (!(adam->epsilon > 0.0f)) return fail(VS_ERR_INVALID, "Adam epsilon must be positive (it scales the moment codec)");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    StageTimer tm(ctx, ST_PROJECT_BWD);
    ProjectUpdateArgs pu{};
    pu.cam = st->cam; pu.num_splats = N; pu.sh_degree = st->degree; pu.log_scale_offset = st->lso;
    pu.transforms = transforms; pu.sh = sh_coeffs; pu.sh_half = st->sh_half; pu.min_scale = st->min_scale; pu.mip = st->mip; pu.raw_opac = raw_opacities; pu.compact = st->compact;
    pu.v_combined = v_combined; pu.w_t = w_t; pu.lr_scale = lr_scale; pu.w_o = w_o;
    pu.beta1 = adam->beta1; pu.beta2 = adam->beta2; pu.inv1 = adam->inv1; pu.inv2 = adam->inv2;
    pu.epsilon = adam->epsilon; pu.lr_opac = adam->lr_opac; pu.opac_reg = adam->opac_reg; pu.round_seed = adam->round_seed;
    pu.color_dir = out->color_dir; pu.v_refine = out->v_refine_weight; pu.grad_sq = out->coeffs_grad_sq;
    VS_HIP(launch_project_update(pu, ctx->stream), "project update");
    return VS_OK;
}

extern "C" vs_status vs_block8_encode(vs_ctx* ctx, const float* values, uint32_t n, uint32_t* codes, float* scales) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (n == 0) return VS_OK;
    if (!values || !codes || !scales) return fail(VS_ERR_INVALID, "null buffer");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_b8_encode(values, n, codes, scales, ctx->stream), "block8 encode");
    return VS_OK;
}

extern "C" vs_status vs_block8_decode(vs_ctx* ctx, const uint32_t* codes, const float* scales, uint32_t n,
                                      float* values) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (n == 0) return VS_OK;
    if (!values || !codes || !scales) return fail(VS_ERR_INVALID, "null buffer");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_b8_decode(codes, scales, n, values, ctx->stream), "block8 decode");
    return VS_OK;
}

extern "C" vs_status vs_block8_zero_rows(vs_ctx* ctx, uint32_t* codes, uint32_t n, const uint32_t* rows,
                                         uint32_t num_rows, uint32_t row_width) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if ((uint64_t)num_rows * row_width == 0 || n == 0) return VS_OK;
    if (!codes || !rows) return fail(VS_ERR_INVALID, "null buffer");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_b8_zero_rows(codes, n, rows, num_rows, row_width, ctx->stream), "block8 zero rows");
    return VS_OK;
}

extern "C" vs_status vs_sh_step(vs_ctx* ctx, uint16_t* sh_coeffs, uint32_t num_splats, uint32_t sh_degree,
                                const float* color_dir, const uint32_t* grad_rows, const float* grad_sq,
                                float* variance, uint32_t* codes, float* scales, const float* lr_scale,
                                const vs_sh_step_params* p) {
    if (!ctx || !p) return fail(VS_ERR_INVALID, "null argument");
    if (sh_degree > 4) return fail(VS_ERR_INVALID, "SH degree must be 0..4 (1, 4, 9, 16 or 25 coefficients)");
    if (num_splats == 0) return VS_OK;
    const uint64_t values = (uint64_t)num_splats * (sh_degree + 1) * (sh_degree + 1) * 3;
    if (values > 0xFFFFFF00ull) return fail(VS_ERR_INVALID, "too many SH values for 32-bit value indices");
    if (!sh_coeffs || !color_dir || !grad_rows || !grad_sq || !variance || !codes || !scales || !lr_scale)
        return fail(VS_ERR_INVALID, "null buffer");
    if (((uintptr_t)sh_coeffs & 7u) || ((uintptr_t)codes & 3u) || ((uintptr_t)scales & 3u))
        return fail(VS_ERR_INVALID, "sh_coeffs must be 8-byte aligned, codes and scales 4-byte aligned");
    if (!(p->epsilon > 0.0f)) return fail(VS_ERR_INVALID, "Adam epsilon must be positive");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    StageTimer tm(ctx, ST_OTHER);
    ShStepArgs a{};
    a.num_splats = num_splats; a.sh_degree = sh_degree;
    a.num_values = (uint32_t)values; a.num_blocks = (uint32_t)((values + 127) / 128);
    a.sh = sh_coeffs; a.color_dir = color_dir; a.grad_rows = grad_rows; a.grad_sq = grad_sq;
    a.variance = variance; a.codes = codes; a.scales = scales; a.lr_scale = lr_scale;
    a.beta1 = p->beta1; a.beta2 = p->beta2; a.inv1 = p->inv1; a.inv2 = p->inv2; a.epsilon = p->epsilon; a.lr = p->lr;
    a.round_seed = p->round_seed; a.first = p->first ? 1u : 0u;
    VS_HIP(launch_sh_step(a, ctx->stream), "SH step");
    return VS_OK;
}

extern "C" vs_status vs_geo_encode(vs_ctx* ctx, const float* m, const float* v, uint32_t n, float epsilon,
                                   uint32_t* words) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (n == 0) return VS_OK;
    if (!m || !v || !words) return fail(VS_ERR_INVALID, "null buffer");
    if (!(epsilon > 0.0f)) return fail(VS_ERR_INVALID, "epsilon must be positive");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_geo_encode(m, v, n, epsilon, words, ctx->stream), "geo encode");
    return VS_OK;
}

extern "C" vs_status vs_geo_decode(vs_ctx* ctx, const uint32_t* words, uint32_t n, float epsilon, float* m, float* v) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (n == 0) return VS_OK;
    if (!m || !v || !words) return fail(VS_ERR_INVALID, "null buffer");
    if (!(epsilon > 0.0f)) return fail(VS_ERR_INVALID, "epsilon must be positive");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_geo_decode(words, n, epsilon, m, v, ctx->stream), "geo decode");
    return VS_OK;
}

extern "C" vs_status vs_geo_zero_rows(vs_ctx* ctx, uint32_t* words, uint64_t num_words, const uint32_t* rows,
                                      uint32_t num_rows, uint32_t row_width) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if ((uint64_t)num_rows * row_width == 0) return VS_OK;
    if (!words || !rows) return fail(VS_ERR_INVALID, "null buffer");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_geo_zero_rows(words, rows, num_rows, row_width, num_words, ctx->stream), "geo zero rows");
    return VS_OK;
}

extern "C" vs_status vs_fwd_state_view(const vs_fwd_state* st, vs_state_view* o) {
    if (!st || !o) return fail(VS_ERR_INVALID, "null argument");
    if (st->tiles_pending && st->I > 0) {
        vs_ctx* ctx = st->ctx;
        VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
        VS_HIP(launch_tiles_from_ranges(st->ranges, st->T, st->I, st->tiles, ctx->stream), "tile ids from ranges");
        VS_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        st->tiles_pending = false;
    }
    o->num_splats = st->N; o->num_visible = st->V; o->num_intersections = st->I; o->num_tiles = st->T;
    o->tile_bw = st->tbw; o->tile_bh = st->tbh;
    o->isect_tiles = st->tiles; o->isect_gids = st->gids; o->intersect_counts = st->counts;
    o->depth_bits = st->depth_bits;
    o->compact_from_global = st->compact;
    // views into the 64-byte rows (VS_PROJ_ROW_FLOATS floats apart)
    o->proj_xy_conic = reinterpret_cast<const float*>(st->proj);
    o->proj_c11_opac_rg = reinterpret_cast<const float*>(st->proj) + 4;
    o->proj_b = reinterpret_cast<const float*>(st->proj) + 8;
    o->proj_aux = reinterpret_cast<const float*>(st->proj_aux);
    o->proj_surf = reinterpret_cast<const float*>(st->proj_surf);
    o->tile_ranges = st->ranges;
    o->listed_intersections = st->I;
    o->depth_cutoff = st->cutoff ? 1u : 0u;
    o->listed_counts = st->cutoff ? st->kept_counts : st->counts;
    if (st->cutoff && st->listed) {
        vs_ctx* ctx = st->ctx;
        VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
        uint32_t listed = 0;
        VS_HIP(hipMemcpyAsync(&listed, st->listed, 4, hipMemcpyDeviceToHost, ctx->stream), "listed count readback");
        VS_HIP(hipStreamSynchronize(ctx->stream), "hipStreamSynchronize");
        o->listed_intersections = std::min(listed, st->I);
    }
    return VS_OK;
}

extern "C" vs_status vs_radix_argsort_u32(vs_ctx* ctx, const uint32_t* keys, const uint32_t* vals, uint32_t n,
                                          const uint32_t* n_dev, uint32_t skip_bits, uint32_t sorting_bits,
                                          uint32_t* out_keys, uint32_t* out_vals) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (skip_bits + sorting_bits > 32) return fail(VS_ERR_INVALID, "Can only sort up to 32 bits");
    if (n == 0) return VS_OK;
    if (!keys || !vals || !out_keys || !out_vals) return fail(VS_ERR_INVALID, "null buffer");
    if (keys == out_keys || vals == out_vals) return fail(VS_ERR_INVALID, "outputs must not alias inputs");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    void* tmp = nullptr;
    VS_HIP(lib_alloc(ctx, &tmp, sort_tmp_bytes(n, false), ctx->stream), "hipMallocAsync(sort tmp)");
    StageTimer tm(ctx, ST_OTHER);
    hipError_t e = radix_sort_pairs(keys, vals, out_keys, out_vals, n, n_dev, false, skip_bits, skip_bits + sorting_bits,
                                    tmp, ctx->dev_flags + FLAG_SORT_STALL, ctx->stream, ctx->spin_limit);
    lib_free(ctx, tmp);
    if (e != hipSuccess) return hip_fail(e, "radix sort");
    return sync_sort_flag(ctx);
}

extern "C" vs_status vs_radix_argsort_u32_noalloc(vs_ctx* ctx, const uint32_t* keys, const uint32_t* vals, uint32_t n,
                                                  const uint32_t* n_dev, uint32_t skip_bits, uint32_t sorting_bits,
                                                  uint32_t* out_keys, uint32_t* out_vals) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (skip_bits + sorting_bits > 32) return fail(VS_ERR_INVALID, "Can only sort up to 32 bits");
    if (n > NOALLOC_SORT_MAX_KEYS)
        return fail(VS_ERR_CAPACITY, "vs_radix_argsort_u32_noalloc sorts at most 4194304 keys (its scratch array's size)");
    if (n == 0) return VS_OK;
    if (!keys || !vals || !out_keys || !out_vals) return fail(VS_ERR_INVALID, "null buffer");
    if (keys == out_keys || vals == out_vals) return fail(VS_ERR_INVALID, "outputs must not alias inputs");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    if (ctx->device < 0 || ctx->device >= MAX_DEVICES) return fail(VS_ERR_INVALID, "device index beyond the library's table");
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    ScratchSlot& sl = g_scratch[ctx->device];
    if (!sl.ptr)
        return fail(VS_ERR_INVALID, "the allocation-free sort's scratch array is unavailable on this device: " +
                                        (sl.tried ? sl.error : std::string("no context was created on it")));
    // Order this sort behind the array's last user on another stream.
    if (sl.used && sl.last != ctx->stream)
        VS_HIP(hipStreamWaitEvent(ctx->stream, sl.done, 0), "hipStreamWaitEvent(scratch)");
    // Stream-ordered, no wait: a pass that gave up sets the context's flag,
    // which the next synchronising call on the context reports.
    const hipError_t e = radix_sort_pairs(keys, vals, out_keys, out_vals, n, n_dev, false, skip_bits,
                                          skip_bits + sorting_bits, sl.ptr, ctx->dev_flags + FLAG_SORT_STALL, ctx->stream,
                                          ctx->spin_limit);
    if (e != hipSuccess) return hip_fail(e, "radix sort");
    VS_HIP(hipEventRecord(sl.done, ctx->stream), "hipEventRecord(scratch)");
    sl.used = true;
    sl.last = ctx->stream;
    return VS_OK;
}

extern "C" vs_status vs_radix_argsort_u64(vs_ctx* ctx, const uint64_t* keys, const uint32_t* vals, uint32_t n,
                                          uint32_t sorting_bits, uint64_t* out_keys, uint32_t* out_vals) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (sorting_bits > 64) return fail(VS_ERR_INVALID, "Can only sort up to 64 bits");
    if (n == 0) return VS_OK;
    if (!keys || !vals || !out_keys || !out_vals) return fail(VS_ERR_INVALID, "null buffer");
    if (keys == out_keys || vals == out_vals) return fail(VS_ERR_INVALID, "outputs must not alias inputs");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    void* tmp = nullptr;
    VS_HIP(lib_alloc(ctx, &tmp, sort_tmp_bytes(n, true), ctx->stream), "hipMallocAsync(sort tmp)");
    StageTimer tm(ctx, ST_OTHER);
    hipError_t e = radix_sort_pairs(keys, vals, out_keys, out_vals, n, nullptr, true, 0, sorting_bits, tmp,
                                    ctx->dev_flags + FLAG_SORT_STALL, ctx->stream, ctx->spin_limit);
    lib_free(ctx, tmp);
    if (e != hipSuccess) return hip_fail(e, "radix sort");
    return sync_sort_flag(ctx);
}

extern "C" vs_status vs_stream_probe(vs_ctx* ctx, void* buf, uint64_t bytes, int32_t mode) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (mode < 0 || mode > 3) return fail(VS_ERR_INVALID, "mode must be 0..3 (vs_probe_mode)");
    const uint64_t width = (mode & 2) ? 4u : 16u;
    if (!buf || ((uintptr_t)buf & (width - 1)) || bytes % width)
        return fail(VS_ERR_INVALID, "buf must be non-null and aligned, bytes a multiple of the word width");
    if (bytes == 0) return VS_OK;
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    void* sink = nullptr;
    if ((mode & 1) == 0) VS_HIP(lib_alloc(ctx, &sink, (size_t)calib_sink_words() * 4, ctx->stream), "hipMallocAsync(sink)");
    const hipError_t e = launch_stream_probe(buf, bytes, mode, static_cast<uint32_t*>(sink), ctx->stream);
    if (sink) lib_free(ctx, sink);
    if (e != hipSuccess) return hip_fail(e, "stream probe");
    return VS_OK;
}

extern "C" vs_status vs_compositing_exp2(vs_ctx* ctx, uint32_t first_bits, uint64_t count, float* out) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (count > (1ull << 32) - first_bits) return fail(VS_ERR_INVALID, "the range passes bit pattern 0xFFFFFFFF");
    if (count == 0) return VS_OK;
    if (!out) return fail(VS_ERR_INVALID, "out is null");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_exp2_range(first_bits, count, out, ctx->stream), "compositing exp2");
    return VS_OK;
}

extern "C" vs_status vs_raster_division(vs_ctx* ctx, float a, const uint32_t* bits, uint64_t count, float* out) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (count == 0) return VS_OK;
    if (!bits || !out) return fail(VS_ERR_INVALID, "null buffer");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_division_values(a, bits, count, out, ctx->stream), "raster division");
    return VS_OK;
}

extern "C" vs_status vs_raster_division_mismatches(vs_ctx* ctx, float a, uint64_t* mismatches) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (!mismatches) return fail(VS_ERR_INVALID, "mismatches is null");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_fill_u32(reinterpret_cast<uint32_t*>(mismatches), 0u, 2u, ctx->stream), "zero mismatch count");
    VS_HIP(launch_division_check(a, reinterpret_cast<unsigned long long*>(mismatches), ctx->stream), "raster division check");
    return VS_OK;
}

extern "C" vs_status vs_prefix_sum_u32(vs_ctx* ctx, const uint32_t* in, uint32_t* out, uint32_t n) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (n == 0) return VS_OK;
    if (!in || !out) return fail(VS_ERR_INVALID, "null buffer");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    void* tmp = nullptr;
    VS_HIP(lib_alloc(ctx, &tmp, scan_tmp_words(n) * 4, ctx->stream), "hipMallocAsync(scan tmp)");
    hipError_t e = scan_u32(in, out, n, true, static_cast<uint32_t*>(tmp), nullptr, ctx->stream);
    lib_free(ctx, tmp);
    if (e != hipSuccess) return hip_fail(e, "prefix sum");
    return VS_OK;
}

extern "C" vs_status vs_scan_in_place_u32(vs_ctx* ctx, uint32_t* data, uint32_t n) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    if (n == 0) return VS_OK;
    if (!data) return fail(VS_ERR_INVALID, "null buffer");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(scan_single_block(data, n, true, nullptr, ctx->stream), "scan in place");
    return VS_OK;
}

namespace {
vs_status loss_args(const float* pred, uint32_t channels, const uint32_t* gt, uint32_t w, uint32_t h,
                    const vs_loss_cfg* cfg, LossArgs& a) {
    if (!pred || !gt || !cfg) return fail(VS_ERR_INVALID, "null argument");
    if (channels != 3 && channels != 4) return fail(VS_ERR_INVALID, "image loss expects 3 or 4 channels");
    if (w == 0 || h == 0) return fail(VS_ERR_INVALID, "empty image");
    a = LossArgs{};
    a.img_w = w; a.img_h = h; a.channels = channels; a.pred = pred; a.gt = gt;
    a.l1_weight = cfg->l1_weight; a.ssim_weight = cfg->ssim_weight; a.alpha_weight_cfg = cfg->alpha_weight;
    a.composite = cfg->composite != 0; a.mask = cfg->mask != 0;
    a.bg[0] = cfg->bg[0]; a.bg[1] = cfg->bg[1]; a.bg[2] = cfg->bg[2];
    // channel_weights (lib.rs:1297-1300)
    const float pixels = (float)(h * w);
    a.rgb_weight = 1.0f / (3.0f * pixels);
    a.alpha_weight = cfg->alpha_weight / pixels;
    return VS_OK;
}
uint32_t loss_planes(const vs_loss_cfg* cfg, uint32_t channels) { return (cfg->alpha_weight > 0.0f && channels == 4) ? 4u : 3u; }
uint32_t loss_tiles(uint32_t w, uint32_t h) { return ((w + 15) / 16) * ((h + 15) / 16); }
} // namespace

extern "C" vs_status vs_image_loss_forward(vs_ctx* ctx, const float* pred, uint32_t channels, const uint32_t* gt_packed,
                                           uint32_t img_w, uint32_t img_h, const vs_loss_cfg* cfg, float* partials,
                                           float* coeffs, float* loss_map, float* total) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    LossArgs a;
    vs_status st = loss_args(pred, channels, gt_packed, img_w, img_h, cfg, a);
    if (st != VS_OK) return st;
    if (total && !partials) return fail(VS_ERR_INVALID, "the total needs the partials buffer");
    a.partials = partials; a.coeffs = coeffs; a.loss_map = loss_map; a.total = total;
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    StageTimer tm(ctx, ST_OTHER);
    VS_HIP(launch_loss_forward(a, ctx->stream), "image loss forward");
    return VS_OK;
}

extern "C" vs_status vs_image_loss_backward(vs_ctx* ctx, const float* pred, uint32_t channels, const uint32_t* gt_packed,
                                            uint32_t img_w, uint32_t img_h, const vs_loss_cfg* cfg,
                                            const float* dl_dpartials, uint32_t dl_count, const float* coeffs,
                                            float* dl_dpred) {
    if (!ctx) return fail(VS_ERR_INVALID, "ctx is null");
    LossArgs a;
    vs_status st = loss_args(pred, channels, gt_packed, img_w, img_h, cfg, a);
    if (st != VS_OK) return st;
    if (!dl_dpartials || !dl_dpred) return fail(VS_ERR_INVALID, "null argument");
    const uint32_t n_partials = loss_planes(cfg, channels) * loss_tiles(img_w, img_h);
    if (dl_count != 1 && dl_count != n_partials)
        return fail(VS_ERR_INVALID, "dl_dpartials must be [1] or [planes, tiles]");
    if (channels == 4 && ((uintptr_t)dl_dpred & 15u)) return fail(VS_ERR_INVALID, "dl_dpred must be 16-byte aligned");
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    hipStream_t s = ctx->stream;
    StageTimer tm(ctx, ST_OTHER);
    void* tmp = nullptr;
    if (!coeffs) {
        // No stored coefficients: the forward recomputes them (the reference's
        // recomputing backward blurs the same quantities in the same order).
        VS_HIP(lib_alloc(ctx, &tmp, (size_t)9 * img_w * img_h * 4, s), "hipMallocAsync(loss coefficients)");
        LossArgs f = a;
        f.coeffs = static_cast<float*>(tmp);
        hipError_t e = launch_loss_forward(f, s);
        if (e != hipSuccess) { lib_free(ctx, tmp); return hip_fail(e, "image loss coefficients"); }
        coeffs = static_cast<const float*>(tmp);
    }
    LossBwdArgs b{};
    b.fwd = a; b.img_w = img_w; b.img_h = img_h; b.channels = channels; b.pred = pred; b.gt = gt_packed;
    b.dl = dl_dpartials; b.coeffs = coeffs; b.dl_dpred = dl_dpred; b.rgb_weight = a.rgb_weight;
    b.alpha_weight = a.alpha_weight;
    hipError_t e = launch_loss_backward(b, dl_count == 1, s);
    if (tmp) lib_free(ctx, tmp);
    if (e != hipSuccess) return hip_fail(e, "image loss backward");
    return VS_OK;
}

// 1 / (3 x the pixels the L1 term averages over): the whole image, or the
// pixels inside the circle mask, counted with the kernels' own f32 test once
// per mask (a training loop passes the same mask every step).
static float l1_inv_count(vs_ctx* ctx, uint32_t w, uint32_t h, float mcx, float mcy, float mr) {
    uint64_t count = (uint64_t)w * h;
    if (mr > 0.0f) {
        const vs_ctx::MaskKey& k = ctx->l1_mask;
        if (!(k.w == w && k.h == h && k.cx == mcx && k.cy == mcy && k.r == mr)) {
            count = 0;
            for (uint32_t y = 0; y < h; ++y)
                for (uint32_t x = 0; x < w; ++x) {
                    const float dx = (float)x + 0.5f - mcx, dy = (float)y + 0.5f - mcy;
                    if (dx * dx + dy * dy <= mr * mr) ++count;
                }
            ctx->l1_mask = vs_ctx::MaskKey{w, h, mcx, mcy, mr};
            ctx->l1_mask_count = count;
        }
        count = ctx->l1_mask_count;
    }
    return count ? 1.0f / (3.0f * (float)count) : 0.0f;
}

static vs_status l1_cotangent(vs_ctx* ctx, const float* pred, uint32_t channels, const void* gt, bool packed, uint32_t w,
                              uint32_t h, float mcx, float mcy, float mr, float* v_out) {
    if (!ctx || !pred || !gt || !v_out) return fail(VS_ERR_INVALID, "null argument");
    if (channels < 3) return fail(VS_ERR_INVALID, "prediction needs at least 3 channels");
    const float inv = l1_inv_count(ctx, w, h, mcx, mcy, mr);
    VS_HIP(hipSetDevice(ctx->device), "hipSetDevice");
    VS_HIP(launch_l1_cotangent(pred, channels, gt, packed, w, h, mcx, mcy, mr, inv, v_out, ctx->stream), "l1 cotangent");
    return VS_OK;
}

extern "C" vs_status vs_l1_cotangent(vs_ctx* ctx, const float* pred, uint32_t channels, const float* gt, uint32_t w,
                                     uint32_t h, float mcx, float mcy, float mr, float* v_out) {
    return l1_cotangent(ctx, pred, channels, gt, false, w, h, mcx, mcy, mr, v_out);
}

extern "C" vs_status vs_l1_cotangent_packed(vs_ctx* ctx, const float* pred, uint32_t channels, const uint32_t* gt_packed,
                                            uint32_t w, uint32_t h, float mcx, float mcy, float mr, float* v_out) {
    return l1_cotangent(ctx, pred, channels, gt_packed, true, w, h, mcx, mcy, mr, v_out);
}
