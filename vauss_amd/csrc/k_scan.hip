// k_scan.hip -- device-wide u32 prefix sums.
//
// Replaces crates/splat-train-scan (prefix_sum, lib.rs:24-83; scan_in_place,
// lib.rs:85-96).  Reduce-then-scan over 1024-element blocks: a reduce kernel
// writes block totals, one workgroup scans the totals, and a scan kernel
// re-reads its block through LDS (coalesced loads, blocked per-thread
// sequential scan, wave shuffles) and adds the block offset.
#include "vs_internal.h"

namespace vs {

constexpr int SCAN_BLOCK = 256;
constexpr int SCAN_ITEMS = 4;
constexpr uint32_t SCAN_TILE = SCAN_BLOCK * SCAN_ITEMS;   // 1024: over 600 blocks for 616k elements
constexpr int SINGLE_BLOCK = 1024;

__device__ __forceinline__ uint32_t wave_incl_scan(uint32_t v, uint32_t lane) {
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(v, o);
        if ((int)lane >= o) v += t;
    }
    return v;
}

// Block-wide exclusive scan of one value per thread; returns the block total.
template <int NT>
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t& excl, uint32_t* s_w) {
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t incl = wave_incl_scan(v, lane);
    if (lane == 63) s_w[wave] = incl;
    __syncthreads();
    if (threadIdx.x < 64) {
        const uint32_t wv = (threadIdx.x < NT / 64) ? s_w[threadIdx.x] : 0u;
        const uint32_t wi = wave_incl_scan(wv, threadIdx.x);
        if (threadIdx.x < NT / 64) s_w[threadIdx.x + 16] = wi - wv;   // exclusive wave offsets
        if (threadIdx.x == NT / 64 - 1) s_w[32] = wi;                 // block total
    }
    __syncthreads();
    excl = s_w[16 + wave] + incl - v;
    const uint32_t total = s_w[32];
    __syncthreads();
    return total;
}

// With a permutation `perm`, element i of the scanned sequence is in[perm[i]]
// and its result is written to out[perm[i]] (out[i] with `in_order`, and then
// also to out2[perm[i]] when out2 is given).  Entries at or past `perm_bound`
// (only a corrupt permutation holds them) read as 0 and are not scattered, so
// a bad permutation cannot index out of bounds.
__device__ __forceinline__ uint32_t scan_load(const uint32_t* __restrict__ in, const uint32_t* __restrict__ perm,
                                              uint64_t idx, uint32_t perm_bound) {
    if (!perm) return in[idx];
    const uint32_t j = perm[idx];
    return j < perm_bound ? in[j] : 0u;
}

// Element count: n, or min(*n_dev, n) when a device count is given.
__device__ __forceinline__ uint64_t scan_count(uint64_t n, const uint32_t* __restrict__ n_dev) {
    return n_dev ? (*n_dev < n ? (uint64_t)*n_dev : n) : n;
}

__global__ void __launch_bounds__(SCAN_BLOCK) scan_reduce_kernel(const uint32_t* __restrict__ in, uint64_t n_cap,
                                                                 uint32_t* __restrict__ sums,
                                                                 const uint32_t* __restrict__ perm,
                                                                 const uint32_t* __restrict__ n_dev, uint32_t perm_bound) {
    const uint64_t n = scan_count(n_cap, n_dev);
    const uint64_t base = (uint64_t)blockIdx.x * SCAN_TILE;
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) {
        const uint64_t idx = base + (uint64_t)i * SCAN_BLOCK + threadIdx.x;
        if (idx < n) acc += scan_load(in, perm, idx, perm_bound);
    }
    __shared__ uint32_t s_w[48];
    uint32_t excl;
    const uint32_t total = block_excl_scan<SCAN_BLOCK>(acc, excl, s_w);
    if (threadIdx.x == 0) sums[blockIdx.x] = total;
}

__global__ void __launch_bounds__(SCAN_BLOCK) scan_block_kernel(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                                uint64_t n_cap, const uint32_t* __restrict__ offsets,
                                                                int inclusive, const uint32_t* __restrict__ perm,
                                                                const uint32_t* __restrict__ n_dev, uint32_t perm_bound,
                                                                int in_order, uint32_t* __restrict__ out2) {
    const uint64_t n = scan_count(n_cap, n_dev);
    __shared__ uint32_t s_data[SCAN_TILE];
    __shared__ uint32_t s_w[48];
    const uint64_t base = (uint64_t)blockIdx.x * SCAN_TILE;
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) {
        const uint32_t li = i * SCAN_BLOCK + threadIdx.x;
        const uint64_t idx = base + li;
        s_data[li] = (idx < n) ? scan_load(in, perm, idx, perm_bound) : 0u;
    }
    __syncthreads();
    uint32_t v[SCAN_ITEMS];
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) { v[i] = s_data[threadIdx.x * SCAN_ITEMS + i]; acc += v[i]; }
    uint32_t excl;
    block_excl_scan<SCAN_BLOCK>(acc, excl, s_w);
    uint32_t run = excl + (offsets ? offsets[blockIdx.x] : 0u);
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) {
        const uint32_t before = run;
        run += v[i];
        s_data[threadIdx.x * SCAN_ITEMS + i] = inclusive ? run : before;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) {
        const uint32_t li = i * SCAN_BLOCK + threadIdx.x;
        const uint64_t idx = base + li;
        if (idx < n) {
            const uint64_t j = (perm && !in_order) ? (uint64_t)perm[idx] : idx;
            if (!perm || in_order || j < perm_bound) out[j] = s_data[li];
            if (out2) {
                const uint32_t k = perm[idx];
                if (k < perm_bound) out2[k] = s_data[li];
            }
        }
    }
}

// One workgroup walks the array in chunks of 1024, carrying the running sum.
__global__ void __launch_bounds__(SINGLE_BLOCK) scan_single_kernel(uint32_t* __restrict__ data, uint32_t n, int inclusive,
                                                                   uint32_t* __restrict__ total_out) {
    __shared__ uint32_t s_w[48];
    uint32_t carry = 0;
    for (uint32_t start = 0; start < n; start += SINGLE_BLOCK) {
        const uint32_t idx = start + threadIdx.x;
        const uint32_t v = (idx < n) ? data[idx] : 0u;
        uint32_t excl;
        const uint32_t total = block_excl_scan<SINGLE_BLOCK>(v, excl, s_w);
        if (idx < n) data[idx] = carry + excl + (inclusive ? v : 0u);
        carry += total;
    }
    if (total_out && threadIdx.x == 0) *total_out = carry;
}

// Single-pass scan with decoupled look-back: each block scans its tile,
// publishes its total, and finds the sum of every earlier tile by reading
// its predecessors' published totals 64 at a time (one per lane of the first
// wavefront) back to the nearest full prefix.  A block only waits on
// lower-indexed blocks, which are dispatched first and publish before they
// wait, so the chain drains; a wait past `spin_limit` polls sets *err and
// proceeds (the result is then wrong and reported).  Status words are 64-bit:
// two flag bits over a 62-bit sum.
constexpr uint64_t LB_AGG = 1ull << 62, LB_PREFIX = 2ull << 62, LB_VAL = (1ull << 62) - 1ull;

__global__ void __launch_bounds__(SCAN_BLOCK) scan_lookback_kernel(const uint32_t* __restrict__ in, uint32_t* __restrict__ out,
                                                                   uint64_t n_cap, const uint32_t* __restrict__ perm,
                                                                   const uint32_t* __restrict__ n_dev, uint32_t perm_bound,
                                                                   uint32_t* __restrict__ out2, uint32_t out2_above,
                                                                   unsigned long long* status, uint32_t* err,
                                                                   uint32_t spin_limit, int write_end) {
    const uint64_t n = scan_count(n_cap, n_dev);
    const uint64_t base = (uint64_t)blockIdx.x * SCAN_TILE;
    if (base >= n) return;   // uniform: no later block has elements either
    __shared__ uint32_t s_data[SCAN_TILE];
    __shared__ uint32_t s_w[48];
    __shared__ unsigned long long s_prefix;
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) {
        const uint32_t li = i * SCAN_BLOCK + threadIdx.x;
        const uint64_t idx = base + li;
        s_data[li] = (idx < n) ? scan_load(in, perm, idx, perm_bound) : 0u;
    }
    __syncthreads();
    uint32_t v[SCAN_ITEMS];
    uint32_t acc = 0;
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) { v[i] = s_data[threadIdx.x * SCAN_ITEMS + i]; acc += v[i]; }
    uint32_t excl;
    const uint32_t total = block_excl_scan<SCAN_BLOCK>(acc, excl, s_w);
    if (threadIdx.x < 64) {
        const uint32_t lane = threadIdx.x;
        const int b = (int)blockIdx.x;
        if (lane == 0)
            __hip_atomic_store(&status[b], (b == 0 ? LB_PREFIX : LB_AGG) | (unsigned long long)total, __ATOMIC_RELAXED,
                               __HIP_MEMORY_SCOPE_AGENT);
        unsigned long long prefix = 0;
        if (b > 0) {
            int top = b - 1;           // the window is [top - 63, top], lane i reads top - i
            uint32_t spins = 0;
            while (true) {
                const int j = top - (int)lane;
                const unsigned long long st =
                    j >= 0 ? __hip_atomic_load(&status[j], __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : LB_PREFIX;
                const unsigned long long flag = st & ~LB_VAL;
                const uint64_t pref = __ballot(flag == LB_PREFIX), unpub = __ballot(flag == 0ull);
                const uint32_t last = pref ? (uint32_t)__builtin_ctzll(pref) : 63u;   // the lanes this window needs
                const uint64_t need = last == 63u ? ~0ull : ((2ull << last) - 1ull);
                if (unpub & need) {   // a needed predecessor has not published yet
                    if (++spins > spin_limit) { if (lane == 0) atomicOr(err, 1u); break; }
                    __builtin_amdgcn_s_sleep(1);
                    continue;
                }
                unsigned long long part = ((need >> lane) & 1ull) ? (st & LB_VAL) : 0ull;
#pragma unroll
                for (int o = 32; o > 0; o >>= 1) part += __shfl_xor(part, o);
                prefix += part;
                if (pref) break;
                top -= 64;
            }
            if (lane == 0)
                __hip_atomic_store(&status[b], LB_PREFIX | (prefix + total), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        }
        if (lane == 0) s_prefix = prefix;
    }
    __syncthreads();
    uint32_t run = excl + (uint32_t)s_prefix;
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) {
        s_data[threadIdx.x * SCAN_ITEMS + i] = run;
        // the scattered copy, for the few elements above the threshold (an
        // element past n loaded as 0, which is never above it)
        if (out2 && v[i] > out2_above) {
            const uint32_t k = perm[base + (uint64_t)threadIdx.x * SCAN_ITEMS + i];
            if (k < perm_bound) out2[k] = run;
        }
        run += v[i];
    }
    // out[n]: the total, from the thread holding element n - 1 (the elements
    // past it loaded as zero)
    if (write_end) {
        const uint64_t first = base + (uint64_t)threadIdx.x * SCAN_ITEMS;
        if (first < n && n <= first + SCAN_ITEMS) out[n] = run;
    }
    __syncthreads();
#pragma unroll
    for (int i = 0; i < SCAN_ITEMS; ++i) {
        const uint32_t li = i * SCAN_BLOCK + threadIdx.x;
        const uint64_t idx = base + li;
        if (idx < n) out[idx] = s_data[li];
    }
}

uint64_t scan_lookback_status_words(uint64_t n) { return 2 * ((n + SCAN_TILE - 1) / SCAN_TILE); }

hipError_t scan_u32_lookback(const uint32_t* in, uint32_t* out, uint64_t n, uint32_t* status, uint32_t* err,
                             hipStream_t s, uint32_t spin_limit, const uint32_t* perm, const uint32_t* n_dev,
                             uint32_t perm_bound, uint32_t* out_scattered, bool write_end, uint32_t scatter_above) {
    if (n == 0) return hipSuccess;
    const uint64_t blocks = (n + SCAN_TILE - 1) / SCAN_TILE;
    scan_lookback_kernel<<<(uint32_t)blocks, SCAN_BLOCK, 0, s>>>(in, out, n, perm, n_dev, perm_bound,
                                                                 perm ? out_scattered : nullptr, scatter_above,
                                                                 reinterpret_cast<unsigned long long*>(status), err,
                                                                 spin_limit, write_end ? 1 : 0);
    return hipGetLastError();
}

size_t scan_tmp_words(uint64_t n) {
    const uint64_t blocks = (n + SCAN_TILE - 1) / SCAN_TILE;
    return (size_t)(blocks ? blocks : 1) + 64;
}

hipError_t scan_single_block(uint32_t* data, uint32_t n, bool inclusive, uint32_t* total_out, hipStream_t s) {
    if (n == 0 && !total_out) return hipSuccess;
    scan_single_kernel<<<1, SINGLE_BLOCK, 0, s>>>(data, n, inclusive ? 1 : 0, total_out);
    return hipGetLastError();
}

hipError_t scan_u32(const uint32_t* in, uint32_t* out, uint64_t n, bool inclusive, uint32_t* tmp,
                    uint32_t* total_out, hipStream_t s, const uint32_t* perm, const uint32_t* n_dev,
                    uint32_t perm_bound, bool out_in_order, uint32_t* out_scattered) {
    const int in_order = out_in_order ? 1 : 0;
    uint32_t* out2 = (perm && out_in_order) ? out_scattered : nullptr;
    if (n == 0) {
        if (total_out) return scan_single_block(tmp, 0, false, total_out, s);
        return hipSuccess;
    }
    const uint64_t blocks = (n + SCAN_TILE - 1) / SCAN_TILE;
    if (blocks == 1) {
        scan_block_kernel<<<1, SCAN_BLOCK, 0, s>>>(in, out, n, nullptr, inclusive ? 1 : 0, perm, n_dev, perm_bound, in_order, out2);
        if (total_out) {
            scan_reduce_kernel<<<1, SCAN_BLOCK, 0, s>>>(in, n, tmp, perm, n_dev, perm_bound);
            hipError_t e = hipGetLastError();
            if (e != hipSuccess) return e;
            return scan_single_block(tmp, 1, true, total_out, s);
        }
        return hipGetLastError();
    }
    scan_reduce_kernel<<<(uint32_t)blocks, SCAN_BLOCK, 0, s>>>(in, n, tmp, perm, n_dev, perm_bound);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    e = scan_single_block(tmp, (uint32_t)blocks, false, total_out, s);
    if (e != hipSuccess) return e;
    scan_block_kernel<<<(uint32_t)blocks, SCAN_BLOCK, 0, s>>>(in, out, n, tmp, inclusive ? 1 : 0, perm, n_dev, perm_bound, in_order, out2);
    return hipGetLastError();
}

} // namespace vs
