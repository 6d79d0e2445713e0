// k_scan.hip -- device-wide u32 prefix sums.
//
// Replaces crates/splat-train-scan (prefix_sum, lib.rs:24-83; scan_in_place,
// lib.rs:85-96).  Reduce-then-scan over 4096-element blocks: a reduce kernel
// writes block totals, one workgroup scans the totals, and a scan kernel
// re-reads its block through LDS (coalesced loads, blocked per-thread
// sequential scan, wave shuffles) and adds the block offset.
#include "vs_internal.h"

namespace vs {

constexpr int SCAN_BLOCK = 256;
constexpr int SCAN_ITEMS = 16;
constexpr uint32_t SCAN_TILE = SCAN_BLOCK * SCAN_ITEMS;   // 4096
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
