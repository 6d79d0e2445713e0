// k_sort.hip -- stable LSD radix sort of (key, u32 value) pairs, 8-bit digits,
// u32 or u64 keys.
//
// Replaces crates/splat-train-sort (radix_argsort*, lib.rs:15-189;
// kernels.rs:35-341).  One pass per digit:
//   upsweep  -- per 2048-key block, an LDS digit histogram written digit-major
//               into a [256 x blocks] table;
//   scan     -- exclusive scan of the table (k_scan.hip) = each block's
//               first output slot per digit;
//   scatter  -- each wavefront ranks its keys in input order with ballot-based
//               digit matching (8 ballots per step, no atomics), the block
//               reorders keys by digit in LDS, and the reordered tile is
//               written out so equal digits land in consecutive addresses.
// Ranking in (wave, step, lane) order with waves owning consecutive key
// ranges keeps every pass stable, so the sort is stable.
#include "vs_internal.h"

namespace vs {

constexpr int SORT_BLOCK = 256;
constexpr int SORT_ITEMS = 8;
constexpr uint32_t SORT_TILE = SORT_BLOCK * SORT_ITEMS;   // 2048 keys per block
constexpr int SORT_WAVES = SORT_BLOCK / 64;
constexpr uint32_t KEYS_PER_WAVE = 64 * SORT_ITEMS;

template <typename K>
__device__ __forceinline__ uint32_t digit_of(K k, uint32_t shift) { return (uint32_t)(k >> shift) & 0xFFu; }

template <typename K>
__global__ void __launch_bounds__(SORT_BLOCK) sort_upsweep_kernel(const K* __restrict__ keys, uint32_t n_cap,
                                                                  const uint32_t* __restrict__ n_dev, uint32_t shift,
                                                                  uint32_t* __restrict__ table, uint32_t nblocks) {
    __shared__ uint32_t hist[SORT_WAVES][256];
    const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
    const uint32_t wave = threadIdx.x >> 6;
    for (uint32_t i = threadIdx.x; i < SORT_WAVES * 256; i += SORT_BLOCK) (&hist[0][0])[i] = 0;
    __syncthreads();
    const uint32_t base = blockIdx.x * SORT_TILE;
#pragma unroll
    for (int i = 0; i < SORT_ITEMS; ++i) {
        const uint32_t idx = base + i * SORT_BLOCK + threadIdx.x;
        if (idx < n) atomicAdd(&hist[wave][digit_of(keys[idx], shift)], 1u);
    }
    __syncthreads();
    const uint32_t d = threadIdx.x;
    uint32_t c = 0;
#pragma unroll
    for (int w = 0; w < SORT_WAVES; ++w) c += hist[w][d];
    table[(size_t)d * nblocks + blockIdx.x] = c;
}

template <typename K>
__global__ void __launch_bounds__(SORT_BLOCK) sort_scatter_kernel(const K* __restrict__ keys_in, const uint32_t* __restrict__ vals_in,
                                                                  K* __restrict__ keys_out, uint32_t* __restrict__ vals_out,
                                                                  uint32_t n_cap, const uint32_t* __restrict__ n_dev, uint32_t shift,
                                                                  const uint32_t* __restrict__ offsets, uint32_t nblocks) {
    __shared__ uint32_t wave_hist[SORT_WAVES][256];
    __shared__ uint32_t digit_start[256];
    __shared__ uint32_t s_tot[8];
    __shared__ K s_keys[SORT_TILE];
    __shared__ uint32_t s_vals[SORT_TILE];

    const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t base = blockIdx.x * SORT_TILE;
    if (base >= n) return;   // uniform per block
    for (uint32_t i = threadIdx.x; i < SORT_WAVES * 256; i += SORT_BLOCK) (&wave_hist[0][0])[i] = 0;
    __syncthreads();

    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    K key[SORT_ITEMS];
    uint32_t val[SORT_ITEMS], dig[SORT_ITEMS], rank[SORT_ITEMS];
    const uint32_t wbase = base + wave * KEYS_PER_WAVE;
#pragma unroll
    for (int s = 0; s < SORT_ITEMS; ++s) {
        const uint32_t idx = wbase + s * 64 + lane;
        const bool valid = idx < n;
        key[s] = valid ? keys_in[idx] : (K)0;
        val[s] = valid ? vals_in[idx] : 0u;
        const uint32_t d = digit_of(key[s], shift);
        dig[s] = valid ? d : 256u;
        uint64_t peers = __ballot(valid);
#pragma unroll
        for (int b = 0; b < 8; ++b) {
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
    // Per-digit totals, wave offsets and the block's digit starts.
    {
        const uint32_t d = threadIdx.x;
        uint32_t run = 0;
#pragma unroll
        for (int w = 0; w < SORT_WAVES; ++w) {
            const uint32_t c = wave_hist[w][d];
            wave_hist[w][d] = run;     // becomes the wave's exclusive offset within digit d
            run += c;
        }
        // exclusive scan of run over the 256 digits
        uint32_t incl = run;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(incl, o);
            if ((int)lane >= o) incl += t;
        }
        if (lane == 63) s_tot[wave] = incl;
        __syncthreads();
        uint32_t wo = 0;
        for (uint32_t w = 0; w < wave; ++w) wo += s_tot[w];
        digit_start[d] = wo + incl - run;
    }
    __syncthreads();
#pragma unroll
    for (int s = 0; s < SORT_ITEMS; ++s) {
        if (dig[s] < 256u) {
            const uint32_t pos = digit_start[dig[s]] + wave_hist[wave][dig[s]] + rank[s];
            s_keys[pos] = key[s];
            s_vals[pos] = val[s];
        }
    }
    __syncthreads();
    const uint32_t count = min(SORT_TILE, n - base);
    for (uint32_t i = threadIdx.x; i < count; i += SORT_BLOCK) {
        const K k = s_keys[i];
        const uint32_t d = digit_of(k, shift);
        const uint32_t gpos = offsets[(size_t)d * nblocks + blockIdx.x] + (i - digit_start[d]);
        if (gpos < n) {   // always true for a consistent table; keeps a bad rank from writing out of bounds
            keys_out[gpos] = k;
            vals_out[gpos] = s_vals[i];
        }
    }
}

static size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }

size_t sort_tmp_bytes(uint64_t n, bool key64) {
    const uint64_t nblocks = (n + SORT_TILE - 1) / SORT_TILE;
    const size_t ks = key64 ? 8 : 4;
    size_t b = 0;
    b += align_up(n * ks, 256);                 // ping-pong keys
    b += align_up(n * 4, 256);                  // ping-pong values
    b += align_up(nblocks * 256 * 4, 256);      // digit table
    b += align_up(scan_tmp_words(nblocks * 256) * 4, 256);
    return b + 256;
}

template <typename K>
static hipError_t sort_impl(const K* keys_in, const uint32_t* vals_in, K* keys_out, uint32_t* vals_out, uint32_t n,
                            const uint32_t* n_dev, uint32_t first_bit, uint32_t end_bit, void* tmp, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint32_t bits = end_bit > first_bit ? end_bit - first_bit : 0;
    const uint32_t passes = (bits + 7) / 8;
    if (passes == 0) {
        hipError_t e = hipMemcpyAsync(keys_out, keys_in, (size_t)n * sizeof(K), hipMemcpyDeviceToDevice, s);
        if (e != hipSuccess) return e;
        return hipMemcpyAsync(vals_out, vals_in, (size_t)n * 4, hipMemcpyDeviceToDevice, s);
    }
    const uint32_t nblocks = (n + SORT_TILE - 1) / SORT_TILE;
    char* p = reinterpret_cast<char*>(align_up(reinterpret_cast<uintptr_t>(tmp), 256));
    K* tk = reinterpret_cast<K*>(p); p += align_up((size_t)n * sizeof(K), 256);
    uint32_t* tv = reinterpret_cast<uint32_t*>(p); p += align_up((size_t)n * 4, 256);
    uint32_t* table = reinterpret_cast<uint32_t*>(p); p += align_up((size_t)nblocks * 256 * 4, 256);
    uint32_t* stmp = reinterpret_cast<uint32_t*>(p);
    const K* src_k = keys_in;
    const uint32_t* src_v = vals_in;
    for (uint32_t pass = 0; pass < passes; ++pass) {
        const bool to_out = ((passes - 1 - pass) % 2) == 0;
        K* dk = to_out ? keys_out : tk;
        uint32_t* dv = to_out ? vals_out : tv;
        const uint32_t shift = first_bit + 8 * pass;
        sort_upsweep_kernel<K><<<nblocks, SORT_BLOCK, 0, s>>>(src_k, n, n_dev, shift, table, nblocks);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        e = scan_u32(table, table, (uint64_t)nblocks * 256, false, stmp, nullptr, s);
        if (e != hipSuccess) return e;
        sort_scatter_kernel<K><<<nblocks, SORT_BLOCK, 0, s>>>(src_k, src_v, dk, dv, n, n_dev, shift, table, nblocks);
        e = hipGetLastError();
        if (e != hipSuccess) return e;
        src_k = dk;
        src_v = dv;
    }
    return hipSuccess;
}

hipError_t radix_sort_pairs(const void* keys_in, const uint32_t* vals_in, void* keys_out, uint32_t* vals_out,
                            uint32_t n, const uint32_t* n_dev, bool key64, uint32_t first_bit, uint32_t end_bit,
                            void* tmp, hipStream_t s) {
    if (key64)
        return sort_impl<uint64_t>(static_cast<const uint64_t*>(keys_in), vals_in, static_cast<uint64_t*>(keys_out),
                                   vals_out, n, n_dev, first_bit, end_bit, tmp, s);
    return sort_impl<uint32_t>(static_cast<const uint32_t*>(keys_in), vals_in, static_cast<uint32_t*>(keys_out),
                               vals_out, n, n_dev, first_bit, end_bit, tmp, s);
}

} // namespace vs
