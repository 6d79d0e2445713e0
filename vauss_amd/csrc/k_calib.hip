// k_calib.hip -- streaming kernels of known traffic for calibrating the
// memory counters (rocprofv3 --pmc) that bench.py turns into HBM bytes per
// kernel.  No reference counterpart: a measurement aid.
//
// Each kernel touches every byte of its buffer exactly once, in contiguous
// per-wavefront runs (grid-stride over W-byte words, W = 16 or 4), so its
// memory traffic is the buffer size: a read kernel's L2->memory read requests
// and a write kernel's write requests, at the request sizes fully coalesced
// streaming produces.  The read kernels fold every word into one u32 per
// block (so no load is dead) written to `sink` [grid].
#include "vs_internal.h"

namespace vs {

constexpr uint32_t CALIB_BLOCK = 256;
constexpr uint32_t CALIB_GRID = 2048;

template <int W>
__global__ void __launch_bounds__(CALIB_BLOCK) stream_read_kernel(const uint32_t* __restrict__ buf, uint64_t words,
                                                                  uint32_t* __restrict__ sink) {
    constexpr int U = W / 4;   // u32 per word
    __shared__ uint32_t s_x[CALIB_BLOCK / 64];
    uint32_t x = 0;
    const uint64_t stride = (uint64_t)gridDim.x * CALIB_BLOCK;
    for (uint64_t i = (uint64_t)blockIdx.x * CALIB_BLOCK + threadIdx.x; i < words; i += stride) {
        if constexpr (U == 4) {
            const uint4 v = reinterpret_cast<const uint4*>(buf)[i];
            x ^= v.x ^ v.y ^ v.z ^ v.w;
        } else {
            x ^= buf[i];
        }
    }
    for (int o = 32; o > 0; o >>= 1) x ^= __shfl_xor(x, o);
    if ((threadIdx.x & 63) == 0) s_x[threadIdx.x >> 6] = x;
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
        for (uint32_t w = 0; w < CALIB_BLOCK / 64; ++w) t ^= s_x[w];
        sink[blockIdx.x] = t;
    }
}

template <int W>
__global__ void __launch_bounds__(CALIB_BLOCK) stream_write_kernel(uint32_t* __restrict__ buf, uint64_t words,
                                                                   uint32_t value) {
    constexpr int U = W / 4;
    const uint64_t stride = (uint64_t)gridDim.x * CALIB_BLOCK;
    for (uint64_t i = (uint64_t)blockIdx.x * CALIB_BLOCK + threadIdx.x; i < words; i += stride) {
        if constexpr (U == 4) {
            reinterpret_cast<uint4*>(buf)[i] = make_uint4(value, value ^ 1u, value ^ 2u, value ^ 3u);
        } else {
            buf[i] = value;
        }
    }
}

uint32_t calib_sink_words() { return CALIB_GRID; }

hipError_t launch_stream_probe(void* buf, uint64_t bytes, int mode, uint32_t* sink, hipStream_t s) {
    const int width = (mode & 2) ? 4 : 16;
    const uint64_t words = bytes / (uint64_t)width;
    if (words == 0) return hipSuccess;
    const uint32_t grid = (uint32_t)std::min<uint64_t>(CALIB_GRID, (words + CALIB_BLOCK - 1) / CALIB_BLOCK);
    uint32_t* b = static_cast<uint32_t*>(buf);
    if ((mode & 1) == 0) {
        if (width == 16) stream_read_kernel<16><<<grid, CALIB_BLOCK, 0, s>>>(b, words, sink);
        else stream_read_kernel<4><<<grid, CALIB_BLOCK, 0, s>>>(b, words, sink);
    } else {
        if (width == 16) stream_write_kernel<16><<<grid, CALIB_BLOCK, 0, s>>>(b, words, 0x5EEDu);
        else stream_write_kernel<4><<<grid, CALIB_BLOCK, 0, s>>>(b, words, 0x5EEDu);
    }
    return hipGetLastError();
}

} // namespace vs
