// valu_rates.hip -- issue rate of each VALU instruction class on this GPU
// (wave64 instructions per second across the chip), the calibration behind
// the instruction-issue ceiling bench.py reports for the compositing kernels.
//
// Each kernel runs 2048 x 16-unrolled iterations of 8 independent chains of one
// instruction per lane (register operands only), 8 waves per SIMD on every CU,
// and is timed with HIP events over 5 launches.  Classes whose rate differs
// are the point: FP32 add/mul/fma, max, compare and select issue in 4 cycles
// per wave64 instruction, integer add / logic, moves and conversions in 2,
// transcendentals in 8.
#include <hip/hip_runtime.h>
#include <cstdint>
#include <cstdio>

namespace {

constexpr int ITERS = 2048;
constexpr int BLOCK = 256;

#define CH8(OP) OP(x0) OP(x1) OP(x2) OP(x3) OP(x4) OP(x5) OP(x6) OP(x7)
#define FINISH out[blockIdx.x * BLOCK + threadIdx.x] = ((x0 + x1) + (x2 + x3)) + ((x4 + x5) + (x6 + x7)) + b
#define INIT float x0 = threadIdx.x, x1 = x0 + 1, x2 = x0 + 2, x3 = x0 + 3, x4 = x0 + 4, x5 = x0 + 5, x6 = x0 + 6, x7 = x0 + 7

__global__ void __launch_bounds__(BLOCK) k_fma(float* out, float a, float b) {
    INIT;
#define OP(x) x = __builtin_fmaf(x, a, b);
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { CH8(OP) }
#undef OP
    FINISH;
}
__global__ void __launch_bounds__(BLOCK) k_add(float* out, float a, float b) {
    INIT;
#define OP(x) x = x + a;
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { CH8(OP) }
#undef OP
    FINISH;
}
__global__ void __launch_bounds__(BLOCK) k_exp(float* out, float a, float b) {
    INIT;
    x0 *= 1e-3f; x1 *= 1e-3f; x2 *= 1e-3f; x3 *= 1e-3f; x4 *= 1e-3f; x5 *= 1e-3f; x6 *= 1e-3f; x7 *= 1e-3f;
#define OP(x) x = __builtin_amdgcn_exp2f(x);
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { CH8(OP) }
#undef OP
    FINISH + a;
}
__global__ void __launch_bounds__(BLOCK) k_int(float* out, float a, float b) {
    uint32_t y0 = threadIdx.x, y1 = y0 * 3, y2 = y0 * 5, y3 = y0 * 7, y4 = y0 * 11, y5 = y0 * 13, y6 = y0 * 17, y7 = y0 * 19;
    const uint32_t k = __float_as_uint(a);
#define OP(y) asm volatile("v_add_u32 %0, %0, %1" : "+v"(y) : "v"(k));
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { OP(y0) OP(y1) OP(y2) OP(y3) OP(y4) OP(y5) OP(y6) OP(y7) }
#undef OP
    out[blockIdx.x * BLOCK + threadIdx.x] = (float)(((y0 + y1) + (y2 + y3)) + ((y4 + y5) + (y6 + y7))) + b;
}
__global__ void __launch_bounds__(BLOCK) k_max(float* out, float a, float b) {
    INIT;
#define OP(x) asm volatile("v_max_f32 %0, %0, %1" : "+v"(x) : "v"(a));
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { CH8(OP) }
#undef OP
    FINISH;
}
__global__ void __launch_bounds__(BLOCK) k_cndmask(float* out, float a, float b) {
    INIT;
    const uint64_t m = __ballot(threadIdx.x & 1);
#define OP(x) asm volatile("v_cndmask_b32_e64 %0, %0, %1, %2" : "+v"(x) : "v"(a), "s"(m));
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { CH8(OP) }
#undef OP
    FINISH;
}
__global__ void __launch_bounds__(BLOCK) k_mov(float* out, float a, float b) {
    INIT;
#define OP(x) asm volatile("v_mov_b32 %0, %1" : "=v"(x) : "v"(a));
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { CH8(OP) }
#undef OP
    FINISH;
}
__global__ void __launch_bounds__(BLOCK) k_cvt(float* out, float a, float b) {
    INIT;
#define OP(x) asm volatile("v_cvt_f32_i32 %0, %0" : "+v"(x));
#pragma unroll 16
    for (int i = 0; i < ITERS; ++i) { CH8(OP) }
#undef OP
    FINISH + a;
}

typedef void (*Kern)(float*, float, float);

}  // namespace

int main() {
    int dev = 0;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) { std::printf("no GPU\n"); return 1; }
    const int blocks = prop.multiProcessorCount * 8;     // 8 workgroups of 4 waves per CU: 8 waves per SIMD
    const double waves = blocks * (BLOCK / 64.0);
    float* out = nullptr;
    if (hipMalloc(&out, (size_t)blocks * BLOCK * sizeof(float)) != hipSuccess) return 1;
    hipEvent_t e0, e1;
    if (hipEventCreate(&e0) != hipSuccess || hipEventCreate(&e1) != hipSuccess) return 1;
    struct { const char* name; Kern k; } ks[] = {
        {"fp32 fma (v_fma_f32)", k_fma}, {"fp32 add (v_add_f32)", k_add}, {"max (v_max_f32)", k_max},
        {"select (v_cndmask_b32)", k_cndmask}, {"int32 add (v_add_u32)", k_int}, {"move (v_mov_b32)", k_mov},
        {"convert (v_cvt_f32_i32)", k_cvt}, {"transcendental (v_exp_f32)", k_exp}};
    const double clock_hz = prop.clockRate * 1e3;
    const double simds = prop.multiProcessorCount * 4.0;
    std::printf("%d CUs, %.0f MHz; %d waves per launch\n", prop.multiProcessorCount, clock_hz / 1e6, (int)waves);
    std::printf("| class | G wave-instr/s | cycles per wave64 instruction |\n|---|---|---|\n");
    for (auto& k : ks) {
        k.k<<<blocks, BLOCK>>>(out, 1.0000001f, 0.5f);
        if (hipEventRecord(e0) != hipSuccess) return 1;
        for (int r = 0; r < 5; ++r) k.k<<<blocks, BLOCK>>>(out, 1.0000001f, 0.5f);
        if (hipEventRecord(e1) != hipSuccess || hipEventSynchronize(e1) != hipSuccess) return 1;
        float ms = 0.0f;
        if (hipEventElapsedTime(&ms, e0, e1) != hipSuccess) return 1;
        const double insts = waves * ITERS * 8.0;
        const double rate = insts / (ms / 5 * 1e-3);
        std::printf("| %s | %.0f | %.2f |\n", k.name, rate / 1e9, simds * clock_hz / rate);
    }
    if (hipGetLastError() != hipSuccess) return 1;
    hipFree(out);
    return 0;
}
