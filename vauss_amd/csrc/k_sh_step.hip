// k_sh_step.hip -- the trainer's SH-coefficient step: lazy Adam on f16
// coefficients whose first moment is stored block-scaled in 8 bits, with the
// coefficient gradient rebuilt from the fused update's colour gradient and
// view direction; plus that moment's codec (encode, decode, zero rows).
//
// Restates crates/splat-train/src/optim.rs:391-498 (step_sh_color,
// step_quantized) and crates/splat-train/src/quant_kernels.rs:582-777
// (step_kernel_w4, sh_basis, stochastic_half), 438-498 (pack_block, unpack,
// encode/decode) and 911-925 (zero_moment_rows_kernel).
//
// Moment layout: the flat [N*K*3] values in blocks of 128; block b has one
// f32 scale (absmax / 127) and 32 u32 words of four biased 8-bit codes,
// value 4w+j in byte j of word w.  gfx950 mapping: one wave64 owns two
// blocks, each 32-lane half one block and each lane one word (four
// consecutive values), so a block's absmax is a 5-step butterfly inside the
// half-wave and no LDS or barrier is needed.
#include "vs_device.h"
#include "vs_sh.h"
#include "vs_internal.h"

namespace vs {

constexpr uint32_t B8_VALUES = 128;            // quant.rs:15
constexpr uint32_t B8_WORDS = B8_VALUES / 4;   // one word per lane of a half-wave
constexpr int SH_STEP_BLOCK = 256;             // 4 waves = 8 moment blocks

// quant_kernels.rs:866-894: round to one of the two f16 values adjacent to
// `value` with probability proportional to distance; a per-value, per-step
// integer hash gives 24 uniform bits.  Values beyond the f16 range (and NaN)
// pass through for the conversion to turn into infinities.
VS_DEV float stochastic_half(float value, uint32_t index, uint32_t step) {
    const float magnitude = __builtin_fabsf(value);
    if (!(magnitude <= 65504.0f)) return value;
    float lower, upper;
    if (magnitude < 6.103515625e-05f) {           // f16 subnormals: spacing 2^-24
        lower = __builtin_floorf(magnitude * 16777216.0f) / 16777216.0f;
        upper = lower + 5.9604644775390625e-08f;
    } else {
        const uint32_t bits = as_u(magnitude) & 0xffffe000u;
        lower = as_f(bits);
        upper = as_f(bits + 8192u);
    }
    uint32_t h = index ^ (step * 0x9e3779b9u);
    h = (h ^ (h >> 16)) * 0x7feb352du;
    h = (h ^ (h >> 15)) * 0x846ca68bu;
    h = h ^ (h >> 16);
    const float uniform = (float)(h >> 8) / 16777216.0f;
    const float probability = (magnitude - lower) / (upper - lower);
    const float r = uniform < probability ? upper : lower;
    return value < 0.0f ? -r : r;
}

// Block absmax over the 32 lanes of this half-wave (NaN-ignoring max).
VS_DEV float half_wave_max(float v) {
#pragma unroll
    for (int off = 16; off > 0; off >>= 1) v = mx(v, __shfl_xor(v, off, 64));
    return v;
}

// pack_block's code: round(clamp(m / scale, -127, 127)) + 128, 128 for a
// zero scale (ties to even).
VS_DEV uint32_t b8_code(float m, float scale) {
    if (!(scale > 0.0f)) return 128u;
    return (uint32_t)(__builtin_rintf(clampf(m / scale, -127.0f, 127.0f)) + 128.0f);
}

VS_DEV float b8_value(uint32_t word, int j, float scale) {
    return ((float)((word >> (8 * j)) & 255u) - 128.0f) * scale;
}

// The second moment, one f32 per splat (optim.rs:447-469), before the step
// reads it: v beta2 + grad_sq (1 - beta2) for splats with gradients, kept for
// culled ones (compact row 0); at the first step grad_sq (1 - beta2) for all.
__global__ void sh_variance_kernel(ShStepArgs a) {
    const uint32_t g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= a.num_splats) return;
    const float c2 = 1.0f - a.beta2;
    const float gsq = a.grad_sq[g];
    if (a.first) a.variance[g] = gsq * c2;
    else if (a.grad_rows[g] != 0u) a.variance[g] = a.variance[g] * a.beta2 + gsq * c2;
}

// step_kernel_w4 (quant_kernels.rs:582-727).  Values of culled splats keep
// their coefficient and moment; a block without a value of a visible splat
// is left untouched; every other block is re-packed from the stepped moments.
template <int DEG>
__global__ void __launch_bounds__(SH_STEP_BLOCK) sh_step_kernel(ShStepArgs a) {
    constexpr uint32_t K = sh_count<DEG>();
    constexpr uint32_t RW = K * 3;                // values per splat row
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t block = (blockIdx.x * SH_STEP_BLOCK + threadIdx.x) >> 5;
    const uint32_t word = block * B8_WORDS + (lane & 31u);
    const uint32_t n = a.num_values;
    const uint32_t first = word * 4u;
    const bool live = block < a.num_blocks;       // the whole half-wave agrees

    // The (at most two) splat rows this word's values fall in.
    const uint32_t row_a = first / RW;
    const uint32_t last = first + 3u < n ? first + 3u : n - 1u;
    const uint32_t row_b = last / RW;
    uint32_t gr_a = 0u, gr_b = 0u;
    if (live && first < n) {
        gr_a = a.grad_rows[row_a];
        gr_b = row_b == row_a ? gr_a : a.grad_rows[row_b];
    }
    const bool any = gr_a != 0u || gr_b != 0u;
    const uint64_t ballot = __ballot(any);
    const uint32_t half_bits = (uint32_t)(ballot >> (lane & 32u));
    if (half_bits == 0u) return;                  // half-wave uniform: no shuffle below mixes halves

    const float old_scale = a.scales[block];
    const uint32_t old = a.codes[word];
    float m[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) m[j] = first + j < n ? b8_value(old, j, old_scale) : 0.0f;

    if (any) {
        const float factor = 1.0f - a.beta1;
        float ya[K], yb[K];
        float cda[3] = {0.0f, 0.0f, 0.0f}, cdb[3] = {0.0f, 0.0f, 0.0f};
        float den_a = 1.0f, den_b = 1.0f;
        if (gr_a != 0u) {
            const float* cd = a.color_dir + (size_t)gr_a * 6;
            cda[0] = cd[0]; cda[1] = cd[1]; cda[2] = cd[2];
            sh_basis<DEG>(F3{cd[3], cd[4], cd[5]}, ya);
            den_a = __builtin_sqrtf(a.variance[row_a] * a.inv2) + a.epsilon;
        }
        if (row_b != row_a && gr_b != 0u) {
            const float* cd = a.color_dir + (size_t)gr_b * 6;
            cdb[0] = cd[0]; cdb[1] = cd[1]; cdb[2] = cd[2];
            sh_basis<DEG>(F3{cd[3], cd[4], cd[5]}, yb);
            den_b = __builtin_sqrtf(a.variance[row_b] * a.inv2) + a.epsilon;
        }
        uint16_t* p = a.sh + first;
        uint16_t ph[4];
        const bool whole = first + 3u < n;
        if (whole) {
            const uint2 q = *reinterpret_cast<const uint2*>(p);
            ph[0] = (uint16_t)(q.x & 0xFFFFu); ph[1] = (uint16_t)(q.x >> 16);
            ph[2] = (uint16_t)(q.y & 0xFFFFu); ph[3] = (uint16_t)(q.y >> 16);
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j) ph[j] = first + j < n ? p[j] : (uint16_t)0;
        }
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t idx = first + j;
            const uint32_t row = idx / RW;
            const bool on_a = row == row_a;
            if (idx >= n || (on_a ? gr_a : gr_b) == 0u) continue;
            const uint32_t col = idx - row * RW;
            const uint32_t k = col / 3u, c = col - k * 3u;
            float basis = 0.0f;
#pragma unroll
            for (uint32_t t = 0; t < K; ++t) basis = t == k ? (on_a ? ya[t] : yb[t]) : basis;
            const float colour = c == 0u ? (on_a ? cda[0] : cdb[0]) : (c == 1u ? (on_a ? cda[1] : cdb[1])
                                                                              : (on_a ? cda[2] : cdb[2]));
            const float gv = basis * colour;
            const float moment = m[j] * a.beta1 + gv * factor;
            const float denom = on_a ? den_a : den_b;
            const float delta = (moment * a.inv1 / denom) * (a.lr_scale[col] * a.lr);
            const float updated = stochastic_half(h2f(ph[j]) - delta, idx, a.round_seed);
            ph[j] = f2h(updated);
            m[j] = moment;
        }
        if (whole) {
            *reinterpret_cast<uint2*>(p) = make_uint2((uint32_t)ph[0] | ((uint32_t)ph[1] << 16),
                                                      (uint32_t)ph[2] | ((uint32_t)ph[3] << 16));
        } else {
#pragma unroll
            for (int j = 0; j < 4; ++j)
                if (first + j < n) p[j] = ph[j];
        }
    }
    const float local = mx(mx(__builtin_fabsf(m[0]), __builtin_fabsf(m[1])),
                           mx(__builtin_fabsf(m[2]), __builtin_fabsf(m[3])));
    const float scale = half_wave_max(local) / 127.0f;
    if ((lane & 31u) == 0u) a.scales[block] = scale;
    uint32_t packed = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) packed |= b8_code(m[j], scale) << (8 * j);
    a.codes[word] = packed;
}

// encode_kernel / pack_block (quant_kernels.rs:438-484): values past n are 0.
__global__ void __launch_bounds__(SH_STEP_BLOCK) b8_encode_kernel(const float* __restrict__ values, uint32_t n,
                                                                  uint32_t num_blocks, uint32_t* __restrict__ codes,
                                                                  float* __restrict__ scales) {
    const uint32_t lane = threadIdx.x & 63u;
    const uint32_t block = (blockIdx.x * SH_STEP_BLOCK + threadIdx.x) >> 5;
    if (block >= num_blocks) return;              // half-wave uniform
    const uint32_t word = block * B8_WORDS + (lane & 31u);
    float v[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) v[j] = word * 4u + j < n ? values[word * 4u + j] : 0.0f;
    const float local = mx(mx(__builtin_fabsf(v[0]), __builtin_fabsf(v[1])), mx(__builtin_fabsf(v[2]), __builtin_fabsf(v[3])));
    const float scale = half_wave_max(local) / 127.0f;
    if ((lane & 31u) == 0u) scales[block] = scale;
    uint32_t packed = 0u;
#pragma unroll
    for (int j = 0; j < 4; ++j) packed |= b8_code(v[j], scale) << (8 * j);
    codes[word] = packed;
}

// decode_kernel / unpack (quant_kernels.rs:486-498).
__global__ void b8_decode_kernel(const uint32_t* __restrict__ codes, const float* __restrict__ scales, uint32_t n,
                                 float* __restrict__ out) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = b8_value(codes[i / 4u], (int)(i % 4u), scales[i / B8_VALUES]);
}

// zero_moment_rows_kernel (quant_kernels.rs:911-925): each value of the
// listed rows gets the zero code 128; rows may share words, so the byte is
// cleared and set with two word atomics that touch only it.  Values past n
// are ignored.
__global__ void b8_zero_rows_kernel(uint32_t* __restrict__ codes, uint32_t n, const uint32_t* __restrict__ rows,
                                    uint32_t num_rows, uint32_t row_width) {
    const uint64_t pos = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (pos >= (uint64_t)num_rows * row_width) return;
    const uint64_t idx = (uint64_t)rows[pos / row_width] * row_width + pos % row_width;
    if (idx >= n) return;
    const uint32_t shift = (uint32_t)(idx % 4u) * 8u;
    atomicAnd(codes + idx / 4u, ~(255u << shift));
    atomicOr(codes + idx / 4u, 128u << shift);
}

hipError_t launch_sh_step(const ShStepArgs& a, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    sh_variance_kernel<<<(a.num_splats + 255) / 256, 256, 0, s>>>(a);
    const uint32_t grid = (a.num_blocks + SH_STEP_BLOCK / 32 - 1) / (SH_STEP_BLOCK / 32);
    switch (a.sh_degree) {
    case 0: sh_step_kernel<0><<<grid, SH_STEP_BLOCK, 0, s>>>(a); break;
    case 1: sh_step_kernel<1><<<grid, SH_STEP_BLOCK, 0, s>>>(a); break;
    case 2: sh_step_kernel<2><<<grid, SH_STEP_BLOCK, 0, s>>>(a); break;
    case 3: sh_step_kernel<3><<<grid, SH_STEP_BLOCK, 0, s>>>(a); break;
    default: sh_step_kernel<4><<<grid, SH_STEP_BLOCK, 0, s>>>(a); break;
    }
    return hipGetLastError();
}

hipError_t launch_b8_encode(const float* values, uint32_t n, uint32_t* codes, float* scales, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint32_t blocks = (n + B8_VALUES - 1) / B8_VALUES;
    b8_encode_kernel<<<(blocks + SH_STEP_BLOCK / 32 - 1) / (SH_STEP_BLOCK / 32), SH_STEP_BLOCK, 0, s>>>(
        values, n, blocks, codes, scales);
    return hipGetLastError();
}

hipError_t launch_b8_decode(const uint32_t* codes, const float* scales, uint32_t n, float* values, hipStream_t s) {
    if (n == 0) return hipSuccess;
    b8_decode_kernel<<<(n + 255) / 256, 256, 0, s>>>(codes, scales, n, values);
    return hipGetLastError();
}

hipError_t launch_b8_zero_rows(uint32_t* codes, uint32_t n, const uint32_t* rows, uint32_t num_rows,
                               uint32_t row_width, hipStream_t s) {
    const uint64_t total = (uint64_t)num_rows * row_width;
    if (total == 0) return hipSuccess;
    b8_zero_rows_kernel<<<(uint32_t)((total + 255) / 256), 256, 0, s>>>(codes, n, rows, num_rows, row_width);
    return hipGetLastError();
}

} // namespace vs
