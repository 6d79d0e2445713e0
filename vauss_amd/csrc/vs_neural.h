// vs_neural.h -- compact neural appearance: one shared decoder evaluated once
// per visible splat in the projection, and its backward.
//
// Restates crates/splat-train-render/src/kernels/neural.rs:1-161 and
// bwd/kernels/neural_backwards.rs:82-283.  Each splat's coefficient row holds
// 12 floats: the base colour as an SH DC coefficient (3), a latent f (8) and a
// pad.  For the unit view direction d:
//   x  = [sin f0, cos f0, ..., sin f7, cos f7, Y0(d) .. Y15(d)]   (bands > degree are 0)
//   h1 = ReLU(W1 x), h2 = ReLU(W2 h1), colour = ReLU(C0 base + tanh(W3 h2) + 0.5)
// with W1 16x32, W2 16x16, W3 3x16 row-major [out][in] packed in one [816]
// array.  Every dot product accumulates in input order from 0 without fused
// multiply-adds, so the CPU restatement reproduces it bit for bit.
#pragma once
#include "vs_device.h"
#include "vs_sh.h"

namespace vs {

constexpr int NEURAL_DEG = -1;                 // the DEG template value of neural mode
constexpr int NEURAL_LATENTS = 8, NEURAL_INPUTS = 32, NEURAL_HIDDEN = 16;
constexpr int NEURAL_W1 = 0, NEURAL_W2 = 512, NEURAL_W3 = 768, NEURAL_LEN = 816;
constexpr int NEURAL_ROW = 12;                 // floats per splat row
constexpr uint32_t NEURAL_MAX_DEGREE = 3;
constexpr float NEURAL_C0 = 0.2820948f;

// write_direction_basis (neural.rs:64-98): real SH bands 0..3 of d into x[16..32).
VS_DEV void direction_basis(float* x, F3 v, uint32_t deg) {
    const float vx = v.x, vy = v.y, vz = v.z;
    const float xy = vx * vy, xz = vx * vz, yz = vy * vz, x2 = vx * vx, y2 = vy * vy, z2 = vz * vz;
    const float m1 = deg >= 1u ? 1.0f : 0.0f, m2 = deg >= 2u ? 1.0f : 0.0f, m3 = deg >= 3u ? 1.0f : 0.0f;
    x[16] = 0.2820948f;
    x[17] = m1 * (-0.4886025f * vy);
    x[18] = m1 * (0.4886025f * vz);
    x[19] = m1 * (-0.4886025f * vx);
    x[20] = m2 * (1.0925484f * xy);
    x[21] = m2 * (-1.0925484f * yz);
    x[22] = m2 * (0.9461747f * z2 - 0.31539157f);
    x[23] = m2 * (-1.0925484f * xz);
    x[24] = m2 * (0.5462742f * x2 - 0.5462742f * y2);
    x[25] = m3 * (0.5900436f * vy * (-3.0f * x2 + y2));
    x[26] = m3 * (2.8906114f * xy * vz);
    x[27] = m3 * (0.4570458f * vy * (1.0f - 5.0f * z2));
    x[28] = m3 * (0.37317633f * vz * (5.0f * z2 - 3.0f));
    x[29] = m3 * (0.4570458f * vx * (1.0f - 5.0f * z2));
    x[30] = m3 * (1.4453057f * vz * (x2 - y2));
    x[31] = m3 * (0.5900436f * vx * (-x2 + 3.0f * y2));
}

// direction_basis_vjp (neural_backwards.rs:82-133).
VS_DEV F3 direction_basis_vjp(const float* dx, F3 v, uint32_t deg) {
    const float x = v.x, y = v.y, z = v.z;
    float gx = 0.0f, gy = 0.0f, gz = 0.0f;
    if (deg >= 1u) {
        const float c1 = 0.4886025f;
        gy += -c1 * dx[17];
        gz += c1 * dx[18];
        gx += -c1 * dx[19];
    }
    if (deg >= 2u) {
        const float a = 1.0925484f;
        gx += a * y * dx[20];
        gy += a * x * dx[20];
        gy += -a * z * dx[21];
        gz += -a * y * dx[21];
        gz += 1.8923494f * z * dx[22];
        gx += -a * z * dx[23];
        gz += -a * x * dx[23];
        gx += a * x * dx[24];
        gy += -a * y * dx[24];
    }
    if (deg >= 3u) {
        const float x2 = x * x, y2 = y * y, z2 = z * z;
        const float b = 1.7701308f, c = 2.8906114f, e = 0.4570458f, f = 4.570458f;
        gx += -3.5402615f * x * y * dx[25];
        gy += (b * y2 - b * x2) * dx[25];
        gx += c * y * z * dx[26];
        gy += c * x * z * dx[26];
        gz += c * x * y * dx[26];
        gy += (e - 2.285229f * z2) * dx[27];
        gz += -f * y * z * dx[27];
        gz += (5.597645f * z2 - 1.119529f) * dx[28];
        gx += (e - 2.285229f * z2) * dx[29];
        gz += -f * x * z * dx[29];
        gx += c * x * z * dx[30];
        gy += -c * y * z * dx[30];
        gz += 1.4453057f * (x2 - y2) * dx[30];
        gx += (b * y2 - b * x2) * dx[31];
        gy += 3.5402615f * x * y * dx[31];
    }
    return F3{gx, gy, gz};
}

// The decoder's forward for one row; `row` holds 12 values (f32 or f16 bits).
template <typename SHT>
VS_DEV void neural_forward(const SHT* __restrict__ row, const float* __restrict__ W, F3 v, uint32_t deg,
                           float* x, float* h1, float* h2, float* o) {
#pragma unroll
    for (int i = 0; i < NEURAL_LATENTS; ++i) sincosf_c(sh_ld(row, 3 + i), x[2 * i], x[2 * i + 1]);
    direction_basis(x, v, deg);
#pragma unroll
    for (int j = 0; j < NEURAL_HIDDEN; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NEURAL_INPUTS; ++k) acc += W[NEURAL_W1 + j * NEURAL_INPUTS + k] * x[k];
        h1[j] = mx(acc, 0.0f);
    }
#pragma unroll
    for (int j = 0; j < NEURAL_HIDDEN; ++j) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NEURAL_HIDDEN; ++k) acc += W[NEURAL_W2 + j * NEURAL_HIDDEN + k] * h1[k];
        h2[j] = mx(acc, 0.0f);
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        float acc = 0.0f;
#pragma unroll
        for (int k = 0; k < NEURAL_HIDDEN; ++k) acc += W[NEURAL_W3 + c * NEURAL_HIDDEN + k] * h2[k];
        o[c] = acc;
    }
}

// neural_color (neural.rs:100-161).
template <typename SHT>
VS_DEV F3 neural_color(const SHT* __restrict__ row, const float* __restrict__ W, F3 v, uint32_t deg) {
    float x[NEURAL_INPUTS], h1[NEURAL_HIDDEN], h2[NEURAL_HIDDEN], o[3];
    neural_forward(row, W, v, deg, x, h1, h2, o);
    return F3{mx(sh_ld(row, 0) * NEURAL_C0 + tanhf_c(o[0]) + 0.5f, 0.0f),
              mx(sh_ld(row, 1) * NEURAL_C0 + tanhf_c(o[1]) + 0.5f, 0.0f),
              mx(sh_ld(row, 2) * NEURAL_C0 + tanhf_c(o[2]) + 0.5f, 0.0f)};
}

}  // namespace vs
