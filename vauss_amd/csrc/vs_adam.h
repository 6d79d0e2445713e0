// vs_adam.h -- packed Adam moments (one u32 per parameter value) and the
// f32 Adam step on them, as the fused projection update uses them.
//
// Restates crates/splat-train-render/src/bwd/kernels/geo_moments.rs:1-127.
// With Adam's epsilon e, u = m / (sqrt(v) + e) and l = ln(1 + sqrt(v) / e).
// Low half of a word: u sign-magnitude, 15-bit magnitude over [0, 8].  High
// half: l as a 16-bit code over [0, 64].  Decode: sqrt(v) = e (exp(l) - 1),
// m = u e exp(l), so word 0 is exactly m = v = 0.  Encoding adds a rounding
// offset in [0, 1) to each code before the floor: 0.5 rounds to nearest, a
// hashed uniform rounds stochastically (one beta2 decay moves l by less than
// half a code step, so round-to-nearest would freeze decaying moments).
//
// The transcendentals are the build's own (expf_c, logf_c) and every
// multiply-add is unfused, so the CPU restatement reproduces the words bit for
// bit.
#pragma once
#include "vs_device.h"

namespace vs {

constexpr float GEO_U_MAX = 8.0f;
constexpr float GEO_U_CODES = 32767.0f;
constexpr float GEO_U_STEP = GEO_U_MAX / GEO_U_CODES;
constexpr float GEO_U_PER_UNIT = GEO_U_CODES / GEO_U_MAX;
constexpr float GEO_L_MAX = 64.0f;
constexpr float GEO_L_CODES = 65535.0f;
constexpr float GEO_L_STEP = GEO_L_MAX / GEO_L_CODES;
constexpr float GEO_L_PER_UNIT = GEO_L_CODES / GEO_L_MAX;

// exp(l) of a word (geo_moments.rs:24-28).
VS_DEV float geo_growth(uint32_t word) { return expf_c((float)(word >> 16) * GEO_L_STEP); }

// Normalized first moment u of a word (geo_moments.rs:30-35).
VS_DEV float geo_normalized(uint32_t word) {
    const float magnitude = (float)(word & 0x7fffu) * GEO_U_STEP;
    return (word & 0x8000u) ? -magnitude : magnitude;
}

// geo_moments.rs:37-56
VS_DEV uint32_t pack_geo(float m, float v, float epsilon, float round_l, float round_u) {
    const float l = logf_c(1.0f + __builtin_sqrtf(mx(v, 0.0f)) / epsilon) * GEO_L_PER_UNIT;
    const float l_code = __builtin_floorf(clampf(l + round_l, 0.0f, GEO_L_CODES));
    const float scale = epsilon * expf_c(l_code * GEO_L_STEP);
    const float u = __builtin_fabsf(m) / scale * GEO_U_PER_UNIT;
    const uint32_t u_code = (uint32_t)__builtin_floorf(clampf(u + round_u, 0.0f, GEO_U_CODES));
    const uint32_t sign = (m < 0.0f) ? 0x8000u : 0u;
    return ((uint32_t)l_code << 16) | sign | u_code;
}

// Per-element, per-step integer hash for the stochastic rounding
// (geo_moments.rs:58-66).
VS_DEV uint32_t mix_hash(uint32_t index, uint32_t step) {
    uint32_t h = index ^ (step * 0x9e3779b9u);
    h = (h ^ (h >> 16)) * 0x7feb352du;
    h = (h ^ (h >> 15)) * 0x846ca68bu;
    return h ^ (h >> 16);
}

// One Adam step of `param` with its packed moments `word` (geo_moments.rs:68-101);
// `index` is the element's flat index, which seeds its rounding stream.
VS_DEV void adam_packed(float& param, uint32_t& word, uint32_t index, float g, float lr, float beta1, float beta2,
                        float inv1, float inv2, float epsilon, uint32_t seed) {
    const float growth = geo_growth(word);
    const float root = epsilon * (growth - 1.0f);
    const float m1 = geo_normalized(word) * (epsilon * growth) * beta1 + g * (1.0f - beta1);
    const float v1 = root * root * beta2 + g * g * (1.0f - beta2);
    const float step = (m1 * inv1) / (__builtin_sqrtf(v1 * inv2) + epsilon);
    param = param - step * lr;
    const uint32_t h = mix_hash(index, seed);
    word = pack_geo(m1, v1, epsilon, (float)(h >> 16) / 65536.0f, (float)(h & 0xffffu) / 65536.0f);
}

} // namespace vs
