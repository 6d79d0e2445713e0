// or_math.h -- oracle-side arithmetic: the f32 transcendental contract and
// the small linear-algebra types of the reference's cube math.
//
// TEST INFRASTRUCTURE ONLY (see vs_oracle.h).
//
// Every expression here is written in the operation order of the reference
// (crates/splat-train-cube/src/lib.rs) and compiled with -ffp-contract=off, so
// a multiply-add is fused only where `std::fma` is written explicitly.
#pragma once
#include <cmath>
#include <cstdint>
#include <cstring>
#include <algorithm>

namespace orc {

static inline uint32_t f2u(float x) { uint32_t u; std::memcpy(&u, &x, 4); return u; }
static inline float u2f(uint32_t u) { float x; std::memcpy(&x, &u, 4); return x; }

// Bit-level finite check, crates/splat-train-cube/src/lib.rs:566-571.
static inline bool is_finite(float x) { return ((f2u(x) >> 23) & 0xFFu) != 0xFFu; }

// ---------------------------------------------------------------------------
// Transcendentals.  The reference leaves exp/log/atan2 to the shader
// compiler's intrinsics, whose last-ulp behaviour no test of the reference
// pins.  The contract fixes one portable evaluation built only from IEEE
// add/mul/fma/divide, rint and ldexp, so the oracle and the GPU kernels agree
// bit for bit.
//
// exp: Cody-Waite reduction x = n ln2 + r, |r| <= ln2/2, then
//      e^r = 1 + (r + r^2 q(r)) with a degree-4 q fitted by least squares on
//      [-ln2/2, ln2/2] (relative error of the result ~1.2 ulp).
//      x < -87.33654 returns 0 (no subnormal results), x > 88.72283 -> +inf.
// ---------------------------------------------------------------------------
static inline float expf_c(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return INFINITY;
    if (x < -87.33654f) return 0.0f;
    const float n = std::rint(x * 1.44269502f);
    float r = std::fma(-n, 0.693145751953125f, x);
    r = std::fma(-n, 1.42860677e-06f, r);
    float q = std::fma(0.00137514074f, r, 0.00836891588f);
    q = std::fma(q, r, 0.0416695327f);
    q = std::fma(q, r, 0.166665182f);
    q = std::fma(q, r, 0.499999881f);
    const float r2 = r * r;
    const float p = std::fma(r2, q, r) + 1.0f;
    return std::ldexp(p, (int)n);
}

// exp2n: 2^x for the compositing loops, whose argument is -sigma in base-2
//      units (sigma log2 e, never positive for a pair that can contribute):
//      x = min(max(x, -127), 128) (NaN -> -127), n = rint(x), f = x - n in
//      [-1/2, 1/2] (exact), 2^f = 1 + f P(f) with P of degree 4 fitted for
//      least maximum relative error on [-1/2, 1/2] (Lawson iterations),
//      result ldexp(p, n); relative error <= 2.1 ulp on [-126, 0].
static inline float exp2n_c(float x) {
    x = std::fmin(std::fmax(x, -127.0f), 128.0f);
    const float n = std::rint(x);
    const float f = x - n;
    float p = std::fma(1.326472731e-03f, f, 9.671512991e-03f);
    p = std::fma(p, f, 5.550733581e-02f);
    p = std::fma(p, f, 2.402224243e-01f);
    p = std::fma(p, f, 6.931470037e-01f);
    p = std::fma(p, f, 1.0f);
    return std::ldexp(p, (int)n);
}
// log2(e) rounded to f32: the compositing loops scale the conic by it so
// sigma comes out in base-2 units.
constexpr float LOG2E_F = 1.44269502f;

// log: x = m 2^e with m in [sqrt(1/2), sqrt(2)); s = (m-1)/(m+1);
//      ln m = 2 atanh(s) = 2s + s * s^2 (2/3 + 2/5 s^2 + 2/7 s^4 + 2/9 s^6)
//      (Taylor terms of atanh; |s| <= 0.1716 so the tail is < 3e-9).
//      ln x = e ln2_hi + (e ln2_lo + ln m).
static inline float logf_c(float x) {
    if (x != x) return x;
    if (x < 0.0f) return NAN;
    if (x == 0.0f) return -INFINITY;
    if (x == INFINITY) return INFINITY;
    int e = 0;
    uint32_t b = f2u(x);
    if (b < 0x00800000u) {            // subnormal input: scale into the normal range
        x = x * 8388608.0f;
        b = f2u(x);
        e = -23;
    }
    e += (int)(b >> 23) - 127;
    float m = u2f((b & 0x007FFFFFu) | 0x3F800000u);
    if (m > 1.41421354f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float s2 = s * s;
    float R = std::fma(s2, 0.222222224f, 0.285714298f);
    R = std::fma(R, s2, 0.400000006f);
    R = std::fma(R, s2, 0.666666687f);
    R = R * s2;
    const float lnm = std::fma(s, R, s + s);
    const float ef = (float)e;
    return std::fma(ef, 0.693145751953125f, std::fma(ef, 1.42860677e-06f, lnm));
}

// atan2: octant reduction to a = min/max in [0,1]; a > tan(pi/8) uses
//        t = (a-1)/(a+1) and pi/4; atan(t) = t + t^3 P(t^2) with a degree-4 P
//        fitted by least squares on [0, tan(pi/8)] (~1 ulp).
static inline float atan2f_c(float y, float x) {
    if (x != x || y != y) return x + y;
    const float ax = std::fabs(x), ay = std::fabs(y);
    float r;
    if (ax == INFINITY || ay == INFINITY) {
        if (ax == INFINITY && ay == INFINITY) r = (x < 0.0f) ? 2.35619449f : 0.785398163f;
        else if (ax == INFINITY) r = (x < 0.0f) ? 3.14159274f : 0.0f;
        else r = 1.57079637f;
        return std::copysign(r, y);
    }
    if (ax == 0.0f && ay == 0.0f) {
        r = std::signbit(x) ? 3.14159274f : 0.0f;
        return std::copysign(r, y);
    }
    const float mx = std::max(ax, ay);
    const float mn = std::min(ax, ay);
    const float a = mn / mx;
    float t, base;
    if (a > 0.414213568f) { t = (a - 1.0f) / (a + 1.0f); base = 0.785398163f; }
    else { t = a; base = 0.0f; }
    const float t2 = t * t;
    float P = std::fma(-0.0609764382f, t2, 0.106022187f);
    P = std::fma(P, t2, -0.142448023f);
    P = std::fma(P, t2, 0.199985489f);
    P = std::fma(P, t2, -0.333333164f);
    const float at = std::fma(t * t2, P, t);
    r = base + at;
    if (ay > ax) r = (1.57079637f - r) + (-4.37113883e-08f);
    if (x < 0.0f) r = (3.14159274f - r) + (-8.74227766e-08f);
    return std::copysign(r, y);
}

// sin and cos of one argument: j = rint(x 2/pi); r = x - j pi/2 in three fma
// steps (pi/2 split into three f32 parts), |r| <= pi/4 plus rounding; Taylor
// polynomials of sin r (through r^11) and cos r (through r^12) in Horner
// form; the quadrant j mod 4 picks and signs them.  Non-finite x -> NaN.
static inline void sincosf_c(float x, float& s, float& c) {
    if (!is_finite(x)) { s = c = NAN; return; }
    const float j = std::rint(x * 0x1.45f306p-1f);
    float r = std::fma(-j, 0x1.921fb6p+0f, x);
    r = std::fma(-j, -0x1.777a5cp-25f, r);
    r = std::fma(-j, -0x1.ee59dap-50f, r);
    const float z = r * r;
    float ps = std::fma(z, -0x1.ae6456p-26f, 0x1.71de3ap-19f);
    ps = std::fma(ps, z, -0x1.a01a02p-13f);
    ps = std::fma(ps, z, 0x1.111112p-7f);
    ps = std::fma(ps, z, -0x1.555556p-3f);
    const float sr = std::fma(r * z, ps, r);
    float pc = std::fma(z, 0x1.1eed8ep-29f, -0x1.27e4fcp-22f);
    pc = std::fma(pc, z, 0x1.a01a02p-16f);
    pc = std::fma(pc, z, -0x1.6c16c2p-10f);
    pc = std::fma(pc, z, 0x1.555556p-5f);
    pc = std::fma(pc, z, -0.5f);
    const float cr = std::fma(z, pc, 1.0f);
    const int q = (int)(j - 4.0f * std::floor(j * 0.25f));
    s = (q == 0) ? sr : (q == 1) ? cr : (q == 2) ? -sr : -cr;
    c = (q == 0) ? cr : (q == 1) ? -sr : (q == 2) ? -cr : sr;
}

// tanh: |x| < 0.5625 -> x + x^3 P(x^2), P the Taylor series of (tanh x - x)/x^3
// through x^16; otherwise 1 - 2 / (exp(2|x|) + 1) with the sign of x (1 once
// exp overflows); signed zeros pass through.
static inline float tanhf_c(float x) {
    if (x != x || x == 0.0f) return x;
    const float a = std::fabs(x);
    if (a < 0.5625f) {
        const float z = x * x;
        float p = std::fma(z, -0x1.f57d78p-13f, 0x1.355824p-11f);
        p = std::fma(p, z, -0x1.7da364p-10f);
        p = std::fma(p, z, 0x1.d6d3d0p-9f);
        p = std::fma(p, z, -0x1.226e36p-7f);
        p = std::fma(p, z, 0x1.664f48p-6f);
        p = std::fma(p, z, -0x1.ba1ba2p-5f);
        p = std::fma(p, z, 0x1.111112p-3f);
        p = std::fma(p, z, -0x1.555556p-2f);
        return std::fma(x * z, p, x);
    }
    const float t = 1.0f - 2.0f / (expf_c(2.0f * a) + 1.0f);
    return std::copysign(t, x);
}

// sigmoid, crates/splat-train-cube/src/lib.rs:561-564.
static inline float sigmoid(float x) { return 1.0f / (1.0f + expf_c(-x)); }

// Rust's f32::min / f32::max / clamp on finite values.
static inline float fmin_(float a, float b) { return (a < b) ? a : ((b == b) ? b : a); }
static inline float fmax_(float a, float b) { return (a > b) ? a : ((b == b) ? b : a); }
static inline float clampf(float v, float lo, float hi) { return fmin_(fmax_(v, lo), hi); }

// ---------------------------------------------------------------------------
// Cube math types, crates/splat-train-cube/src/lib.rs:40-559, in the same
// operation order.
// ---------------------------------------------------------------------------
struct V3 { float x, y, z; };
static inline V3 v3(float x, float y, float z) { return V3{x, y, z}; }
static inline V3 add(V3 a, V3 b) { return V3{a.x + b.x, a.y + b.y, a.z + b.z}; }
static inline V3 sub(V3 a, V3 b) { return V3{a.x - b.x, a.y - b.y, a.z - b.z}; }
static inline V3 scale(V3 a, float s) { return V3{a.x * s, a.y * s, a.z * s}; }
// Vec3A::dot sums four lanes, the padding lane being 0 * 0.
static inline float dot(V3 a, V3 b) { return ((a.x * b.x + a.y * b.y) + a.z * b.z) + 0.0f * 0.0f; }
static inline float length(V3 a) { return std::sqrt(dot(a, a)); }
static inline V3 normalize(V3 a) { return scale(a, 1.0f / length(a)); }
static inline bool finite3(V3 a) { return is_finite(a.x) && is_finite(a.y) && is_finite(a.z); }

struct V2 { float x, y; };
static inline V2 add2(V2 a, V2 b) { return V2{a.x + b.x, a.y + b.y}; }
static inline V2 scale2(V2 a, float s) { return V2{a.x * s, a.y * s}; }
static inline float dot2(V2 a, V2 b) { return a.x * b.x + a.y * b.y; }

struct Q4 { float w, x, y, z; };
static inline float qdot(Q4 a, Q4 b) { return ((a.w * b.w + a.x * b.x) + a.y * b.y) + a.z * b.z; }
static inline Q4 qscale(Q4 a, float s) { return Q4{a.w * s, a.x * s, a.y * s, a.z * s}; }
static inline Q4 qnormalize(Q4 a) { return qscale(a, 1.0f / std::sqrt(qdot(a, a))); }

// Column-major 3x3: c[i] is column i.
struct M3 { V3 c0, c1, c2; };
static inline M3 quat_to_mat3(Q4 q) {
    const float w = q.w, qx = q.x, qy = q.y, qz = q.z;
    const float x2 = qx * qx, y2 = qy * qy, z2 = qz * qz;
    const float xy = qx * qy, xz = qx * qz, yz = qy * qz;
    const float wx = w * qx, wy = w * qy, wz = w * qz;
    M3 m;
    m.c0 = V3{1.0f - 2.0f * (y2 + z2), 2.0f * (xy + wz), 2.0f * (xz - wy)};
    m.c1 = V3{2.0f * (xy - wz), 1.0f - 2.0f * (x2 + z2), 2.0f * (yz + wx)};
    m.c2 = V3{2.0f * (xz + wy), 2.0f * (yz - wx), 1.0f - 2.0f * (x2 + y2)};
    return m;
}
static inline V3 mul_vec3(M3 m, V3 v) { return add(add(scale(m.c0, v.x), scale(m.c1, v.y)), scale(m.c2, v.z)); }
static inline V3 tmul_vec3(M3 m, V3 v) { return V3{dot(m.c0, v), dot(m.c1, v), dot(m.c2, v)}; }
static inline M3 mul_mat3(M3 a, M3 b) { return M3{mul_vec3(a, b.c0), mul_vec3(a, b.c1), mul_vec3(a, b.c2)}; }
static inline M3 mul_diag(M3 a, V3 s) { return M3{scale(a.c0, s.x), scale(a.c1, s.y), scale(a.c2, s.z)}; }
static inline V3 row0(M3 m) { return V3{m.c0.x, m.c1.x, m.c2.x}; }
static inline V3 row1(M3 m) { return V3{m.c0.y, m.c1.y, m.c2.y}; }
static inline V3 row2(M3 m) { return V3{m.c0.z, m.c1.z, m.c2.z}; }

struct S2 { float c00, c01, c11; };
struct S3 { float c00, c01, c02, c11, c12, c22; };
static inline S3 outer_self(M3 m) {
    const V3 r0 = row0(m), r1 = row1(m), r2 = row2(m);
    return S3{dot(r0, r0), dot(r0, r1), dot(r0, r2), dot(r1, r1), dot(r1, r2), dot(r2, r2)};
}
static inline V2 s2_mul_vec2(S2 s, V2 v) { return add2(scale2(V2{s.c00, s.c01}, v.x), scale2(V2{s.c01, s.c11}, v.y)); }
static inline S2 s2_scale(S2 s, float k) { return S2{s.c00 * k, s.c01 * k, s.c11 * k}; }
static inline float s2_max_abs(S2 s) { return fmax_(fmax_(std::fabs(s.c00), std::fabs(s.c11)), std::fabs(s.c01)); }
static inline S2 s2_inverse(S2 s) {
    const float det = s.c00 * s.c11 - s.c01 * s.c01;
    const float inv_det = (det > 0.0f) ? 1.0f / det : 0.0f;
    return S2{s.c11 * inv_det, -s.c01 * inv_det, s.c00 * inv_det};
}
static inline bool s2_finite(S2 s) { return is_finite(s.c00) && is_finite(s.c11) && is_finite(s.c01); }

static inline V3 s3_row0(S3 s) { return V3{s.c00, s.c01, s.c02}; }
static inline V3 s3_row1(S3 s) { return V3{s.c01, s.c11, s.c12}; }
static inline V3 s3_row2(S3 s) { return V3{s.c02, s.c12, s.c22}; }
static inline V3 s3_mul_vec3(S3 s, V3 v) { return add(add(scale(s3_row0(s), v.x), scale(s3_row1(s), v.y)), scale(s3_row2(s), v.z)); }
static inline S3 s3_scale(S3 s, float k) { return S3{s.c00 * k, s.c01 * k, s.c02 * k, s.c11 * k, s.c12 * k, s.c22 * k}; }
static inline M3 s3_mul_mat3(S3 s, M3 m) { return M3{s3_mul_vec3(s, m.c0), s3_mul_vec3(s, m.c1), s3_mul_vec3(s, m.c2)}; }
static inline S3 s3_congruence(S3 s, M3 m) {
    const V3 sr0 = s3_mul_vec3(s, row0(m)), sr1 = s3_mul_vec3(s, row1(m)), sr2 = s3_mul_vec3(s, row2(m));
    return S3{dot(row0(m), sr0), dot(row0(m), sr1), dot(row0(m), sr2), dot(row1(m), sr1), dot(row1(m), sr2), dot(row2(m), sr2)};
}
static inline S3 s3_tcongruence(S3 s, M3 m) {
    const V3 sc0 = s3_mul_vec3(s, m.c0), sc1 = s3_mul_vec3(s, m.c1), sc2 = s3_mul_vec3(s, m.c2);
    return S3{dot(m.c0, sc0), dot(m.c0, sc1), dot(m.c0, sc2), dot(m.c1, sc1), dot(m.c1, sc2), dot(m.c2, sc2)};
}

// 2x3 column-major.
struct M23 { V2 c0, c1, c2; };
static inline V2 m23_mul_vec3(M23 m, V3 v) { return add2(add2(scale2(m.c0, v.x), scale2(m.c1, v.y)), scale2(m.c2, v.z)); }
static inline M23 m23_mul_mat3(M23 m, M3 n) { return M23{m23_mul_vec3(m, n.c0), m23_mul_vec3(m, n.c1), m23_mul_vec3(m, n.c2)}; }
static inline V3 m23_row0(M23 m) { return V3{m.c0.x, m.c1.x, m.c2.x}; }
static inline V3 m23_row1(M23 m) { return V3{m.c0.y, m.c1.y, m.c2.y}; }
static inline S3 m23_tcongruence_s2(M23 m, S2 s) {
    const V2 sc0 = s2_mul_vec2(s, m.c0), sc1 = s2_mul_vec2(s, m.c1), sc2 = s2_mul_vec2(s, m.c2);
    return S3{dot2(m.c0, sc0), dot2(m.c0, sc1), dot2(m.c0, sc2), dot2(m.c1, sc1), dot2(m.c1, sc2), dot2(m.c2, sc2)};
}
static inline S2 m23_gram(M23 m) {
    const float c00 = (m.c0.x * m.c0.x + m.c1.x * m.c1.x) + m.c2.x * m.c2.x;
    const float c01 = (m.c0.x * m.c0.y + m.c1.x * m.c1.y) + m.c2.x * m.c2.y;
    const float c11 = (m.c0.y * m.c0.y + m.c1.y * m.c1.y) + m.c2.y * m.c2.y;
    return S2{c00, c01, c11};
}
static inline M23 s2_mul_m23(S2 s, M23 n) { return M23{s2_mul_vec2(s, n.c0), s2_mul_vec2(s, n.c1), s2_mul_vec2(s, n.c2)}; }

// calc_sigma, crates/splat-train-cube/src/lib.rs:574-579 (tile test form).
static inline float calc_sigma(float px, float py, S2 c, float x, float y) {
    const float dx = px - x;
    const float dy = py - y;
    return 0.5f * (c.c00 * dx * dx + c.c11 * dy * dy) + c.c01 * dx * dy;
}

} // namespace orc
