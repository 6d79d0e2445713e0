// vs_device.h -- device math shared by the gfx950 kernels.
//
// Build contract: every translation unit is compiled with -ffp-contract=off,
// so a multiply-add is fused only where __builtin_fmaf is written.  f32
// division and sqrt are the correctly-rounded sequences hipcc emits by
// default, f32 denormals are IEEE.  Together with the transcendentals below
// this makes projection, tile binning, key order and compositing reproducible
// bit for bit by any IEEE-754 implementation of the same operation sequence.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

#define VS_DEV __device__ __forceinline__

namespace vs {

constexpr uint32_t TILE_W = 16;                 // kernels/helpers.rs:15
constexpr uint32_t TILE_PIX = TILE_W * TILE_W;  // kernels/helpers.rs:16
constexpr float ALPHA_MID = 1.0f / 255.0f;      // kernels/helpers.rs:23
constexpr float ALPHA_BAND = 1.0e-3f;           // kernels/helpers.rs:24
constexpr float T_STOP = 1.0e-4f;               // kernels/rasterize.rs:323
constexpr float ALPHA_CAP = 0.999f;             // kernels/rasterize.rs:313

VS_DEV uint32_t as_u(float x) { return __float_as_uint(x); }
VS_DEV float as_f(uint32_t u) { return __uint_as_float(u); }
VS_DEV bool finite(float x) { return ((as_u(x) >> 23) & 0xFFu) != 0xFFu; }
// IEEE binary16 <-> f32: widening is exact; narrowing rounds to nearest even
// (f16 subnormals kept, overflow to infinity).
VS_DEV float h2f(uint16_t b) { return (float)__builtin_bit_cast(_Float16, b); }
VS_DEV uint16_t f2h(float f) { return __builtin_bit_cast(uint16_t, (_Float16)f); }

// Min/max/clamp with the semantics of Rust's f32::min/max on NaN (return
// the other operand), written out so the result never depends on the
// target's min/max NaN convention.
VS_DEV float mn(float a, float b) { return (a < b) ? a : ((b == b) ? b : a); }
VS_DEV float mx(float a, float b) { return (a > b) ? a : ((b == b) ? b : a); }
VS_DEV float clampf(float v, float lo, float hi) { return mn(mx(v, lo), hi); }

// ---- transcendentals --------------------------------------------------------
// exp: n = rint(x log2 e); r = x - n ln2 in two fma steps (Cody-Waite split
// 0.693145751953125 + 1.42860677e-06); e^r = 1 + (r + r^2 q(r)) with q of
// degree 4 fitted by least squares on [-ln2/2, ln2/2]; result ldexp(p, n).
// x < -87.33654 -> 0 (results never subnormal), x > 88.72283 -> +inf.
VS_DEV float expf_c(float x) {
    if (x != x) return x;
    if (x > 88.72283f) return __builtin_inff();
    if (x < -87.33654f) return 0.0f;
    const float n = __builtin_rintf(x * 1.44269502f);
    float r = __builtin_fmaf(-n, 0.693145751953125f, x);
    r = __builtin_fmaf(-n, 1.42860677e-06f, r);
    float q = __builtin_fmaf(0.00137514074f, r, 0.00836891588f);
    q = __builtin_fmaf(q, r, 0.0416695327f);
    q = __builtin_fmaf(q, r, 0.166665182f);
    q = __builtin_fmaf(q, r, 0.499999881f);
    const float r2 = r * r;
    const float p = __builtin_fmaf(r2, q, r) + 1.0f;
    return __builtin_ldexpf(p, (int)n);
}

// 2^x for the compositing loops, whose argument is -sigma in base-2 units
// (the conic is staged pre-scaled by LOG2E_F): the hardware's v_exp_f32, one
// transcendental instruction (the degree-5 polynomial it replaced took nine
// VALU instructions per pixel and splat).  On [-126, 0] it is within 1 ulp of
// 2^x; below -126 it returns less than 2^-126 (or 0), so opacity x G stays
// under every cutoff (1/255 - 5e-4 at the lowest) and the pair is rejected.
// A NaN argument (a NaN sigma) gives NaN, and the sigma >= 0 test rejects the
// pair.  vs_compositing_exp2 returns this function's values for checking.
constexpr float LOG2E_F = 1.44269502f;
VS_DEV float comp_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// a / b with the IEEE division's result, in six instructions for the
// divisors that matter: for 2^-100 <= |b| <= 2^100 the hardware reciprocal
// (1 ulp), one Newton step on it and one remainder correction of a times it
// (Markstein's sequence) give the correctly rounded quotient, for a = 1 and
// a = 0.2 at every such b (all 2^32 bit patterns are compared with the
// division by vs_raster_division_mismatches); any other b takes the
// division itself.  The surfel backward's replay takes the ray-plane
// sample's 1 / q.z from it (the forward divides: the range branch costs its
// busier scalar unit more than the division).
VS_DEV float div_cr(float a, float b) {
    const float ab = __builtin_fabsf(b);
    if (!(ab >= 0x1p-100f && ab <= 0x1p100f)) return a / b;
    const float r0 = __builtin_amdgcn_rcpf(b);
    const float r1 = __builtin_fmaf(__builtin_fmaf(-b, r0, 1.0f), r0, r0);
    const float q0 = a * r1;
    return __builtin_fmaf(__builtin_fmaf(-b, q0, a), r1, q0);
}

// log: m = x 2^-e in [sqrt(1/2), sqrt(2)), s = (m-1)/(m+1),
// ln m = 2s + s^3 (2/3 + 2/5 s^2 + 2/7 s^4 + 2/9 s^6), ln x = e ln2 + ln m.
VS_DEV float logf_c(float x) {
    if (x != x) return x;
    if (x < 0.0f) return __builtin_nanf("");
    if (x == 0.0f) return -__builtin_inff();
    if (x == __builtin_inff()) return x;
    int e = 0;
    uint32_t b = as_u(x);
    if (b < 0x00800000u) { x = x * 8388608.0f; b = as_u(x); e = -23; }
    e += (int)(b >> 23) - 127;
    float m = as_f((b & 0x007FFFFFu) | 0x3F800000u);
    if (m > 1.41421354f) { m = m * 0.5f; e += 1; }
    const float f = m - 1.0f;
    const float s = f / (2.0f + f);
    const float s2 = s * s;
    float R = __builtin_fmaf(s2, 0.222222224f, 0.285714298f);
    R = __builtin_fmaf(R, s2, 0.400000006f);
    R = __builtin_fmaf(R, s2, 0.666666687f);
    R = R * s2;
    const float lnm = __builtin_fmaf(s, R, s + s);
    const float ef = (float)e;
    return __builtin_fmaf(ef, 0.693145751953125f, __builtin_fmaf(ef, 1.42860677e-06f, lnm));
}

// atan2: a = min(|x|,|y|)/max(|x|,|y|); a > tan(pi/8) -> t = (a-1)/(a+1)
// around pi/4; atan t = t + t^3 P(t^2) with P of degree 4 fitted by least
// squares on [0, tan(pi/8)]; octant and sign fixups with pi/2, pi in
// hi + lo parts.
VS_DEV float atan2f_c(float y, float x) {
    if (x != x || y != y) return x + y;
    const float ax = __builtin_fabsf(x), ay = __builtin_fabsf(y);
    float r;
    const float inf = __builtin_inff();
    if (ax == inf || ay == inf) {
        if (ax == inf && ay == inf) r = (x < 0.0f) ? 2.35619449f : 0.785398163f;
        else if (ax == inf) r = (x < 0.0f) ? 3.14159274f : 0.0f;
        else r = 1.57079637f;
        return __builtin_copysignf(r, y);
    }
    if (ax == 0.0f && ay == 0.0f) {
        r = __builtin_signbit(x) ? 3.14159274f : 0.0f;
        return __builtin_copysignf(r, y);
    }
    const float hi = (ax > ay) ? ax : ay;
    const float lo = (ax > ay) ? ay : ax;
    const float a = lo / hi;
    float t, base;
    if (a > 0.414213568f) { t = (a - 1.0f) / (a + 1.0f); base = 0.785398163f; }
    else { t = a; base = 0.0f; }
    const float t2 = t * t;
    float P = __builtin_fmaf(-0.0609764382f, t2, 0.106022187f);
    P = __builtin_fmaf(P, t2, -0.142448023f);
    P = __builtin_fmaf(P, t2, 0.199985489f);
    P = __builtin_fmaf(P, t2, -0.333333164f);
    const float at = __builtin_fmaf(t * t2, P, t);
    r = base + at;
    if (ay > ax) r = (1.57079637f - r) + (-4.37113883e-08f);
    if (x < 0.0f) r = (3.14159274f - r) + (-8.74227766e-08f);
    return __builtin_copysignf(r, y);
}

// sin and cos of one argument: j = rint(x 2/pi); r = x - j pi/2 in three fma
// steps (pi/2 split into three f32 parts), |r| <= pi/4 plus rounding; Taylor
// polynomials of sin r (through r^11) and cos r (through r^12) in Horner
// form; the quadrant j mod 4 picks and signs them.  Non-finite x -> NaN.
VS_DEV void sincosf_c(float x, float& s, float& c) {
    if (!finite(x)) { s = c = __builtin_nanf(""); return; }
    const float j = __builtin_rintf(x * 0x1.45f306p-1f);
    float r = __builtin_fmaf(-j, 0x1.921fb6p+0f, x);
    r = __builtin_fmaf(-j, -0x1.777a5cp-25f, r);
    r = __builtin_fmaf(-j, -0x1.ee59dap-50f, r);
    const float z = r * r;
    float ps = __builtin_fmaf(z, -0x1.ae6456p-26f, 0x1.71de3ap-19f);
    ps = __builtin_fmaf(ps, z, -0x1.a01a02p-13f);
    ps = __builtin_fmaf(ps, z, 0x1.111112p-7f);
    ps = __builtin_fmaf(ps, z, -0x1.555556p-3f);
    const float sr = __builtin_fmaf(r * z, ps, r);
    float pc = __builtin_fmaf(z, 0x1.1eed8ep-29f, -0x1.27e4fcp-22f);
    pc = __builtin_fmaf(pc, z, 0x1.a01a02p-16f);
    pc = __builtin_fmaf(pc, z, -0x1.6c16c2p-10f);
    pc = __builtin_fmaf(pc, z, 0x1.555556p-5f);
    pc = __builtin_fmaf(pc, z, -0.5f);
    const float cr = __builtin_fmaf(z, pc, 1.0f);
    const int q = (int)(j - 4.0f * __builtin_floorf(j * 0.25f));
    s = (q == 0) ? sr : (q == 1) ? cr : (q == 2) ? -sr : -cr;
    c = (q == 0) ? cr : (q == 1) ? -sr : (q == 2) ? -cr : sr;
}

// tanh: |x| < 0.5625 -> x + x^3 P(x^2), P the Taylor series of (tanh x - x)/x^3
// through x^16; otherwise 1 - 2 / (exp(2|x|) + 1) with the sign of x (1 once
// exp overflows); signed zeros pass through.
VS_DEV float tanhf_c(float x) {
    if (x != x || x == 0.0f) return x;
    const float a = __builtin_fabsf(x);
    if (a < 0.5625f) {
        const float z = x * x;
        float p = __builtin_fmaf(z, -0x1.f57d78p-13f, 0x1.355824p-11f);
        p = __builtin_fmaf(p, z, -0x1.7da364p-10f);
        p = __builtin_fmaf(p, z, 0x1.d6d3d0p-9f);
        p = __builtin_fmaf(p, z, -0x1.226e36p-7f);
        p = __builtin_fmaf(p, z, 0x1.664f48p-6f);
        p = __builtin_fmaf(p, z, -0x1.ba1ba2p-5f);
        p = __builtin_fmaf(p, z, 0x1.111112p-3f);
        p = __builtin_fmaf(p, z, -0x1.555556p-2f);
        return __builtin_fmaf(x * z, p, x);
    }
    const float t = 1.0f - 2.0f / (expf_c(2.0f * a) + 1.0f);
    return __builtin_copysignf(t, x);
}

// crates/splat-train-cube/src/lib.rs:561-564
VS_DEV float sigmoid(float x) { return 1.0f / (1.0f + expf_c(-x)); }

// ---- small linear algebra (crates/splat-train-cube/src/lib.rs:40-559) ---------
struct F3 { float x, y, z; };
struct F2 { float x, y; };
struct Qt { float w, x, y, z; };
struct M3 { F3 c0, c1, c2; };            // column-major
struct S2 { float c00, c01, c11; };
struct S3 { float c00, c01, c02, c11, c12, c22; };
struct M23 { F2 c0, c1, c2; };           // 2x3 column-major

VS_DEV F3 f3(float x, float y, float z) { return F3{x, y, z}; }
VS_DEV F3 operator+(F3 a, F3 b) { return F3{a.x + b.x, a.y + b.y, a.z + b.z}; }
VS_DEV F3 operator-(F3 a, F3 b) { return F3{a.x - b.x, a.y - b.y, a.z - b.z}; }
VS_DEV F3 operator*(F3 a, float s) { return F3{a.x * s, a.y * s, a.z * s}; }
// Vec3A::dot adds a zero padding lane last.
VS_DEV float dot(F3 a, F3 b) { return ((a.x * b.x + a.y * b.y) + a.z * b.z) + 0.0f; }
VS_DEV float length(F3 a) { return __builtin_sqrtf(dot(a, a)); }
VS_DEV F3 normalize(F3 a) { return a * (1.0f / length(a)); }
VS_DEV bool finite(F3 a) { return finite(a.x) && finite(a.y) && finite(a.z); }

VS_DEV F2 operator+(F2 a, F2 b) { return F2{a.x + b.x, a.y + b.y}; }
VS_DEV F2 operator*(F2 a, float s) { return F2{a.x * s, a.y * s}; }
VS_DEV float dot(F2 a, F2 b) { return a.x * b.x + a.y * b.y; }

VS_DEV float dot(Qt a, Qt b) { return ((a.w * b.w + a.x * b.x) + a.y * b.y) + a.z * b.z; }
VS_DEV Qt operator*(Qt a, float s) { return Qt{a.w * s, a.x * s, a.y * s, a.z * s}; }
VS_DEV Qt normalize(Qt a) { return a * (1.0f / __builtin_sqrtf(dot(a, a))); }

VS_DEV M3 to_mat3(Qt q) {
    const float x2 = q.x * q.x, y2 = q.y * q.y, z2 = q.z * q.z;
    const float xy = q.x * q.y, xz = q.x * q.z, yz = q.y * q.z;
    const float wx = q.w * q.x, wy = q.w * q.y, wz = q.w * q.z;
    return M3{F3{1.0f - 2.0f * (y2 + z2), 2.0f * (xy + wz), 2.0f * (xz - wy)},
              F3{2.0f * (xy - wz), 1.0f - 2.0f * (x2 + z2), 2.0f * (yz + wx)},
              F3{2.0f * (xz + wy), 2.0f * (yz - wx), 1.0f - 2.0f * (x2 + y2)}};
}
VS_DEV F3 mul(M3 m, F3 v) { return (m.c0 * v.x + m.c1 * v.y) + m.c2 * v.z; }
VS_DEV F3 tmul(M3 m, F3 v) { return F3{dot(m.c0, v), dot(m.c1, v), dot(m.c2, v)}; }
VS_DEV M3 mul(M3 a, M3 b) { return M3{mul(a, b.c0), mul(a, b.c1), mul(a, b.c2)}; }
VS_DEV M3 mul_diag(M3 a, F3 s) { return M3{a.c0 * s.x, a.c1 * s.y, a.c2 * s.z}; }
VS_DEV F3 row0(M3 m) { return F3{m.c0.x, m.c1.x, m.c2.x}; }
VS_DEV F3 row1(M3 m) { return F3{m.c0.y, m.c1.y, m.c2.y}; }
VS_DEV F3 row2(M3 m) { return F3{m.c0.z, m.c1.z, m.c2.z}; }
VS_DEV S3 outer_self(M3 m) {
    const F3 r0 = row0(m), r1 = row1(m), r2 = row2(m);
    return S3{dot(r0, r0), dot(r0, r1), dot(r0, r2), dot(r1, r1), dot(r1, r2), dot(r2, r2)};
}

VS_DEV F2 mul(S2 s, F2 v) { return F2{s.c00, s.c01} * v.x + F2{s.c01, s.c11} * v.y; }
VS_DEV S2 scale(S2 s, float k) { return S2{s.c00 * k, s.c01 * k, s.c11 * k}; }
VS_DEV float max_abs(S2 s) { return mx(mx(__builtin_fabsf(s.c00), __builtin_fabsf(s.c11)), __builtin_fabsf(s.c01)); }
VS_DEV S2 inverse(S2 s) {
    const float det = s.c00 * s.c11 - s.c01 * s.c01;
    const float inv_det = (det > 0.0f) ? 1.0f / det : 0.0f;
    return S2{s.c11 * inv_det, -s.c01 * inv_det, s.c00 * inv_det};
}
VS_DEV bool finite(S2 s) { return finite(s.c00) && finite(s.c11) && finite(s.c01); }

VS_DEV F3 srow0(S3 s) { return F3{s.c00, s.c01, s.c02}; }
VS_DEV F3 srow1(S3 s) { return F3{s.c01, s.c11, s.c12}; }
VS_DEV F3 srow2(S3 s) { return F3{s.c02, s.c12, s.c22}; }
VS_DEV F3 mul(S3 s, F3 v) { return (srow0(s) * v.x + srow1(s) * v.y) + srow2(s) * v.z; }
VS_DEV S3 scale(S3 s, float k) { return S3{s.c00 * k, s.c01 * k, s.c02 * k, s.c11 * k, s.c12 * k, s.c22 * k}; }
VS_DEV M3 mul(S3 s, M3 m) { return M3{mul(s, m.c0), mul(s, m.c1), mul(s, m.c2)}; }
VS_DEV S3 congruence(S3 s, M3 m) {   // m s m^T
    const F3 a = mul(s, row0(m)), b = mul(s, row1(m)), c = mul(s, row2(m));
    return S3{dot(row0(m), a), dot(row0(m), b), dot(row0(m), c), dot(row1(m), b), dot(row1(m), c), dot(row2(m), c)};
}
VS_DEV S3 tcongruence(S3 s, M3 m) {  // m^T s m
    const F3 a = mul(s, m.c0), b = mul(s, m.c1), c = mul(s, m.c2);
    return S3{dot(m.c0, a), dot(m.c0, b), dot(m.c0, c), dot(m.c1, b), dot(m.c1, c), dot(m.c2, c)};
}

VS_DEV F2 mul(M23 m, F3 v) { return (m.c0 * v.x + m.c1 * v.y) + m.c2 * v.z; }
VS_DEV M23 mul(M23 m, M3 n) { return M23{mul(m, n.c0), mul(m, n.c1), mul(m, n.c2)}; }
VS_DEV F3 mrow0(M23 m) { return F3{m.c0.x, m.c1.x, m.c2.x}; }
VS_DEV F3 mrow1(M23 m) { return F3{m.c0.y, m.c1.y, m.c2.y}; }
VS_DEV S3 tcongruence(M23 m, S2 s) {  // m^T s m
    const F2 a = mul(s, m.c0), b = mul(s, m.c1), c = mul(s, m.c2);
    return S3{dot(m.c0, a), dot(m.c0, b), dot(m.c0, c), dot(m.c1, b), dot(m.c1, c), dot(m.c2, c)};
}
VS_DEV S2 gram(M23 m) {
    return S2{(m.c0.x * m.c0.x + m.c1.x * m.c1.x) + m.c2.x * m.c2.x,
              (m.c0.x * m.c0.y + m.c1.x * m.c1.y) + m.c2.x * m.c2.y,
              (m.c0.y * m.c0.y + m.c1.y * m.c1.y) + m.c2.y * m.c2.y};
}
VS_DEV M23 mul(S2 s, M23 n) { return M23{mul(s, n.c0), mul(s, n.c1), mul(s, n.c2)}; }

// calc_sigma in the tile-test form, crates/splat-train-cube/src/lib.rs:574-579.
VS_DEV float calc_sigma(float px, float py, S2 c, float x, float y) {
    const float dx = px - x;
    const float dy = py - y;
    return 0.5f * (c.c00 * dx * dx + c.c11 * dy * dy) + c.c01 * dx * dy;
}

// Compositing form of sigma (contract), in base-2 units with the staged
// A = (c00/2) log2 e, B = c01 log2 e, C = (c11/2) log2 e.
VS_DEV float raster_sigma(float A, float B, float C, float dx, float dy) {
    return __builtin_fmaf(__builtin_fmaf(A, dx, B * dy), dx, (C * dy) * dy);
}

// kernels/helpers.rs:26-47
VS_DEV float cutoff_weight(float alpha) {
    const float t = clampf((alpha - (ALPHA_MID - 0.5f * ALPHA_BAND)) / ALPHA_BAND, 0.0f, 1.0f);
    return t * t * (3.0f - 2.0f * t);
}
VS_DEV float cutoff_weight_deriv(float alpha) {
    const float lo = ALPHA_MID - 0.5f * ALPHA_BAND, hi = ALPHA_MID + 0.5f * ALPHA_BAND;
    const float t = (alpha - lo) / ALPHA_BAND;
    return (alpha > lo && alpha < hi) ? (6.0f * t - 6.0f * t * t) / ALPHA_BAND : 0.0f;
}

// Rust float -> u32 `as` cast (truncate, saturate, NaN -> 0).
VS_DEV uint32_t f2u_sat(float v) {
    if (!(v > 0.0f)) return 0u;
    if (v >= 4294967296.0f) return 0xFFFFFFFFu;
    return (uint32_t)v;
}

} // namespace vs
