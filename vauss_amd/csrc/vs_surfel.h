// vs_surfel.h -- surfel (2DGS) geometry shared by the projection, the raster
// kernels and the projection backward.
//
// Restates crates/splat-train-render/src/kernels/helpers.rs:56-69,316-423
// and the per-pixel ray-plane sample of kernels/rasterize.rs:267-301.  A
// surfel is the disk spanned by its first two scaled axes; M = K [a b c] with
// a = s_u W R e0, b = s_v W R e1, c = the view-space centre maps (u, v, 1) on
// the disk to the screen.  Surfels are pinhole-only.
#pragma once
#include "vs_device.h"
#include "vs_camera.h"

namespace vs {

constexpr int SURFEL_MODEL = 16;            // the MODEL template value of surfel projection (pinhole camera)
constexpr float SURFEL_NEAR = 0.01f;         // kernels/helpers.rs:66-68
constexpr int SURFEL_GRADS = 17;             // M rows (9), normal (3), rgb (3), alpha, refine

struct SurfelProj { F3 r0, r1, r2; float bin_x, bin_y; S2 bin_conic; bool valid; };

// surfel_project (helpers.rs:331-412): M's rows and the screen ellipse that
// covers the opacity cutoff footprint u^2 + v^2 <= 2 power (dual conic
// M diag(k2, k2, -1) M^T) grown by the low-pass disk of radius sqrt(power);
// invalid when the footprint touches the camera plane.
VS_DEV SurfelProj surfel_project(F3 sc, Qt q, F3 mc, const vs_camera& u, float power) {
    const M3 rot = mul(view_rot(u), to_mat3(q));
    const F3 a = rot.c0 * sc.x, b = rot.c1 * sc.y;
    const F3 ka{u.fx * a.x + u.cx * a.z, u.fy * a.y + u.cy * a.z, a.z};
    const F3 kb{u.fx * b.x + u.cx * b.z, u.fy * b.y + u.cy * b.z, b.z};
    const F3 kc{u.fx * mc.x + u.cx * mc.z, u.fy * mc.y + u.cy * mc.z, mc.z};
    SurfelProj p;
    p.r0 = F3{ka.x, kb.x, kc.x};
    p.r1 = F3{ka.y, kb.y, kc.y};
    p.r2 = F3{ka.z, kb.z, kc.z};
    const F3 r0 = p.r0, r1 = p.r1, r2 = p.r2;
    const float k2 = 2.0f * power;
    const float d00 = k2 * (r0.x * r0.x + r0.y * r0.y) - r0.z * r0.z;
    const float d01 = k2 * (r0.x * r1.x + r0.y * r1.y) - r0.z * r1.z;
    const float d11 = k2 * (r1.x * r1.x + r1.y * r1.y) - r1.z * r1.z;
    const float d02 = k2 * (r0.x * r2.x + r0.y * r2.y) - r0.z * r2.z;
    const float d12 = k2 * (r1.x * r2.x + r1.y * r2.y) - r1.z * r2.z;
    const float d22 = k2 * (r2.x * r2.x + r2.y * r2.y) - r2.z * r2.z;
    const float n = -d22;
    const bool front = n > 1.0e-12f;
    const float inv_n = front ? 1.0f / n : 0.0f;
    const float x0 = -d02 * inv_n, y0 = -d12 * inv_n;
    const float s00 = d00 * inv_n + x0 * x0, s01 = d01 * inv_n + x0 * y0, s11 = d11 * inv_n + y0 * y0;
    const float r2f = mx(power, 0.0f);
    const float half_tr = mx(0.5f * (s00 + s11), 1.0e-12f);
    // t = mean semi-axis / filter radius makes the Minkowski bound tight for a circle
    const float t = clampf(__builtin_sqrtf(half_tr / mx(r2f, 1.0e-12f)), 1.0e-3f, 1.0e3f);
    const float ga = 1.0f + 1.0f / t, gb = (1.0f + t) * r2f;
    const S2 grown{ga * s00 + gb, ga * s01, ga * s11 + gb};
    const float det = grown.c00 * grown.c11 - grown.c01 * grown.c01;
    const S2 inv = inverse(grown);
    p.bin_conic = S2{inv.c00 * k2, inv.c01 * k2, inv.c11 * k2};
    p.bin_x = x0;
    p.bin_y = y0;
    p.valid = front && det > 0.0f && finite(x0) && finite(y0) && finite(p.bin_conic);
    return p;
}

// surfel_normal (helpers.rs:414-419): the rotated local +Z, facing the camera.
VS_DEV F3 surfel_normal(Qt q, F3 mc, const vs_camera& u) {
    const F3 n = mul(view_rot(u), to_mat3(q)).c2;
    return n * (dot(n, mc) > 0.0f ? -1.0f : 1.0f);
}

// The pixel ray's sample (rasterize.rs:267-301): h_u = M0 - x M2,
// h_v = M1 - y M2, q = h_u x h_v, (u, v) = (q.x, q.y) / q.z, depth
// z = M2 . (u, v, 1); the low-pass offsets from the projected centre; sigma =
// min(u^2 + v^2, 2 |pixel - centre|^2) / 2.  `m` is the staged row: M rows
// (m0.xyzw, m1.xyzw, m2.x), centre (m2.yz), normal (m2.w, m3.xy); `smax`
// (m3.z) bounds the footprint.  A pixel whose two sigma candidates both
// certainly exceed smax (u^2 + v^2 tested as q.x^2 + q.y^2 against
// 2 smax q.z^2 with a 2e-4 margin, far above the few ulp of the divided
// form) comes back invalid before the divisions: such a pair has alpha below
// every cutoff, so skipping it changes no result.
struct SurfelHit { float hux, huy, huz, hvx, hvy, hvz, qz, rq, su, sv, s3d, z, dxs, dys, s2d, sigma; bool valid; };
// EARLY: a pixel far outside both the plane disk and the low-pass disk
// returns at once (invalid, the other fields unset); otherwise every field is
// computed and such a pixel is marked invalid all the same.  REFINED: 1 / q.z
// from div_cr (the same bits as the division; cheaper where the caller's
// scalar unit has room for its range branch: the backward's replay).
template <bool EARLY = true, bool REFINED = false>
VS_DEV SurfelHit surfel_hit(float4 m0, float4 m1, float4 m2, float smax, float px, float py) {
    // Fused multiply-adds where written (the oracle fuses the same ones; each
    // rounds once where the unfused form rounded twice, so the culling's
    // rounding bounds on q still hold).
    SurfelHit h;
    const float m20 = m1.z, m21 = m1.w, m22 = m2.x;
    h.hux = __builtin_fmaf(-px, m20, m0.x); h.huy = __builtin_fmaf(-px, m21, m0.y); h.huz = __builtin_fmaf(-px, m22, m0.z);
    h.hvx = __builtin_fmaf(-py, m20, m0.w); h.hvy = __builtin_fmaf(-py, m21, m1.x); h.hvz = __builtin_fmaf(-py, m22, m1.y);
    const float qx = __builtin_fmaf(h.huy, h.hvz, -(h.huz * h.hvy));
    const float qy = __builtin_fmaf(h.huz, h.hvx, -(h.hux * h.hvz));
    h.qz = __builtin_fmaf(h.hux, h.hvy, -(h.huy * h.hvx));
    h.dxs = px - m2.y;
    h.dys = py - m2.z;
    h.s2d = 2.0f * __builtin_fmaf(h.dxs, h.dxs, h.dys * h.dys);
    h.valid = false;
    const bool far = 0.5f * h.s2d > smax && __builtin_fmaf(qx, qx, qy * qy) > (2.0004f * smax) * (h.qz * h.qz);
    if (EARLY && far) return h;
    // the quotients as products with the correctly rounded 1 / q.z (the oracle's form)
    h.rq = REFINED ? div_cr(1.0f, h.qz) : 1.0f / h.qz;
    h.su = qx * h.rq;
    h.sv = qy * h.rq;
    h.s3d = __builtin_fmaf(h.su, h.su, h.sv * h.sv);
    h.z = __builtin_fmaf(m20, h.su, __builtin_fmaf(m21, h.sv, m22));
    h.sigma = 0.5f * mn(h.s3d, h.s2d);
    h.valid = !far && finite(h.z) && h.z >= SURFEL_NEAR;
    return h;
}

}  // namespace vs
