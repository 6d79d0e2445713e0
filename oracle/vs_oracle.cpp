// vs_oracle.cpp -- CPU restatement of the reference Gaussian-splat render path.
//
// TEST INFRASTRUCTURE ONLY.  Loaded by tests/, __graft_entry__.smoke() and the
// cpu_baseline leg of bench.py as the checker; the product never links it.
//
// Each stage cites the reference function it restates (paths relative to
// crates/splat-train-render/src unless they name another crate).  The stage
// order follows render.rs:401-979 (`render_cube`):
//   project_forward (cull + count, kernels/project_forward.rs:26-261)
//   project_visible (kernels/project_visible.rs:97-174, aux 182-312)
//   depth sort      (render.rs:689-694: stable, raw f32 bits)
//   count scan      (kernels/map_gaussians.rs:215-269)
//   map/emit        (kernels/map_gaussians.rs:23-174)
//   tile sort       (render.rs:792-794: stable by tile id)
//   tile offsets    (get_tile_offset.rs:11-59)
//   rasterize       (kernels/rasterize.rs:109-420)
//   raster VJP      (bwd/kernels/rasterize_backwards_planes.rs:112-682)
//   projection VJP  (bwd/kernels/project_backwards.rs:132-424)
//
// The reference compacts visible splats with an atomic counter, so its
// compaction order (and the order of exactly tied depths) is whatever the
// atomics produced.  The oracle fixes that order to increasing global id, one
// of the orders the reference can produce; every tie below is therefore
// broken by global id.
//
// Arithmetic contract shared with the GPU kernels (both sides implement it
// independently):
//  * projection-side math: the reference's operation order, no contraction;
//  * exp/log/atan2: the portable evaluations of or_math.h;
//  * compositing: dx = px - x, dy = py - y, and sigma in base-2 units
//      s2 = fma(fma(A, dx, B*dy), dx, (C*dy)*dy),
//      A = (c00/2) L, B = c01 L, C = (c11/2) L, L = log2(e) in f32
//    (the reference's 0.5(c00 dx^2 + c11 dy^2) + c01 dx dy times log2 e, up to
//    rounding and the contraction its shader compiler is also free to apply;
//    s2 >= 0 exactly when sigma >= 0), G = 2^(-s2) (comp_exp2_c below: the
//    GPU's exp2 instruction from an installed table of its values, else
//    exp2n of or_math.h), alpha = min(0.999, opac G), T' = T (1 - alpha),
//    colour += max(c,0) * (alpha T) as an fma, final = fma(T, bg, colour).
//    Surfels: G = 2^(-(sigma L)) of their ray-plane sigma.
#include "vs_oracle.h"
#include "or_math.h"

#include <vector>
#include <numeric>
#include <algorithm>
#include <cstdlib>
#include <cstring>
#include <memory>
#ifdef _OPENMP
#include <omp.h>
#endif

using namespace orc;

namespace {

// G = 2^x of the compositing loops.  The GPU kernels take it from the
// hardware's exp2 instruction, whose bits no CPU routine reproduces; a caller
// that holds that instruction's values for a range of f32 bit patterns
// (normally every x from -0 down to -128) installs them with
// or_set_comp_exp2_table and the loops composite with the same G.  Outside
// the table, and with none installed, G is exp2n_c (or_math.h).  That covers
// x < -128, where both give less than 2^-127 and every cutoff rejects the
// pair; a NaN x, whose sigma the sigma >= 0 test rejects; and +0, which takes
// the value of -0 (both are 1).
const float* g_exp2_tab = nullptr;
uint32_t g_exp2_first = 0;
uint64_t g_exp2_count = 0;
inline float comp_exp2_c(float x) {
    if (g_exp2_tab) {
        uint32_t b;
        std::memcpy(&b, &x, 4);
        if (b == 0u) b = 0x80000000u;
        if (b >= g_exp2_first && (uint64_t)(b - g_exp2_first) < g_exp2_count) return g_exp2_tab[b - g_exp2_first];
    }
    return exp2n_c(x);
}

constexpr uint32_t TILE_W = 16;                 // kernels/helpers.rs:15-16
constexpr float ALPHA_CUTOFF_MID = 1.0f / 255.0f;   // kernels/helpers.rs:23
constexpr float ALPHA_CUTOFF_BAND = 1.0e-3f;        // kernels/helpers.rs:24
constexpr float DIST_NEAR = 0.2f, DIST_FAR = 100.0f; // kernels/helpers.rs:93-94

// kernels/helpers.rs:26-47
float alpha_cutoff_weight(float alpha) {
    const float t = clampf((alpha - (ALPHA_CUTOFF_MID - 0.5f * ALPHA_CUTOFF_BAND)) / ALPHA_CUTOFF_BAND, 0.0f, 1.0f);
    return t * t * (3.0f - 2.0f * t);
}
float alpha_cutoff_weight_deriv(float alpha) {
    const float low = ALPHA_CUTOFF_MID - 0.5f * ALPHA_CUTOFF_BAND;
    const float high = ALPHA_CUTOFF_MID + 0.5f * ALPHA_CUTOFF_BAND;
    const bool inside = alpha > low && alpha < high;
    const float t = (alpha - low) / ALPHA_CUTOFF_BAND;
    return inside ? (6.0f * t - 6.0f * t * t) / ALPHA_CUTOFF_BAND : 0.0f;
}
// kernels/helpers.rs:100-103
float dist_depth(float z) { return DIST_FAR / (DIST_FAR - DIST_NEAR) * (1.0f - DIST_NEAR / fmax_(z, DIST_NEAR)); }

M3 view_rot(const or_camera& u) {
    return M3{V3{u.viewmat[0], u.viewmat[1], u.viewmat[2]},
              V3{u.viewmat[3], u.viewmat[4], u.viewmat[5]},
              V3{u.viewmat[6], u.viewmat[7], u.viewmat[8]}};
}
V3 view_trans(const or_camera& u) { return V3{u.viewmat[9], u.viewmat[10], u.viewmat[11]}; }
// kernels/helpers.rs:472-475
V3 world_to_cam(V3 mean, const or_camera& u) { return add(mul_vec3(view_rot(u), mean), view_trans(u)); }

// --- camera models -----------------------------------------------------------
// kernels/camera_model/pinhole.rs:165-171
void project_pinhole(V3 p, const or_camera& u, float& ou, float& ov) {
    const float inv_z = 1.0f / p.z;
    ou = u.fx * p.x * inv_z + u.cx;
    ov = u.fy * p.y * inv_z + u.cy;
}
// kernels/camera_model/kannala_brandt_4.rs:18-54
void project_kb4(V3 p, const or_camera& u, float& ou, float& ov) {
    const float x = p.x, y = p.y, z = p.z;
    const float k1 = u.kb4[0], k2 = u.kb4[1], k3 = u.kb4[2], k4 = u.kb4[3];
    const float inv_z = 1.0f / z;
    const float pin_u = u.fx * x * inv_z + u.cx;
    const float pin_v = u.fy * y * inv_z + u.cy;
    const float r = std::sqrt(x * x + y * y);
    const float theta = atan2f_c(r, z);
    const float th2 = theta * theta, th4 = th2 * th2, th6 = th2 * th4, th8 = th4 * th4;
    const float d = theta * (1.0f + k1 * th2 + k2 * th4 + k3 * th6 + k4 * th8);
    const float inv_r = 1.0f / r;
    const float fu = u.fx * (d * x * inv_r) + u.cx;
    const float fv = u.fy * (d * y * inv_r) + u.cy;
    const bool near_axis = r < 1e-6f;
    ou = near_axis ? pin_u : fu;
    ov = near_axis ? pin_v : fv;
}
// kernels/camera_model/thin_prism_fisheye.rs:37-63: N_u, N_v (delta = N / z^2)
// and their (x, y) derivatives, in camera-space x, y.
struct TpPolys { float nu, nv, dnu_dx, dnu_dy, dnv_dx, dnv_dy; };
TpPolys thin_prism_polys(float x, float y, const or_camera& u) {
    const float p1 = u.dist[0], p2 = u.dist[1], sx1 = u.dist[2], sy1 = u.dist[3];
    const float x2 = x * x, y2 = y * y, xy = x * y, r2 = x2 + y2;
    TpPolys t;
    t.nu = 2.0f * p1 * xy + p2 * (3.0f * x2 + y2) + sx1 * r2;
    t.nv = 2.0f * p2 * xy + p1 * (x2 + 3.0f * y2) + sy1 * r2;
    t.dnu_dx = 2.0f * (p1 * y + (3.0f * p2 + sx1) * x);
    t.dnu_dy = 2.0f * (p1 * x + (p2 + sx1) * y);
    t.dnv_dx = 2.0f * (p2 * y + (p1 + sy1) * x);
    t.dnv_dy = 2.0f * (p2 * x + (3.0f * p1 + sy1) * y);
    return t;
}

// kernels/camera_model/radial_tangential_8.rs:23-62
void project_rt8(V3 p, const or_camera& u, float& ou, float& ov) {
    const float k1 = u.dist[0], k2 = u.dist[1], k3 = u.dist[2], k4 = u.dist[3], k5 = u.dist[4], k6 = u.dist[5];
    const float p1 = u.dist[6], p2 = u.dist[7];
    const float xn = p.x / p.z, yn = p.y / p.z;
    const float xn2 = xn * xn, yn2 = yn * yn;
    const float r2 = xn2 + yn2, r4 = r2 * r2, r6 = r4 * r2;
    const float radial = (1.0f + k1 * r2 + k2 * r4 + k3 * r6) / (1.0f + k4 * r2 + k5 * r4 + k6 * r6);
    const float xyn = xn * yn;
    const float xd = xn * radial + 2.0f * p1 * xyn + p2 * (r2 + 2.0f * xn2);
    const float yd = yn * radial + 2.0f * p2 * xyn + p1 * (r2 + 2.0f * yn2);
    ou = u.fx * xd + u.cx;
    ov = u.fy * yd + u.cy;
}
// kernels/camera_model/thin_prism_fisheye.rs:65-82
void project_tpf(V3 p, const or_camera& u, float& ou, float& ov) {
    float ku, kv;
    project_kb4(p, u, ku, kv);
    const float inv_z = 1.0f / p.z, inv_z2 = inv_z * inv_z;
    const TpPolys t = thin_prism_polys(p.x, p.y, u);
    ou = ku + u.fx * t.nu * inv_z2;
    ov = kv + u.fy * t.nv * inv_z2;
}
void project(V3 p, const or_camera& u, float& ou, float& ov) {
    switch (u.model) {
    case OR_MODEL_KB4: project_kb4(p, u, ou, ov); break;
    case OR_MODEL_RT8: project_rt8(p, u, ou, ov); break;
    case OR_MODEL_TPF: project_tpf(p, u, ou, ov); break;
    default: project_pinhole(p, u, ou, ov); break;
    }
}
// kernels/camera_model/pinhole.rs:173-197
M23 jac_pinhole(V3 p, const or_camera& u) {
    const float inv_z = 1.0f / p.z;
    const float dx = u.fx * inv_z;
    const float dy = u.fy * inv_z;
    const float cx = clampf(p.x * inv_z, u.lim_neg_x, u.lim_pos_x);
    const float cy = clampf(p.y * inv_z, u.lim_neg_y, u.lim_pos_y);
    return M23{V2{dx, 0.0f}, V2{0.0f, dy}, V2{-dx * cx, -dy * cy}};
}
// kernels/camera_model/kannala_brandt_4.rs:58-152
M23 jac_kb4(V3 p, const or_camera& u) {
    const float k1 = u.kb4[0], k2 = u.kb4[1], k3 = u.kb4[2], k4 = u.kb4[3];
    const float x = p.x, y = p.y, z = p.z;
    const float inv_z = 1.0f / z;
    const float x2 = x * x, y2 = y * y, xy = x * y;
    const float r2 = x2 + y2;
    const float r = std::sqrt(r2);
    const float inv_r = 1.0f / r;
    const float inv_r3 = inv_r * inv_r * inv_r;
    const float rho2 = r2 + z * z;
    const float inv_rho2 = 1.0f / rho2;
    const float inv_rho2_r = inv_rho2 * inv_r;
    const float theta = atan2f_c(r, z);
    const float th2 = theta * theta, th4 = th2 * th2, th6 = th4 * th2, th8 = th4 * th4;
    const float d = theta * (1.0f + k1 * th2 + k2 * th4 + k3 * th6 + k4 * th8);
    const float dd = 1.0f + 3.0f * k1 * th2 + 5.0f * k2 * th4 + 7.0f * k3 * th6 + 9.0f * k4 * th8;
    const float dth_dx = x * z * inv_rho2_r;
    const float dth_dy = y * z * inv_rho2_r;
    const float dth_dz = -r * inv_rho2;
    const float dd_dx = dd * dth_dx, dd_dy = dd * dth_dy, dd_dz = dd * dth_dz;
    const float xr = x * inv_r;
    const float dxr_dx = y2 * inv_r3;
    const float dxr_dy = -xy * inv_r3;
    const float du_dx = u.fx * (dd_dx * xr + d * dxr_dx);
    const float du_dy = u.fx * (dd_dy * xr + d * dxr_dy);
    const float du_dz = u.fx * (dd_dz * xr);
    const float yr = y * inv_r;
    const float dyr_dx = -xy * inv_r3;
    const float dyr_dy = x2 * inv_r3;
    const float dv_dx = u.fy * (dd_dx * yr + d * dyr_dx);
    const float dv_dy = u.fy * (dd_dy * yr + d * dyr_dy);
    const float dv_dz = u.fy * (dd_dz * yr);
    const bool near_axis = r < 1e-6f;
    const float pdx = u.fx * inv_z, pdy = u.fy * inv_z;
    const float p_du_dz = -pdx * x * inv_z;
    const float p_dv_dz = -pdy * y * inv_z;
    return M23{V2{near_axis ? pdx : du_dx, near_axis ? 0.0f : dv_dx},
               V2{near_axis ? 0.0f : du_dy, near_axis ? pdy : dv_dy},
               V2{near_axis ? p_du_dz : du_dz, near_axis ? p_dv_dz : dv_dz}};
}
// kernels/camera_model/radial_tangential_8.rs:64-149
M23 jac_rt8(V3 p, const or_camera& u) {
    const float k1 = u.dist[0], k2 = u.dist[1], k3 = u.dist[2], k4 = u.dist[3], k5 = u.dist[4], k6 = u.dist[5];
    const float p1 = u.dist[6], p2 = u.dist[7];
    const float z = p.z, inv_z = 1.0f / z, inv_z2 = inv_z * inv_z;
    const float xb = clampf(p.x * inv_z, u.lim_neg_x, u.lim_pos_x);
    const float yb = clampf(p.y * inv_z, u.lim_neg_y, u.lim_pos_y);
    const float rb = std::sqrt(xb * xb + yb * yb);
    const float sc = rb > u.lim_r ? u.lim_r / rb : 1.0f;
    const float xn = xb * sc, yn = yb * sc;
    const float xc = xn * z, yc = yn * z;
    const float r2 = xn * xn + yn * yn, r4 = r2 * r2, r6 = r4 * r2;
    const float N = 1.0f + k1 * r2 + k2 * r4 + k3 * r6;
    const float D = 1.0f + k4 * r2 + k5 * r4 + k6 * r6;
    const float Np = k1 + 2.0f * k2 * r2 + 3.0f * k3 * r4;
    const float Dp = k4 + 2.0f * k5 * r2 + 3.0f * k6 * r4;
    const float iD = 1.0f / D, iD2 = iD * iD;
    const float R0 = N * iD, R1 = (Np * D - N * Dp) * iD2;
    const float a00 = R0 + 2.0f * xn * xn * R1 + 2.0f * p1 * yn + 6.0f * p2 * xn;
    const float a01 = 2.0f * xn * yn * R1 + 2.0f * p1 * xn + 2.0f * p2 * yn;
    const float a10 = a01;
    const float a11 = R0 + 2.0f * yn * yn * R1 + 6.0f * p1 * yn + 2.0f * p2 * xn;
    return M23{V2{u.fx * a00 * inv_z, u.fy * a10 * inv_z},
               V2{u.fx * a01 * inv_z, u.fy * a11 * inv_z},
               V2{-u.fx * (a00 * xc + a01 * yc) * inv_z2, -u.fy * (a10 * xc + a11 * yc) * inv_z2}};
}
// kernels/camera_model/thin_prism_fisheye.rs:84-116
M23 jac_tpf(V3 p, const or_camera& u) {
    const M23 k = jac_kb4(p, u);
    const float inv_z = 1.0f / p.z, inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
    const TpPolys t = thin_prism_polys(p.x, p.y, u);
    return M23{V2{k.c0.x + u.fx * t.dnu_dx * inv_z2, k.c0.y + u.fy * t.dnv_dx * inv_z2},
               V2{k.c1.x + u.fx * t.dnu_dy * inv_z2, k.c1.y + u.fy * t.dnv_dy * inv_z2},
               V2{k.c2.x + -2.0f * u.fx * t.nu * inv_z3, k.c2.y + -2.0f * u.fy * t.nv * inv_z3}};
}
M23 project_jacobian(V3 p, const or_camera& u) {
    switch (u.model) {
    case OR_MODEL_KB4: return jac_kb4(p, u);
    case OR_MODEL_RT8: return jac_rt8(p, u);
    case OR_MODEL_TPF: return jac_tpf(p, u);
    default: return jac_pinhole(p, u);
    }
}

// kernels/camera_model/pinhole.rs:199-265
V3 projection_vjp_pinhole(M23 J, V3 mc, S3 cov_c, const or_camera& u, S2 v_cov2d, V2 v_mean2d) {
    const float fx = u.fx, fy = u.fy;
    const float mx = mc.x, my = mc.y, mz = mc.z;
    const float inv_z = 1.0f / mz;
    const float mx_rz_raw = mx * inv_z, my_rz_raw = my * inv_z;
    const float mx_rz = clampf(mx_rz_raw, u.lim_neg_x, u.lim_pos_x);
    const float my_rz = clampf(my_rz_raw, u.lim_neg_y, u.lim_pos_y);
    const bool in_x = mx_rz_raw <= u.lim_pos_x && mx_rz_raw >= u.lim_neg_x;
    const bool in_y = my_rz_raw <= u.lim_pos_y && my_rz_raw >= u.lim_neg_y;
    const float inv_z2 = inv_z * inv_z;
    const float inv_z3 = inv_z2 * inv_z;
    float v_mx = fx * inv_z * v_mean2d.x;
    float v_my = fy * inv_z * v_mean2d.y;
    float v_mz = -(fx * mx * v_mean2d.x + fy * my * v_mean2d.y) * inv_z2;
    const M23 tmp = s2_mul_m23(v_cov2d, J);
    const float vj00 = 2.0f * dot(m23_row0(tmp), s3_row0(cov_c));
    const float vj11 = 2.0f * dot(m23_row1(tmp), s3_row1(cov_c));
    const float vj20 = 2.0f * dot(m23_row0(tmp), s3_row2(cov_c));
    const float vj21 = 2.0f * dot(m23_row1(tmp), s3_row2(cov_c));
    const float tx = mz * mx_rz;
    const float ty = mz * my_rz;
    if (in_x) v_mx += -fx * inv_z2 * vj20; else v_mz += -fx * inv_z3 * vj20 * tx;
    if (in_y) v_my += -fy * inv_z2 * vj21; else v_mz += -fy * inv_z3 * vj21 * ty;
    v_mz += -fx * inv_z2 * vj00 - fy * inv_z2 * vj11 + 2.0f * fx * tx * inv_z3 * vj20 + 2.0f * fy * ty * inv_z3 * vj21;
    return V3{v_mx, v_my, v_mz};
}

// kernels/camera_model/kannala_brandt_4.rs:154-337
V3 projection_vjp_kb4(M23 J, V3 mc, S3 cov_c, const or_camera& u, S2 v_cov2d, V2 v_mean2d) {
    const float fx = u.fx, fy = u.fy;
    const float k1 = u.kb4[0], k2 = u.kb4[1], k3 = u.kb4[2], k4 = u.kb4[3];
    const float mx = mc.x, my = mc.y, mz = mc.z;
    const float r2 = mx * mx + my * my;
    const float r = fmax_(std::sqrt(r2), 1.0e-8f);
    const float rho2 = r2 + mz * mz;
    const float theta = atan2f_c(r, mz);
    const float th2 = theta * theta, th4 = th2 * th2, th6 = th4 * th2, th8 = th4 * th4;
    const float theta_d = theta * (1.0f + k1 * th2 + k2 * th4 + k3 * th6 + k4 * th8);
    const float p1 = 1.0f + 3.0f * k1 * th2 + 5.0f * k2 * th4 + 7.0f * k3 * th6 + 9.0f * k4 * th8;
    const float p2 = 6.0f * k1 * theta + 20.0f * k2 * theta * th2 + 42.0f * k3 * theta * th4 + 72.0f * k4 * theta * th6;
    const float inv_r = 1.0f / r;
    const float inv_r3 = inv_r * inv_r * inv_r;
    const float inv_r5 = inv_r3 * inv_r * inv_r;
    const float inv_rho2 = 1.0f / rho2;
    const float inv_rho2_sq = inv_rho2 * inv_rho2;
    const float inv_rho2_r = inv_rho2 * inv_r;
    const float dth_x = mx * mz * inv_rho2_r;
    const float dth_y = my * mz * inv_rho2_r;
    const float dth_z = -r * inv_rho2;
    const float xr = mx * inv_r, yr = my * inv_r;
    const float dxr_x = my * my * inv_r3;
    const float dxr_y = -mx * my * inv_r3;
    const float dyr_x = dxr_y;
    const float dyr_y = mx * mx * inv_r3;
    const float dg_x = p1 * dth_x, dg_y = p1 * dth_y, dg_z = p1 * dth_z;
    float v_mx = dot2(v_mean2d, J.c0);
    float v_my = dot2(v_mean2d, J.c1);
    float v_mz = dot2(v_mean2d, J.c2);
    const M23 tmp = s2_mul_m23(v_cov2d, J);
    const float vj_u0 = 2.0f * dot(m23_row0(tmp), s3_row0(cov_c));
    const float vj_u1 = 2.0f * dot(m23_row0(tmp), s3_row1(cov_c));
    const float vj_u2 = 2.0f * dot(m23_row0(tmp), s3_row2(cov_c));
    const float vj_v0 = 2.0f * dot(m23_row1(tmp), s3_row0(cov_c));
    const float vj_v1 = 2.0f * dot(m23_row1(tmp), s3_row1(cov_c));
    const float vj_v2 = 2.0f * dot(m23_row1(tmp), s3_row2(cov_c));
    const float three_r2_z2 = 3.0f * r2 + mz * mz;
    const float r2_minus_z2 = r2 - mz * mz;
    const float h_th_00 = mz * (r2 * rho2 - mx * mx * three_r2_z2) * inv_r3 * inv_rho2_sq;
    const float h_th_11 = mz * (r2 * rho2 - my * my * three_r2_z2) * inv_r3 * inv_rho2_sq;
    const float h_th_01 = -mx * my * mz * three_r2_z2 * inv_r3 * inv_rho2_sq;
    const float h_th_02 = mx * r2_minus_z2 * inv_r * inv_rho2_sq;
    const float h_th_12 = my * r2_minus_z2 * inv_r * inv_rho2_sq;
    const float h_th_22 = 2.0f * mz * r * inv_rho2_sq;
    const float two_x2_my2 = 2.0f * mx * mx - my * my;
    const float two_y2_mx2 = 2.0f * my * my - mx * mx;
    const float h_xr_00 = -3.0f * mx * my * my * inv_r5;
    const float h_xr_01 = my * two_x2_my2 * inv_r5;
    const float h_xr_11 = mx * two_y2_mx2 * inv_r5;
    const float h_yr_00 = my * two_x2_my2 * inv_r5;
    const float h_yr_01 = mx * two_y2_mx2 * inv_r5;
    const float h_yr_11 = -3.0f * mx * mx * my * inv_r5;
    {
        const float d2g = p2 * dth_x * dth_x + p1 * h_th_00;
        const float d_ju = fx * (d2g * xr + dg_x * dxr_x + dg_x * dxr_x + theta_d * h_xr_00);
        const float d_jv = fy * (d2g * yr + dg_x * dyr_x + dg_x * dyr_x + theta_d * h_yr_00);
        v_mx += vj_u0 * d_ju + vj_v0 * d_jv;
    }
    {
        const float d2g = p2 * dth_y * dth_x + p1 * h_th_01;
        const float d_ju = fx * (d2g * xr + dg_y * dxr_x + dg_x * dxr_y + theta_d * h_xr_01);
        const float d_jv = fy * (d2g * yr + dg_y * dyr_x + dg_x * dyr_y + theta_d * h_yr_01);
        v_mx += vj_u1 * d_ju + vj_v1 * d_jv;
    }
    {
        const float d2g = p2 * dth_z * dth_x + p1 * h_th_02;
        const float d_ju = fx * (d2g * xr + dg_x * 0.0f + dg_z * dxr_x);
        const float d_jv = fy * (d2g * yr + dg_x * 0.0f + dg_z * dyr_x);
        v_mx += vj_u2 * d_ju + vj_v2 * d_jv;
    }
    {
        const float d2g = p2 * dth_x * dth_y + p1 * h_th_01;
        const float d_ju = fx * (d2g * xr + dg_x * dxr_y + dg_y * dxr_x + theta_d * h_xr_01);
        const float d_jv = fy * (d2g * yr + dg_x * dyr_y + dg_y * dyr_x + theta_d * h_yr_01);
        v_my += vj_u0 * d_ju + vj_v0 * d_jv;
    }
    {
        const float d2g = p2 * dth_y * dth_y + p1 * h_th_11;
        const float d_ju = fx * (d2g * xr + dg_y * dxr_y + dg_y * dxr_y + theta_d * h_xr_11);
        const float d_jv = fy * (d2g * yr + dg_y * dyr_y + dg_y * dyr_y + theta_d * h_yr_11);
        v_my += vj_u1 * d_ju + vj_v1 * d_jv;
    }
    {
        const float d2g = p2 * dth_z * dth_y + p1 * h_th_12;
        const float d_ju = fx * (d2g * xr + dg_y * 0.0f + dg_z * dxr_y);
        const float d_jv = fy * (d2g * yr + dg_y * 0.0f + dg_z * dyr_y);
        v_my += vj_u2 * d_ju + vj_v2 * d_jv;
    }
    {
        const float d2g = p2 * dth_x * dth_z + p1 * h_th_02;
        const float d_ju = fx * (d2g * xr + dg_z * dxr_x + dg_x * 0.0f);
        const float d_jv = fy * (d2g * yr + dg_z * dyr_x + dg_x * 0.0f);
        v_mz += vj_u0 * d_ju + vj_v0 * d_jv;
    }
    {
        const float d2g = p2 * dth_y * dth_z + p1 * h_th_12;
        const float d_ju = fx * (d2g * xr + dg_z * dxr_y + dg_y * 0.0f);
        const float d_jv = fy * (d2g * yr + dg_z * dyr_y + dg_y * 0.0f);
        v_mz += vj_u1 * d_ju + vj_v1 * d_jv;
    }
    {
        const float d2g = p2 * dth_z * dth_z + p1 * h_th_22;
        const float d_ju = fx * (d2g * xr);
        const float d_jv = fy * (d2g * yr);
        v_mz += vj_u2 * d_ju + vj_v2 * d_jv;
    }
    return V3{v_mx, v_my, v_mz};
}

// kernels/camera_model/radial_tangential_8.rs:151-393: the Jacobian at the
// clamped, radially capped surrogate point and its derivative; clamped or
// capped coordinates act as constants of the mean.
V3 projection_vjp_rt8(V3 mc, S3 cov_c, const or_camera& u, S2 v_cov2d, V2 v_mean2d) {
    const float fx = u.fx, fy = u.fy;
    const float k1 = u.dist[0], k2 = u.dist[1], k3 = u.dist[2], k4 = u.dist[3], k5 = u.dist[4], k6 = u.dist[5];
    const float p1 = u.dist[6], p2 = u.dist[7];
    const float mz = mc.z, inv_z = 1.0f / mz;
    const float xr_raw = mc.x * inv_z, yr_raw = mc.y * inv_z;
    const float xr_box = clampf(xr_raw, u.lim_neg_x, u.lim_pos_x);
    const float yr_box = clampf(yr_raw, u.lim_neg_y, u.lim_pos_y);
    const float r_box = std::sqrt(xr_box * xr_box + yr_box * yr_box);
    const bool capped = r_box > u.lim_r;
    const float r_scale = capped ? u.lim_r / r_box : 1.0f;
    const float xr = xr_box * r_scale, yr = yr_box * r_scale;
    const bool in_x = xr_raw <= u.lim_pos_x && xr_raw >= u.lim_neg_x && !capped;
    const bool in_y = yr_raw <= u.lim_pos_y && yr_raw >= u.lim_neg_y && !capped;
    const float xc = xr * mz, yc = yr * mz;
    const float inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
    const float x = xc * inv_z, y = yc * inv_z;
    const float r2 = x * x + y * y, r4 = r2 * r2;
    const float N = 1.0f + k1 * r2 + k2 * r4 + k3 * r2 * r4;
    const float D = 1.0f + k4 * r2 + k5 * r4 + k6 * r2 * r4;
    const float Np = k1 + 2.0f * k2 * r2 + 3.0f * k3 * r4;
    const float Dp = k4 + 2.0f * k5 * r2 + 3.0f * k6 * r4;
    const float Npp = 2.0f * k2 + 6.0f * k3 * r2;
    const float Dpp = 2.0f * k5 + 6.0f * k6 * r2;
    const float iD = 1.0f / D, iD2 = iD * iD, iD3 = iD2 * iD;
    const float R0 = N * iD;
    const float R1 = (Np * D - N * Dp) * iD2;
    const float R2 = (Npp * D * D - 2.0f * Np * D * Dp - N * Dpp * D + 2.0f * N * Dp * Dp) * iD3;
    const float Rx = 2.0f * x * R1, Ry = 2.0f * y * R1;
    const float R1x = 2.0f * x * R2, R1y = 2.0f * y * R2;
    const float a00 = R0 + 2.0f * x * x * R1 + 2.0f * p1 * y + 6.0f * p2 * x;
    const float a01 = 2.0f * x * y * R1 + 2.0f * p1 * x + 2.0f * p2 * y;
    const float a10 = a01;
    const float a11 = R0 + 2.0f * y * y * R1 + 6.0f * p1 * y + 2.0f * p2 * x;
    const float s00 = fx * a00 * inv_z, s01 = fx * a01 * inv_z, s02 = -fx * (a00 * xc + a01 * yc) * inv_z2;
    const float s10 = fy * a10 * inv_z, s11 = fy * a11 * inv_z, s12 = -fy * (a10 * xc + a11 * yc) * inv_z2;
    const float e00 = in_x ? s00 : 0.0f, e10 = in_x ? s10 : 0.0f;
    const float e01 = in_y ? s01 : 0.0f, e11 = in_y ? s11 : 0.0f;
    const float e02 = ((in_x ? 0.0f : xr * s00) + (in_y ? 0.0f : yr * s01)) + s02;
    const float e12 = ((in_x ? 0.0f : xr * s10) + (in_y ? 0.0f : yr * s11)) + s12;
    float v_x = e00 * v_mean2d.x + e10 * v_mean2d.y;
    float v_y = e01 * v_mean2d.x + e11 * v_mean2d.y;
    float v_z = e02 * v_mean2d.x + e12 * v_mean2d.y;
    const M23 tmp = s2_mul_m23(v_cov2d, M23{V2{e00, e10}, V2{e01, e11}, V2{e02, e12}});
    const float gu0 = 2.0f * dot(m23_row0(tmp), s3_row0(cov_c)), gu1 = 2.0f * dot(m23_row0(tmp), s3_row1(cov_c));
    const float gu2 = 2.0f * dot(m23_row0(tmp), s3_row2(cov_c));
    const float gv0 = 2.0f * dot(m23_row1(tmp), s3_row0(cov_c)), gv1 = 2.0f * dot(m23_row1(tmp), s3_row1(cov_c));
    const float gv2 = 2.0f * dot(m23_row1(tmp), s3_row2(cov_c));
    const float wu0 = in_x ? gu0 : xr * gu2, wv0 = in_x ? gv0 : xr * gv2;
    const float wu1 = in_y ? gu1 : yr * gu2, wv1 = in_y ? gv1 : yr * gv2;
    const float wu2 = gu2, wv2 = gv2;
    // derivatives of the distortion Jacobian entries in (x, y)
    const float a00x = Rx + 4.0f * x * R1 + 2.0f * x * x * R1x + 6.0f * p2;
    const float a00y = Ry + 2.0f * x * x * R1y + 2.0f * p1;
    const float a01x = 2.0f * y * R1 + 2.0f * x * y * R1x + 2.0f * p1;
    const float a01y = 2.0f * x * R1 + 2.0f * x * y * R1y + 2.0f * p2;
    const float a10x = a01x, a10y = a01y;
    const float a11x = Rx + 2.0f * y * y * R1x + 2.0f * p2;
    const float a11y = Ry + 4.0f * y * R1 + 2.0f * y * y * R1y + 6.0f * p1;
    // ... in (xc, yc, Z)
    const float a00_xc = a00x * inv_z, a00_yc = a00y * inv_z, a00_z = -(xc * a00x + yc * a00y) * inv_z2;
    const float a01_xc = a01x * inv_z, a01_yc = a01y * inv_z, a01_z = -(xc * a01x + yc * a01y) * inv_z2;
    const float a10_xc = a10x * inv_z, a10_yc = a10y * inv_z, a10_z = -(xc * a10x + yc * a10y) * inv_z2;
    const float a11_xc = a11x * inv_z, a11_yc = a11y * inv_z, a11_z = -(xc * a11x + yc * a11y) * inv_z2;
    const float s00_xc = fx * a00_xc * inv_z, s00_yc = fx * a00_yc * inv_z, s00_z = fx * (a00_z * inv_z - a00 * inv_z2);
    const float s01_xc = fx * a01_xc * inv_z, s01_yc = fx * a01_yc * inv_z, s01_z = fx * (a01_z * inv_z - a01 * inv_z2);
    const float s10_xc = fy * a10_xc * inv_z, s10_yc = fy * a10_yc * inv_z, s10_z = fy * (a10_z * inv_z - a10 * inv_z2);
    const float s11_xc = fy * a11_xc * inv_z, s11_yc = fy * a11_yc * inv_z, s11_z = fy * (a11_z * inv_z - a11 * inv_z2);
    const float s02_xc = -fx * (a00_xc * xc + a00 + a01_xc * yc) * inv_z2;
    const float s02_yc = -fx * (a00_yc * xc + a01_yc * yc + a01) * inv_z2;
    const float s02_z = -fx * ((a00_z * xc + a01_z * yc) * inv_z2 - 2.0f * (a00 * xc + a01 * yc) * inv_z3);
    const float s12_xc = -fy * (a10_xc * xc + a10 + a11_xc * yc) * inv_z2;
    const float s12_yc = -fy * (a10_yc * xc + a11_yc * yc + a11) * inv_z2;
    const float s12_z = -fy * ((a10_z * xc + a11_z * yc) * inv_z2 - 2.0f * (a10 * xc + a11 * yc) * inv_z3);
    const float c_xc = wu0 * s00_xc + wu1 * s01_xc + wu2 * s02_xc + wv0 * s10_xc + wv1 * s11_xc + wv2 * s12_xc;
    const float c_yc = wu0 * s00_yc + wu1 * s01_yc + wu2 * s02_yc + wv0 * s10_yc + wv1 * s11_yc + wv2 * s12_yc;
    const float c_z = wu0 * s00_z + wu1 * s01_z + wu2 * s02_z + wv0 * s10_z + wv1 * s11_z + wv2 * s12_z;
    if (in_x) v_x += c_xc;
    if (in_y) v_y += c_yc;
    v_z += c_z;
    if (!in_x) v_z += xr * c_xc;
    if (!in_y) v_z += yr * c_yc;
    return V3{v_x, v_y, v_z};
}

// kernels/camera_model/thin_prism_fisheye.rs:118-203
V3 projection_vjp_tpf(M23 J, V3 mc, S3 cov_c, const or_camera& u, S2 v_cov2d, V2 v_mean2d) {
    const V3 kg = projection_vjp_kb4(J, mc, cov_c, u, v_cov2d, v_mean2d);
    const float fx = u.fx, fy = u.fy;
    const float p1 = u.dist[0], p2 = u.dist[1], sx1 = u.dist[2], sy1 = u.dist[3];
    const float inv_z = 1.0f / mc.z, inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z, inv_z4 = inv_z2 * inv_z2;
    const TpPolys t = thin_prism_polys(mc.x, mc.y, u);
    const float nu_xx = 6.0f * p2 + 2.0f * sx1, nu_yy = 2.0f * p2 + 2.0f * sx1, nu_xy = 2.0f * p1;
    const float nv_xx = 2.0f * p1 + 2.0f * sy1, nv_yy = 6.0f * p1 + 2.0f * sy1, nv_xy = 2.0f * p2;
    const float hu00 = nu_xx * inv_z2, hu01 = nu_xy * inv_z2, hu11 = nu_yy * inv_z2;
    const float hu02 = -2.0f * t.dnu_dx * inv_z3, hu12 = -2.0f * t.dnu_dy * inv_z3, hu22 = 6.0f * t.nu * inv_z4;
    const float hv00 = nv_xx * inv_z2, hv01 = nv_xy * inv_z2, hv11 = nv_yy * inv_z2;
    const float hv02 = -2.0f * t.dnv_dx * inv_z3, hv12 = -2.0f * t.dnv_dy * inv_z3, hv22 = 6.0f * t.nv * inv_z4;
    const M23 tmp = s2_mul_m23(v_cov2d, J);
    const float gu0 = 2.0f * dot(m23_row0(tmp), s3_row0(cov_c)), gu1 = 2.0f * dot(m23_row0(tmp), s3_row1(cov_c));
    const float gu2 = 2.0f * dot(m23_row0(tmp), s3_row2(cov_c));
    const float gv0 = 2.0f * dot(m23_row1(tmp), s3_row0(cov_c)), gv1 = 2.0f * dot(m23_row1(tmp), s3_row1(cov_c));
    const float gv2 = 2.0f * dot(m23_row1(tmp), s3_row2(cov_c));
    const float ax = fx * (gu0 * hu00 + gu1 * hu01 + gu2 * hu02) + fy * (gv0 * hv00 + gv1 * hv01 + gv2 * hv02);
    const float ay = fx * (gu0 * hu01 + gu1 * hu11 + gu2 * hu12) + fy * (gv0 * hv01 + gv1 * hv11 + gv2 * hv12);
    const float az = fx * (gu0 * hu02 + gu1 * hu12 + gu2 * hu22) + fy * (gv0 * hv02 + gv1 * hv12 + gv2 * hv22);
    return V3{kg.x + ax, kg.y + ay, kg.z + az};
}

V3 projection_vjp(M23 J, V3 mc, S3 cov_c, const or_camera& u, S2 v_cov2d, V2 v_mean2d) {
    switch (u.model) {
    case OR_MODEL_KB4: return projection_vjp_kb4(J, mc, cov_c, u, v_cov2d, v_mean2d);
    case OR_MODEL_RT8: return projection_vjp_rt8(mc, cov_c, u, v_cov2d, v_mean2d);
    case OR_MODEL_TPF: return projection_vjp_tpf(J, mc, cov_c, u, v_cov2d, v_mean2d);
    default: return projection_vjp_pinhole(J, mc, cov_c, u, v_cov2d, v_mean2d);
    }
}

// --- covariance ----------------------------------------------------------------
// kernels/helpers.rs:195-225
S2 calc_cov2d(V3 scale_, Q4 quat, V3 mean_c, const or_camera& u) {
    const M3 ns = mul_diag(mul_mat3(view_rot(u), quat_to_mat3(quat)), scale_);
    const M23 J = project_jacobian(mean_c, u);
    const M23 v = m23_mul_mat3(J, ns);
    const S2 raw = m23_gram(v);
    const float lim = 1.0e18f;
    const float max_abs = s2_max_abs(raw);
    const float scale_down = (max_abs > lim) ? lim / max_abs : 1.0f;
    return s2_scale(raw, scale_down);
}
// compensate_cov2d, kernels/helpers.rs:227-245: +0.3 on the diagonal (Default)
// or +0.1 with the compensation sqrt(max(det, 0) / det_blurred) (Mip).
S2 compensate_cov2d(S2 c, bool mip, float& filter_comp) {
    const float blur = mip ? 0.1f : 0.3f;
    const S2 b{c.c00 + blur, c.c01, c.c11 + blur};
    filter_comp = 1.0f;
    if (mip) {
        const float det_raw = fmax_(c.c00 * c.c11 - c.c01 * c.c01, 0.0f);
        const float det_blurred = b.c00 * b.c11 - b.c01 * b.c01;
        filter_comp = std::sqrt(det_raw / det_blurred);
    }
    return b;
}

// apply_scale_floor, kernels/helpers.rs:497-553: s' = sqrt(s^2 + f^2) per
// axis, opacity sigmoid(raw) prod(s / s') clamped to [1e-6, 1 - 1e-6].
struct ScaleFloor { V3 scale; float opac, coef; V3 ratio_sq; bool opac_open; };
ScaleFloor apply_scale_floor(V3 s, float opac_sig, const float* min_scale, uint32_t g) {
    ScaleFloor r{s, opac_sig, 1.0f, v3(1.0f, 1.0f, 1.0f), true};
    if (min_scale) {
        const float f = min_scale[g], f2 = f * f;
        r.scale = v3(std::sqrt(s.x * s.x + f2), std::sqrt(s.y * s.y + f2), std::sqrt(s.z * s.z + f2));
        const float rx = s.x / r.scale.x, ry = s.y / r.scale.y, rz = s.z / r.scale.z;
        r.coef = rx * ry * rz;
        r.ratio_sq = v3(rx * rx, ry * ry, rz * rz);
        const float o = opac_sig * r.coef;
        r.opac_open = o > 1.0e-6f && o < 1.0f - 1.0e-6f;
        r.opac = clampf(o, 1.0e-6f, 1.0f - 1.0e-6f);
    }
    return r;
}

// kernels/helpers.rs:133-144
void bbox_extent(S2 conic, float power, float& ex, float& ey) {
    const float det = conic.c00 * conic.c11 - conic.c01 * conic.c01;
    const bool degenerate = det <= 0.0f;
    const float inv_det = degenerate ? 0.0f : 1.0f / det;
    const float ex_ = std::sqrt(2.0f * power * conic.c11 * inv_det);
    const float ey_ = std::sqrt(2.0f * power * conic.c00 * inv_det);
    ex = degenerate ? -1.0f : ex_;
    ey = degenerate ? -1.0f : ey_;
}
struct TileBbox { uint32_t min_x, min_y, max_x, max_y; };
// Rust's float -> u32 `as` cast: truncation, saturating, NaN -> 0.
uint32_t f2u32_sat(float v) {
    if (!(v > 0.0f)) return 0u;
    if (v >= 4294967296.0f) return 0xFFFFFFFFu;
    return (uint32_t)v;
}
// kernels/helpers.rs:160-190
TileBbox tile_bbox(float cx, float cy, float ex, float ey, uint32_t bw, uint32_t bh) {
    const float tw = (float)TILE_W;
    const float x = cx / tw, y = cy / tw, dx = ex / tw, dy = ey / tw;
    const float bwf = (float)bw, bhf = (float)bh;
    return TileBbox{f2u32_sat(clampf(x - dx, 0.0f, bwf)), f2u32_sat(clampf(y - dy, 0.0f, bhf)),
                    f2u32_sat(clampf(x + dx + 1.0f, 0.0f, bwf)), f2u32_sat(clampf(y + dy + 1.0f, 0.0f, bhf))};
}
// kernels/helpers.rs:275-314 (StopThePop conservative ellipse-rect test)
bool will_contribute(uint32_t tx, uint32_t ty, float mx, float my, S2 conic, float power) {
    const float min_x = (float)(tx * TILE_W), min_y = (float)(ty * TILE_W);
    const float max_x = min_x + (float)TILE_W, max_y = min_y + (float)TILE_W;
    const bool x_left = mx < min_x, x_right = mx > max_x;
    const bool in_x = !(x_left || x_right);
    const bool y_above = my < min_y, y_below = my > max_y;
    const bool in_y = !(y_above || y_below);
    bool hit = in_x && in_y;
    if (!hit) {
        const float corner_x = x_left ? min_x : max_x;
        const float corner_y = y_above ? min_y : max_y;
        const float width = max_x - min_x, height = max_y - min_y;
        const float dxf = x_left ? width : -width;
        const float dyf = y_above ? height : -height;
        const float diff_x = mx - corner_x, diff_y = my - corner_y;
        const float tx_raw = (dxf * conic.c00 * diff_x + dxf * conic.c01 * diff_y) / (dxf * conic.c00 * dxf);
        const float ty_raw = (dyf * conic.c01 * diff_x + dyf * conic.c11 * diff_y) / (dyf * conic.c11 * dyf);
        const float tx_ = in_y ? 0.0f : clampf(tx_raw, 0.0f, 1.0f);
        const float ty_ = in_x ? 0.0f : clampf(ty_raw, 0.0f, 1.0f);
        const float px = corner_x + tx_ * dxf;
        const float py = corner_y + ty_ * dyf;
        hit = calc_sigma(px, py, conic, mx, my) <= power;
    }
    return hit;
}

// --- SH -------------------------------------------------------------------------
// kernels/sh.rs:51-140 basis values in the order the reference accumulates them.
int sh_basis(uint32_t degree, V3 v, float* Y) {
    Y[0] = 0.2820948f;
    int n = 1;
    if (degree >= 1) {
        const float f0a = 0.4886025f;
        Y[1] = -f0a * v.y; Y[2] = f0a * v.z; Y[3] = -f0a * v.x; n = 4;
        if (degree >= 2) {
            const float z2 = v.z * v.z;
            const float f0b = -1.0925485f * v.z;
            const float f1a = 0.54627424f;
            const float fc1 = v.x * v.x - v.y * v.y;
            const float fs1 = 2.0f * v.x * v.y;
            Y[4] = f1a * fs1; Y[5] = f0b * v.y; Y[6] = 0.9461747f * z2 - 0.31539157f;
            Y[7] = f0b * v.x; Y[8] = f1a * fc1; n = 9;
            if (degree >= 3) {
                const float f0c = -2.285229f * z2 + 0.4570458f;
                const float f1b = 1.4453057f * v.z;
                const float f2a = -0.5900436f;
                const float fc2 = v.x * fc1 - v.y * fs1;
                const float fs2 = v.x * fs1 + v.y * fc1;
                const float p12 = v.z * (1.8658817f * z2 - 1.119529f);
                Y[9] = f2a * fs2; Y[10] = f1b * fs1; Y[11] = f0c * v.y; Y[12] = p12;
                Y[13] = f0c * v.x; Y[14] = f1b * fc1; Y[15] = f2a * fc2; n = 16;
                if (degree >= 4) {
                    const float f0d = v.z * (-4.683326f * z2 + 2.0071396f);
                    const float f1c = 3.3116114f * z2 - 0.47308735f;
                    const float f2b = -1.7701308f * v.z;
                    const float f3a = 0.62583575f;
                    const float fc3 = v.x * fc2 - v.y * fs2;
                    const float fs3 = v.x * fs2 + v.y * fc2;
                    const float p6 = Y[6];
                    Y[16] = f3a * fs3; Y[17] = f2b * fs2; Y[18] = f1c * fs1; Y[19] = f0d * v.y;
                    Y[20] = 1.9843135f * v.z * p12 - 1.0062306f * p6;
                    Y[21] = f0d * v.x; Y[22] = f1c * fc1; Y[23] = f2b * fc2; Y[24] = f3a * fc3; n = 25;
                }
            }
        }
    }
    return n;
}
// kernels/sh.rs:51-140: colour = C0 c0 + sum_k Y_k c_k, each term added in order.
V3 sh_to_color(const float* coeffs, uint32_t degree, V3 v) {
    float Y[25];
    const int n = sh_basis(degree, v, Y);
    V3 color = scale(v3(coeffs[0], coeffs[1], coeffs[2]), Y[0]);
    for (int k = 1; k < n; ++k) color = add(color, scale(v3(coeffs[3 * k], coeffs[3 * k + 1], coeffs[3 * k + 2]), Y[k]));
    return color;
}
// kernels/project_visible.rs:25-61 (SH branch)
V3 splat_color(const float* coeffs, uint32_t degree, V3 mean, const or_camera& u) {
    const V3 v = normalize(sub(mean, V3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]}));
    const V3 raw = sh_to_color(coeffs, degree, v);
    const V3 c = V3{raw.x + 0.5f, raw.y + 0.5f, raw.z + 0.5f};
    return V3{clampf(is_finite(c.x) ? c.x : 0.0f, -100.0f, 100.0f),
              clampf(is_finite(c.y) ? c.y : 0.0f, -100.0f, 100.0f),
              clampf(is_finite(c.z) ? c.z : 0.0f, -100.0f, 100.0f)};
}
// kernels/sh.rs:147-274
V3 sh_viewdir_vjp(const float* cb, uint32_t degree, V3 v, V3 vc) {
    auto co = [&](int k) { return v3(cb[3 * k], cb[3 * k + 1], cb[3 * k + 2]); };
    float gx = 0.0f, gy = 0.0f, gz = 0.0f;
    if (degree >= 1) {
        const float f0a = 0.4886025f;
        const float s_n1 = dot(co(1), vc), s_z0 = dot(co(2), vc), s_p1 = dot(co(3), vc);
        gx += -f0a * s_p1; gy += -f0a * s_n1; gz += f0a * s_z0;
        if (degree >= 2) {
            const float z = v.z, x = v.x, y = v.y;
            const float c2 = -1.0925485f, f1a = 0.54627424f;
            const float s_n2 = dot(co(4), vc), s_n1b = dot(co(5), vc), s_z0b = dot(co(6), vc), s_p1b = dot(co(7), vc), s_p2 = dot(co(8), vc);
            gx += 2.0f * f1a * y * s_n2 + c2 * z * s_p1b + 2.0f * f1a * x * s_p2;
            gy += 2.0f * f1a * x * s_n2 + c2 * z * s_n1b - 2.0f * f1a * y * s_p2;
            gz += c2 * y * s_n1b + 2.0f * 0.9461747f * z * s_z0b + c2 * x * s_p1b;
            if (degree >= 3) {
                const float z2 = z * z, x2 = x * x, y2 = y * y;
                const float f2a = -0.5900436f, c1b = 1.4453057f;
                const float f1b = c1b * z;
                const float c0c = -2.285229f;
                const float f0c = c0c * z2 + 0.4570458f;
                const float f0c_dz = 2.0f * c0c * z;
                const float s_n3 = dot(co(9), vc), s_n2c = dot(co(10), vc), s_n1c = dot(co(11), vc), s_z0c = dot(co(12), vc);
                const float s_p1c = dot(co(13), vc), s_p2c = dot(co(14), vc), s_p3 = dot(co(15), vc);
                const float d12_z = 3.0f * 1.8658817f * z2 - 1.119529f;
                gx += f2a * 6.0f * x * y * s_n3 + 2.0f * f1b * y * s_n2c + f0c * s_p1c + 2.0f * f1b * x * s_p2c + f2a * 3.0f * (x2 - y2) * s_p3;
                gy += f2a * 3.0f * (x2 - y2) * s_n3 + 2.0f * f1b * x * s_n2c + f0c * s_n1c + (-2.0f) * f1b * y * s_p2c + f2a * (-6.0f) * x * y * s_p3;
                gz += 2.0f * c1b * x * y * s_n2c + f0c_dz * y * s_n1c + d12_z * s_z0c + f0c_dz * x * s_p1c + c1b * (x2 - y2) * s_p2c;
                if (degree >= 4) {
                    const float fc1 = x2 - y2, fs1 = 2.0f * x * y;
                    const float fc2 = x * fc1 - y * fs1, fs2 = x * fs1 + y * fc1;
                    const float f0d = z * (-4.683326f * z2 + 2.0071396f);
                    const float f0d_dz = -14.049978f * z2 + 2.0071396f;
                    const float f1c = 3.3116114f * z2 - 0.47308735f;
                    const float f1c_dz = 2.0f * 3.3116114f * z;
                    const float f2b_c = -1.7701308f;
                    const float f2b = f2b_c * z;
                    const float f3a = 0.62583575f;
                    const float p_sh12 = z * (1.8658817f * z2 - 1.119529f);
                    const float dp12 = 3.0f * 1.8658817f * z2 - 1.119529f;
                    const float dp6 = 2.0f * 0.9461747f * z;
                    const float dp20 = 1.9843135f * (p_sh12 + z * dp12) - 1.0062306f * dp6;
                    const float s_n4 = dot(co(16), vc), s_n3d = dot(co(17), vc), s_n2d = dot(co(18), vc), s_n1d = dot(co(19), vc);
                    const float s_z0d = dot(co(20), vc), s_p1d = dot(co(21), vc), s_p2d = dot(co(22), vc), s_p3d = dot(co(23), vc), s_p4 = dot(co(24), vc);
                    gx += f3a * 4.0f * fs2 * s_n4 + f2b * 3.0f * fs1 * s_n3d + f1c * 2.0f * y * s_n2d + f0d * s_p1d + f1c * 2.0f * x * s_p2d + f2b * 3.0f * fc1 * s_p3d + f3a * 4.0f * fc2 * s_p4;
                    gy += f3a * 4.0f * fc2 * s_n4 + f2b * 3.0f * fc1 * s_n3d + f1c * 2.0f * x * s_n2d + f0d * s_n1d + f1c * (-2.0f) * y * s_p2d + f2b * (-3.0f) * fs1 * s_p3d + f3a * (-4.0f) * fs2 * s_p4;
                    gz += f2b_c * fs2 * s_n3d + f1c_dz * fs1 * s_n2d + f0d_dz * y * s_n1d + dp20 * s_z0d + f0d_dz * x * s_p1d + f1c_dz * fc1 * s_p2d + f2b_c * fc2 * s_p3d;
                }
            }
        }
    }
    return V3{gx, gy, gz};
}

// --- projection VJP helpers, bwd/kernels/project_backwards.rs:18-98 ----------
Q4 apply_normalize_vjp(Q4 q, Q4 g) {
    const float lsq = qdot(q, q);
    const float l = std::sqrt(lsq);
    const float inv = 1.0f / (l * lsq);
    const float qw = q.w, qx = q.x, qy = q.y, qz = q.z;
    const float gw = g.w, gx = g.x, gy = g.y, gz = g.z;
    const float cc0 = -qw * qx, cc1 = -qx * qy, cc2 = -qy * qw;
    const float cs0 = -qw * qz, cs1 = -qx * qz, cs2 = -qy * qz;
    const float sw = qw * qw, sx = qx * qx, sy = qy * qy, sz = qz * qz;
    return Q4{((lsq - sw) * gw + cc0 * gx + cc2 * gy + cs0 * gz) * inv,
              (cc0 * gw + (lsq - sx) * gx + cc1 * gy + cs1 * gz) * inv,
              (cc2 * gw + cc1 * gx + (lsq - sy) * gy + cs2 * gz) * inv,
              (cs0 * gw + cs1 * gx + cs2 * gy + (lsq - sz) * gz) * inv};
}
Q4 quat_to_mat_vjp(Q4 q, M3 v) {
    const float qw = q.w, qx = q.x, qy = q.y, qz = q.z;
    const float w_grad = qx * (v.c1.z - v.c2.y) + qy * (v.c2.x - v.c0.z) + qz * (v.c0.y - v.c1.x);
    const float x_grad = -2.0f * qx * (v.c1.y + v.c2.z) + qy * (v.c0.y + v.c1.x) + qz * (v.c0.z + v.c2.x) + qw * (v.c1.z - v.c2.y);
    const float y_grad = qx * (v.c0.y + v.c1.x) - 2.0f * qy * (v.c0.x + v.c2.z) + qz * (v.c1.z + v.c2.y) + qw * (v.c2.x - v.c0.z);
    const float z_grad = qx * (v.c0.z + v.c2.x) + qy * (v.c1.z + v.c2.y) - 2.0f * qz * (v.c0.x + v.c1.y) + qw * (v.c0.y - v.c1.x);
    return Q4{2.0f * w_grad, 2.0f * x_grad, 2.0f * y_grad, 2.0f * z_grad};
}
S2 inverse2x2_vjp(S2 minv, S2 v) {
    const float t00 = -minv.c00 * v.c00 + -minv.c01 * v.c01;
    const float t01 = -minv.c01 * v.c00 + -minv.c11 * v.c01;
    const float t10 = -minv.c00 * v.c01 + -minv.c01 * v.c11;
    const float t11 = -minv.c01 * v.c01 + -minv.c11 * v.c11;
    return S2{t00 * minv.c00 + t10 * minv.c01, t01 * minv.c00 + t11 * minv.c01, t01 * minv.c01 + t11 * minv.c11};
}

// ---- compact neural appearance, kernels/neural.rs:1-161 -------------------------
// Row of 12 floats per splat: base colour as an SH DC coefficient (3), latent
// f (8), pad.  x = [sin f0, cos f0, ..., sin f7, cos f7, Y0(d) .. Y15(d)],
// h1 = ReLU(W1 x), h2 = ReLU(W2 h1), colour = ReLU(C0 base + tanh(W3 h2) + 0.5);
// W1 16x32, W2 16x16, W3 3x16 row-major [out][in], packed in one [816].
constexpr int NEURAL_LATENTS = 8, NEURAL_INPUTS = 32, NEURAL_HIDDEN = 16;
constexpr int NEURAL_W1 = 0, NEURAL_W2 = 512, NEURAL_W3 = 768, NEURAL_LEN = 816, NEURAL_ROW = 12;
constexpr float SH_C0 = 0.2820948f;

// write_direction_basis (neural.rs:64-98): real SH bands 0..3 of the unit
// direction into x[16..32); bands above `deg` are 0.
static void direction_basis(float* x, V3 v, uint32_t deg) {
    const float vx = v.x, vy = v.y, vz = v.z;
    const float xy = vx * vy, xz = vx * vz, yz = vy * vz, x2 = vx * vx, y2 = vy * vy, z2 = vz * vz;
    const float m1 = deg >= 1 ? 1.0f : 0.0f, m2 = deg >= 2 ? 1.0f : 0.0f, m3 = deg >= 3 ? 1.0f : 0.0f;
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

// direction_basis_vjp (neural_backwards.rs:82-133): d x[17..32) / d v applied to dx.
static V3 direction_basis_vjp(const float* dx, V3 v, uint32_t deg) {
    const float x = v.x, y = v.y, z = v.z;
    float gx = 0.0f, gy = 0.0f, gz = 0.0f;
    if (deg >= 1) {
        const float c1 = 0.4886025f;
        gy += -c1 * dx[17];
        gz += c1 * dx[18];
        gx += -c1 * dx[19];
    }
    if (deg >= 2) {
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
    if (deg >= 3) {
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
    return V3{gx, gy, gz};
}

struct NeuralAct { float x[NEURAL_INPUTS], h1[NEURAL_HIDDEN], h2[NEURAL_HIDDEN], o[3]; };

// The decoder's forward for one row (neural.rs:100-151); sums run in input order.
static void neural_forward(const float* row, const float* W, V3 v, uint32_t deg, NeuralAct& a) {
    for (int i = 0; i < NEURAL_LATENTS; ++i) sincosf_c(row[3 + i], a.x[2 * i], a.x[2 * i + 1]);
    direction_basis(a.x, v, deg);
    for (int j = 0; j < NEURAL_HIDDEN; ++j) {
        float acc = 0.0f;
        for (int k = 0; k < NEURAL_INPUTS; ++k) acc += W[NEURAL_W1 + j * NEURAL_INPUTS + k] * a.x[k];
        a.h1[j] = fmax_(acc, 0.0f);
    }
    for (int j = 0; j < NEURAL_HIDDEN; ++j) {
        float acc = 0.0f;
        for (int k = 0; k < NEURAL_HIDDEN; ++k) acc += W[NEURAL_W2 + j * NEURAL_HIDDEN + k] * a.h1[k];
        a.h2[j] = fmax_(acc, 0.0f);
    }
    for (int c = 0; c < 3; ++c) {
        float acc = 0.0f;
        for (int k = 0; k < NEURAL_HIDDEN; ++k) acc += W[NEURAL_W3 + c * NEURAL_HIDDEN + k] * a.h2[k];
        a.o[c] = acc;
    }
}

// neural_color (neural.rs:100-161).
static V3 neural_color(const float* row, const float* W, V3 v, uint32_t deg) {
    NeuralAct a;
    neural_forward(row, W, v, deg, a);
    return V3{fmax_(row[0] * SH_C0 + tanhf_c(a.o[0]) + 0.5f, 0.0f),
              fmax_(row[1] * SH_C0 + tanhf_c(a.o[1]) + 0.5f, 0.0f),
              fmax_(row[2] * SH_C0 + tanhf_c(a.o[2]) + 0.5f, 0.0f)};
}

// ---- surfels (2DGS), kernels/helpers.rs:56-69,316-423 ---------------------------
constexpr float SURFEL_NEAR = 0.01f;
constexpr int SURFEL_AUX = 14;          // M rows (9), low-pass centre (2), normal (3)
constexpr int SURFEL_GRADS = 17;        // M rows (9), normal (3), rgb (3), alpha, refine
struct SurfelProj { V3 r0, r1, r2; float bin_x, bin_y; S2 bin_conic; bool valid; };

// surfel_project (helpers.rs:331-412): M = K [s_u W R e0, s_v W R e1, p_c]
// (rows r0..r2) and the screen ellipse covering the opacity cutoff footprint
// u^2 + v^2 <= 2 power and the low-pass disk of radius sqrt(power).
static SurfelProj surfel_project(V3 sc, Q4 q, V3 mc, const or_camera& u, float power) {
    const M3 rot = mul_mat3(view_rot(u), quat_to_mat3(q));
    const V3 a = scale(rot.c0, sc.x), b = scale(rot.c1, sc.y);
    const V3 ka{u.fx * a.x + u.cx * a.z, u.fy * a.y + u.cy * a.z, a.z};
    const V3 kb{u.fx * b.x + u.cx * b.z, u.fy * b.y + u.cy * b.z, b.z};
    const V3 kc{u.fx * mc.x + u.cx * mc.z, u.fy * mc.y + u.cy * mc.z, mc.z};
    SurfelProj p;
    p.r0 = V3{ka.x, kb.x, kc.x};
    p.r1 = V3{ka.y, kb.y, kc.y};
    p.r2 = V3{ka.z, kb.z, kc.z};
    const V3 r0 = p.r0, r1 = p.r1, r2 = p.r2;
    const float k2 = 2.0f * power;
    const float d00 = k2 * (r0.x * r0.x + r0.y * r0.y) - r0.z * r0.z;
    const float d01 = k2 * (r0.x * r1.x + r0.y * r1.y) - r0.z * r1.z;
    const float d11 = k2 * (r1.x * r1.x + r1.y * r1.y) - r1.z * r1.z;
    const float d02 = k2 * (r0.x * r2.x + r0.y * r2.y) - r0.z * r2.z;
    const float d12 = k2 * (r1.x * r2.x + r1.y * r2.y) - r1.z * r2.z;
    const float d22 = k2 * (r2.x * r2.x + r2.y * r2.y) - r2.z * r2.z;
    const float n = -d22;
    const bool front = n > 1.0e-12f;                     // the ellipse lies in front of the camera
    const float inv_n = front ? 1.0f / n : 0.0f;
    const float x0 = -d02 * inv_n, y0 = -d12 * inv_n;
    const float s00 = d00 * inv_n + x0 * x0, s01 = d01 * inv_n + x0 * y0, s11 = d11 * inv_n + y0 * y0;
    const float r2f = fmax_(power, 0.0f);
    const float half_tr = fmax_(0.5f * (s00 + s11), 1.0e-12f);
    const float t = clampf(std::sqrt(half_tr / fmax_(r2f, 1.0e-12f)), 1.0e-3f, 1.0e3f);
    const float ga = 1.0f + 1.0f / t, gb = (1.0f + t) * r2f;
    const S2 grown{ga * s00 + gb, ga * s01, ga * s11 + gb};
    const float det = grown.c00 * grown.c11 - grown.c01 * grown.c01;
    const S2 inv = s2_inverse(grown);
    p.bin_conic = S2{inv.c00 * k2, inv.c01 * k2, inv.c11 * k2};
    p.bin_x = x0; p.bin_y = y0;
    p.valid = front && det > 0.0f && is_finite(x0) && is_finite(y0) && s2_finite(p.bin_conic);
    return p;
}
// surfel_normal (helpers.rs:414-419): the rotated local +Z, facing the camera.
static V3 surfel_normal(Q4 q, V3 mc, const or_camera& u) {
    const V3 n = mul_mat3(view_rot(u), quat_to_mat3(q)).c2;
    return scale(n, dot(n, mc) > 0.0f ? -1.0f : 1.0f);
}
// The ray-plane sample of a pixel (rasterize.rs:267-301): (u, v), the
// intersection depth z, the low-pass offsets and sigma = min(s3d, s2d) / 2;
// false when the ray misses or meets the plane before the near limit.  The
// quotients q.x / q.z and q.y / q.z are taken as products with the correctly
// rounded 1 / q.z (one division for both; each within one rounding of the
// quotient), and the products that feed a sum or a difference are fused
// multiply-adds where written, as the kernels do.
struct SurfelHit { float hux, huy, huz, hvx, hvy, hvz, qz, su, sv, s3d, z, dxs, dys, s2d, sigma; bool valid; };
static SurfelHit surfel_hit(const float* a, float px, float py) {
    SurfelHit h;
    const float m20 = a[6], m21 = a[7], m22 = a[8];
    h.hux = std::fmaf(-px, m20, a[0]); h.huy = std::fmaf(-px, m21, a[1]); h.huz = std::fmaf(-px, m22, a[2]);
    h.hvx = std::fmaf(-py, m20, a[3]); h.hvy = std::fmaf(-py, m21, a[4]); h.hvz = std::fmaf(-py, m22, a[5]);
    const float qx = std::fmaf(h.huy, h.hvz, -(h.huz * h.hvy));
    const float qy = std::fmaf(h.huz, h.hvx, -(h.hux * h.hvz));
    h.qz = std::fmaf(h.hux, h.hvy, -(h.huy * h.hvx));
    const float rq = 1.0f / h.qz;
    h.su = qx * rq;
    h.sv = qy * rq;
    h.s3d = std::fmaf(h.su, h.su, h.sv * h.sv);
    h.z = std::fmaf(m20, h.su, std::fmaf(m21, h.sv, m22));
    h.dxs = px - a[9]; h.dys = py - a[10];
    h.s2d = 2.0f * std::fmaf(h.dxs, h.dxs, h.dys * h.dys);
    h.sigma = 0.5f * fmin_(h.s3d, h.s2d);
    h.valid = is_finite(h.z) && h.z >= SURFEL_NEAR;
    return h;
}

struct RasterSplat { float x, y, A, B, C, opac, r, g, b, c00, c01, c11; uint32_t gid; float z, nx, ny, nz; const float* surf; };

} // namespace

struct or_fwd {
    or_camera cam;
    uint32_t W = 0, H = 0, N = 0, degree = 0, K = 0;
    float lso = 0.0f;
    float bg[3] = {0, 0, 0};
    int flags = 0;
    uint32_t tbw = 0, tbh = 0, T = 0, out_ch = 4;
    const float* transforms = nullptr;   // borrowed for the backward (caller keeps alive)
    const float* sh = nullptr;
    const float* raw_opac = nullptr;
    const float* min_scale = nullptr;    // NULL: no scale floor
    bool mip = false;
    const float* decoder = nullptr;      // [816] neural appearance, NULL: SH colour
    std::vector<float> transforms_copy, sh_copy, opac_copy, min_scale_copy, decoder_copy;
    uint32_t V = 0;
    uint64_t evals = 0;
    std::vector<uint32_t> intersect_counts;
    std::vector<float> max_radius, opacities, visible;
    std::vector<uint32_t> global_from_compact;
    std::vector<float> depths, projected, aux, surf;   // surf: [V,14] surfel aux (M rows, centre, normal)
    bool surfel = false;
    std::vector<uint32_t> isect_tile, isect_cid;   // sorted, sentinel-free prefix of length I
    std::vector<uint32_t> tile_offsets, tile_offsets_shrunk;
    std::vector<float> out_img;
    std::vector<uint32_t> out_packed;
};

static int resolve_threads(int threads) {
#ifdef _OPENMP
    return threads > 0 ? threads : omp_get_max_threads();
#else
    (void)threads;
    return 1;
#endif
}

extern "C" int or_max_threads(void) { return resolve_threads(0); }

extern "C" int or_render_forward(const or_camera* cam_in, uint32_t W, uint32_t H,
                                 const float* transforms, const float* sh, uint32_t degree,
                                 const float* raw_opac, uint32_t N, float lso, const float* min_scale,
                                 const float* decoder, const float bg[3], int flags, int threads, or_fwd** out) {
    if (!cam_in || !out || W == 0 || H == 0 || degree > 4 || (decoder && degree > 3)) return 1;
    const int nthreads = resolve_threads(threads);
    auto f = std::make_unique<or_fwd>();
    f->cam = *cam_in;
    const or_camera& u = f->cam;
    // Neural rows hold 4 coefficients; `degree` is then the decoder's direction band.
    f->W = W; f->H = H; f->N = N; f->degree = degree; f->K = decoder ? 4u : (degree + 1) * (degree + 1); f->lso = lso;
    f->bg[0] = bg[0]; f->bg[1] = bg[1]; f->bg[2] = bg[2];
    f->flags = flags;
    const bool bwd_info = flags & OR_FLAG_BWD_INFO;
    const bool surfel = flags & OR_FLAG_SURFEL;
    // Surfel training renders always carry the geometry channels (render.rs:471-473).
    const bool geometry = (flags & OR_FLAG_GEOMETRY) || (surfel && bwd_info);
    const bool surf_crit = surfel && (flags & OR_FLAG_SURFACE);
    const bool smooth = flags & OR_FLAG_SMOOTH_CUTOFF;
    const bool brute = flags & OR_FLAG_BRUTE_FORCE;
    f->tbw = (W + TILE_W - 1) / TILE_W; f->tbh = (H + TILE_W - 1) / TILE_W; f->T = f->tbw * f->tbh;
    f->out_ch = geometry ? 12 : 4;
    const uint32_t K = f->K;
    // Keep private copies so the backward never depends on caller lifetimes.
    f->transforms_copy.assign(transforms, transforms + (size_t)N * 10);
    f->sh_copy.assign(sh, sh + (size_t)N * K * 3);
    f->opac_copy.assign(raw_opac, raw_opac + N);
    f->transforms = f->transforms_copy.data(); f->sh = f->sh_copy.data(); f->raw_opac = f->opac_copy.data();
    transforms = f->transforms; sh = f->sh; raw_opac = f->raw_opac;
    if (min_scale) {
        f->min_scale_copy.assign(min_scale, min_scale + N);
        f->min_scale = f->min_scale_copy.data();
    }
    if (decoder) {
        f->decoder_copy.assign(decoder, decoder + NEURAL_LEN);
        f->decoder = f->decoder_copy.data();
    }
    f->mip = (flags & OR_FLAG_MIP) != 0;
    f->surfel = surfel;
    const bool mip = f->mip;

    // ---- project_forward: cull + count, kernels/project_forward.rs:26-261 ----
    f->intersect_counts.assign(N, 0u);
    f->max_radius.assign(N, 0.0f);
    f->opacities.assign(N, 0.0f);
    std::vector<uint8_t> vis_flag(N, 0);
    std::vector<float> depth_g(N, 0.0f);
    const uint32_t tbw = f->tbw, tbh = f->tbh;
    #pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t gi = 0; gi < (int64_t)N; ++gi) {
        const uint32_t g = (uint32_t)gi;
        const float* t = transforms + (size_t)g * 10;
        const V3 mean_c = world_to_cam(v3(t[0], t[1], t[2]), u);
        if (!(finite3(mean_c) && mean_c.z <= 1.0e10f)) continue;
        if (u.model == OR_MODEL_PINHOLE || surfel) {   // the fisheye models cull by angle; surfels are pinhole
            if (mean_c.z < 0.01f) continue;
        } else {
            const float r = std::sqrt(mean_c.x * mean_c.x + mean_c.y * mean_c.y);
            const float theta = atan2f_c(r, mean_c.z);
            if (theta > u.half_max_render_fov) continue;
        }
        const V3 sc = v3(expf_c(t[7] + lso), expf_c(t[8] + lso), expf_c(t[9] + lso));
        if (!finite3(sc)) continue;
        const Q4 qu{t[3], t[4], t[5], t[6]};
        const float qn = qdot(qu, qu);
        if (!(qn >= 1.0e-6f && is_finite(qn))) continue;
        const float ro = raw_opac[g];
        if (!is_finite(ro)) continue;
        const Q4 q = qnormalize(qu);
        const ScaleFloor fl = apply_scale_floor(sc, sigmoid(ro), f->min_scale, g);
        f->opacities[g] = fl.opac;
        float mx, my, power;
        S2 conic;
        if (surfel) {
            // project_forward.rs:128-147: bin by the ellipse covering the cutoff
            // footprint and the low-pass disk; no 2-D blur compensation.
            if (!(fl.opac >= 1.0f / 255.0f)) continue;
            power = logf_c(fl.opac * 255.0f);
            const SurfelProj sp = surfel_project(fl.scale, q, mean_c, u, power);
            if (!sp.valid) continue;
            conic = sp.bin_conic; mx = sp.bin_x; my = sp.bin_y;
        } else {
            float filter_comp;
            const S2 cov = compensate_cov2d(calc_cov2d(fl.scale, q, mean_c, u), mip, filter_comp);
            const float opac = fl.opac * filter_comp;
            if (!s2_finite(cov)) continue;
            project(mean_c, u, mx, my);
            if (!(opac >= 1.0f / 255.0f)) continue;
            power = logf_c(opac * 255.0f);
            conic = s2_inverse(cov);
        }
        float ex, ey;
        bbox_extent(conic, power, ex, ey);
        if (!(ex >= 0.0f && ey >= 0.0f)) continue;
        const float wf = (float)W, hf = (float)H;
        const bool on_screen = mx + ex > 0.0f && mx - ex < wf && my + ey > 0.0f && my - ey < hf;
        if (!on_screen) continue;
        const TileBbox bb = tile_bbox(mx, my, ex, ey, tbw, tbh);
        const float radius = fmax_(ex / wf, ey / hf);
        // count_contributing_tiles, kernels/helpers.rs:253-273
        const uint32_t bw = bb.max_x - bb.min_x;
        const uint32_t nb = (bb.max_y - bb.min_y) * bw;
        uint32_t hits = 0;
        for (uint32_t i = 0; i < nb; ++i) {
            const uint32_t tx = i % bw + bb.min_x, ty = i / bw + bb.min_y;
            if (will_contribute(tx, ty, mx, my, conic, power)) ++hits;
        }
        f->intersect_counts[g] = hits;
        f->max_radius[g] = radius;
        vis_flag[g] = 1;
        depth_g[g] = mean_c.z;
    }
    // Compaction: increasing global id (see header).
    for (uint32_t g = 0; g < N; ++g) if (vis_flag[g]) f->global_from_compact.push_back(g);
    const uint32_t V = (uint32_t)f->global_from_compact.size();
    f->V = V;
    f->depths.resize(V);
    for (uint32_t c = 0; c < V; ++c) f->depths[c] = depth_g[f->global_from_compact[c]];

    // ---- project_visible, kernels/project_visible.rs:97-174 / 182-312 ----------
    f->projected.assign((size_t)V * 9, 0.0f);
    if (geometry && !surfel) f->aux.assign((size_t)V * 4, 0.0f);
    if (surfel) f->surf.assign((size_t)V * SURFEL_AUX, 0.0f);
    #pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t ci = 0; ci < (int64_t)V; ++ci) {
        const uint32_t c = (uint32_t)ci;
        const uint32_t g = f->global_from_compact[c];
        const float* t = transforms + (size_t)g * 10;
        const V3 mean = v3(t[0], t[1], t[2]);
        const V3 sc = v3(expf_c(t[7] + lso), expf_c(t[8] + lso), expf_c(t[9] + lso));
        const Q4 q = qnormalize(Q4{t[3], t[4], t[5], t[6]});
        const ScaleFloor fl = apply_scale_floor(sc, sigmoid(raw_opac[g]), f->min_scale, g);
        const V3 mean_c = world_to_cam(mean, u);
        float filter_comp;
        const S2 cov = compensate_cov2d(calc_cov2d(fl.scale, q, mean_c, u), mip, filter_comp);
        const float opac = fl.opac * filter_comp;
        const S2 conic = s2_inverse(cov);
        float mx, my;
        project(mean_c, u, mx, my);
        V3 col;
        if (f->decoder) {
            // kernels/project_visible.rs:25-61, neural branch: the same scrub and clamp
            const V3 c3 = neural_color(sh + (size_t)g * NEURAL_ROW, f->decoder,
                                       normalize(sub(mean, V3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]})), degree);
            col = V3{clampf(is_finite(c3.x) ? c3.x : 0.0f, -100.0f, 100.0f),
                     clampf(is_finite(c3.y) ? c3.y : 0.0f, -100.0f, 100.0f),
                     clampf(is_finite(c3.z) ? c3.z : 0.0f, -100.0f, 100.0f)};
        } else {
            col = splat_color(sh + (size_t)g * K * 3, degree, mean, u);
        }
        float* row = &f->projected[(size_t)c * 9];
        if (surfel) {
            // project_visible.rs:231-273: the row carries the binning ellipse and
            // the floored opacity; the coverage reads the aux row.
            const SurfelProj sp = surfel_project(fl.scale, q, mean_c, u, logf_c(fl.opac * 255.0f));
            const V3 nrm = surfel_normal(q, mean_c, u);
            float* a = &f->surf[(size_t)c * SURFEL_AUX];
            a[0] = sp.r0.x; a[1] = sp.r0.y; a[2] = sp.r0.z; a[3] = sp.r1.x; a[4] = sp.r1.y; a[5] = sp.r1.z;
            a[6] = sp.r2.x; a[7] = sp.r2.y; a[8] = sp.r2.z;
            project_pinhole(mean_c, u, a[9], a[10]);
            a[11] = nrm.x; a[12] = nrm.y; a[13] = nrm.z;
            row[0] = sp.bin_x; row[1] = sp.bin_y; row[2] = sp.bin_conic.c00; row[3] = sp.bin_conic.c01;
            row[4] = sp.bin_conic.c11; row[5] = fl.opac; row[6] = col.x; row[7] = col.y; row[8] = col.z;
            continue;
        }
        row[0] = mx; row[1] = my; row[2] = conic.c00; row[3] = conic.c01; row[4] = conic.c11;
        row[5] = opac; row[6] = col.x; row[7] = col.y; row[8] = col.z;
        if (geometry) {
            const M3 rot = mul_mat3(view_rot(u), quat_to_mat3(q));
            const V3 fs = fl.scale;               // the normal's axis is the floored scales' smallest
            const bool x_min = fs.x <= fs.y && fs.x <= fs.z;
            const bool y_min = !x_min && fs.y <= fs.z;
            const V3 axis = x_min ? rot.c0 : (y_min ? rot.c1 : rot.c2);
            const float flip = (dot(axis, mean_c) > 0.0f) ? -1.0f : 1.0f;
            float* a = &f->aux[(size_t)c * 4];
            a[0] = mean_c.z; a[1] = axis.x * flip; a[2] = axis.y * flip; a[3] = axis.z * flip;
        }
    }

    // ---- depth sort: stable on raw f32 bits, render.rs:689-694 -------------------
    std::vector<uint32_t> sorted(V);
    std::iota(sorted.begin(), sorted.end(), 0u);
    std::stable_sort(sorted.begin(), sorted.end(), [&](uint32_t a, uint32_t b) {
        return f2u(f->depths[a]) < f2u(f->depths[b]);
    });

    // ---- count scan in depth order, kernels/map_gaussians.rs:215-269 -----------
    std::vector<uint64_t> cum(V + 1, 0);
    for (uint32_t j = 0; j < V; ++j) cum[j + 1] = cum[j] + f->intersect_counts[f->global_from_compact[sorted[j]]];
    const uint64_t I = cum[V];
    if (I > 0xFFFFFFFFull) return 2;

    // ---- map: emit (tile, compact id) in depth order, kernels/map_gaussians.rs:23-174
    std::vector<uint32_t> tile_of(I), cid_of(I);
    const uint32_t sentinel = f->T;
    #pragma omp parallel for schedule(dynamic, 256) num_threads(nthreads)
    for (int64_t ji = 0; ji < (int64_t)V; ++ji) {
        const uint32_t j = (uint32_t)ji;
        const uint32_t c = sorted[j];
        const float* row = &f->projected[(size_t)c * 9];
        const S2 conic{row[2], row[3], row[4]};
        const float power = logf_c(row[5] * 255.0f);
        float ex, ey;
        bbox_extent(conic, power, ex, ey);
        const TileBbox bb = tile_bbox(row[0], row[1], ex, ey, tbw, tbh);
        const uint64_t base = cum[j];
        const uint32_t pf_count = (uint32_t)(cum[j + 1] - cum[j]);
        const uint32_t bw = bb.max_x - bb.min_x;
        const uint32_t nb = (bb.max_y - bb.min_y) * bw;
        uint32_t hits = 0;
        for (uint32_t i = 0; i < nb; ++i) {
            const uint32_t tx = i % bw + bb.min_x, ty = i / bw + bb.min_y;
            if (will_contribute(tx, ty, row[0], row[1], conic, power) && hits < pf_count) {
                tile_of[base + hits] = tx + ty * tbw;
                cid_of[base + hits] = c;
                ++hits;
            }
        }
        for (uint32_t p = hits; p < pf_count; ++p) { tile_of[base + p] = sentinel; cid_of[base + p] = c; }
    }

    // ---- tile sort: stable by tile id, render.rs:792-794 -----------------------
    // A counting sort: tile ids are < T + 1, and scattering in input order
    // into each tile's bucket keeps equal ids in emission (depth) order.
    std::vector<uint64_t> bucket((size_t)f->T + 2, 0);
    for (uint64_t i = 0; i < I; ++i) ++bucket[(size_t)tile_of[i] + 1];
    for (size_t t = 1; t < bucket.size(); ++t) bucket[t] += bucket[t - 1];
    const uint64_t I_valid = bucket[sentinel];    // sentinels sort last and are never read
    f->isect_tile.resize(I_valid);
    f->isect_cid.resize(I_valid);
    for (uint64_t i = 0; i < I; ++i) {
        const uint32_t t = tile_of[i];
        if (t >= sentinel) continue;
        const uint64_t o = bucket[t]++;
        f->isect_tile[o] = t;
        f->isect_cid[o] = cid_of[i];
    }

    // ---- tile offsets, get_tile_offset.rs:11-59 ---------------------------------
    f->tile_offsets.assign((size_t)f->T * 2, 0u);
    for (uint64_t i = 0; i < I_valid; ++i) {
        const uint32_t tid = f->isect_tile[i];
        if (i == 0 || f->isect_tile[i - 1] != tid) f->tile_offsets[(size_t)tid * 2] = (uint32_t)i;
        if (i + 1 == I_valid || f->isect_tile[i + 1] != tid) f->tile_offsets[(size_t)tid * 2 + 1] = (uint32_t)(i + 1);
    }
    f->tile_offsets_shrunk = f->tile_offsets;

    // ---- rasterize, kernels/rasterize.rs:109-420 --------------------------------
    const uint32_t C = f->out_ch;
    if (bwd_info) f->out_img.assign((size_t)W * H * C, 0.0f); else f->out_packed.assign((size_t)W * H, 0u);
    f->visible.assign(N, 0.0f);
    uint64_t evals_total = 0;
    #pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads) reduction(+ : evals_total)
    for (int64_t ti = 0; ti < (int64_t)f->T; ++ti) {
        const uint32_t tile = (uint32_t)ti;
        const uint32_t tx = tile % tbw, ty = tile / tbw;
        const uint32_t lo = brute ? 0u : f->tile_offsets[(size_t)tile * 2];
        const uint32_t hi = brute ? V : f->tile_offsets[(size_t)tile * 2 + 1];
        std::vector<RasterSplat> list(hi - lo);
        for (uint32_t i = lo; i < hi; ++i) {
            const uint32_t c = brute ? sorted[i] : f->isect_cid[i];
            const float* row = &f->projected[(size_t)c * 9];
            RasterSplat s;
            s.x = row[0]; s.y = row[1]; s.c00 = row[2]; s.c01 = row[3]; s.c11 = row[4];
            s.A = (0.5f * row[2]) * LOG2E_F; s.B = row[3] * LOG2E_F; s.C = (0.5f * row[4]) * LOG2E_F;
            s.opac = row[5]; s.r = row[6]; s.g = row[7]; s.b = row[8];
            s.gid = f->global_from_compact[c];
            s.surf = surfel ? &f->surf[(size_t)c * SURFEL_AUX] : nullptr;
            if (surfel) { s.z = 0.0f; s.nx = s.surf[11]; s.ny = s.surf[12]; s.nz = s.surf[13]; }
            else if (geometry) { const float* a = &f->aux[(size_t)c * 4]; s.z = a[0]; s.nx = a[1]; s.ny = a[2]; s.nz = a[3]; }
            else { s.z = s.nx = s.ny = s.nz = 0.0f; }
            list[i - lo] = s;
        }
        uint32_t max_useful = lo;
        for (uint32_t py = ty * TILE_W; py < ty * TILE_W + TILE_W; ++py) {
            for (uint32_t px = tx * TILE_W; px < tx * TILE_W + TILE_W; ++px) {
                if (px >= W || py >= H) continue;
                const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
                float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
                float depth_acc = 0.0f, median = 0.0f, dist_b = 0.0f, dist_c = 0.0f, nx = 0.0f, ny = 0.0f, nz = 0.0f;
                uint32_t median_id = 0xFFFFFFFFu;
                uint32_t last_useful = lo;
                float surf_o = 0.0f;
                bool surf_found = false;
                for (uint32_t i = lo; i < hi; ++i) {
                    const RasterSplat& s = list[i - lo];
                    ++evals_total;
                    float sigma, z = s.z, G;
                    if (surfel) {
                        const SurfelHit hit = surfel_hit(s.surf, pcx, pcy);
                        if (!hit.valid) continue;          // no intersection in front of the near limit
                        sigma = hit.sigma;
                        z = hit.z;
                        G = comp_exp2_c(-(sigma * LOG2E_F));
                    } else {
                        const float dx = pcx - s.x, dy = pcy - s.y;
                        sigma = std::fma(std::fma(s.A, dx, s.B * dy), dx, (s.C * dy) * dy);   // base 2
                        G = comp_exp2_c(-sigma);
                    }
                    const float alpha = fmin_(0.999f, s.opac * G);
                    const float w_cut = smooth ? alpha_cutoff_weight(alpha) : ((alpha >= ALPHA_CUTOFF_MID) ? 1.0f : 0.0f);
                    if (!(sigma >= 0.0f && w_cut > 0.0f)) continue;
                    const float alpha_eff = alpha * w_cut;
                    const float next_t = T * (1.0f - alpha_eff);
                    if (next_t <= 1.0e-4f) break;
                    if (bwd_info) f->visible[s.gid] = 1.0f;   // benign race: every writer stores 1
                    const float vis = alpha_eff * T;
                    cr = std::fma(fmax_(s.r, 0.0f), vis, cr);
                    cg = std::fma(fmax_(s.g, 0.0f), vis, cg);
                    cb = std::fma(fmax_(s.b, 0.0f), vis, cb);
                    if (geometry) {
                        depth_acc = std::fma(z, vis, depth_acc);
                        if (surf_crit) {
                            // unbiased-depth surface criterion (rasterize.rs:346-354)
                            surf_o += alpha_eff + 0.1f * G;
                            if (!surf_found && (surf_o > 0.6f || T > 0.5f)) {
                                median = z; median_id = i; surf_found = surf_o > 0.6f;
                            }
                        } else if (T > 0.5f) {
                            median = z; median_id = i;
                        }
                        const float m = dist_depth(z);
                        dist_b = std::fma(m, vis, dist_b);
                        dist_c = std::fma(m * m, vis, dist_c);
                        nx = std::fma(s.nx, vis, nx);
                        ny = std::fma(s.ny, vis, ny);
                        nz = std::fma(s.nz, vis, nz);
                    }
                    T = next_t;
                    last_useful = i + 1;
                }
                max_useful = std::max(max_useful, last_useful);
                const float fr = std::fma(T, f->bg[0], cr);
                const float fg = std::fma(T, f->bg[1], cg);
                const float fb = std::fma(T, f->bg[2], cb);
                const float fa = 1.0f - T;
                const size_t pid = (size_t)py * W + px;
                if (bwd_info) {
                    float* o = &f->out_img[pid * C];
                    o[0] = fr; o[1] = fg; o[2] = fb; o[3] = fa;
                    if (geometry) {
                        o[4] = depth_acc; o[5] = median; o[6] = nx; o[7] = ny; o[8] = nz;
                        o[9] = dist_b; o[10] = dist_c; o[11] = u2f(median_id);
                    }
                } else {
                    const uint32_t r8 = f2u32_sat(clampf(fr * 255.0f, 0.0f, 255.0f));
                    const uint32_t g8 = f2u32_sat(clampf(fg * 255.0f, 0.0f, 255.0f));
                    const uint32_t b8 = f2u32_sat(clampf(fb * 255.0f, 0.0f, 255.0f));
                    const uint32_t a8 = f2u32_sat(clampf(fa * 255.0f, 0.0f, 255.0f));
                    f->out_packed[pid] = r8 | (g8 << 8) | (b8 << 16) | (a8 << 24);
                }
            }
        }
        if (bwd_info && !brute) f->tile_offsets_shrunk[(size_t)tile * 2 + 1] = max_useful;
    }
    f->evals = evals_total;
    *out = f.release();
    return 0;
}

extern "C" void or_fwd_get_info(const or_fwd* f, or_fwd_info* info) {
    info->num_splats = f->N;
    info->num_visible = f->V;
    info->num_intersections = (uint32_t)f->isect_tile.size();
    info->num_tiles = f->T;
    info->tile_bw = f->tbw; info->tile_bh = f->tbh;
    info->img_w = f->W; info->img_h = f->H;
    info->out_channels = (f->flags & OR_FLAG_BWD_INFO) ? f->out_ch : 1;
    info->num_evaluations = f->evals;
}

extern "C" int or_fwd_get(const or_fwd* f, int field, void* dst) {
    auto cp = [&](const auto& v) { if (!v.empty()) std::memcpy(dst, v.data(), v.size() * sizeof(v[0])); return 0; };
    switch (field) {
    case OR_F_INTERSECT_COUNTS: return cp(f->intersect_counts);
    case OR_F_MAX_RADIUS: return cp(f->max_radius);
    case OR_F_OPACITIES: return cp(f->opacities);
    case OR_F_GLOBAL_FROM_COMPACT: return cp(f->global_from_compact);
    case OR_F_DEPTHS: return cp(f->depths);
    case OR_F_PROJECTED: return cp(f->projected);
    case OR_F_AUX: return cp(f->aux);
    case OR_F_ISECT_TILE: return cp(f->isect_tile);
    case OR_F_ISECT_GID: {
        uint32_t* d = (uint32_t*)dst;
        for (size_t i = 0; i < f->isect_cid.size(); ++i) d[i] = f->global_from_compact[f->isect_cid[i]];
        return 0;
    }
    case OR_F_TILE_OFFSETS: return cp(f->tile_offsets);
    case OR_F_TILE_OFFSETS_SHRUNK: return cp(f->tile_offsets_shrunk);
    case OR_F_VISIBLE: return cp(f->visible);
    case OR_F_OUT_IMG: return (f->flags & OR_FLAG_BWD_INFO) ? cp(f->out_img) : cp(f->out_packed);
    case OR_F_SURFEL_AUX: return cp(f->surf);
    default: return 1;
    }
}

extern "C" void or_fwd_free(or_fwd* f) { delete f; }

static int project_vjp(const or_fwd* f, const float* vcf, int nthreads, float* v_transforms, float* v_sh,
                       float* v_raw_opac, float* v_refine);

extern "C" int or_render_backward(const or_fwd* f, const float* v_out, int threads,
                                  float* v_combined_out, float* v_transforms, float* v_sh,
                                  float* v_raw_opac, float* v_refine) {
    if (!f || !v_out || !(f->flags & OR_FLAG_BWD_INFO)) return 1;
    const int nthreads = resolve_threads(threads);
    const uint32_t W = f->W, H = f->H, N = f->N, C = f->out_ch;
    const bool smooth = f->flags & OR_FLAG_SMOOTH_CUTOFF;
    // Per-(tile, splat) partial sums of the raster VJP, one row per sorted
    // intersection inside the shrunk tile ranges (the only ones a pixel
    // evaluates), summed afterwards in intersection order so the result does
    // not depend on the thread count.  row_of[tile] + (i - lo) is the row.
    std::vector<uint64_t> row_of((size_t)f->T + 1, 0);
    for (uint32_t t = 0; t < f->T; ++t) {
        const uint32_t lo = f->tile_offsets_shrunk[(size_t)t * 2], hi = f->tile_offsets_shrunk[(size_t)t * 2 + 1];
        row_of[t + 1] = row_of[t] + (hi > lo ? hi - lo : 0);
    }
    const int NG = f->surfel ? SURFEL_GRADS : 10;     // gradient components per splat
    std::vector<double> part((size_t)row_of[f->T] * NG, 0.0);
    const float img_w = (float)W, img_h = (float)H;

    // ---- raster VJP, bwd/kernels/rasterize_backwards_planes.rs:112-682 ----------
    #pragma omp parallel for schedule(dynamic, 1) num_threads(nthreads)
    for (int64_t ti = 0; ti < (int64_t)f->T; ++ti) {
        const uint32_t tile = (uint32_t)ti;
        const uint32_t tx = tile % f->tbw, ty = tile / f->tbw;
        const uint32_t lo = f->tile_offsets_shrunk[(size_t)tile * 2], hi = f->tile_offsets_shrunk[(size_t)tile * 2 + 1];
        if (hi <= lo) continue;
        for (uint32_t py = ty * TILE_W; py < ty * TILE_W + TILE_W; ++py) {
            for (uint32_t px = tx * TILE_W; px < tx * TILE_W + TILE_W; ++px) {
                if (px >= W || py >= H) continue;
                const size_t base = ((size_t)py * W + px) * C;
                const float final_a = f->out_img[base + 3];
                const float t_final = 1.0f - final_a;
                float sr = f->out_img[base] - t_final * f->bg[0];
                float sg = f->out_img[base + 1] - t_final * f->bg[1];
                float sb = f->out_img[base + 2] - t_final * f->bg[2];
                float T = 1.0f;
                const float vr = v_out[base], vg = v_out[base + 1], vb = v_out[base + 2];
                const float v_t = (v_out[base + 3] - (f->bg[0] * vr + f->bg[1] * vg + f->bg[2] * vb)) * t_final;
                const float refine_scale = 1.0f / fmax_(final_a, 1.0e-5f);
                const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
                if (f->surfel) {
                    // rasterize_backwards_planes.rs:266-480: the surfel replay, with the
                    // geometry channels composited like colours without a background.
                    double sz = f->out_img[base + 4], snx = f->out_img[base + 6], sny = f->out_img[base + 7];
                    double snz = f->out_img[base + 8], sdb = f->out_img[base + 9], sdc = f->out_img[base + 10];
                    double srd = sr, sgd = sg, sbd = sb;
                    const uint32_t med_id = f2u(f->out_img[base + 11]);
                    const double vz = v_out[base + 4], vmed = v_out[base + 5], vnx = v_out[base + 6];
                    const double vny = v_out[base + 7], vnz = v_out[base + 8], vdb = v_out[base + 9], vdc = v_out[base + 10];
                    for (uint32_t i = lo; i < hi && T > 1.0e-4f; ++i) {
                        const uint32_t c = f->isect_cid[i];
                        const float* row = &f->projected[(size_t)c * 9];
                        const float* a = &f->surf[(size_t)c * SURFEL_AUX];
                        const float opac = row[5], cr = row[6], cgc = row[7], cbc = row[8];
                        const SurfelHit h = surfel_hit(a, pcx, pcy);
                        if (!h.valid) continue;
                        const float sigma = h.sigma;
                        const float G = comp_exp2_c(-(sigma * LOG2E_F));
                        const float alpha = fmin_(0.999f, opac * G);
                        const float w_cut = smooth ? alpha_cutoff_weight(alpha) : ((alpha >= ALPHA_CUTOFF_MID) ? 1.0f : 0.0f);
                        if (!(sigma >= 0.0f && w_cut > 0.0f)) continue;
                        const float alpha_eff = alpha * w_cut;
                        const float next_t = T * (1.0f - alpha_eff);
                        if (next_t <= 1.0e-4f) { T = 0.0f; break; }
                        const float vis = alpha_eff * T;
                        double* p = &part[(size_t)(row_of[tile] + (i - lo)) * NG];
                        const double clr = fmax_(cr, 0.0f), clg = fmax_(cgc, 0.0f), clb = fmax_(cbc, 0.0f);
                        const double z = h.z, nx = a[11], ny = a[12], nz = a[13];
                        const double m = dist_depth(h.z);
                        const double dm_dz = (h.z > DIST_NEAR) ? (double)DIST_FAR / (DIST_FAR - DIST_NEAR) * DIST_NEAR / (z * z) : 0.0;
                        if (cr >= 0.0f) p[12] += (double)vis * vr;
                        if (cgc >= 0.0f) p[13] += (double)vis * vg;
                        if (cbc >= 0.0f) p[14] += (double)vis * vb;
                        p[9] += vis * vnx; p[10] += vis * vny; p[11] += vis * vnz;
                        const double Td = T;
                        const double ra = 1.0 / (1.0 - (double)alpha_eff);
                        const double dot = ((Td * clr - srd) * vr + (Td * clg - sgd) * vg + (Td * clb - sbd) * vb +
                                            (Td * z - sz) * vz + (Td * nx - snx) * vnx + (Td * ny - sny) * vny +
                                            (Td * nz - snz) * vnz + (Td * m - sdb) * vdb + (Td * m * m - sdc) * vdc) * ra;
                        const double v_alpha_eff = dot + (double)v_t * ra;
                        const double v_alpha = smooth ? v_alpha_eff * ((double)w_cut + (double)alpha * alpha_cutoff_weight_deriv(alpha)) : v_alpha_eff;
                        const double v_z = (double)vis * (vz + (vdb + 2.0 * m * vdc) * dm_dz) + (i == med_id ? vmed : 0.0);
                        const bool unsat = opac * G <= 0.999f;
                        const double v_sigma = unsat ? -(double)alpha * v_alpha : 0.0;
                        if (unsat) p[15] += v_alpha * (double)G;
                        const bool use_3d = h.s3d <= h.s2d;
                        const double su = h.su, sv = h.sv;
                        const double v_su = (use_3d ? v_sigma * su : 0.0) + v_z * a[6];
                        const double v_sv = (use_3d ? v_sigma * sv : 0.0) + v_z * a[7];
                        const double v_cx = use_3d ? 0.0 : -2.0 * v_sigma * h.dxs;
                        const double v_cy = use_3d ? 0.0 : -2.0 * v_sigma * h.dys;
                        const double inv_qz = 1.0 / (double)h.qz;
                        const double vqx = v_su * inv_qz, vqy = v_sv * inv_qz, vqz = -(v_su * su + v_sv * sv) * inv_qz;
                        // q = h_u x h_v: v_hu = h_v x v_q, v_hv = v_q x h_u
                        const double vhux = h.hvy * vqz - h.hvz * vqy, vhuy = h.hvz * vqx - h.hvx * vqz, vhuz = h.hvx * vqy - h.hvy * vqx;
                        const double vhvx = vqy * h.huz - vqz * h.huy, vhvy = vqz * h.hux - vqx * h.huz, vhvz = vqx * h.huy - vqy * h.hux;
                        const double inv_r2z = 1.0 / (double)a[8];
                        const double g0 = vhux, g1 = vhuy, g2 = vhuz + v_cx * inv_r2z;
                        const double g3 = vhvx, g4 = vhvy, g5 = vhvz + v_cy * inv_r2z;
                        const double g6 = v_z * su - pcx * vhux - pcy * vhvx;
                        const double g7 = v_z * sv - pcx * vhuy - pcy * vhvy;
                        const double g8 = v_z - pcx * vhuz - pcy * vhvz - (v_cx * a[9] + v_cy * a[10]) * inv_r2z;
                        p[0] += g0; p[1] += g1; p[2] += g2; p[3] += g3; p[4] += g4; p[5] += g5;
                        p[6] += g6; p[7] += g7; p[8] += g8;
                        // refine weight: the gradient of a screen-space shift of the surfel (M -> T M)
                        const double shx = g0 * a[6] + g1 * a[7] + g2 * a[8];
                        const double shy = g3 * a[6] + g4 * a[7] + g5 * a[8];
                        p[16] += std::sqrt(shx * img_w * shx * img_w + shy * img_h * shy * img_h) * (double)refine_scale;
                        srd -= vis * clr; sgd -= vis * clg; sbd -= vis * clb;
                        sz -= vis * z; snx -= vis * nx; sny -= vis * ny; snz -= vis * nz;
                        sdb -= vis * m; sdc -= vis * m * m;
                        T = next_t;
                    }
                    continue;
                }
                for (uint32_t i = lo; i < hi && T > 1.0e-4f; ++i) {
                    const float* row = &f->projected[(size_t)f->isect_cid[i] * 9];
                    const float x = row[0], y = row[1], c00 = row[2], c01 = row[3], c11 = row[4];
                    const float opac = row[5], cr = row[6], cgc = row[7], cbc = row[8];
                    const float dx = pcx - x, dy = pcy - y;
                    const float sigma = std::fma(std::fma((0.5f * c00) * LOG2E_F, dx, (c01 * LOG2E_F) * dy), dx,
                                                 (((0.5f * c11) * LOG2E_F) * dy) * dy);   // base 2, as the forward's
                    const float G = comp_exp2_c(-sigma);
                    const float alpha = fmin_(0.999f, opac * G);
                    const float w_cut = smooth ? alpha_cutoff_weight(alpha) : ((alpha >= ALPHA_CUTOFF_MID) ? 1.0f : 0.0f);
                    if (!(sigma >= 0.0f && w_cut > 0.0f)) continue;
                    const float alpha_eff = alpha * w_cut;
                    const float next_t = T * (1.0f - alpha_eff);
                    if (next_t <= 1.0e-4f) { T = 0.0f; break; }
                    const float vis = alpha_eff * T;
                    double* p = &part[(size_t)(row_of[tile] + (i - lo)) * NG];
                    const float clr = fmax_(cr, 0.0f), clg = fmax_(cgc, 0.0f), clb = fmax_(cbc, 0.0f);
                    if (cr >= 0.0f) p[5] += (double)vis * vr;
                    if (cgc >= 0.0f) p[6] += (double)vis * vg;
                    if (cbc >= 0.0f) p[7] += (double)vis * vb;
                    const double ra = 1.0 / (1.0 - (double)alpha_eff);
                    const double dot_rgb = (((double)T * clr - sr) * vr + ((double)T * clg - sg) * vg + ((double)T * clb - sb) * vb) * ra;
                    const double v_alpha_eff = dot_rgb + (double)v_t * ra;
                    const double v_alpha = smooth ? v_alpha_eff * ((double)w_cut + (double)alpha * alpha_cutoff_weight_deriv(alpha)) : v_alpha_eff;
                    const double v_sigma = -(double)alpha * v_alpha;
                    const double bdx = -(double)dx, bdy = -(double)dy;   // x - pixel
                    const double vxy_x = v_sigma * ((double)c00 * bdx + (double)c01 * bdy);
                    const double vxy_y = v_sigma * ((double)c01 * bdx + (double)c11 * bdy);
                    if (opac * G <= 0.999f) {
                        p[2] += 0.5 * v_sigma * bdx * bdx;
                        p[3] += v_sigma * bdx * bdy;
                        p[4] += 0.5 * v_sigma * bdy * bdy;
                        p[0] += vxy_x;
                        p[1] += vxy_y;
                        p[8] += v_alpha * (double)G;
                        p[9] += std::sqrt(vxy_x * img_w * vxy_x * img_w + vxy_y * img_h * vxy_y * img_h) * (double)refine_scale;
                    }
                    sr = sr - vis * clr;
                    sg = sg - vis * clg;
                    sb = sb - vis * clb;
                    T = next_t;
                }
            }
        }
    }
    // Per-splat sums in sorted-intersection order.
    std::vector<double> vc((size_t)N * NG, 0.0);
    for (uint32_t t = 0; t < f->T; ++t) {
        const uint32_t lo = f->tile_offsets_shrunk[(size_t)t * 2], hi = f->tile_offsets_shrunk[(size_t)t * 2 + 1];
        for (uint32_t i = lo; i < hi; ++i) {
            const uint32_t g = f->global_from_compact[f->isect_cid[i]];
            const double* p = &part[(size_t)(row_of[t] + (i - lo)) * NG];
            for (int k = 0; k < NG; ++k) vc[(size_t)g * NG + k] += p[k];
        }
    }
    std::vector<float> vcf((size_t)N * NG);
    for (size_t i = 0; i < (size_t)N * NG; ++i) vcf[i] = (float)vc[i];
    if (v_combined_out) std::memcpy(v_combined_out, vcf.data(), sizeof(float) * vcf.size());
    return project_vjp(f, vcf.data(), nthreads, v_transforms, v_sh, v_raw_opac, v_refine);
}

// ---- projection VJP, bwd/kernels/project_backwards.rs:132-424 -------------------
struct SplatVjp { V3 v_mean; Q4 v_q; V3 v_log; float v_raw; V3 vdir; };

// splat_vjp (project_backwards.rs:132-274) of global splat g with parameters
// row t [10] and raw opacity `raw` on its raster gradients rg [10].
static SplatVjp splat_vjp(const or_fwd* f, uint32_t g, const float* t, float raw, const float rg[10]) {
    const or_camera& u = f->cam;
    const uint32_t K = f->K, degree = f->degree;
    const float* cb = f->sh + (size_t)g * K * 3;
    const V3 mean = v3(t[0], t[1], t[2]);
    const V3 sc_raw = v3(expf_c(t[7] + f->lso), expf_c(t[8] + f->lso), expf_c(t[9] + f->lso));
    const Q4 qu{t[3], t[4], t[5], t[6]};
    const Q4 q = qnormalize(qu);
    const float opac_sig = sigmoid(raw);
    const ScaleFloor fl = apply_scale_floor(sc_raw, opac_sig, f->min_scale, g);
    const V3 sc = fl.scale;
    // SH + view-direction VJP
    const V3 u_world = sub(mean, V3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]});
    const float u_len = length(u_world);
    const V3 vdir = scale(u_world, 1.0f / u_len);
    const V3 v_color = v3(rg[5], rg[6], rg[7]);
    // Neural appearance adds its own view-direction term after (neural_backwards.rs).
    const V3 v_v_sh = f->decoder ? V3{0.0f, 0.0f, 0.0f} : sh_viewdir_vjp(cb, degree, vdir, v_color);
    const float v_dot = dot(vdir, v_v_sh);
    const V3 v_mean_sh = f->decoder ? V3{0.0f, 0.0f, 0.0f} : scale(sub(v_v_sh, scale(vdir, v_dot)), 1.0f / u_len);
    const V3 mean_c = world_to_cam(mean, u);
    const M3 R = quat_to_mat3(q);
    const M3 Mm = mul_diag(R, sc);
    float filter_comp;
    const S2 cov = compensate_cov2d(calc_cov2d(sc, q, mean_c, u), f->mip, filter_comp);
    // the compensated opacity's gradient (no path through filter_comp), 0 where the floor clamps
    const float v_opac_base = fl.opac_open ? filter_comp * rg[8] : 0.0f;
    const S2 conic_inv = s2_inverse(cov);
    const S2 v_inv{rg[2], rg[3] * 0.5f, rg[4]};
    const S2 v_cov2d = inverse2x2_vjp(conic_inv, v_inv);
    const S3 covar = outer_self(Mm);
    const M3 vrot = view_rot(u);
    const S3 cov_c = s3_congruence(covar, vrot);
    const M23 J = project_jacobian(mean_c, u);
    const V3 v_mean_c = projection_vjp(J, mean_c, cov_c, u, v_cov2d, V2{rg[0], rg[1]});
    const S3 vcc = m23_tcongruence_s2(J, v_cov2d);
    SplatVjp r;
    r.v_mean = add(tmul_vec3(vrot, v_mean_c), v_mean_sh);
    const M3 v_m = s3_mul_mat3(s3_scale(s3_tcongruence(vcc, vrot), 2.0f), Mm);
    const V3 v_log{dot(R.c0, v_m.c0) * sc.x, dot(R.c1, v_m.c1) * sc.y, dot(R.c2, v_m.c2) * sc.z};
    // through the floor: d log s' / d log s = ratio_sq, plus the opacity
    // compensation's d(opac) / d(log s_i) = opac (1 - ratio_sq_i)
    r.v_log = V3{v_log.x * fl.ratio_sq.x + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.x),
                 v_log.y * fl.ratio_sq.y + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.y),
                 v_log.z * fl.ratio_sq.z + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.z)};
    const Q4 q_grad = quat_to_mat_vjp(q, mul_diag(v_m, sc));
    r.v_q = apply_normalize_vjp(qu, q_grad);
    r.v_raw = v_opac_base * fl.coef * opac_sig * (1.0f - opac_sig);
    r.vdir = vdir;
    return r;
}

// surfel_backwards (project_backwards.rs:426-570) of global splat g from its
// 17 raster gradients [M rows (9), normal (3), rgb (3), alpha, refine]:
// M = K [s_u W R e0, s_v W R e1, W p + t], n = +-W R e2.
static void surfel_vjp(const or_fwd* f, uint32_t g, const float* rg, float* v_transforms, float* v_sh,
                       float* v_raw_opac, float* v_refine) {
    const or_camera& u = f->cam;
    const uint32_t K = f->K, degree = f->degree;
    const float* t = f->transforms + (size_t)g * 10;
    const float* cb = f->sh + (size_t)g * K * 3;
    const V3 mean = v3(t[0], t[1], t[2]);
    const V3 sc_raw = v3(expf_c(t[7] + f->lso), expf_c(t[8] + f->lso), expf_c(t[9] + f->lso));
    const Q4 qu{t[3], t[4], t[5], t[6]};
    const Q4 q = qnormalize(qu);
    const float opac_sig = sigmoid(f->raw_opac[g]);
    const ScaleFloor fl = apply_scale_floor(sc_raw, opac_sig, f->min_scale, g);
    const V3 sc = fl.scale;
    const V3 vc0{rg[0], rg[3], rg[6]}, vc1{rg[1], rg[4], rg[7]}, vc2{rg[2], rg[5], rg[8]};
    const V3 v_n{rg[9], rg[10], rg[11]}, v_color{rg[12], rg[13], rg[14]};
    const V3 u_world = sub(mean, V3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]});
    const float u_len = length(u_world);
    const V3 vdir = scale(u_world, 1.0f / u_len);
    if (v_sh) {
        float Y[25];
        const int n = sh_basis(degree, vdir, Y);
        float* o = v_sh + (size_t)g * K * 3;
        for (int k = 0; k < n; ++k) { o[3 * k] = v_color.x * Y[k]; o[3 * k + 1] = v_color.y * Y[k]; o[3 * k + 2] = v_color.z * Y[k]; }
    }
    const V3 v_v_sh = sh_viewdir_vjp(cb, degree, vdir, v_color);
    const V3 v_mean_sh = scale(sub(v_v_sh, scale(vdir, dot(vdir, v_v_sh))), 1.0f / u_len);
    const float v_opac_base = fl.opac_open ? rg[15] : 0.0f;         // no 2-D blur compensation
    if (v_raw_opac) v_raw_opac[g] = v_opac_base * fl.coef * opac_sig * (1.0f - opac_sig);
    if (v_refine) v_refine[g] = clampf(is_finite(rg[16]) ? rg[16] : 0.0f, 0.0f, 1.0e32f);
    // M = K X  =>  v_X = K^T v_M, column by column
    const V3 v_a{u.fx * vc0.x, u.fy * vc0.y, u.cx * vc0.x + u.cy * vc0.y + vc0.z};
    const V3 v_b{u.fx * vc1.x, u.fy * vc1.y, u.cx * vc1.x + u.cy * vc1.y + vc1.z};
    const V3 v_c{u.fx * vc2.x, u.fy * vc2.y, u.cx * vc2.x + u.cy * vc2.y + vc2.z};
    const M3 W = view_rot(u);
    const M3 wr = mul_mat3(W, quat_to_mat3(q));
    const V3 mean_c = world_to_cam(mean, u);
    const float v_su = dot(wr.c0, v_a), v_sv = dot(wr.c1, v_b);
    const float flip = dot(wr.c2, mean_c) > 0.0f ? -1.0f : 1.0f;
    const M3 v_r{scale(tmul_vec3(W, v_a), sc.x), scale(tmul_vec3(W, v_b), sc.y), scale(tmul_vec3(W, v_n), flip)};
    const Q4 v_q = apply_normalize_vjp(qu, quat_to_mat_vjp(q, v_r));
    const V3 v_mean = add(tmul_vec3(W, v_c), v_mean_sh);
    if (v_transforms) {
        float* o = v_transforms + (size_t)g * 10;
        o[0] = v_mean.x; o[1] = v_mean.y; o[2] = v_mean.z;
        o[3] = v_q.w; o[4] = v_q.x; o[5] = v_q.y; o[6] = v_q.z;
        o[7] = v_su * sc.x * fl.ratio_sq.x + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.x);
        o[8] = v_sv * sc.y * fl.ratio_sq.y + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.y);
        o[9] = v_opac_base * fl.opac * (1.0f - fl.ratio_sq.z);
    }
}

// Dense per-splat gradients from the raster VJP's v_combined [N,10]; rows of
// splats that were culled, or whose v_combined row is all zero, stay zero
// (bwd/kernels/project_backwards.rs:311-382).
static int project_vjp(const or_fwd* f, const float* vcf, int nthreads, float* v_transforms, float* v_sh,
                       float* v_raw_opac, float* v_refine) {
    const uint32_t N = f->N, K = f->K;
    if (v_transforms) std::memset(v_transforms, 0, sizeof(float) * (size_t)N * 10);
    if (v_sh) std::memset(v_sh, 0, sizeof(float) * (size_t)N * K * 3);
    if (v_raw_opac) std::memset(v_raw_opac, 0, sizeof(float) * N);
    if (v_refine) std::memset(v_refine, 0, sizeof(float) * N);
    const uint32_t degree = f->degree;
    #pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t ci = 0; ci < (int64_t)f->V; ++ci) {
        const uint32_t g = f->global_from_compact[(size_t)ci];
        if (f->surfel) {
            const float* rs = vcf + (size_t)g * SURFEL_GRADS;
            bool any_s = false;
            for (int k = 0; k < SURFEL_GRADS; ++k) any_s = any_s || rs[k] != 0.0f;
            if (any_s) surfel_vjp(f, g, rs, v_transforms, v_sh, v_raw_opac, v_refine);
            continue;
        }
        float rg[10];
        bool any = false;
        for (int k = 0; k < 10; ++k) { rg[k] = vcf[(size_t)g * 10 + k]; any = any || rg[k] != 0.0f; }
        if (!any) continue;
        const SplatVjp r = splat_vjp(f, g, f->transforms + (size_t)g * 10, f->raw_opac[g], rg);
        if (v_sh && !f->decoder) {
            // sh.rs:281-359: v_coeff_k = Y_k(v) v_colour
            float Y[25];
            const int n = sh_basis(degree, r.vdir, Y);
            float* o = v_sh + (size_t)g * K * 3;
            for (int k = 0; k < n; ++k) { o[3 * k] = rg[5] * Y[k]; o[3 * k + 1] = rg[6] * Y[k]; o[3 * k + 2] = rg[7] * Y[k]; }
        }
        if (v_raw_opac) v_raw_opac[g] = r.v_raw;
        if (v_refine) v_refine[g] = clampf(is_finite(rg[9]) ? rg[9] : 0.0f, 0.0f, 1.0e32f);
        if (v_transforms) {
            float* o = v_transforms + (size_t)g * 10;
            o[0] = r.v_mean.x; o[1] = r.v_mean.y; o[2] = r.v_mean.z;
            o[3] = r.v_q.w; o[4] = r.v_q.x; o[5] = r.v_q.y; o[6] = r.v_q.z;
            o[7] = r.v_log.x; o[8] = r.v_log.y; o[9] = r.v_log.z;
        }
    }
    return 0;
}

// ---- packed Adam moments, bwd/kernels/geo_moments.rs:1-127 ----------------------
// With Adam's epsilon e: u = m / (sqrt(v) + e) in the low 16 bits (sign +
// 15-bit magnitude over [0, 8]), l = ln(1 + sqrt(v) / e) as a 16-bit code over
// [0, 64] in the high half; sqrt(v) = e (exp(l) - 1), m = u e exp(l).
static const float GEO_U_CODES = 32767.0f, GEO_U_STEP = 8.0f / 32767.0f, GEO_U_PER_UNIT = 32767.0f / 8.0f;
static const float GEO_L_CODES = 65535.0f, GEO_L_STEP = 64.0f / 65535.0f, GEO_L_PER_UNIT = 65535.0f / 64.0f;

static float geo_growth(uint32_t word) { return expf_c((float)(word >> 16) * GEO_L_STEP); }      // :24-28
static float geo_normalized(uint32_t word) {                                                   // :30-35
    const float magnitude = (float)(word & 0x7fffu) * GEO_U_STEP;
    return (word & 0x8000u) ? -magnitude : magnitude;
}
static uint32_t pack_geo(float m, float v, float epsilon, float round_l, float round_u) {      // :37-56
    const float l = logf_c(1.0f + std::sqrt(fmax_(v, 0.0f)) / epsilon) * GEO_L_PER_UNIT;
    const float l_code = std::floor(clampf(l + round_l, 0.0f, GEO_L_CODES));
    const float sc = epsilon * expf_c(l_code * GEO_L_STEP);
    const float uu = std::fabs(m) / sc * GEO_U_PER_UNIT;
    const uint32_t u_code = (uint32_t)std::floor(clampf(uu + round_u, 0.0f, GEO_U_CODES));
    const uint32_t sign = (m < 0.0f) ? 0x8000u : 0u;
    return ((uint32_t)l_code << 16) | sign | u_code;
}
static uint32_t mix_hash(uint32_t index, uint32_t step) {                                      // :58-66
    uint32_t h = index ^ (step * 0x9e3779b9u);
    h = (h ^ (h >> 16)) * 0x7feb352du;
    h = (h ^ (h >> 15)) * 0x846ca68bu;
    return h ^ (h >> 16);
}
static void adam_packed(float& param, uint32_t& word, uint32_t index, float g, float lr, const or_adam& a,
                        uint32_t seed) {                                                          // :68-101
    const float growth = geo_growth(word);
    const float root = a.epsilon * (growth - 1.0f);
    const float m1 = geo_normalized(word) * (a.epsilon * growth) * a.beta1 + g * (1.0f - a.beta1);
    const float v1 = root * root * a.beta2 + g * g * (1.0f - a.beta2);
    const float step = (m1 * a.inv1) / (std::sqrt(v1 * a.inv2) + a.epsilon);
    param = param - step * lr;
    const uint32_t h = mix_hash(index, seed);
    word = pack_geo(m1, v1, a.epsilon, (float)(h >> 16) / 65536.0f, (float)(h & 0xffffu) / 65536.0f);
}

extern "C" uint32_t or_geo_encode(float m, float v, float epsilon) { return pack_geo(m, v, epsilon, 0.5f, 0.5f); }
extern "C" void or_geo_decode(uint32_t word, float epsilon, float* m, float* v) {
    const float growth = geo_growth(word);
    const float root = epsilon * (growth - 1.0f);
    *m = geo_normalized(word) * (epsilon * growth);
    *v = root * root;
}
extern "C" uint32_t or_geo_pack(float m, float v, float epsilon, float round_l, float round_u) {
    return pack_geo(m, v, epsilon, round_l, round_u);
}
extern "C" uint32_t or_mix_hash(uint32_t index, uint32_t step) { return mix_hash(index, step); }
extern "C" void or_adam_packed(float* param, uint32_t* word, uint32_t index, float g, float lr, const or_adam* a,
                               uint32_t seed) {
    adam_packed(*param, *word, index, g, lr, *a, seed);
}

// ---- IEEE binary16, the SH step's coefficient storage ------------------------------
namespace {
float f16_to_f32(uint16_t h) {
    const uint32_t sign = (uint32_t)(h & 0x8000u) << 16, e = (h >> 10) & 0x1Fu, man = h & 0x3FFu;
    if (e == 0) {
        const float v = (float)man * 5.9604644775390625e-08f;      // man * 2^-24, exact
        return (h & 0x8000u) ? -v : v;
    }
    if (e == 31) return u2f(sign | 0x7F800000u | (man << 13));
    return u2f(sign | ((e + 112u) << 23) | (man << 13));
}
// Round to nearest even; subnormals kept; >= 65520 in magnitude -> infinity.
uint16_t f32_to_f16(float f) {
    const uint32_t x = f2u(f), sign = (x >> 16) & 0x8000u, ax = x & 0x7FFFFFFFu;
    if (ax > 0x7F800000u) return (uint16_t)(sign | 0x7E00u | ((ax >> 13) & 0x3FFu));
    if (ax >= 0x477FF000u) return (uint16_t)(sign | 0x7C00u);
    if (ax < 0x38800000u) return (uint16_t)(sign | (uint32_t)std::nearbyint(u2f(ax) * 16777216.0f));
    const uint32_t r = ax - 0x38000000u;
    return (uint16_t)(sign | ((r + 0x0FFFu + ((r >> 13) & 1u)) >> 13));
}

// quant_kernels.rs:866-894.
float stochastic_half(float value, uint32_t index, uint32_t step) {
    const float magnitude = std::fabs(value);
    if (!(magnitude <= 65504.0f)) return value;
    float lower, upper;
    if (magnitude < 6.103515625e-05f) {
        lower = std::floor(magnitude * 16777216.0f) / 16777216.0f;
        upper = lower + 5.9604644775390625e-08f;
    } else {
        const uint32_t bits = f2u(magnitude) & 0xffffe000u;
        lower = u2f(bits);
        upper = u2f(bits + 8192u);
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

// Block-scaled 8-bit moment (quant.rs; pack_block / unpack, quant_kernels.rs:438-484).
constexpr uint32_t B8 = 128;
float b8_get(const uint32_t* codes, const float* scales, uint64_t i) {
    const uint32_t code = (codes[i / 4] >> ((i % 4) * 8)) & 255u;
    return ((float)code - 128.0f) * scales[i / B8];
}
// Pack one block's 128 moments (values past the end are 0).
void b8_pack(const float* m, uint64_t block, uint32_t* codes, float* scales) {
    float absmax = 0.0f;
    for (uint32_t i = 0; i < B8; ++i) absmax = fmax_(absmax, std::fabs(m[i]));
    const float scale = absmax / 127.0f;
    scales[block] = scale;
    for (uint32_t w = 0; w < B8 / 4; ++w) {
        uint32_t word = 0;
        for (uint32_t j = 0; j < 4; ++j) {
            uint32_t code = 128u;
            if (scale > 0.0f) code = (uint32_t)(std::nearbyint(clampf(m[4 * w + j] / scale, -127.0f, 127.0f)) + 128.0f);
            word |= code << (8 * j);
        }
        codes[block * (B8 / 4) + w] = word;
    }
}
} // namespace

extern "C" uint16_t or_f32_to_f16(float f) { return f32_to_f16(f); }
extern "C" float or_f16_to_f32(uint16_t h) { return f16_to_f32(h); }
extern "C" float or_stochastic_half(float value, uint32_t index, uint32_t step) {
    return stochastic_half(value, index, step);
}
extern "C" void or_block8_encode(const float* values, uint64_t n, uint32_t* codes, float* scales) {
    const uint64_t blocks = (n + B8 - 1) / B8;
    float m[B8];
    for (uint64_t b = 0; b < blocks; ++b) {
        for (uint32_t i = 0; i < B8; ++i) m[i] = b * B8 + i < n ? values[b * B8 + i] : 0.0f;
        b8_pack(m, b, codes, scales);
    }
}
extern "C" void or_block8_decode(const uint32_t* codes, const float* scales, uint64_t n, float* values) {
    for (uint64_t i = 0; i < n; ++i) values[i] = b8_get(codes, scales, i);
}
extern "C" void or_block8_zero_rows(uint32_t* codes, uint64_t n, const uint32_t* rows, uint32_t num_rows,
                                    uint32_t row_width) {
    for (uint32_t r = 0; r < num_rows; ++r)
        for (uint32_t c = 0; c < row_width; ++c) {
            const uint64_t i = (uint64_t)rows[r] * row_width + c;
            if (i >= n) continue;
            const uint32_t shift = (uint32_t)(i % 4) * 8;
            codes[i / 4] = (codes[i / 4] & ~(255u << shift)) | (128u << shift);
        }
}

// AdamScaled::step_sh_color (crates/splat-train/src/optim.rs:391-498) with
// the moment step of quant_kernels.rs:582-727, block by block: the second
// moment first (optim.rs:447-469), then each block holding a value of a splat
// with a gradient row is decoded, its values of such splats stepped (the
// coefficient gradient rebuilt as Y_k(dir) colour_c, quant_kernels.rs:569-577
// and 673-700) and the block re-packed; other blocks stay as they are.
extern "C" int or_sh_step(uint16_t* sh, uint32_t N, uint32_t degree, const float* color_dir, const uint32_t* grad_rows,
                          const float* grad_sq, float* variance, uint32_t* codes, float* scales, const float* lr_scale,
                          float beta1, float beta2, float inv1, float inv2, float epsilon, float lr,
                          uint32_t round_seed, int first) {
    if (degree > 4) return 1;
    const uint32_t K = (degree + 1) * (degree + 1), RW = K * 3;
    const uint64_t n = (uint64_t)N * RW, blocks = (n + B8 - 1) / B8;
    const float c2 = 1.0f - beta2;
    for (uint32_t g = 0; g < N; ++g) {
        if (first) variance[g] = grad_sq[g] * c2;
        else if (grad_rows[g] != 0u) variance[g] = variance[g] * beta2 + grad_sq[g] * c2;
    }
    const float factor = 1.0f - beta1;
    float m[B8];
    float Y[25];
    for (uint64_t b = 0; b < blocks; ++b) {
        bool any = false;
        for (uint32_t i = 0; i < B8 && !any; ++i) {
            const uint64_t idx = b * B8 + i;
            any = idx < n && grad_rows[idx / RW] != 0u;
        }
        if (!any) continue;
        for (uint32_t i = 0; i < B8; ++i) {
            const uint64_t idx = b * B8 + i;
            m[i] = idx < n ? b8_get(codes, scales, idx) : 0.0f;
            if (idx >= n) continue;
            const uint64_t row = idx / RW;
            const uint32_t gr = grad_rows[row];
            if (gr == 0u) continue;
            const uint32_t col = (uint32_t)(idx % RW), k = col / 3, c = col % 3;
            const float* cd = color_dir + (uint64_t)gr * 6;
            sh_basis(degree, v3(cd[3], cd[4], cd[5]), Y);
            const float gv = Y[k] * cd[c];
            const float moment = m[i] * beta1 + gv * factor;
            const float denom = std::sqrt(variance[row] * inv2) + epsilon;
            const float delta = (moment * inv1 / denom) * (lr_scale[col] * lr);
            sh[idx] = f32_to_f16(stochastic_half(f16_to_f32(sh[idx]) - delta, (uint32_t)idx, round_seed));
            m[i] = moment;
        }
        b8_pack(m, b, codes, scales);
    }
    return 0;
}

// ---- fused projection VJP + Adam, bwd/kernels/project_update.rs:40-178 ------------
extern "C" int or_project_update(const or_fwd* f, const float* v_combined, float* transforms, float* raw_opac,
                                 uint32_t* w_t, const float* lr_scale, uint32_t* w_o, const or_adam* a,
                                 float* color_dir, float* v_refine, float* grad_sq, int threads) {
    if (!f || !v_combined || !transforms || !raw_opac || !w_t || !lr_scale || !w_o || !a ||
        !(f->flags & OR_FLAG_BWD_INFO))
        return 1;
    const uint32_t N = f->N;
    std::vector<uint8_t> visible(N, 0);
    for (uint32_t c = 0; c < f->V; ++c) visible[f->global_from_compact[c]] = 1;
    if (color_dir) for (int k = 0; k < 6; ++k) color_dir[k] = 0.0f;
    const uint32_t seed_t = a->round_seed ^ (10u << 24), seed_o = a->round_seed ^ (1u << 24);
    #pragma omp parallel for schedule(static) num_threads(resolve_threads(threads))
    for (int64_t gi = 0; gi < (int64_t)N; ++gi) {
        const uint32_t g = (uint32_t)gi;
        float* t = transforms + (size_t)g * 10;
        float grad[10] = {0, 0, 0, 0, 0, 0, 0, 0, 0, 0};
        float g_opac = 0.0f, refine = 0.0f, gsq = 0.0f;
        if (visible[g]) {
            const float* rg = v_combined + (size_t)g * 10;
            bool any = false;
            for (int k = 0; k < 10; ++k) any = any || rg[k] != 0.0f;
            float* cd = color_dir ? color_dir + (size_t)(g + 1) * 6 : nullptr;
            if (any) {
                const SplatVjp r = splat_vjp(f, g, t, raw_opac[g], rg);
                if (cd) { cd[0] = rg[5]; cd[1] = rg[6]; cd[2] = rg[7]; cd[3] = r.vdir.x; cd[4] = r.vdir.y; cd[5] = r.vdir.z; }
                grad[0] = r.v_mean.x; grad[1] = r.v_mean.y; grad[2] = r.v_mean.z;
                grad[3] = r.v_q.w; grad[4] = r.v_q.x; grad[5] = r.v_q.y; grad[6] = r.v_q.z;
                grad[7] = r.v_log.x; grad[8] = r.v_log.y; grad[9] = r.v_log.z;
                g_opac = r.v_raw;
                refine = clampf(is_finite(rg[9]) ? rg[9] : 0.0f, 0.0f, 1.0e32f);
                // project_update.rs:133-140: the SH row's mean square from its DC
                // entries (SH C0 = 0.2820948, kernels/sh.rs:17)
                const float c0 = 0.2820948f * rg[5], c1 = 0.2820948f * rg[6], c2 = 0.2820948f * rg[7];
                gsq = (c0 * c0 + c1 * c1 + c2 * c2) / 3.0f;
            } else if (cd) {
                for (int k = 0; k < 6; ++k) cd[k] = 0.0f;
            }
        } else if (color_dir) {
            for (int k = 0; k < 6; ++k) color_dir[(size_t)(g + 1) * 6 + k] = 0.0f;
        }
        if (v_refine) v_refine[g] = refine;
        if (grad_sq) grad_sq[g] = gsq;
        float raw = raw_opac[g];
        const float o = 1.0f / (1.0f + expf_c(-raw));
        g_opac += a->opac_reg * o * (1.0f - o);
        for (int k = 0; k < 10; ++k)
            adam_packed(t[k], w_t[(size_t)g * 10 + k], g * 10u + (uint32_t)k, grad[k], lr_scale[k], *a, seed_t);
        adam_packed(raw, w_o[g], g, g_opac, a->lr_opac, *a, seed_o);
        raw_opac[g] = raw;
    }
    return 0;
}

// ---- neural appearance backward, bwd/kernels/neural_backwards.rs:141-283 ---------
// One visible splat with a colour gradient: its row gradient [base (DC
// units), latents, 0] and the row's mean square, its view-direction mean
// gradient, and its decoder weight products added to dW (f64).
static void neural_row_backward(const or_fwd* f, uint32_t g, V3 vc, float* v_row, float& sq_out, V3& v_mean,
                                double* dW, double* dW_abs) {
    const or_camera& u = f->cam;
    const float* W = f->decoder;
    const float* row = f->sh + (size_t)g * NEURAL_ROW;
    const float* t = f->transforms + (size_t)g * 10;
    const V3 u_world = sub(v3(t[0], t[1], t[2]), V3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]});
    const float u_len = length(u_world);
    const V3 dir = scale(u_world, 1.0f / u_len);
    NeuralAct a;
    neural_forward(row, W, dir, f->degree, a);
    const float gc3[3] = {vc.x, vc.y, vc.z};
    float sq = 0.0f, go[3];
    for (int c = 0; c < 3; ++c) {
        const float th = tanhf_c(a.o[c]);
        const float base = row[c] * SH_C0;
        const float gcol = (base + th + 0.5f > 0.0f) ? gc3[c] : 0.0f;     // ReLU of the colour
        v_row[c] = gcol * SH_C0;
        sq += (gcol * SH_C0) * (gcol * SH_C0);
        go[c] = gcol * (1.0f - th * th);
    }
    float d2[NEURAL_HIDDEN], d1[NEURAL_HIDDEN], dx[NEURAL_INPUTS];
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
        float acc = 0.0f;
        for (int c = 0; c < 3; ++c) acc += W[NEURAL_W3 + c * NEURAL_HIDDEN + k] * go[c];
        d2[k] = (a.h2[k] > 0.0f) ? acc : 0.0f;
    }
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
        float acc = 0.0f;
        for (int j = 0; j < NEURAL_HIDDEN; ++j) acc += W[NEURAL_W2 + j * NEURAL_HIDDEN + k] * d2[j];
        d1[k] = (a.h1[k] > 0.0f) ? acc : 0.0f;
    }
    for (int k = 0; k < NEURAL_INPUTS; ++k) {
        float acc = 0.0f;
        for (int j = 0; j < NEURAL_HIDDEN; ++j) acc += W[NEURAL_W1 + j * NEURAL_INPUTS + k] * d1[j];
        dx[k] = acc;
    }
    // latents through sin / cos
    for (int i = 0; i < NEURAL_LATENTS; ++i) {
        const float gl = dx[2 * i] * a.x[2 * i + 1] - dx[2 * i + 1] * a.x[2 * i];
        v_row[3 + i] = gl;
        sq += gl * gl;
    }
    v_row[11] = 0.0f;
    sq_out = sq / (float)NEURAL_ROW;
    const V3 g_dir = direction_basis_vjp(dx, dir, f->degree);
    v_mean = scale(sub(g_dir, scale(dir, dot(dir, g_dir))), 1.0f / u_len);
    auto add = [&](int w, float p) { dW[w] += (double)p; dW_abs[w] += std::fabs((double)p); };
    for (int j = 0; j < NEURAL_HIDDEN; ++j)
        for (int k = 0; k < NEURAL_INPUTS; ++k) add(NEURAL_W1 + j * NEURAL_INPUTS + k, d1[j] * a.x[k]);
    for (int j = 0; j < NEURAL_HIDDEN; ++j)
        for (int k = 0; k < NEURAL_HIDDEN; ++k) add(NEURAL_W2 + j * NEURAL_HIDDEN + k, d2[j] * a.h1[k]);
    for (int c = 0; c < 3; ++c)
        for (int k = 0; k < NEURAL_HIDDEN; ++k) add(NEURAL_W3 + c * NEURAL_HIDDEN + k, go[c] * a.h2[k]);
}

// project_bwd_neural's neural half (bwd/render_bwd.rs:390-435): rows [N,12],
// their mean squares [N], the decoder gradient [816] summed in f64, and each
// row's view-direction term added to v_transforms' mean (in/out; may be NULL).
extern "C" int or_neural_backward(const or_fwd* f, const float* v_combined, int threads, float* v_transforms,
                                  float* v_rows, float* v_rows_sq, float* v_decoder, double* v_decoder_abs) {
    if (!f || !v_combined || !f->decoder || !(f->flags & OR_FLAG_BWD_INFO)) return 1;
    const uint32_t N = f->N;
    if (v_rows) std::memset(v_rows, 0, sizeof(float) * (size_t)N * NEURAL_ROW);
    if (v_rows_sq) std::memset(v_rows_sq, 0, sizeof(float) * N);
    const int nthreads = resolve_threads(threads);
    std::vector<double> dW((size_t)nthreads * NEURAL_LEN, 0.0), dW_abs((size_t)nthreads * NEURAL_LEN, 0.0);
    std::vector<float> means((size_t)N * 3, 0.0f);
    std::vector<uint8_t> active(N, 0);
    #pragma omp parallel num_threads(nthreads)
    {
#ifdef _OPENMP
        double* mine = &dW[(size_t)omp_get_thread_num() * NEURAL_LEN];
        double* mine_abs = &dW_abs[(size_t)omp_get_thread_num() * NEURAL_LEN];
#else
        double* mine = dW.data();
        double* mine_abs = dW_abs.data();
#endif
        #pragma omp for schedule(static)
        for (int64_t ci = 0; ci < (int64_t)f->V; ++ci) {
            const uint32_t g = f->global_from_compact[(size_t)ci];
            const float* rg = v_combined + (size_t)g * 10;
            const V3 vc = v3(rg[5], rg[6], rg[7]);
            if (vc.x == 0.0f && vc.y == 0.0f && vc.z == 0.0f) continue;
            float row[NEURAL_ROW], sq;
            V3 vm;
            neural_row_backward(f, g, vc, row, sq, vm, mine, mine_abs);
            if (v_rows) std::memcpy(v_rows + (size_t)g * NEURAL_ROW, row, sizeof(row));
            if (v_rows_sq) v_rows_sq[g] = sq;
            means[(size_t)g * 3] = vm.x; means[(size_t)g * 3 + 1] = vm.y; means[(size_t)g * 3 + 2] = vm.z;
            active[g] = 1;
        }
    }
    if (v_transforms)
        for (uint32_t g = 0; g < N; ++g)
            if (active[g])
                for (int k = 0; k < 3; ++k) v_transforms[(size_t)g * 10 + k] += means[(size_t)g * 3 + k];
    if (v_decoder)
        for (int w = 0; w < NEURAL_LEN; ++w) {
            double acc = 0.0;
            for (int t = 0; t < nthreads; ++t) acc += dW[(size_t)t * NEURAL_LEN + w];
            v_decoder[w] = (float)acc;
        }
    if (v_decoder_abs)
        for (int w = 0; w < NEURAL_LEN; ++w) {
            double acc = 0.0;
            for (int t = 0; t < nthreads; ++t) acc += dW_abs[(size_t)t * NEURAL_LEN + w];
            v_decoder_abs[w] = acc;
        }
    return 0;
}

// ---- camera gradient, bwd/kernels/pose_backwards.rs:1-191 -------------------------
// The camera is perturbed by x_c' = (I + A) x_c + b after the world-to-camera
// transform; A pivots on the camera centre, which b moves by -M^-1 b.
static V3 cross3(V3 a, V3 b) {
    return V3{a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}
// pose_backwards.rs:61-74: M^-T g from the column cross products over det M.
static V3 inverse_transpose_mul(M3 m, V3 g) {
    const V3 k0 = cross3(m.c1, m.c2), k1 = cross3(m.c2, m.c0), k2 = cross3(m.c0, m.c1);
    return scale(add(add(scale(k0, g.x), scale(k1, g.y)), scale(k2, g.z)), 1.0f / dot(m.c0, k0));
}
// pose_backwards_kernel (pose_backwards.rs:88-191) for global splat g: the row
// [v x^T + 2 V S (row-major 3x3), db]; false (zero row) when the raster
// gradients of position, conic and colour are all zero.
static bool pose_row(const or_fwd* f, uint32_t g, const float rg[10], float row[12]) {
    for (int k = 0; k < 12; ++k) row[k] = 0.0f;
    bool any = false;
    for (int k = 0; k < 8; ++k) any = any || rg[k] != 0.0f;
    if (!any) return false;
    const or_camera& u = f->cam;
    const float* t = f->transforms + (size_t)g * 10;
    const V3 mean = v3(t[0], t[1], t[2]);
    const V3 sc_raw = v3(expf_c(t[7] + f->lso), expf_c(t[8] + f->lso), expf_c(t[9] + f->lso));
    const Q4 q = qnormalize(Q4{t[3], t[4], t[5], t[6]});
    const V3 sc = apply_scale_floor(sc_raw, sigmoid(f->raw_opac[g]), f->min_scale, g).scale;
    // SH view direction: only the camera centre moves it.
    const V3 u_world = sub(mean, V3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]});
    const float u_len = length(u_world);
    const V3 dir = scale(u_world, 1.0f / u_len);
    const V3 v_dir = sh_viewdir_vjp(f->sh + (size_t)g * f->K * 3, f->degree, dir, v3(rg[5], rg[6], rg[7]));
    const V3 v_mean_sh = scale(sub(v_dir, scale(dir, dot(dir, v_dir))), 1.0f / u_len);
    const V3 mean_c = world_to_cam(mean, u);
    float filter_comp;
    const S2 cov = compensate_cov2d(calc_cov2d(sc, q, mean_c, u), f->mip, filter_comp);
    const S2 v_cov2d = inverse2x2_vjp(s2_inverse(cov), S2{rg[2], rg[3] * 0.5f, rg[4]});
    const M3 vrot = view_rot(u);
    const S3 cov_c = s3_congruence(outer_self(mul_diag(quat_to_mat3(q), sc)), vrot);
    const M23 J = project_jacobian(mean_c, u);
    const V3 v = projection_vjp(J, mean_c, cov_c, u, v_cov2d, V2{rg[0], rg[1]});
    const S3 V = m23_tcongruence_s2(J, v_cov2d);
    const V3 vb = add(v, inverse_transpose_mul(vrot, v_mean_sh));
    const V3 vr[3] = {V3{V.c00, V.c01, V.c02}, V3{V.c01, V.c11, V.c12}, V3{V.c02, V.c12, V.c22}};
    const V3 sr[3] = {V3{cov_c.c00, cov_c.c01, cov_c.c02}, V3{cov_c.c01, cov_c.c11, cov_c.c12},
                      V3{cov_c.c02, cov_c.c12, cov_c.c22}};
    const float vv[3] = {v.x, v.y, v.z}, xx[3] = {mean_c.x, mean_c.y, mean_c.z};
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) row[3 * i + j] = vv[i] * xx[j] + 2.0f * dot(vr[i], sr[j]);
    row[9] = vb.x; row[10] = vb.y; row[11] = vb.z;
    return true;
}

// SplatBwdOps::pose_bwd (bwd/render_bwd.rs:224-288): the rows summed over the
// visible splats in f64; `rows` [N,12] (optional) receives each splat's row.
extern "C" int or_pose_backward(const or_fwd* f, const float* v_combined, int threads, double* v_pose, float* rows) {
    if (!f || !v_combined || !v_pose || !(f->flags & OR_FLAG_BWD_INFO)) return 1;
    const uint32_t N = f->N;
    std::vector<float> all((size_t)N * 12, 0.0f);
    const int nthreads = resolve_threads(threads);
    #pragma omp parallel for schedule(static) num_threads(nthreads)
    for (int64_t ci = 0; ci < (int64_t)f->V; ++ci) {
        const uint32_t g = f->global_from_compact[(size_t)ci];
        pose_row(f, g, v_combined + (size_t)g * 10, &all[(size_t)g * 12]);
    }
    for (int k = 0; k < 12; ++k) v_pose[k] = 0.0;
    for (uint32_t ci = 0; ci < f->V; ++ci) {
        const uint32_t g = f->global_from_compact[ci];
        for (int k = 0; k < 12; ++k) v_pose[k] += (double)all[(size_t)g * 12 + k];
    }
    if (rows) std::memcpy(rows, all.data(), sizeof(float) * all.size());
    return 0;
}

extern "C" int or_project_backward(const or_fwd* f, const float* v_combined, int threads, float* v_transforms,
                                   float* v_sh, float* v_raw_opac, float* v_refine) {
    if (!f || !v_combined || !(f->flags & OR_FLAG_BWD_INFO)) return 1;
    return project_vjp(f, v_combined, resolve_threads(threads), v_transforms, v_sh, v_raw_opac, v_refine);
}

// ---- sort & scan ---------------------------------------------------------------
extern "C" void or_radix_argsort_u32(const uint32_t* keys, const uint32_t* vals, uint32_t n,
                                     uint32_t skip_bits, uint32_t sorting_bits,
                                     uint32_t* out_keys, uint32_t* out_vals) {
    if (n == 0) return;
    if (sorting_bits == 0) {
        std::memcpy(out_keys, keys, sizeof(uint32_t) * n);
        std::memcpy(out_vals, vals, sizeof(uint32_t) * n);
        return;
    }
    const uint32_t passes = (sorting_bits + 7) / 8;
    const uint32_t width = passes * 8;
    const uint64_t mask = (width >= 64) ? ~0ull : ((1ull << width) - 1ull);
    std::vector<uint32_t> idx(n);
    std::iota(idx.begin(), idx.end(), 0u);
    std::stable_sort(idx.begin(), idx.end(), [&](uint32_t a, uint32_t b) {
        return (((uint64_t)keys[a] >> skip_bits) & mask) < (((uint64_t)keys[b] >> skip_bits) & mask);
    });
    for (uint32_t i = 0; i < n; ++i) { out_keys[i] = keys[idx[i]]; out_vals[i] = vals[idx[i]]; }
}

extern "C" void or_prefix_sum_u32(const uint32_t* in, uint32_t* out, uint32_t n) {
    uint32_t acc = 0;
    for (uint32_t i = 0; i < n; ++i) { acc += in[i]; out[i] = acc; }
}

// ---- exported math -------------------------------------------------------------
extern "C" float or_expf(float x) { return expf_c(x); }
extern "C" void or_exp2n_n(const float* x, float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = exp2n_c(x[i]);
}
extern "C" void or_set_comp_exp2_table(const float* tab, uint32_t first_bits, uint64_t count) {
    g_exp2_tab = (tab && count) ? tab : nullptr;
    g_exp2_first = first_bits;
    g_exp2_count = g_exp2_tab ? count : 0;
}
extern "C" float or_logf(float x) { return logf_c(x); }
extern "C" float or_atan2f(float y, float x) { return atan2f_c(y, x); }
extern "C" void or_expf_n(const float* x, float* y, uint64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) y[i] = expf_c(x[i]);
}
extern "C" void or_logf_n(const float* x, float* y, uint64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) y[i] = logf_c(x[i]);
}
extern "C" void or_sincosf_n(const float* x, float* s, float* c, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) sincosf_c(x[i], s[i], c[i]);
}
extern "C" void or_tanhf_n(const float* x, float* y, uint64_t n) {
    for (uint64_t i = 0; i < n; ++i) y[i] = tanhf_c(x[i]);
}
// The neural decoder's colour for one row and direction (test hook).
extern "C" void or_neural_color(const float row[12], const float decoder[816], const float dir[3], uint32_t degree,
                                float out[3]) {
    const V3 c = neural_color(row, decoder, V3{dir[0], dir[1], dir[2]}, degree);
    out[0] = c.x; out[1] = c.y; out[2] = c.z;
}
extern "C" void or_atan2f_n(const float* y, const float* x, float* r, uint64_t n) {
    #pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < (int64_t)n; ++i) r[i] = atan2f_c(y[i], x[i]);
}
extern "C" void or_sh_basis(uint32_t degree, const float v[3], float* out) {
    sh_basis(degree, v3(v[0], v[1], v[2]), out);
}

// ---- camera host math, camera.rs:99-237 (f64) ----------------------------------
namespace {
double kb4_d(double th, const float* k) {
    const double t2 = th * th, t3 = t2 * th, t5 = t3 * t2, t7 = t5 * t2, t9 = t7 * t2;
    return th + (double)k[0] * t3 + (double)k[1] * t5 + (double)k[2] * t7 + (double)k[3] * t9;
}
double kb4_dd(double th, const float* k) {
    const double t2 = th * th, t4 = t2 * t2, t6 = t4 * t2, t8 = t6 * t2;
    return 1.0 + 3.0 * (double)k[0] * t2 + 5.0 * (double)k[1] * t4 + 7.0 * (double)k[2] * t6 + 9.0 * (double)k[3] * t8;
}
double kb4_fold(const float* k) {
    const int STEPS = 128;
    const double step = M_PI / STEPS;
    double lo = 0.0, hi = M_PI;
    bool found = false;
    for (int i = 1; i <= STEPS; ++i) {
        const double th = i * step;
        if (kb4_dd(th, k) <= 0.0) { hi = th; found = true; break; }
        lo = th;
    }
    if (!found) return M_PI;
    for (int it = 0; it < 64; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (kb4_dd(mid, k) > 0.0) lo = mid; else hi = mid;
        if (hi - lo < 1e-12) break;
    }
    return 0.5 * (lo + hi);
}
double kb4_inv(double target, const float* k) {
    if (target <= 0.0) return 0.0;
    const double fold = kb4_fold(k);
    if (target >= kb4_d(fold, k)) return fold;
    double lo = 0.0, hi = fold;
    for (int it = 0; it < 100; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (kb4_d(mid, k) < target) lo = mid; else hi = mid;
        if (hi - lo < 1e-14) break;
    }
    return 0.5 * (lo + hi);
}
// camera.rs:238-303: the RT8 radial factor and its two inverses.
double rt8_radial(double r, const float* k) {
    const double r2 = r * r, r4 = r2 * r2, r6 = r4 * r2;
    return (1.0 + (double)k[0] * r2 + (double)k[1] * r4 + (double)k[2] * r6) /
           (1.0 + (double)k[3] * r2 + (double)k[4] * r4 + (double)k[5] * r6);
}
double rt8_undistort(double r_d, const float* k) {
    double r = r_d;
    for (int it = 0; it < 30; ++it) {
        const double f = rt8_radial(r, k);
        if (std::fabs(f) < 1e-12) break;
        const double nr = r_d / f;
        if (std::fabs(nr - r) < 1e-12) { r = nr; break; }
        r = nr;
    }
    return r;
}
double rt8_corner(double r_d, const float* k) {     // < 0: no crossing below r = 16
    const double step = 16.0 / 4096;
    double lo = 0.0, hi = -1.0;
    for (int i = 1; i <= 4096; ++i) {
        const double r = i * step;
        if (r * rt8_radial(r, k) >= r_d) { hi = r; break; }
        lo = r;
    }
    if (hi < 0.0) return -1.0;
    for (int it = 0; it < 64; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (mid * rt8_radial(mid, k) < r_d) lo = mid; else hi = mid;
        if (hi - lo < 1e-12) break;
    }
    return 0.5 * (lo + hi);
}
} // namespace

extern "C" double or_rt8_radial(double r, const float dist[8]) { return rt8_radial(r, dist); }
extern "C" double or_rt8_undistort_radius(double r_d, const float dist[8]) { return rt8_undistort(r_d, dist); }
extern "C" double or_rt8_undistort_corner_radius(double r_d, const float dist[8]) { return rt8_corner(r_d, dist); }
// calculate_jacobian_clamp_limits (camera.rs:305-374) for a model and pinhole
// parameters: out = lim_pos_x, lim_pos_y, lim_neg_x, lim_neg_y, lim_r.
extern "C" void or_clamp_limits(int model, uint32_t img_w, uint32_t img_h, float fx, float fy, float cx, float cy,
                                const float dist[8], float out[5]) {
    const float w = (float)img_w, h = (float)img_h;
    out[0] = out[1] = out[2] = out[3] = 0.0f;
    out[4] = 3.40282347e+38f;
    const float epx = (1.15f * w - cx) / fx, epy = (1.15f * h - cy) / fy;
    const float enx = (-0.15f * w - cx) / fx, eny = (-0.15f * h - cy) / fy;
    if (model == OR_MODEL_PINHOLE) {
        out[0] = epx; out[1] = epy; out[2] = enx; out[3] = eny;
    } else if (model == OR_MODEL_RT8) {
        auto und = [&](float e) {
            const float sgn = std::signbit(e) ? -1.0f : 1.0f;
            return (float)rt8_undistort((double)std::fabs(e), dist) * sgn;
        };
        out[0] = und(epx); out[1] = und(epy); out[2] = und(enx); out[3] = und(eny);
        const double cd = std::hypot((double)fmax_(std::fabs(epx), std::fabs(enx)),
                                     (double)fmax_(std::fabs(epy), std::fabs(eny)));
        const double r = rt8_corner(cd, dist);
        if (r >= 0.0) out[4] = (float)r;
    }
}

extern "C" double or_kb4_d(double theta, const float kb4[4]) { return kb4_d(theta, kb4); }
extern "C" double or_kb4_dd_dtheta(double theta, const float kb4[4]) { return kb4_dd(theta, kb4); }
extern "C" double or_kb4_invert_d(double target, const float kb4[4]) { return kb4_inv(target, kb4); }
// params: kb4 k1..k4 then dist[8]
extern "C" double or_fov_to_focal(double fov, uint32_t pixels, int model, const float params[12]) {
    const double half = fov / 2.0;
    const double r_pix = (double)pixels / 2.0;
    double projected;
    if (model == OR_MODEL_KB4 || model == OR_MODEL_TPF) projected = kb4_d(half, params);
    else if (model == OR_MODEL_RT8) { const double r = std::tan(half); projected = r * rt8_radial(r, params + 4); }
    else projected = std::tan(half);
    return r_pix / projected;
}
extern "C" double or_focal_to_fov(double focal, uint32_t pixels, int model, const float params[12]) {
    const double r_pix = (double)pixels / 2.0;
    const double r_norm = r_pix / focal;
    double half;
    if (model == OR_MODEL_KB4 || model == OR_MODEL_TPF) half = kb4_inv(r_norm, params);
    else if (model == OR_MODEL_RT8) half = std::atan(rt8_undistort(r_norm, params + 4));
    else half = std::atan(r_norm);
    return 2.0 * half;
}
extern "C" double or_max_render_theta(int model, const float params[12]) {
    return (model == OR_MODEL_KB4 || model == OR_MODEL_TPF) ? kb4_fold(params) : M_PI;
}

// ---- image loss: L1 + SSIM, crates/splat-train-loss/src/lib.rs:226-1306 ------------
// gauss_taps() (lib.rs:48-62): exp(-x^2 / 4.5), x = -5..5, in f32, normalised
// by their f32 sum; the literals are those f32 values.
static const float LOSS_GW[11] = {0x1.0d957p-10f, 0x1.f1fe04p-8f, 0x1.26eb18p-5f, 0x1.bff1p-4f, 0x1.b43c4p-3f,
                                  0x1.106562p-2f, 0x1.b43c4p-3f, 0x1.bff1p-4f, 0x1.26eb18p-5f, 0x1.f1fe04p-8f,
                                  0x1.0d957p-10f};
static const float LOSS_C1 = 0.01f * 0.01f, LOSS_C2 = 0.03f * 0.03f, LOSS_INV_255 = 1.0f / 255.0f;
static const uint32_t LOSS_TILE = 16;

namespace {
struct LossImg {
    uint32_t h, w, cn;
    const float* pred;
    const uint32_t* gt;
    const or_loss_cfg* cfg;
    float gt_c(uint32_t y, uint32_t x, uint32_t c) const { return (float)((gt[(size_t)y * w + x] >> (c * 8)) & 0xffu) * LOSS_INV_255; }
    float gt_a(uint32_t y, uint32_t x) const { return (float)((gt[(size_t)y * w + x] >> 24) & 0xffu) * LOSS_INV_255; }
    // read_gt + compositing (lib.rs:161-183, 318-323)
    float gt_eff(uint32_t y, uint32_t x, uint32_t c) const {
        const float g = gt_c(y, x, c);
        return cfg->composite ? g + (1.0f - gt_a(y, x)) * cfg->bg[c] : g;
    }
    float p(uint32_t y, uint32_t x, uint32_t c) const { return pred[((size_t)y * w + x) * cn + c]; }
    uint32_t tiles_x() const { return (w + LOSS_TILE - 1) / LOSS_TILE; }
    uint32_t tiles() const { return tiles_x() * ((h + LOSS_TILE - 1) / LOSS_TILE); }
    uint32_t tile_of(uint32_t y, uint32_t x) const { return (y / LOSS_TILE) * tiles_x() + x / LOSS_TILE; }
};

// Separable 11-tap blur of `n` per-pixel values with zero outside the image,
// in the kernels' order: per tap distance d = 1..5, sum += (left + right) * w,
// then the centre tap; rows first, then columns (lib.rs:326-414).
// src(y, x, k) gives value k at an in-image pixel; out is [h][w][n].
template <typename F>
void blur(const LossImg& im, int n, F src, std::vector<float>& out) {
    const uint32_t h = im.h, w = im.w;
    std::vector<float> hs((size_t)h * w * n);
    std::vector<float> row((size_t)(w + 10) * n);
    for (uint32_t y = 0; y < h; ++y) {
        std::fill(row.begin(), row.end(), 0.0f);
        for (uint32_t x = 0; x < w; ++x)
            for (int k = 0; k < n; ++k) row[(size_t)(x + 5) * n + k] = src(y, x, k);
        for (uint32_t x = 0; x < w; ++x)
            for (int k = 0; k < n; ++k) {
                float s = 0.0f;
                for (int d = 1; d <= 5; ++d) s += (row[(size_t)(x + 5 - d) * n + k] + row[(size_t)(x + 5 + d) * n + k]) * LOSS_GW[5 - d];
                s += row[(size_t)(x + 5) * n + k] * LOSS_GW[5];
                hs[((size_t)y * w + x) * n + k] = s;
            }
    }
    out.assign((size_t)h * w * n, 0.0f);
    auto hv = [&](int64_t y, uint32_t x, int k) { return (y < 0 || y >= (int64_t)h) ? 0.0f : hs[((size_t)y * w + x) * n + k]; };
    for (uint32_t y = 0; y < h; ++y)
        for (uint32_t x = 0; x < w; ++x)
            for (int k = 0; k < n; ++k) {
                float s = 0.0f;
                for (int d = 1; d <= 5; ++d) s += (hv((int64_t)y - d, x, k) + hv((int64_t)y + d, x, k)) * LOSS_GW[5 - d];
                s += hv(y, x, k) * LOSS_GW[5];
                out[((size_t)y * w + x) * n + k] = s;
            }
}

// Sum of a 16x16 tile's 256 values (tid = row * 16 + col, zero past the
// image) by the halving tree tile_sum (lib.rs:112-128) uses.
float tile_tree_sum(float* v) {
    for (uint32_t stride = 128; stride >= 1; stride >>= 1)
        for (uint32_t t = 0; t < stride; ++t) v[t] += v[t + stride];
    return v[0];
}
} // namespace

// image_loss_forward_kernel (lib.rs:238-478) for every plane, writing the
// reduced partials [planes, tiles], the per-pixel SSIM coefficients [3][3][H,W]
// (dmu1, dsigma1, dsigma12 per channel) and the loss map [H,W,cn]; NULL skips.
extern "C" int or_image_loss_forward(const float* pred, uint32_t cn, const uint32_t* gt, uint32_t w, uint32_t h,
                                     const or_loss_cfg* cfg, float* partials, float* coeffs, float* loss_map) {
    if (!pred || !gt || !cfg || (cn != 3 && cn != 4) || w == 0 || h == 0) return 1;
    const LossImg im{h, w, cn, pred, gt, cfg};
    const bool alpha_match = cfg->alpha_weight > 0.0f && cn == 4;
    const float pixels = (float)(h * w);
    const float rgb_weight = 1.0f / (3.0f * pixels);
    const float alpha_weight = cfg->alpha_weight / pixels;
    const uint32_t T = im.tiles();
    std::vector<float> lossv((size_t)h * w);
    std::vector<float> bl;
    for (uint32_t c = 0; c < 3; ++c) {
        blur(im, 5, [&](uint32_t y, uint32_t x, int k) {
            const float xv = im.p(y, x, c), yv = im.gt_eff(y, x, c);
            switch (k) {
            case 0: return xv;
            case 1: return xv * xv;
            case 2: return yv;
            case 3: return yv * yv;
            default: return xv * yv;
            }
        }, bl);
        for (uint32_t y = 0; y < h; ++y)
            for (uint32_t x = 0; x < w; ++x) {
                const float* o = &bl[((size_t)y * w + x) * 5];
                const float mu1 = o[0], mu2 = o[2];
                const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
                const float sigma1_sq = fmax_(0.0f, o[1] - mu1_sq);
                const float sigma2_sq = fmax_(0.0f, o[3] - mu2_sq);
                const float sigma12 = o[4] - mu1 * mu2;
                const float a = mu1_sq + mu2_sq + LOSS_C1;
                const float b = sigma1_sq + sigma2_sq + LOSS_C2;
                const float c_top = 2.0f * mu1 * mu2 + LOSS_C1;
                const float d_top = 2.0f * sigma12 + LOSS_C2;
                const float raw = (c_top * d_top) / (a * b);
                const float val = clampf(raw, -1.0f, 1.0f);
                if (coeffs) {
                    const float inv_b = 1.0f / b;
                    const float inv_ab = 1.0f / (a * b);
                    const float cd = c_top * d_top * inv_ab;
                    const bool clamped = cd < -1.0f || cd > 1.0f;
                    const size_t plane = (size_t)h * w, at = (size_t)c * 3 * plane + (size_t)y * w + x;
                    coeffs[at] = clamped ? 0.0f : 2.0f * inv_ab * (mu2 * (d_top - c_top) - mu1 * cd * (b - a));
                    coeffs[at + plane] = clamped ? 0.0f : -cd * inv_b;
                    coeffs[at + 2 * plane] = clamped ? 0.0f : 2.0f * c_top * inv_ab;
                }
                const float l1 = std::fabs(im.p(y, x, c) - im.gt_eff(y, x, c));
                float lv = cfg->l1_weight * l1 + cfg->ssim_weight * val;
                if (cfg->mask) lv = lv * im.gt_a(y, x);
                lossv[(size_t)y * w + x] = lv;
                if (loss_map) loss_map[((size_t)y * w + x) * cn + c] = lv;
            }
        if (partials)
            for (uint32_t t = 0; t < T; ++t) {
                float v[256];
                const uint32_t ty = t / im.tiles_x(), tx = t % im.tiles_x();
                for (uint32_t i = 0; i < 256; ++i) {
                    const uint32_t y = ty * 16 + i / 16, x = tx * 16 + i % 16;
                    v[i] = (y < h && x < w) ? lossv[(size_t)y * w + x] : 0.0f;
                }
                partials[(size_t)c * T + t] = tile_tree_sum(v) * rgb_weight;
            }
    }
    if (alpha_match) {
        // lib.rs:266-285: |pred.a - gt.a| (times gt.a when masking), no blur
        for (uint32_t y = 0; y < h; ++y)
            for (uint32_t x = 0; x < w; ++x) {
                const float ga = im.gt_a(y, x);
                float v = std::fabs(im.p(y, x, 3) - ga);
                if (cfg->mask) v = v * ga;
                lossv[(size_t)y * w + x] = v;
                if (loss_map) loss_map[((size_t)y * w + x) * cn + 3] = v;
            }
        if (partials)
            for (uint32_t t = 0; t < T; ++t) {
                float v[256];
                const uint32_t ty = t / im.tiles_x(), tx = t % im.tiles_x();
                for (uint32_t i = 0; i < 256; ++i) {
                    const uint32_t y = ty * 16 + i / 16, x = tx * 16 + i % 16;
                    v[i] = (y < h && x < w) ? lossv[(size_t)y * w + x] : 0.0f;
                }
                partials[(size_t)3 * T + t] = tile_tree_sum(v) * alpha_weight;
            }
    }
    return 0;
}

// image_loss_backward_coeffs_kernel (lib.rs:821-1020): dL/dpred [H,W,cn] from
// the forward's coefficients and dl_dpartials ([1] gradient of the total when
// scalar_grad, else one per partial [planes, tiles]).
extern "C" int or_image_loss_backward(const float* pred, uint32_t cn, const uint32_t* gt, uint32_t w, uint32_t h,
                                      const or_loss_cfg* cfg, const float* dl_dpartials, int scalar_grad,
                                      const float* coeffs, float* dl_dpred) {
    if (!pred || !gt || !cfg || !dl_dpartials || !coeffs || !dl_dpred || (cn != 3 && cn != 4)) return 1;
    const LossImg im{h, w, cn, pred, gt, cfg};
    const bool alpha_match = cfg->alpha_weight > 0.0f && cn == 4;
    const float pixels = (float)(h * w);
    const float rgb_weight = 1.0f / (3.0f * pixels);
    const float alpha_weight = cfg->alpha_weight / pixels;
    const uint32_t T = im.tiles();
    const size_t plane = (size_t)h * w;
    // chain_at (lib.rs:141-159)
    auto chain_at = [&](uint32_t c, uint32_t y, uint32_t x, float weight) {
        const float g = scalar_grad ? dl_dpartials[0] : dl_dpartials[(size_t)c * T + im.tile_of(y, x)];
        return g * weight;
    };
    std::vector<float> bl;
    for (uint32_t c = 0; c < 3; ++c) {
        blur(im, 3, [&](uint32_t y, uint32_t x, int k) {
            float chain = chain_at(c, y, x, rgb_weight);
            if (cfg->mask) chain = chain * im.gt_a(y, x);
            return coeffs[(size_t)c * 3 * plane + (size_t)k * plane + (size_t)y * w + x] * chain;
        }, bl);
        for (uint32_t y = 0; y < h; ++y)
            for (uint32_t x = 0; x < w; ++x) {
                const float* s = &bl[((size_t)y * w + x) * 3];
                const float p1 = im.p(y, x, c), ge = im.gt_eff(y, x, c);
                const float ssim_grad = s[0] + (2.0f * p1) * s[1] + ge * s[2];
                const float diff = p1 - ge;
                const float sign = diff > 0.0f ? 1.0f : (diff < 0.0f ? -1.0f : 0.0f);
                float cc = chain_at(c, y, x, rgb_weight);
                if (cfg->mask) cc = cc * im.gt_a(y, x);
                dl_dpred[((size_t)y * w + x) * cn + c] = cfg->ssim_weight * ssim_grad + cfg->l1_weight * sign * cc;
            }
    }
    if (cn == 4)
        for (uint32_t y = 0; y < h; ++y)
            for (uint32_t x = 0; x < w; ++x) {
                float g = 0.0f;
                if (alpha_match) {
                    const float ga = im.gt_a(y, x);
                    const float diff = im.p(y, x, 3) - ga;
                    const float sign = diff > 0.0f ? 1.0f : (diff < 0.0f ? -1.0f : 0.0f);
                    float chain = chain_at(3, y, x, alpha_weight);
                    if (cfg->mask) chain = chain * ga;
                    g = sign * chain;
                }
                dl_dpred[((size_t)y * w + x) * cn + 3] = g;
            }
    return 0;
}
