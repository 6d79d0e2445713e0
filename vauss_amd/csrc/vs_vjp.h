// vs_vjp.h -- the projection VJP of one visible splat, shared by the dense
// projection backward (k_project_bwd.hip) and the fused update
// (k_project_update.hip).
//
// Restates crates/splat-train-render/src/bwd/kernels/project_backwards.rs
// (splat_vjp :132-274) for the Default and Mip render modes, with or without
// the scale floor.
#pragma once
#include "vs_device.h"
#include "vs_camera.h"
#include "vs_sh.h"

namespace vs {

// project_backwards.rs:18-51
VS_DEV Qt normalize_vjp(Qt q, Qt g) {
    const float lsq = dot(q, q);
    const float l = __builtin_sqrtf(lsq);
    const float inv = 1.0f / (l * lsq);
    const float cc0 = -q.w * q.x, cc1 = -q.x * q.y, cc2 = -q.y * q.w;
    const float cs0 = -q.w * q.z, cs1 = -q.x * q.z, cs2 = -q.y * q.z;
    const float sw = q.w * q.w, sx = q.x * q.x, sy = q.y * q.y, sz = q.z * q.z;
    return Qt{((lsq - sw) * g.w + cc0 * g.x + cc2 * g.y + cs0 * g.z) * inv,
              (cc0 * g.w + (lsq - sx) * g.x + cc1 * g.y + cs1 * g.z) * inv,
              (cc2 * g.w + cc1 * g.x + (lsq - sy) * g.y + cs2 * g.z) * inv,
              (cs0 * g.w + cs1 * g.x + cs2 * g.y + (lsq - sz) * g.z) * inv};
}
// project_backwards.rs:53-78
VS_DEV Qt quat_to_mat_vjp(Qt q, M3 v) {
    const float wg = q.x * (v.c1.z - v.c2.y) + q.y * (v.c2.x - v.c0.z) + q.z * (v.c0.y - v.c1.x);
    const float xg = -2.0f * q.x * (v.c1.y + v.c2.z) + q.y * (v.c0.y + v.c1.x) + q.z * (v.c0.z + v.c2.x) + q.w * (v.c1.z - v.c2.y);
    const float yg = q.x * (v.c0.y + v.c1.x) - 2.0f * q.y * (v.c0.x + v.c2.z) + q.z * (v.c1.z + v.c2.y) + q.w * (v.c2.x - v.c0.z);
    const float zg = q.x * (v.c0.z + v.c2.x) + q.y * (v.c1.z + v.c2.y) - 2.0f * q.z * (v.c0.x + v.c1.y) + q.w * (v.c0.y - v.c1.x);
    return Qt{2.0f * wg, 2.0f * xg, 2.0f * yg, 2.0f * zg};
}
// project_backwards.rs:80-98
VS_DEV S2 inverse_vjp(S2 m, S2 v) {
    const float t00 = -m.c00 * v.c00 + -m.c01 * v.c01;
    const float t01 = -m.c01 * v.c00 + -m.c11 * v.c01;
    const float t10 = -m.c00 * v.c01 + -m.c01 * v.c11;
    const float t11 = -m.c01 * v.c01 + -m.c11 * v.c11;
    return S2{t00 * m.c00 + t10 * m.c01, t01 * m.c00 + t11 * m.c01, t01 * m.c01 + t11 * m.c11};
}


struct SplatVjp {
    F3 v_mean;      // d/d mean
    Qt v_q;         // d/d unnormalised quaternion (w, x, y, z)
    F3 v_log;       // d/d log-scale
    float v_raw;    // d/d raw opacity
    F3 vdir;        // unit view direction (the SH basis argument)
};

// rg: the splat's raster gradients [xy(2), conic(3), rgb(3), opacity, refine].
// `scl_raw` is exp(log-scale + offset); `min_scale` (NULL: no floor) and
// `mip` select the render mode's forward, as in the projection.
template <int DEG, int MODEL, typename SHT>
VS_DEV SplatVjp splat_vjp(const vs_camera& u, const SHT* __restrict__ sh_row, F3 mean, F3 scl_raw, Qt qu, float raw,
                          const float rg[10], const float* __restrict__ min_scale, uint32_t g, bool mip) {
    const Qt q = normalize(qu);
    const float opac_sig = sigmoid(raw);
    const ScaleFloor fl = apply_scale_floor(scl_raw, opac_sig, min_scale, g);
    const F3 scl = fl.scale;

    // SH and view-direction VJP, project_backwards.rs:174-201
    const F3 u_world = mean - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]};
    const float u_len = length(u_world);
    const F3 vdir = u_world * (1.0f / u_len);
    const F3 v_color{rg[5], rg[6], rg[7]};
    F3 v_mean_sh{0.0f, 0.0f, 0.0f};   // neural appearance (DEG < 0) adds its own term after
    if constexpr (DEG >= 0) {
        const F3 v_v_sh = sh_viewdir_vjp<DEG>(sh_row, vdir, v_color);
        const float v_dot = dot(vdir, v_v_sh);
        v_mean_sh = (v_v_sh - vdir * v_dot) * (1.0f / u_len);
    }

    // Covariance / projection VJP, project_backwards.rs:203-274
    const F3 mc = world_to_cam(mean, u);
    const M3 R = to_mat3(q);
    const M3 Mm = mul_diag(R, scl);
    float filter_comp;
    const S2 cov = compensate_cov2d(cov2d_raw<MODEL>(scl, q, mc, u), mip, filter_comp);
    // the compensated opacity's gradient (no path through filter_comp), 0 where the floor clamps
    const float v_opac_base = fl.opac_open ? filter_comp * rg[8] : 0.0f;
    const S2 conic = inverse(cov);
    const S2 v_cov2d = inverse_vjp(conic, S2{rg[2], rg[3] * 0.5f, rg[4]});
    const S3 covar = outer_self(Mm);
    const M3 vrot = view_rot(u);
    const S3 cov_c = congruence(covar, vrot);
    const M23 J = project_jacobian<MODEL>(mc, u);
    F3 v_mean_c;
    v_mean_c = projection_vjp<MODEL>(J, mc, cov_c, u, v_cov2d, F2{rg[0], rg[1]});
    const S3 vcc = tcongruence(J, v_cov2d);
    SplatVjp r;
    r.v_mean = tmul(vrot, v_mean_c) + v_mean_sh;
    const M3 v_m = mul(scale(tcongruence(vcc, vrot), 2.0f), Mm);
    // project_backwards.rs:256-265: through the floor (ratio_sq) plus the
    // opacity compensation's d(opac) / d(log s_i) = opac (1 - ratio_sq_i)
    const F3 v_lf{dot(R.c0, v_m.c0) * scl.x, dot(R.c1, v_m.c1) * scl.y, dot(R.c2, v_m.c2) * scl.z};
    r.v_log = F3{v_lf.x * fl.ratio_sq.x + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.x),
                 v_lf.y * fl.ratio_sq.y + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.y),
                 v_lf.z * fl.ratio_sq.z + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.z)};
    const Qt q_grad = quat_to_mat_vjp(q, mul_diag(v_m, scl));
    r.v_q = normalize_vjp(qu, q_grad);
    r.v_raw = v_opac_base * fl.coef * opac_sig * (1.0f - opac_sig);
    r.vdir = vdir;
    return r;
}

// ---- camera gradient, bwd/kernels/pose_backwards.rs ------------------------------
// The camera is perturbed by x_c' = (I + A) x_c + b after the world-to-camera
// transform; A pivots on the camera centre, which b moves by -M^-1 b.
VS_DEV F3 cross(F3 a, F3 b) { return F3{a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x}; }
// pose_backwards.rs:61-74: M^-T g from the column cross products over det M.
VS_DEV F3 inverse_transpose_mul(M3 m, F3 g) {
    const F3 k0 = cross(m.c1, m.c2), k1 = cross(m.c2, m.c0), k2 = cross(m.c0, m.c1);
    return ((k0 * g.x + k1 * g.y) + k2 * g.z) * (1.0f / dot(m.c0, k0));
}

// pose_backwards_kernel (pose_backwards.rs:88-191) for one splat whose raster
// gradients of position, conic or colour are not all zero: the row
// [v x^T + 2 V S (row-major 3x3), db] with v, V the camera-space mean and
// covariance gradients and x, S the camera-space mean and covariance.
template <int DEG, int MODEL, typename SHT>
VS_DEV void pose_row(const vs_camera& u, const SHT* __restrict__ sh_row, F3 mean, F3 scl_raw, Qt qu, float raw,
                     const float rg[10], const float* __restrict__ min_scale, uint32_t g, bool mip, float row[12]) {
    const Qt q = normalize(qu);
    const F3 scl = apply_scale_floor(scl_raw, sigmoid(raw), min_scale, g).scale;
    // SH view direction: only the camera centre moves it.
    const F3 u_world = mean - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]};
    const float u_len = length(u_world);
    const F3 dir = u_world * (1.0f / u_len);
    const F3 v_dir = sh_viewdir_vjp<DEG>(sh_row, dir, F3{rg[5], rg[6], rg[7]});
    const F3 v_mean_sh = (v_dir - dir * dot(dir, v_dir)) * (1.0f / u_len);
    const F3 mc = world_to_cam(mean, u);
    float filter_comp;
    const S2 cov = compensate_cov2d(cov2d_raw<MODEL>(scl, q, mc, u), mip, filter_comp);
    const S2 v_cov2d = inverse_vjp(inverse(cov), S2{rg[2], rg[3] * 0.5f, rg[4]});
    const M3 vrot = view_rot(u);
    const S3 S = congruence(outer_self(mul_diag(to_mat3(q), scl)), vrot);
    const M23 J = project_jacobian<MODEL>(mc, u);
    const F3 v = projection_vjp<MODEL>(J, mc, S, u, v_cov2d, F2{rg[0], rg[1]});
    const S3 V = tcongruence(J, v_cov2d);
    const F3 vb = v + inverse_transpose_mul(vrot, v_mean_sh);
    const F3 vr[3] = {srow0(V), srow1(V), srow2(V)};
    const F3 sr[3] = {srow0(S), srow1(S), srow2(S)};
    const float vv[3] = {v.x, v.y, v.z}, xx[3] = {mc.x, mc.y, mc.z};
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) row[3 * i + j] = vv[i] * xx[j] + 2.0f * dot(vr[i], sr[j]);
    row[9] = vb.x; row[10] = vb.y; row[11] = vb.z;
}

} // namespace vs
