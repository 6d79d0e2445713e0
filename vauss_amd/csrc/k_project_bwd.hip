// k_project_bwd.hip -- projection VJP: raster gradient rows -> dense
// parameter gradients.
//
// Restates crates/splat-train-render/src/bwd/kernels/project_backwards.rs
// (splat_vjp :132-274, project_backwards_kernel :282-424) for the Default
// render mode without a scale floor.  One lane per global splat; rows whose
// ten raster gradients are all zero (culled or never blended) get zero
// gradients, which is the reference's dense result after gathering its compact
// rows through compact_from_global (bwd/burn_glue.rs:355-395).
#include "vs_device.h"
#include "vs_camera.h"
#include "vs_sh.h"
#include "vs_internal.h"

namespace vs {

constexpr int PBWD_BLOCK = 256;

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

template <int DEG, int MODEL>
__global__ void __launch_bounds__(PBWD_BLOCK) project_bwd_kernel(ProjectBwdArgs a) {
    constexpr int K = sh_count<DEG>();
    const uint32_t g = blockIdx.x * PBWD_BLOCK + threadIdx.x;
    if (g >= a.num_splats) return;
    const vs_camera& u = a.cam;
    const float2* r2 = reinterpret_cast<const float2*>(a.v_combined + (size_t)g * 10);
    const float2 r01 = r2[0], r23 = r2[1], r45 = r2[2], r67 = r2[3], r89 = r2[4];
    const float rg[10] = {r01.x, r01.y, r23.x, r23.y, r45.x, r45.y, r67.x, r67.y, r89.x, r89.y};
    bool any = false;
#pragma unroll
    for (int k = 0; k < 10; ++k) any = any || rg[k] != 0.0f;
    float* vsh = a.v_sh ? a.v_sh + (size_t)g * K * 3 : nullptr;
    if (!any) {
        if (a.v_transforms) {
            float2* o = reinterpret_cast<float2*>(a.v_transforms + (size_t)g * 10);
#pragma unroll
            for (int k = 0; k < 5; ++k) o[k] = make_float2(0.0f, 0.0f);
        }
        if (vsh) {
#pragma unroll
            for (int k = 0; k < K * 3; ++k) vsh[k] = 0.0f;
        }
        if (a.v_raw_opac) a.v_raw_opac[g] = 0.0f;
        if (a.v_refine) a.v_refine[g] = 0.0f;
        return;
    }
    const float2* t2 = reinterpret_cast<const float2*>(a.transforms + (size_t)g * 10);
    const float2 t01 = t2[0], t23 = t2[1], t45 = t2[2], t67 = t2[3], t89 = t2[4];
    const float lso = a.log_scale_offset;
    const F3 mean{t01.x, t01.y, t23.x};
    const F3 scl{expf_c(t67.y + lso), expf_c(t89.x + lso), expf_c(t89.y + lso)};
    const Qt qu{t23.y, t45.x, t45.y, t67.x};
    const float raw = a.raw_opac[g];
    const Qt q = normalize(qu);
    const float opac_sig = sigmoid(raw);

    // SH and view-direction VJP, project_backwards.rs:174-201
    const F3 u_world = mean - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]};
    const float u_len = length(u_world);
    const F3 vdir = u_world * (1.0f / u_len);
    const F3 v_color{rg[5], rg[6], rg[7]};
    if (vsh) {
        float Y[K];
        sh_basis<DEG>(vdir, Y);
#pragma unroll
        for (int k = 0; k < K; ++k) {
            vsh[3 * k] = v_color.x * Y[k];
            vsh[3 * k + 1] = v_color.y * Y[k];
            vsh[3 * k + 2] = v_color.z * Y[k];
        }
    }
    const F3 v_v_sh = sh_viewdir_vjp<DEG>(a.sh + (size_t)g * K * 3, vdir, v_color);
    const float v_dot = dot(vdir, v_v_sh);
    const F3 v_mean_sh = (v_v_sh - vdir * v_dot) * (1.0f / u_len);

    // Covariance / projection VJP, project_backwards.rs:203-274
    const F3 mc = world_to_cam(mean, u);
    const M3 R = to_mat3(q);
    const M3 Mm = mul_diag(R, scl);
    const S2 cov = cov2d_blurred<MODEL>(scl, q, mc, u);
    const float v_opac_base = 1.0f * rg[8];
    const S2 conic = inverse(cov);
    const S2 v_cov2d = inverse_vjp(conic, S2{rg[2], rg[3] * 0.5f, rg[4]});
    const S3 covar = outer_self(Mm);
    const M3 vrot = view_rot(u);
    const S3 cov_c = congruence(covar, vrot);
    const M23 J = project_jacobian<MODEL>(mc, u);
    F3 v_mean_c;
    if constexpr (MODEL == VS_CAMERA_KB4) v_mean_c = projection_vjp_kb4(J, mc, cov_c, u, v_cov2d, F2{rg[0], rg[1]});
    else v_mean_c = projection_vjp_pinhole(J, mc, cov_c, u, v_cov2d, F2{rg[0], rg[1]});
    const S3 vcc = tcongruence(J, v_cov2d);
    const F3 v_mean = tmul(vrot, v_mean_c) + v_mean_sh;
    const M3 v_m = mul(scale(tcongruence(vcc, vrot), 2.0f), Mm);
    const F3 v_log{dot(R.c0, v_m.c0) * scl.x, dot(R.c1, v_m.c1) * scl.y, dot(R.c2, v_m.c2) * scl.z};
    const Qt q_grad = quat_to_mat_vjp(q, mul_diag(v_m, scl));
    const Qt v_q = normalize_vjp(qu, q_grad);
    const float v_raw = v_opac_base * 1.0f * opac_sig * (1.0f - opac_sig);

    if (a.v_raw_opac) a.v_raw_opac[g] = v_raw;
    if (a.v_refine) a.v_refine[g] = clampf(finite(rg[9]) ? rg[9] : 0.0f, 0.0f, 1.0e32f);
    if (a.v_transforms) {
        float2* o = reinterpret_cast<float2*>(a.v_transforms + (size_t)g * 10);
        o[0] = make_float2(v_mean.x, v_mean.y);
        o[1] = make_float2(v_mean.z, v_q.w);
        o[2] = make_float2(v_q.x, v_q.y);
        o[3] = make_float2(v_q.z, v_log.x);
        o[4] = make_float2(v_log.y, v_log.z);
    }
}

template <int DEG>
static void launch_pbwd_model(const ProjectBwdArgs& a, dim3 grid, hipStream_t s) {
    if (a.cam.model == VS_CAMERA_KB4) project_bwd_kernel<DEG, VS_CAMERA_KB4><<<grid, PBWD_BLOCK, 0, s>>>(a);
    else project_bwd_kernel<DEG, VS_CAMERA_PINHOLE><<<grid, PBWD_BLOCK, 0, s>>>(a);
}

hipError_t launch_project_bwd(const ProjectBwdArgs& a, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    const dim3 grid((a.num_splats + PBWD_BLOCK - 1) / PBWD_BLOCK);
    switch (a.sh_degree) {
    case 0: launch_pbwd_model<0>(a, grid, s); break;
    case 1: launch_pbwd_model<1>(a, grid, s); break;
    case 2: launch_pbwd_model<2>(a, grid, s); break;
    case 3: launch_pbwd_model<3>(a, grid, s); break;
    default: launch_pbwd_model<4>(a, grid, s); break;
    }
    return hipGetLastError();
}

} // namespace vs
