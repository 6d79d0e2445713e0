// k_project_bwd.hip -- projection VJP: raster gradient rows -> dense
// parameter gradients.
//
// Restates crates/splat-train-render/src/bwd/kernels/project_backwards.rs
// (splat_vjp :132-274, project_backwards_kernel :282-424) for the Default
// render mode without a scale floor.  One lane per global splat; rows whose
// ten raster gradients are all zero (culled or never blended) get zero
// gradients, which is the reference's dense result after gathering its compact
// rows through compact_from_global (bwd/burn_glue.rs:355-395).
#include "vs_vjp.h"
#include "vs_neural.h"
#include "vs_surfel.h"
#include "vs_internal.h"

namespace vs {

constexpr int PBWD_BLOCK = 256;

// surfel_backwards (bwd/kernels/project_backwards.rs:426-570): the raster
// gradients of M = K [s_u W R e0, s_v W R e1, W p + t] (rows), the normal
// n = +-W R e2, colour, opacity and refine weight [17] to the parameters.
template <int DEG, typename SHT>
VS_DEV void surfel_bwd(const ProjectBwdArgs& a, uint32_t g) {
    constexpr int K = sh_count<DEG>();
    const vs_camera& u = a.cam;
    const float* rs = a.v_combined + (size_t)g * SURFEL_GRADS;
    float rg[SURFEL_GRADS];
    bool any = false;
#pragma unroll
    for (int k = 0; k < SURFEL_GRADS; ++k) { rg[k] = rs[k]; any = any || rg[k] != 0.0f; }
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
    const F3 scl_raw{expf_c(t67.y + lso), expf_c(t89.x + lso), expf_c(t89.y + lso)};
    const Qt qu{t23.y, t45.x, t45.y, t67.x};
    const Qt q = normalize(qu);
    const float opac_sig = sigmoid(a.raw_opac[g]);
    const ScaleFloor fl = apply_scale_floor(scl_raw, opac_sig, a.min_scale, g);
    const F3 sc = fl.scale;
    const F3 vc0{rg[0], rg[3], rg[6]}, vc1{rg[1], rg[4], rg[7]}, vc2{rg[2], rg[5], rg[8]};
    const F3 v_n{rg[9], rg[10], rg[11]}, v_color{rg[12], rg[13], rg[14]};
    const F3 u_world = mean - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]};
    const float u_len = length(u_world);
    const F3 vdir = u_world * (1.0f / u_len);
    const SHT* sh_row = static_cast<const SHT*>(a.sh) + (size_t)g * K * 3;
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
    const F3 v_v_sh = sh_viewdir_vjp<DEG>(sh_row, vdir, v_color);
    const F3 v_mean_sh = (v_v_sh - vdir * dot(vdir, v_v_sh)) * (1.0f / u_len);
    const float v_opac_base = fl.opac_open ? rg[15] : 0.0f;         // no 2-D blur compensation
    if (a.v_raw_opac) a.v_raw_opac[g] = v_opac_base * fl.coef * opac_sig * (1.0f - opac_sig);
    if (a.v_refine) a.v_refine[g] = clampf(finite(rg[16]) ? rg[16] : 0.0f, 0.0f, 1.0e32f);
    // M = K X  =>  v_X = K^T v_M, column by column
    const F3 v_a{u.fx * vc0.x, u.fy * vc0.y, u.cx * vc0.x + u.cy * vc0.y + vc0.z};
    const F3 v_b{u.fx * vc1.x, u.fy * vc1.y, u.cx * vc1.x + u.cy * vc1.y + vc1.z};
    const F3 v_c{u.fx * vc2.x, u.fy * vc2.y, u.cx * vc2.x + u.cy * vc2.y + vc2.z};
    const M3 W = view_rot(u);
    const M3 wr = mul(W, to_mat3(q));
    const F3 mc = world_to_cam(mean, u);
    const float v_su = dot(wr.c0, v_a), v_sv = dot(wr.c1, v_b);
    const float flip = dot(wr.c2, mc) > 0.0f ? -1.0f : 1.0f;
    const M3 v_r{tmul(W, v_a) * sc.x, tmul(W, v_b) * sc.y, tmul(W, v_n) * flip};
    const Qt v_q = normalize_vjp(qu, quat_to_mat_vjp(q, v_r));
    const F3 v_mean = tmul(W, v_c) + v_mean_sh;
    if (a.v_transforms) {
        float2* o = reinterpret_cast<float2*>(a.v_transforms + (size_t)g * 10);
        o[0] = make_float2(v_mean.x, v_mean.y);
        o[1] = make_float2(v_mean.z, v_q.w);
        o[2] = make_float2(v_q.x, v_q.y);
        o[3] = make_float2(v_q.z, v_su * sc.x * fl.ratio_sq.x + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.x));
        o[4] = make_float2(v_sv * sc.y * fl.ratio_sq.y + v_opac_base * fl.opac * (1.0f - fl.ratio_sq.y),
                           v_opac_base * fl.opac * (1.0f - fl.ratio_sq.z));
    }
}

template <int DEG, int MODEL, typename SHT>
__global__ void __launch_bounds__(PBWD_BLOCK) project_bwd_kernel(ProjectBwdArgs a) {
    // Neural rows (DEG < 0) and their gradients belong to the neural backward.
    constexpr int K = DEG >= 0 ? sh_count<DEG>() : 0;
    const uint32_t g = blockIdx.x * PBWD_BLOCK + threadIdx.x;
    if (g >= a.num_splats) return;
    if constexpr (MODEL == SURFEL_MODEL) {
        surfel_bwd<DEG, SHT>(a, g);
    } else {
        const vs_camera& u = a.cam;
        const float2* r2 = reinterpret_cast<const float2*>(a.v_combined + (size_t)g * 10);
        const float2 r01 = r2[0], r23 = r2[1], r45 = r2[2], r67 = r2[3], r89 = r2[4];
        const float rg[10] = {r01.x, r01.y, r23.x, r23.y, r45.x, r45.y, r67.x, r67.y, r89.x, r89.y};
        bool any = false;
#pragma unroll
        for (int k = 0; k < 10; ++k) any = any || rg[k] != 0.0f;
        float* vsh = (DEG >= 0 && a.v_sh) ? a.v_sh + (size_t)g * K * 3 : nullptr;
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
        const SplatVjp r = splat_vjp<DEG, MODEL>(u, static_cast<const SHT*>(a.sh) + (size_t)g * K * 3, mean, scl, qu, a.raw_opac[g], rg,
                                                  a.min_scale, g, a.mip != 0u);
        if constexpr (DEG >= 0) {
            if (vsh) {
                // sh.rs:281-359: v_coeff_k = Y_k(v) v_colour
                float Y[K];
                sh_basis<DEG>(r.vdir, Y);
#pragma unroll
                for (int k = 0; k < K; ++k) {
                    vsh[3 * k] = rg[5] * Y[k];
                    vsh[3 * k + 1] = rg[6] * Y[k];
                    vsh[3 * k + 2] = rg[7] * Y[k];
                }
            }
        }
        if (a.v_raw_opac) a.v_raw_opac[g] = r.v_raw;
        if (a.v_refine) a.v_refine[g] = clampf(finite(rg[9]) ? rg[9] : 0.0f, 0.0f, 1.0e32f);
        if (a.v_transforms) {
            float2* o = reinterpret_cast<float2*>(a.v_transforms + (size_t)g * 10);
            o[0] = make_float2(r.v_mean.x, r.v_mean.y);
            o[1] = make_float2(r.v_mean.z, r.v_q.w);
            o[2] = make_float2(r.v_q.x, r.v_q.y);
            o[3] = make_float2(r.v_q.z, r.v_log.x);
            o[4] = make_float2(r.v_log.y, r.v_log.z);
        }
    }
}

template <int DEG, typename SHT>
static void launch_pbwd_type(const ProjectBwdArgs& a, dim3 grid, hipStream_t s) {
    if constexpr (DEG >= 0) {           // surfels take SH colour only
        if (a.surfel) {
            project_bwd_kernel<DEG, SURFEL_MODEL, SHT><<<grid, PBWD_BLOCK, 0, s>>>(a);
            return;
        }
    }
    switch (a.cam.model) {
    case VS_CAMERA_KB4: project_bwd_kernel<DEG, VS_CAMERA_KB4, SHT><<<grid, PBWD_BLOCK, 0, s>>>(a); break;
    case VS_CAMERA_RT8: project_bwd_kernel<DEG, VS_CAMERA_RT8, SHT><<<grid, PBWD_BLOCK, 0, s>>>(a); break;
    case VS_CAMERA_TPF: project_bwd_kernel<DEG, VS_CAMERA_TPF, SHT><<<grid, PBWD_BLOCK, 0, s>>>(a); break;
    default: project_bwd_kernel<DEG, VS_CAMERA_PINHOLE, SHT><<<grid, PBWD_BLOCK, 0, s>>>(a); break;
    }
}
template <int DEG>
static void launch_pbwd_model(const ProjectBwdArgs& a, dim3 grid, hipStream_t s) {
    if (a.sh_half) launch_pbwd_type<DEG, uint16_t>(a, grid, s);
    else launch_pbwd_type<DEG, float>(a, grid, s);
}

hipError_t launch_project_bwd(const ProjectBwdArgs& a, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    const dim3 grid((a.num_splats + PBWD_BLOCK - 1) / PBWD_BLOCK);
    if (a.decoder) {
        launch_pbwd_model<NEURAL_DEG>(a, grid, s);
        return hipGetLastError();
    }
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
