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
// With STAGE the SH gradient row is left to the caller: `any` says whether
// the splat has gradients, and the row is v_color (out) times the SH basis
// of vdir (out).
template <int DEG, typename SHT, bool STAGE>
VS_DEV void surfel_bwd(const ProjectBwdArgs& a, uint32_t g, bool& any_out, F3& vcol_out, F3& vdir_out) {
    constexpr int K = sh_count<DEG>();
    const vs_camera& u = a.cam;
    const float* rs = a.v_combined + (size_t)g * SURFEL_GRADS;
    float rg[SURFEL_GRADS];
    bool any = false;
#pragma unroll
    for (int k = 0; k < SURFEL_GRADS; ++k) { rg[k] = rs[k]; any = any || rg[k] != 0.0f; }
    any_out = any;
    float* vsh = (a.v_sh && !STAGE) ? a.v_sh + (size_t)g * K * 3 : nullptr;
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
    vcol_out = v_color;
    vdir_out = vdir;
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

// SH gradient rows whose length is a multiple of 4 floats (degrees 1 and 3)
// leave through LDS: each lane writes its row there, and the wavefront then
// stores its 64 contiguous rows as float4s, consecutive lanes on consecutive
// 16 bytes (instead of 3K scattered 4-byte stores per lane).
template <int DEG>
constexpr bool stage_sh_rows() { return DEG >= 0 && (sh_count<DEG>() * 3) % 4 == 0; }

template <int DEG, int MODEL, typename SHT>
__global__ void __launch_bounds__(PBWD_BLOCK) project_bwd_kernel(ProjectBwdArgs a) {
    // Neural rows (DEG < 0) and their gradients belong to the neural backward.
    constexpr int K = DEG >= 0 ? sh_count<DEG>() : 0;
    constexpr bool STAGE = stage_sh_rows<DEG>();
    constexpr int Q = STAGE ? K * 3 / 4 : 1;      // float4s per SH row
    __shared__ float4 s_rows[STAGE ? PBWD_BLOCK / 64 : 1][STAGE ? 64 * Q : 1];
    const uint32_t g = blockIdx.x * PBWD_BLOCK + threadIdx.x;
    const bool valid = g < a.num_splats;
    bool any = false;
    F3 vdir{0.0f, 0.0f, 0.0f}, vcol{0.0f, 0.0f, 0.0f};
    if constexpr (MODEL == SURFEL_MODEL) {
        if (valid) surfel_bwd<DEG, SHT, STAGE>(a, g, any, vcol, vdir);
    } else {
        const vs_camera& u = a.cam;
        float rg[10] = {};
        if (valid) {
            const float2* r2 = reinterpret_cast<const float2*>(a.v_combined + (size_t)g * 10);
            const float2 r01 = r2[0], r23 = r2[1], r45 = r2[2], r67 = r2[3], r89 = r2[4];
            rg[0] = r01.x; rg[1] = r01.y; rg[2] = r23.x; rg[3] = r23.y; rg[4] = r45.x;
            rg[5] = r45.y; rg[6] = r67.x; rg[7] = r67.y; rg[8] = r89.x; rg[9] = r89.y;
#pragma unroll
            for (int k = 0; k < 10; ++k) any = any || rg[k] != 0.0f;
        }
        float* vsh = (DEG >= 0 && a.v_sh && valid) ? a.v_sh + (size_t)g * K * 3 : nullptr;
        vcol = F3{rg[5], rg[6], rg[7]};
        if (valid && !any) {
            if (a.v_transforms) {
                float2* o = reinterpret_cast<float2*>(a.v_transforms + (size_t)g * 10);
#pragma unroll
                for (int k = 0; k < 5; ++k) o[k] = make_float2(0.0f, 0.0f);
            }
            if constexpr (!STAGE) {
                if (vsh) {
#pragma unroll
                    for (int k = 0; k < K * 3; ++k) vsh[k] = 0.0f;
                }
            }
            if (a.v_raw_opac) a.v_raw_opac[g] = 0.0f;
            if (a.v_refine) a.v_refine[g] = 0.0f;
        } else if (valid) {
            const float2* t2 = reinterpret_cast<const float2*>(a.transforms + (size_t)g * 10);
            const float2 t01 = t2[0], t23 = t2[1], t45 = t2[2], t67 = t2[3], t89 = t2[4];
            const float lso = a.log_scale_offset;
            const F3 mean{t01.x, t01.y, t23.x};
            const F3 scl{expf_c(t67.y + lso), expf_c(t89.x + lso), expf_c(t89.y + lso)};
            const Qt qu{t23.y, t45.x, t45.y, t67.x};
            const SplatVjp r = splat_vjp<DEG, MODEL>(u, static_cast<const SHT*>(a.sh) + (size_t)g * K * 3, mean, scl, qu,
                                                      a.raw_opac[g], rg, a.min_scale, g, a.mip != 0u);
            vdir = r.vdir;
            if constexpr (DEG >= 0 && !STAGE) {
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
    if constexpr (STAGE) {
        if (a.v_sh) {   // uniform
            // sh.rs:281-359: v_coeff_k = Y_k(v) v_colour (zero rows for splats without gradients)
            const uint32_t lane = threadIdx.x & 63u, w = threadIdx.x >> 6;
            float row[K * 3];
            if (any) {
                float Y[K];
                sh_basis<DEG>(vdir, Y);
#pragma unroll
                for (int k = 0; k < K; ++k) { row[3 * k] = vcol.x * Y[k]; row[3 * k + 1] = vcol.y * Y[k]; row[3 * k + 2] = vcol.z * Y[k]; }
            } else {
#pragma unroll
                for (int k = 0; k < K * 3; ++k) row[k] = 0.0f;
            }
#pragma unroll
            for (int q = 0; q < Q; ++q)
                s_rows[w][lane * Q + q] = make_float4(row[4 * q], row[4 * q + 1], row[4 * q + 2], row[4 * q + 3]);
            __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
            __builtin_amdgcn_wave_barrier();
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
            const uint32_t g0 = blockIdx.x * PBWD_BLOCK + w * 64;
            const uint32_t rows = g0 < a.num_splats ? min(64u, a.num_splats - g0) : 0u;
            float* dst = a.v_sh + (size_t)g0 * K * 3;
            if (((uintptr_t)a.v_sh & 15u) == 0u) {
                for (uint32_t c = lane; c < rows * Q; c += 64) reinterpret_cast<float4*>(dst)[c] = s_rows[w][c];
            } else {   // a caller's array aligned to 4 bytes only: the same order in single floats
                const float* src = reinterpret_cast<const float*>(s_rows[w]);
                for (uint32_t c = lane; c < rows * Q * 4; c += 64) dst[c] = src[c];
            }
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
