// k_project_update.hip -- projection VJP fused with the Adam step of the
// transforms and raw opacities, on packed moments; plus the moment codec's
// encode / decode / row-reset kernels.
//
// Restates crates/splat-train-render/src/bwd/kernels/project_update.rs:40-178
// (and bwd/project_update.rs:80-220 for the outputs) for the Default render
// mode without a scale floor.  One lane per splat.  A splat with raster
// gradients runs the projection VJP in registers and feeds it straight into
// Adam, so no dense gradient is written; every splat steps (culled ones decay
// their moments with a zero gradient and take the opacity regulariser).  The
// colour gradient and view direction go to `color_dir` for the SH step, which
// rebuilds the coefficient gradient Y_k(dir) colour itself.
#include "vs_vjp.h"
#include "vs_adam.h"
#include "vs_internal.h"

namespace vs {

constexpr int PUPD_BLOCK = 256;

template <int DEG, int MODEL, typename SHT>
__global__ void __launch_bounds__(PUPD_BLOCK) project_update_kernel(ProjectUpdateArgs a) {
    constexpr int K = sh_count<DEG>();
    const uint32_t g = blockIdx.x * PUPD_BLOCK + threadIdx.x;
    if (g >= a.num_splats) return;
    if (g == 0 && a.color_dir) {
#pragma unroll
        for (int k = 0; k < 6; ++k) a.color_dir[k] = 0.0f;
    }
    float2* t2 = reinterpret_cast<float2*>(a.transforms + (size_t)g * 10);
    const float2 t01 = t2[0], t23 = t2[1], t45 = t2[2], t67 = t2[3], t89 = t2[4];
    float t[10] = {t01.x, t01.y, t23.x, t23.y, t45.x, t45.y, t67.x, t67.y, t89.x, t89.y};
    float raw = a.raw_opac[g];

    float grad[10];
#pragma unroll
    for (int k = 0; k < 10; ++k) grad[k] = 0.0f;
    float g_opac = 0.0f, refine = 0.0f, grad_sq = 0.0f;
    const uint32_t row = a.compact[g];
    if (row > 0u) {
        const float2* r2 = reinterpret_cast<const float2*>(a.v_combined + (size_t)g * 10);
        const float2 r01 = r2[0], r23 = r2[1], r45 = r2[2], r67 = r2[3], r89 = r2[4];
        const float rg[10] = {r01.x, r01.y, r23.x, r23.y, r45.x, r45.y, r67.x, r67.y, r89.x, r89.y};
        bool any = false;
#pragma unroll
        for (int k = 0; k < 10; ++k) any = any || rg[k] != 0.0f;
        float* cd = a.color_dir ? a.color_dir + (size_t)row * 6 : nullptr;
        if (any) {
            const float lso = a.log_scale_offset;
            const F3 mean{t[0], t[1], t[2]};
            const F3 scl{expf_c(t[7] + lso), expf_c(t[8] + lso), expf_c(t[9] + lso)};
            const Qt qu{t[3], t[4], t[5], t[6]};
            const SplatVjp r = splat_vjp<DEG, MODEL>(a.cam, static_cast<const SHT*>(a.sh) + (size_t)g * K * 3, mean,
                                                     scl, qu, raw, rg, a.min_scale, g, a.mip != 0u);
            if (cd) {
                cd[0] = rg[5]; cd[1] = rg[6]; cd[2] = rg[7];
                cd[3] = r.vdir.x; cd[4] = r.vdir.y; cd[5] = r.vdir.z;
            }
            grad[0] = r.v_mean.x; grad[1] = r.v_mean.y; grad[2] = r.v_mean.z;
            grad[3] = r.v_q.w; grad[4] = r.v_q.x; grad[5] = r.v_q.y; grad[6] = r.v_q.z;
            grad[7] = r.v_log.x; grad[8] = r.v_log.y; grad[9] = r.v_log.z;
            g_opac = r.v_raw;
            refine = clampf(finite(rg[9]) ? rg[9] : 0.0f, 0.0f, 1.0e32f);
            // Mean square of the SH gradient row from its DC entries
            // (project_update.rs:133-140: sum_k Y_k^2 = (d+1)^2 / 4 pi).
            const float c0 = SH_C0 * rg[5], c1 = SH_C0 * rg[6], c2 = SH_C0 * rg[7];
            grad_sq = (c0 * c0 + c1 * c1 + c2 * c2) / 3.0f;
        } else if (cd) {
#pragma unroll
            for (int k = 0; k < 6; ++k) cd[k] = 0.0f;
        }
    } else if (a.color_dir) {
        // A culled splat's row (g + 1) is never gathered (its compact row is
        // 0); it is zeroed anyway so the output does not depend on old memory.
#pragma unroll
        for (int k = 0; k < 6; ++k) a.color_dir[(size_t)(g + 1) * 6 + k] = 0.0f;
    }
    if (a.v_refine) a.v_refine[g] = refine;
    if (a.grad_sq) a.grad_sq[g] = grad_sq;

    // Opacity regulariser w * mean(opacity) on every splat: d/d raw = (w / N) o (1 - o).
    const float o = 1.0f / (1.0f + expf_c(-raw));
    g_opac += a.opac_reg * o * (1.0f - o);
    // Separate rounding streams for transforms and opacity, which share indices.
    const uint32_t seed_t = a.round_seed ^ (10u << 24);
    const uint32_t seed_o = a.round_seed ^ (1u << 24);
    uint32_t* wt = a.w_t + (size_t)g * 10;
#pragma unroll
    for (int k = 0; k < 10; ++k) {
        uint32_t w = wt[k];
        adam_packed(t[k], w, g * 10u + (uint32_t)k, grad[k], a.lr_scale[k], a.beta1, a.beta2, a.inv1, a.inv2, a.epsilon,
                    seed_t);
        wt[k] = w;
    }
    t2[0] = make_float2(t[0], t[1]);
    t2[1] = make_float2(t[2], t[3]);
    t2[2] = make_float2(t[4], t[5]);
    t2[3] = make_float2(t[6], t[7]);
    t2[4] = make_float2(t[8], t[9]);
    uint32_t wo = a.w_o[g];
    adam_packed(raw, wo, g, g_opac, a.lr_opac, a.beta1, a.beta2, a.inv1, a.inv2, a.epsilon, seed_o);
    a.w_o[g] = wo;
    a.raw_opac[g] = raw;
}

// geo_moments.rs:104-127: round-to-nearest encode, decode.
__global__ void geo_encode_kernel(const float* __restrict__ m, const float* __restrict__ v, uint32_t n, float epsilon,
                                  uint32_t* __restrict__ words) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) words[i] = pack_geo(m[i], v[i], epsilon, 0.5f, 0.5f);
}
__global__ void geo_decode_kernel(const uint32_t* __restrict__ words, uint32_t n, float epsilon, float* __restrict__ m,
                                  float* __restrict__ v) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint32_t w = words[i];
    const float growth = geo_growth(w);
    const float root = epsilon * (growth - 1.0f);
    m[i] = geo_normalized(w) * (epsilon * growth);
    v[i] = root * root;
}
// geo_moments.rs:129-137: zero `row_width` words of each listed row.
__global__ void geo_zero_rows_kernel(uint32_t* __restrict__ words, const uint32_t* __restrict__ rows, uint32_t num_rows,
                                     uint32_t row_width, uint64_t num_words) {
    const uint64_t pos = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (pos >= (uint64_t)num_rows * row_width) return;
    const uint64_t idx = (uint64_t)rows[pos / row_width] * row_width + pos % row_width;
    if (idx < num_words) words[idx] = 0u;
}

template <int DEG, typename SHT>
static void launch_pupd_type(const ProjectUpdateArgs& a, dim3 grid, hipStream_t s) {
    switch (a.cam.model) {
    case VS_CAMERA_KB4: project_update_kernel<DEG, VS_CAMERA_KB4, SHT><<<grid, PUPD_BLOCK, 0, s>>>(a); break;
    case VS_CAMERA_RT8: project_update_kernel<DEG, VS_CAMERA_RT8, SHT><<<grid, PUPD_BLOCK, 0, s>>>(a); break;
    case VS_CAMERA_TPF: project_update_kernel<DEG, VS_CAMERA_TPF, SHT><<<grid, PUPD_BLOCK, 0, s>>>(a); break;
    default: project_update_kernel<DEG, VS_CAMERA_PINHOLE, SHT><<<grid, PUPD_BLOCK, 0, s>>>(a); break;
    }
}
template <int DEG>
static void launch_pupd_model(const ProjectUpdateArgs& a, dim3 grid, hipStream_t s) {
    if (a.sh_half) launch_pupd_type<DEG, uint16_t>(a, grid, s);
    else launch_pupd_type<DEG, float>(a, grid, s);
}

hipError_t launch_project_update(const ProjectUpdateArgs& a, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    const dim3 grid((a.num_splats + PUPD_BLOCK - 1) / PUPD_BLOCK);
    switch (a.sh_degree) {
    case 0: launch_pupd_model<0>(a, grid, s); break;
    case 1: launch_pupd_model<1>(a, grid, s); break;
    case 2: launch_pupd_model<2>(a, grid, s); break;
    case 3: launch_pupd_model<3>(a, grid, s); break;
    default: launch_pupd_model<4>(a, grid, s); break;
    }
    return hipGetLastError();
}

hipError_t launch_geo_encode(const float* m, const float* v, uint32_t n, float epsilon, uint32_t* words, hipStream_t s) {
    if (n == 0) return hipSuccess;
    geo_encode_kernel<<<(n + 255) / 256, 256, 0, s>>>(m, v, n, epsilon, words);
    return hipGetLastError();
}
hipError_t launch_geo_decode(const uint32_t* words, uint32_t n, float epsilon, float* m, float* v, hipStream_t s) {
    if (n == 0) return hipSuccess;
    geo_decode_kernel<<<(n + 255) / 256, 256, 0, s>>>(words, n, epsilon, m, v);
    return hipGetLastError();
}
hipError_t launch_geo_zero_rows(uint32_t* words, const uint32_t* rows, uint32_t num_rows, uint32_t row_width,
                                uint64_t num_words, hipStream_t s) {
    const uint64_t total = (uint64_t)num_rows * row_width;
    if (total == 0) return hipSuccess;
    geo_zero_rows_kernel<<<(uint32_t)((total + 255) / 256), 256, 0, s>>>(words, rows, num_rows, row_width, num_words);
    return hipGetLastError();
}

} // namespace vs
