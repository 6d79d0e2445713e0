// k_pose.hip -- camera gradient from the raster gradient rows.
//
// Restates crates/splat-train-render/src/bwd/kernels/pose_backwards.rs
// (pose_backwards_kernel :88-191) and its reduction in
// bwd/render_bwd.rs:224-288.  One lane per global splat computes the row
// [dA (row-major 3x3), db] of a splat whose position, conic or colour
// gradients are not all zero (culled splats have none), zero otherwise; each
// 256-splat block sums its rows (wave butterflies, then the four waves in
// order) into one partial, and a single block sums the partials in f64 in a
// fixed order, so the result does not depend on scheduling.
#include "vs_vjp.h"
#include "vs_internal.h"

namespace vs {

constexpr int POSE_BLOCK = 256;
constexpr int POSE_DIM = 12;

template <int DEG, int MODEL, typename SHT>
__global__ void __launch_bounds__(POSE_BLOCK) pose_bwd_kernel(PoseBwdArgs a) {
    constexpr int K = sh_count<DEG>();
    __shared__ float s_part[POSE_BLOCK / 64][POSE_DIM];
    const uint32_t g = blockIdx.x * POSE_BLOCK + threadIdx.x;
    float row[POSE_DIM];
#pragma unroll
    for (int k = 0; k < POSE_DIM; ++k) row[k] = 0.0f;
    if (g < a.num_splats) {
        const float2* r2 = reinterpret_cast<const float2*>(a.v_combined + (size_t)g * 10);
        const float2 r01 = r2[0], r23 = r2[1], r45 = r2[2], r67 = r2[3];
        const float rg[10] = {r01.x, r01.y, r23.x, r23.y, r45.x, r45.y, r67.x, r67.y, 0.0f, 0.0f};
        bool any = false;
#pragma unroll
        for (int k = 0; k < 8; ++k) any = any || rg[k] != 0.0f;
        if (any) {
            const float2* t2 = reinterpret_cast<const float2*>(a.transforms + (size_t)g * 10);
            const float2 t01 = t2[0], t23 = t2[1], t45 = t2[2], t67 = t2[3], t89 = t2[4];
            const float lso = a.log_scale_offset;
            const F3 mean{t01.x, t01.y, t23.x};
            const F3 scl{expf_c(t67.y + lso), expf_c(t89.x + lso), expf_c(t89.y + lso)};
            const Qt qu{t23.y, t45.x, t45.y, t67.x};
            pose_row<DEG, MODEL>(a.cam, static_cast<const SHT*>(a.sh) + (size_t)g * K * 3, mean, scl, qu,
                                 a.raw_opac[g], rg, a.min_scale, g, a.mip != 0u, row);
        }
    }
    const uint32_t lane = threadIdx.x & 63u, wave = threadIdx.x >> 6;
#pragma unroll
    for (int k = 0; k < POSE_DIM; ++k) {
        float v = row[k];
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
        if (lane == 0) s_part[wave][k] = v;
    }
    __syncthreads();
    if (threadIdx.x < POSE_DIM) {
        float v = s_part[0][threadIdx.x];
#pragma unroll
        for (int w = 1; w < POSE_BLOCK / 64; ++w) v += s_part[w][threadIdx.x];
        a.partials[(size_t)blockIdx.x * POSE_DIM + threadIdx.x] = v;
    }
}

// One block of 192 lanes: 16 lanes per component stride the [nblocks, 12]
// partials in f64 (independent loads, so the pass is not one long chain),
// then each component adds its 16 sums in a fixed order.
constexpr int POSE_SUM_PARTS = 16;
__global__ void __launch_bounds__(POSE_DIM * POSE_SUM_PARTS) pose_sum_kernel(const float* __restrict__ partials,
                                                                            uint32_t nblocks, float* __restrict__ out) {
    __shared__ double s_part[POSE_SUM_PARTS][POSE_DIM];
    const uint32_t k = threadIdx.x % POSE_DIM, part = threadIdx.x / POSE_DIM;
    double v = 0.0;
#pragma unroll 8
    for (uint32_t b = part; b < nblocks; b += POSE_SUM_PARTS) v += (double)partials[(size_t)b * POSE_DIM + k];
    s_part[part][k] = v;
    __syncthreads();
    if (threadIdx.x < POSE_DIM) {
        double t = s_part[0][k];
        for (int p = 1; p < POSE_SUM_PARTS; ++p) t += s_part[p][k];
        out[k] = (float)t;
    }
}

template <int DEG, typename SHT>
static void launch_pose_type(const PoseBwdArgs& a, dim3 grid, hipStream_t s) {
    switch (a.cam.model) {
    case VS_CAMERA_KB4: pose_bwd_kernel<DEG, VS_CAMERA_KB4, SHT><<<grid, POSE_BLOCK, 0, s>>>(a); break;
    case VS_CAMERA_RT8: pose_bwd_kernel<DEG, VS_CAMERA_RT8, SHT><<<grid, POSE_BLOCK, 0, s>>>(a); break;
    case VS_CAMERA_TPF: pose_bwd_kernel<DEG, VS_CAMERA_TPF, SHT><<<grid, POSE_BLOCK, 0, s>>>(a); break;
    default: pose_bwd_kernel<DEG, VS_CAMERA_PINHOLE, SHT><<<grid, POSE_BLOCK, 0, s>>>(a); break;
    }
}
template <int DEG>
static void launch_pose_model(const PoseBwdArgs& a, dim3 grid, hipStream_t s) {
    if (a.sh_half) launch_pose_type<DEG, uint16_t>(a, grid, s);
    else launch_pose_type<DEG, float>(a, grid, s);
}

uint32_t pose_bwd_blocks(uint32_t num_splats) { return (num_splats + POSE_BLOCK - 1) / POSE_BLOCK; }

hipError_t launch_pose_bwd(const PoseBwdArgs& a, hipStream_t s) {
    const uint32_t nb = pose_bwd_blocks(a.num_splats);
    if (nb > 0) {
        const dim3 grid(nb);
        switch (a.sh_degree) {
        case 0: launch_pose_model<0>(a, grid, s); break;
        case 1: launch_pose_model<1>(a, grid, s); break;
        case 2: launch_pose_model<2>(a, grid, s); break;
        case 3: launch_pose_model<3>(a, grid, s); break;
        default: launch_pose_model<4>(a, grid, s); break;
        }
    }
    pose_sum_kernel<<<1, POSE_DIM * POSE_SUM_PARTS, 0, s>>>(a.partials, nb, a.v_pose);
    return hipGetLastError();
}

} // namespace vs
