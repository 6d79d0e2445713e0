// k_loss.hip -- the image loss after the render: L1 + SSIM over an [H,W,C]
// f32 prediction and RGBA8-packed ground truth, its per-tile partial sums,
// and its gradient.
//
// Restates crates/splat-train-loss/src/lib.rs: image_loss_forward_kernel
// (:238-478) and image_loss_backward_coeffs_kernel (:821-1020).  SSIM uses an
// 11-tap Gaussian window (sigma 1.5) applied separably with zero padding,
// C1 = 0.01^2, C2 = 0.03^2, clamped to [-1, 1]; the per-pixel loss is
// l1_w |p - g| + ssim_w SSIM (ssim_w negative for training), optionally
// times gt.a (mask), with g composited over a background when asked.  The
// forward also keeps, per pixel and channel, the partials of SSIM w.r.t. the
// blurred moments (<x>, <x^2>, <xy>), so the backward blurs chain x partial
// once instead of re-running the forward's blurs.
//
// One 256-lane workgroup per 16x16 tile handles all three colour channels, so
// each halo pixel's prediction and packed ground truth are loaded once.  Sums
// follow one fixed order everywhere (per tap distance d = 1..5 add
// (left + right) * w, then the centre; rows, then columns; tile sums by a
// halving tree), which the CPU restatement repeats bit for bit.
#include "vs_device.h"
#include "vs_internal.h"

namespace vs {

// gauss_taps() (lib.rs:48-62) in f32: exp(-x^2 / 4.5) rounded to f32, divided
// by their f32 sum.
__device__ constexpr float LGW[6] = {0x1.0d957p-10f, 0x1.f1fe04p-8f, 0x1.26eb18p-5f, 0x1.bff1p-4f, 0x1.b43c4p-3f,
                                     0x1.106562p-2f};
constexpr float LOSS_C1 = 0.01f * 0.01f;
constexpr float LOSS_C2 = 0.03f * 0.03f;
constexpr float LOSS_INV_255 = 1.0f / 255.0f;
constexpr int LT = 16;              // tile edge
constexpr int LH = 5;               // window half width
constexpr int LS = LT + 2 * LH;     // 26: tile plus halo
constexpr int LBLOCK = LT * LT;

__device__ __forceinline__ float gt_byte(uint32_t v, uint32_t c) { return (float)((v >> (c * 8u)) & 0xffu) * LOSS_INV_255; }

// Sum of s[0..256) by the halving tree (s is overwritten); all lanes call it.
__device__ __forceinline__ float tile_tree(float* s) {
#pragma unroll
    for (uint32_t stride = 128; stride >= 1; stride >>= 1) {
        if (threadIdx.x < stride) s[threadIdx.x] += s[threadIdx.x + stride];
        __syncthreads();
    }
    return s[0];
}

template <bool COMPOSITE, bool MASK>
__device__ __forceinline__ float gt_eff(uint32_t v, uint32_t c, const LossArgs& a) {
    const float g = gt_byte(v, c);
    if constexpr (COMPOSITE) return g + (1.0f - gt_byte(v, 3)) * a.bg[c];
    return g;
}

template <bool COMPOSITE, bool MASK, bool ALPHA>
__global__ void __launch_bounds__(LBLOCK) loss_fwd_kernel(LossArgs a) {
    __shared__ float s_pg[3][LS * LS][2];        // (pred, effective gt) per channel, tile + halo
    __shared__ float s_h[3][LS * LT][5];         // row blur of x, x^2, y, y^2, xy
    __shared__ float s_red[4][LBLOCK];
    const uint32_t tid = threadIdx.x;
    const uint32_t lx = tid % LT, ly = tid / LT;
    const int tx0 = (int)(blockIdx.x * LT), ty0 = (int)(blockIdx.y * LT);
    const uint32_t w = a.img_w, h = a.img_h, cn = a.channels;

    for (uint32_t i = tid; i < LS * LS; i += LBLOCK) {
        const int gy = ty0 + (int)(i / LS) - LH, gx = tx0 + (int)(i % LS) - LH;
        float p[3] = {0.0f, 0.0f, 0.0f}, g[3] = {0.0f, 0.0f, 0.0f};
        if (gy >= 0 && gx >= 0 && gy < (int)h && gx < (int)w) {
            const size_t pix = (size_t)gy * w + gx;
            const uint32_t v = a.gt[pix];
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                p[c] = a.pred[pix * cn + c];
                g[c] = gt_eff<COMPOSITE, MASK>(v, c, a);
            }
        }
#pragma unroll
        for (int c = 0; c < 3; ++c) { s_pg[c][i][0] = p[c]; s_pg[c][i][1] = g[c]; }
    }
    __syncthreads();

    // Row blur at the tile's 16 columns for all 26 rows.
    for (uint32_t i = tid; i < LS * LT; i += LBLOCK) {
        const uint32_t r = i / LT, col = i % LT + LH;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            float sx = 0.0f, sx2 = 0.0f, sy = 0.0f, sy2 = 0.0f, sxy = 0.0f;
#pragma unroll
            for (int d = 1; d <= 5; ++d) {
                const float wd = LGW[5 - d];
                const float* L = s_pg[c][r * LS + col - d];
                const float* R = s_pg[c][r * LS + col + d];
                const float xl = L[0], yl = L[1], xr = R[0], yr = R[1];
                sx += (xl + xr) * wd;
                sx2 += (xl * xl + xr * xr) * wd;
                sy += (yl + yr) * wd;
                sy2 += (yl * yl + yr * yr) * wd;
                sxy += (xl * yl + xr * yr) * wd;
            }
            const float* M = s_pg[c][r * LS + col];
            const float xc = M[0], yc = M[1], wc = LGW[5];
            sx += xc * wc;
            sx2 += xc * xc * wc;
            sy += yc * wc;
            sy2 += yc * yc * wc;
            sxy += xc * yc * wc;
            float* o = s_h[c][i];
            o[0] = sx; o[1] = sx2; o[2] = sy; o[3] = sy2; o[4] = sxy;
        }
    }
    __syncthreads();

    const uint32_t px = (uint32_t)tx0 + lx, py = (uint32_t)ty0 + ly;
    const bool in = px < w && py < h;
    const size_t pix = (size_t)py * w + px;
    const uint32_t gv = in ? a.gt[pix] : 0u;
    const size_t plane = (size_t)h * w;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        float out[5];
#pragma unroll
        for (int k = 0; k < 5; ++k) {
            float s = 0.0f;
#pragma unroll
            for (int d = 1; d <= 5; ++d)
                s += (s_h[c][(ly + LH - d) * LT + lx][k] + s_h[c][(ly + LH + d) * LT + lx][k]) * LGW[5 - d];
            s += s_h[c][(ly + LH) * LT + lx][k] * LGW[5];
            out[k] = s;
        }
        float lv = 0.0f;
        if (in) {
            const float mu1 = out[0], mu2 = out[2];
            const float mu1_sq = mu1 * mu1, mu2_sq = mu2 * mu2;
            const float sigma1_sq = mx(0.0f, out[1] - mu1_sq);
            const float sigma2_sq = mx(0.0f, out[3] - mu2_sq);
            const float sigma12 = out[4] - mu1 * mu2;
            const float A = mu1_sq + mu2_sq + LOSS_C1;
            const float B = sigma1_sq + sigma2_sq + LOSS_C2;
            const float c_top = 2.0f * mu1 * mu2 + LOSS_C1;
            const float d_top = 2.0f * sigma12 + LOSS_C2;
            const float val = clampf((c_top * d_top) / (A * B), -1.0f, 1.0f);
            if (a.coeffs) {
                const float inv_b = 1.0f / B;
                const float inv_ab = 1.0f / (A * B);
                const float cd = c_top * d_top * inv_ab;
                const bool clamped = cd < -1.0f || cd > 1.0f;
                const size_t at = (size_t)c * 3 * plane + pix;
                a.coeffs[at] = clamped ? 0.0f : 2.0f * inv_ab * (mu2 * (d_top - c_top) - mu1 * cd * (B - A));
                a.coeffs[at + plane] = clamped ? 0.0f : -cd * inv_b;
                a.coeffs[at + 2 * plane] = clamped ? 0.0f : 2.0f * c_top * inv_ab;
            }
            const float* M = s_pg[c][(ly + LH) * LS + lx + LH];
            lv = a.l1_weight * __builtin_fabsf(M[0] - M[1]) + a.ssim_weight * val;
            if constexpr (MASK) lv = lv * gt_byte(gv, 3);
            if (a.loss_map) a.loss_map[pix * cn + c] = lv;
        }
        s_red[c][tid] = lv;
    }
    if constexpr (ALPHA) {
        // lib.rs:266-285: |pred.a - gt.a| (times gt.a when masking), no blur
        float v = 0.0f;
        if (in) {
            const float ga = gt_byte(gv, 3);
            v = __builtin_fabsf(a.pred[pix * cn + 3] - ga);
            if constexpr (MASK) v = v * ga;
            if (a.loss_map) a.loss_map[pix * cn + 3] = v;
        }
        s_red[3][tid] = v;
    }
    __syncthreads();
    if (a.partials) {
        const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
        const uint32_t T = gridDim.x * gridDim.y;
        constexpr int PL = ALPHA ? 4 : 3;
        // halving trees of the planes side by side (same order as one tree each)
#pragma unroll
        for (uint32_t stride = 128; stride >= 1; stride >>= 1) {
            if (tid < stride) {
#pragma unroll
                for (int c = 0; c < PL; ++c) s_red[c][tid] += s_red[c][tid + stride];
            }
            __syncthreads();
        }
        if (tid < PL) a.partials[(size_t)tid * T + tile] = s_red[tid][0] * (tid < 3 ? a.rgb_weight : a.alpha_weight);
    }
}

template <bool COMPOSITE, bool MASK, bool ALPHA, bool SCALAR>
__global__ void __launch_bounds__(LBLOCK) loss_bwd_kernel(LossBwdArgs a) {
    __shared__ float s_c[LS * LS][9];      // chain x coefficient, 3 per channel, tile + halo
    __shared__ float s_h[LS * LT][9];      // their row blur
    const uint32_t tid = threadIdx.x;
    const uint32_t lx = tid % LT, ly = tid / LT;
    const int tx0 = (int)(blockIdx.x * LT), ty0 = (int)(blockIdx.y * LT);
    const uint32_t w = a.img_w, h = a.img_h, cn = a.channels;
    const uint32_t tiles_x = (w + LT - 1) / LT;
    const uint32_t T = tiles_x * ((h + LT - 1) / LT);
    const size_t plane = (size_t)h * w;

    // chain_at (lib.rs:141-159): the upstream gradient of a pixel's tile sum times its weight.
    auto chain_at = [&](uint32_t c, uint32_t y, uint32_t x, float weight) {
        const float g = SCALAR ? a.dl[0] : a.dl[(size_t)c * T + (y / LT) * tiles_x + x / LT];
        return g * weight;
    };

    for (uint32_t i = tid; i < LS * LS; i += LBLOCK) {
        const int gy = ty0 + (int)(i / LS) - LH, gx = tx0 + (int)(i % LS) - LH;
        float v[9];
#pragma unroll
        for (int k = 0; k < 9; ++k) v[k] = 0.0f;
        if (gy >= 0 && gx >= 0 && gy < (int)h && gx < (int)w) {
            const size_t pix = (size_t)gy * w + gx;
            float ga = 1.0f;
            if constexpr (MASK) ga = gt_byte(a.gt[pix], 3);
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                float chain = chain_at(c, (uint32_t)gy, (uint32_t)gx, a.rgb_weight);
                if constexpr (MASK) chain = chain * ga;
#pragma unroll
                for (int k = 0; k < 3; ++k) v[c * 3 + k] = a.coeffs[(size_t)(c * 3 + k) * plane + pix] * chain;
            }
        }
#pragma unroll
        for (int k = 0; k < 9; ++k) s_c[i][k] = v[k];
    }
    __syncthreads();

    for (uint32_t i = tid; i < LS * LT; i += LBLOCK) {
        const uint32_t r = i / LT, col = i % LT + LH;
#pragma unroll
        for (int k = 0; k < 9; ++k) {
            float s = 0.0f;
#pragma unroll
            for (int d = 1; d <= 5; ++d) s += (s_c[r * LS + col - d][k] + s_c[r * LS + col + d][k]) * LGW[5 - d];
            s += s_c[r * LS + col][k] * LGW[5];
            s_h[i][k] = s;
        }
    }
    __syncthreads();

    const uint32_t px = (uint32_t)tx0 + lx, py = (uint32_t)ty0 + ly;
    if (px >= w || py >= h) return;
    const size_t pix = (size_t)py * w + px;
    const uint32_t gv = a.gt[pix];
    float out[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        float s3[3];
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            float s = 0.0f;
#pragma unroll
            for (int d = 1; d <= 5; ++d)
                s += (s_h[(ly + LH - d) * LT + lx][c * 3 + k] + s_h[(ly + LH + d) * LT + lx][c * 3 + k]) * LGW[5 - d];
            s += s_h[(ly + LH) * LT + lx][c * 3 + k] * LGW[5];
            s3[k] = s;
        }
        const float p1 = a.pred[pix * cn + c];
        const float ge = gt_eff<COMPOSITE, MASK>(gv, c, a.fwd);
        const float ssim_grad = s3[0] + (2.0f * p1) * s3[1] + ge * s3[2];
        const float diff = p1 - ge;
        const float sign = diff > 0.0f ? 1.0f : (diff < 0.0f ? -1.0f : 0.0f);
        float cc = chain_at(c, py, px, a.rgb_weight);
        if constexpr (MASK) cc = cc * gt_byte(gv, 3);
        out[c] = a.fwd.ssim_weight * ssim_grad + a.fwd.l1_weight * sign * cc;
    }
    if (cn == 4) {
        if constexpr (ALPHA) {
            const float ga = gt_byte(gv, 3);
            const float diff = a.pred[pix * 4 + 3] - ga;
            const float sign = diff > 0.0f ? 1.0f : (diff < 0.0f ? -1.0f : 0.0f);
            float chain = chain_at(3, py, px, a.alpha_weight);
            if constexpr (MASK) chain = chain * ga;
            out[3] = sign * chain;
        }
        reinterpret_cast<float4*>(a.dl_dpred)[pix] = make_float4(out[0], out[1], out[2], out[3]);
    } else {
        a.dl_dpred[pix * 3] = out[0];
        a.dl_dpred[pix * 3 + 1] = out[1];
        a.dl_dpred[pix * 3 + 2] = out[2];
    }
}

// Sum of the partials in one fixed order (per-lane strided sums, then a tree).
// The total of the weighted tile partials: one 1024-lane block, four
// independent loads in flight per lane, then a wave64 butterfly and a
// 16-entry LDS sum.  The summation order is fixed but differs from the tile
// tree's; the total is a convenience (the partials are the exact outputs).
constexpr int TOTAL_BLOCK = 1024;
__global__ void __launch_bounds__(TOTAL_BLOCK) loss_total_kernel(const float* __restrict__ partials, uint32_t n,
                                                                 float* __restrict__ total) {
    __shared__ float s[TOTAL_BLOCK / 64];
    float a0 = 0.0f, a1 = 0.0f, a2 = 0.0f, a3 = 0.0f;
    uint32_t i = threadIdx.x;
    for (; i + 3u * TOTAL_BLOCK < n; i += 4u * TOTAL_BLOCK) {
        a0 += partials[i];
        a1 += partials[i + TOTAL_BLOCK];
        a2 += partials[i + 2u * TOTAL_BLOCK];
        a3 += partials[i + 3u * TOTAL_BLOCK];
    }
    for (; i < n; i += TOTAL_BLOCK) a0 += partials[i];
    float v = (a0 + a1) + (a2 + a3);
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63u) == 0u) s[threadIdx.x >> 6] = v;
    __syncthreads();
    if (threadIdx.x == 0) {
        float t = 0.0f;
#pragma unroll
        for (int w = 0; w < TOTAL_BLOCK / 64; ++w) t += s[w];
        *total = t;
    }
}

template <bool C, bool M, bool A>
static void launch_fwd3(const LossArgs& a, dim3 grid, hipStream_t s) {
    loss_fwd_kernel<C, M, A><<<grid, LBLOCK, 0, s>>>(a);
}
hipError_t launch_loss_forward(const LossArgs& a, hipStream_t s) {
    const dim3 grid((a.img_w + LT - 1) / LT, (a.img_h + LT - 1) / LT);
    const bool alpha = a.alpha_weight_cfg > 0.0f && a.channels == 4;
    const int sel = (a.composite ? 4 : 0) | (a.mask ? 2 : 0) | (alpha ? 1 : 0);
    switch (sel) {
    case 0: launch_fwd3<false, false, false>(a, grid, s); break;
    case 1: launch_fwd3<false, false, true>(a, grid, s); break;
    case 2: launch_fwd3<false, true, false>(a, grid, s); break;
    case 3: launch_fwd3<false, true, true>(a, grid, s); break;
    case 4: launch_fwd3<true, false, false>(a, grid, s); break;
    case 5: launch_fwd3<true, false, true>(a, grid, s); break;
    case 6: launch_fwd3<true, true, false>(a, grid, s); break;
    default: launch_fwd3<true, true, true>(a, grid, s); break;
    }
    hipError_t e = hipGetLastError();
    if (e != hipSuccess || !a.total || !a.partials) return e;
    const uint32_t planes = alpha ? 4u : 3u;
    loss_total_kernel<<<1, TOTAL_BLOCK, 0, s>>>(a.partials, planes * grid.x * grid.y, a.total);
    return hipGetLastError();
}

template <bool C, bool M, bool A>
static void launch_bwd3(const LossBwdArgs& a, dim3 grid, bool scalar, hipStream_t s) {
    if (scalar) loss_bwd_kernel<C, M, A, true><<<grid, LBLOCK, 0, s>>>(a);
    else loss_bwd_kernel<C, M, A, false><<<grid, LBLOCK, 0, s>>>(a);
}
hipError_t launch_loss_backward(const LossBwdArgs& a, bool scalar, hipStream_t s) {
    const dim3 grid((a.img_w + LT - 1) / LT, (a.img_h + LT - 1) / LT);
    const bool alpha = a.fwd.alpha_weight_cfg > 0.0f && a.channels == 4;
    const int sel = (a.fwd.composite ? 4 : 0) | (a.fwd.mask ? 2 : 0) | (alpha ? 1 : 0);
    switch (sel) {
    case 0: launch_bwd3<false, false, false>(a, grid, scalar, s); break;
    case 1: launch_bwd3<false, false, true>(a, grid, scalar, s); break;
    case 2: launch_bwd3<false, true, false>(a, grid, scalar, s); break;
    case 3: launch_bwd3<false, true, true>(a, grid, scalar, s); break;
    case 4: launch_bwd3<true, false, false>(a, grid, scalar, s); break;
    case 5: launch_bwd3<true, false, true>(a, grid, scalar, s); break;
    case 6: launch_bwd3<true, true, false>(a, grid, scalar, s); break;
    default: launch_bwd3<true, true, true>(a, grid, scalar, s); break;
    }
    return hipGetLastError();
}

} // namespace vs
