// k_neural.hip -- backward of the compact neural appearance.
//
// Restates crates/splat-train-render/src/bwd/kernels/neural_backwards.rs
// (row_backward :141-283, neural_backwards_kernel :285-442) and the partial
// sum of bwd/render_bwd.rs:390-435.  A bounded grid strides over the global
// splat ids, one row per lane per step.  A splat with a colour gradient
// recomputes the decoder's activations (vs_neural.h) and writes its row
// gradient [base (DC units), latents, 0], the row's mean square, and adds its
// view-direction term to the mean gradient the projection backward wrote;
// every other row is written as zeros.  The decoder gradient is three small
// products over rows: each step stages every lane's activations in LDS
// (x | d1 and h1 | d2 | h2, plus the output adjoints) and each lane adds the
// products of the weights it owns over the step's rows in registers; a block
// writes one [816] partial, and one pass sums the partials per weight in f64,
// in block order.  No float atomics, and the result does not depend on
// scheduling.
#include "vs_neural.h"
#include "vs_internal.h"

namespace vs {

constexpr int NB_BLOCK = 128;
constexpr int NB_STRIDE = 49;                   // 48 staged floats per row + 1 (odd: conflict-free row writes)
constexpr int NB_W1_PER = NEURAL_HIDDEN * NEURAL_INPUTS / NB_BLOCK;   // 4
constexpr int NB_W2_PER = NEURAL_HIDDEN * NEURAL_HIDDEN / NB_BLOCK;   // 2
constexpr uint32_t NB_MAX_BLOCKS = 1024;

// One row's backward (neural_backwards.rs:141-283).  Stages x, d1 into A and
// h1, d2, h2 into B; returns the output adjoints in go.
template <typename SHT>
VS_DEV void neural_row_bwd(const NeuralBwdArgs& a, uint32_t g, F3 vc, float* A, float* B, float* go) {
    const float* __restrict__ W = a.decoder;
    const SHT* row = static_cast<const SHT*>(a.rows) + (size_t)g * NEURAL_ROW;
    const float* t = a.transforms + (size_t)g * 10;
    const vs_camera& u = a.cam;
    const F3 u_world = F3{t[0], t[1], t[2]} - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]};
    const float u_len = length(u_world);
    const F3 dir = u_world * (1.0f / u_len);
    float x[NEURAL_INPUTS], h1[NEURAL_HIDDEN], h2[NEURAL_HIDDEN], o[3];
    neural_forward(row, W, dir, a.degree, x, h1, h2, o);
    const float gc[3] = {vc.x, vc.y, vc.z};
    float vrow[NEURAL_ROW];
    float sq = 0.0f;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float th = tanhf_c(o[c]);
        const float base = sh_ld(row, c) * NEURAL_C0;
        const float gcol = (base + th + 0.5f > 0.0f) ? gc[c] : 0.0f;     // ReLU of the colour
        vrow[c] = gcol * NEURAL_C0;
        sq += (gcol * NEURAL_C0) * (gcol * NEURAL_C0);
        go[c] = gcol * (1.0f - th * th);
    }
    float d2[NEURAL_HIDDEN], d1[NEURAL_HIDDEN], dx[NEURAL_INPUTS];
#pragma unroll
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
        float acc = 0.0f;
#pragma unroll
        for (int c = 0; c < 3; ++c) acc += W[NEURAL_W3 + c * NEURAL_HIDDEN + k] * go[c];
        d2[k] = (h2[k] > 0.0f) ? acc : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NEURAL_HIDDEN; ++j) acc += W[NEURAL_W2 + j * NEURAL_HIDDEN + k] * d2[j];
        d1[k] = (h1[k] > 0.0f) ? acc : 0.0f;
    }
#pragma unroll
    for (int k = 0; k < NEURAL_INPUTS; ++k) {
        float acc = 0.0f;
#pragma unroll
        for (int j = 0; j < NEURAL_HIDDEN; ++j) acc += W[NEURAL_W1 + j * NEURAL_INPUTS + k] * d1[j];
        dx[k] = acc;
    }
#pragma unroll
    for (int i = 0; i < NEURAL_LATENTS; ++i) {           // latents through sin / cos
        const float gl = dx[2 * i] * x[2 * i + 1] - dx[2 * i + 1] * x[2 * i];
        vrow[3 + i] = gl;
        sq += gl * gl;
    }
    vrow[11] = 0.0f;
    if (a.v_rows) {
        float4* o4 = reinterpret_cast<float4*>(a.v_rows + (size_t)g * NEURAL_ROW);
        o4[0] = make_float4(vrow[0], vrow[1], vrow[2], vrow[3]);
        o4[1] = make_float4(vrow[4], vrow[5], vrow[6], vrow[7]);
        o4[2] = make_float4(vrow[8], vrow[9], vrow[10], vrow[11]);
    }
    if (a.v_rows_sq) a.v_rows_sq[g] = sq / (float)NEURAL_ROW;
    if (a.v_transforms) {
        const F3 g_dir = direction_basis_vjp(dx, dir, a.degree);
        const F3 vm = (g_dir - dir * dot(dir, g_dir)) * (1.0f / u_len);
        float* vt = a.v_transforms + (size_t)g * 10;
        vt[0] += vm.x;
        vt[1] += vm.y;
        vt[2] += vm.z;
    }
#pragma unroll
    for (int k = 0; k < NEURAL_INPUTS; ++k) A[k] = x[k];
#pragma unroll
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
        A[NEURAL_INPUTS + k] = d1[k];
        B[k] = h1[k];
        B[16 + k] = d2[k];
        B[32 + k] = h2[k];
    }
}

template <typename SHT>
__global__ void __launch_bounds__(NB_BLOCK) neural_bwd_kernel(NeuralBwdArgs a, uint32_t iters) {
    __shared__ float s_a[NB_BLOCK * NB_STRIDE];
    __shared__ float s_b[NB_BLOCK * NB_STRIDE];
    __shared__ float s_go[NB_BLOCK * 3];
    const uint32_t t = threadIdx.x;
    float acc1[NB_W1_PER], acc2[NB_W2_PER], acc3 = 0.0f;
#pragma unroll
    for (int i = 0; i < NB_W1_PER; ++i) acc1[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < NB_W2_PER; ++i) acc2[i] = 0.0f;
    float* A = s_a + t * NB_STRIDE;
    float* B = s_b + t * NB_STRIDE;
    float* GO = s_go + t * 3;
    const uint32_t stride = gridDim.x * NB_BLOCK;
    uint32_t g = blockIdx.x * NB_BLOCK + t;
    for (uint32_t it = 0; it < iters; ++it, g += stride) {
        bool active = false;
        if (g < a.num_splats) {
            const float* rg = a.v_combined + (size_t)g * 10;
            const F3 vc{rg[5], rg[6], rg[7]};
            active = vc.x != 0.0f || vc.y != 0.0f || vc.z != 0.0f;
            if (active) {
                neural_row_bwd<SHT>(a, g, vc, A, B, GO);
            } else {
                if (a.v_rows) {
                    float4* o4 = reinterpret_cast<float4*>(a.v_rows + (size_t)g * NEURAL_ROW);
                    o4[0] = o4[1] = o4[2] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
                if (a.v_rows_sq) a.v_rows_sq[g] = 0.0f;
            }
        }
        if (!active) {
            for (int k = 0; k < 48; ++k) { A[k] = 0.0f; B[k] = 0.0f; }
            GO[0] = GO[1] = GO[2] = 0.0f;
        }
        if (__syncthreads_or(active)) {
            // dW1[j][k] += d1[j] x[k]: this lane owns k = t % 32, j = t / 32 + 4 i.
            const uint32_t k1 = t % NEURAL_INPUTS, j1 = t / NEURAL_INPUTS;
            float a1[NB_W1_PER];
#pragma unroll
            for (int i = 0; i < NB_W1_PER; ++i) a1[i] = 0.0f;
            for (int r = 0; r < NB_BLOCK; ++r) {
                const float* R = s_a + r * NB_STRIDE;
                const float xk = R[k1];
#pragma unroll
                for (int i = 0; i < NB_W1_PER; ++i) a1[i] += R[NEURAL_INPUTS + j1 + 4 * i] * xk;
            }
#pragma unroll
            for (int i = 0; i < NB_W1_PER; ++i) acc1[i] += a1[i];
            // dW2[j][k] += d2[j] h1[k]: k = t % 16, j = t / 16 + 8 i; dW3[c][k] += go[c] h2[k] for t < 48.
            const uint32_t k2 = t % NEURAL_HIDDEN, j2 = t / NEURAL_HIDDEN;
            float a2[NB_W2_PER];
#pragma unroll
            for (int i = 0; i < NB_W2_PER; ++i) a2[i] = 0.0f;
            float a3 = 0.0f;
            const uint32_t c3 = (t < 48u) ? t / NEURAL_HIDDEN : 0u;
            for (int r = 0; r < NB_BLOCK; ++r) {
                const float* R = s_b + r * NB_STRIDE;
                const float hk = R[k2];
#pragma unroll
                for (int i = 0; i < NB_W2_PER; ++i) a2[i] += R[16 + j2 + 8 * i] * hk;
                a3 += s_go[r * 3 + c3] * R[32 + k2];
            }
#pragma unroll
            for (int i = 0; i < NB_W2_PER; ++i) acc2[i] += a2[i];
            acc3 += a3;
        }
        __syncthreads();        // the next step overwrites the staged rows
    }
    float* p = a.partials + (size_t)blockIdx.x * NEURAL_LEN;
#pragma unroll
    for (int i = 0; i < NB_W1_PER; ++i) p[NEURAL_W1 + (t % NEURAL_INPUTS) + (t / NEURAL_INPUTS + 4 * i) * NEURAL_INPUTS] = acc1[i];
#pragma unroll
    for (int i = 0; i < NB_W2_PER; ++i) p[NEURAL_W2 + (t % NEURAL_HIDDEN) + (t / NEURAL_HIDDEN + 8 * i) * NEURAL_HIDDEN] = acc2[i];
    if (t < 48u) p[NEURAL_W3 + t] = acc3;
}

// One lane per weight: the column of the [blocks, 816] partials, in f64.
__global__ void __launch_bounds__(256) neural_sum_kernel(const float* __restrict__ partials, uint32_t nblocks,
                                                         float* __restrict__ out) {
    const uint32_t w = blockIdx.x * 256 + threadIdx.x;
    if (w >= (uint32_t)NEURAL_LEN) return;
    double acc = 0.0;
    for (uint32_t b = 0; b < nblocks; ++b) acc += (double)partials[(size_t)b * NEURAL_LEN + w];
    out[w] = (float)acc;
}

uint32_t neural_bwd_blocks(uint32_t num_splats) {
    const uint32_t b = (num_splats + NB_BLOCK - 1) / NB_BLOCK;
    return b < 1u ? 1u : (b > NB_MAX_BLOCKS ? NB_MAX_BLOCKS : b);
}

hipError_t launch_neural_bwd(const NeuralBwdArgs& a, hipStream_t s) {
    const uint32_t nb = neural_bwd_blocks(a.num_splats);
    const uint32_t iters = (a.num_splats + nb * NB_BLOCK - 1) / (nb * NB_BLOCK);
    if (a.half) neural_bwd_kernel<uint16_t><<<nb, NB_BLOCK, 0, s>>>(a, iters);
    else neural_bwd_kernel<float><<<nb, NB_BLOCK, 0, s>>>(a, iters);
    if (a.v_decoder) neural_sum_kernel<<<(NEURAL_LEN + 255) / 256, 256, 0, s>>>(a.partials, nb, a.v_decoder);
    return hipGetLastError();
}

}  // namespace vs
