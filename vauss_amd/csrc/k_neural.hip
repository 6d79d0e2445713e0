// k_neural.hip -- backward of the compact neural appearance.
//
// Restates crates/splat-train-render/src/bwd/kernels/neural_backwards.rs
// (row_backward :141-283, neural_backwards_kernel :285-442) and the partial
// sum of bwd/render_bwd.rs:390-435.  Each block owns a chunk of splats: rows
// without a colour gradient get zero outputs, the others are compacted into
// an LDS list, so every lane of a step has a row.  A row recomputes the
// decoder's activations from the LDS copy of the weights and writes its row
// gradient [base (DC units), latents, 0], the row's mean square, and adds its
// view-direction term to the mean gradient the projection backward wrote.
// The decoder gradient is three small products over rows: each step's
// activations stay in LDS (x | d1 and h1 | d2 | h2, plus the output
// adjoints) and each lane adds the products of the weights it owns over the
// step's rows in registers; a block writes one [816] partial, and one pass
// sums the partials per weight in f64 in a fixed order.  No float atomics,
// and the result does not depend on scheduling.
#include "vs_neural.h"
#include "vs_internal.h"

namespace vs {

constexpr int NB_BLOCK = 128;                   // lanes per block, and rows per step
constexpr int NB_CHUNK = NB_BLOCK * 16;         // splats per block
constexpr int NB_STRIDE = 49;                   // 48 staged floats per row + 1 (odd: conflict-free row writes)
constexpr int NB_W1_PER = NEURAL_HIDDEN * NEURAL_INPUTS / NB_BLOCK;   // 4
constexpr int NB_W2_PER = NEURAL_HIDDEN * NEURAL_HIDDEN / NB_BLOCK;   // 2

// The decoder in LDS: row-major [out][in] and the two transposes [in][out],
// so every layer reads 4 consecutive weights per (uniform-address) load.
struct NeuralLds {
    float w[NEURAL_LEN];
    float w1t[NEURAL_INPUTS * NEURAL_HIDDEN];
    float w2t[NEURAL_HIDDEN * NEURAL_HIDDEN];
};

// One row's backward (neural_backwards.rs:141-283) with the row's
// activations kept in its LDS staging rows: A = x (32) | d1 (16),
// B = h1 (16) | d2 (16) | h2 (16), go = the output adjoints.  Every layer
// loops over its inputs and keeps one register accumulator per output, which
// adds each output's terms in input order, as the forward's dot products do.
template <typename SHT>
VS_DEV void neural_row_bwd(const NeuralBwdArgs& a, const NeuralLds& L, uint32_t g, F3 vc, float* A, float* B,
                           float* go) {
    const SHT* row = static_cast<const SHT*>(a.rows) + (size_t)g * NEURAL_ROW;
    const float* t = a.transforms + (size_t)g * 10;
    const vs_camera& u = a.cam;
    const F3 u_world = F3{t[0], t[1], t[2]} - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]};
    const float u_len = length(u_world);
    const F3 dir = u_world * (1.0f / u_len);
#pragma unroll
    for (int i = 0; i < NEURAL_LATENTS; ++i) sincosf_c(sh_ld(row, 3 + i), A[2 * i], A[2 * i + 1]);
    direction_basis(A, dir, a.degree);
    float acc[NEURAL_INPUTS];
    // h1 = ReLU(W1 x)
#pragma unroll
    for (int j = 0; j < NEURAL_HIDDEN; ++j) acc[j] = 0.0f;
#pragma unroll 1
    for (int k = 0; k < NEURAL_INPUTS; ++k) {
        const float xk = A[k];
        const float4* w4 = reinterpret_cast<const float4*>(L.w1t + k * NEURAL_HIDDEN);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 w = w4[q];
            acc[4 * q] += w.x * xk; acc[4 * q + 1] += w.y * xk; acc[4 * q + 2] += w.z * xk; acc[4 * q + 3] += w.w * xk;
        }
    }
#pragma unroll
    for (int j = 0; j < NEURAL_HIDDEN; ++j) B[j] = mx(acc[j], 0.0f);
    // h2 = ReLU(W2 h1)
#pragma unroll
    for (int j = 0; j < NEURAL_HIDDEN; ++j) acc[j] = 0.0f;
#pragma unroll 1
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
        const float hk = B[k];
        const float4* w4 = reinterpret_cast<const float4*>(L.w2t + k * NEURAL_HIDDEN);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 w = w4[q];
            acc[4 * q] += w.x * hk; acc[4 * q + 1] += w.y * hk; acc[4 * q + 2] += w.z * hk; acc[4 * q + 3] += w.w * hk;
        }
    }
    float h2[NEURAL_HIDDEN];
#pragma unroll
    for (int j = 0; j < NEURAL_HIDDEN; ++j) { h2[j] = mx(acc[j], 0.0f); B[32 + j] = h2[j]; }
    // o = W3 h2; colour = ReLU(C0 base + tanh(o) + 0.5)
    float o[3] = {0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
#pragma unroll
        for (int c = 0; c < 3; ++c) o[c] += L.w[NEURAL_W3 + c * NEURAL_HIDDEN + k] * h2[k];
    }
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
    // d2 = [h2 > 0] W3^T go
#pragma unroll
    for (int k = 0; k < NEURAL_HIDDEN; ++k) {
        float s2 = 0.0f;
#pragma unroll
        for (int c = 0; c < 3; ++c) s2 += L.w[NEURAL_W3 + c * NEURAL_HIDDEN + k] * go[c];
        B[16 + k] = (h2[k] > 0.0f) ? s2 : 0.0f;
    }
    // d1 = [h1 > 0] W2^T d2
#pragma unroll
    for (int k = 0; k < NEURAL_HIDDEN; ++k) acc[k] = 0.0f;
#pragma unroll 1
    for (int j = 0; j < NEURAL_HIDDEN; ++j) {
        const float dj = B[16 + j];
        const float4* w4 = reinterpret_cast<const float4*>(L.w + NEURAL_W2 + j * NEURAL_HIDDEN);
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const float4 w = w4[q];
            acc[4 * q] += w.x * dj; acc[4 * q + 1] += w.y * dj; acc[4 * q + 2] += w.z * dj; acc[4 * q + 3] += w.w * dj;
        }
    }
#pragma unroll
    for (int k = 0; k < NEURAL_HIDDEN; ++k) A[NEURAL_INPUTS + k] = (B[k] > 0.0f) ? acc[k] : 0.0f;
    // dx = W1^T d1
#pragma unroll
    for (int k = 0; k < NEURAL_INPUTS; ++k) acc[k] = 0.0f;
#pragma unroll 1
    for (int j = 0; j < NEURAL_HIDDEN; ++j) {
        const float dj = A[NEURAL_INPUTS + j];
        const float4* w4 = reinterpret_cast<const float4*>(L.w + NEURAL_W1 + j * NEURAL_INPUTS);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const float4 w = w4[q];
            acc[4 * q] += w.x * dj; acc[4 * q + 1] += w.y * dj; acc[4 * q + 2] += w.z * dj; acc[4 * q + 3] += w.w * dj;
        }
    }
#pragma unroll
    for (int i = 0; i < NEURAL_LATENTS; ++i) {           // latents through sin / cos
        const float gl = acc[2 * i] * A[2 * i + 1] - acc[2 * i + 1] * A[2 * i];
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
        const F3 g_dir = direction_basis_vjp(acc, dir, a.degree);
        const F3 vm = (g_dir - dir * dot(dir, g_dir)) * (1.0f / u_len);
        float* vt = a.v_transforms + (size_t)g * 10;
        vt[0] += vm.x;
        vt[1] += vm.y;
        vt[2] += vm.z;
    }
}

// One block per NB_CHUNK splats: rows without a colour gradient get zero
// outputs; the others are compacted (in id order) into an LDS list and run
// NB_BLOCK at a time, each step followed by the weight products of its rows.
template <typename SHT>
__global__ void __launch_bounds__(NB_BLOCK) neural_bwd_kernel(NeuralBwdArgs a) {
    __shared__ NeuralLds L;
    __shared__ float s_a[NB_BLOCK * NB_STRIDE];
    __shared__ float s_b[NB_BLOCK * NB_STRIDE];
    __shared__ float s_go[NB_BLOCK * 3];
    __shared__ uint32_t s_list[NB_CHUNK];
    __shared__ uint32_t s_wcnt[NB_BLOCK / 64];
    __shared__ uint32_t s_cnt;
    const uint32_t t = threadIdx.x;
    const uint32_t lane = t & 63u, wave = t >> 6;
    for (uint32_t i = t; i < (uint32_t)NEURAL_LEN; i += NB_BLOCK) {
        const float v = a.decoder[i];
        L.w[i] = v;
        if (i < (uint32_t)NEURAL_W2) L.w1t[(i % NEURAL_INPUTS) * NEURAL_HIDDEN + i / NEURAL_INPUTS] = v;
        else if (i < (uint32_t)NEURAL_W3) {
            const uint32_t r = i - NEURAL_W2;
            L.w2t[(r % NEURAL_HIDDEN) * NEURAL_HIDDEN + r / NEURAL_HIDDEN] = v;
        }
    }
    if (t == 0) s_cnt = 0;
    __syncthreads();

    // Compaction of the chunk's rows with a colour gradient.
    const uint32_t base = blockIdx.x * NB_CHUNK;
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    for (uint32_t sub = 0; sub < (uint32_t)(NB_CHUNK / NB_BLOCK); ++sub) {
        const uint32_t g = base + sub * NB_BLOCK + t;
        bool act = false;
        if (g < a.num_splats) {
            const float* rg = a.v_combined + (size_t)g * 10;
            act = rg[5] != 0.0f || rg[6] != 0.0f || rg[7] != 0.0f;
            if (!act) {
                if (a.v_rows) {
                    float4* o4 = reinterpret_cast<float4*>(a.v_rows + (size_t)g * NEURAL_ROW);
                    o4[0] = o4[1] = o4[2] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                }
                if (a.v_rows_sq) a.v_rows_sq[g] = 0.0f;
            }
        }
        const uint64_t m = __ballot(act);
        if (lane == 0) s_wcnt[wave] = (uint32_t)__popcll(m);
        __syncthreads();
        uint32_t off = s_cnt;
        for (uint32_t w = 0; w < wave; ++w) off += s_wcnt[w];
        if (act) s_list[off + (uint32_t)__popcll(m & lt_mask)] = g;
        __syncthreads();
        if (t == 0) {
            uint32_t total = s_cnt;
            for (uint32_t w = 0; w < (uint32_t)(NB_BLOCK / 64); ++w) total += s_wcnt[w];
            s_cnt = total;
        }
        __syncthreads();
    }
    const uint32_t n_act = s_cnt;

    float acc1[NB_W1_PER], acc2[NB_W2_PER], acc3 = 0.0f;
#pragma unroll
    for (int i = 0; i < NB_W1_PER; ++i) acc1[i] = 0.0f;
#pragma unroll
    for (int i = 0; i < NB_W2_PER; ++i) acc2[i] = 0.0f;
    float* A = s_a + t * NB_STRIDE;
    float* B = s_b + t * NB_STRIDE;
    float* GO = s_go + t * 3;
    const uint32_t k1 = t % NEURAL_INPUTS, j1 = t / NEURAL_INPUTS;
    const uint32_t k2 = t % NEURAL_HIDDEN, j2 = t / NEURAL_HIDDEN;
    const uint32_t c3 = (t < 48u) ? t / NEURAL_HIDDEN : 0u;
    for (uint32_t b0 = 0; b0 < n_act; b0 += NB_BLOCK) {
        if (b0 + t < n_act) {
            const uint32_t g = s_list[b0 + t];
            const float* rg = a.v_combined + (size_t)g * 10;
            neural_row_bwd<SHT>(a, L, g, F3{rg[5], rg[6], rg[7]}, A, B, GO);
        }
        __syncthreads();
        const uint32_t nrows = (n_act - b0 < (uint32_t)NB_BLOCK) ? n_act - b0 : (uint32_t)NB_BLOCK;
        // dW1[j][k] += d1[j] x[k]: this lane owns k = t % 32, j = t / 32 + 4 i.
        float a1[NB_W1_PER];
#pragma unroll
        for (int i = 0; i < NB_W1_PER; ++i) a1[i] = 0.0f;
        for (uint32_t r = 0; r < nrows; ++r) {
            const float* R = s_a + r * NB_STRIDE;
            const float xk = R[k1];
#pragma unroll
            for (int i = 0; i < NB_W1_PER; ++i) a1[i] += R[NEURAL_INPUTS + j1 + 4 * i] * xk;
        }
#pragma unroll
        for (int i = 0; i < NB_W1_PER; ++i) acc1[i] += a1[i];
        // dW2[j][k] += d2[j] h1[k]: k = t % 16, j = t / 16 + 8 i; dW3[c][k] += go[c] h2[k] for t < 48.
        float a2[NB_W2_PER];
#pragma unroll
        for (int i = 0; i < NB_W2_PER; ++i) a2[i] = 0.0f;
        float a3 = 0.0f;
        for (uint32_t r = 0; r < nrows; ++r) {
            const float* R = s_b + r * NB_STRIDE;
            const float hk = R[k2];
#pragma unroll
            for (int i = 0; i < NB_W2_PER; ++i) a2[i] += R[16 + j2 + 8 * i] * hk;
            a3 += s_go[r * 3 + c3] * R[32 + k2];
        }
#pragma unroll
        for (int i = 0; i < NB_W2_PER; ++i) acc2[i] += a2[i];
        acc3 += a3;
        __syncthreads();        // the next step overwrites the staged rows
    }
    float* p = a.partials + (size_t)blockIdx.x * NEURAL_LEN;
#pragma unroll
    for (int i = 0; i < NB_W1_PER; ++i) p[NEURAL_W1 + k1 + (j1 + 4 * i) * NEURAL_INPUTS] = acc1[i];
#pragma unroll
    for (int i = 0; i < NB_W2_PER; ++i) p[NEURAL_W2 + k2 + (j2 + 8 * i) * NEURAL_HIDDEN] = acc2[i];
    if (t < 48u) p[NEURAL_W3 + t] = acc3;
}

// The [blocks, 816] partials summed per weight in f64: 64 weights per block,
// four lanes per weight striding the partial rows, combined in a fixed order.
__global__ void __launch_bounds__(256) neural_sum_kernel(const float* __restrict__ partials, uint32_t nblocks,
                                                         float* __restrict__ out) {
    __shared__ double s_part[4][64];
    const uint32_t c = threadIdx.x & 63u, part = threadIdx.x >> 6;
    const uint32_t w = blockIdx.x * 64 + c;
    double acc = 0.0;
    if (w < (uint32_t)NEURAL_LEN) {
#pragma unroll 8
        for (uint32_t b = part; b < nblocks; b += 4) acc += (double)partials[(size_t)b * NEURAL_LEN + w];
    }
    s_part[part][c] = acc;
    __syncthreads();
    if (part == 0 && w < (uint32_t)NEURAL_LEN) out[w] = (float)(((s_part[0][c] + s_part[1][c]) + s_part[2][c]) + s_part[3][c]);
}

uint32_t neural_bwd_blocks(uint32_t num_splats) {
    const uint32_t b = (num_splats + NB_CHUNK - 1) / NB_CHUNK;
    return b < 1u ? 1u : b;
}

hipError_t launch_neural_bwd(const NeuralBwdArgs& a, hipStream_t s) {
    const uint32_t nb = neural_bwd_blocks(a.num_splats);
    if (a.half) neural_bwd_kernel<uint16_t><<<nb, NB_BLOCK, 0, s>>>(a);
    else neural_bwd_kernel<float><<<nb, NB_BLOCK, 0, s>>>(a);
    if (a.v_decoder) neural_sum_kernel<<<(NEURAL_LEN + 63) / 64, 256, 0, s>>>(a.partials, nb, a.v_decoder);
    return hipGetLastError();
}

}  // namespace vs
