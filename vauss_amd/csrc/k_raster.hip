// k_raster.hip -- tile ranges, forward alpha compositing and its VJP.
//
// Both kernels split a 16x16 tile into four 8x8 quadrants and stage the
// tile's depth-sorted splats into LDS in batches.  While staging, each lane
// tests its splat against the four quadrants (quadrant_mask), so no cycle is
// spent on a (splat, quadrant) pair whose every pixel stays below the alpha
// cutoff.
//
// Forward: crates/splat-train-render/src/kernels/rasterize.rs:109-420.  One
// 256-lane workgroup per tile, one pixel per lane in Morton order so each
// wavefront owns one quadrant (kernels/helpers.rs:105-128).  Batches of 256
// splats are staged as float4 pairs that lanes read as broadcasts; the
// workgroup compacts, per quadrant, the live batch slots, and each wavefront
// walks its own list.  The tile stops at the first batch boundary where every
// pixel has reached T <= 1e-4.  (Four wavefronts per tile hide the long exp
// dependency chain better than one wavefront with four pixels per lane.)
//
// Backward: bwd/kernels/rasterize_backwards_planes.rs:112-682.  One 64-lane
// wavefront per tile; lane L owns pixel (L % 8, L / 8) of each quadrant, so
// the quadrant masks become uniform branches and the per-splat work (one
// reduction, one atomic instruction) is shared by the whole tile.  Each lane
// replays its pixels front to back with the forward's exact arithmetic (so
// termination decisions agree bit for bit), sums its pixels' ten gradient
// components in registers, and the wavefront reduce-scatters them with
// permlane swaps and DPP (no LDS traffic), so each (tile, splat) pair issues
// one atomic instruction of at most ten lanes.
#include <hip/hip_ext.h>
#include "vs_device.h"
#include "vs_surfel.h"
#include "vs_internal.h"

namespace vs {

constexpr int BWD_BATCH = 64;

// get_tile_offset.rs:11-59: [start, end) of each tile in the sorted ids.
// Four sorted entries per thread (one 16-byte load): a tile's range starts
// where its id differs from the entry before and ends where it differs from
// the entry after.
__global__ void __launch_bounds__(256) tile_ranges_kernel(const uint32_t* __restrict__ tiles, uint32_t n_cap,
                                                          uint32_t num_tiles, uint32_t* __restrict__ ranges,
                                                          const uint32_t* __restrict__ n_dev) {
    const uint32_t n = n_dev ? min(*n_dev, n_cap) : n_cap;
    const uint64_t i0 = ((uint64_t)blockIdx.x * 256 + threadIdx.x) * 4;
    if (i0 >= n) return;
    uint32_t v[5];
    if (i0 + 4 <= n) {
        const uint4 q = reinterpret_cast<const uint4*>(tiles)[i0 / 4];
        v[0] = q.x; v[1] = q.y; v[2] = q.z; v[3] = q.w;
    } else {
#pragma unroll
        for (int k = 0; k < 4; ++k) v[k] = (i0 + k < n) ? tiles[i0 + k] : 0xFFFFFFFFu;
    }
    v[4] = (i0 + 4 < n) ? tiles[i0 + 4] : 0xFFFFFFFFu;
    uint32_t prev = i0 ? tiles[i0 - 1] : 0xFFFFFFFFu;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const uint64_t i = i0 + k;
        const uint32_t tile = v[k];
        if (i < n && tile < num_tiles) {   // sentinel rows sort last and own no tile
            if (prev != tile) ranges[tile * 2] = (uint32_t)i;
            if (v[k + 1] != tile) ranges[tile * 2 + 1] = (uint32_t)i + 1;
        }
        prev = tile;
    }
}

// DIST_NEAR / DIST_FAR depth map, kernels/helpers.rs:91-103.
VS_DEV float dist_depth(float z) { return 100.0f / (100.0f - 0.2f) * (1.0f - 0.2f / mx(z, 0.2f)); }

// Workgroups are dealt to the 8 XCDs round-robin; give XCD k the contiguous
// band of tiles [k*per, (k+1)*per) so neighbouring tiles, which share most of
// their splats, gather the same projected rows through the same L2.
VS_DEV uint32_t xcd_tile(uint32_t block, uint32_t num_tiles) {
    const uint32_t per = (num_tiles + 7) / 8;
    return (block % 8) * per + block / 8;
}
static uint32_t xcd_grid(uint32_t num_tiles) { return 8 * ((num_tiles + 7) / 8); }

// Tile of workgroup `block`: order[block] when a dispatch order is given
// (tile_order_kernel; entries past the tiles hold 0xFFFFFFFF), else the
// banded mapping above.
VS_DEV uint32_t block_tile(const uint32_t* order, uint32_t block, uint32_t num_tiles) {
    return order ? order[block] : xcd_tile(block, num_tiles);
}

// Dispatch order of the raster kernels.  Each XCD starts its workgroups in
// increasing index order as slots free up, so a long tile dealt out late
// ends the launch alone (the backward runs one wavefront per tile and holds
// about 1.6 tiles per slot at C3).  XCD k keeps its contiguous band of tiles
// [k per, (k + 1) per) (neighbouring tiles share splats, whose rows then stay
// in one L2) but takes them longest list first: block i * 8 + k gets the
// i-th longest tile of band k.  One workgroup per band counts its tiles into
// ORDER_BINS bins of 8 sqrt(list length) (LDS atomics: the order inside a
// bin is arbitrary, which changes no result) and scatters them by bin,
// longest bin first.
constexpr int ORDER_BLOCK = 1024;
constexpr int ORDER_BINS = 2048;
static_assert(ORDER_BINS == 2 * ORDER_BLOCK, "each thread of the order scan owns two bins");

VS_DEV uint32_t order_bin(uint32_t lo, uint32_t hi) {
    const float len = (float)(hi > lo ? hi - lo : 0u);
    const uint32_t key = min((uint32_t)(__builtin_sqrtf(len) * 8.0f), (uint32_t)ORDER_BINS - 1u);
    return (uint32_t)ORDER_BINS - 1u - key;   // ascending bin = descending length
}

__global__ void __launch_bounds__(ORDER_BLOCK) tile_order_kernel(uint32_t* ranges, uint32_t num_tiles,
                                                                 uint32_t* __restrict__ order,
                                                                 uint32_t* __restrict__ shrunk_init, int fix_empty,
                                                                 const uint32_t* __restrict__ flags_from,
                                                                 uint32_t* flags_to, uint32_t nflags,
                                                                 uint32_t* __restrict__ aux_out,
                                                                 float* __restrict__ zero, uint64_t zero_floats) {
    // Blocks past the eight bands clear `zero` (8-byte aligned; the backward's
    // gradient rows), which would otherwise take a launch of its own.
    if (blockIdx.x >= 8u) {
        const uint64_t stride = (uint64_t)(gridDim.x - 8u) * ORDER_BLOCK, pairs = zero_floats / 2;
        const uint64_t first = (uint64_t)(blockIdx.x - 8u) * ORDER_BLOCK + threadIdx.x;
        float2* z2 = reinterpret_cast<float2*>(zero);
        for (uint64_t i = first; i < pairs; i += stride) z2[i] = make_float2(0.0f, 0.0f);
        if (first == 0 && (zero_floats & 1u)) zero[zero_floats - 1] = 0.0f;
        return;
    }
    if (blockIdx.x == 0 && threadIdx.x < nflags) flags_to[threadIdx.x] = flags_from[threadIdx.x];
    __shared__ uint32_t s_bin[ORDER_BINS];
    __shared__ uint32_t s_wave[ORDER_BLOCK / 64];
    const uint32_t per = (num_tiles + 7) / 8;
    const uint32_t band = blockIdx.x;
    const uint32_t t0 = band * per, t1 = min(num_tiles, t0 + per);
    const uint32_t tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    for (uint32_t i = tid; i < ORDER_BINS; i += ORDER_BLOCK) s_bin[i] = 0u;
    __syncthreads();
    for (uint32_t t = t0 + tid; t < t1; t += ORDER_BLOCK) {
        uint32_t lo = ranges[2 * t];
        const uint32_t hi = ranges[2 * t + 1];
        if (fix_empty && lo == 0xFFFFFFFFu) {   // a tile the sort's range pass never saw: empty, (0, 0)
            lo = 0u;
            ranges[2 * t] = 0u;
        }
        atomicAdd(&s_bin[order_bin(lo, hi)], 1u);
        if (shrunk_init) {   // the forward's shrunk ranges start empty at the range start
            shrunk_init[2 * t] = lo;
            shrunk_init[2 * t + 1] = lo;
        }
        if (aux_out) {
            aux_out[2 * t] = lo;
            aux_out[2 * t + 1] = shrunk_init ? lo : hi;
        }
    }
    __syncthreads();
    // exclusive scan of the bins: each thread owns bins 2 tid and 2 tid + 1
    const uint32_t c0 = s_bin[2 * tid], c1 = s_bin[2 * tid + 1];
    uint32_t incl = c0 + c1;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t v = __shfl_up(incl, o);
        if ((int)lane >= o) incl += v;
    }
    if (lane == 63) s_wave[wave] = incl;
    __syncthreads();
    uint32_t before = 0;
    for (uint32_t w = 0; w < wave; ++w) before += s_wave[w];
    const uint32_t excl = before + incl - (c0 + c1);
    __syncthreads();                      // every count is read before the offsets replace them
    s_bin[2 * tid] = excl;
    s_bin[2 * tid + 1] = excl + c0;
    __syncthreads();
    for (uint32_t t = t0 + tid; t < t1; t += ORDER_BLOCK) {
        const uint32_t pos = atomicAdd(&s_bin[order_bin(ranges[2 * t], ranges[2 * t + 1])], 1u);
        order[(size_t)pos * 8 + band] = t;
    }
    for (uint32_t i = (t1 > t0 ? t1 - t0 : 0u) + tid; i < per; i += ORDER_BLOCK) order[(size_t)i * 8 + band] = 0xFFFFFFFFu;
}

// ---- quadrant culling -------------------------------------------------------
// A tile is four 8x8 quadrants.  For each staged splat the kernels compute a
// 4-bit mask of the quadrants in which some pixel centre may pass the alpha
// cutoff, and a wavefront skips (splat, quadrant) pairs outside the mask.
// The test is conservative, so skipping changes no result bit: a pixel that
// is skipped would have failed `alpha >= 1/255` (or, with the smooth cutoff,
// `alpha > 1/255 - 5e-4`: kernels/helpers.rs:23-47) and left every
// accumulator untouched.
//
// alpha = min(0.999, opac e^-sigma) is below the cutoff c whenever
// sigma > ln(opac / c).  The kernels hold the conic in base-2 units
// (s2 = sigma log2 e = A dx^2 + B dx dy + C dy^2 with the staged A, B, C), so a
// quadrant is dead when the minimum of s2 over the rectangle spanned by its
// pixel centres exceeds (1.01 ln(opac / c) + 0.01) log2 e.  The 1% + 0.01 margin dwarfs the
// f32 rounding of both this minimum and the per-pixel sigma, which is at most
// a few ulp of (A dx^2 + |B dx dy| + C dy^2) <= 2 sigma / (1 - rho) with
// rho = |B| / (2 sqrt(AC)); splats with 1 - rho^2 <= 0.01 (and any
// non-positive-definite or non-finite conic) keep all four quadrants.
constexpr float QUAD_MARGIN_REL = 1.01f;
constexpr float QUAD_MARGIN_ABS = 0.01f;
constexpr float QUAD_MIN_DECORR = 0.01f;

// Minimum over t in [lo, hi] of sigma on the edge where the other offset is
// fixed at u:  a u^2 + b u t + c t^2, minimised at t = k u (k = -b / 2c).
VS_DEV float edge_min(float a, float b, float c, float k, float u, float lo, float hi) {
    const float t = __builtin_fminf(__builtin_fmaxf(k * u, lo), hi);
    return (a * u + b * t) * u + c * t * t;
}

// The dead-quadrant bound (1.01 ln(opac / c) + 0.01) log2 e from the row's
// power = ln(255 opac): ln(opac / c) = power for c = 1/255 (up to a few ulp,
// far inside the 0.01 margin) and power + ln(1 / (255 c)) = power + 0.13640
// for the smooth cutoff's c = 1/255 - 5e-4 (0.1365 rounds that up).
constexpr float QUAD_SMOOTH_SHIFT = 0.1365f;
VS_DEV float quad_threshold(float power, bool smooth) {
    return (QUAD_MARGIN_REL * (smooth ? power + QUAD_SMOOTH_SHIFT : power) + QUAD_MARGIN_ABS) * LOG2E_F;
}

// Bit q (q = qy * 2 + qx) set when quadrant q of the tile whose first pixel
// centre is (x0, y0) may hold a pixel that passes the cutoff (power: the
// row's ln(255 opacity)).
VS_DEV uint32_t quadrant_mask(float x0, float y0, float mx_, float my_, float A, float B, float C, float power,
                              bool smooth) {
    const float thr = quad_threshold(power, smooth);
    const float four_ac = 4.0f * A * C;
    if (!(A > 0.0f && C > 0.0f && four_ac - B * B > QUAD_MIN_DECORR * four_ac && thr < 3.0e38f)) return 0xFu;
    const float kx = -B / (2.0f * C);   // vertical edges: dy* = kx dx
    const float ky = -B / (2.0f * A);   // horizontal edges: dx* = ky dy
    uint32_t mask = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float a0 = (x0 + (float)(8 * (q & 1))) - mx_, a1 = a0 + 7.0f;
        const float b0 = (y0 + (float)(8 * (q >> 1))) - my_, b1 = b0 + 7.0f;
        const bool inside = a0 <= 0.0f && a1 >= 0.0f && b0 <= 0.0f && b1 >= 0.0f;
        float m = __builtin_fminf(edge_min(A, B, C, kx, a0, b0, b1), edge_min(A, B, C, kx, a1, b0, b1));
        m = __builtin_fminf(m, __builtin_fminf(edge_min(C, B, A, ky, b0, a0, a1), edge_min(C, B, A, ky, b1, a0, a1)));
        if (inside || !(m > thr)) mask |= 1u << q;
    }
    return mask;
}

// The same test for one quadrant whose first pixel centre is (x0, y0): true
// when some pixel of its 8 x 8 block may pass the cutoff.
VS_DEV bool quadrant_live(float x0, float y0, float mx_, float my_, float A, float B, float C, float power, bool smooth) {
    const float thr = quad_threshold(power, smooth);
    const float four_ac = 4.0f * A * C;
    if (!(A > 0.0f && C > 0.0f && four_ac - B * B > QUAD_MIN_DECORR * four_ac && thr < 3.0e38f)) return true;
    const float kx = -B / (2.0f * C);
    const float ky = -B / (2.0f * A);
    const float a0 = x0 - mx_, a1 = a0 + 7.0f;
    const float b0 = y0 - my_, b1 = b0 + 7.0f;
    const bool inside = a0 <= 0.0f && a1 >= 0.0f && b0 <= 0.0f && b1 >= 0.0f;
    float m = __builtin_fminf(edge_min(A, B, C, kx, a0, b0, b1), edge_min(A, B, C, kx, a1, b0, b1));
    m = __builtin_fminf(m, __builtin_fminf(edge_min(C, B, A, ky, b0, a0, a1), edge_min(C, B, A, ky, b1, a0, a1)));
    return inside || !(m > thr);
}

// Morton order of the 64 lanes over an 8 x 8 quadrant (kernels/helpers.rs:
// 105-113 lay a tile out the same way): lane l holds pixel
// (even bits of l, odd bits of l).
VS_DEV uint32_t compact_bits_16(uint32_t v) {
    uint32_t x = v & 0x55555555u;
    x = (x | (x >> 1)) & 0x33333333u;
    x = (x | (x >> 2)) & 0x0F0F0F0Fu;
    x = (x | (x >> 4)) & 0x00FF00FFu;
    x = (x | (x >> 8)) & 0x0000FFFFu;
    return x;
}

// Surfel quadrant culling.  A surfel's pixel sigma is
// 0.5 min(u^2 + v^2, 2 |pixel - centre|^2) (surfel_hit), and alpha is below
// the cutoff c whenever sigma > ln(opac / c); with s = 1.01 ln(opac / c) +
// 0.01 a quadrant is dead when, over its pixel centres, both
//   * the low-pass disk misses: |pixel - centre|^2 > s, and
//   * the ray-plane disk misses: q.x^2 + q.y^2 > 2 s q.z^2,
// where q = h_u x h_v and (u, v) = (q.x, q.y) / q.z (a pixel with q.z = 0
// gets a non-finite depth and is no hit; the 1 % of s covers the rounding of
// the quotients).  The exact q is affine in the pixel:
// q(x, y) = R0 x R1 + x (R1 x R2) - y (R0 x R2) (R0, R1, R2 the rows of M), so
// over the quadrant it is P + t1 A + t2 B, t in [0, 1]^2, with P the q at its
// first pixel centre, A = 7 (R1 x R2) and B = -7 (R0 x R2).  Per component,
// the f32 q of surfel_hit at any of its pixels is within
// E = 6.5 ulp (H_y V_z + H_z V_y) (and so on) of the exact q (h_u within
// 2 ulp of H = |R0| + |x| |R2|, h_v of V = |R1| + |y| |R2|, one rounding of
// each product and of the difference), and the model built from the f32 P, A
// and B within E + 4.1 ulp of 7 (|.| |.| + |.| |.|) of the exact q; d is the
// sum.  f = q.x^2 + q.y^2 - 2 s q.z^2 is then a quadratic in t, a pixel's f is
// at least the model's minus 2 (|q.x| d.x + |q.y| d.y) + 2 s (2 |q.z| + d.z)
// d.z, and the f32 evaluation of the model's minimum errs by far less than
// 1e-4 of (|q.x| + |q.y|)^2 + 2 s q.z^2.  The minimum is at a corner, at the
// vertex of an edge parabola (value f - k^2 / h), or at the interior critical
// point when the Hessian is positive definite: then q.xy = 0 at some point of
// the pixel plane, the unconstrained minimum is <= 0, and a critical point
// inside the square keeps the quadrant.  Non-finite or huge values keep the
// quadrant.
VS_DEV float3 surf_q(float4 m0, float4 m1, float4 m2, float px, float py) {
    const float hux = m0.x - px * m1.z, huy = m0.y - px * m1.w, huz = m0.z - px * m2.x;
    const float hvx = m0.w - py * m1.z, hvy = m1.x - py * m1.w, hvz = m1.y - py * m2.x;
    return make_float3(huy * hvz - huz * hvy, huz * hvx - hux * hvz, hux * hvy - huy * hvx);
}
VS_DEV float surf_f(float3 p, float s2) { return p.x * p.x + p.y * p.y - s2 * (p.z * p.z); }
VS_DEV float surf_dot(float3 p, float3 d, float s2) { return p.x * d.x + p.y * d.y - s2 * (p.z * d.z); }
// Minimum over t in [0, 1] of f + 2 k t + h t^2 is below thr (the ends are
// tested separately): only a vertex inside the edge matters.
VS_DEV bool surf_edge_low(float f, float k, float h, float thr) {
    return h > 0.0f && k < 0.0f && -k < h && !(f - k * (k * __builtin_amdgcn_rcpf(h)) > thr);
}

VS_DEV bool surfel_quadrant_live(float x0, float y0, float4 m0, float4 m1, float4 m2, float opac, bool smooth) {
    const float cut = smooth ? (ALPHA_MID - 0.5f * ALPHA_BAND) : ALPHA_MID;
    const float s = QUAD_MARGIN_REL * logf_c(opac / cut) + QUAD_MARGIN_ABS;
    if (!(s < 3.0e38f)) return true;
    // low-pass disk around the projected centre (m2.y, m2.z)
    const float a0 = x0 - m2.y, a1 = a0 + 7.0f, b0 = y0 - m2.z, b1 = b0 + 7.0f;
    const float nx_ = __builtin_fminf(__builtin_fmaxf(0.0f, a0), a1), ny_ = __builtin_fminf(__builtin_fmaxf(0.0f, b0), b1);
    if (!(nx_ * nx_ + ny_ * ny_ > s)) return true;
    // pixel centres x0 + i, y0 + j exact in f32
    if (!(fabsf(x0) < 4.0e6f && fabsf(y0) < 4.0e6f)) return true;
    const float r0x = m0.x, r0y = m0.y, r0z = m0.z, r1x = m0.w, r1y = m1.x, r1z = m1.y;
    const float r2x = m1.z, r2y = m1.w, r2z = m2.x;
    const float xm = __builtin_fmaxf(fabsf(x0), fabsf(x0 + 7.0f)), ym = __builtin_fmaxf(fabsf(y0), fabsf(y0 + 7.0f));
    const float Hx = fabsf(r0x) + xm * fabsf(r2x), Hy = fabsf(r0y) + xm * fabsf(r2y), Hz = fabsf(r0z) + xm * fabsf(r2z);
    const float Vx = fabsf(r1x) + ym * fabsf(r2x), Vy = fabsf(r1y) + ym * fabsf(r2y), Vz = fabsf(r1z) + ym * fabsf(r2z);
    constexpr float ULP = 5.9604645e-8f;
    const float3 A = make_float3(7.0f * (r1y * r2z - r1z * r2y), 7.0f * (r1z * r2x - r1x * r2z), 7.0f * (r1x * r2y - r1y * r2x));
    const float3 B = make_float3(7.0f * (r0z * r2y - r0y * r2z), 7.0f * (r0x * r2z - r0z * r2x), 7.0f * (r0y * r2x - r0x * r2y));
    const float ax_ = fabsf(r2x), ay_ = fabsf(r2y), az_ = fabsf(r2z);
    const float dx = (13.0f * ULP) * (Hy * Vz + Hz * Vy) +
                     (28.7f * ULP) * ((fabsf(r1y) + fabsf(r0y)) * az_ + (fabsf(r1z) + fabsf(r0z)) * ay_);
    const float dy = (13.0f * ULP) * (Hz * Vx + Hx * Vz) +
                     (28.7f * ULP) * ((fabsf(r1z) + fabsf(r0z)) * ax_ + (fabsf(r1x) + fabsf(r0x)) * az_);
    const float dz = (13.0f * ULP) * (Hx * Vy + Hy * Vx) +
                     (28.7f * ULP) * ((fabsf(r1x) + fabsf(r0x)) * ay_ + (fabsf(r1y) + fabsf(r0y)) * ax_);
    const float3 p00 = surf_q(m0, m1, m2, x0, y0);
    const float3 p10 = make_float3(p00.x + A.x, p00.y + A.y, p00.z + A.z);
    const float3 p01 = make_float3(p00.x + B.x, p00.y + B.y, p00.z + B.z);
    const float3 p11 = make_float3(p10.x + B.x, p10.y + B.y, p10.z + B.z);
    const float s2 = 2.0f * s;
    const float qx = __builtin_fmaxf(__builtin_fmaxf(fabsf(p00.x), fabsf(p10.x)), __builtin_fmaxf(fabsf(p01.x), fabsf(p11.x)));
    const float qy = __builtin_fmaxf(__builtin_fmaxf(fabsf(p00.y), fabsf(p10.y)), __builtin_fmaxf(fabsf(p01.y), fabsf(p11.y)));
    const float qz = __builtin_fmaxf(__builtin_fmaxf(fabsf(p00.z), fabsf(p10.z)), __builtin_fmaxf(fabsf(p01.z), fabsf(p11.z)));
    const float qxy = qx + qy;
    const float M = qxy * qxy + s2 * (qz * qz);
    if (!(M < 1.0e36f)) return true;
    const float thr = 2.0f * (qx * dx + qy * dy) + s2 * ((2.0f * qz + dz) * dz) + 1.0e-4f * M;
    const float f00 = surf_f(p00, s2), f10 = surf_f(p10, s2), f01 = surf_f(p01, s2), f11 = surf_f(p11, s2);
    if (!(f00 > thr && f10 > thr && f01 > thr && f11 > thr)) return true;
    const float hA = surf_f(A, s2), hB = surf_f(B, s2), hAB = surf_dot(A, B, s2);
    const float g1 = surf_dot(p00, A, s2), g2 = surf_dot(p00, B, s2);
    if (surf_edge_low(f00, g1, hA, thr) || surf_edge_low(f01, surf_dot(p01, A, s2), hA, thr) ||
        surf_edge_low(f00, g2, hB, thr) || surf_edge_low(f10, surf_dot(p10, B, s2), hB, thr))
        return true;
    // interior critical point of a positive definite Hessian (scaled by 1/M)
    const float c = __builtin_amdgcn_rcpf(M);
    const float ha = hA * c, hb = hB * c, hab = hAB * c, ga = g1 * c, gb = g2 * c;
    const float det = ha * hb - hab * hab;
    if (ha > 0.0f && det > 0.0f) {
        const float n1 = hab * gb - hb * ga, n2 = hab * ga - ha * gb, lo = -1.0e-3f * det, hi = 1.001f * det;
        if (n1 >= lo && n1 <= hi && n2 >= lo && n2 <= hi) return true;
    }
    return false;
}

constexpr int FWD_BATCH = 64;

// Forward, kernels/rasterize.rs:109-420.  One 64-lane wavefront, its own
// workgroup, per 8 x 8 quadrant of a 16 x 16 tile, one pixel per lane.  The
// four quadrant workgroups of a tile are dealt to one XCD one after another
// (XCD b % 8 starts its blocks in index order; its i-th is quadrant i % 4 of
// the tile in dispatch slot i / 4), so the tile's splat rows are shared in
// one L2, yet no quadrant waits on another: each stages the tile's
// depth-sorted splats 64 at a time into its LDS, keeps in a compacted list
// those that may reach the quadrant (quadrant_live, surfel_quadrant_live), walks
// the list, and leaves as soon as its 64 pixels are done.  The tile's shrunk
// range end (one past its last blended intersection) is the maximum over its
// quadrants, kept with an atomic max on an end the dispatch-order pass set
// to the range start.
// The L1 term's cotangent at pixel (x, y) (crates/splat-train-loss/src/lib.rs:
// 786-811): sign(pred - gt) * inv_count on rgb inside the circle mask of
// radius mr about (mcx, mcy) (none for mr <= 0), 0 on alpha and outside; a
// packed target channel is its byte x (1/255) in f32 (lib.rs:93,1042-1044).
// l1_cotangent_kernel and the forward's fused epilogue both use these.
constexpr float L1_INV_255 = 1.0f / 255.0f;
VS_DEV float l1_sign(float p, float g, float inv) { const float d = p - g; return (d > 0.0f) ? inv : ((d < 0.0f) ? -inv : 0.0f); }
VS_DEV bool l1_in_mask(uint32_t x, uint32_t y, float mcx, float mcy, float mr) {
    if (!(mr > 0.0f)) return true;
    const float dx = (float)x + 0.5f - mcx, dy = (float)y + 0.5f - mcy;
    return dx * dx + dy * dy <= mr * mr;
}
VS_DEV float l1_unpack(uint32_t q, int c) { return (float)((q >> (8 * c)) & 0xFFu) * L1_INV_255; }

template <bool BWD, bool GEOM, bool SMOOTH, bool SURF>
__global__ void __launch_bounds__(FWD_BATCH) raster_fwd_kernel(RasterArgs a) {
    // Every per-splat array has 16-byte slots, so one LDS address, the slot's
    // byte offset kept in the list, serves all reads of a splat.
    // (surfels read neither the conic nor s_c: their blue channel rides in the
    // pad word of the fourth surfel row, and the smaller LDS footprint lets a
    // sixth wavefront onto each SIMD)
    __shared__ float4 s_a[SURF ? 1 : FWD_BATCH];    // x, y, A, B (the conic in base-2 units)
    __shared__ float4 s_b[FWD_BATCH];    // C, opacity, max(r,0), max(g,0)
    __shared__ float4 s_c[SURF ? 1 : FWD_BATCH];    // max(b,0), -, -, -
    __shared__ float4 s_d[(GEOM && !SURF) ? FWD_BATCH : 1];
    __shared__ float4 s_s[SURF ? FWD_BATCH * 4 : 1];   // row k of slot t at s_s[k * FWD_BATCH + t]
    __shared__ uint4 s_hit[BWD ? FWD_BATCH : 1];   // .x = 1 once the slot blended a pixel, .y once it stopped one
    __shared__ __align__(16) uint32_t s_list[FWD_BATCH];   // live slots as byte offsets (slot * 16)

    const uint32_t xcd = blockIdx.x % 8, idx = blockIdx.x / 8;
    const uint32_t q = idx % 4;
    const uint32_t slot = (idx / 4) * 8 + xcd;
    const uint32_t tile = block_tile(a.order, slot, a.num_tiles);
    if (tile >= a.num_tiles) return;   // uniform: padding of the dispatch order
    const uint32_t tx = tile % a.tile_bw, ty = tile / a.tile_bw;
    const uint32_t l = threadIdx.x;
    const uint32_t qx0 = tx * TILE_W + 8u * (q & 1u), qy0 = ty * TILE_W + 8u * (q >> 1);
    const uint32_t px = qx0 + compact_bits_16(l);
    const uint32_t py = qy0 + compact_bits_16(l >> 1);
    const bool inside = px < a.img_w && py < a.img_h;
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
    const float x0 = (float)qx0 + 0.5f, y0 = (float)qy0 + 0.5f;   // the quadrant's first pixel centre
    const uint32_t lo = a.ranges[tile * 2], hi = a.ranges[tile * 2 + 1];

    float T = 1.0f, cr = 0.0f, cg = 0.0f, cb = 0.0f;
    float depth_acc = 0.0f, median = 0.0f, dist_b = 0.0f, dist_c = 0.0f, nx = 0.0f, ny = 0.0f, nz = 0.0f;
    uint32_t median_id = 0xFFFFFFFFu;
    float surf_o = 0.0f;
    bool surf_found = false;
    bool done = !inside;
    uint32_t last = lo;
    const char* const lds_a = reinterpret_cast<const char*>(s_a);
    const char* const lds_b = reinterpret_cast<const char*>(s_b);
    const char* const lds_c = reinterpret_cast<const char*>(s_c);
    const char* const lds_d = reinterpret_cast<const char*>(s_d);
    const char* const lds_s = reinterpret_cast<const char*>(s_s);

    for (uint32_t start = lo; start < hi; start += FWD_BATCH) {
        if (__ballot(!done) == 0ull) break;           // every pixel of the quadrant is done
        const uint32_t rem = min((uint32_t)FWD_BATCH, hi - start);
        const uint32_t gid = (l < rem) ? a.gids[start + l] : 0xFFFFFFFFu;
        bool live = false;
        __syncthreads();                              // the previous batch's LDS reads are complete
        // whole 16-byte slots: lanes write consecutive addresses (a narrower
        // store at the 16-byte stride puts eight lanes on each bank)
        if constexpr (BWD) s_hit[l] = make_uint4(0u, 0u, 0u, 0u);
        if (gid < a.num_splats) {   // else: past the batch, or a corrupt id (dead slot)
            const float4* row = a.proj + (size_t)gid * PROJ_Q;
            const float4 pa = row[0];
            const float4 pb = row[1];
            const float4 pc = row[2];
            const float cb = pc.x;
            // the conic in base-2 units: sigma log2 e comes out of the same fma chain
            const float4 sa = make_float4(pa.x, pa.y, (0.5f * pa.z) * LOG2E_F, pa.w * LOG2E_F);
            const float4 sb = make_float4((0.5f * pb.x) * LOG2E_F, pb.y, mx(pb.z, 0.0f), mx(pb.w, 0.0f));
            if constexpr (!SURF) {
                s_a[l] = sa;
                s_c[l] = make_float4(mx(cb, 0.0f), 0.0f, 0.0f, 0.0f);
            }
            s_b[l] = sb;
            if constexpr (GEOM && !SURF) s_d[l] = a.proj_aux[gid];
            if constexpr (SURF) {
                const float4* ps = a.proj_surf + (size_t)gid * 4;
                float4 r[4];
#pragma unroll
                for (int k = 0; k < 4; ++k) r[k] = ps[k];
                r[3].w = mx(cb, 0.0f);   // the pad word
#pragma unroll
                for (int k = 0; k < 4; ++k) s_s[k * FWD_BATCH + l] = r[k];
                live = surfel_quadrant_live(x0, y0, r[0], r[1], r[2], pb.y, SMOOTH);
            } else {
                live = quadrant_live(x0, y0, sa.x, sa.y, sa.z, sa.w, sb.x, pc.y, SMOOTH);
            }
        }
        // the live slots in slot (= depth) order: the mask is walked in
        // scalar registers, lowest set bit first
        const uint64_t lm = __ballot(live);
        if (live) s_list[__builtin_amdgcn_mbcnt_hi((uint32_t)(lm >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)lm, 0u))] =
            l * 16u;
        __syncthreads();
        const uint32_t nlist = (uint32_t)__popcll(lm);
        uint32_t done_v = done ? 1u : 0u;   // carried in a vector register through the loop
        uint32_t stop_off = 0xFFFFFFFFu;    // the slot at which the lane's pixel stopped in this batch
        // A uniform loop over the list: every lane evaluates every pair and a
        // done lane only fails the blend test.  One divergent branch per pair
        // (the blend) keeps the scalar exec-mask work per pair small; the
        // scalar unit is shared by the CU's four SIMDs, and a per-lane loop
        // exit or a guard around the whole body costs it more per pair than
        // the vector work the masked lanes would skip.  One list entry: the
        // slot at LDS byte offset `off`.
        auto entry = [&](uint32_t off) {
            const float4 sb = *reinterpret_cast<const float4*>(lds_b + off);
            float sigma, zs = 0.0f, G;
            bool valid = true;
            if constexpr (SURF) {
                const float4* ss = reinterpret_cast<const float4*>(lds_s + off);
                const SurfelHit hit = surfel_hit(ss[0], ss[FWD_BATCH], ss[2 * FWD_BATCH], ss[3 * FWD_BATCH].z, pcx, pcy);
                valid = hit.valid;              // the ray misses the plane or meets it before the near limit
                sigma = hit.sigma;
                zs = hit.z;
                G = comp_exp2(-(sigma * LOG2E_F));
            } else {
                const float4 sa = *reinterpret_cast<const float4*>(lds_a + off);
                const float dx = pcx - sa.x, dy = pcy - sa.y;
                sigma = raster_sigma(sa.z, sa.w, sb.x, dx, dy);   // base 2
                G = comp_exp2(-sigma);
            }
            // min(0.999, .) of a product that is NaN only when sigma is
            // (then the sigma test below rejects the pair): same value as mn().
            const float alpha = __builtin_fminf(ALPHA_CAP, sb.y * G);
            const float w_cut = SMOOTH ? cutoff_weight(alpha) : ((alpha >= ALPHA_MID) ? 1.0f : 0.0f);
            const float ae = SMOOTH ? alpha * w_cut : alpha;
            const float nt = T * (1.0f - ae);
            const bool pass = done_v == 0u && valid && sigma >= 0.0f && w_cut > 0.0f;
            const bool stop = nt <= T_STOP;
            done_v = (pass && stop) ? 1u : done_v;
            if constexpr (BWD) stop_off = (pass && stop) ? off : stop_off;
            {
                if (pass && !stop) {
                    if constexpr (BWD) reinterpret_cast<uint4*>(reinterpret_cast<char*>(s_hit) + off)->x = 1u;
                    const float vis = ae * T;
                    const float cbv = SURF ? reinterpret_cast<const float4*>(lds_s + off)[3 * FWD_BATCH].w
                                           : reinterpret_cast<const float4*>(lds_c + off)->x;
                    cr = __builtin_fmaf(sb.z, vis, cr);
                    cg = __builtin_fmaf(sb.w, vis, cg);
                    cb = __builtin_fmaf(cbv, vis, cb);
                    if constexpr (GEOM) {
                        float4 d;
                        if constexpr (SURF) {
                            const float4* ss = reinterpret_cast<const float4*>(lds_s + off);
                            const float4 s2 = ss[2 * FWD_BATCH], s3 = ss[3 * FWD_BATCH];
                            d = make_float4(zs, s2.w, s3.x, s3.y);
                        } else {
                            d = *reinterpret_cast<const float4*>(lds_d + off);
                        }
                        const uint32_t t = off >> 4;
                        depth_acc = __builtin_fmaf(d.x, vis, depth_acc);
                        if (SURF && a.surf_crit) {
                            // unbiased-depth surface criterion (rasterize.rs:181-187, 346-354)
                            surf_o += ae + 0.1f * G;
                            if (!surf_found && (surf_o > 0.6f || T > 0.5f)) {
                                median = d.x; median_id = start + t; surf_found = surf_o > 0.6f;
                            }
                        } else if (T > 0.5f) {
                            median = d.x; median_id = start + t;
                        }
                        const float m = dist_depth(d.x);
                        dist_b = __builtin_fmaf(m, vis, dist_b);
                        dist_c = __builtin_fmaf(m * m, vis, dist_c);
                        nx = __builtin_fmaf(d.y, vis, nx);
                        ny = __builtin_fmaf(d.z, vis, ny);
                        nz = __builtin_fmaf(d.w, vis, nz);
                    }
                    T = nt;
                }
            }
        };
        // Full groups of eight entries (two 16-byte list reads each) run
        // without a bound test per entry (scalar compare-and-branch work the
        // CU's shared scalar unit would do); the last, partial group has its
        // own loop, so no entry is shared between the two paths (a shared
        // first entry made the compiler copy the accumulators there).
        uint32_t j0 = 0;
        for (; j0 + 8u <= nlist; j0 += 8u) {
            const uint4 la = *reinterpret_cast<const uint4*>(&s_list[j0]);
            const uint4 lb = *reinterpret_cast<const uint4*>(&s_list[j0 + 4u]);
            entry(la.x); entry(la.y); entry(la.z); entry(la.w);
            entry(lb.x); entry(lb.y); entry(lb.z); entry(lb.w);
            if (__ballot(done_v == 0u) == 0ull) break;   // every pixel of the quadrant is done (uniform)
        }
        // after a break every pixel is done and the ballot skips the rest
        if (j0 < nlist && __ballot(done_v == 0u) != 0ull) {
            // j0 <= 56: both reads stay inside the 64-entry list
            const uint4 la = *reinterpret_cast<const uint4*>(&s_list[j0]);
            const uint4 lb = *reinterpret_cast<const uint4*>(&s_list[j0 + 4u]);
            const uint32_t offs[8] = {la.x, la.y, la.z, la.w, lb.x, lb.y, lb.z, lb.w};
#pragma unroll
            for (uint32_t jj = 0; jj < 8u; ++jj) {
                if (j0 + jj >= nlist) break;                 // uniform
                entry(offs[jj]);
            }
        }
        done = done_v != 0u;
        if constexpr (BWD) {
            // A slot passes in this quadrant when one of its pixels blended it
            // or stopped at it (the backward's replay changes a pixel's state
            // only there), recorded per list entry for the backward.
            if (stop_off != 0xFFFFFFFFu) reinterpret_cast<uint4*>(reinterpret_cast<char*>(s_hit) + stop_off)->y = 1u;
            __syncthreads();
            const uint4 h = s_hit[l];
            const bool hit = gid < a.num_splats && h.x;
            if (hit) a.visible[gid] = 1.0f;
            if (l < rem && a.qpass) a.qpass[(size_t)(start + l) * 4 + q] = (h.x | h.y) ? (uint8_t)(1u << q) : (uint8_t)0u;
            // batches run in increasing order, so the batch's last blended
            // slot is the quadrant's last so far
            const uint64_t hm = __ballot(hit);
            if (hm != 0ull) last = start + 64u - (uint32_t)__builtin_clzll(hm);
        }
    }

    const float fr = __builtin_fmaf(T, a.bg_r, cr);
    const float fg = __builtin_fmaf(T, a.bg_g, cg);
    const float fb = __builtin_fmaf(T, a.bg_b, cb);
    const float fa = 1.0f - T;
    const size_t pid = (size_t)py * a.img_w + px;
    if (inside) {
        if constexpr (GEOM) {
            float4* o = reinterpret_cast<float4*>(a.out) + pid * 3;
            o[0] = make_float4(fr, fg, fb, fa);
            o[1] = make_float4(depth_acc, median, nx, ny);
            o[2] = make_float4(nz, dist_b, dist_c, as_f(median_id));
        } else if constexpr (BWD) {
            reinterpret_cast<float4*>(a.out)[pid] = make_float4(fr, fg, fb, fa);
            if (a.l1_v) {   // uniform: the L1 cotangent of this image (vs_render_forward_l1)
                const uint32_t q = a.l1_gt[pid];
                const float inv = a.l1_inv;
                reinterpret_cast<float4*>(a.l1_v)[pid] =
                    l1_in_mask(px, py, a.l1_mcx, a.l1_mcy, a.l1_mr)
                        ? make_float4(l1_sign(fr, l1_unpack(q, 0), inv), l1_sign(fg, l1_unpack(q, 1), inv),
                                      l1_sign(fb, l1_unpack(q, 2), inv), 0.0f)
                        : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
            }
        } else {
            const uint32_t r8 = f2u_sat(clampf(fr * 255.0f, 0.0f, 255.0f));
            const uint32_t g8 = f2u_sat(clampf(fg * 255.0f, 0.0f, 255.0f));
            const uint32_t b8 = f2u_sat(clampf(fb * 255.0f, 0.0f, 255.0f));
            const uint32_t a8 = f2u_sat(clampf(fa * 255.0f, 0.0f, 255.0f));
            reinterpret_cast<uint32_t*>(a.out)[pid] = r8 | (g8 << 8) | (b8 << 16) | (a8 << 24);
        }
    }
    if constexpr (BWD) {
        if (l == 0 && last > lo) {
            atomicMax(&a.ranges_shrunk[tile * 2 + 1], last);
            if (a.aux_ranges) atomicMax(&a.aux_ranges[tile * 2 + 1], last);
        }
    }
}

// 10-component reduce-scatter over a 64-lane wavefront, built from gfx950's
// cross-lane data paths instead of LDS permutes:
//   bit 5: v_permlane32_swap (5 pairs)   bit 4: v_permlane16_swap (3 pairs)
//   bit 3: DPP row_ror:8      (2 pairs)   bit 2: DPP row_half_mirror (1 pair)
//   bits 1, 0: DPP quad_perm full sums.
// A swap exchanges the upper lanes of its first operand with the lower lanes
// of its second, so after it "first + second" is, in every lane, the pair
// sum of the value that lane keeps.  Afterwards lane L holds the wave sum of
// component 5*b5 + 3*b4 + 2*b3 + b2 (b = bits of L) when that is < 10 and the
// sub-indices are not padding; lanes with L & 3 == 0 write it.
VS_DEV float swap32_sum(float keep_lo, float keep_hi) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(keep_lo), __float_as_uint(keep_hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
VS_DEV float swap16_sum(float keep_lo, float keep_hi) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(keep_lo), __float_as_uint(keep_hi), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
template <int CTRL>
VS_DEV float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, false));
}
constexpr int DPP_QUAD_XOR1 = 0xB1;       // quad_perm [1,0,3,2]
constexpr int DPP_QUAD_XOR2 = 0x4E;       // quad_perm [2,3,0,1]
constexpr int DPP_ROW_ROR8 = 0x128;       // rotate a 16-lane row by 8 (= lane ^ 8)
constexpr int DPP_ROW_HALF_MIRROR = 0x141; // lane i <-> 7 - i within each 8 lanes

VS_DEV int scatter_component(uint32_t lane) {
    const int i3 = ((lane & 8) ? 2 : 0) + ((lane & 4) ? 1 : 0);    // 3 = padding
    const int i5 = ((lane & 16) ? 3 : 0) + i3;                      // 5 = padding
    return (i3 < 3 && i5 < 5) ? ((lane & 32) ? 5 : 0) + i5 : -1;
}

// Sets a register to +0 where it lives.
VS_DEV void zero_in_place(float& x) { asm volatile("v_mov_b32 %0, 0" : "=v"(x)); }
// Sets a register pair to +0 with one 64-bit move.
VS_DEV void zero_pair(float& x, float& y) {
    double z;
    asm volatile("v_mov_b64 %0, 0" : "=v"(z));
    const unsigned long long u = (unsigned long long)__double_as_longlong(z);
    x = __uint_as_float((uint32_t)u);
    y = __uint_as_float((uint32_t)(u >> 32));
}

VS_DEV float reduce_scatter10(const float v[10], uint32_t lane) {
    float w[5];
#pragma unroll
    for (int i = 0; i < 5; ++i) w[i] = swap32_sum(v[i], v[i + 5]);
    float x[3];
    x[0] = swap16_sum(w[0], w[3]);
    x[1] = swap16_sum(w[1], w[4]);
    x[2] = swap16_sum(w[2], 0.0f);
    const bool h8 = lane & 8, h4 = lane & 4;
    const float y0 = (h8 ? x[2] : x[0]) + dpp<DPP_ROW_ROR8>(h8 ? x[0] : x[2]);
    const float y1 = (h8 ? 0.0f : x[1]) + dpp<DPP_ROW_ROR8>(h8 ? x[1] : 0.0f);
    float z = (h4 ? y1 : y0) + dpp<DPP_ROW_HALF_MIRROR>(h4 ? y0 : y1);
    z += dpp<DPP_QUAD_XOR2>(z);
    z += dpp<DPP_QUAD_XOR1>(z);
    return z;
}

// 17-component reduce-scatter on the same data paths (surfel gradients):
// bit 5 pairs component i with i + 9, bit 4 pairs 5 apart, bit 3 pairs 3
// apart, bit 2 pairs 2 apart, bit 1 pairs neighbours, bit 0 completes the
// sum.  Lane L then holds the wave sum of component
// 9*b5 + 5*b4 + 3*b3 + 2*b2 + b1 unless a sub-index is padding
// (scatter_component17 < 0); lanes with L & 1 == 0 write it.
VS_DEV int scatter_component17(uint32_t lane) {
    const int k = ((lane & 4) ? 2 : 0) + ((lane & 2) ? 1 : 0);      // 3 = padding
    const int j = ((lane & 8) ? 3 : 0) + k;                          // 5 = padding
    const int i = ((lane & 16) ? 5 : 0) + j;                         // 9 = padding
    const int c = ((lane & 32) ? 9 : 0) + i;                         // 17 = padding
    return (k < 3 && j < 5 && i < 9 && c < 17) ? c : -1;
}

VS_DEV float reduce_scatter17(const float v[17], uint32_t lane) {
    float w[9];
#pragma unroll
    for (int i = 0; i < 8; ++i) w[i] = swap32_sum(v[i], v[i + 9]);
    w[8] = swap32_sum(v[8], 0.0f);
    float x[5];
#pragma unroll
    for (int j = 0; j < 4; ++j) x[j] = swap16_sum(w[j], w[j + 5]);
    x[4] = swap16_sum(w[4], 0.0f);
    const bool h8 = lane & 8, h4 = lane & 4, h2 = lane & 2;
    const float y0 = (h8 ? x[3] : x[0]) + dpp<DPP_ROW_ROR8>(h8 ? x[0] : x[3]);
    const float y1 = (h8 ? x[4] : x[1]) + dpp<DPP_ROW_ROR8>(h8 ? x[1] : x[4]);
    const float y2 = (h8 ? 0.0f : x[2]) + dpp<DPP_ROW_ROR8>(h8 ? x[2] : 0.0f);
    const float z0 = (h4 ? y2 : y0) + dpp<DPP_ROW_HALF_MIRROR>(h4 ? y0 : y2);
    const float z1 = (h4 ? 0.0f : y1) + dpp<DPP_ROW_HALF_MIRROR>(h4 ? y1 : 0.0f);
    float u = (h2 ? z1 : z0) + dpp<DPP_QUAD_XOR2>(h2 ? z0 : z1);
    u += dpp<DPP_QUAD_XOR1>(u);
    return u;
}

// One 64-lane wavefront per tile; lane L owns pixel (L % 8, L / 8) of each
// 8x8 quadrant k (k = 0..3), so the quadrant masks turn into uniform branches.
// A lane sums its pixels' contributions in registers and the wavefront
// reduces each splat once.  PX = 1: images of fewer than BWD_QUAD_TILES
// tiles, which leave most SIMDs idle with one wavefront per tile, take one
// wavefront per quadrant instead (the four of a tile on one XCD, as in the
// forward); each reduces and adds its own sums.
constexpr int BWD_PX = 4;
constexpr uint32_t BWD_QUAD_TILES = 2048;

template <bool SMOOTH, int PX>
__global__ void __launch_bounds__(64) raster_bwd_kernel(RasterBwdArgs a) {
    // Per-splat values are formed once at staging, where one instruction
    // serves the 64 splats of a batch, not per (splat, wavefront) in the loop.
    __shared__ float4 s_a[BWD_BATCH];       // x, y, A, B (the forward's conic in base-2 units)
    __shared__ float4 s_b[BWD_BATCH];       // C, opacity, max(r,0), max(g,0)
    __shared__ float4 s_c[BWD_BATCH];       // max(b,0), c00, c11, colour gates (bits r,g,b >= 0, bit 3 set)
    __shared__ float4 s_d[BWD_BATCH];       // the conic's rows scaled to pixels: c00 W, c01 W, c01 H, c11 H
    __shared__ float s_c01[BWD_BATCH];      // c01

    uint32_t slot = blockIdx.x, q0 = 0u;      // q0: the first quadrant the wavefront owns
    if constexpr (PX == 1) {
        const uint32_t xcd = blockIdx.x % 8, idx = blockIdx.x / 8;
        q0 = idx % 4;
        slot = (idx / 4) * 8 + xcd;
    }
    const uint32_t tile = block_tile(a.order, slot, a.num_tiles);
    if (tile >= a.num_tiles) return;   // uniform: padding blocks of the XCD mapping
    const uint32_t lo = a.ranges[tile * 2], hi = a.ranges[tile * 2 + 1];
    if (lo >= hi) return;   // uniform per tile
    const uint32_t tx = tile % a.tile_bw, ty = tile / a.tile_bw;
    const uint32_t lane = threadIdx.x;
    const float img_w = (float)a.img_w, img_h = (float)a.img_h;
    const float x0 = (float)(tx * TILE_W) + 0.5f, y0 = (float)(ty * TILE_W) + 0.5f;

    // Pixel replay state, bwd/kernels/rasterize_backwards_planes.rs:194-209.
    // The reference carries the remaining colour S (3 channels) to form
    // v_alpha = (sum_c (T max(c,0) - S_c) v_c + v_t) / (1 - alpha); only
    // D = S . v - v_t enters it, so a lane carries that per pixel:
    // v_alpha = (T (max(c,0) . v) - D) / (1 - alpha), D -= vis (max(c,0) . v).
    float pcx[PX], pcy[PX], D[PX], T[PX];
    float vr[PX], vg[PX], vb[PX], rscale[PX];
    bool cot = false;   // a pixel of the lane has a nonzero (or non-finite) cotangent
#pragma unroll
    for (int k = 0; k < PX; ++k) {
        const uint32_t qk = q0 + (uint32_t)k;
        const uint32_t px = tx * TILE_W + 8 * (qk & 1) + (lane & 7);
        const uint32_t py = ty * TILE_W + 8 * (qk >> 1) + (lane >> 3);
        pcx[k] = (float)px + 0.5f;
        pcy[k] = (float)py + 0.5f;
        D[k] = T[k] = vr[k] = vg[k] = vb[k] = rscale[k] = 0.0f;
        if (px < a.img_w && py < a.img_h) {
            const size_t base = ((size_t)py * a.img_w + px) * a.channels;
            const float4 o = *reinterpret_cast<const float4*>(a.out_img + base);
            const float4 v = *reinterpret_cast<const float4*>(a.v_out + base);
            cot = cot || v.x != 0.0f || v.y != 0.0f || v.z != 0.0f || v.w != 0.0f;
            const float t_final = 1.0f - o.w;
            const float sr = o.x - t_final * a.bg_r;
            const float sg = o.y - t_final * a.bg_g;
            const float sb = o.z - t_final * a.bg_b;
            const float vt = (v.w - (a.bg_r * v.x + a.bg_g * v.y + a.bg_b * v.z)) * t_final;
            D[k] = (sr * v.x + sg * v.y + sb * v.z) - vt;
            T[k] = 1.0f;
            vr[k] = v.x; vg[k] = v.y; vb[k] = v.z;
            rscale[k] = __builtin_amdgcn_rcpf(mx(o.w, 1.0e-5f));
        }
    }
    // every gradient term is linear in the cotangent: a tile whose pixels all
    // have a zero one (outside a loss mask) adds nothing
    if (__ballot(cot) == 0ull) return;
    const int comp = scatter_component(lane);
    // Per-lane factor applied to the reduced sum: the conic sums are carried
    // as sum nv dx^2, nv dx dy, nv dy^2 with nv = alpha v_alpha = -v_sigma,
    // so v_conic = (-1/2, -1, -1/2) times them (exact scalings).
    const float comp_scale = (comp == 2 || comp == 4) ? -0.5f : ((comp == 3) ? -1.0f : 1.0f);
    // the colour rows (5, 6, 7) take the splat's c >= 0 gate, the rest bit 3 (always set)
    const uint32_t gate_shift = (comp >= 5 && comp <= 7) ? (uint32_t)(comp - 5) : 3u;
    float g[10];
#pragma unroll
    for (int i = 0; i < 10; ++i) g[i] = 0.0f;

    for (uint32_t start = lo; start < hi; start += BWD_BATCH) {
        uint32_t alive = 0;   // quadrants with a pixel still above T_STOP (uniform)
#pragma unroll
        for (int k = 0; k < PX; ++k) alive |= (__ballot(T[k] > T_STOP) != 0ull) ? (1u << k) : 0u;
        if (alive == 0) break;                              // every pixel of the tile is done
        // uniform; kept in a scalar register so the splat loop counts in SALU
        const uint32_t rem = __builtin_amdgcn_readfirstlane(min((uint32_t)BWD_BATCH, hi - start));
        __syncthreads();
        const uint32_t gid = (lane < rem) ? a.gids[start + lane] : 0xFFFFFFFFu;
        // Lane t stages splat t: its live-quadrant mask and id stay in this
        // lane's registers and reach the splat loop by readlane (a corrupt id
        // keeps mask 0: no quadrant).
        uint32_t mask = 0u;
        if (gid < a.num_splats) {
            const float4* row = a.proj + (size_t)gid * PROJ_Q;
            const float4 pa = row[0];
            const float4 pb = row[1];
            const float4 pc = row[2];
            const float cb = pc.x;
            // the forward's base-2 conic for the replay; c00, c01, c11 for the gradients
            const float4 sa = make_float4(pa.x, pa.y, (0.5f * pa.z) * LOG2E_F, pa.w * LOG2E_F);
            const float c2 = (0.5f * pb.x) * LOG2E_F;
            const uint32_t gates = (pb.z >= 0.0f ? 1u : 0u) | (pb.w >= 0.0f ? 2u : 0u) | (cb >= 0.0f ? 4u : 0u) | 8u;
            s_a[lane] = sa;
            s_b[lane] = make_float4(c2, pb.y, mx(pb.z, 0.0f), mx(pb.w, 0.0f));
            s_c[lane] = make_float4(mx(cb, 0.0f), pa.z, pb.x, as_f(gates));
            s_d[lane] = make_float4(pa.z * img_w, pa.w * img_w, pa.w * img_h, pb.x * img_h);
            s_c01[lane] = pa.w;
            if (a.qpass) {
                // the quadrants where the forward's replay passed this entry:
                // the others' pixels neither blend nor stop there
                const uint32_t w = a.qpass[start + lane];
                mask = (w | (w >> 8) | (w >> 16) | (w >> 24)) & 0xFu;
            } else {
                mask = quadrant_mask(x0, y0, sa.x, sa.y, sa.z, sa.w, c2, pc.y, SMOOTH);
            }
        }
        __syncthreads();
        for (uint32_t t = 0; t < rem; ++t) {
            const uint32_t live = (__builtin_amdgcn_readlane(mask, t) >> q0) & alive;
            if (live == 0) continue;                        // uniform: no quadrant reaches the cutoff
            const float4 sa = s_a[t];
            const float4 sbv = s_b[t];
            const float4 scv = s_c[t];
            const float4 sdv = s_d[t];
            const float opac = sbv.y;
            const float cl_r = sbv.z, cl_g = sbv.w, cl_b = scv.x;
#pragma unroll
            for (int k = 0; k < PX; ++k) {
                if (!((live >> k) & 1u)) continue;          // uniform
                // a done pixel (T = 0, as is a pixel outside the image) fails
                // the stop test below; a per-pixel guard here costs more than
                // the arithmetic it would mask
                const float Tk = T[k];
                const float dx = pcx[k] - sa.x, dy = pcy[k] - sa.y;
                const float sigma = raster_sigma(sa.z, sa.w, sbv.x, dx, dy);   // base 2, as the forward's
                const float G = comp_exp2(-sigma);
                const float alpha = __builtin_fminf(ALPHA_CAP, opac * G);   // == mn(): see the forward
                const float w_cut = SMOOTH ? cutoff_weight(alpha) : ((alpha >= ALPHA_MID) ? 1.0f : 0.0f);
                if (!(sigma >= 0.0f && w_cut > 0.0f)) continue;
                const float ae = SMOOTH ? alpha * w_cut : alpha;
                const float one_m = 1.0f - ae;
                const float nt = Tk * one_m;
                T[k] = (nt <= T_STOP) ? 0.0f : nt;
                if (nt <= T_STOP) continue;
                const float vis = ae * Tk;
                // colour: the c >= 0 gate is per splat, applied after the reduction
                g[5] = __builtin_fmaf(vis, vr[k], g[5]);
                g[6] = __builtin_fmaf(vis, vg[k], g[6]);
                g[7] = __builtin_fmaf(vis, vb[k], g[7]);
                const float cv = __builtin_fmaf(cl_b, vb[k], __builtin_fmaf(cl_g, vg[k], cl_r * vr[k]));
                const float ra = __builtin_amdgcn_rcpf(one_m);
                const float v_ae = __builtin_fmaf(Tk, cv, -D[k]) * ra;
                const float v_alpha = SMOOTH ? v_ae * (w_cut + alpha * cutoff_weight_deriv(alpha)) : v_ae;
                D[k] = __builtin_fmaf(-vis, cv, D[k]);
                if (opac * G <= ALPHA_CAP) {
                    const float nv = alpha * v_alpha;                // = -v_sigma
                    const float tx_ = nv * dx, ty_ = nv * dy;        // nv (pixel - mean)
                    // the mean gradient is conic . sum nv (pixel - mean): the conic is
                    // applied once per splat below; here only the sums
                    g[0] += tx_;
                    g[1] += ty_;
                    g[2] = __builtin_fmaf(tx_, dx, g[2]);
                    g[3] = __builtin_fmaf(tx_, dy, g[3]);
                    g[4] = __builtin_fmaf(ty_, dy, g[4]);
                    g[8] = __builtin_fmaf(v_alpha, G, g[8]);
                    // this pixel's mean gradient in pixels: (W (c00 tx + c01 ty), H (c01 tx + c11 ty))
                    const float ux = __builtin_fmaf(sdv.y, ty_, sdv.x * tx_);
                    const float uy = __builtin_fmaf(sdv.w, ty_, sdv.z * tx_);
                    g[9] = __builtin_fmaf(__builtin_amdgcn_sqrtf(__builtin_fmaf(ux, ux, uy * uy)), rscale[k], g[9]);
                }
            }
            // Every live splat is reduced: one whose live quadrants hold no
            // blending pixel (the forward only stopped pixels there) sums
            // zeros and adds nothing, and is rare enough that a ballot to
            // skip it (materialised from the exec masks per splat) cost more.
            {
                const float c00 = scv.y, c01 = s_c01[t], c11 = scv.z;
                const float sx = g[0], sy = g[1];
                g[0] = __builtin_fmaf(c01, sy, c00 * sx);
                g[1] = __builtin_fmaf(c11, sy, c01 * sx);
            }
            float val = reduce_scatter10(g, lane);
            // the sums restart at zero for the next splat, cleared in their own
            // registers (a plain assignment makes the compiler rebuild the
            // zeros at every branch of the next splat's quadrant loop)
#pragma unroll
            for (int i = 0; i < 10; i += 2) zero_pair(g[i], g[i + 1]);
            // the gate bit sign-extended to a mask: +0 where the gate is off
            val = __uint_as_float(__float_as_uint(val * comp_scale) &
                                  (uint32_t)__builtin_amdgcn_sbfe((int)as_u(scv.w), gate_shift, 1u));
            const uint32_t gid_t = __builtin_amdgcn_readlane(gid, t);
            if ((lane & 3) == 0 && comp >= 0 && val != 0.0f)
                atomicAdd(&a.v_combined[(size_t)gid_t * 10 + comp], val);
        }
    }
}

// Surfel (2DGS) backward, bwd/kernels/rasterize_backwards_planes.rs:266-480:
// a 256-thread workgroup per tile, one 64-lane wavefront per 8x8 quadrant and
// one pixel per lane.  Each pixel replays the forward with the remaining
// colour, depth, normal and distortion sums and their cotangents (the
// geometry channels composite like colours without a background).  Per batch
// of 64 splats, each wavefront walks the splats that may reach its quadrant
// (surfel_quadrant_live, the forward's test), reduce-scatters its pixels' 17
// gradient components [M rows, normal, rgb, alpha, refine] per splat
// (reduce_scatter17) and adds the 17 wave sums into the batch's LDS
// accumulator; after the batch the workgroup adds each splat's nonzero sums
// to v_combined [N,17], one atomic per component and tile.
// Six waves per SIMD (80 VGPRs, five values spilled) instead of the 89
// registers' five: 1.61 -> 1.56 ms at C3 (the loop is issue-bound, and a
// sixth wave hides more of its LDS and transcendental latency).
constexpr int SURF_BWD_BLOCK = 256;
template <bool SMOOTH>
__global__ void __launch_bounds__(SURF_BWD_BLOCK) __attribute__((amdgpu_waves_per_eu(6))) raster_bwd_surfel_kernel(RasterBwdArgs a) {
    __shared__ float4 s_s[BWD_BATCH * 4];   // M rows, centre, normal (vs_surfel.h layout): row k of splat t at
                                            // s_s[k * BWD_BATCH + t], so each wavefront's staging store is consecutive
    __shared__ float4 s_b[BWD_BATCH];       // opacity, max(r, 0), max(g, 0), max(b, 0)
    __shared__ uint32_t s_gate[BWD_BATCH];  // bit c: colour channel c is >= 0 (its gradient passes the clamp)
    __shared__ uint32_t s_gid[BWD_BATCH];
    __shared__ float s_acc[BWD_BATCH * SURFEL_GRADS];
    // per wavefront: whether any lane holds a nonzero cotangent / a pixel still
    // running (a ballot and one barrier in place of a workgroup OR-reduction)
    __shared__ uint4 s_any_cot, s_any_run;

    const uint32_t tile = block_tile(a.order, blockIdx.x, a.num_tiles);
    if (tile >= a.num_tiles) return;   // uniform: padding blocks of the XCD mapping
    const uint32_t lo = a.ranges[tile * 2], hi = a.ranges[tile * 2 + 1];
    if (lo >= hi) return;   // uniform per tile
    const uint32_t tx = tile % a.tile_bw, ty = tile / a.tile_bw;
    const uint32_t lane = threadIdx.x & 63u, q = threadIdx.x >> 6;
    const float img_w = (float)a.img_w, img_h = (float)a.img_h;
    const uint32_t qx0 = tx * TILE_W + 8u * (q & 1u), qy0 = ty * TILE_W + 8u * (q >> 1);
    const float x0 = (float)qx0 + 0.5f, y0 = (float)qy0 + 0.5f;   // the quadrant's first pixel centre

    const uint32_t px = qx0 + (lane & 7u), py = qy0 + (lane >> 3);
    const float pcx = (float)px + 0.5f, pcy = (float)py + 0.5f;
    float T = 0.0f, rscale = 0.0f;
    float sr = 0.0f, sg = 0.0f, sb = 0.0f, sz = 0.0f, snx = 0.0f, sny = 0.0f, snz = 0.0f, sdb = 0.0f, sdc = 0.0f;
    float vr = 0.0f, vg = 0.0f, vb = 0.0f, vt = 0.0f, vz = 0.0f, vmed = 0.0f, vnx = 0.0f, vny = 0.0f, vnz = 0.0f;
    float vdb = 0.0f, vdc = 0.0f;
    uint32_t med = 0xFFFFFFFFu;
    bool cot = false;   // the pixel has a nonzero (or non-finite) cotangent
    if (px < a.img_w && py < a.img_h) {
        const size_t base = ((size_t)py * a.img_w + px) * a.channels;
        const float4 o0 = *reinterpret_cast<const float4*>(a.out_img + base);
        const float4 o1 = *reinterpret_cast<const float4*>(a.out_img + base + 4);
        const float4 o2 = *reinterpret_cast<const float4*>(a.out_img + base + 8);
        const float4 v0 = *reinterpret_cast<const float4*>(a.v_out + base);
        const float4 v1 = *reinterpret_cast<const float4*>(a.v_out + base + 4);
        const float4 v2 = *reinterpret_cast<const float4*>(a.v_out + base + 8);
        cot = v0.x != 0.0f || v0.y != 0.0f || v0.z != 0.0f || v0.w != 0.0f || v1.x != 0.0f || v1.y != 0.0f ||
              v1.z != 0.0f || v1.w != 0.0f || v2.x != 0.0f || v2.y != 0.0f || v2.z != 0.0f || v2.w != 0.0f;
        const float t_final = 1.0f - o0.w;
        sr = o0.x - t_final * a.bg_r;
        sg = o0.y - t_final * a.bg_g;
        sb = o0.z - t_final * a.bg_b;
        T = 1.0f;
        vr = v0.x; vg = v0.y; vb = v0.z;
        vt = (v0.w - (a.bg_r * v0.x + a.bg_g * v0.y + a.bg_b * v0.z)) * t_final;
        rscale = 1.0f / mx(o0.w, 1.0e-5f);
        sz = o1.x; snx = o1.z; sny = o1.w; snz = o2.x; sdb = o2.y; sdc = o2.z;
        med = as_u(o2.w);
        vz = v1.x; vmed = v1.y; vnx = v1.z; vny = v1.w; vnz = v2.x; vdb = v2.y; vdc = v2.z;
    }
    // S.v: the channels still to come behind the current splat, dotted with the
    // cotangent (the only use of those sums); each blend takes vis (c.v) off it
    float sv_rest = sr * vr + sg * vg + sb * vb + sz * vz + snx * vnx + sny * vny + snz * vnz + sdb * vdb + sdc * vdc;
    // every gradient term is linear in the cotangent: a tile whose pixels all
    // have a zero one (outside a loss mask) adds nothing
    {
        const bool w = __ballot(cot) != 0ull;
        if (lane == 0) reinterpret_cast<uint32_t*>(&s_any_cot)[q] = w ? 1u : 0u;
        __syncthreads();
        const uint4 f = s_any_cot;
        if ((f.x | f.y | f.z | f.w) == 0u) return;
    }
    const int comp = (lane & 1u) ? -1 : scatter_component17(lane);   // the gradient component this lane adds
    const int gate_bit = (comp >= 12 && comp <= 14) ? comp - 12 : -1;  // rgb components: their clamp's gate
    for (uint32_t i = threadIdx.x; i < BWD_BATCH * SURFEL_GRADS; i += SURF_BWD_BLOCK) s_acc[i] = 0.0f;

    for (uint32_t start = lo; start < hi; start += BWD_BATCH) {
        // every pixel of the tile is done: the whole workgroup leaves together
        // (the previous batch's reads of s_any_run are behind its two barriers)
        {
            const bool w = __ballot(T > T_STOP) != 0ull;
            if (lane == 0) reinterpret_cast<uint32_t*>(&s_any_run)[q] = w ? 1u : 0u;
            __syncthreads();
            const uint4 f = s_any_run;
            if ((f.x | f.y | f.z | f.w) == 0u) break;
        }
        const uint32_t rem = min((uint32_t)BWD_BATCH, hi - start);
        // wavefront q stages row q of each splat's surfel record; wavefront 0 the rest
        if (lane < rem) {
            const uint32_t gid = a.gids[start + lane];
            if (gid < a.num_splats) {
                float4 row = a.proj_surf[(size_t)gid * 4 + q];
                if (q == 3) row.w = 1.0f / a.proj_surf[(size_t)gid * 4 + 2].x;   // 1 / M[2][2] in the pad slot
                s_s[q * BWD_BATCH + lane] = row;
                if (q == 0) {
                    const float4 pb = a.proj[(size_t)gid * PROJ_Q + 1];
                    const float cb_ = a.proj[(size_t)gid * PROJ_Q + 2].x;
                    s_b[lane] = make_float4(pb.y, mx(pb.z, 0.0f), mx(pb.w, 0.0f), mx(cb_, 0.0f));
                    s_gate[lane] = (pb.z >= 0.0f ? 1u : 0u) | (pb.w >= 0.0f ? 2u : 0u) | (cb_ >= 0.0f ? 4u : 0u);
                    s_gid[lane] = gid;
                }
            } else {   // a corrupt id: zero opacity never reaches the cutoff
                s_s[q * BWD_BATCH + lane] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
                if (q == 0) { s_b[lane] = make_float4(0.0f, 0.0f, 0.0f, 0.0f); s_gate[lane] = 0u; s_gid[lane] = 0u; }
            }
        }
        __syncthreads();
        // the batch's splats that may reach this quadrant, in depth order: with
        // the forward's pass bytes, exactly those at which a pixel of the
        // quadrant blended or stopped (the others change no pixel's state)
        bool live_t = false;
        if (lane < rem) {
            live_t = a.qpass ? ((a.qpass[start + lane] >> (8u * q)) & 0xFFu) != 0u
                             : surfel_quadrant_live(x0, y0, s_s[lane], s_s[BWD_BATCH + lane], s_s[2 * BWD_BATCH + lane],
                                                    s_b[lane].x, SMOOTH);
        }
        uint64_t live = __ballot(live_t);
        if (__ballot(T > T_STOP) == 0ull) live = 0ull;       // this quadrant is done
        while (live) {
            const uint32_t t = (uint32_t)__builtin_ctzll(live);
            live &= live - 1ull;
            const float4 m0 = s_s[t], m1 = s_s[BWD_BATCH + t], m2 = s_s[2 * BWD_BATCH + t], m3 = s_s[3 * BWD_BATCH + t];
            const float4 cb = s_b[t];
            const float opac = cb.x, cl_r = cb.y, cl_g = cb.z, cl_b = cb.w;
            const float r2x = m1.z, r2y = m1.w, r2z = m2.x, cen_x = m2.y, cen_y = m2.z;
            const float nrm_x = m2.w, nrm_y = m3.x, nrm_z = m3.y;
            const float inv_r2z = m3.w;
            // the projection's logf(opac / (1/255 - 5e-4)) + 1e-3: alpha is below the cutoff band beyond it
            const float sigma_max = m3.z;
            const uint32_t isect = start + t;
            // the replayed forward: which lanes blend this splat (every field of the
            // hit is computed, so the gradient below runs on every lane and one
            // select per component keeps the blending lanes' values)
            const SurfelHit h = surfel_hit<false, true>(m0, m1, m2, m3.z, pcx, pcy);
            const float G = comp_exp2(-(h.sigma * LOG2E_F));
            const float alpha = __builtin_fminf(ALPHA_CAP, opac * G);
            const float w_cut = SMOOTH ? cutoff_weight(alpha) : ((alpha >= ALPHA_MID) ? 1.0f : 0.0f);
            const float ae = alpha * w_cut;
            const float nt = T * (1.0f - ae);
            const bool blend = T > T_STOP && h.valid && h.sigma <= sigma_max && h.sigma >= 0.0f && w_cut > 0.0f;
            const bool stop = blend && nt <= T_STOP;
            const bool contrib = blend && !stop;
            if (stop) T = 0.0f;
            if (__ballot(contrib) == 0ull) continue;          // uniform: no lane blends it
            // Lanes that do not blend this splat must add exact zeros: every
            // component below is a product with vis, v_alpha or v_z, or with the
            // ray-plane terms su, sv, 1/q.z, and those (the only ones that can
            // be non-finite off the disk) are zeroed on such lanes, so each
            // gradient component is 0 there without a select of its own.
            // The gradient terms below are not part of the replay: they take
            // fused multiply-adds (the build contracts nothing by itself, so
            // that the replay above rounds as the forward does), and the
            // hardware reciprocal and square root (1 ulp) where the replay
            // keeps IEEE division.
            const float z = contrib ? h.z : 0.0f;
            // the distortion map and its slope from one hardware reciprocal
            // r = 1 / max(z, 0.2) (1 ulp): m = K (1 - 0.2 r), dm/dz = 0.2 K r^2
            // above z = 0.2 (m is flat below)
            const float rz = __builtin_amdgcn_rcpf(mx(z, 0.2f));
            const float m = 100.0f / (100.0f - 0.2f) * (1.0f - 0.2f * rz);
            const float dm_dz = (z > 0.2f) ? (100.0f / (100.0f - 0.2f) * 0.2f) * (rz * rz) : 0.0f;
            const float Tk = T;
            const float vis = contrib ? ae * Tk : 0.0f;
            float gs[SURFEL_GRADS];
            gs[12] = vis * vr;      // the colour clamps' gates apply to the wave sums below
            gs[13] = vis * vg;
            gs[14] = vis * vb;
            gs[9] = vis * vnx;
            gs[10] = vis * vny;
            gs[11] = vis * vnz;
            const float ra = __builtin_amdgcn_rcpf(1.0f - ae);
            // this splat's channels at the pixel, dotted with the cotangent
            float cv = cl_r * vr;
            cv = __builtin_fmaf(cl_g, vg, cv);
            cv = __builtin_fmaf(cl_b, vb, cv);
            cv = __builtin_fmaf(z, vz, cv);
            cv = __builtin_fmaf(nrm_x, vnx, cv);
            cv = __builtin_fmaf(nrm_y, vny, cv);
            cv = __builtin_fmaf(nrm_z, vnz, cv);
            cv = __builtin_fmaf(m, __builtin_fmaf(m, vdc, vdb), cv);
            const float v_ae = __builtin_fmaf(vt, ra, __builtin_fmaf(Tk, cv, -sv_rest) * ra);
            const float v_alpha_c = SMOOTH ? v_ae * (w_cut + alpha * cutoff_weight_deriv(alpha)) : v_ae;
            const bool unsat = contrib && opac * G <= ALPHA_CAP;
            const float v_alpha = unsat ? v_alpha_c : 0.0f;
            const float v_z = __builtin_fmaf(vis, __builtin_fmaf(__builtin_fmaf(m + m, vdc, vdb), dm_dz, vz), (contrib && isect == med) ? vmed : 0.0f);
            const float v_sigma = -alpha * v_alpha;
            gs[15] = v_alpha * G;
            const float su = contrib ? h.su : 0.0f, sv = contrib ? h.sv : 0.0f;
            const bool use_3d = h.s3d <= h.s2d;
            const float v_su = __builtin_fmaf(v_z, r2x, use_3d ? v_sigma * su : 0.0f);
            const float v_sv = __builtin_fmaf(v_z, r2y, use_3d ? v_sigma * sv : 0.0f);
            const float v_s2 = use_3d ? 0.0f : -2.0f * v_sigma;
            const float v_cx = v_s2 * h.dxs, v_cy = v_s2 * h.dys;
            const float inv_qz = contrib ? h.rq : 0.0f;   // the replay's 1 / q.z
            const float vqx = v_su * inv_qz, vqy = v_sv * inv_qz, vqz = -__builtin_fmaf(v_su, su, v_sv * sv) * inv_qz;
            // q = h_u x h_v: v_hu = h_v x v_q, v_hv = v_q x h_u
            const float vhux = __builtin_fmaf(h.hvy, vqz, -(h.hvz * vqy)), vhuy = __builtin_fmaf(h.hvz, vqx, -(h.hvx * vqz));
            const float vhuz = __builtin_fmaf(h.hvx, vqy, -(h.hvy * vqx));
            const float vhvx = __builtin_fmaf(vqy, h.huz, -(vqz * h.huy)), vhvy = __builtin_fmaf(vqz, h.hux, -(vqx * h.huz));
            const float vhvz = __builtin_fmaf(vqx, h.huy, -(vqy * h.hux));
            const float g0 = vhux, g1 = vhuy, g2 = __builtin_fmaf(v_cx, inv_r2z, vhuz);
            const float g3 = vhvx, g4 = vhvy, g5 = __builtin_fmaf(v_cy, inv_r2z, vhvz);
            gs[0] = g0; gs[1] = g1; gs[2] = g2; gs[3] = g3; gs[4] = g4; gs[5] = g5;
            gs[6] = __builtin_fmaf(v_z, su, -__builtin_fmaf(pcx, vhux, pcy * vhvx));
            gs[7] = __builtin_fmaf(v_z, sv, -__builtin_fmaf(pcx, vhuy, pcy * vhvy));
            gs[8] = v_z - __builtin_fmaf(pcx, vhuz, __builtin_fmaf(pcy, vhvz, __builtin_fmaf(v_cx, cen_x, v_cy * cen_y) * inv_r2z));
            // refine weight: this pixel's gradient of a screen-space shift of the surfel (M -> T M)
            const float shx = __builtin_fmaf(g0, r2x, __builtin_fmaf(g1, r2y, g2 * r2z));
            const float shy = __builtin_fmaf(g3, r2x, __builtin_fmaf(g4, r2y, g5 * r2z));
            const float ux = shx * img_w, uy = shy * img_h;
            gs[16] = __builtin_amdgcn_sqrtf(__builtin_fmaf(ux, ux, uy * uy)) * rscale;
            if (contrib) {
                sv_rest = __builtin_fmaf(-vis, cv, sv_rest);
                T = nt;
            }
            float mine = reduce_scatter17(gs, lane);
            if (gate_bit >= 0 && !((s_gate[t] >> gate_bit) & 1u)) mine = 0.0f;
            if (comp >= 0 && mine != 0.0f) atomicAdd(&s_acc[t * SURFEL_GRADS + comp], mine);
        }
        __syncthreads();
        for (uint32_t i = threadIdx.x; i < rem * SURFEL_GRADS; i += SURF_BWD_BLOCK) {
            const float v = s_acc[i];
            if (v != 0.0f) {
                atomicAdd(&a.v_combined[(size_t)s_gid[i / SURFEL_GRADS] * SURFEL_GRADS + i % SURFEL_GRADS], v);
                s_acc[i] = 0.0f;
            }
        }
    }
}

// sign(pred - gt) * inv_count on rgb, 0 on the other channels and outside
// the mask (l1_sign, l1_in_mask).  Images whose channel count is a multiple
// of 4 (RGBA, the 12-channel geometry render) are read and written as
// float4s: the first holds rgb, the rest are zero.  A PACKED target is [H,W]
// RGBA8 (r in the low byte, l1_unpack).

template <bool VEC4, bool PACKED>
__global__ void l1_cotangent_kernel(const float* __restrict__ pred, uint32_t C, const void* __restrict__ gt_in, uint32_t w,
                                    uint32_t h, float mcx, float mcy, float mr, float inv_count, float* __restrict__ v) {
    const uint32_t pid = blockIdx.x * blockDim.x + threadIdx.x;
    if (pid >= w * h) return;
    const uint32_t x = pid % w, y = pid / w;
    const bool in_mask = l1_in_mask(x, y, mcx, mcy, mr);
    const float inv = in_mask ? inv_count : 0.0f;
    float g0, g1, g2;
    if constexpr (PACKED) {
        const uint32_t q = static_cast<const uint32_t*>(gt_in)[pid];
        g0 = l1_unpack(q, 0);
        g1 = l1_unpack(q, 1);
        g2 = l1_unpack(q, 2);
    } else {
        const float* gt = static_cast<const float*>(gt_in);
        g0 = gt[(size_t)pid * 3]; g1 = gt[(size_t)pid * 3 + 1]; g2 = gt[(size_t)pid * 3 + 2];
    }
    if constexpr (VEC4) {
        const uint32_t q4 = C / 4;
        const float4 p = reinterpret_cast<const float4*>(pred)[(size_t)pid * q4];
        float4* o = reinterpret_cast<float4*>(v) + (size_t)pid * q4;
        o[0] = in_mask ? make_float4(l1_sign(p.x, g0, inv), l1_sign(p.y, g1, inv), l1_sign(p.z, g2, inv), 0.0f)
                       : make_float4(0.0f, 0.0f, 0.0f, 0.0f);
        for (uint32_t k = 1; k < q4; ++k) o[k] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    } else {
        const float gg[3] = {g0, g1, g2};
        for (uint32_t c = 0; c < C; ++c)
            v[(size_t)pid * C + c] = (c < 3 && in_mask) ? l1_sign(pred[(size_t)pid * C + c], gg[c], inv) : 0.0f;
    }
}

// Every tile's range starts as (0xFFFFFFFF, 0): the sort's range pass
// lowers starts and raises ends.
__global__ void ranges_init_kernel(uint32_t* __restrict__ ranges, uint32_t num_tiles) {
    const uint32_t t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t < num_tiles) reinterpret_cast<uint2*>(ranges)[t] = make_uint2(0xFFFFFFFFu, 0u);
}
hipError_t launch_ranges_init(uint32_t* ranges, uint32_t num_tiles, hipStream_t s) {
    if (num_tiles == 0) return hipSuccess;
    ranges_init_kernel<<<(num_tiles + 255) / 256, 256, 0, s>>>(ranges, num_tiles);
    return hipGetLastError();
}

// The sorted tile ids, rebuilt from the ranges (one workgroup per tile; the
// caller fills the list with the sentinel first).
__global__ void tiles_from_ranges_kernel(const uint32_t* __restrict__ ranges, uint32_t n, uint32_t* __restrict__ tiles) {
    const uint32_t t = blockIdx.x;
    const uint32_t lo = ranges[2 * t], hi = min(ranges[2 * t + 1], n);
    for (uint32_t i = lo + threadIdx.x; i < hi; i += blockDim.x) tiles[i] = t;
}
hipError_t launch_tiles_from_ranges(const uint32_t* ranges, uint32_t num_tiles, uint32_t n, uint32_t* tiles,
                                    hipStream_t s) {
    if (n == 0) return hipSuccess;
    hipError_t e = launch_fill_u32(tiles, num_tiles, n, s);
    if (e != hipSuccess || num_tiles == 0) return e;
    tiles_from_ranges_kernel<<<num_tiles, 256, 0, s>>>(ranges, n, tiles);
    return hipGetLastError();
}

hipError_t launch_tile_ranges(const uint32_t* tiles, uint32_t n, uint32_t num_tiles, uint32_t* ranges, hipStream_t s,
                              const uint32_t* n_dev) {
    if (n == 0) return hipSuccess;
    tile_ranges_kernel<<<(uint32_t)(((uint64_t)n + 1023) / 1024), 256, 0, s>>>(tiles, n, num_tiles, ranges, n_dev);
    return hipGetLastError();
}

hipError_t launch_tile_order(uint32_t* ranges, uint32_t num_tiles, uint32_t* order, hipStream_t s,
                             uint32_t* shrunk_init, bool fix_empty, const uint32_t* flags_from, uint32_t* flags_to,
                             uint32_t nflags, uint32_t* aux_out, float* zero, uint64_t zero_floats) {
    if (num_tiles == 0) return hipSuccess;
    if (!flags_to) nflags = 0;
    // the clearing blocks store float2
    if (zero && ((uintptr_t)zero & 7u)) return hipErrorInvalidValue;
    if (!zero) zero_floats = 0;
    const uint64_t pairs = zero_floats / 2;
    const uint32_t fill_blocks =
        zero_floats ? (uint32_t)std::min<uint64_t>((pairs + ORDER_BLOCK * 4 - 1) / (ORDER_BLOCK * 4) + 1, 2048) : 0u;
    tile_order_kernel<<<8 + fill_blocks, ORDER_BLOCK, 0, s>>>(ranges, num_tiles, order, shrunk_init, fix_empty ? 1 : 0,
                                                              flags_from, flags_to, nflags, aux_out, zero, zero_floats);
    return hipGetLastError();
}

hipError_t launch_raster_fwd(const RasterArgs& a, bool bwd_info, bool geometry, bool smooth, hipStream_t s) {
    if (a.num_tiles == 0) return hipSuccess;
    const dim3 grid(4 * xcd_grid(a.num_tiles));   // four quadrant workgroups per dispatch slot
    if (a.proj_surf) {           // surfels: every bwd-info pass carries the geometry channels
        if (!bwd_info) raster_fwd_kernel<false, false, false, true><<<grid, FWD_BATCH, 0, s>>>(a);
        else if (smooth) raster_fwd_kernel<true, true, true, true><<<grid, FWD_BATCH, 0, s>>>(a);
        else raster_fwd_kernel<true, true, false, true><<<grid, FWD_BATCH, 0, s>>>(a);
    } else if (!bwd_info) raster_fwd_kernel<false, false, false, false><<<grid, FWD_BATCH, 0, s>>>(a);
    else if (geometry) raster_fwd_kernel<true, true, false, false><<<grid, FWD_BATCH, 0, s>>>(a);
    else if (smooth) raster_fwd_kernel<true, false, true, false><<<grid, FWD_BATCH, 0, s>>>(a);
    else raster_fwd_kernel<true, false, false, false><<<grid, FWD_BATCH, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_raster_bwd(const RasterBwdArgs& a, bool smooth, hipStream_t s, hipEvent_t start, hipEvent_t stop) {
    if (a.num_tiles == 0) return hipSuccess;
    dim3 grid(xcd_grid(a.num_tiles));
    void (*k)(RasterBwdArgs);
    uint32_t block = 64;
    if (a.proj_surf) {
        k = smooth ? raster_bwd_surfel_kernel<true> : raster_bwd_surfel_kernel<false>;
        block = SURF_BWD_BLOCK;
    } else if (a.num_tiles < BWD_QUAD_TILES) {
        k = smooth ? raster_bwd_kernel<true, 1> : raster_bwd_kernel<false, 1>;
        grid = dim3(4 * xcd_grid(a.num_tiles));   // four quadrant wavefronts per dispatch slot
    } else {
        k = smooth ? raster_bwd_kernel<true, BWD_PX> : raster_bwd_kernel<false, BWD_PX>;
    }
    if (start) hipExtLaunchKernelGGL(k, grid, dim3(block), 0, s, start, stop, 0u, a);
    else k<<<grid, block, 0, s>>>(a);
    return hipGetLastError();
}

// out[i] = comp_exp2(x) for the f32 x whose bit pattern is first_bits + i.
__global__ void __launch_bounds__(256) exp2_range_kernel(uint32_t first_bits, uint64_t count, float* __restrict__ out) {
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < count; i += stride)
        out[i] = comp_exp2(__uint_as_float(first_bits + (uint32_t)i));
}

// out[i] = div_cr(a, b) for the f32 b whose bit pattern is bits[i].
__global__ void __launch_bounds__(256) division_values_kernel(float a, const uint32_t* __restrict__ bits, uint64_t count,
                                                              float* __restrict__ out) {
    const uint64_t stride = (uint64_t)gridDim.x * 256u;
    for (uint64_t i = (uint64_t)blockIdx.x * 256u + threadIdx.x; i < count; i += stride)
        out[i] = div_cr(a, __uint_as_float(bits[i]));
}
// *mismatches += the bit patterns b, of all 2^32, at which div_cr(a, b) and the
// division a / b differ (two NaNs agree); each thread takes 256 consecutive b.
constexpr uint32_t DIV_CHECK_PER_THREAD = 256;
__global__ void __launch_bounds__(256) division_check_kernel(float a, unsigned long long* __restrict__ mismatches) {
    const uint64_t base = ((uint64_t)blockIdx.x * 256u + threadIdx.x) * DIV_CHECK_PER_THREAD;
    uint32_t bad = 0;
    for (uint32_t k = 0; k < DIV_CHECK_PER_THREAD; ++k) {
        const float b = __uint_as_float((uint32_t)(base + k));
        const float x = div_cr(a, b), y = a / b;
        bad += (__float_as_uint(x) != __float_as_uint(y) && !(x != x && y != y)) ? 1u : 0u;
    }
    uint32_t wave_bad = bad;
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) wave_bad += (uint32_t)__shfl_xor((int)wave_bad, o);
    if ((threadIdx.x & 63u) == 0u && wave_bad) atomicAdd(mismatches, (unsigned long long)wave_bad);
}

hipError_t launch_division_values(float a, const uint32_t* bits, uint64_t count, float* out, hipStream_t s) {
    if (count == 0) return hipSuccess;
    const uint32_t grid = (uint32_t)std::min<uint64_t>(16384u, (count + 255u) / 256u);
    division_values_kernel<<<grid, 256, 0, s>>>(a, bits, count, out);
    return hipGetLastError();
}
hipError_t launch_division_check(float a, unsigned long long* mismatches, hipStream_t s) {
    // 2^32 patterns: 65536 blocks x 256 threads x 256 patterns
    division_check_kernel<<<(uint32_t)((1ull << 32) / (256ull * DIV_CHECK_PER_THREAD)), 256, 0, s>>>(a, mismatches);
    return hipGetLastError();
}

hipError_t launch_exp2_range(uint32_t first_bits, uint64_t count, float* out, hipStream_t s) {
    if (count == 0) return hipSuccess;
    const uint32_t grid = (uint32_t)std::min<uint64_t>(16384u, (count + 255u) / 256u);
    exp2_range_kernel<<<grid, 256, 0, s>>>(first_bits, count, out);
    return hipGetLastError();
}

hipError_t launch_l1_cotangent(const float* pred, uint32_t channels, const void* gt, bool packed, uint32_t w, uint32_t h,
                               float mcx, float mcy, float mr, float inv_count, float* v_out, hipStream_t s) {
    const uint32_t n = w * h;
    if (n == 0) return hipSuccess;
    const bool vec4 = channels >= 4 && channels % 4 == 0 && ((uintptr_t)pred & 15u) == 0 && ((uintptr_t)v_out & 15u) == 0;
    const dim3 grid((n + 255) / 256);
    if (vec4 && packed) l1_cotangent_kernel<true, true><<<grid, 256, 0, s>>>(pred, channels, gt, w, h, mcx, mcy, mr, inv_count, v_out);
    else if (vec4) l1_cotangent_kernel<true, false><<<grid, 256, 0, s>>>(pred, channels, gt, w, h, mcx, mcy, mr, inv_count, v_out);
    else if (packed) l1_cotangent_kernel<false, true><<<grid, 256, 0, s>>>(pred, channels, gt, w, h, mcx, mcy, mr, inv_count, v_out);
    else l1_cotangent_kernel<false, false><<<grid, 256, 0, s>>>(pred, channels, gt, w, h, mcx, mcy, mr, inv_count, v_out);
    return hipGetLastError();
}

} // namespace vs
