// k_project.hip -- projection, culling, tile counting and intersection emission.
//
// One fused kernel replaces the reference's project_forward + project_visible
// (crates/splat-train-render/src/kernels/project_forward.rs:26-261,
// kernels/project_visible.rs:97-312): each lane owns one splat, culls it, and a
// surviving splat reads its SH row, writes its projected row at its global id
// (no compaction of the rows) and counts the tiles its ellipse touches.
//
// Binning then follows the reference's order of work (render.rs:689-794) on
// smaller keys: the splats that hit a tile are compacted in global-id order
// with their depth bits (less the minimum) as u32 keys, a stable radix sort
// puts them in depth order (ties in global-id order), a scan of their tile
// counts in that order gives each one its slot range, and emission writes one
// u32 tile id per hit tile into that range.  A stable sort by tile id then
// yields each tile's list in (depth bits, global id) order.  Counting and
// emission test only the tiles near the ellipse's boundary (see walk_rows).
#include <algorithm>
#include "vs_device.h"
#include "vs_camera.h"
#include "vs_sh.h"
#include "vs_neural.h"
#include "vs_surfel.h"
#include "vs_internal.h"

namespace vs {

constexpr int PROJ_BLOCK = 256;

struct TileBox { uint32_t x0, y0, x1, y1; };

// kernels/helpers.rs:133-144
VS_DEV void bbox_extent(S2 c, float power, float& ex, float& ey) {
    const float det = c.c00 * c.c11 - c.c01 * c.c01;
    const bool degenerate = det <= 0.0f;
    const float inv_det = degenerate ? 0.0f : 1.0f / det;
    const float ex_ = __builtin_sqrtf(2.0f * power * c.c11 * inv_det);
    const float ey_ = __builtin_sqrtf(2.0f * power * c.c00 * inv_det);
    ex = degenerate ? -1.0f : ex_;
    ey = degenerate ? -1.0f : ey_;
}
// kernels/helpers.rs:160-190
VS_DEV TileBox tile_box(float cx, float cy, float ex, float ey, uint32_t bw, uint32_t bh) {
    const float x = cx / 16.0f, y = cy / 16.0f, dx = ex / 16.0f, dy = ey / 16.0f;
    const float bwf = (float)bw, bhf = (float)bh;
    return TileBox{f2u_sat(clampf(x - dx, 0.0f, bwf)), f2u_sat(clampf(y - dy, 0.0f, bhf)),
                   f2u_sat(clampf(x + dx + 1.0f, 0.0f, bwf)), f2u_sat(clampf(y + dy + 1.0f, 0.0f, bhf))};
}
// kernels/helpers.rs:275-314 (StopThePop conservative ellipse-rectangle test)
VS_DEV bool will_contribute(uint32_t tx, uint32_t ty, float mx_, float my_, S2 c, float power) {
    const float x0 = (float)(tx * TILE_W), y0 = (float)(ty * TILE_W);
    const float x1 = x0 + (float)TILE_W, y1 = y0 + (float)TILE_W;
    const bool xl = mx_ < x0, xr = mx_ > x1;
    const bool in_x = !(xl || xr);
    const bool ya = my_ < y0, yb = my_ > y1;
    const bool in_y = !(ya || yb);
    if (in_x && in_y) return true;
    const float cx = xl ? x0 : x1, cy = ya ? y0 : y1;
    const float w = x1 - x0, h = y1 - y0;
    const float dxf = xl ? w : -w, dyf = ya ? h : -h;
    const float ddx = mx_ - cx, ddy = my_ - cy;
    const float txr = (dxf * c.c00 * ddx + dxf * c.c01 * ddy) / (dxf * c.c00 * dxf);
    const float tyr = (dyf * c.c01 * ddx + dyf * c.c11 * ddy) / (dyf * c.c11 * dyf);
    const float tx_ = in_y ? 0.0f : clampf(txr, 0.0f, 1.0f);
    const float ty_ = in_x ? 0.0f : clampf(tyr, 0.0f, 1.0f);
    return calc_sigma(cx + tx_ * dxf, cy + ty_ * dyf, c, mx_, my_) <= power;
}

VS_DEV uint32_t lane_id() { return __lane_id(); }
VS_DEV float rl(float v, int lane) { return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane)); }
VS_DEV uint32_t rl(uint32_t v, int lane) { return (uint32_t)__builtin_amdgcn_readlane((int)v, lane); }

// ---- tile walk: exact ranges per tile row, tests only at the boundary --------
// The reference tests every tile of a box, a small box per thread and a large
// one per subgroup (kernels/map_gaussians.rs:17-19, project_forward.rs:198-247).
// Here each tile row of a box is split, from the ellipse's chords in double
// precision (square roots within 1e-11 relative, chord_sqrt), into
//   * tiles outside an outer range, which the test cannot pass: they lie
//     outside the ellipse sigma <= P (1 + 4e-3) + 1e-4 with half a pixel to
//     spare, while the test evaluates sigma at a point of the tile (within
//     5e-4 px of it) in f32, within 5 ulp x (1 + rho) / (1 - rho) = 1.3e-3
//     relative for the conics admitted below (rho = |c01| / sqrt(c00 c11));
//   * tiles inside an interior (certain) range, which it must pass: each
//     holds, 0.05 px inside its edges, a point with sigma <= P (1 - 4e-3)
//     - 1e-4 (the range spans the x extent of that ellipse over the row);
//   * the rest, on which will_contribute runs as the reference's does: at
//     most a tile or two at each end of a row.
// Conics with c01^2 > 0.999 c00 c11 (f32 sigma too inexact to rely on) test
// every tile of the box.  All of it is load-balanced over the wavefront: its
// box rows are laid end to end and walked 64 at a time, and each step's
// boundary tiles (and, for emission, interior tiles) likewise.  The set of
// tiles that pass is exactly the reference's; emission writes a splat's tiles
// in an order of its own, which the stable tile sort makes irrelevant (a
// splat has one entry per tile, and entries of one tile keep slot order).
constexpr float BAND_OUT = 0.5f;      // px of slack around the outer range
constexpr float BAND_IN = 0.05f;      // px of slack inside the interior range

struct RowLds {
    float4 geo[64];       // per splat: px, py, c00, c01
    float2 geo2[64];      // c11, power
    uint4 box[64];        // x0, x1, y0, exact ranges (1) or every tile (0)
    uint4 word[64];       // caller words: slot base, global id, count
    uint32_t acc[64];     // per splat: tiles that passed (count) / slots taken (emission)
    uint32_t mark[64];    // per step: lane whose run starts at this position
    uint32_t mark2[64];
    uint4 row[64];        // per row of the step: owner, ty, oa, ia
    uint4 row2[64];       // ib, ob, first interior slot, -
    uint32_t tmp[64];
};

VS_DEV void wave_sync() { __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront"); __builtin_amdgcn_wave_barrier();
                          __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront"); }

// One step of an enumeration over per-lane runs of n items, laid end to end.
struct EnumStep {
    bool active, head;    // head: first lane of its run within the step
    uint32_t owner;       // lane whose run holds this lane's item
    uint32_t idx;         // the item's index within that run
    uint64_t seg;         // lanes of the step holding items of the same run
};
// Every lane calls this together; `visit(EnumStep)` runs once per step on
// every lane.  `mark` is the wavefront's 64-word LDS scratch for the step.
template <typename Visit>
VS_DEV void wave_enum(uint32_t* mark, uint32_t n, Visit&& visit) {
    const uint32_t lane = __lane_id();
    uint32_t incl = n;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o);
        if ((int)lane >= o) incl += t;
    }
    const uint32_t excl = incl - n;
    const uint32_t total = (uint32_t)__builtin_amdgcn_readlane((int)incl, 63);
    const uint64_t le = (lane == 63) ? ~0ull : ((2ull << lane) - 1ull);
    for (uint32_t c0 = 0; c0 < total; c0 += 64) {
        mark[lane] = 0xFFFFFFFFu;
        wave_sync();
        if (n > 0 && excl >= c0 && excl - c0 < 64u) mark[excl - c0] = lane;
        wave_sync();
        const uint64_t starts = __ballot(mark[lane] != 0xFFFFFFFFu);
        const uint64_t carry = __ballot(n > 0 && excl < c0 && incl > c0);   // run begun in an earlier step
        const uint64_t below = starts & le;
        const uint32_t seg_lo = below ? 63u - (uint32_t)__builtin_clzll(below) : 0u;
        EnumStep st;
        st.owner = below ? mark[seg_lo] : (carry ? (uint32_t)__builtin_ctzll(carry) : 0u);
        st.active = c0 + lane < total;
        st.idx = c0 + lane - (uint32_t)__shfl((int)excl, (int)st.owner);
        const uint64_t above = starts & ~le;
        const uint32_t seg_hi = above ? (uint32_t)__builtin_ctzll(above) : 64u;
        st.seg = (~0ull << seg_lo) & (seg_hi == 64u ? ~0ull : ((1ull << seg_hi) - 1ull));
        st.head = st.active && lane == seg_lo;
        visit(st);
        wave_sync();
    }
}
VS_DEV uint32_t lanes_below(uint64_t m) {
    const uint32_t lane = __lane_id();
    return (uint32_t)__popcll(m & (lane == 0 ? 0ull : (~0ull >> (64 - lane))));
}

// sqrt(x) for x >= 0 from the reciprocal-square-root instruction and one
// Newton step: relative error below 1e-11 (the step squares the
// instruction's), a chord end within 1e-7 px for half-widths up to 1e4 px,
// far inside the ranges' margins (0.05 px inside, 0.5 px outside).  The
// correctly rounded sqrt took ~15 instructions per chord (C4's projection
// walks 3.3e7 box rows of four chords: 0.90 -> 0.82 ms).
VS_DEV double chord_sqrt(double x) {
    if (!(x > 0.0)) return 0.0;
    const double y = __builtin_amdgcn_rsq(x);
    const double yr = y * (1.5 - (0.5 * x) * (y * y));
    return x * yr;
}

// Ellipse chord at height dy (sigma = 0.5 (a dx^2 + c dy^2) + b dx dy <= P):
// [l, r], or false when the line misses it (`touch`: a line at the ellipse's
// top or bottom, where rounding may leave the discriminant just below 0,
// still gets its one point).
VS_DEV bool chord(double a, double b, double det, double inva, double two_a_p, double dy, double& l, double& r,
                  bool touch = false) {
    double disc = two_a_p - det * dy * dy;
    if (touch) disc = fmax(disc, 0.0);
    if (!(disc >= 0.0)) return false;
    const double s = chord_sqrt(disc);
    l = (-b * dy - s) * inva;
    r = (-b * dy + s) * inva;
    return true;
}

// Tiles [ia, ib) of row ty, within [lo, hi), whose corners (widened by
// BAND_IN) lie inside the ellipse sigma <= P (1 - 4e-3) - 1e-4; ia and ib are
// left alone when there are none.
VS_DEV void row_interior(float px, float py, S2 cf, double P, uint32_t ty, uint32_t lo, uint32_t hi, uint32_t& ia,
                         uint32_t& ib) {
    const double a = cf.c00, b = cf.c01, c = cf.c11;
    const double det = a * c - b * b, inva = 1.0 / a;
    const double mx_ = px, my_ = py;
    const double p_in = P * 0.996 - 1e-4;
    if (!(p_in > 0.0)) return;
    const double e0 = (double)(ty * TILE_W) - my_ - BAND_IN, e1 = e0 + (double)TILE_W + 2.0 * BAND_IN;
    double l0, r0, l1, r1;
    if (!chord(a, b, det, inva, 2.0 * a * p_in, e0, l0, r0) || !chord(a, b, det, inva, 2.0 * a * p_in, e1, l1, r1)) return;
    const double fi = ceil((mx_ + fmax(l0, l1) + BAND_IN) / TILE_W), fj = floor((mx_ + fmin(r0, r1) - BAND_IN) / TILE_W);
    const double ci = fmin(fmax(fi, (double)lo), (double)hi), cj = fmin(fmax(fj, (double)lo), (double)hi);
    if (ci < cj) { ia = (uint32_t)ci; ib = (uint32_t)cj; }
}

// The per-splat terms of the row ranges, formed once per splat and handed to
// the lanes that walk its rows: the outer ellipse sigma <= p_out (y extent ey,
// leftmost point at dy = kx) and the inner one sigma <= p_in (ey_in, kx_in;
// NaN when p_in <= 0: no certain tiles).
struct RangeK { double det, inva, two_a_pout, ey, kx, two_a_pin, ey_in, kx_in; };
VS_DEV RangeK range_consts(S2 cf, float power) {
    const double a = cf.c00, b = cf.c01, c = cf.c11, P = power;
    RangeK k;
    k.det = a * c - b * b;
    k.inva = 1.0 / a;
    const double p_out = P * 1.004 + 1e-4;
    const double ex = sqrt(2.0 * c * p_out / k.det);
    k.ey = sqrt(2.0 * a * p_out / k.det);
    k.two_a_pout = 2.0 * a * p_out;
    k.kx = b * ex / c;                  // -b ex / c is its exact negation
    const double p_in = P * 0.996 - 1e-4;
    k.two_a_pin = (p_in > 0.0) ? 2.0 * a * p_in : __builtin_nan("");   // NaN: no interior chord
    // both ellipses share their axes: the inner extents are the outer ones
    // scaled by sqrt(p_in / p_out)
    const double s_in = sqrt(p_in / p_out);
    k.ey_in = k.ey * s_in;
    k.kx_in = k.kx * s_in;
    return k;
}
VS_DEV RangeK shfl_k(const RangeK& k, uint32_t src) {
    const int s = (int)src;
    return RangeK{__shfl(k.det, s), __shfl(k.inva, s), __shfl(k.two_a_pout, s), __shfl(k.ey, s), __shfl(k.kx, s),
                  __shfl(k.two_a_pin, s), __shfl(k.ey_in, s), __shfl(k.kx_in, s)};
}

// Tile-x ranges of row ty of a splat's box: [oa, ob) may pass, [ia, ib) must
// (b = c01, k: the splat's range_consts).
VS_DEV void row_ranges_k(float px, float py, double b, const RangeK& k, uint4 box, uint32_t ty, uint32_t& oa,
                         uint32_t& ia, uint32_t& ib, uint32_t& ob) {
    const uint32_t x0 = box.x, x1 = box.y;
    oa = x0; ob = x1; ia = ib = x1;
    if (!box.w) return;
    const double mx_ = px, my_ = py;
    const double d0 = (double)(ty * TILE_W) - my_ - BAND_OUT, d1 = d0 + (double)TILE_W + 2.0 * BAND_OUT;
    const double lo = fmax(d0, -k.ey), hi = fmin(d1, k.ey);
    if (!(lo <= hi)) { oa = ob = x0; ia = ib = x0; return; }
    double l, r, t;
    chord(0.0, b, k.det, k.inva, k.two_a_pout, fmin(fmax(k.kx, lo), hi), l, t, true);
    chord(0.0, b, k.det, k.inva, k.two_a_pout, fmin(fmax(-k.kx, lo), hi), t, r, true);
    const double fo = floor((mx_ + l - BAND_OUT) / TILE_W), fe = floor((mx_ + r + BAND_OUT) / TILE_W) + 1.0;
    oa = (uint32_t)fmin(fmax(fo, (double)x0), (double)x1);
    ob = (uint32_t)fmin(fmax(fe, (double)oa), (double)x1);
    ia = ib = ob;
    // The certain range: tiles whose x span overlaps, by BAND_IN, the x extent
    // of the inner ellipse over the row band shrunk by BAND_IN.  The ellipse
    // meets the band in a convex set, so each such tile holds a point of the
    // band with sigma <= p_in, and the exact minimum of sigma over the tile
    // (which the StopThePop test evaluates) is no larger: the test passes with
    // the p_in margin (0.4 % of sigma + 1e-4, 0.05 px) to spare against its f32
    // rounding, as for a tile wholly inside.  The leftmost point of the set is
    // at dy = kx_in clamped to the band (the left chord end is convex in dy),
    // the rightmost at -kx_in.
    const double f0 = (double)(ty * TILE_W) - my_ + BAND_IN, f1 = f0 + (double)TILE_W - 2.0 * BAND_IN;
    const double lo_i = fmax(f0, -k.ey_in), hi_i = fmin(f1, k.ey_in);
    if (!(lo_i <= hi_i)) return;
    double li, ri;
    if (!chord(0.0, b, k.det, k.inva, k.two_a_pin, fmin(fmax(k.kx_in, lo_i), hi_i), li, t) ||
        !chord(0.0, b, k.det, k.inva, k.two_a_pin, fmin(fmax(-k.kx_in, lo_i), hi_i), t, ri))
        return;   // also for a NaN inner ellipse (p_in <= 0)
    const double fi = floor((mx_ + li + BAND_IN) / TILE_W), fj = ceil((mx_ + ri - BAND_IN) / TILE_W);
    const double ci = fmin(fmax(fi, (double)oa), (double)ob), cj = fmin(fmax(fj, (double)oa), (double)ob);
    if (ci < cj) { ia = (uint32_t)ci; ib = (uint32_t)cj; }
}

// Whether a conic admits the exact ranges (positive definite, |corr| <= sqrt(0.999)).
VS_DEV uint32_t ranges_ok(S2 c, float power) {
    const double a = c.c00, b = c.c01, cc = c.c11;
    return (a > 0.0 && cc > 0.0 && b * b <= 0.999 * a * cc && power >= 0.0f && finite(c) && finite(power)) ? 1u : 0u;
}

// The depth cutoff's per-tile tables (null cut: no cutoff).
struct CutFilter {
    const uint8_t* cut;       // [T] last depth bin the tile keeps
    const uint16_t* allow;    // [bh][CUT_BINS][bw + 1] tiles before x in row ty keeping bin b
};
// Depth bin of raw depth bits in [dmin, dmax]: equal spans of the bits, so
// about equal ratios of depth (monotone, as the depth order is).
VS_DEV uint32_t cut_bin(uint32_t dbits, uint32_t dmin, uint32_t dmax) {
    const uint64_t span = (uint64_t)(dmax - dmin) + 1ull;
    return (uint32_t)min(((uint64_t)(dbits - dmin) * CUT_BINS) / span, (uint64_t)(CUT_BINS - 1u));
}

// Walks the boxes of the wavefront (every lane calls it; nb == 0: no box).
// EMIT: writes each passing tile id (and the global id) into the splat's slot
// range [word0, word0 + count), at most `count` of them and below `capacity`;
// otherwise counts them.  On return acc[lane] holds the lane's tiles.
// FILTER: only tiles whose cutoff bin is at least the splat's depth bin
// (`bin`) count: interior runs by the row's prefix counts of such tiles (the
// k-th found by bisection when emitting), boundary tiles before their test.
template <bool EMIT, bool FILTER = false>
VS_DEV void walk_rows(RowLds& L, bool has, TileBox bb, float px, float py, S2 cf, float power, uint32_t base,
                      uint32_t gid, uint32_t cnt, uint32_t tile_bw, uint32_t* tiles, uint32_t* vals, uint32_t capacity,
                      CutFilter cutf = CutFilter{nullptr, nullptr}, uint32_t bin = 0u) {
    const uint32_t lane = __lane_id();
    L.geo[lane] = make_float4(px, py, cf.c00, cf.c01);
    L.geo2[lane] = make_float2(cf.c11, power);
    L.box[lane] = make_uint4(bb.x0, bb.x1, bb.y0, has ? ranges_ok(cf, power) : 0u);
    L.word[lane] = make_uint4(base, gid, cnt, bin);
    L.acc[lane] = 0u;
    const uint32_t rows = has ? bb.y1 - bb.y0 : 0u;
    const RangeK myk = range_consts(cf, power);
    wave_enum(L.mark, rows, [&](const EnumStep& rs) {
        // this lane's row: ranges, then a walk over the step's boundary tiles
        const uint32_t o = rs.owner;
        uint32_t oa = 0, ia = 0, ib = 0, ob = 0, ty = 0;
        const float4 g = L.geo[o];
        const RangeK ok = shfl_k(myk, o);   // every lane, before any branch
        const uint16_t* ar = nullptr;   // FILTER: the row's prefix counts of tiles keeping the splat's bin
        if (rs.active) {
            const uint4 bx = L.box[o];
            ty = bx.z + rs.idx;
            if (FILTER) ar = cutf.allow + ((size_t)ty * CUT_BINS + L.word[o].w) * (tile_bw + 1u);
            // a row of the box without such a tile is skipped whole
            if (!FILTER || ar[bx.y] != ar[bx.x]) row_ranges_k(g.x, g.y, (double)g.w, ok, bx, ty, oa, ia, ib, ob);
            if (FILTER && ar[ob] == ar[oa]) oa = ia = ib = ob;
        }
        uint32_t n_in = ib - ia;
        if (FILTER && rs.active && n_in) n_in = (uint32_t)ar[ib] - (uint32_t)ar[ia];
        uint32_t first_in = 0;
        if (rs.active && n_in) {
            if (EMIT) first_in = atomicAdd(&L.acc[o], n_in);
            else atomicAdd(&L.acc[o], n_in);
        }
        L.row[lane] = make_uint4(o, ty, oa, ia);
        L.row2[lane] = make_uint4(ib, ob, first_in, n_in);
        wave_sync();
        const uint32_t n_bd = rs.active ? (ia - oa) + (ob - ib) : 0u;
        wave_enum(L.mark2, n_bd, [&](const EnumStep& bs) {
            const uint4 rw = L.row[bs.owner];
            const uint4 rw2 = L.row2[bs.owner];
            const uint32_t left = rw.w - rw.z;
            const uint32_t tx = bs.idx < left ? rw.z + bs.idx : rw2.x + (bs.idx - left);
            const float4 sg = L.geo[rw.x];
            const float2 sg2 = L.geo2[rw.x];
            const bool kept = !FILTER || (bs.active && (uint32_t)cutf.cut[rw.y * tile_bw + tx] >= L.word[rw.x].w);
            const bool hit = bs.active && kept && will_contribute(tx, rw.y, sg.x, sg.y, S2{sg.z, sg.w, sg2.x}, sg2.y);
            const uint64_t hm = __ballot(hit);
            const uint32_t seg_hits = (uint32_t)__popcll(hm & bs.seg);
            if (!EMIT) {
                if (bs.head && seg_hits) atomicAdd(&L.acc[rw.x], seg_hits);
            } else {
                if (bs.head) L.tmp[lane] = seg_hits ? atomicAdd(&L.acc[rw.x], seg_hits) : 0u;
                wave_sync();
                if (hit) {
                    const uint32_t seg_lo = (uint32_t)__builtin_ctzll(bs.seg);
                    const uint32_t k = L.tmp[seg_lo] + lanes_below(hm & bs.seg);
                    const uint4 w = L.word[rw.x];
                    if (k < w.z && w.x + k < capacity) {
                        tiles[w.x + k] = tx + rw.y * tile_bw;
                        vals[w.x + k] = w.y;
                    }
                }
            }
        });
        if (EMIT) {
            wave_enum(L.mark2, rs.active ? n_in : 0u, [&](const EnumStep& is) {
                if (!is.active) return;
                const uint4 rw = L.row[is.owner];
                const uint4 rw2 = L.row2[is.owner];
                const uint4 w = L.word[rw.x];
                const uint32_t k = rw2.z + is.idx;
                uint32_t tx = rw.w + is.idx;
                if (FILTER && rw2.w != rw2.x - rw.w) {
                    // the idx-th kept tile of [ia, ib) (a run that keeps every
                    // tile needs no search): the first x with ar[x + 1] > ar[ia] + idx
                    const uint16_t* ar = cutf.allow + ((size_t)rw.y * CUT_BINS + w.w) * (tile_bw + 1u);
                    const uint32_t target = (uint32_t)ar[rw.w] + is.idx;
                    uint32_t lo = rw.w, hi = rw2.x - 1u;
                    while (lo < hi) {
                        const uint32_t mid = (lo + hi) >> 1;
                        if ((uint32_t)ar[mid + 1u] > target) hi = mid; else lo = mid + 1u;
                    }
                    tx = lo;
                }
                if (k < w.z && w.x + k < capacity) {
                    tiles[w.x + k] = tx + rw.y * tile_bw;
                    vals[w.x + k] = w.y;
                }
            });
        }
    });
}

VS_DEV uint32_t wave_sum(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o);
    return v;
}
VS_DEV uint32_t wave_min(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { const uint32_t w = __shfl_xor(v, o); v = w < v ? w : v; }
    return v;
}
VS_DEV uint32_t wave_max(uint32_t v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) { const uint32_t w = __shfl_xor(v, o); v = w > v ? w : v; }
    return v;
}

// One workgroup reduces the projection's block statistics: the 64-bit total of
// tile hits, the visible count, the depth-bit range, and the exclusive scan
// (in place) of the per-block counts of splats that hit at least one tile,
// which are the compaction offsets of those splats.
constexpr int FIN_BLOCK = 1024;
__global__ void __launch_bounds__(FIN_BLOCK) finalize_counts_kernel(uint32_t* __restrict__ stats, uint32_t nb,
                                                                   uint32_t* __restrict__ counters,
                                                                   uint32_t isect_capacity, uint32_t* host_copy) {
    __shared__ uint32_t s_w[FIN_BLOCK / 64];
    __shared__ uint32_t s_vis[FIN_BLOCK / 64], s_min[FIN_BLOCK / 64], s_max[FIN_BLOCK / 64];
    __shared__ unsigned long long s_hits[FIN_BLOCK / 64];
    const uint32_t lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const uint32_t* hits = stats + (size_t)BS_HITS * nb;
    const uint32_t* vis = stats + (size_t)BS_VISIBLE * nb;
    const uint32_t* dmin = stats + (size_t)BS_DMIN * nb;
    const uint32_t* dmax = stats + (size_t)BS_DMAX * nb;
    uint32_t* emit = stats + (size_t)BS_EMIT * nb;
    // Each thread takes a contiguous chunk of the blocks: one read of every
    // row (the chunk's loads in flight together), one block scan of the
    // chunks' emitter counts, then the chunk's offsets written from a second
    // (L2-resident) read of its counts.
    const uint32_t per = (nb + FIN_BLOCK - 1) / FIN_BLOCK;
    const uint32_t b0 = min(nb, threadIdx.x * per), b1 = min(nb, b0 + per);
    unsigned long long h_acc = 0;
    uint32_t v_acc = 0, mn_acc = 0xFFFFFFFFu, mx_acc = 0u, e_acc = 0;
#pragma unroll 4
    for (uint32_t i = b0; i < b1; ++i) {
        e_acc += emit[i];
        h_acc += hits[i];
        v_acc += vis[i];
        mn_acc = min(mn_acc, dmin[i]);
        mx_acc = max(mx_acc, dmax[i]);
    }
    uint32_t incl = e_acc;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t t = __shfl_up(incl, o);
        if ((int)lane >= o) incl += t;
    }
    if (lane == 63) s_w[wave] = incl;
    __syncthreads();
    uint32_t before = 0, carry = 0;
    for (uint32_t w = 0; w < FIN_BLOCK / 64; ++w) {
        if (w < wave) before += s_w[w];
        carry += s_w[w];
    }
    uint32_t run = before + incl - e_acc;
    for (uint32_t i = b0; i < b1; ++i) {
        const uint32_t x = emit[i];
        emit[i] = run;
        run += x;
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) h_acc += __shfl_xor(h_acc, o);
    const uint32_t wv = wave_sum(v_acc), wmn = wave_min(mn_acc), wmx = wave_max(mx_acc);
    if (lane == 0) { s_vis[wave] = wv; s_min[wave] = wmn; s_max[wave] = wmx; s_hits[wave] = h_acc; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t tv = 0, tmn = 0xFFFFFFFFu, tmx = 0u;
        unsigned long long th = 0;
        for (int w = 0; w < FIN_BLOCK / 64; ++w) {
            tv += s_vis[w]; tmn = min(tmn, s_min[w]); tmx = max(tmx, s_max[w]); th += s_hits[w];
        }
        uint32_t c[CNT_COUNT] = {};
        c[CNT_VISIBLE] = tv;
        c[CNT_DEPTH_MIN] = tmn;
        c[CNT_DEPTH_MAX] = tmx;
        c[CNT_EMITTERS] = carry;
        c[CNT_ISECT64] = (uint32_t)th;
        c[CNT_ISECT64 + 1] = (uint32_t)(th >> 32);
        c[CNT_BOUNDED] = th < (unsigned long long)isect_capacity ? (uint32_t)th : isect_capacity;
        for (int i = 0; i < CNT_COUNT; ++i) counters[i] = c[i];
        if (host_copy)
            for (int i = 0; i < CNT_COUNT; ++i) host_copy[i] = c[i];
    }
}

// A splat's SH row as f32: f32 rows in float4 loads where the row size
// allows; f16 rows (raw binary16) in 16- or 8-byte loads where it allows.
template <int DEG>
VS_DEV void load_sh_row(const uint16_t* __restrict__ sh, uint32_t g, float* c) {
    constexpr int N = sh_count<DEG>() * 3;
    const uint16_t* row = sh + (size_t)g * N;
    if constexpr (N % 8 == 0) {
        const uint4* r = reinterpret_cast<const uint4*>(row);
#pragma unroll
        for (int i = 0; i < N / 8; ++i) {
            const uint4 q = r[i];
            const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                c[8 * i + 2 * j] = h2f((uint16_t)(w[j] & 0xFFFFu));
                c[8 * i + 2 * j + 1] = h2f((uint16_t)(w[j] >> 16));
            }
        }
    } else if constexpr (N % 4 == 0) {
        const uint2* r = reinterpret_cast<const uint2*>(row);
#pragma unroll
        for (int i = 0; i < N / 4; ++i) {
            const uint2 q = r[i];
            c[4 * i] = h2f((uint16_t)(q.x & 0xFFFFu)); c[4 * i + 1] = h2f((uint16_t)(q.x >> 16));
            c[4 * i + 2] = h2f((uint16_t)(q.y & 0xFFFFu)); c[4 * i + 3] = h2f((uint16_t)(q.y >> 16));
        }
    } else {
#pragma unroll
        for (int i = 0; i < N; ++i) c[i] = h2f(row[i]);
    }
}
template <int DEG>
VS_DEV void load_sh_row(const float* __restrict__ sh, uint32_t g, float* c) {
    constexpr int K = sh_count<DEG>();
    const float* row = sh + (size_t)g * (K * 3);
    if constexpr ((K * 3) % 4 == 0) {
        const float4* r4 = reinterpret_cast<const float4*>(row);
#pragma unroll
        for (int i = 0; i < K * 3 / 4; ++i) {
            const float4 q = r4[i];
            c[4 * i] = q.x; c[4 * i + 1] = q.y; c[4 * i + 2] = q.z; c[4 * i + 3] = q.w;
        }
    } else {
#pragma unroll
        for (int i = 0; i < K * 3; ++i) c[i] = row[i];
    }
}

template <int DEG, typename SHT>
VS_DEV F3 load_color(const SHT* __restrict__ sh, uint32_t g, F3 mean, const vs_camera& u) {
    float c[sh_count<DEG>() * 3];
    load_sh_row<DEG>(sh, g, c);
    // kernels/project_visible.rs:25-61
    const F3 v = normalize(mean - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]});
    const F3 raw = sh_color<DEG>(c, v);
    const float r = raw.x + 0.5f, gg = raw.y + 0.5f, b = raw.z + 0.5f;
    return F3{clampf(finite(r) ? r : 0.0f, -100.0f, 100.0f),
              clampf(finite(gg) ? gg : 0.0f, -100.0f, 100.0f),
              clampf(finite(b) ? b : 0.0f, -100.0f, 100.0f)};
}

template <int DEG, int MODEL, bool GEOM, typename SHT>
__global__ void __launch_bounds__(PROJ_BLOCK) project_kernel(ProjectArgs a) {
    const vs_camera& u = a.cam;
    const uint32_t g = blockIdx.x * PROJ_BLOCK + threadIdx.x;
    bool visible = false;
    float px = 0.0f, py = 0.0f, power = 0.0f, radius = 0.0f, opac_out = 0.0f;
    S2 conic{0.0f, 0.0f, 0.0f};
    TileBox bb{0, 0, 0, 0};
    uint32_t dbits = 0;
    F3 fscl{0.0f, 0.0f, 0.0f};      // floored scale (the geometry normal picks its smallest axis)
    if (g < a.num_splats) {
        const float2* t2 = reinterpret_cast<const float2*>(a.transforms + (size_t)g * 10);
        const float2 t01 = t2[0], t23 = t2[1], t45 = t2[2], t67 = t2[3], t89 = t2[4];
        const float raw_op = a.raw_opac[g];
        // kernels/project_forward.rs:62-194, culls in the reference's order.
        do {
            const F3 mean{t01.x, t01.y, t23.x};
            const F3 mc = world_to_cam(mean, u);
            if (!(finite(mc) && mc.z <= 1.0e10f)) break;
            if constexpr (MODEL == VS_CAMERA_PINHOLE || MODEL == SURFEL_MODEL) {
                if (mc.z < 0.01f) break;
            } else {
                const float r = __builtin_sqrtf(mc.x * mc.x + mc.y * mc.y);
                if (atan2f_c(r, mc.z) > u.half_max_render_fov) break;
            }
            const float lso = a.log_scale_offset;
            const F3 scl{expf_c(t67.y + lso), expf_c(t89.x + lso), expf_c(t89.y + lso)};
            if (!finite(scl)) break;
            const Qt qu{t23.y, t45.x, t45.y, t67.x};
            const float qn = dot(qu, qu);
            if (!(qn >= 1.0e-6f && finite(qn))) break;
            if (!finite(raw_op)) break;
            const Qt q = normalize(qu);
            const ScaleFloor fl = apply_scale_floor(scl, sigmoid(raw_op), a.min_scale, g);
            opac_out = fl.opac;
            float opac;
            SurfelProj sp{};
            if constexpr (MODEL == SURFEL_MODEL) {
                // project_forward.rs:128-147: bin by the ellipse covering the
                // cutoff footprint and the low-pass disk; no 2-D blur compensation.
                opac = fl.opac;
                if (!(opac >= 1.0f / 255.0f)) break;
                power = logf_c(opac * 255.0f);
                sp = surfel_project(fl.scale, q, mc, u, power);
                if (!sp.valid) break;
                conic = sp.bin_conic;
                px = sp.bin_x;
                py = sp.bin_y;
            } else {
                float filter_comp;
                const S2 cov = compensate_cov2d(cov2d_raw<MODEL>(fl.scale, q, mc, u), a.mip != 0u, filter_comp);
                opac = fl.opac * filter_comp;
                fscl = fl.scale;
                if (!finite(cov)) break;
                project_point<MODEL>(mc, u, px, py);
                if (!(opac >= 1.0f / 255.0f)) break;
                power = logf_c(opac * 255.0f);
                conic = inverse(cov);
            }
            float ex, ey;
            bbox_extent(conic, power, ex, ey);
            if (!(ex >= 0.0f && ey >= 0.0f)) break;
            const float wf = (float)a.img_w, hf = (float)a.img_h;
            if (!(px + ex > 0.0f && px - ex < wf && py + ey > 0.0f && py - ey < hf)) break;
            bb = tile_box(px, py, ex, ey, a.tile_bw, a.tile_bh);
            radius = mx(ex / wf, ey / hf);
            dbits = as_u(mc.z);
            visible = true;
            // Projected row (kernels/project_visible.rs:150-173), written at the global id.
            F3 col;
            if constexpr (DEG == NEURAL_DEG) {
                // kernels/project_visible.rs:25-61, neural branch: the same scrub and clamp
                const F3 vd = normalize(mean - F3{u.cam_pos[0], u.cam_pos[1], u.cam_pos[2]});
                const F3 c3 = neural_color(static_cast<const SHT*>(a.sh) + (size_t)g * NEURAL_ROW, a.decoder, vd,
                                           a.sh_degree);
                col = F3{clampf(finite(c3.x) ? c3.x : 0.0f, -100.0f, 100.0f),
                         clampf(finite(c3.y) ? c3.y : 0.0f, -100.0f, 100.0f),
                         clampf(finite(c3.z) ? c3.z : 0.0f, -100.0f, 100.0f)};
            } else {
                col = load_color<DEG>(static_cast<const SHT*>(a.sh), g, mean, u);
            }
            float4* row = a.proj + (size_t)g * PROJ_Q;
            row[0] = make_float4(px, py, conic.c00, conic.c01);
            row[1] = make_float4(conic.c11, opac, col.x, col.y);
            row[2] = make_float4(col.z, power, 0.0f, 0.0f);
            if constexpr (MODEL == SURFEL_MODEL) {
                // project_visible.rs:231-273: M rows, the low-pass centre (the
                // pinhole projection of the centre) and the camera-facing normal
                float cx_, cy_;
                project_point<VS_CAMERA_PINHOLE>(mc, u, cx_, cy_);
                const F3 nrm = surfel_normal(q, mc, u);
                float4* o = a.proj_surf + (size_t)g * 4;
                o[0] = make_float4(sp.r0.x, sp.r0.y, sp.r0.z, sp.r1.x);
                o[1] = make_float4(sp.r1.y, sp.r1.z, sp.r2.x, sp.r2.y);
                o[2] = make_float4(sp.r2.z, cx_, cy_, nrm.x);
                // the raster kernels' footprint bound: sigma beyond it leaves alpha
                // below the lowest cutoff (ALPHA_MID - ALPHA_BAND / 2) by a factor e^-1e-3
                const float smax = logf_c(opac / (ALPHA_MID - 0.5f * ALPHA_BAND)) + 1.0e-3f;
                o[3] = make_float4(nrm.y, nrm.z, smax, 0.0f);
            }
            if constexpr (GEOM) {
                // kernels/project_visible.rs:271-289
                const M3 rot = mul(view_rot(u), to_mat3(q));
                const bool x_min = fscl.x <= fscl.y && fscl.x <= fscl.z;
                const bool y_min = !x_min && fscl.y <= fscl.z;
                const F3 axis = x_min ? rot.c0 : (y_min ? rot.c1 : rot.c2);
                const float flip = (dot(axis, mc) > 0.0f) ? -1.0f : 1.0f;
                a.proj_aux[g] = make_float4(mc.z, axis.x * flip, axis.y * flip, axis.z * flip);
            }
        } while (false);
    }

    // Tile counting (kernels/helpers.rs:253-273): the StopThePop test on every
    // tile of the box, in a load-balanced walk over the wavefront's boxes.
    __shared__ RowLds s_walk[PROJ_BLOCK / 64];
    const uint32_t lane = lane_id();
    RowLds& L = s_walk[threadIdx.x / 64];
    uint32_t hits = 0u;
    if (__ballot(visible) != 0ull) {   // a wavefront without a visible splat skips the walk
        walk_rows<false>(L, visible, bb, px, py, conic, power, 0u, 0u, 0u, a.tile_bw, nullptr, nullptr, 0u);
        hits = L.acc[lane];
    }

    if (g < a.num_splats) {
        a.opacities[g] = opac_out;
        a.max_radius[g] = radius;
        a.counts[g] = hits;
        a.depth_bits[g] = dbits;
        a.compact[g] = visible ? g + 1u : 0u;
        if (a.visible) a.visible[g] = 0.0f;
    }
    // every tile's range starts as (0xFFFFFFFF, 0): the tile sort's range pass
    // lowers starts and raises ends
    for (uint32_t t = g; t < a.num_tiles; t += gridDim.x * PROJ_BLOCK)
        reinterpret_cast<uint2*>(a.ranges)[t] = make_uint2(0xFFFFFFFFu, 0u);

    // Block statistics, reduced by finalize_counts_kernel (no global atomics:
    // a same-address atomic from every wave serialises across the XCDs).
    __shared__ uint32_t s_sum[PROJ_BLOCK / 64], s_vis[PROJ_BLOCK / 64], s_min[PROJ_BLOCK / 64], s_max[PROJ_BLOCK / 64];
    __shared__ uint32_t s_emit[PROJ_BLOCK / 64];
    const uint32_t wsum = wave_sum(hits);
    const uint32_t wvis = (uint32_t)__popcll(__ballot(visible));
    const uint32_t wemit = (uint32_t)__popcll(__ballot(hits > 0u));
    const uint32_t wmin = wave_min(visible ? dbits : 0xFFFFFFFFu);
    const uint32_t wmax = wave_max(visible ? dbits : 0u);
    const uint32_t wave = threadIdx.x / 64;
    if (lane == 0) { s_sum[wave] = wsum; s_vis[wave] = wvis; s_min[wave] = wmin; s_max[wave] = wmax; s_emit[wave] = wemit; }
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t bs = 0, bv = 0, bmn = 0xFFFFFFFFu, bmx = 0u, be = 0;
#pragma unroll
        for (int w = 0; w < PROJ_BLOCK / 64; ++w) {
            bs += s_sum[w]; bv += s_vis[w]; bmn = min(bmn, s_min[w]); bmx = max(bmx, s_max[w]); be += s_emit[w];
        }
        const uint32_t nb = gridDim.x;
        a.block_stats[BS_HITS * nb + blockIdx.x] = bs;
        a.block_stats[BS_VISIBLE * nb + blockIdx.x] = bv;
        a.block_stats[BS_DMIN * nb + blockIdx.x] = bmn;
        a.block_stats[BS_DMAX * nb + blockIdx.x] = bmx;
        a.block_stats[BS_EMIT * nb + blockIdx.x] = be;
    }
}

// Compaction of the splats that hit a tile, in global-id order, as (depth
// bits - minimum, global id) pairs: the input of the depth sort (the
// reference's depth argsort of render.rs:689-694, keyed on raw f32 bits).
// Blocks match the projection's, whose scanned emitter counts give the base.
__global__ void __launch_bounds__(PROJ_BLOCK) compact_kernel(CompactArgs a) {
    const uint32_t g = blockIdx.x * PROJ_BLOCK + threadIdx.x;
    const uint32_t lane = lane_id(), wave = threadIdx.x / 64;
    const bool e = g < a.num_splats && a.counts[g] > 0u;
    const uint64_t m = __ballot(e);
    const uint64_t lt_mask = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    __shared__ uint32_t s_w[PROJ_BLOCK / 64];
    if (lane == 0) s_w[wave] = (uint32_t)__popcll(m);
    __syncthreads();
    uint32_t base = a.block_offsets[blockIdx.x];
    for (uint32_t w = 0; w < wave; ++w) base += s_w[w];
    if (e) {
        const uint32_t o = base + (uint32_t)__popcll(m & lt_mask);
        a.keys[o] = a.depth_bits[g] - a.counters[CNT_DEPTH_MIN];
        a.vals[o] = g;
    }
    for (uint64_t i = g; i < a.zero_words; i += (uint64_t)gridDim.x * PROJ_BLOCK) a.zero[i] = 0u;
    for (uint64_t i = g; i < a.zero2_words; i += (uint64_t)gridDim.x * PROJ_BLOCK) a.zero2[i] = 0u;
}

// Emission (kernels/map_gaussians.rs:23-174): a splat with hits owns the
// slots [base, base + count), which the scan in depth order assigned, and
// writes there the ids of the tiles that pass the tile test, in row-major box
// order.  One launch, two kinds of blocks:
//  * the first emit_big_blocks(N) blocks walk the splats of more than
//    EMIT_SMALL_LIST slots, one lane per splat in global-id order, where long
//    lists are spread evenly over the wavefronts (in depth order the nearest,
//    largest ones would share the first wavefronts); their slot bases come
//    from the scan's copy by global id, which it writes for them alone;
//  * the rest walk the other splats in depth order, one lane per emitter:
//    neighbouring lanes own neighbouring slot ranges, so a wavefront's stores
//    fill one contiguous stretch of the list.
// Both kinds know a splat's count before reading its row, so each reads only
// the rows it emits.  If the recomputed test finds fewer tiles than the
// projection counted, the rest of a splat's slots get the sentinel tile id T,
// which sorts last and owns no range.
VS_DEV uint32_t emit_big_blocks(uint32_t n) { return (n + PROJ_BLOCK - 1) / PROJ_BLOCK; }

template <bool FILTER>
__global__ void __launch_bounds__(PROJ_BLOCK) emit_kernel(EmitArgs a) {
    const uint32_t lane = lane_id();
    const uint32_t big_blocks = emit_big_blocks(a.num_splats);
    const bool big = blockIdx.x < big_blocks;
    uint32_t g = 0xFFFFFFFFu, base = 0u, cnt = 0u;
    if (big) {
        g = blockIdx.x * PROJ_BLOCK + threadIdx.x;
        cnt = (g < a.num_splats) ? a.counts[g] : 0u;
        if (cnt <= EMIT_SMALL_LIST) cnt = 0u;         // the depth-order blocks emit it
    } else {
        const uint32_t j = (blockIdx.x - big_blocks) * PROJ_BLOCK + threadIdx.x;
        const uint32_t m = a.m_dev ? min(*a.m_dev, a.num_emitters) : a.num_emitters;
        if (j < m) {
            g = a.order[j];
            base = a.slot_base[j];
            // the count from the slot bases in depth order (slot_base[m] is the
            // total) rather than a gather from the counts in id order
            cnt = (g < a.num_splats) ? a.slot_base[j + 1] - base : 0u;
            if (cnt > EMIT_SMALL_LIST) cnt = 0u;      // the global-id blocks emit it
        }
    }
    float px = 0.0f, py = 0.0f, power = 0.0f;
    S2 conic{0.0f, 0.0f, 0.0f};
    TileBox bb{0, 0, 0, 0};
    uint32_t bin = 0u;
    if (cnt > 0) {
        // Recompute the box from the projected row as kernels/map_gaussians.rs:61-66 does
        // (power = logf(255 opacity) as the projection computed it).
        const float4* row = a.proj + (size_t)g * PROJ_Q;
        const float4 pa = row[0];
        const float c11 = row[1].x;
        power = row[2].y;
        px = pa.x; py = pa.y;
        conic = S2{pa.z, pa.w, c11};
        float ex, ey;
        bbox_extent(conic, power, ex, ey);
        bb = tile_box(px, py, ex, ey, a.tile_bw, a.tile_bh);
        if (FILTER) bin = cut_bin(a.depth_bits[g], a.counters[CNT_DEPTH_MIN], a.counters[CNT_DEPTH_MAX]);
    }
    if (big && cnt > 0) base = a.slot_base_g[g];
    __shared__ RowLds s_walk[PROJ_BLOCK / 64];
    RowLds& L = s_walk[threadIdx.x / 64];
    // a splat's count bounds its slots; slots past the arena are dropped.  A
    // wavefront with nothing to emit (most of the global-id blocks' ones)
    // skips the walk and its per-lane setup (the walk is wavefront-local).
    uint32_t emitted = 0u;
    if (__ballot(cnt > 0) != 0ull) {
        walk_rows<true, FILTER>(L, cnt > 0, bb, px, py, conic, power, base, g, cnt, a.tile_bw, a.tiles, a.vals,
                                a.capacity, CutFilter{a.cut, a.allow}, bin);
        emitted = L.acc[lane];
    }
    const uint32_t sentinel = a.tile_bw * a.tile_bh;
    for (uint32_t k = emitted; k < cnt && base + k < a.capacity; ++k) {
        a.tiles[base + k] = sentinel;
        a.vals[base + k] = g;
    }
    for (uint64_t i = (uint64_t)blockIdx.x * PROJ_BLOCK + threadIdx.x; i < a.zero_words; i += (uint64_t)gridDim.x * PROJ_BLOCK)
        a.zero[i] = 0u;
    // the list's length: the last emitter's slot range ends it
    if (a.listed && blockIdx.x == 0 && threadIdx.x == 0) {
        const uint32_t m = a.m_dev ? min(*a.m_dev, a.num_emitters) : a.num_emitters;
        *a.listed = m ? a.slot_base[m] : 0u;
    }
}

// ---- depth cutoff ---------------------------------------------------------------
// A splat's alpha at a pixel is min(ALPHA_CAP, opac G) with G = exp(-sigma).
// Inside its core ellipse sigma <= ln(opac / a), a = CUT_LEVEL min(opac,
// ALPHA_CAP), every pixel of a tile that row_interior places inside (0.4 %
// of sigma and 0.05 px to spare against the f32 evaluation) gets alpha >= a,
// and a >= CUT_MIN_ALPHA lies above the cutoff band, so a pixel that still
// runs blends the splat with (1 - alpha) <= (1 - a).  Such a tile lists the
// splat (its core lies inside the footprint the tile test passes).  The
// fixed-point masses floor(-ln(1 - a) CUT_SCALE 0.999) of the cores covering a tile, summed
// over the depth bins up to b, bound -ln T at every pixel after the tile's
// splats of bins <= b from below; once they reach CUT_NEED, ln(1 / T_STOP)
// + 0.25 nats (the margin covers the f32 rounding of T over two million
// blends), every pixel has stopped by the end of bin b, and splats of later
// bins are never evaluated there.  The rasterised image, the ranges a
// forward consumes and everything downstream are those of the full list.
constexpr float CUT_LEVEL = 0.5f;
constexpr float CUT_MIN_ALPHA = 0.01f;
constexpr uint32_t CUT_NEED = 38750;   // ceil((ln(1e4) + 0.25) * CUT_SCALE)

// Per splat with tiles: the mass of its core added to the difference rows of
// its depth bin, +m at the first interior tile, -m past the last (u32
// arithmetic wraps; the prefix sums recover the masses; the row's entry bw
// is never read).  A core narrower than a tile covers none.
//
// Two passes.  The front one adds the splats of bins < CUT_FRONT; a tile
// whose masses over those bins reach CUT_NEED has its cutoff bin among them
// (cut_pending_kernel marks the others pending).  The back one adds the
// splats of later bins whose box holds a pending tile: a box without one
// lies over tiles whose cutoff bins all precede the splat's bin, where its
// mass would only raise bins past the cutoff, which decide nothing.  The
// cutoff bins are those of every mass added (a heavy-tailed view 2560 x 1440
// has every cutoff bin below 8 while all but 0.5 % of 2.7 M cores lie behind).
template <bool BACK>
__global__ void __launch_bounds__(PROJ_BLOCK) cut_mass_kernel(CutArgs a) {
    const uint32_t g = blockIdx.x * PROJ_BLOCK + threadIdx.x;
    const uint32_t lane = lane_id();
    if (BACK && *a.pend_total == 0u) return;   // every cutoff bin lies among the front bins
    if (!BACK && g == 0u) *a.pend_total = 0u;   // cut_pending_kernel sums it next
    bool has = g < a.num_splats && a.counts[g] > 0u;
    float px = 0.0f, py = 0.0f, pc = 0.0f;
    S2 cf{0.0f, 0.0f, 0.0f};
    uint32_t m = 0u, bin = 0u;
    TileBox bb{0, 0, 0, 0};
    if (has) {
        bin = cut_bin(a.depth_bits[g], a.counters[CNT_DEPTH_MIN], a.counters[CNT_DEPTH_MAX]);
        has = BACK ? bin >= CUT_FRONT : bin < CUT_FRONT;
    }
    if (has) {
        const float4 pa = a.proj[(size_t)g * PROJ_Q], pb = a.proj[(size_t)g * PROJ_Q + 1];
        px = pa.x; py = pa.y;
        cf = S2{pa.z, pa.w, pb.x};
        const float opac = pb.y, ac = CUT_LEVEL * __builtin_fminf(opac, ALPHA_CAP);
        pc = logf_c(opac / ac);
        const float fm = floorf(-logf_c(1.0f - ac) * (CUT_SCALE * 0.999f));
        has = ac >= CUT_MIN_ALPHA && pc > 0.0f && ranges_ok(cf, pc) && fm >= 1.0f && fm < 1.0e6f;
        if (has) {
            m = (uint32_t)fm;
            float ex, ey;
            bbox_extent(cf, pc, ex, ey);
            has = ex >= 0.5f * TILE_W && ey >= 0.5f * TILE_W;
            bb = tile_box(px, py, ex, ey, a.tile_bw, a.tile_bh);
        }
    }
    if (BACK && has) {
        // summed over every row of the box: with an exit at the first pending
        // row the loop's flag came out of the last iteration's compare, which
        // clears it for lanes that left earlier
        const size_t w1 = (size_t)a.tile_bw + 1u;
        const uint32_t* p = a.pend + (size_t)bb.y0 * w1;
        uint32_t k = 0u;
        for (uint32_t y = bb.y0; y < bb.y1; ++y, p += w1) k += p[bb.x1] - p[bb.x0];
        has = k > 0u;
    }
    __shared__ RowLds s_walk[PROJ_BLOCK / 64];
    RowLds& L = s_walk[threadIdx.x / 64];
    L.geo[lane] = make_float4(px, py, cf.c00, cf.c01);
    L.geo2[lane] = make_float2(cf.c11, pc);
    L.box[lane] = make_uint4(bb.x0, bb.x1, bb.y0, 0u);
    L.word[lane] = make_uint4(m, bin, 0u, 0u);
    const uint32_t rows = has ? bb.y1 - bb.y0 : 0u;
    wave_enum(L.mark, rows, [&](const EnumStep& rs) {
        if (!rs.active) return;
        const uint32_t o = rs.owner;
        const float4 g4 = L.geo[o];
        const float2 g2 = L.geo2[o];
        const uint4 bx = L.box[o];
        const uint4 w = L.word[o];
        const uint32_t ty = bx.z + rs.idx;
        uint32_t ia = bx.y, ib = bx.y;
        row_interior(g4.x, g4.y, S2{g4.z, g4.w, g2.x}, g2.y, ty, bx.x, bx.y, ia, ib);
        if (ia < ib) {
            uint32_t* row = a.mass + ((size_t)ty * CUT_BINS + w.y) * (a.tile_bw + 1u);
            atomicAdd(&row[ia], w.x);
            if (ib < a.tile_bw) atomicAdd(&row[ib], 0u - w.x);
        }
    });
}

// After the front pass, one wavefront per tile row: each tile's masses over
// the front bins (prefix sums of their difference rows, which stay as they
// are) and
// pend[ty][x] = the row's tiles left of x where they stay below CUT_NEED
// (pend[ty][bw]: all of them).
constexpr int CUT_PEND_BLOCK = 64;
__global__ void __launch_bounds__(CUT_PEND_BLOCK) cut_pending_kernel(CutArgs a) {
    const uint32_t ty = blockIdx.x, bw = a.tile_bw, lane = lane_id();
    const size_t w1 = (size_t)bw + 1u;
    const uint32_t* mrow = a.mass + (size_t)ty * CUT_BINS * w1;
    uint32_t* p = a.pend + (size_t)ty * w1;
    uint32_t carry[CUT_FRONT];
#pragma unroll
    for (uint32_t b = 0; b < CUT_FRONT; ++b) carry[b] = 0u;
    uint32_t pc = 0u;
    for (uint32_t x0 = 0; x0 < bw; x0 += 64) {
        const uint32_t x = x0 + lane;
        uint32_t v[CUT_FRONT];
#pragma unroll
        for (uint32_t b = 0; b < CUT_FRONT; ++b) v[b] = x < bw ? mrow[b * w1 + x] : 0u;
        uint64_t cum = 0;
#pragma unroll
        for (uint32_t b = 0; b < CUT_FRONT; ++b) {
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(v[b], o);
                if ((int)lane >= o) v[b] += t;
            }
            cum += v[b] + carry[b];
            carry[b] += (uint32_t)__shfl((int)v[b], 63);
        }
        const uint32_t k = (x < bw && cum < CUT_NEED) ? 1u : 0u;
        uint32_t c = k;
#pragma unroll
        for (int o = 1; o < 64; o <<= 1) {
            const uint32_t t = __shfl_up(c, o);
            if ((int)lane >= o) c += t;
        }
        if (x < bw) p[x] = pc + c - k;
        pc += (uint32_t)__shfl((int)c, 63);
    }
    if (lane == 0) {
        p[bw] = pc;
        if (pc) atomicAdd(a.pend_total, pc);
    }
}

// One workgroup per tile row: the masses per (bin, tile) by prefix sums of
// the differences (in place), each tile's cutoff bin (the first whose
// cumulative mass reaches CUT_NEED; the last bin when none does), and per
// bin the prefix counts of the row's tiles that keep it.
constexpr int CUT_ROW_BLOCK = 256;
__global__ void __launch_bounds__(CUT_ROW_BLOCK) cut_rows_kernel(CutArgs a) {
    __shared__ uint8_t s_cut[CUT_MAX_BW];
    const uint32_t ty = blockIdx.x, bw = a.tile_bw, lane = lane_id(), wave = threadIdx.x / 64;
    const size_t w1 = (size_t)bw + 1u;
    uint32_t* mrow = a.mass + (size_t)ty * CUT_BINS * w1;
    for (uint32_t b = wave; b < CUT_BINS; b += CUT_ROW_BLOCK / 64) {
        uint32_t* r = mrow + b * w1;
        uint32_t carry = 0u;
        for (uint32_t x0 = 0; x0 < bw; x0 += 64) {
            const uint32_t x = x0 + lane;
            uint32_t v = x < bw ? r[x] : 0u;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(v, o);
                if ((int)lane >= o) v += t;
            }
            if (x < bw) r[x] = v + carry;
            carry += (uint32_t)__shfl((int)v, 63);
        }
    }
    __syncthreads();
    for (uint32_t x = threadIdx.x; x < bw; x += CUT_ROW_BLOCK) {
        uint64_t cum = 0;
        uint32_t c = CUT_BINS - 1u;
        for (uint32_t b = 0; b < CUT_BINS; ++b) {
            cum += mrow[b * w1 + x];
            if (cum >= CUT_NEED) { c = b; break; }
        }
        s_cut[x] = (uint8_t)c;
        a.cut[(size_t)ty * bw + x] = (uint8_t)c;
    }
    __syncthreads();
    for (uint32_t b = wave; b < CUT_BINS; b += CUT_ROW_BLOCK / 64) {
        uint16_t* r = a.allow + ((size_t)ty * CUT_BINS + b) * w1;
        uint32_t carry = 0u;
        for (uint32_t x0 = 0; x0 < bw; x0 += 64) {
            const uint32_t x = x0 + lane;
            const uint32_t k = (x < bw && (uint32_t)s_cut[x] >= b) ? 1u : 0u;
            uint32_t v = k;
#pragma unroll
            for (int o = 1; o < 64; o <<= 1) {
                const uint32_t t = __shfl_up(v, o);
                if ((int)lane >= o) v += t;
            }
            if (x < bw) r[x] = (uint16_t)(carry + v - k);
            carry += (uint32_t)__shfl((int)v, 63);
        }
        if (lane == 0) r[bw] = (uint16_t)carry;
    }
}

// The kept-tile prefix counts summed over rows: sat[ty][b][x] = the tiles of
// rows 0..ty left of column x that keep bin b.  One thread per (bin, column)
// runs down the rows.
constexpr int CUT_SAT_BLOCK = 256;
__global__ void __launch_bounds__(CUT_SAT_BLOCK) cut_sat_kernel(CutArgs a) {
    const uint32_t w1 = a.tile_bw + 1u;
    const uint32_t i = blockIdx.x * CUT_SAT_BLOCK + threadIdx.x;
    if (i >= CUT_BINS * w1) return;
    const size_t stride = (size_t)CUT_BINS * w1;
    const uint16_t* __restrict__ src = a.allow + i;   // (bin, column) i of row 0: [b * w1 + x]
    uint32_t* __restrict__ dst = a.sat + i;
    uint32_t sum = 0u;
#pragma unroll 8
    for (uint32_t y = 0; y < a.tile_bh; ++y) {
        sum += src[y * stride];
        dst[y * stride] = sum;
    }
}

// Tiles of the box [x0, x1) x [y0, y1) that keep bin b (the box is not empty).
VS_DEV uint32_t box_keeps(const uint32_t* sat, uint32_t tile_bw, TileBox bb, uint32_t b) {
    const size_t w1 = (size_t)tile_bw + 1u;
    const uint32_t* hi = sat + ((size_t)(bb.y1 - 1u) * CUT_BINS + b) * w1;
    uint32_t k = hi[bb.x1] - hi[bb.x0];
    if (bb.y0 > 0u) {
        const uint32_t* lo = sat + ((size_t)(bb.y0 - 1u) * CUT_BINS + b) * w1;
        k -= lo[bb.x1] - lo[bb.x0];
    }
    return k;
}

// Per splat with tiles: the tiles it keeps under the cutoff (the emission's
// walk).  A splat whose box holds no tile keeping its depth bin (at C4 all
// but a few thousand of the listed splats) keeps none, without a walk.
__global__ void __launch_bounds__(PROJ_BLOCK) count_kept_kernel(EmitArgs a) {
    const uint32_t g = blockIdx.x * PROJ_BLOCK + threadIdx.x;
    const uint32_t lane = lane_id();
    const uint32_t cnt = (g < a.num_splats) ? a.counts[g] : 0u;
    float px = 0.0f, py = 0.0f, power = 0.0f;
    S2 conic{0.0f, 0.0f, 0.0f};
    TileBox bb{0, 0, 0, 0};
    uint32_t bin = 0u;
    bool has = false;
    if (cnt > 0) {
        bin = cut_bin(a.depth_bits[g], a.counters[CNT_DEPTH_MIN], a.counters[CNT_DEPTH_MAX]);
        // the image's tiles keeping the bin (the summed table's last row, past
        // its last column): none, and the projected row is never read
        const size_t w1 = (size_t)a.tile_bw + 1u;
        has = a.sat[((size_t)(a.tile_bh - 1u) * CUT_BINS + bin) * w1 + a.tile_bw] > 0u;
    }
    if (has) {
        const float4* row = a.proj + (size_t)g * PROJ_Q;
        const float4 pa = row[0];
        px = pa.x; py = pa.y;
        conic = S2{pa.z, pa.w, row[1].x};
        power = row[2].y;
        float ex, ey;
        bbox_extent(conic, power, ex, ey);
        bb = tile_box(px, py, ex, ey, a.tile_bw, a.tile_bh);
        has = bb.x1 > bb.x0 && bb.y1 > bb.y0 && box_keeps(a.sat, a.tile_bw, bb, bin) > 0u;
    }
    uint32_t kept = 0u;
    if (__ballot(has) != 0ull) {   // a wavefront with nothing to walk skips the walk
        __shared__ RowLds s_walk[PROJ_BLOCK / 64];
        RowLds& L = s_walk[threadIdx.x / 64];
        walk_rows<false, true>(L, has, bb, px, py, conic, power, 0u, 0u, 0u, a.tile_bw, nullptr, nullptr, 0u,
                               CutFilter{a.cut, a.allow}, bin);
        kept = L.acc[lane];
    }
    if (g < a.num_splats) a.counts_out[g] = kept;
    // the block's splats that keep a pair: the compaction takes them alone
    __shared__ uint32_t s_k[PROJ_BLOCK / 64];
    const uint64_t km = __ballot(kept > 0u);
    if (lane == 0) s_k[threadIdx.x / 64] = (uint32_t)__popcll(km);
    __syncthreads();
    if (threadIdx.x == 0) {
        uint32_t t = 0;
#pragma unroll
        for (int w = 0; w < PROJ_BLOCK / 64; ++w) t += s_k[w];
        a.kept_blocks[blockIdx.x] = t;
    }
}

// One workgroup: v[0, n) scanned in place (exclusive), the sum to *total.
// Each thread scans a contiguous chunk after the workgroup's scan of the
// chunk sums.
constexpr int SCAN_BLOCKS_BLOCK = 1024;
__global__ void __launch_bounds__(SCAN_BLOCKS_BLOCK) scan_blocks_kernel(uint32_t* v, uint32_t n, uint32_t* total) {
    __shared__ uint32_t s_w[SCAN_BLOCKS_BLOCK / 64];
    const uint32_t t = threadIdx.x, lane = t & 63u, wave = t >> 6;
    const uint32_t per = (n + SCAN_BLOCKS_BLOCK - 1) / SCAN_BLOCKS_BLOCK;
    const uint32_t lo = (uint32_t)min((uint64_t)t * per, (uint64_t)n), hi = (uint32_t)min((uint64_t)lo + per, (uint64_t)n);
    uint32_t sum = 0u;
    for (uint32_t i = lo; i < hi; ++i) sum += v[i];
    uint32_t incl = sum;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
        const uint32_t u = __shfl_up(incl, o);
        if ((int)lane >= o) incl += u;
    }
    if (lane == 63u) s_w[wave] = incl;
    __syncthreads();
    uint32_t wbase = 0u;
    for (uint32_t w = 0; w < wave; ++w) wbase += s_w[w];
    uint32_t run = wbase + incl - sum;
    for (uint32_t i = lo; i < hi; ++i) {
        const uint32_t x = v[i];
        v[i] = run;
        run += x;
    }
    if (t == SCAN_BLOCKS_BLOCK - 1) *total = wbase + incl;
}

__global__ void fill_u32_kernel(uint32_t* p, uint32_t v, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) p[i] = v;
}
__global__ void fill_f32_kernel(float* p, float v, uint64_t n) {
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += (uint64_t)gridDim.x * blockDim.x) p[i] = v;
}

static uint32_t fill_grid(uint64_t n) {
    const uint64_t b = (n + 255) / 256;
    return (uint32_t)(b < 8192 ? (b ? b : 1) : 8192);
}

hipError_t launch_finalize_counts(uint32_t* block_stats, uint32_t nblocks, uint32_t* counters, uint32_t isect_capacity,
                                  hipStream_t s, uint32_t* host_copy) {
    finalize_counts_kernel<<<1, FIN_BLOCK, 0, s>>>(block_stats, nblocks, counters, isect_capacity, host_copy);
    return hipGetLastError();
}

template <int DEG, int MODEL, typename SHT>
static void launch_project_geom(const ProjectArgs& a, dim3 grid, hipStream_t s, bool geom) {
    if (geom) project_kernel<DEG, MODEL, true, SHT><<<grid, PROJ_BLOCK, 0, s>>>(a);
    else project_kernel<DEG, MODEL, false, SHT><<<grid, PROJ_BLOCK, 0, s>>>(a);
}
template <int DEG, int MODEL>
static void launch_project_type(const ProjectArgs& a, dim3 grid, hipStream_t s, bool geom) {
    if (a.sh_half) launch_project_geom<DEG, MODEL, uint16_t>(a, grid, s, geom);
    else launch_project_geom<DEG, MODEL, float>(a, grid, s, geom);
}
template <int DEG>
static void launch_project_model(const ProjectArgs& a, dim3 grid, hipStream_t s, bool geom) {
    if (a.proj_surf) {                       // surfels: pinhole camera, no gaussian geometry normal
        launch_project_type<DEG, SURFEL_MODEL>(a, grid, s, false);
        return;
    }
    switch (a.cam.model) {
    case VS_CAMERA_KB4: launch_project_type<DEG, VS_CAMERA_KB4>(a, grid, s, geom); break;
    case VS_CAMERA_RT8: launch_project_type<DEG, VS_CAMERA_RT8>(a, grid, s, geom); break;
    case VS_CAMERA_TPF: launch_project_type<DEG, VS_CAMERA_TPF>(a, grid, s, geom); break;
    default: launch_project_type<DEG, VS_CAMERA_PINHOLE>(a, grid, s, geom); break;
    }
}

hipError_t launch_project(const ProjectArgs& a, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    const dim3 grid((a.num_splats + PROJ_BLOCK - 1) / PROJ_BLOCK);
    const bool geom = a.proj_aux != nullptr;
    if (a.decoder) {
        launch_project_model<NEURAL_DEG>(a, grid, s, geom);
        return hipGetLastError();
    }
    switch (a.sh_degree) {
    case 0: launch_project_model<0>(a, grid, s, geom); break;
    case 1: launch_project_model<1>(a, grid, s, geom); break;
    case 2: launch_project_model<2>(a, grid, s, geom); break;
    case 3: launch_project_model<3>(a, grid, s, geom); break;
    default: launch_project_model<4>(a, grid, s, geom); break;
    }
    return hipGetLastError();
}

hipError_t launch_compact(const CompactArgs& a, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    compact_kernel<<<(a.num_splats + PROJ_BLOCK - 1) / PROJ_BLOCK, PROJ_BLOCK, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_emit(const EmitArgs& a, hipStream_t s) {
    if (a.num_emitters == 0 || a.num_splats == 0) return hipSuccess;
    const uint32_t big_blocks = (a.num_splats + PROJ_BLOCK - 1) / PROJ_BLOCK;   // emit_big_blocks
    const uint32_t grid = big_blocks + (a.num_emitters + PROJ_BLOCK - 1) / PROJ_BLOCK;
    if (a.cut) emit_kernel<true><<<grid, PROJ_BLOCK, 0, s>>>(a);
    else emit_kernel<false><<<grid, PROJ_BLOCK, 0, s>>>(a);
    return hipGetLastError();
}

hipError_t launch_cut_mass(const CutArgs& a, bool back, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    if (!a.pend_total || (back && !a.pend)) return hipErrorInvalidValue;
    const uint32_t grid = (a.num_splats + PROJ_BLOCK - 1) / PROJ_BLOCK;
    if (back) cut_mass_kernel<true><<<grid, PROJ_BLOCK, 0, s>>>(a);
    else cut_mass_kernel<false><<<grid, PROJ_BLOCK, 0, s>>>(a);
    return hipGetLastError();
}
hipError_t launch_cut_pending(const CutArgs& a, hipStream_t s) {
    if (a.tile_bh == 0 || a.tile_bw == 0) return hipSuccess;
    if (a.tile_bw > CUT_MAX_BW || !a.pend || !a.pend_total) return hipErrorInvalidValue;
    cut_pending_kernel<<<a.tile_bh, CUT_PEND_BLOCK, 0, s>>>(a);
    return hipGetLastError();
}
hipError_t launch_cut_rows(const CutArgs& a, hipStream_t s) {
    if (a.tile_bh == 0 || a.tile_bw == 0) return hipSuccess;
    if (a.tile_bw > CUT_MAX_BW) return hipErrorInvalidValue;
    cut_rows_kernel<<<a.tile_bh, CUT_ROW_BLOCK, 0, s>>>(a);
    return hipGetLastError();
}
hipError_t launch_cut_sat(const CutArgs& a, hipStream_t s) {
    if (a.tile_bh == 0 || a.tile_bw == 0) return hipSuccess;
    const uint32_t cols = CUT_BINS * (a.tile_bw + 1u);
    cut_sat_kernel<<<(cols + CUT_SAT_BLOCK - 1) / CUT_SAT_BLOCK, CUT_SAT_BLOCK, 0, s>>>(a);
    return hipGetLastError();
}
hipError_t launch_scan_blocks(uint32_t* v, uint32_t n, uint32_t* total, hipStream_t s) {
    if (!v || !total) return hipErrorInvalidValue;
    scan_blocks_kernel<<<1, SCAN_BLOCKS_BLOCK, 0, s>>>(v, n, total);
    return hipGetLastError();
}
hipError_t launch_count_kept(const EmitArgs& a, hipStream_t s) {
    if (a.num_splats == 0) return hipSuccess;
    if (!a.sat || !a.kept_blocks) return hipErrorInvalidValue;
    count_kept_kernel<<<(a.num_splats + PROJ_BLOCK - 1) / PROJ_BLOCK, PROJ_BLOCK, 0, s>>>(a);
    return hipGetLastError();
}

// One lane per element, per-wavefront ballots before the global atomics.
template <bool HALF>
__global__ void __launch_bounds__(256) validate_kernel(const void* __restrict__ p, uint64_t n, uint32_t row,
                                                       uint32_t col0, uint32_t col1, float lo, float hi,
                                                       uint32_t* __restrict__ stats) {
    uint32_t nan = 0, inf = 0, below = 0, above = 0, first_nan = 0xFFFFFFFFu, first_inf = 0xFFFFFFFFu;
    const uint64_t stride = (uint64_t)gridDim.x * blockDim.x;
    for (uint64_t i = (uint64_t)blockIdx.x * blockDim.x + threadIdx.x; i < n; i += stride) {
        const uint32_t col = (uint32_t)(i % row);
        if (col < col0 || col >= col1) continue;
        const float v = HALF ? h2f(static_cast<const uint16_t*>(p)[i]) : static_cast<const float*>(p)[i];
        if (v != v) { ++nan; first_nan = min(first_nan, (uint32_t)min(i, (uint64_t)0xFFFFFFFEu)); }
        else if (!finite(v)) { ++inf; first_inf = min(first_inf, (uint32_t)min(i, (uint64_t)0xFFFFFFFEu)); }
        else { below += v < lo; above += v > hi; }
    }
    const uint64_t any = __ballot(nan | inf | below | above);
    if (any == 0ull) return;
    if (nan) { atomicAdd(&stats[VAL_NAN], nan); atomicMin(&stats[VAL_FIRST_NAN], first_nan); }
    if (inf) { atomicAdd(&stats[VAL_INF], inf); atomicMin(&stats[VAL_FIRST_INF], first_inf); }
    if (below) atomicAdd(&stats[VAL_BELOW], below);
    if (above) atomicAdd(&stats[VAL_ABOVE], above);
}

hipError_t launch_validate(const void* p, bool half, uint64_t n, uint32_t row, uint32_t col0, uint32_t col1, float lo,
                           float hi, uint32_t* stats, hipStream_t s) {
    if (n == 0) return hipSuccess;
    const uint32_t grid = (uint32_t)std::min<uint64_t>((n + 255) / 256, 4096);
    if (half) validate_kernel<true><<<grid, 256, 0, s>>>(p, n, row, col0, col1, lo, hi, stats);
    else validate_kernel<false><<<grid, 256, 0, s>>>(p, n, row, col0, col1, lo, hi, stats);
    return hipGetLastError();
}

hipError_t launch_fill_u32(uint32_t* p, uint32_t value, uint64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    fill_u32_kernel<<<fill_grid(n), 256, 0, s>>>(p, value, n);
    return hipGetLastError();
}
hipError_t launch_fill_f32(float* p, float value, uint64_t n, hipStream_t s) {
    if (n == 0) return hipSuccess;
    fill_f32_kernel<<<fill_grid(n), 256, 0, s>>>(p, value, n);
    return hipGetLastError();
}

} // namespace vs
