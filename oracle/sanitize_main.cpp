// sanitize_main.cpp -- drives every entry point of the CPU oracle on small
// seeded scenes, for a build with AddressSanitizer and UndefinedBehavior-
// Sanitizer (`make -C oracle sanitize`): an out-of-bounds access, a use of
// freed memory or undefined arithmetic in the oracle aborts the run.
//
// TEST INFRASTRUCTURE ONLY (the oracle is the checker, never the product).
#include <cmath>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <cstring>
#include <vector>

#include "vs_oracle.h"

namespace {

uint64_t g_state = 0;
uint64_t next_u64() {   // SplitMix64
    uint64_t z = (g_state += 0x9E3779B97F4A7C15ull);
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}
float uni(float lo, float hi) { return lo + (float)((double)(next_u64() >> 11) * 0x1.0p-53) * (hi - lo); }

struct Scene {
    uint32_t n = 0, degree = 0, k = 1;
    std::vector<float> transforms, sh, raw_opac, min_scale, decoder;
};

Scene make_scene(uint32_t n, uint32_t degree, uint64_t seed, float log_scale_lo, float log_scale_hi) {
    g_state = seed;
    Scene s;
    s.n = n;
    s.degree = degree;
    s.k = (degree + 1) * (degree + 1);
    s.transforms.resize((size_t)n * 10);
    s.sh.resize((size_t)n * s.k * 3);
    s.raw_opac.resize(n);
    s.min_scale.resize(n);
    for (uint32_t i = 0; i < n; ++i) {
        float* t = &s.transforms[(size_t)i * 10];
        t[0] = uni(-1.5f, 1.5f); t[1] = uni(-1.5f, 1.5f); t[2] = uni(-1.5f, 1.5f);
        for (int j = 3; j < 7; ++j) t[j] = uni(-1.0f, 1.0f);
        for (int j = 7; j < 10; ++j) t[j] = uni(log_scale_lo, log_scale_hi);
        for (uint32_t j = 0; j < s.k * 3; ++j) s.sh[(size_t)i * s.k * 3 + j] = j < 3 ? uni(0.0f, 1.0f) : uni(-0.1f, 0.1f);
        s.raw_opac[i] = uni(-1.0f, 3.0f);
        s.min_scale[i] = uni(0.0f, 0.01f);
    }
    // a few degenerate rows: zero quaternion, non-finite mean, behind the camera
    if (n > 8) {
        for (int j = 3; j < 7; ++j) s.transforms[3 * 10 + j] = 0.0f;
        s.transforms[5 * 10 + 0] = NAN;
        s.transforms[7 * 10 + 2] = -50.0f;
    }
    s.decoder.resize(816);
    for (auto& w : s.decoder) w = uni(-0.3f, 0.3f);
    return s;
}

or_camera camera(int model, uint32_t w, uint32_t h) {
    or_camera c;
    std::memset(&c, 0, sizeof(c));
    c.model = model;
    c.fx = c.fy = 0.8f * (float)w;
    c.cx = 0.5f * (float)w;
    c.cy = 0.5f * (float)h;
    c.viewmat[0] = c.viewmat[4] = c.viewmat[8] = 1.0f;   // identity rotation, camera at z = -5
    c.viewmat[11] = 5.0f;
    c.cam_pos[2] = -5.0f;
    c.half_max_render_fov = model == OR_MODEL_PINHOLE ? 3.1415f : 1.4f;
    c.lim_pos_x = (1.15f * (float)w - c.cx) / c.fx;
    c.lim_pos_y = (1.15f * (float)h - c.cy) / c.fy;
    c.lim_neg_x = (-0.15f * (float)w - c.cx) / c.fx;
    c.lim_neg_y = (-0.15f * (float)h - c.cy) / c.fy;
    c.lim_r = 0.0f;
    const float kb4[4] = {0.02f, -0.01f, 0.005f, -0.001f};
    const float rt8[8] = {-0.05f, 0.02f, -0.005f, 0.01f, 0.004f, -0.002f, 0.001f, -0.001f};
    if (model == OR_MODEL_KB4 || model == OR_MODEL_TPF) std::memcpy(c.kb4, kb4, sizeof(kb4));
    if (model == OR_MODEL_RT8) std::memcpy(c.dist, rt8, sizeof(rt8));
    if (model == OR_MODEL_TPF) { c.dist[0] = 0.001f; c.dist[1] = -0.001f; c.dist[2] = 0.002f; c.dist[3] = -0.002f; }
    return c;
}

int g_failures = 0;
uint64_t g_visible = 0, g_isects = 0, g_renders = 0;
void check(int rc, const char* what) {
    if (rc != 0) { std::fprintf(stderr, "%s returned %d\n", what, rc); ++g_failures; }
}

void render_case(const Scene& s, int model, int flags, bool floor, bool neural, uint32_t w, uint32_t h) {
    const or_camera cam = camera(model, w, h);
    const float bg[3] = {0.1f, 0.2f, 0.3f};
    or_fwd* f = nullptr;
    const uint32_t degree = neural ? 3u : s.degree;
    check(or_render_forward(&cam, w, h, s.transforms.data(), s.sh.data(), degree, s.raw_opac.data(), s.n, 0.0f,
                            floor ? s.min_scale.data() : nullptr, neural ? s.decoder.data() : nullptr, bg, flags, 2,
                            &f),
          "or_render_forward");
    if (!f) return;
    or_fwd_info info;
    or_fwd_get_info(f, &info);
    g_visible += info.num_visible;
    g_isects += info.num_intersections;
    g_renders += 1;
    const size_t n = info.num_splats, v = info.num_visible, i = info.num_intersections, t = info.num_tiles;
    const size_t pix = (size_t)info.img_w * info.img_h;
    const size_t sizes[14] = {n * 4, n * 4, n * 4, v * 4, v * 4, v * 36, v * 16, i * 4, i * 4, t * 8, t * 8, n * 4,
                              pix * (info.out_channels ? info.out_channels : 1) * 4, v * 56};
    std::vector<float> img;
    for (int field = 0; field < 14; ++field) {
        std::vector<uint8_t> buf(sizes[field] + 4);
        check(or_fwd_get(f, field, buf.data()), "or_fwd_get");
        if (field == OR_F_OUT_IMG && (flags & OR_FLAG_BWD_INFO)) {
            img.resize(pix * info.out_channels);
            std::memcpy(img.data(), buf.data(), img.size() * 4);
        }
    }
    if (flags & OR_FLAG_BWD_INFO) {
        const uint32_t ch = info.out_channels;
        const uint32_t ng = (flags & OR_FLAG_SURFEL) ? 17u : 10u;
        std::vector<float> v_out(pix * ch);
        for (size_t p = 0; p < pix; ++p)
            for (uint32_t c = 0; c < ch; ++c) v_out[p * ch + c] = (c < 3) ? ((img[p * ch + c] > 0.3f) ? 1e-3f : -1e-3f) : 0.0f;
        const uint32_t k = neural ? 4u : s.k;
        std::vector<float> vc(n * ng), vt(n * 10), vs(n * k * 3), vo(n), vr(n);
        check(or_render_backward(f, v_out.data(), 2, vc.data(), vt.data(), vs.data(), vo.data(), vr.data()),
              "or_render_backward");
        check(or_project_backward(f, vc.data(), 2, vt.data(), vs.data(), vo.data(), vr.data()), "or_project_backward");
        if (neural) {
            std::vector<float> rows(n * 12), sq(n), dec(816);
            std::vector<double> dabs(816);
            check(or_neural_backward(f, vc.data(), 2, vt.data(), rows.data(), sq.data(), dec.data(), dabs.data()),
                  "or_neural_backward");
        } else if (!(flags & OR_FLAG_SURFEL)) {
            double pose[12];
            std::vector<float> rows(n * 12);
            check(or_pose_backward(f, vc.data(), 2, pose, rows.data()), "or_pose_backward");
            std::vector<float> tr(s.transforms), op(s.raw_opac), lr(10, 1e-3f), cd((n + 1) * 6), rw(n), gsq(n);
            std::vector<uint32_t> wt(n * 10, 0u), wo(n, 0u);
            const or_adam adam{0.9f, 0.999f, 10.0f, 1000.0f, 1e-15f, 0.05f, 1e-4f, 3u};
            check(or_project_update(f, vc.data(), tr.data(), op.data(), wt.data(), lr.data(), wo.data(), &adam, cd.data(),
                                    rw.data(), gsq.data(), 2),
                  "or_project_update");
            if (s.degree > 0) {
                std::vector<uint16_t> sh16(s.sh.size());
                for (size_t j = 0; j < sh16.size(); ++j) sh16[j] = or_f32_to_f16(s.sh[j]);
                std::vector<uint32_t> rows_u(n);
                for (size_t j = 0; j < n; ++j) rows_u[j] = (uint32_t)((j % 3 == 0) ? 0 : j + 1);
                const size_t values = sh16.size(), blocks = (values + 127) / 128;
                std::vector<uint32_t> codes(blocks * 32, 0x80808080u);
                std::vector<float> scales(blocks, 0.0f), var(n, 0.0f), lrs(s.k * 3, 1.0f);
                check(or_sh_step(sh16.data(), (uint32_t)n, s.degree, cd.data(), rows_u.data(), gsq.data(), var.data(),
                                 codes.data(), scales.data(), lrs.data(), 0.9f, 0.999f, 10.0f, 1000.0f, 1e-15f, 1e-3f, 3u,
                                 1),
                      "or_sh_step");
            }
        }
        // the image loss on this render
        std::vector<uint32_t> gt(pix);
        for (size_t p = 0; p < pix; ++p) gt[p] = (uint32_t)(next_u64() & 0xFFFFFFFFu);
        const or_loss_cfg cfg{0.8f, -0.2f, 0.1f, 1, {0.1f, 0.2f, 0.3f}, 1};
        const uint32_t tiles = ((info.img_w + 15) / 16) * ((info.img_h + 15) / 16);
        std::vector<float> part((size_t)4 * tiles), coeffs(9 * pix), lmap(pix * 4), dpred(pix * 4), dl(1, 1.0f);
        std::vector<float> pred4(pix * 4);
        for (size_t p = 0; p < pix; ++p)
            for (int c = 0; c < 4; ++c) pred4[p * 4 + c] = img[p * ch + c];
        check(or_image_loss_forward(pred4.data(), 4, gt.data(), info.img_w, info.img_h, &cfg, part.data(), coeffs.data(),
                                    lmap.data()),
              "or_image_loss_forward");
        check(or_image_loss_backward(pred4.data(), 4, gt.data(), info.img_w, info.img_h, &cfg, dl.data(), 1,
                                     coeffs.data(), dpred.data()),
              "or_image_loss_backward");
    }
    or_fwd_free(f);
}

}  // namespace

int main() {
    const Scene sh0 = make_scene(600, 0, 0xA5A5, -4.0f, -2.0f);
    const Scene sh3 = make_scene(500, 3, 0x5A5A, -4.5f, -1.5f);
    const Scene big = make_scene(60, 2, 0x0B16, -1.0f, 0.5f);   // splats covering many tiles
    for (int model = OR_MODEL_PINHOLE; model <= OR_MODEL_TPF; ++model) {
        render_case(sh0, model, OR_FLAG_BWD_INFO, false, false, 64, 48);
        render_case(sh3, model, OR_FLAG_BWD_INFO | OR_FLAG_MIP, true, false, 80, 64);
        render_case(sh3, model, OR_FLAG_BWD_INFO | OR_FLAG_GEOMETRY, false, false, 72, 40);
        render_case(sh3, model, OR_FLAG_BWD_INFO | OR_FLAG_SMOOTH_CUTOFF, false, false, 64, 64);
        render_case(big, model, OR_FLAG_BWD_INFO | OR_FLAG_BRUTE_FORCE, false, false, 48, 48);
        render_case(sh3, model, 0, false, false, 64, 48);                    // packed forward
        render_case(sh3, model, OR_FLAG_BWD_INFO, false, true, 64, 48);      // neural appearance
    }
    render_case(sh3, OR_MODEL_PINHOLE, OR_FLAG_BWD_INFO | OR_FLAG_SURFEL, false, false, 64, 48);
    render_case(sh3, OR_MODEL_PINHOLE, OR_FLAG_BWD_INFO | OR_FLAG_SURFEL | OR_FLAG_SURFACE, true, false, 64, 48);
    render_case(big, OR_MODEL_PINHOLE, OR_FLAG_BWD_INFO | OR_FLAG_SURFEL | OR_FLAG_SMOOTH_CUTOFF, false, false, 40, 40);

    // sort, scan, codecs and transcendentals
    g_state = 0x50F7;
    std::vector<uint32_t> keys(5000), vals(5000), ok(5000), ov(5000), ps(5000);
    for (size_t j = 0; j < keys.size(); ++j) { keys[j] = (uint32_t)next_u64(); vals[j] = (uint32_t)j; }
    or_radix_argsort_u32(keys.data(), vals.data(), 5000, 0, 32, ok.data(), ov.data());
    or_radix_argsort_u32(keys.data(), vals.data(), 5000, 4, 13, ok.data(), ov.data());
    or_prefix_sum_u32(vals.data(), ps.data(), 5000);
    std::vector<float> x(1000), y(1000), z(1000);
    for (size_t j = 0; j < x.size(); ++j) { x[j] = uni(-100.0f, 100.0f); y[j] = uni(-3.0f, 3.0f); }
    or_expf_n(x.data(), z.data(), 1000);
    or_logf_n(x.data(), z.data(), 1000);
    or_atan2f_n(x.data(), y.data(), z.data(), 1000);
    or_sincosf_n(x.data(), y.data(), z.data(), 1000);
    or_tanhf_n(x.data(), z.data(), 1000);
    std::vector<uint32_t> codes(32 * 8);
    std::vector<float> scales(8), dec(1000);
    or_block8_encode(x.data(), 1000, codes.data(), scales.data());
    or_block8_decode(codes.data(), scales.data(), 1000, dec.data());
    const uint32_t zero_rows[2] = {1, 7};
    or_block8_zero_rows(codes.data(), 1000, zero_rows, 2, 48);
    for (int j = 0; j < 200; ++j) {
        float m = 0.0f, v = 0.0f;
        or_geo_decode(or_geo_encode(uni(-1.0f, 1.0f), uni(0.0f, 1.0f), 1e-15f), 1e-15f, &m, &v);
        (void)or_stochastic_half(uni(-10.0f, 10.0f), (uint32_t)j, 5u);
    }
    if (g_failures) {
        std::fprintf(stderr, "%d oracle calls failed\n", g_failures);
        return 1;
    }
    std::printf("oracle sanitizer run: ok (%llu renders, %llu visible splats, %llu intersections)\n",
                (unsigned long long)g_renders, (unsigned long long)g_visible, (unsigned long long)g_isects);
    return 0;
}
