// camera.cpp -- host camera math behind vs_camera_uniforms().
//
// Restates crates/splat-train-render/src/camera.rs (f64 fov/focal conversions,
// KB4 fold search, Jacobian clamp limits) and the uniform assembly of
// render.rs:478-503.  The pose algebra follows glam's f32 formulas
// (Affine3A::from_rotation_translation, Mat3A::inverse via cross products),
// which is what the reference's `Camera::world_to_local` evaluates.
#include <cmath>
#include <cstring>
#include "../../include/vsplat.h"

namespace {

constexpr double PI64 = 3.14159265358979323846;

double kb4_d(double th, const float* k) {
    const double t2 = th * th, t3 = t2 * th, t5 = t3 * t2, t7 = t5 * t2, t9 = t7 * t2;
    return th + (double)k[0] * t3 + (double)k[1] * t5 + (double)k[2] * t7 + (double)k[3] * t9;
}
double kb4_dd(double th, const float* k) {
    const double t2 = th * th, t4 = t2 * t2, t6 = t4 * t2, t8 = t6 * t2;
    return 1.0 + 3.0 * (double)k[0] * t2 + 5.0 * (double)k[1] * t4 + 7.0 * (double)k[2] * t6 + 9.0 * (double)k[3] * t8;
}
// camera.rs:174-208: coarse scan for the first sign change of d', then bisection.
double kb4_fold(const float* k) {
    const int steps = 128;
    const double step = PI64 / steps;
    double lo = 0.0, hi = PI64;
    bool found = false;
    for (int i = 1; i <= steps; ++i) {
        const double th = i * step;
        if (kb4_dd(th, k) <= 0.0) { hi = th; found = true; break; }
        lo = th;
    }
    if (!found) return PI64;
    for (int it = 0; it < 64; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (kb4_dd(mid, k) > 0.0) lo = mid; else hi = mid;
        if (hi - lo < 1e-12) break;
    }
    return 0.5 * (lo + hi);
}
// camera.rs:210-237: bisection on the rising branch, clamped at the fold.
double kb4_invert(double target, const float* k) {
    if (target <= 0.0) return 0.0;
    const double fold = kb4_fold(k);
    if (target >= kb4_d(fold, k)) return fold;
    double lo = 0.0, hi = fold;
    for (int it = 0; it < 100; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (kb4_d(mid, k) < target) lo = mid; else hi = mid;
        if (hi - lo < 1e-14) break;
    }
    return 0.5 * (lo + hi);
}

// camera.rs:238-248: RT8 radial factor N(r^2) / D(r^2); d = k1..k6.
double rt8_radial(double r, const float* d) {
    const double r2 = r * r, r4 = r2 * r2, r6 = r4 * r2;
    const double num = 1.0 + (double)d[0] * r2 + (double)d[1] * r4 + (double)d[2] * r6;
    const double den = 1.0 + (double)d[3] * r2 + (double)d[4] * r4 + (double)d[5] * r6;
    return num / den;
}
// camera.rs:250-266: undistorted r with r radial(r) = r_d by fixed-point iteration.
double rt8_undistort_radius(double r_d, const float* d) {
    double r = r_d;
    for (int i = 0; i < 30; ++i) {
        const double factor = rt8_radial(r, d);
        if (std::fabs(factor) < 1e-12) break;
        const double r_new = r_d / factor;
        if (std::fabs(r_new - r) < 1e-12) { r = r_new; break; }
        r = r_new;
    }
    return r;
}
// camera.rs:268-303: the first crossing of r radial(r) = r_d below r = 16 by
// a 4096-step scan and bisection; false when the polynomial folds first.
bool rt8_undistort_corner_radius(double r_d, const float* d, double& out) {
    const double r_max = 16.0;
    const int steps = 4096;
    const double step = r_max / steps;
    double lo = 0.0, hi = 0.0;
    bool found = false;
    for (int i = 1; i <= steps; ++i) {
        const double r = i * step;
        if (r * rt8_radial(r, d) >= r_d) { hi = r; found = true; break; }
        lo = r;
    }
    if (!found) return false;
    for (int it = 0; it < 64; ++it) {
        const double mid = 0.5 * (lo + hi);
        if (mid * rt8_radial(mid, d) < r_d) lo = mid; else hi = mid;
        if (hi - lo < 1e-12) break;
    }
    out = 0.5 * (lo + hi);
    return true;
}
float signum(float x) { return x != x ? x : (std::signbit(x) ? -1.0f : 1.0f); }

struct V3f { float x, y, z; };
V3f cross(V3f a, V3f b) { return V3f{a.y * b.z - b.y * a.z, a.z * b.x - b.z * a.x, a.x * b.y - b.x * a.y}; }
float dot3(V3f a, V3f b) { return (a.x * b.x + a.y * b.y) + a.z * b.z; }
struct M3f { V3f c0, c1, c2; };
V3f mulv(const M3f& m, V3f v) {
    return V3f{(m.c0.x * v.x + m.c1.x * v.y) + m.c2.x * v.z,
               (m.c0.y * v.x + m.c1.y * v.y) + m.c2.y * v.z,
               (m.c0.z * v.x + m.c1.z * v.y) + m.c2.z * v.z};
}
// glam Mat3A::from_quat
M3f from_quat(const float q[4]) {
    const float x = q[0], y = q[1], z = q[2], w = q[3];
    const float x2 = x + x, y2 = y + y, z2 = z + z;
    const float xx = x * x2, xy = x * y2, xz = x * z2;
    const float yy = y * y2, yz = y * z2, zz = z * z2;
    const float wx = w * x2, wy = w * y2, wz = w * z2;
    return M3f{V3f{1.0f - (yy + zz), xy + wz, xz - wy},
               V3f{xy - wz, 1.0f - (xx + zz), yz + wx},
               V3f{xz + wy, yz - wx, 1.0f - (xx + yy)}};
}
// glam Mat3A::inverse
M3f inverse(const M3f& m) {
    const V3f t0 = cross(m.c1, m.c2), t1 = cross(m.c2, m.c0), t2 = cross(m.c0, m.c1);
    const float det = dot3(m.c2, t2);
    const float inv = 1.0f / det;
    const V3f a{t0.x * inv, t0.y * inv, t0.z * inv};
    const V3f b{t1.x * inv, t1.y * inv, t1.z * inv};
    const V3f c{t2.x * inv, t2.y * inv, t2.z * inv};
    // transpose of from_cols(a, b, c)
    return M3f{V3f{a.x, b.x, c.x}, V3f{a.y, b.y, c.y}, V3f{a.z, b.z, c.z}};
}

} // namespace

// `params`: kb4 k1..k4 then dist[8] (12 floats).
extern "C" double vs_fov_to_focal(double fov, uint32_t pixels, int32_t model, const float* params) {
    const double half = fov / 2.0;
    const double r_pix = (double)pixels / 2.0;
    double projected = std::tan(half);
    if (model == VS_CAMERA_KB4 || model == VS_CAMERA_TPF) projected = kb4_d(half, params);
    else if (model == VS_CAMERA_RT8) projected = projected * rt8_radial(projected, params + 4);
    return r_pix / projected;
}

extern "C" double vs_focal_to_fov(double focal, uint32_t pixels, int32_t model, const float* params) {
    const double r_pix = (double)pixels / 2.0;
    const double r_norm = r_pix / focal;
    double half;
    if (model == VS_CAMERA_KB4 || model == VS_CAMERA_TPF) half = kb4_invert(r_norm, params);
    else if (model == VS_CAMERA_RT8) half = std::atan(rt8_undistort_radius(r_norm, params + 4));
    else half = std::atan(r_norm);
    return 2.0 * half;
}

extern "C" double vs_max_render_theta(int32_t model, const float* params) {
    return (model == VS_CAMERA_KB4 || model == VS_CAMERA_TPF) ? kb4_fold(params) : PI64;
}

extern "C" vs_status vs_camera_uniforms(const vs_pose* pose, uint32_t img_w, uint32_t img_h, vs_camera* out) {
    if (!pose || !out || img_w == 0 || img_h == 0) return VS_ERR_INVALID;
    if (pose->model < VS_CAMERA_PINHOLE || pose->model > VS_CAMERA_TPF) return VS_ERR_INVALID;
    vs_camera c;
    std::memset(&c, 0, sizeof(c));
    c.model = pose->model;
    if (pose->model == VS_CAMERA_KB4 || pose->model == VS_CAMERA_TPF) std::memcpy(c.kb4, pose->kb4, sizeof(c.kb4));
    if (pose->model == VS_CAMERA_RT8) std::memcpy(c.dist, pose->dist, sizeof(c.dist));
    if (pose->model == VS_CAMERA_TPF) std::memcpy(c.dist, pose->dist, 4 * sizeof(float));
    float params[12];
    std::memcpy(params, c.kb4, sizeof(c.kb4));
    std::memcpy(params + 4, c.dist, sizeof(c.dist));
    // camera.rs:55-79
    c.fx = (float)vs_fov_to_focal(pose->fov_x, img_w, pose->model, params);
    c.fy = (float)vs_fov_to_focal(pose->fov_y, img_h, pose->model, params);
    c.cx = pose->center_uv[0] * (float)img_w;
    c.cy = pose->center_uv[1] * (float)img_h;
    // render.rs:478-480 (f32 arithmetic, std::f32::consts::PI)
    const float pi32 = 3.14159265358979323846f;
    const float diag = std::hypot((float)pose->fov_x, (float)pose->fov_y) * 1.05f;
    const float capped = std::fmin(diag, 2.0f * pi32 - 1e-6f) * 0.5f;
    c.half_max_render_fov = std::fmin(capped, (float)vs_max_render_theta(pose->model, params));
    // camera.rs:90-96: world_to_local = (R, t)^-1
    const M3f R = from_quat(pose->rotation);
    const M3f Ri = inverse(R);
    const V3f t{pose->position[0], pose->position[1], pose->position[2]};
    const V3f ti = mulv(Ri, t);
    const V3f trans{-ti.x, -ti.y, -ti.z};
    c.viewmat[0] = Ri.c0.x; c.viewmat[1] = Ri.c0.y; c.viewmat[2] = Ri.c0.z;
    c.viewmat[3] = Ri.c1.x; c.viewmat[4] = Ri.c1.y; c.viewmat[5] = Ri.c1.z;
    c.viewmat[6] = Ri.c2.x; c.viewmat[7] = Ri.c2.y; c.viewmat[8] = Ri.c2.z;
    c.viewmat[9] = trans.x; c.viewmat[10] = trans.y; c.viewmat[11] = trans.z;
    // render.rs:485: centre = world_to_local.inverse().translation
    const M3f Rb = inverse(Ri);
    const V3f tb = mulv(Rb, trans);
    c.cam_pos[0] = -tb.x; c.cam_pos[1] = -tb.y; c.cam_pos[2] = -tb.z;
    // camera.rs:305-374: the pinhole margin; RT8 inverts it through the
    // radial model and caps the radius at the same-margin image corner's;
    // the fisheye models leave the limits at zero.
    c.lim_r = 3.40282347e+38f;
    const float w = (float)img_w, h = (float)img_h;
    if (pose->model == VS_CAMERA_PINHOLE) {
        c.lim_pos_x = (1.15f * w - c.cx) / c.fx;
        c.lim_pos_y = (1.15f * h - c.cy) / c.fy;
        c.lim_neg_x = (-0.15f * w - c.cx) / c.fx;
        c.lim_neg_y = (-0.15f * h - c.cy) / c.fy;
    } else if (pose->model == VS_CAMERA_RT8) {
        auto undistort = [&](float edge) {
            return (float)rt8_undistort_radius((double)std::fabs(edge), c.dist) * signum(edge);
        };
        const float edge_pos_x = (1.15f * w - c.cx) / c.fx, edge_pos_y = (1.15f * h - c.cy) / c.fy;
        const float edge_neg_x = (-0.15f * w - c.cx) / c.fx, edge_neg_y = (-0.15f * h - c.cy) / c.fy;
        c.lim_pos_x = undistort(edge_pos_x);
        c.lim_pos_y = undistort(edge_pos_y);
        c.lim_neg_x = undistort(edge_neg_x);
        c.lim_neg_y = undistort(edge_neg_y);
        const double corner_d = std::hypot((double)std::fmax(std::fabs(edge_pos_x), std::fabs(edge_neg_x)),
                                           (double)std::fmax(std::fabs(edge_pos_y), std::fabs(edge_neg_y)));
        double r;
        if (rt8_undistort_corner_radius(corner_d, c.dist, r)) c.lim_r = (float)r;
    }
    *out = c;
    return VS_OK;
}
