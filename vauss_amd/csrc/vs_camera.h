// vs_camera.h -- device camera models: projection, Jacobian and projection VJP
// for the pinhole and Kannala-Brandt-4 ("OpenCV fisheye") models.
// Restates crates/splat-train-render/src/kernels/camera_model/{pinhole,kannala_brandt_4}.rs
// in their operation order.
#pragma once
#include "vs_device.h"
#include "../../include/vsplat.h"

namespace vs {

VS_DEV M3 view_rot(const vs_camera& u) {
    return M3{F3{u.viewmat[0], u.viewmat[1], u.viewmat[2]},
              F3{u.viewmat[3], u.viewmat[4], u.viewmat[5]},
              F3{u.viewmat[6], u.viewmat[7], u.viewmat[8]}};
}
// kernels/helpers.rs:472-475
VS_DEV F3 world_to_cam(F3 m, const vs_camera& u) {
    return mul(view_rot(u), m) + F3{u.viewmat[9], u.viewmat[10], u.viewmat[11]};
}

// pinhole.rs:165-171 / kannala_brandt_4.rs:18-54
template <int MODEL>
VS_DEV void project_point(F3 p, const vs_camera& u, float& ou, float& ov) {
    const float inv_z = 1.0f / p.z;
    if constexpr (MODEL == VS_CAMERA_PINHOLE) {
        ou = u.fx * p.x * inv_z + u.cx;
        ov = u.fy * p.y * inv_z + u.cy;
    } else {
        const float pin_u = u.fx * p.x * inv_z + u.cx;
        const float pin_v = u.fy * p.y * inv_z + u.cy;
        const float r = __builtin_sqrtf(p.x * p.x + p.y * p.y);
        const float th = atan2f_c(r, p.z);
        const float t2 = th * th, t4 = t2 * t2, t6 = t2 * t4, t8 = t4 * t4;
        const float d = th * (1.0f + u.kb4[0] * t2 + u.kb4[1] * t4 + u.kb4[2] * t6 + u.kb4[3] * t8);
        const float inv_r = 1.0f / r;
        const float fu = u.fx * (d * p.x * inv_r) + u.cx;
        const float fv = u.fy * (d * p.y * inv_r) + u.cy;
        const bool near_axis = r < 1e-6f;
        ou = near_axis ? pin_u : fu;
        ov = near_axis ? pin_v : fv;
    }
}

// pinhole.rs:173-197 / kannala_brandt_4.rs:58-152
template <int MODEL>
VS_DEV M23 project_jacobian(F3 p, const vs_camera& u) {
    if constexpr (MODEL == VS_CAMERA_PINHOLE) {
        const float inv_z = 1.0f / p.z;
        const float dx = u.fx * inv_z, dy = u.fy * inv_z;
        const float cx = clampf(p.x * inv_z, u.lim_neg_x, u.lim_pos_x);
        const float cy = clampf(p.y * inv_z, u.lim_neg_y, u.lim_pos_y);
        return M23{F2{dx, 0.0f}, F2{0.0f, dy}, F2{-dx * cx, -dy * cy}};
    } else {
        const float k1 = u.kb4[0], k2 = u.kb4[1], k3 = u.kb4[2], k4 = u.kb4[3];
        const float x = p.x, y = p.y, z = p.z;
        const float inv_z = 1.0f / z;
        const float x2 = x * x, y2 = y * y, xy = x * y;
        const float r2 = x2 + y2;
        const float r = __builtin_sqrtf(r2);
        const float inv_r = 1.0f / r;
        const float inv_r3 = inv_r * inv_r * inv_r;
        const float rho2 = r2 + z * z;
        const float inv_rho2 = 1.0f / rho2;
        const float inv_rho2_r = inv_rho2 * inv_r;
        const float th = atan2f_c(r, z);
        const float t2 = th * th, t4 = t2 * t2, t6 = t4 * t2, t8 = t4 * t4;
        const float d = th * (1.0f + k1 * t2 + k2 * t4 + k3 * t6 + k4 * t8);
        const float dd = 1.0f + 3.0f * k1 * t2 + 5.0f * k2 * t4 + 7.0f * k3 * t6 + 9.0f * k4 * t8;
        const float dth_dx = x * z * inv_rho2_r, dth_dy = y * z * inv_rho2_r, dth_dz = -r * inv_rho2;
        const float dd_dx = dd * dth_dx, dd_dy = dd * dth_dy, dd_dz = dd * dth_dz;
        const float xr = x * inv_r, dxr_dx = y2 * inv_r3, dxr_dy = -xy * inv_r3;
        const float du_dx = u.fx * (dd_dx * xr + d * dxr_dx);
        const float du_dy = u.fx * (dd_dy * xr + d * dxr_dy);
        const float du_dz = u.fx * (dd_dz * xr);
        const float yr = y * inv_r, dyr_dx = -xy * inv_r3, dyr_dy = x2 * inv_r3;
        const float dv_dx = u.fy * (dd_dx * yr + d * dyr_dx);
        const float dv_dy = u.fy * (dd_dy * yr + d * dyr_dy);
        const float dv_dz = u.fy * (dd_dz * yr);
        const bool na = r < 1e-6f;
        const float pdx = u.fx * inv_z, pdy = u.fy * inv_z;
        const float pdu_dz = -pdx * x * inv_z, pdv_dz = -pdy * y * inv_z;
        return M23{F2{na ? pdx : du_dx, na ? 0.0f : dv_dx},
                   F2{na ? 0.0f : du_dy, na ? pdy : dv_dy},
                   F2{na ? pdu_dz : du_dz, na ? pdv_dz : dv_dz}};
    }
}

// pinhole.rs:199-265
VS_DEV F3 projection_vjp_pinhole(M23 J, F3 mc, S3 cov_c, const vs_camera& u, S2 v_cov2d, F2 v_mean2d) {
    const float fx = u.fx, fy = u.fy;
    const float mx_ = mc.x, my_ = mc.y, mz = mc.z;
    const float inv_z = 1.0f / mz;
    const float xr_raw = mx_ * inv_z, yr_raw = my_ * inv_z;
    const float xr = clampf(xr_raw, u.lim_neg_x, u.lim_pos_x);
    const float yr = clampf(yr_raw, u.lim_neg_y, u.lim_pos_y);
    const bool in_x = xr_raw <= u.lim_pos_x && xr_raw >= u.lim_neg_x;
    const bool in_y = yr_raw <= u.lim_pos_y && yr_raw >= u.lim_neg_y;
    const float inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
    float v_mx = fx * inv_z * v_mean2d.x;
    float v_my = fy * inv_z * v_mean2d.y;
    float v_mz = -(fx * mx_ * v_mean2d.x + fy * my_ * v_mean2d.y) * inv_z2;
    const M23 tmp = mul(v_cov2d, J);
    const float vj00 = 2.0f * dot(mrow0(tmp), srow0(cov_c));
    const float vj11 = 2.0f * dot(mrow1(tmp), srow1(cov_c));
    const float vj20 = 2.0f * dot(mrow0(tmp), srow2(cov_c));
    const float vj21 = 2.0f * dot(mrow1(tmp), srow2(cov_c));
    const float tx = mz * xr, ty = mz * yr;
    if (in_x) v_mx += -fx * inv_z2 * vj20; else v_mz += -fx * inv_z3 * vj20 * tx;
    if (in_y) v_my += -fy * inv_z2 * vj21; else v_mz += -fy * inv_z3 * vj21 * ty;
    v_mz += -fx * inv_z2 * vj00 - fy * inv_z2 * vj11 + 2.0f * fx * tx * inv_z3 * vj20 + 2.0f * fy * ty * inv_z3 * vj21;
    return F3{v_mx, v_my, v_mz};
}

// kannala_brandt_4.rs:154-337
VS_DEV F3 projection_vjp_kb4(M23 J, F3 mc, S3 cov_c, const vs_camera& u, S2 v_cov2d, F2 v_mean2d) {
    const float fx = u.fx, fy = u.fy;
    const float k1 = u.kb4[0], k2 = u.kb4[1], k3 = u.kb4[2], k4 = u.kb4[3];
    const float X = mc.x, Y = mc.y, Z = mc.z;
    const float r2 = X * X + Y * Y;
    const float r = mx(__builtin_sqrtf(r2), 1.0e-8f);
    const float rho2 = r2 + Z * Z;
    const float th = atan2f_c(r, Z);
    const float t2 = th * th, t4 = t2 * t2, t6 = t4 * t2, t8 = t4 * t4;
    const float thd = th * (1.0f + k1 * t2 + k2 * t4 + k3 * t6 + k4 * t8);
    const float p1 = 1.0f + 3.0f * k1 * t2 + 5.0f * k2 * t4 + 7.0f * k3 * t6 + 9.0f * k4 * t8;
    const float p2 = 6.0f * k1 * th + 20.0f * k2 * th * t2 + 42.0f * k3 * th * t4 + 72.0f * k4 * th * t6;
    const float inv_r = 1.0f / r, inv_r3 = inv_r * inv_r * inv_r, inv_r5 = inv_r3 * inv_r * inv_r;
    const float inv_rho2 = 1.0f / rho2, inv_rho2_sq = inv_rho2 * inv_rho2, inv_rho2_r = inv_rho2 * inv_r;
    const float dth_x = X * Z * inv_rho2_r, dth_y = Y * Z * inv_rho2_r, dth_z = -r * inv_rho2;
    const float xr = X * inv_r, yr = Y * inv_r;
    const float dxr_x = Y * Y * inv_r3, dxr_y = -X * Y * inv_r3, dyr_x = dxr_y, dyr_y = X * X * inv_r3;
    const float dg_x = p1 * dth_x, dg_y = p1 * dth_y, dg_z = p1 * dth_z;
    float v_mx = dot(v_mean2d, J.c0), v_my = dot(v_mean2d, J.c1), v_mz = dot(v_mean2d, J.c2);
    const M23 tmp = mul(v_cov2d, J);
    const float vu0 = 2.0f * dot(mrow0(tmp), srow0(cov_c)), vu1 = 2.0f * dot(mrow0(tmp), srow1(cov_c)), vu2 = 2.0f * dot(mrow0(tmp), srow2(cov_c));
    const float vv0 = 2.0f * dot(mrow1(tmp), srow0(cov_c)), vv1 = 2.0f * dot(mrow1(tmp), srow1(cov_c)), vv2 = 2.0f * dot(mrow1(tmp), srow2(cov_c));
    const float a3 = 3.0f * r2 + Z * Z, rz = r2 - Z * Z;
    const float h00 = Z * (r2 * rho2 - X * X * a3) * inv_r3 * inv_rho2_sq;
    const float h11 = Z * (r2 * rho2 - Y * Y * a3) * inv_r3 * inv_rho2_sq;
    const float h01 = -X * Y * Z * a3 * inv_r3 * inv_rho2_sq;
    const float h02 = X * rz * inv_r * inv_rho2_sq;
    const float h12 = Y * rz * inv_r * inv_rho2_sq;
    const float h22 = 2.0f * Z * r * inv_rho2_sq;
    const float tx2y = 2.0f * X * X - Y * Y, ty2x = 2.0f * Y * Y - X * X;
    const float hx00 = -3.0f * X * Y * Y * inv_r5, hx01 = Y * tx2y * inv_r5, hx11 = X * ty2x * inv_r5;
    const float hy00 = Y * tx2y * inv_r5, hy01 = X * ty2x * inv_r5, hy11 = -3.0f * X * X * Y * inv_r5;
    {
        const float d2g = p2 * dth_x * dth_x + p1 * h00;
        const float ju = fx * (d2g * xr + dg_x * dxr_x + dg_x * dxr_x + thd * hx00);
        const float jv = fy * (d2g * yr + dg_x * dyr_x + dg_x * dyr_x + thd * hy00);
        v_mx += vu0 * ju + vv0 * jv;
    }
    {
        const float d2g = p2 * dth_y * dth_x + p1 * h01;
        const float ju = fx * (d2g * xr + dg_y * dxr_x + dg_x * dxr_y + thd * hx01);
        const float jv = fy * (d2g * yr + dg_y * dyr_x + dg_x * dyr_y + thd * hy01);
        v_mx += vu1 * ju + vv1 * jv;
    }
    {
        const float d2g = p2 * dth_z * dth_x + p1 * h02;
        const float ju = fx * (d2g * xr + dg_x * 0.0f + dg_z * dxr_x);
        const float jv = fy * (d2g * yr + dg_x * 0.0f + dg_z * dyr_x);
        v_mx += vu2 * ju + vv2 * jv;
    }
    {
        const float d2g = p2 * dth_x * dth_y + p1 * h01;
        const float ju = fx * (d2g * xr + dg_x * dxr_y + dg_y * dxr_x + thd * hx01);
        const float jv = fy * (d2g * yr + dg_x * dyr_y + dg_y * dyr_x + thd * hy01);
        v_my += vu0 * ju + vv0 * jv;
    }
    {
        const float d2g = p2 * dth_y * dth_y + p1 * h11;
        const float ju = fx * (d2g * xr + dg_y * dxr_y + dg_y * dxr_y + thd * hx11);
        const float jv = fy * (d2g * yr + dg_y * dyr_y + dg_y * dyr_y + thd * hy11);
        v_my += vu1 * ju + vv1 * jv;
    }
    {
        const float d2g = p2 * dth_z * dth_y + p1 * h12;
        const float ju = fx * (d2g * xr + dg_y * 0.0f + dg_z * dxr_y);
        const float jv = fy * (d2g * yr + dg_y * 0.0f + dg_z * dyr_y);
        v_my += vu2 * ju + vv2 * jv;
    }
    {
        const float d2g = p2 * dth_x * dth_z + p1 * h02;
        const float ju = fx * (d2g * xr + dg_z * dxr_x + dg_x * 0.0f);
        const float jv = fy * (d2g * yr + dg_z * dyr_x + dg_x * 0.0f);
        v_mz += vu0 * ju + vv0 * jv;
    }
    {
        const float d2g = p2 * dth_y * dth_z + p1 * h12;
        const float ju = fx * (d2g * xr + dg_z * dxr_y + dg_y * 0.0f);
        const float jv = fy * (d2g * yr + dg_z * dyr_y + dg_y * 0.0f);
        v_mz += vu1 * ju + vv1 * jv;
    }
    {
        const float d2g = p2 * dth_z * dth_z + p1 * h22;
        v_mz += vu2 * (fx * (d2g * xr)) + vv2 * (fy * (d2g * yr));
    }
    return F3{v_mx, v_my, v_mz};
}

// calc_cov2d, kernels/helpers.rs:195-225: (J W R S)(J W R S)^T, scaled so no
// entry exceeds 1e18.
template <int MODEL>
VS_DEV S2 cov2d_raw(F3 scl, Qt q, F3 mean_c, const vs_camera& u) {
    const M3 ns = mul_diag(mul(view_rot(u), to_mat3(q)), scl);
    const M23 J = project_jacobian<MODEL>(mean_c, u);
    const S2 raw = gram(mul(J, ns));
    const float ma = max_abs(raw);
    const float sd = (ma > 1.0e18f) ? 1.0e18f / ma : 1.0f;
    return scale(raw, sd);
}

// compensate_cov2d, kernels/helpers.rs:227-245: +0.3 on the diagonal
// (Default), or +0.1 and the opacity factor sqrt(max(det, 0) / det_blurred)
// (Mip).
VS_DEV S2 compensate_cov2d(S2 c, bool mip, float& filter_comp) {
    const float blur = mip ? 0.1f : 0.3f;
    const S2 b{c.c00 + blur, c.c01, c.c11 + blur};
    filter_comp = 1.0f;
    if (mip) {
        const float det_raw = mx(c.c00 * c.c11 - c.c01 * c.c01, 0.0f);
        const float det_blurred = b.c00 * b.c11 - b.c01 * b.c01;
        filter_comp = __builtin_sqrtf(det_raw / det_blurred);
    }
    return b;
}

// apply_scale_floor, kernels/helpers.rs:497-553 (the Mip-Splatting 3D
// filter): s' = sqrt(s^2 + f^2) per axis; the opacity keeps the splat's mass,
// sigmoid(raw) prod(s / s'), clamped to [1e-6, 1 - 1e-6].  Without a floor
// (min_scale NULL) the identity.
struct ScaleFloor {
    F3 scale;
    float opac, coef;
    F3 ratio_sq;          // d log s' / d log s
    bool opac_open;       // the clamp passes gradient
};
VS_DEV ScaleFloor apply_scale_floor(F3 s, float opac_sig, const float* __restrict__ min_scale, uint32_t g) {
    ScaleFloor r{s, opac_sig, 1.0f, F3{1.0f, 1.0f, 1.0f}, true};
    if (min_scale) {
        const float f = min_scale[g], f2 = f * f;
        r.scale = F3{__builtin_sqrtf(s.x * s.x + f2), __builtin_sqrtf(s.y * s.y + f2), __builtin_sqrtf(s.z * s.z + f2)};
        const float rx = s.x / r.scale.x, ry = s.y / r.scale.y, rz = s.z / r.scale.z;
        r.coef = rx * ry * rz;
        r.ratio_sq = F3{rx * rx, ry * ry, rz * rz};
        const float o = opac_sig * r.coef;
        r.opac_open = o > 1.0e-6f && o < 1.0f - 1.0e-6f;
        r.opac = clampf(o, 1.0e-6f, 1.0f - 1.0e-6f);
    }
    return r;
}

} // namespace vs
