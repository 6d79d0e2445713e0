// vs_camera.h -- device camera models: projection, Jacobian and projection VJP
// for the pinhole, Kannala-Brandt-4 ("OpenCV fisheye"), radial-tangential-8
// (OpenCV rational) and thin-prism fisheye (COLMAP) models.
// Restates crates/splat-train-render/src/kernels/camera_model/
// {pinhole,kannala_brandt_4,radial_tangential_8,thin_prism_fisheye}.rs in their
// operation order.
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

// thin_prism_fisheye.rs:37-63: the order-2 tangential + thin-prism
// polynomials N_u, N_v of camera-space (x, y) (delta = N / z^2) and their
// (x, y) derivatives.
struct TpPolys { float nu, nv, dnu_dx, dnu_dy, dnv_dx, dnv_dy; };
VS_DEV TpPolys thin_prism_polys(float x, float y, const vs_camera& u) {
    const float p1 = u.dist[0], p2 = u.dist[1], sx1 = u.dist[2], sy1 = u.dist[3];
    const float x2 = x * x, y2 = y * y, xy = x * y, r2 = x2 + y2;
    return TpPolys{2.0f * p1 * xy + p2 * (3.0f * x2 + y2) + sx1 * r2,
                   2.0f * p2 * xy + p1 * (x2 + 3.0f * y2) + sy1 * r2,
                   2.0f * (p1 * y + (3.0f * p2 + sx1) * x),
                   2.0f * (p1 * x + (p2 + sx1) * y),
                   2.0f * (p2 * y + (p1 + sy1) * x),
                   2.0f * (p2 * x + (3.0f * p1 + sy1) * y)};
}

// pinhole.rs:165-171 / kannala_brandt_4.rs:18-54 / radial_tangential_8.rs:23-62 /
// thin_prism_fisheye.rs:65-82
template <int MODEL>
VS_DEV void project_point(F3 p, const vs_camera& u, float& ou, float& ov) {
    const float inv_z = 1.0f / p.z;
    if constexpr (MODEL == VS_CAMERA_PINHOLE) {
        ou = u.fx * p.x * inv_z + u.cx;
        ov = u.fy * p.y * inv_z + u.cy;
    } else if constexpr (MODEL == VS_CAMERA_RT8) {
        const float k1 = u.dist[0], k2 = u.dist[1], k3 = u.dist[2], k4 = u.dist[3], k5 = u.dist[4], k6 = u.dist[5];
        const float p1 = u.dist[6], p2 = u.dist[7];
        const float x_ = p.x / p.z, y_ = p.y / p.z;
        const float x_2 = x_ * x_, y_2 = y_ * y_;
        const float r2 = x_2 + y_2, r4 = r2 * r2, r6 = r4 * r2;
        const float d = (1.0f + k1 * r2 + k2 * r4 + k3 * r6) / (1.0f + k4 * r2 + k5 * r4 + k6 * r6);
        const float x_y_ = x_ * y_;
        const float x__ = x_ * d + 2.0f * p1 * x_y_ + p2 * (r2 + 2.0f * x_2);
        const float y__ = y_ * d + 2.0f * p2 * x_y_ + p1 * (r2 + 2.0f * y_2);
        ou = u.fx * x__ + u.cx;
        ov = u.fy * y__ + u.cy;
    } else if constexpr (MODEL == VS_CAMERA_TPF) {
        float ku, kv;
        project_point<VS_CAMERA_KB4>(p, u, ku, kv);
        const float inv_z2 = inv_z * inv_z;
        const TpPolys tp = thin_prism_polys(p.x, p.y, u);
        ou = ku + u.fx * tp.nu * inv_z2;
        ov = kv + u.fy * tp.nv * inv_z2;
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

// pinhole.rs:173-197 / kannala_brandt_4.rs:58-152 / radial_tangential_8.rs:64-149 /
// thin_prism_fisheye.rs:84-116
template <int MODEL>
VS_DEV M23 project_jacobian(F3 p, const vs_camera& u) {
    if constexpr (MODEL == VS_CAMERA_PINHOLE) {
        const float inv_z = 1.0f / p.z;
        const float dx = u.fx * inv_z, dy = u.fy * inv_z;
        const float cx = clampf(p.x * inv_z, u.lim_neg_x, u.lim_pos_x);
        const float cy = clampf(p.y * inv_z, u.lim_neg_y, u.lim_pos_y);
        return M23{F2{dx, 0.0f}, F2{0.0f, dy}, F2{-dx * cx, -dy * cy}};
    } else if constexpr (MODEL == VS_CAMERA_RT8) {
        const float k1 = u.dist[0], k2 = u.dist[1], k3 = u.dist[2], k4 = u.dist[3], k5 = u.dist[4], k6 = u.dist[5];
        const float p1 = u.dist[6], p2 = u.dist[7];
        const float z = p.z;
        const float inv_z = 1.0f / z, inv_z2 = inv_z * inv_z;
        const float x_b = clampf(p.x * inv_z, u.lim_neg_x, u.lim_pos_x);
        const float y_b = clampf(p.y * inv_z, u.lim_neg_y, u.lim_pos_y);
        // radial cap at the image corner's undistorted radius
        const float r_b = __builtin_sqrtf(x_b * x_b + y_b * y_b);
        const float r_scale = (r_b > u.lim_r) ? u.lim_r / r_b : 1.0f;
        const float x_n = x_b * r_scale, y_n = y_b * r_scale;
        const float xc = x_n * z, yc = y_n * z;
        const float r2 = x_n * x_n + y_n * y_n, r4 = r2 * r2, r6 = r4 * r2;
        const float n_poly = 1.0f + k1 * r2 + k2 * r4 + k3 * r6;
        const float dn_poly = 1.0f + k4 * r2 + k5 * r4 + k6 * r6;
        const float np_poly = k1 + 2.0f * k2 * r2 + 3.0f * k3 * r4;
        const float dnp_poly = k4 + 2.0f * k5 * r2 + 3.0f * k6 * r4;
        const float inv_dn = 1.0f / dn_poly, inv_dn2 = inv_dn * inv_dn;
        const float r_val = n_poly * inv_dn;
        const float rp_val = (np_poly * dn_poly - n_poly * dnp_poly) * inv_dn2;
        const float d00 = r_val + 2.0f * x_n * x_n * rp_val + 2.0f * p1 * y_n + 6.0f * p2 * x_n;
        const float d01 = 2.0f * x_n * y_n * rp_val + 2.0f * p1 * x_n + 2.0f * p2 * y_n;
        const float d10 = d01;
        const float d11 = r_val + 2.0f * y_n * y_n * rp_val + 6.0f * p1 * y_n + 2.0f * p2 * x_n;
        return M23{F2{u.fx * d00 * inv_z, u.fy * d10 * inv_z},
                   F2{u.fx * d01 * inv_z, u.fy * d11 * inv_z},
                   F2{-u.fx * (d00 * xc + d01 * yc) * inv_z2, -u.fy * (d10 * xc + d11 * yc) * inv_z2}};
    } else if constexpr (MODEL == VS_CAMERA_TPF) {
        const M23 kj = project_jacobian<VS_CAMERA_KB4>(p, u);
        const float inv_z = 1.0f / p.z, inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
        const TpPolys tp = thin_prism_polys(p.x, p.y, u);
        return M23{F2{kj.c0.x + u.fx * tp.dnu_dx * inv_z2, kj.c0.y + u.fy * tp.dnv_dx * inv_z2},
                   F2{kj.c1.x + u.fx * tp.dnu_dy * inv_z2, kj.c1.y + u.fy * tp.dnv_dy * inv_z2},
                   F2{kj.c2.x + -2.0f * u.fx * tp.nu * inv_z3, kj.c2.y + -2.0f * u.fy * tp.nv * inv_z3}};
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

namespace vs {

// radial_tangential_8.rs:151-393.  Computes its own Jacobian at the clamped
// (and radially capped) surrogate point; clamped or capped coordinates are
// constants of the mean, routed through S = d(xc, yc, Z) / d(X, Y, Z).
VS_DEV F3 projection_vjp_rt8(F3 mc, S3 cov_c, const vs_camera& u, S2 v_cov2d, F2 v_mean2d) {
    const float fx = u.fx, fy = u.fy;
    const float k1 = u.dist[0], k2 = u.dist[1], k3 = u.dist[2], k4 = u.dist[3], k5 = u.dist[4], k6 = u.dist[5];
    const float p1 = u.dist[6], p2 = u.dist[7];
    const float mz = mc.z;
    const float inv_z = 1.0f / mz;
    const float mx_rz_raw = mc.x * inv_z, my_rz_raw = mc.y * inv_z;
    const float mx_rz_box = clampf(mx_rz_raw, u.lim_neg_x, u.lim_pos_x);
    const float my_rz_box = clampf(my_rz_raw, u.lim_neg_y, u.lim_pos_y);
    const float r_box = __builtin_sqrtf(mx_rz_box * mx_rz_box + my_rz_box * my_rz_box);
    const bool capped = r_box > u.lim_r;
    const float r_scale = capped ? u.lim_r / r_box : 1.0f;
    const float mx_rz = mx_rz_box * r_scale, my_rz = my_rz_box * r_scale;
    const bool in_x = mx_rz_raw <= u.lim_pos_x && mx_rz_raw >= u.lim_neg_x && !capped;
    const bool in_y = my_rz_raw <= u.lim_pos_y && my_rz_raw >= u.lim_neg_y && !capped;
    const float xc = mx_rz * mz, yc = my_rz * mz;
    const float inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z;
    const float x = xc * inv_z, y = yc * inv_z;
    const float r2 = x * x + y * y, r4 = r2 * r2;
    const float n_poly = 1.0f + k1 * r2 + k2 * r4 + k3 * r2 * r4;
    const float dn_poly = 1.0f + k4 * r2 + k5 * r4 + k6 * r2 * r4;
    const float np_poly = k1 + 2.0f * k2 * r2 + 3.0f * k3 * r4;
    const float dnp_poly = k4 + 2.0f * k5 * r2 + 3.0f * k6 * r4;
    const float npp_poly = 2.0f * k2 + 6.0f * k3 * r2;
    const float dnpp_poly = 2.0f * k5 + 6.0f * k6 * r2;
    const float inv_dn = 1.0f / dn_poly, inv_dn2 = inv_dn * inv_dn, inv_dn3 = inv_dn2 * inv_dn;
    const float rr = n_poly * inv_dn;
    const float rrp = (np_poly * dn_poly - n_poly * dnp_poly) * inv_dn2;
    const float rrpp = (npp_poly * dn_poly * dn_poly - 2.0f * np_poly * dn_poly * dnp_poly -
                        n_poly * dnpp_poly * dn_poly + 2.0f * n_poly * dnp_poly * dnp_poly) * inv_dn3;
    const float rx = 2.0f * x * rrp, ry = 2.0f * y * rrp;
    const float rpx = 2.0f * x * rrpp, rpy = 2.0f * y * rrpp;
    const float d00 = rr + 2.0f * x * x * rrp + 2.0f * p1 * y + 6.0f * p2 * x;
    const float d01 = 2.0f * x * y * rrp + 2.0f * p1 * x + 2.0f * p2 * y;
    const float d10 = d01;
    const float d11 = rr + 2.0f * y * y * rrp + 6.0f * p1 * y + 2.0f * p2 * x;
    const float js00 = fx * d00 * inv_z, js01 = fx * d01 * inv_z, js02 = -fx * (d00 * xc + d01 * yc) * inv_z2;
    const float js10 = fy * d10 * inv_z, js11 = fy * d11 * inv_z, js12 = -fy * (d10 * xc + d11 * yc) * inv_z2;
    const float je00 = in_x ? js00 : 0.0f, je10 = in_x ? js10 : 0.0f;
    const float je01 = in_y ? js01 : 0.0f, je11 = in_y ? js11 : 0.0f;
    const float je02 = ((in_x ? 0.0f : mx_rz * js00) + (in_y ? 0.0f : my_rz * js01)) + js02;
    const float je12 = ((in_x ? 0.0f : mx_rz * js10) + (in_y ? 0.0f : my_rz * js11)) + js12;
    // path 1: J_eff^T v_mean2d
    float v_mx = je00 * v_mean2d.x + je10 * v_mean2d.y;
    float v_my = je01 * v_mean2d.x + je11 * v_mean2d.y;
    float v_mz = je02 * v_mean2d.x + je12 * v_mean2d.y;
    // v_J_eff = 2 sym(v_cov2d) J_eff cov_c, pulled back to the surrogate Jacobian
    const M23 tmp = mul(v_cov2d, M23{F2{je00, je10}, F2{je01, je11}, F2{je02, je12}});
    const float ve_u0 = 2.0f * dot(mrow0(tmp), srow0(cov_c)), ve_u1 = 2.0f * dot(mrow0(tmp), srow1(cov_c));
    const float ve_u2 = 2.0f * dot(mrow0(tmp), srow2(cov_c));
    const float ve_v0 = 2.0f * dot(mrow1(tmp), srow0(cov_c)), ve_v1 = 2.0f * dot(mrow1(tmp), srow1(cov_c));
    const float ve_v2 = 2.0f * dot(mrow1(tmp), srow2(cov_c));
    const float vs_u0 = in_x ? ve_u0 : mx_rz * ve_u2, vs_v0 = in_x ? ve_v0 : mx_rz * ve_v2;
    const float vs_u1 = in_y ? ve_u1 : my_rz * ve_u2, vs_v1 = in_y ? ve_v1 : my_rz * ve_v2;
    const float vs_u2 = ve_u2, vs_v2 = ve_v2;
    // second derivatives of the distortion Jacobian entries in (x, y)
    const float dd00_dx = rx + 4.0f * x * rrp + 2.0f * x * x * rpx + 6.0f * p2;
    const float dd00_dy = ry + 2.0f * x * x * rpy + 2.0f * p1;
    const float dd01_dx = 2.0f * y * rrp + 2.0f * x * y * rpx + 2.0f * p1;
    const float dd01_dy = 2.0f * x * rrp + 2.0f * x * y * rpy + 2.0f * p2;
    const float dd10_dx = dd01_dx, dd10_dy = dd01_dy;
    const float dd11_dx = rx + 2.0f * y * y * rpx + 2.0f * p2;
    const float dd11_dy = ry + 4.0f * y * rrp + 2.0f * y * y * rpy + 6.0f * p1;
    const float dd00_dxc = dd00_dx * inv_z, dd00_dyc = dd00_dy * inv_z, dd00_dz = -(xc * dd00_dx + yc * dd00_dy) * inv_z2;
    const float dd01_dxc = dd01_dx * inv_z, dd01_dyc = dd01_dy * inv_z, dd01_dz = -(xc * dd01_dx + yc * dd01_dy) * inv_z2;
    const float dd10_dxc = dd10_dx * inv_z, dd10_dyc = dd10_dy * inv_z, dd10_dz = -(xc * dd10_dx + yc * dd10_dy) * inv_z2;
    const float dd11_dxc = dd11_dx * inv_z, dd11_dyc = dd11_dy * inv_z, dd11_dz = -(xc * dd11_dx + yc * dd11_dy) * inv_z2;
    const float djs00_dxc = fx * dd00_dxc * inv_z, djs00_dyc = fx * dd00_dyc * inv_z;
    const float djs00_dz = fx * (dd00_dz * inv_z - d00 * inv_z2);
    const float djs01_dxc = fx * dd01_dxc * inv_z, djs01_dyc = fx * dd01_dyc * inv_z;
    const float djs01_dz = fx * (dd01_dz * inv_z - d01 * inv_z2);
    const float djs10_dxc = fy * dd10_dxc * inv_z, djs10_dyc = fy * dd10_dyc * inv_z;
    const float djs10_dz = fy * (dd10_dz * inv_z - d10 * inv_z2);
    const float djs11_dxc = fy * dd11_dxc * inv_z, djs11_dyc = fy * dd11_dyc * inv_z;
    const float djs11_dz = fy * (dd11_dz * inv_z - d11 * inv_z2);
    const float djs02_dxc = -fx * (dd00_dxc * xc + d00 + dd01_dxc * yc) * inv_z2;
    const float djs02_dyc = -fx * (dd00_dyc * xc + dd01_dyc * yc + d01) * inv_z2;
    const float djs02_dz = -fx * ((dd00_dz * xc + dd01_dz * yc) * inv_z2 - 2.0f * (d00 * xc + d01 * yc) * inv_z3);
    const float djs12_dxc = -fy * (dd10_dxc * xc + d10 + dd11_dxc * yc) * inv_z2;
    const float djs12_dyc = -fy * (dd10_dyc * xc + dd11_dyc * yc + d11) * inv_z2;
    const float djs12_dz = -fy * ((dd10_dz * xc + dd11_dz * yc) * inv_z2 - 2.0f * (d10 * xc + d11 * yc) * inv_z3);
    const float c_xc = vs_u0 * djs00_dxc + vs_u1 * djs01_dxc + vs_u2 * djs02_dxc + vs_v0 * djs10_dxc +
                       vs_v1 * djs11_dxc + vs_v2 * djs12_dxc;
    const float c_yc = vs_u0 * djs00_dyc + vs_u1 * djs01_dyc + vs_u2 * djs02_dyc + vs_v0 * djs10_dyc +
                       vs_v1 * djs11_dyc + vs_v2 * djs12_dyc;
    const float c_z = vs_u0 * djs00_dz + vs_u1 * djs01_dz + vs_u2 * djs02_dz + vs_v0 * djs10_dz + vs_v1 * djs11_dz +
                      vs_v2 * djs12_dz;
    if (in_x) v_mx += c_xc;
    if (in_y) v_my += c_yc;
    v_mz += c_z;
    if (!in_x) v_mz += mx_rz * c_xc;
    if (!in_y) v_mz += my_rz * c_yc;
    return F3{v_mx, v_my, v_mz};
}

// thin_prism_fisheye.rs:118-203: the KB4 VJP on the full Jacobian plus the
// thin-prism terms' second-derivative contractions.
VS_DEV F3 projection_vjp_tpf(M23 J, F3 mc, S3 cov_c, const vs_camera& u, S2 v_cov2d, F2 v_mean2d) {
    const F3 kg = projection_vjp_kb4(J, mc, cov_c, u, v_cov2d, v_mean2d);
    const float fx = u.fx, fy = u.fy;
    const float p1 = u.dist[0], p2 = u.dist[1], sx1 = u.dist[2], sy1 = u.dist[3];
    const float inv_z = 1.0f / mc.z, inv_z2 = inv_z * inv_z, inv_z3 = inv_z2 * inv_z, inv_z4 = inv_z2 * inv_z2;
    const TpPolys tp = thin_prism_polys(mc.x, mc.y, u);
    const float d2nu_dxx = 6.0f * p2 + 2.0f * sx1, d2nu_dyy = 2.0f * p2 + 2.0f * sx1, d2nu_dxy = 2.0f * p1;
    const float d2nv_dxx = 2.0f * p1 + 2.0f * sy1, d2nv_dyy = 6.0f * p1 + 2.0f * sy1, d2nv_dxy = 2.0f * p2;
    const float h_u_00 = d2nu_dxx * inv_z2, h_u_01 = d2nu_dxy * inv_z2, h_u_11 = d2nu_dyy * inv_z2;
    const float h_u_02 = -2.0f * tp.dnu_dx * inv_z3, h_u_12 = -2.0f * tp.dnu_dy * inv_z3, h_u_22 = 6.0f * tp.nu * inv_z4;
    const float h_v_00 = d2nv_dxx * inv_z2, h_v_01 = d2nv_dxy * inv_z2, h_v_11 = d2nv_dyy * inv_z2;
    const float h_v_02 = -2.0f * tp.dnv_dx * inv_z3, h_v_12 = -2.0f * tp.dnv_dy * inv_z3, h_v_22 = 6.0f * tp.nv * inv_z4;
    const M23 tmp = mul(v_cov2d, J);
    const float vj_u0 = 2.0f * dot(mrow0(tmp), srow0(cov_c)), vj_u1 = 2.0f * dot(mrow0(tmp), srow1(cov_c));
    const float vj_u2 = 2.0f * dot(mrow0(tmp), srow2(cov_c));
    const float vj_v0 = 2.0f * dot(mrow1(tmp), srow0(cov_c)), vj_v1 = 2.0f * dot(mrow1(tmp), srow1(cov_c));
    const float vj_v2 = 2.0f * dot(mrow1(tmp), srow2(cov_c));
    const float v_mx = fx * (vj_u0 * h_u_00 + vj_u1 * h_u_01 + vj_u2 * h_u_02) +
                       fy * (vj_v0 * h_v_00 + vj_v1 * h_v_01 + vj_v2 * h_v_02);
    const float v_my = fx * (vj_u0 * h_u_01 + vj_u1 * h_u_11 + vj_u2 * h_u_12) +
                       fy * (vj_v0 * h_v_01 + vj_v1 * h_v_11 + vj_v2 * h_v_12);
    const float v_mz = fx * (vj_u0 * h_u_02 + vj_u1 * h_u_12 + vj_u2 * h_u_22) +
                       fy * (vj_v0 * h_v_02 + vj_v1 * h_v_12 + vj_v2 * h_v_22);
    return F3{kg.x + v_mx, kg.y + v_my, kg.z + v_mz};
}

// calculate_projection_vjp (camera_model/mod.rs:82-120)
template <int MODEL>
VS_DEV F3 projection_vjp(M23 J, F3 mc, S3 cov_c, const vs_camera& u, S2 v_cov2d, F2 v_mean2d) {
    if constexpr (MODEL == VS_CAMERA_PINHOLE) return projection_vjp_pinhole(J, mc, cov_c, u, v_cov2d, v_mean2d);
    else if constexpr (MODEL == VS_CAMERA_KB4) return projection_vjp_kb4(J, mc, cov_c, u, v_cov2d, v_mean2d);
    else if constexpr (MODEL == VS_CAMERA_RT8) return projection_vjp_rt8(mc, cov_c, u, v_cov2d, v_mean2d);
    else return projection_vjp_tpf(J, mc, cov_c, u, v_cov2d, v_mean2d);
}

} // namespace vs
