// vs_sh.h -- real spherical harmonics up to degree 4: basis, colour and the
// view-direction VJP, restating crates/splat-train-render/src/kernels/sh.rs
// (Sloan, "Efficient Spherical Harmonic Evaluation", JCGT 2013) in its
// accumulation order.  Coefficients are [K,3] per splat, K = (d+1)^2.
#pragma once
#include "vs_device.h"

namespace vs {

constexpr float SH_C0 = 0.2820948f;   // kernels/sh.rs:17

// Basis values Y_0..Y_{K-1}; the order is the order sh.rs adds terms.
template <int DEG>
VS_DEV void sh_basis(F3 v, float* Y) {
    Y[0] = SH_C0;
    if constexpr (DEG >= 1) {
        const float f0a = 0.4886025f;
        Y[1] = -f0a * v.y; Y[2] = f0a * v.z; Y[3] = -f0a * v.x;
    }
    if constexpr (DEG >= 2) {
        const float z2 = v.z * v.z;
        const float f0b = -1.0925485f * v.z;
        const float f1a = 0.54627424f;
        const float fc1 = v.x * v.x - v.y * v.y;
        const float fs1 = 2.0f * v.x * v.y;
        Y[4] = f1a * fs1; Y[5] = f0b * v.y; Y[6] = 0.9461747f * z2 - 0.31539157f;
        Y[7] = f0b * v.x; Y[8] = f1a * fc1;
        if constexpr (DEG >= 3) {
            const float f0c = -2.285229f * z2 + 0.4570458f;
            const float f1b = 1.4453057f * v.z;
            const float f2a = -0.5900436f;
            const float fc2 = v.x * fc1 - v.y * fs1;
            const float fs2 = v.x * fs1 + v.y * fc1;
            const float p12 = v.z * (1.8658817f * z2 - 1.119529f);
            Y[9] = f2a * fs2; Y[10] = f1b * fs1; Y[11] = f0c * v.y; Y[12] = p12;
            Y[13] = f0c * v.x; Y[14] = f1b * fc1; Y[15] = f2a * fc2;
            if constexpr (DEG >= 4) {
                const float f0d = v.z * (-4.683326f * z2 + 2.0071396f);
                const float f1c = 3.3116114f * z2 - 0.47308735f;
                const float f2b = -1.7701308f * v.z;
                const float f3a = 0.62583575f;
                const float fc3 = v.x * fc2 - v.y * fs2;
                const float fs3 = v.x * fs2 + v.y * fc2;
                Y[16] = f3a * fs3; Y[17] = f2b * fs2; Y[18] = f1c * fs1; Y[19] = f0d * v.y;
                Y[20] = 1.9843135f * v.z * p12 - 1.0062306f * Y[6];
                Y[21] = f0d * v.x; Y[22] = f1c * fc1; Y[23] = f2b * fc2; Y[24] = f3a * fc3;
            }
        }
    }
}

template <int DEG> constexpr int sh_count() { return (DEG + 1) * (DEG + 1); }

// One coefficient of an f32 or f16 (raw binary16 bits) row, as f32.
VS_DEV float sh_ld(const float* __restrict__ p, int i) { return p[i]; }
VS_DEV float sh_ld(const uint16_t* __restrict__ p, int i) { return h2f(p[i]); }

// sh.rs:51-140 -- colour = c_0 C0 + sum_k c_k Y_k, terms added in order.
template <int DEG>
VS_DEV F3 sh_color(const float* __restrict__ c, F3 v) {
    float Y[sh_count<DEG>()];
    sh_basis<DEG>(v, Y);
    F3 col = F3{c[0], c[1], c[2]} * Y[0];
#pragma unroll
    for (int k = 1; k < sh_count<DEG>(); ++k) col = col + F3{c[3 * k], c[3 * k + 1], c[3 * k + 2]} * Y[k];
    return col;
}

// sh.rs:147-274 -- d colour . vc / d v.
template <int DEG, typename T>
VS_DEV F3 sh_viewdir_vjp(const T* __restrict__ cb, F3 v, F3 vc) {
    auto co = [&](int k) { return F3{sh_ld(cb, 3 * k), sh_ld(cb, 3 * k + 1), sh_ld(cb, 3 * k + 2)}; };
    float gx = 0.0f, gy = 0.0f, gz = 0.0f;
    if constexpr (DEG >= 1) {
        const float f0a = 0.4886025f;
        const float s_n1 = dot(co(1), vc), s_z0 = dot(co(2), vc), s_p1 = dot(co(3), vc);
        gx += -f0a * s_p1; gy += -f0a * s_n1; gz += f0a * s_z0;
    }
    if constexpr (DEG >= 2) {
        const float z = v.z, x = v.x, y = v.y;
        const float c2 = -1.0925485f, f1a = 0.54627424f;
        const float s_n2 = dot(co(4), vc), s_n1 = dot(co(5), vc), s_z0 = dot(co(6), vc), s_p1 = dot(co(7), vc), s_p2 = dot(co(8), vc);
        gx += 2.0f * f1a * y * s_n2 + c2 * z * s_p1 + 2.0f * f1a * x * s_p2;
        gy += 2.0f * f1a * x * s_n2 + c2 * z * s_n1 - 2.0f * f1a * y * s_p2;
        gz += c2 * y * s_n1 + 2.0f * 0.9461747f * z * s_z0 + c2 * x * s_p1;
    }
    if constexpr (DEG >= 3) {
        const float z = v.z, x = v.x, y = v.y;
        const float z2 = z * z, x2 = x * x, y2 = y * y;
        const float f2a = -0.5900436f, c1b = 1.4453057f;
        const float f1b = c1b * z;
        const float c0c = -2.285229f;
        const float f0c = c0c * z2 + 0.4570458f;
        const float f0c_dz = 2.0f * c0c * z;
        const float s_n3 = dot(co(9), vc), s_n2 = dot(co(10), vc), s_n1 = dot(co(11), vc), s_z0 = dot(co(12), vc);
        const float s_p1 = dot(co(13), vc), s_p2 = dot(co(14), vc), s_p3 = dot(co(15), vc);
        const float d12_z = 3.0f * 1.8658817f * z2 - 1.119529f;
        gx += f2a * 6.0f * x * y * s_n3 + 2.0f * f1b * y * s_n2 + f0c * s_p1 + 2.0f * f1b * x * s_p2 + f2a * 3.0f * (x2 - y2) * s_p3;
        gy += f2a * 3.0f * (x2 - y2) * s_n3 + 2.0f * f1b * x * s_n2 + f0c * s_n1 + (-2.0f) * f1b * y * s_p2 + f2a * (-6.0f) * x * y * s_p3;
        gz += 2.0f * c1b * x * y * s_n2 + f0c_dz * y * s_n1 + d12_z * s_z0 + f0c_dz * x * s_p1 + c1b * (x2 - y2) * s_p2;
    }
    if constexpr (DEG >= 4) {
        const float z = v.z, x = v.x, y = v.y;
        const float z2 = z * z, x2 = x * x, y2 = y * y;
        const float fc1 = x2 - y2, fs1 = 2.0f * x * y;
        const float fc2 = x * fc1 - y * fs1, fs2 = x * fs1 + y * fc1;
        const float f0d = z * (-4.683326f * z2 + 2.0071396f);
        const float f0d_dz = -14.049978f * z2 + 2.0071396f;
        const float f1c = 3.3116114f * z2 - 0.47308735f;
        const float f1c_dz = 2.0f * 3.3116114f * z;
        const float f2b_c = -1.7701308f;
        const float f2b = f2b_c * z;
        const float f3a = 0.62583575f;
        const float p12 = z * (1.8658817f * z2 - 1.119529f);
        const float dp12 = 3.0f * 1.8658817f * z2 - 1.119529f;
        const float dp6 = 2.0f * 0.9461747f * z;
        const float dp20 = 1.9843135f * (p12 + z * dp12) - 1.0062306f * dp6;
        const float s_n4 = dot(co(16), vc), s_n3 = dot(co(17), vc), s_n2 = dot(co(18), vc), s_n1 = dot(co(19), vc);
        const float s_z0 = dot(co(20), vc), s_p1 = dot(co(21), vc), s_p2 = dot(co(22), vc), s_p3 = dot(co(23), vc), s_p4 = dot(co(24), vc);
        gx += f3a * 4.0f * fs2 * s_n4 + f2b * 3.0f * fs1 * s_n3 + f1c * 2.0f * y * s_n2 + f0d * s_p1 + f1c * 2.0f * x * s_p2 + f2b * 3.0f * fc1 * s_p3 + f3a * 4.0f * fc2 * s_p4;
        gy += f3a * 4.0f * fc2 * s_n4 + f2b * 3.0f * fc1 * s_n3 + f1c * 2.0f * x * s_n2 + f0d * s_n1 + f1c * (-2.0f) * y * s_p2 + f2b * (-3.0f) * fs1 * s_p3 + f3a * (-4.0f) * fs2 * s_p4;
        gz += f2b_c * fs2 * s_n3 + f1c_dz * fs1 * s_n2 + f0d_dz * y * s_n1 + dp20 * s_z0 + f0d_dz * x * s_p1 + f1c_dz * fc1 * s_p2 + f2b_c * fc2 * s_p3;
    }
    return F3{gx, gy, gz};
}

} // namespace vs
