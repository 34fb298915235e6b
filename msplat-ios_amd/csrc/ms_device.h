// ms_device.h -- device math shared by the gfx950 kernels.
//
// Arithmetic contract: every kernel is compiled with -ffp-contract=off, so
// each multiply-add written here is either an explicit __builtin_fmaf or a
// separately rounded multiply and add; '/' and sqrtf lower to IEEE
// correctly-rounded sequences on gfx950; exp is ms_expf below.  Given
// identical inputs the forward kernels therefore reproduce a scalar IEEE
// restatement of the reference bit for bit.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "msplat_engine.h"

namespace msd {

struct f3 {
    float x, y, z;
};

__host__ __device__ __forceinline__ float dot3(f3 a, f3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
__host__ __device__ __forceinline__ f3 mul3(f3 a, f3 b) { return {a.x * b.x, a.y * b.y, a.z * b.z}; }
__host__ __device__ __forceinline__ f3 cross3(f3 a, f3 b) {
    return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}

// Constants of msplat_metal.metal:19-44 and :204-212.
constexpr float SH_C0 = 0.28209479177387814f;
constexpr float SH_C1 = 0.4886025119029199f;
__device__ constexpr float SH_C2[5] = {1.0925484305920792f, -1.0925484305920792f,
                                       0.31539156525252005f, -1.0925484305920792f,
                                       0.5462742152960396f};
__device__ constexpr float SH_C3[7] = {-0.5900435899266435f, 2.890611442640554f,
                                       -0.4570457994644658f, 0.3731763325901154f,
                                       -0.4570457994644658f, 1.445305721320277f,
                                       -0.5900435899266435f};
__device__ constexpr float SH_C4[9] = {2.5033429417967046f, -1.7701307697799304f,
                                       0.9461746957575601f, -0.6690465435572892f,
                                       0.10578554691520431f, -0.6690465435572892f,
                                       0.47308734787878004f, -1.7701307697799304f,
                                       0.6258357354491761f};
constexpr float FILTER_SIZE = 0.707106f;  // low-pass cutoff sqrt(2)/2
constexpr float FILTER_INV_SQ = 2.0f;
constexpr float NEAR_N = 0.2f;            // distortion-depth near / far
constexpr float FAR_N = 100.0f;

__device__ __forceinline__ int num_sh_bases(int degree) {
    return degree == 0 ? 1 : degree == 1 ? 4 : degree == 2 ? 9 : degree == 3 ? 16 : 25;
}

// Single-precision exp after S. L. Moshier's Cephes expf: Cody-Waite
// reduction x = k*ln2 + r (ln2 = 0.693359375 - 2.12194440e-4), a degree-7
// polynomial for e^r, then an exact two-step scaling by 2^k (k split in two
// halves so that both factors are normal numbers).
__device__ __forceinline__ float ms_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283905206835f) return __builtin_inff();
    if (x < -103.97208f) return 0.0f;
    float z = __builtin_rintf(x * 1.44269504088896341f);
    float r = __builtin_fmaf(z, -0.693359375f, x);
    r = __builtin_fmaf(z, 2.12194440e-4f, r);
    float r2 = r * r;
    float p = 1.9875691500E-4f;
    p = __builtin_fmaf(p, r, 1.3981999507E-3f);
    p = __builtin_fmaf(p, r, 8.3334519073E-3f);
    p = __builtin_fmaf(p, r, 4.1665795894E-2f);
    p = __builtin_fmaf(p, r, 1.6666665459E-1f);
    p = __builtin_fmaf(p, r, 5.0000001201E-1f);
    p = __builtin_fmaf(p, r2, r);
    p = p + 1.0f;
    int k = (int)z;
    int k1 = k / 2;
    int k2 = k - k1;
    float s1 = __int_as_float((k1 + 127) << 23);
    float s2 = __int_as_float((k2 + 127) << 23);
    return (p * s1) * s2;
}

__device__ __forceinline__ float ms_sigmoid(float x) { return 1.0f / (1.0f + ms_expf(-x)); }

// The rasterizer's Gaussian falloff exp(-rho / 2), rho >= 0, shared bit for
// bit with the golden model's orc_gauss: t = rho * (-log2(e) / 2) (one
// rounding; the constant is log2(e) as a float, halved exactly), clamped at
// -124 (NaN becomes -124), z = rint(t), f = t - z (exact, |f| <= 1/2), 2^f
// as the degree-6 Taylor polynomial of e^(f ln 2) (truncation error below
// 1.2e-7 relative), then ldexp(., z).  The rounding of t dominates: within
// 8 ulp (5e-7 relative) of exp, and a normal number everywhere (>= 4e-38),
// which is all the 1/255 alpha threshold needs far out.
__host__ __device__ __forceinline__ float ms_gauss(float rho) {
    const float t = __builtin_fmaxf(rho * -0.721347510814666748046875f, -124.0f);
    const float z = __builtin_rintf(t);
    const float f = t - z;
    float p = 1.5403530393381606e-4f;
    p = __builtin_fmaf(p, f, 1.3333558146428443e-3f);
    p = __builtin_fmaf(p, f, 9.6181291076284772e-3f);
    p = __builtin_fmaf(p, f, 5.5504108664821580e-2f);
    p = __builtin_fmaf(p, f, 2.4022650695910071e-1f);
    p = __builtin_fmaf(p, f, 6.9314718055994531e-1f);
    p = __builtin_fmaf(p, f, 1.0f);
    return __builtin_ldexpf(p, (int)z);
}

// ms_gauss for 0 <= rho <= kGaussRhoCap, without the clamp: there t is at
// least fl(171 * -log2(e) / 2) = -123.35 > -124, so the clamp never acts and
// the result is ms_gauss(rho) bit for bit.  A caller that caps a larger rho
// (or NaN) at kGaussRhoCap gets ms_gauss(171) ~ 1e-37 instead of
// ms_gauss(rho) <= that, which is as far below any alpha threshold.
constexpr float kGaussRhoCap = 171.0f;
__host__ __device__ __forceinline__ float ms_gauss_capped(float rho) {
    const float t = rho * -0.721347510814666748046875f;
    const float z = __builtin_rintf(t);
    const float f = t - z;
    float p = 1.5403530393381606e-4f;
    p = __builtin_fmaf(p, f, 1.3333558146428443e-3f);
    p = __builtin_fmaf(p, f, 9.6181291076284772e-3f);
    p = __builtin_fmaf(p, f, 5.5504108664821580e-2f);
    p = __builtin_fmaf(p, f, 2.4022650695910071e-1f);
    p = __builtin_fmaf(p, f, 6.9314718055994531e-1f);
    p = __builtin_fmaf(p, f, 1.0f);
    return __builtin_ldexpf(p, (int)z);
}

// Saturating truncation (the tile-rectangle (int) casts of get_bbox,
// msplat_metal.metal:70-73, are undefined outside the int range).
__device__ __forceinline__ int f2i(float x) {
    x = __builtin_fmaxf(x, -2147483648.0f);
    x = __builtin_fminf(x, 2147483520.0f);
    return (int)x;
}

// quat_to_rotmat (msplat_metal.metal:116-136): columns of R.
__device__ __forceinline__ void quat_to_rotmat(const float q[4], f3 &c0, f3 &c1, f3 &c2) {
    float s = 1.0f / __builtin_sqrtf(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
    float w = q[0] * s, x = q[1] * s, y = q[2] * s, z = q[3] * s;
    c0 = {1.f - 2.f * (y * y + z * z), 2.f * (x * y + w * z), 2.f * (x * z - w * y)};
    c1 = {2.f * (x * y - w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z + w * x)};
    c2 = {2.f * (x * z + w * y), 2.f * (y * z - w * x), 1.f - 2.f * (x * x + y * y)};
}

// quat_to_rotmat_vjp (msplat_metal.metal:1252-1295); vR[c] is column c.
__device__ __forceinline__ void quat_to_rotmat_vjp(const float q[4], const f3 vR[3], float out[4]) {
    float s = 1.0f / __builtin_sqrtf(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
    float w = q[0] * s, x = q[1] * s, y = q[2] * s, z = q[3] * s;
    const float R00 = vR[0].x, R01 = vR[0].y, R02 = vR[0].z;
    const float R10 = vR[1].x, R11 = vR[1].y, R12 = vR[1].z;
    const float R20 = vR[2].x, R21 = vR[2].y, R22 = vR[2].z;
    out[0] = 2.f * (x * (R12 - R21) + y * (R20 - R02) + z * (R01 - R10));
    out[1] = 2.f * (-2.f * x * (R11 + R22) + y * (R01 + R10) + z * (R02 + R20) + w * (R12 - R21));
    out[2] = 2.f * (x * (R01 + R10) - 2.f * y * (R00 + R22) + z * (R12 + R21) + w * (R20 - R02));
    out[3] = 2.f * (x * (R02 + R20) + y * (R12 + R21) - 2.f * z * (R00 + R11) + w * (R01 - R10));
}

// Rows 0..3 of projmat applied to the tangent vectors (w = 0) and the centre
// (w = 1): the clip-space columns of compute_transmat_2dgs
// (msplat_metal.metal:246-269).
struct ClipCols {
    float tu[4], tv[4], pc[4];
};

__device__ __forceinline__ ClipCols clip_columns(const float p[3], f3 tu, f3 tv, const float *pm) {
    ClipCols c;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
        c.tu[r] = pm[4 * r + 0] * tu.x + pm[4 * r + 1] * tu.y + pm[4 * r + 2] * tu.z;
        c.tv[r] = pm[4 * r + 0] * tv.x + pm[4 * r + 1] * tv.y + pm[4 * r + 2] * tv.z;
        c.pc[r] = pm[4 * r + 0] * p[0] + pm[4 * r + 1] * p[1] + pm[4 * r + 2] * p[2] + pm[4 * r + 3];
    }
    return c;
}

__device__ __forceinline__ f3 normalize3(f3 v) {
    float inv = 1.0f / __builtin_sqrtf(v.x * v.x + v.y * v.y + v.z * v.z);
    return {v.x * inv, v.y * inv, v.z * inv};
}

// sh_coeffs_to_color (msplat_metal.metal:756-823).
__device__ __forceinline__ void sh_eval(int degree, f3 d, const float *dc, const float *r, float col[3]) {
#pragma unroll
    for (int c = 0; c < 3; ++c) col[c] = SH_C0 * dc[c];
    if (degree < 1) return;
    const float x = d.x, y = d.y, z = d.z;
    const float xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        col[c] += SH_C1 * (-y * r[0 * 3 + c] + z * r[1 * 3 + c] - x * r[2 * 3 + c]);
        if (degree < 2) continue;
        col[c] += (SH_C2[0] * xy * r[3 * 3 + c] + SH_C2[1] * yz * r[4 * 3 + c] +
                   SH_C2[2] * (2.f * zz - xx - yy) * r[5 * 3 + c] + SH_C2[3] * xz * r[6 * 3 + c] +
                   SH_C2[4] * (xx - yy) * r[7 * 3 + c]);
        if (degree < 3) continue;
        col[c] += (SH_C3[0] * y * (3.f * xx - yy) * r[8 * 3 + c] + SH_C3[1] * xy * z * r[9 * 3 + c] +
                   SH_C3[2] * y * (4.f * zz - xx - yy) * r[10 * 3 + c] +
                   SH_C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy) * r[11 * 3 + c] +
                   SH_C3[4] * x * (4.f * zz - xx - yy) * r[12 * 3 + c] +
                   SH_C3[5] * z * (xx - yy) * r[13 * 3 + c] + SH_C3[6] * x * (xx - 3.f * yy) * r[14 * 3 + c]);
        if (degree < 4) continue;
        col[c] += (SH_C4[0] * xy * (xx - yy) * r[15 * 3 + c] + SH_C4[1] * yz * (3.f * xx - yy) * r[16 * 3 + c] +
                   SH_C4[2] * xy * (7.f * zz - 1.f) * r[17 * 3 + c] +
                   SH_C4[3] * yz * (7.f * zz - 3.f) * r[18 * 3 + c] +
                   SH_C4[4] * (zz * (35.f * zz - 30.f) + 3.f) * r[19 * 3 + c] +
                   SH_C4[5] * xz * (7.f * zz - 3.f) * r[20 * 3 + c] +
                   SH_C4[6] * (xx - yy) * (7.f * zz - 1.f) * r[21 * 3 + c] +
                   SH_C4[7] * xz * (xx - 3.f * yy) * r[22 * 3 + c] +
                   SH_C4[8] * (xx * (xx - 3.f * yy) - yy * (3.f * xx - yy)) * r[23 * 3 + c]);
    }
}

// Basis values of sh_coeffs_to_color_vjp (msplat_metal.metal:825-912):
// b[k-1] multiplies v_colors for rest basis k.  Only the first
// num_sh_bases(degree)-1 entries are written.
__device__ __forceinline__ void sh_vjp_basis(int degree, f3 d, float b[24]) {
    if (degree < 1) return;
    const float x = d.x, y = d.y, z = d.z;
    const float xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
    b[0] = -SH_C1 * y;
    b[1] = SH_C1 * z;
    b[2] = -SH_C1 * x;
    if (degree < 2) return;
    b[3] = SH_C2[0] * xy;
    b[4] = SH_C2[1] * yz;
    b[5] = SH_C2[2] * (2.f * zz - xx - yy);
    b[6] = SH_C2[3] * xz;
    b[7] = SH_C2[4] * (xx - yy);
    if (degree < 3) return;
    b[8] = SH_C3[0] * y * (3.f * xx - yy);
    b[9] = SH_C3[1] * xy * z;
    b[10] = SH_C3[2] * y * (4.f * zz - xx - yy);
    b[11] = SH_C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy);
    b[12] = SH_C3[4] * x * (4.f * zz - xx - yy);
    b[13] = SH_C3[5] * z * (xx - yy);
    b[14] = SH_C3[6] * x * (xx - 3.f * yy);
    if (degree < 4) return;
    b[15] = SH_C4[0] * xy * (xx - yy);
    b[16] = SH_C4[1] * yz * (3.f * xx - yy);
    b[17] = SH_C4[2] * xy * (7.f * zz - 1.f);
    b[18] = SH_C4[3] * yz * (7.f * zz - 3.f);
    b[19] = SH_C4[4] * (zz * (35.f * zz - 30.f) + 3.f);
    b[20] = SH_C4[5] * xz * (7.f * zz - 3.f);
    b[21] = SH_C4[6] * (xx - yy) * (7.f * zz - 1.f);
    b[22] = SH_C4[7] * xz * (xx - 3.f * yy);
    b[23] = SH_C4[8] * (xx * (xx - 3.f * yy) - yy * (3.f * xx - yy));
}

// sh_color_dL_ddir (msplat_metal.metal:925-1013); degree-4 bases do not
// contribute to the view-direction gradient.
__device__ __forceinline__ f3 sh_dL_ddir(int degree, f3 d, const float *fr, const float vc[3]) {
    if (degree < 1) return {0.f, 0.f, 0.f};
    const float x = d.x, y = d.y, z = d.z;
    float dx[3], dy[3], dz[3];
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        dx[c] = -SH_C1 * fr[2 * 3 + c];
        dy[c] = -SH_C1 * fr[0 * 3 + c];
        dz[c] = SH_C1 * fr[1 * 3 + c];
    }
    if (degree >= 2) {
        const float xx = x * x, yy = y * y, zz = z * z;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float s4 = fr[3 * 3 + c], s5 = fr[4 * 3 + c], s6 = fr[5 * 3 + c];
            const float s7 = fr[6 * 3 + c], s8 = fr[7 * 3 + c];
            dx[c] += SH_C2[0] * y * s4 + SH_C2[2] * (-2.f * x) * s6 + SH_C2[3] * z * s7 + SH_C2[4] * (2.f * x) * s8;
            dy[c] += SH_C2[0] * x * s4 + SH_C2[1] * z * s5 + SH_C2[2] * (-2.f * y) * s6 + SH_C2[4] * (-2.f * y) * s8;
            dz[c] += SH_C2[1] * y * s5 + SH_C2[2] * (4.f * z) * s6 + SH_C2[3] * x * s7;
        }
        if (degree >= 3) {
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const float s9 = fr[8 * 3 + c], s10 = fr[9 * 3 + c], s11 = fr[10 * 3 + c];
                const float s12 = fr[11 * 3 + c], s13 = fr[12 * 3 + c];
                const float s14 = fr[13 * 3 + c], s15 = fr[14 * 3 + c];
                dx[c] += SH_C3[0] * s9 * (6.f * x * y) + SH_C3[1] * s10 * (y * z) +
                         SH_C3[2] * s11 * (-2.f * x * y) + SH_C3[3] * s12 * (-6.f * x * z) +
                         SH_C3[4] * s13 * (-3.f * xx + 4.f * zz - yy) + SH_C3[5] * s14 * (2.f * x * z) +
                         SH_C3[6] * s15 * (3.f * (xx - yy));
                dy[c] += SH_C3[0] * s9 * (3.f * (xx - yy)) + SH_C3[1] * s10 * (x * z) +
                         SH_C3[2] * s11 * (-3.f * yy + 4.f * zz - xx) + SH_C3[3] * s12 * (-6.f * y * z) +
                         SH_C3[4] * s13 * (-2.f * x * y) + SH_C3[5] * s14 * (-2.f * y * z) +
                         SH_C3[6] * s15 * (-6.f * x * y);
                dz[c] += SH_C3[1] * s10 * (x * y) + SH_C3[2] * s11 * (8.f * y * z) +
                         SH_C3[3] * s12 * (3.f * (2.f * zz - xx - yy)) + SH_C3[4] * s13 * (8.f * x * z) +
                         SH_C3[5] * s14 * (xx - yy);
            }
        }
    }
    f3 r = {0.f, 0.f, 0.f};
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        r.x += dx[c] * vc[c];
        r.y += dy[c] * vc[c];
        r.z += dz[c] * vc[c];
    }
    return r;
}

// dnormvdv (msplat_metal.metal:1017-1025).
__device__ __forceinline__ f3 dnormvdv(f3 v, f3 dv) {
    float sum2 = v.x * v.x + v.y * v.y + v.z * v.z;
    float invsum32 = 1.0f / __builtin_sqrtf(sum2 * sum2 * sum2);
    return {((sum2 - v.x * v.x) * dv.x - v.y * v.x * dv.y - v.z * v.x * dv.z) * invsum32,
            (-v.x * v.y * dv.x + (sum2 - v.y * v.y) * dv.y - v.z * v.y * dv.z) * invsum32,
            (-v.x * v.z * dv.x - v.y * v.z * dv.y + (sum2 - v.z * v.z) * dv.z) * invsum32};
}

// Splat record (MSPLAT_REC_FLOATS = 20 floats, five float4):
//   q0 = (Tu.x Tu.y Tu.z Tv.x)   q1 = (Tv.y Tv.z Tw.x Tw.y)
//   q2 = (Tw.z xy.x xy.y opacity) q3 = (n.x n.y n.z r)   q4 = (g b tau 0)
// with opacity = sigmoid(logit), rgb = max(raw SH + 0.5, 0) and tau the
// reach of the splat: alpha >= 1/255 needs min(rho3d, rho2d) <= tau.
struct Rec {
    float4 q0, q1, q2, q3, q4;
};

// tau = 2 ln(255 opacity) with a margin that covers the rounding of rho, exp
// and the alpha product; -1 when the splat can never reach alpha >= 1/255
// (opacity * G <= opacity and G <= 1).
__device__ __forceinline__ float splat_reach(float opa) {
    const float a = 255.0f * opa;
    if (!(a >= 0.999f)) return -1.0f;
    const float t = __builtin_fmaxf(2.0f * __logf(a), 0.0f);
    return t * 1.0001f + 1e-3f;
}

// Conservative screen box (xmin, xmax, ymin, ymax) of the pixels where a
// splat can reach alpha >= 1/255: the union of the low-pass disc
// rho2d <= tau and the image of the splat-plane disc u^2+v^2 <= tau, whose
// bounding box follows compute_aabb_2dgs (msplat_metal.metal:302-330) with
// cutoff sqrt(tau).  When that disc is not entirely in front of the camera
// (d >= 0) or the bound degenerates, the box is unbounded.
__host__ __device__ __forceinline__ float4 splat_box(const float4 &q0, const float4 &q1, const float4 &q2, float tau) {
    const float inf = __builtin_inff();
    if (!(tau >= 0.0f)) return make_float4(inf, -inf, inf, -inf);
    const f3 T0 = {q0.x, q0.y, q0.z}, T1 = {q0.w, q1.x, q1.y}, T2 = {q1.z, q1.w, q2.x};
    const float r2 = __builtin_sqrtf(0.5f * tau);
    float x0 = q2.y - r2, x1 = q2.y + r2, y0 = q2.z - r2, y1 = q2.z + r2;
    const float d = tau * (T2.x * T2.x + T2.y * T2.y) - T2.z * T2.z;
    bool bounded = d < 0.0f;
    if (bounded) {
        const float inv = 1.0f / d;
        const f3 f = {tau * inv, tau * inv, -inv};
        const float cx = dot3(f, mul3(T0, T2)), cy = dot3(f, mul3(T1, T2));
        const float hx2 = cx * cx - dot3(f, mul3(T0, T0)), hy2 = cy * cy - dot3(f, mul3(T1, T1));
        bounded = hx2 >= 0.0f && hy2 >= 0.0f && cx == cx && cy == cy;
        if (bounded) {
            const float hx = __builtin_sqrtf(hx2), hy = __builtin_sqrtf(hy2);
            x0 = __builtin_fminf(x0, cx - hx);
            x1 = __builtin_fmaxf(x1, cx + hx);
            y0 = __builtin_fminf(y0, cy - hy);
            y1 = __builtin_fmaxf(y1, cy + hy);
        }
    }
    if (!bounded) return make_float4(-inf, inf, -inf, inf);
    const float mx = 1.0f + 1e-3f * (__builtin_fabsf(x0) + __builtin_fabsf(x1));
    const float my = 1.0f + 1e-3f * (__builtin_fabsf(y0) + __builtin_fabsf(y1));
    return make_float4(x0 - mx, x1 + mx, y0 - my, y1 + my);
}

// The ray of pixel p through a splat, k x l with k = px Tw - Tu and
// l = py Tw - Tv (msplat_metal.metal:655-658), expanded about the splat
// centre (xs, ys): ray(p) = R0 + (xs - px) nAx + (ys - py) nAy with
// kc = xs Tw - Tu, lc = ys Tw - Tv, R0 = kc x lc, nAx = lc x Tw,
// nAy = Tw x kc (the (px - xs)(py - ys) term is Tw x Tw = 0).  Exact in real
// arithmetic; every term stays at the splat's own scale, and a pixel needs
// six fmas.  Computed once per splat, shared with the golden model.
__host__ __device__ __forceinline__ void centred_rows(f3 Tu, f3 Tv, f3 Tw, float xs, float ys, f3 &R0, f3 &nAx,
                                                      f3 &nAy) {
    const f3 kc = {__builtin_fmaf(xs, Tw.x, -Tu.x), __builtin_fmaf(xs, Tw.y, -Tu.y), __builtin_fmaf(xs, Tw.z, -Tu.z)};
    const f3 lc = {__builtin_fmaf(ys, Tw.x, -Tv.x), __builtin_fmaf(ys, Tw.y, -Tv.y), __builtin_fmaf(ys, Tw.z, -Tv.z)};
    R0 = cross3(kc, lc);
    nAx = cross3(lc, Tw);
    nAy = cross3(Tw, kc);
}

// 1 / x: the hardware reciprocal and one Newton step.  Equal to the
// correctly rounded 1 / x for every normal |x| < 2^126 (checked
// exhaustively on gfx950, and at every library initialisation over one
// binade); outside that range callers fall back to the division.
__device__ __forceinline__ float ms_rcp_nr(float x) {
    const float y = __builtin_amdgcn_rcpf(x);
    return __builtin_fmaf(__builtin_fmaf(-x, y, 1.0f), y, y);
}
__device__ __forceinline__ bool ms_rcp_nr_exact(float x) {
    const float a = __builtin_fabsf(x);
    return a >= 0x1p-126f && a < 0x1p126f;
}

// The correctly rounded 1 / x for every x: ms_rcp_nr, with the division
// only where some lane's x is outside its exact range (a wave-uniform
// branch, so the common case skips it).  Called by the whole wave.
__device__ __forceinline__ float ms_recip(float x) {
    float r = ms_rcp_nr(x);
    const bool odd = !ms_rcp_nr_exact(x);
    if (__builtin_amdgcn_ballot_w64(odd)) {
        float z = x;
        asm volatile("" : "+v"(z));  // keeps the division inside the branch
        if (odd) r = 1.0f / z;
    }
    return r;
}

// One (pixel, splat) evaluation: the ray-splat intersection, low-pass
// filter and alpha of nd_rasterize_forward_2dgs_kernel
// (msplat_metal.metal:651-683), on the centred ray (centred_rows) of the
// staged planes p0 = (R0, nAx.x), p1 = (nAx.yz, nAy.xy), p2 = (nAy.z, xs,
// ys, opacity), p3 = (Tw, .).  Bit for bit the golden model's eval_pair.
struct PairEval {
    f3 ray;
    float inv_z, u, v, rho3d, rho2d, depth, G, alpha;
};

__device__ __forceinline__ uint64_t eval_pair(float px, float py, const float4 &p0, const float4 &p1,
                                              const float4 &p2, const float4 &p3, PairEval &e) {
    // Straight-line: every value is computed, then the reference's
    // rejections are applied with their exact comparisons (a NaN compares
    // false in each, as in the reference's early returns), each as the
    // wave's lane mask, so the wave needs no exec-mask branches.  Returns the
    // mask of the wave's lanes whose pair passes; called by the whole wave.
    const float dxs = p2.y - px, dys = p2.z - py;
    e.ray = {__builtin_fmaf(dxs, p0.w, __builtin_fmaf(dys, p1.z, p0.x)),
             __builtin_fmaf(dxs, p1.x, __builtin_fmaf(dys, p1.w, p0.y)),
             __builtin_fmaf(dxs, p1.y, __builtin_fmaf(dys, p2.x, p0.z))};
    // infinite when ray.z == 0; that pair is rejected below
    e.inv_z = ms_rcp_nr(e.ray.z);
    {
        // the division only where some lane's ray.z is outside the exact
        // range (a wave-uniform branch, so the common case skips it)
        const bool odd = !ms_rcp_nr_exact(e.ray.z);
        if (__builtin_amdgcn_ballot_w64(odd)) {
            float z = e.ray.z;
            asm volatile("" : "+v"(z));  // keeps the division inside the branch
            if (odd) e.inv_z = 1.0f / z;
        }
    }
    e.u = e.ray.x * e.inv_z;
    e.v = e.ray.y * e.inv_z;
    e.rho3d = __builtin_fmaf(e.u, e.u, e.v * e.v);
    e.rho2d = FILTER_INV_SQ * __builtin_fmaf(dxs, dxs, dys * dys);
    // capped for ms_gauss_capped (one v_min3): beyond the cap ms_gauss is
    // below 1e-37, so alpha < 1/255 either way and every decision, hence
    // every output, is the one ms_gauss(min(rho3d, rho2d)) gives
    const float rho = __builtin_fminf(__builtin_fminf(e.rho3d, e.rho2d), kGaussRhoCap);
    e.depth = __builtin_fmaf(e.u, p3.x, __builtin_fmaf(e.v, p3.y, p3.z));
    // The reference's power > 0 rejection (msplat_metal.metal:676-677) never
    // fires: rho is a minimum of sums of squares (>= 0, +inf or NaN), so
    // power = -rho / 2 is <= 0, -inf or NaN.
    e.G = ms_gauss_capped(rho);
    e.alpha = __builtin_fminf(0.99f, p2.w * e.G);
    return __builtin_amdgcn_ballot_w64(!(e.ray.z == 0.0f)) & __builtin_amdgcn_ballot_w64(!(e.depth < NEAR_N)) &
           __builtin_amdgcn_ballot_w64(!(e.alpha < 1.0f / 255.0f));
}

// Pixels of a 16x16 tile handled by wave w of a 256-thread rasterizer
// workgroup: an 8x8 quadrant (w & 1 selects the column, w >> 1 the row), lane
// l at (l & 7, l >> 3) inside it.  Square blocks meet fewer splat footprints
// than 16x4 strips of the same area.
constexpr int kWaveW = 8, kWaveH = 8;
__host__ __device__ constexpr int wave_x0(int w) { return (w & 1) * kWaveW; }
__host__ __device__ constexpr int wave_y0(int w) { return (w >> 1) * kWaveH; }
__host__ __device__ constexpr int lane_px(int w, int lane) { return wave_x0(w) + (lane & 7); }
__host__ __device__ constexpr int lane_py(int w, int lane) { return wave_y0(w) + (lane >> 3); }

// The 3DGS mode's screen box (xmin, xmax, ymin, ymax) of the pixels where a
// Gaussian centred at (xs, ys) with 2D covariance C = c2 (xx, xy, yy) can
// reach alpha >= 1/255 under the fp32 pair rule on its fp32 conic K:
// rho_f = fl(d^T K d) <= tau.
//  - d^T C^-1 d <= T spans sqrt(T C_xx) in x and sqrt(T C_yy) in y.
//  - Rounding: evaluating rho (five roundings over terms whose magnitudes
//    sum to at most 3 cond rho, cond = lambda_max / lambda_min of C) and
//    K's own rounding from C (the determinant cancels to ~2 cond ulp) keep
//    rho_f >= d^T C^-1 d (1 - 40 u cond), u = 2^-24; so T = tau (1 + 40 u
//    cond) / (1 - 40 u cond) bounds the reach.  Beyond 40 u cond = 1/4 the
//    box is unbounded (the tile rectangle alone limits the splat).
//  - The extents are grown by 0.1% and 1e-3 px for the rounding of the box
//    itself.  Empty when tau < 0 (the Gaussian never reaches 1/255).
__host__ __device__ __forceinline__ float4 gauss3_box(float xs, float ys, const float c2[3], float tau) {
    const float inf = __builtin_inff();
    if (!(tau >= 0.0f)) return make_float4(inf, -inf, inf, -inf);
    const float b = 0.5f * (c2[0] + c2[2]);
    const float det = c2[0] * c2[2] - c2[1] * c2[1];
    const float lmax = b + __builtin_sqrtf(__builtin_fmaxf(b * b - det, 0.0f));
    const float lmin = det / lmax;
    const float k = 40.0f * 5.9604645e-8f * (lmax / lmin);
    if (!(lmin > 0.0f) || !(k < 0.25f)) return make_float4(-inf, inf, -inf, inf);
    const float t = tau * (1.0f + k) / (1.0f - k);
    const float hx = __builtin_sqrtf(t * c2[0]) * 1.001f + 1e-3f;
    const float hy = __builtin_sqrtf(t * c2[2]) * 1.001f + 1e-3f;
    return make_float4(xs - hx, xs + hx, ys - hy, ys + hy);
}

// Bit w (w = 0..3) set when the splat box meets the pixel block of wave w
// of the tile whose top-left pixel is (sx0, sy0).
__host__ __device__ __forceinline__ int strip_mask(const float4 &b, float sx0, float sy0) {
    int m = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const float x0 = sx0 + wave_x0(w), y0 = sy0 + wave_y0(w);
        if (!(b.x > x0 + (kWaveW - 1) || b.y < x0 || b.z > y0 + (kWaveH - 1) || b.w < y0)) m |= 1 << w;
    }
    return m;
}

// Quadrant masks.  Bit w of a (tile, splat) mask is set when a pixel centre
// of wave w's 8x8 block may reach alpha >= 1/255, i.e. u^2+v^2 <= tau or
// rho2d <= tau.  On the centred rows (centred_rows) the ray of pixel p is,
// with delta = p - (xs, ys),
//   ray = R0 - delta.x nAx - delta.y nAy,
// linear in delta, so u^2+v^2 <= tau is the quadratic region
//   g(delta) = ray.x^2 + ray.y^2 - tau ray.z^2 <= 0,
//   g = a x^2 + 2 b x y + c y^2 + 2 d x + 2 e y + f,
// an ellipse when g's quadratic part is positive definite.  A block
// rectangle (grown by half a pixel) meets a convex region iff the region's
// centre lies in it or one of its four edges meets the region.  On a
// vertical line delta.x = X the ellipse {g <= tol} is the chord
//   |y - (ye - kv (X - xe))| <= sqrt(Av - Bv (X - xe)^2)
// about its centre (xe, ye), with kv = b / c, Av = (tol - gmin) / c,
// Bv = det / c^2 (gmin = g(xe, ye), det = a c - b^2), and likewise on a
// horizontal line with a for c.  Everything that depends on the splat alone
// is computed once per splat (mask_record, in the projection); per tile the
// 2x2 blocks share 3 vertical and 3 horizontal lines, so the test is six
// chords, each compared with two edge segments through squared distances
// (no root, no division), plus the low-pass disc.  The ellipse is that of
// a 1% larger tau with a rounding allowance tol = 1e-5 M^2 (M bounds the
// ray's magnitude over every tile of the splat's rectangle), so every test
// is conservative: masked-out splats are exactly pairs eval_pair rejects.
// Ill-conditioned or unbounded regions keep the screen-box mask.
struct MaskRec {
    float4 box;  // splat_box (xmin, xmax, ymin, ymax)
    float4 e;    // (xe, ye, kv, kh): ellipse centre (delta frame), chord slopes
    float4 h;    // (Av, Bv, Ah, Bh): chord half-width^2 = A - B t^2
};

// Per-splat part.  q0..q2 are the splat's first three record planes (T
// rows, centre, opacity), tau its reach, R0 / nAx / nAy its centred rows and
// [tx0, tx1) x [ty0, ty1) its tile rectangle; lp_r2 receives the squared
// radius (delta frame) of its low-pass disc, -1 when it can never blend.
__host__ __device__ __forceinline__ MaskRec mask_record(const float4 &q0, const float4 &q1, const float4 &q2,
                                                        float tau, f3 R0, f3 nAx, f3 nAy, int tx0, int ty0, int tx1,
                                                        int ty1, float &lp_r2) {
    MaskRec m;
    m.box = splat_box(q0, q1, q2, tau);
    // no ellipse: every chord empty, centre outside every block
    m.e = make_float4(1e15f, 1e15f, 0.f, 0.f);
    m.h = make_float4(-1.f, 0.f, -1.f, 0.f);
    lp_r2 = -1.f;
    if (!(tau >= 0.0f)) return m;
    const float tt = tau * 1.01f;
    lp_r2 = 0.5f * tt + 1e-3f;
    const f3 c0 = {-nAx.x, -nAx.y, -nAx.z}, c1 = {-nAy.x, -nAy.y, -nAy.z}, r0 = R0;
    const float a = c0.x * c0.x + c0.y * c0.y - tt * c0.z * c0.z;
    const float b = c0.x * c1.x + c0.y * c1.y - tt * c0.z * c1.z;
    const float c = c1.x * c1.x + c1.y * c1.y - tt * c1.z * c1.z;
    const float d = c0.x * r0.x + c0.y * r0.y - tt * c0.z * r0.z;
    const float e = c1.x * r0.x + c1.y * r0.y - tt * c1.z * r0.z;
    const float f = r0.x * r0.x + r0.y * r0.y - tt * r0.z * r0.z;
    const float det = a * c - b * b;
    if (!(a > 0.0f && c > 0.0f && det > 1e-3f * (a * c))) {
        // ill-conditioned: every chord covers every segment (the box decides)
        m.e = make_float4(0.f, 0.f, 0.f, 0.f);
        m.h = make_float4(1e30f, 0.f, 1e30f, 0.f);
        return m;
    }
    // largest |delta| over the grown pixel rectangles of every listed tile
    const float xs = q2.y, ys = q2.z;
    const float ex = __builtin_fmaxf(__builtin_fabsf((float)(16 * tx0) - 0.5f - xs),
                                     __builtin_fabsf((float)(16 * tx1) - 0.5f - xs));
    const float ey = __builtin_fmaxf(__builtin_fabsf((float)(16 * ty0) - 0.5f - ys),
                                     __builtin_fabsf((float)(16 * ty1) - 0.5f - ys));
    const float st = __builtin_sqrtf(tt);
    const float M = __builtin_fabsf(r0.x) + __builtin_fabsf(r0.y) + st * __builtin_fabsf(r0.z) +
                    ex * (__builtin_fabsf(c0.x) + __builtin_fabsf(c0.y) + st * __builtin_fabsf(c0.z)) +
                    ey * (__builtin_fabsf(c1.x) + __builtin_fabsf(c1.y) + st * __builtin_fabsf(c1.z));
    const float tol = 1e-5f * M * M;
    const float inv_det = 1.0f / det;
    const float xe = (b * e - c * d) * inv_det, ye = (b * d - a * e) * inv_det;
    const float gmin = f + d * xe + e * ye;  // g at the ellipse centre
    if (!(gmin <= tol)) return m;           // empty: the low-pass disc alone
    const float span = tol - gmin;
    // chord half-widths^2 with 1e-4 relative and 1e-4 px^2 absolute slack
    // for the rounding of the per-tile evaluation (and of the reciprocals,
    // a few ulp)
    const float ic = 1.0f / c, ia = 1.0f / a;
    m.e = make_float4(xe, ye, b * ic, b * ia);
    m.h = make_float4(__builtin_fmaf(span * ic, 1.0001f, 1e-4f), det * ic * ic, __builtin_fmaf(span * ia, 1.0001f, 1e-4f),
                      det * ia * ia);
    return m;
}

// Squared distance from t to the segment [lo, hi].
__host__ __device__ __forceinline__ float seg_dist2(float t, float lo, float hi) {
    const float dd = __builtin_fmaxf(__builtin_fmaxf(lo - t, t - hi), 0.0f);
    return dd * dd;
}

// Per-(tile, splat) part: the 4-bit mask for the tile whose top-left pixel
// centre is (sx0, sy0), of the splat centred at (xs, ys).
__host__ __device__ __forceinline__ int quad_mask(const MaskRec &m, float lp_r2, float xs, float ys, float sx0,
                                                  float sy0) {
    const int mbox = strip_mask(m.box, sx0, sy0);
    if (mbox == 0) return 0;
    // block edges in the delta frame: x = V[i], y = L[j], i, j = 0..2
    const float ox = (sx0 - xs) - 0.5f, oy = (sy0 - ys) - 0.5f;
    const float V[3] = {ox, ox + (float)kWaveW, ox + (float)(2 * kWaveW)};
    const float L[3] = {oy, oy + (float)kWaveH, oy + (float)(2 * kWaveH)};
    const float xe = m.e.x, ye = m.e.y;
    // vh[i][j]: the chord on x = V[i] meets segment [L[j], L[j+1]];
    // hh[j][i]: the chord on y = L[j] meets segment [V[i], V[i+1]]
    bool vh[3][2], hh[3][2];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const float dx = V[k] - xe;
        const float hv2 = __builtin_fmaf(-m.h.y, dx * dx, m.h.x);
        const float ym = __builtin_fmaf(-m.e.z, dx, ye);
        vh[k][0] = seg_dist2(ym, L[0], L[1]) <= hv2;
        vh[k][1] = seg_dist2(ym, L[1], L[2]) <= hv2;
        const float dy = L[k] - ye;
        const float hh2 = __builtin_fmaf(-m.h.w, dy * dy, m.h.z);
        const float xm = __builtin_fmaf(-m.e.w, dy, xe);
        hh[k][0] = seg_dist2(xm, V[0], V[1]) <= hh2;
        hh[k][1] = seg_dist2(xm, V[1], V[2]) <= hh2;
    }
    // low-pass disc, centred on the splat centre (delta = 0)
    const float lx0 = __builtin_fminf(__builtin_fmaxf(0.0f, V[0]), V[1]);
    const float lx1 = __builtin_fminf(__builtin_fmaxf(0.0f, V[1]), V[2]);
    const float ly0 = __builtin_fminf(__builtin_fmaxf(0.0f, L[0]), L[1]);
    const float ly1 = __builtin_fminf(__builtin_fmaxf(0.0f, L[1]), L[2]);
    const float lxs[2] = {lx0 * lx0, lx1 * lx1}, lys[2] = {ly0 * ly0, ly1 * ly1};
    int msk = 0;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const int i = w & 1, j = w >> 1;
        const bool centre = xe >= V[i] && xe <= V[i + 1] && ye >= L[j] && ye <= L[j + 1];
        const bool edge = vh[i][j] || vh[i + 1][j] || hh[j][i] || hh[j + 1][i];
        const bool lp = lxs[i] + lys[j] <= lp_r2;
        if (centre || edge || lp) msk |= 1 << w;
    }
    return msk & mbox;
}

// Wave-cooperative enumeration of the tile rectangles held by the 64 lanes
// of a wave.  Lane L owns `count` tiles (its rectangle area, 0 if none); the
// wave walks the concatenation of all 64 lists 64 entries at a time, so each
// lane issues independent per-tile work (no per-lane serial loops whose
// length differs across lanes).  For entry j the owner is the smallest lane
// whose inclusive prefix exceeds j (6-step binary search over shuffles).
// Must be called by all 64 lanes; fn(owner, local_index, active) receives
// owner-side values through shuffles taken by every lane.
template <typename F>
__device__ __forceinline__ void wave_expand(int count, F &&fn) {
    const int lane = threadIdx.x & 63;
    int incl = count;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    const int total = __shfl(incl, 63, 64);
    for (int base = 0; base < total; base += 64) {
        const int j = base + lane;
        int lo = 0, hi = 63;
#pragma unroll
        for (int s = 0; s < 6; ++s) {
            const int mid = (lo + hi) >> 1;
            if (__shfl(incl, mid, 64) <= j)
                lo = mid + 1;
            else
                hi = mid;
        }
        const int o_excl = __shfl(incl, lo, 64) - __shfl(count, lo, 64);
        fn(lo, j - o_excl, j < total);
    }
}

// XCD-aware tile order: MI355X dispatches workgroup i to XCD (i mod 8), so
// giving XCD x the contiguous band of tiles [x*per, (x+1)*per) keeps
// neighbouring tiles -- which share splats -- in one XCD's L2.
__device__ __forceinline__ int xcd_tile(int block, int num_tiles) {
    const int per = (num_tiles + 7) >> 3;
    return (block & 7) * per + (block >> 3);
}

// XCD bands walked in column strips: XCD x owns tile rows
// [x * ty / 8, (x + 1) * ty / 8) (split as evenly as integers allow) and
// takes them in strips kStripW tiles wide, each strip row by row, so the
// ~200 workgroups an XCD runs at once cover a compact block of tiles whose
// splats fit its L2, rather than most of one tile row.  Returns the tile of
// workgroup `block`, or -1 for the padding of a grid of
// xcd_strip_grid(tx, ty) workgroups.  A bijection onto [0, tx * ty).
constexpr int kStripW = 8;
__host__ __device__ __forceinline__ int xcd_strip_grid(int tx, int ty) { return 8 * ((ty + 7) / 8) * tx; }
__host__ __device__ __forceinline__ int xcd_strip_tile(int block, int tx, int ty) {
    const int x = block & 7, k = block >> 3;
    const int base = ty >> 3, extra = ty & 7;
    const int r0 = x * base + (x < extra ? x : extra), bh = base + (x < extra ? 1 : 0);
    if (k >= bh * tx) return -1;
    const int s = k / (kStripW * bh);
    const int idx = k - s * kStripW * bh;
    const int c0 = s * kStripW, w = tx - c0 < kStripW ? tx - c0 : kStripW;
    const int row = idx / w;
    return (r0 + row) * tx + c0 + (idx - row * w);
}

}  // namespace msd
