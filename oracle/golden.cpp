/*
 * golden.cpp -- CPU golden model (oracle) of the msplat 2DGS training step.
 *
 * TEST INFRASTRUCTURE ONLY: linked by tests/, __graft_entry__.smoke() and the
 * cpu_baseline leg of bench.py as the checker; never by the product.
 *
 * Every function cites the reference kernel it restates
 * (msplat_metal.metal = core/metal/msplat_metal.metal, etc.).  Expression
 * association follows the reference source left to right; contractions are
 * spelled out with fmaf (see golden.h for the arithmetic contract).
 *
 * Parity pins (tests/test_oracle.py): orc_expf against libm (ulp bound);
 * SH constants and evaluation against an independent fp64 real-SH
 * evaluation; SSIM window against the closed form; SSIM forward against a
 * brute-force 2D 11x11 window; project, raster and loss backward against
 * fp64 central finite differences of the forward; binning against brute-force
 * rectangle enumeration; sort against std::sort; Adam against the one-step
 * closed form; densify against a serial stable-partition restatement.
 */
#include "golden.h"

#include <algorithm>
#include <chrono>
#include <climits>
#include <cmath>
#include <cstring>
#include <vector>

#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

/* ---- constants (msplat_metal.metal:19-44, 204-212, 2804-2816) ---------- */
const float SH_C0 = 0.28209479177387814f;
const float SH_C1 = 0.4886025119029199f;
const float SH_C2[5] = {1.0925484305920792f, -1.0925484305920792f,
                        0.31539156525252005f, -1.0925484305920792f,
                        0.5462742152960396f};
const float SH_C3[7] = {-0.5900435899266435f, 2.890611442640554f,
                        -0.4570457994644658f, 0.3731763325901154f,
                        -0.4570457994644658f, 1.445305721320277f,
                        -0.5900435899266435f};
const float SH_C4[9] = {2.5033429417967046f, -1.7701307697799304f,
                        0.9461746957575601f, -0.6690465435572892f,
                        0.10578554691520431f, -0.6690465435572892f,
                        0.47308734787878004f, -1.7701307697799304f,
                        0.6258357354491761f};
const float FILTER_SIZE = 0.707106f;   /* :204 */
const float FILTER_INV_SQ = 2.0f;      /* :206 */
const float NEAR_N = 0.2f;             /* :210 */
const float FAR_N = 100.0f;            /* :211 */
const int BLOCK = 16;

struct f3 { float x, y, z; };

inline float dot3(f3 a, f3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }
inline f3 mul3(f3 a, f3 b) { return {a.x * b.x, a.y * b.y, a.z * b.z}; }

int num_sh_bases(int degree) {  /* msplat_metal.metal:46-57 */
    if (degree == 0) return 1;
    if (degree == 1) return 4;
    if (degree == 2) return 9;
    if (degree == 3) return 16;
    return 25;
}

/* Saturating float -> int truncation (NaN -> INT_MIN before clamping to
 * the tile range).  The reference's (int) cast (msplat_metal.metal:70-73) is
 * undefined outside the int range; both implementations define it this way. */
inline int f2i(float x) {
    x = fmaxf(x, -2147483648.0f);
    x = fminf(x, 2147483520.0f);
    return (int)x;
}

/* quat_to_rotmat (msplat_metal.metal:116-136); returns the three columns. */
void quat_to_rotmat(const float *q, f3 &c0, f3 &c1, f3 &c2) {
    float s = 1.0f / sqrtf(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
    float w = q[0] * s, x = q[1] * s, y = q[2] * s, z = q[3] * s;
    c0 = {1.f - 2.f * (y * y + z * z), 2.f * (x * y + w * z), 2.f * (x * z - w * y)};
    c1 = {2.f * (x * y - w * z), 1.f - 2.f * (x * x + z * z), 2.f * (y * z + w * x)};
    c2 = {2.f * (x * z + w * y), 2.f * (y * z - w * x), 1.f - 2.f * (x * x + y * y)};
}

/* quat_to_rotmat_vjp (msplat_metal.metal:1252-1295); vR[c] is column c. */
void quat_to_rotmat_vjp(const float *q, const f3 vR[3], float out[4]) {
    float s = 1.0f / sqrtf(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
    float w = q[0] * s, x = q[1] * s, y = q[2] * s, z = q[3] * s;
    const float R00 = vR[0].x, R01 = vR[0].y, R02 = vR[0].z;
    const float R10 = vR[1].x, R11 = vR[1].y, R12 = vR[1].z;
    const float R20 = vR[2].x, R21 = vR[2].y, R22 = vR[2].z;
    out[0] = 2.f * (x * (R12 - R21) + y * (R20 - R02) + z * (R01 - R10));
    out[1] = 2.f * (-2.f * x * (R11 + R22) + y * (R01 + R10) + z * (R02 + R20) +
                    w * (R12 - R21));
    out[2] = 2.f * (x * (R01 + R10) - 2.f * y * (R00 + R22) + z * (R12 + R21) +
                    w * (R20 - R02));
    out[3] = 2.f * (x * (R02 + R20) + y * (R12 + R21) - 2.f * z * (R00 + R11) +
                    w * (R01 - R10));
}

/* Column u, v, o of the 2DGS homography (compute_transmat_2dgs,
 * msplat_metal.metal:226-295), shared by forward and backward. */
struct ClipCols {
    float tu[4], tv[4], pc[4];
};

ClipCols clip_columns(const float *p, f3 tu, f3 tv, const float *pm) {
    ClipCols c;
    for (int r = 0; r < 4; ++r) {
        c.tu[r] = pm[4 * r + 0] * tu.x + pm[4 * r + 1] * tu.y + pm[4 * r + 2] * tu.z;
        c.tv[r] = pm[4 * r + 0] * tv.x + pm[4 * r + 1] * tv.y + pm[4 * r + 2] * tv.z;
        c.pc[r] = pm[4 * r + 0] * p[0] + pm[4 * r + 1] * p[1] + pm[4 * r + 2] * p[2] +
                  pm[4 * r + 3];
    }
    return c;
}

/* sh_coeffs_to_color (msplat_metal.metal:756-823). */
void sh_eval(int degree, f3 d, const float *dc, const float *rest, float *col) {
    for (int c = 0; c < 3; ++c) col[c] = SH_C0 * dc[c];
    if (degree < 1) return;
    float x = d.x, y = d.y, z = d.z;
    float xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
    for (int c = 0; c < 3; ++c) {
        const float *r = rest;
        col[c] += SH_C1 * (-y * r[0 * 3 + c] + z * r[1 * 3 + c] - x * r[2 * 3 + c]);
        if (degree < 2) continue;
        col[c] += (SH_C2[0] * xy * r[3 * 3 + c] + SH_C2[1] * yz * r[4 * 3 + c] +
                   SH_C2[2] * (2.f * zz - xx - yy) * r[5 * 3 + c] +
                   SH_C2[3] * xz * r[6 * 3 + c] + SH_C2[4] * (xx - yy) * r[7 * 3 + c]);
        if (degree < 3) continue;
        col[c] += (SH_C3[0] * y * (3.f * xx - yy) * r[8 * 3 + c] +
                   SH_C3[1] * xy * z * r[9 * 3 + c] +
                   SH_C3[2] * y * (4.f * zz - xx - yy) * r[10 * 3 + c] +
                   SH_C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy) * r[11 * 3 + c] +
                   SH_C3[4] * x * (4.f * zz - xx - yy) * r[12 * 3 + c] +
                   SH_C3[5] * z * (xx - yy) * r[13 * 3 + c] +
                   SH_C3[6] * x * (xx - 3.f * yy) * r[14 * 3 + c]);
        if (degree < 4) continue;
        col[c] += (SH_C4[0] * xy * (xx - yy) * r[15 * 3 + c] +
                   SH_C4[1] * yz * (3.f * xx - yy) * r[16 * 3 + c] +
                   SH_C4[2] * xy * (7.f * zz - 1.f) * r[17 * 3 + c] +
                   SH_C4[3] * yz * (7.f * zz - 3.f) * r[18 * 3 + c] +
                   SH_C4[4] * (zz * (35.f * zz - 30.f) + 3.f) * r[19 * 3 + c] +
                   SH_C4[5] * xz * (7.f * zz - 3.f) * r[20 * 3 + c] +
                   SH_C4[6] * (xx - yy) * (7.f * zz - 1.f) * r[21 * 3 + c] +
                   SH_C4[7] * xz * (xx - 3.f * yy) * r[22 * 3 + c] +
                   SH_C4[8] * (xx * (xx - 3.f * yy) - yy * (3.f * xx - yy)) *
                       r[23 * 3 + c]);
    }
}

/* sh_coeffs_to_color_vjp (msplat_metal.metal:825-912). */
void sh_vjp(int degree, f3 d, const float *vc, float *vdc, float *vrest) {
    for (int c = 0; c < 3; ++c) vdc[c] = SH_C0 * vc[c];
    if (degree < 1) return;
    float x = d.x, y = d.y, z = d.z;
    float xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
    for (int c = 0; c < 3; ++c) {
        float v1 = -SH_C1 * y, v2 = SH_C1 * z, v3 = -SH_C1 * x;
        vrest[0 * 3 + c] = v1 * vc[c];
        vrest[1 * 3 + c] = v2 * vc[c];
        vrest[2 * 3 + c] = v3 * vc[c];
        if (degree < 2) continue;
        float v4 = SH_C2[0] * xy, v5 = SH_C2[1] * yz, v6 = SH_C2[2] * (2.f * zz - xx - yy);
        float v7 = SH_C2[3] * xz, v8 = SH_C2[4] * (xx - yy);
        vrest[3 * 3 + c] = v4 * vc[c];
        vrest[4 * 3 + c] = v5 * vc[c];
        vrest[5 * 3 + c] = v6 * vc[c];
        vrest[6 * 3 + c] = v7 * vc[c];
        vrest[7 * 3 + c] = v8 * vc[c];
        if (degree < 3) continue;
        float v9 = SH_C3[0] * y * (3.f * xx - yy);
        float v10 = SH_C3[1] * xy * z;
        float v11 = SH_C3[2] * y * (4.f * zz - xx - yy);
        float v12 = SH_C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy);
        float v13 = SH_C3[4] * x * (4.f * zz - xx - yy);
        float v14 = SH_C3[5] * z * (xx - yy);
        float v15 = SH_C3[6] * x * (xx - 3.f * yy);
        vrest[8 * 3 + c] = v9 * vc[c];
        vrest[9 * 3 + c] = v10 * vc[c];
        vrest[10 * 3 + c] = v11 * vc[c];
        vrest[11 * 3 + c] = v12 * vc[c];
        vrest[12 * 3 + c] = v13 * vc[c];
        vrest[13 * 3 + c] = v14 * vc[c];
        vrest[14 * 3 + c] = v15 * vc[c];
        if (degree < 4) continue;
        float v16 = SH_C4[0] * xy * (xx - yy);
        float v17 = SH_C4[1] * yz * (3.f * xx - yy);
        float v18 = SH_C4[2] * xy * (7.f * zz - 1.f);
        float v19 = SH_C4[3] * yz * (7.f * zz - 3.f);
        float v20 = SH_C4[4] * (zz * (35.f * zz - 30.f) + 3.f);
        float v21 = SH_C4[5] * xz * (7.f * zz - 3.f);
        float v22 = SH_C4[6] * (xx - yy) * (7.f * zz - 1.f);
        float v23 = SH_C4[7] * xz * (xx - 3.f * yy);
        float v24 = SH_C4[8] * (xx * (xx - 3.f * yy) - yy * (3.f * xx - yy));
        vrest[15 * 3 + c] = v16 * vc[c];
        vrest[16 * 3 + c] = v17 * vc[c];
        vrest[17 * 3 + c] = v18 * vc[c];
        vrest[18 * 3 + c] = v19 * vc[c];
        vrest[19 * 3 + c] = v20 * vc[c];
        vrest[20 * 3 + c] = v21 * vc[c];
        vrest[21 * 3 + c] = v22 * vc[c];
        vrest[22 * 3 + c] = v23 * vc[c];
        vrest[23 * 3 + c] = v24 * vc[c];
    }
}

/* sh_color_dL_ddir (msplat_metal.metal:925-1013); degree-4 terms are not
 * part of the reference's view-direction gradient. */
f3 sh_dL_ddir(int degree, f3 d, const float *fr, const float *vc) {
    if (degree < 1) return {0.f, 0.f, 0.f};
    const float x = d.x, y = d.y, z = d.z;
    float dx[3], dy[3], dz[3];
    for (int c = 0; c < 3; ++c) {
        dx[c] = -SH_C1 * fr[2 * 3 + c];
        dy[c] = -SH_C1 * fr[0 * 3 + c];
        dz[c] = SH_C1 * fr[1 * 3 + c];
    }
    if (degree >= 2) {
        const float xx = x * x, yy = y * y, zz = z * z;
        for (int c = 0; c < 3; ++c) {
            const float s4 = fr[3 * 3 + c], s5 = fr[4 * 3 + c], s6 = fr[5 * 3 + c];
            const float s7 = fr[6 * 3 + c], s8 = fr[7 * 3 + c];
            dx[c] += SH_C2[0] * y * s4 + SH_C2[2] * (-2.f * x) * s6 + SH_C2[3] * z * s7 +
                     SH_C2[4] * (2.f * x) * s8;
            dy[c] += SH_C2[0] * x * s4 + SH_C2[1] * z * s5 + SH_C2[2] * (-2.f * y) * s6 +
                     SH_C2[4] * (-2.f * y) * s8;
            dz[c] += SH_C2[1] * y * s5 + SH_C2[2] * (4.f * z) * s6 + SH_C2[3] * x * s7;
        }
        if (degree >= 3) {
            for (int c = 0; c < 3; ++c) {
                const float s9 = fr[8 * 3 + c], s10 = fr[9 * 3 + c], s11 = fr[10 * 3 + c];
                const float s12 = fr[11 * 3 + c], s13 = fr[12 * 3 + c];
                const float s14 = fr[13 * 3 + c], s15 = fr[14 * 3 + c];
                dx[c] += SH_C3[0] * s9 * (6.f * x * y) + SH_C3[1] * s10 * (y * z) +
                         SH_C3[2] * s11 * (-2.f * x * y) + SH_C3[3] * s12 * (-6.f * x * z) +
                         SH_C3[4] * s13 * (-3.f * xx + 4.f * zz - yy) +
                         SH_C3[5] * s14 * (2.f * x * z) + SH_C3[6] * s15 * (3.f * (xx - yy));
                dy[c] += SH_C3[0] * s9 * (3.f * (xx - yy)) + SH_C3[1] * s10 * (x * z) +
                         SH_C3[2] * s11 * (-3.f * yy + 4.f * zz - xx) +
                         SH_C3[3] * s12 * (-6.f * y * z) + SH_C3[4] * s13 * (-2.f * x * y) +
                         SH_C3[5] * s14 * (-2.f * y * z) + SH_C3[6] * s15 * (-6.f * x * y);
                dz[c] += SH_C3[1] * s10 * (x * y) + SH_C3[2] * s11 * (8.f * y * z) +
                         SH_C3[3] * s12 * (3.f * (2.f * zz - xx - yy)) +
                         SH_C3[4] * s13 * (8.f * x * z) + SH_C3[5] * s14 * (xx - yy);
            }
        }
    }
    f3 r = {0.f, 0.f, 0.f};
    for (int c = 0; c < 3; ++c) {
        r.x += dx[c] * vc[c];
        r.y += dy[c] * vc[c];
        r.z += dz[c] * vc[c];
    }
    return r;
}

/* dnormvdv (msplat_metal.metal:1017-1025). */
f3 dnormvdv(f3 v, f3 dv) {
    float sum2 = v.x * v.x + v.y * v.y + v.z * v.z;
    float invsum32 = 1.0f / sqrtf(sum2 * sum2 * sum2);
    return {((sum2 - v.x * v.x) * dv.x - v.y * v.x * dv.y - v.z * v.x * dv.z) * invsum32,
            (-v.x * v.y * dv.x + (sum2 - v.y * v.y) * dv.y - v.z * v.y * dv.z) * invsum32,
            (-v.x * v.z * dv.x - v.y * v.z * dv.y + (sum2 - v.z * v.z) * dv.z) * invsum32};
}

inline f3 normalize3(f3 v) {
    float inv = 1.0f / sqrtf(v.x * v.x + v.y * v.y + v.z * v.z);
    return {v.x * inv, v.y * inv, v.z * inv};
}

inline float sigmoid(float x) { return 1.0f / (1.0f + orc_expf(-x)); }

/* Ray-splat evaluation shared by the rasterizer forward and backward
 * (msplat_metal.metal:663-701).  Returns false when the pair is skipped. */
struct PairEval {
    f3 k, l, ray;
    float u, v, rho3d, rho2d, dxs, dys, depth, G, alpha;
};

inline f3 cross3(f3 a, f3 b) {
    return {a.y * b.z - a.z * b.y, a.z * b.x - a.x * b.z, a.x * b.y - a.y * b.x};
}

/* The reference builds k = px Tw - Tu, l = py Tw - Tv and the ray k x l per
 * pixel (msplat_metal.metal:655-658).  The same ray expanded about the splat
 * centre (xs, ys): ray = R0 + (xs - px) nAx + (ys - py) nAy with
 * kc = xs Tw - Tu, lc = ys Tw - Tv, R0 = kc x lc, nAx = lc x Tw,
 * nAy = Tw x kc (the (px - xs)(py - ys) term is Tw x Tw = 0).  Exact in real
 * arithmetic, every term at the splat's own scale; C = (R0, nAx, nAy) once
 * per splat, by the kernels' operations (centred_rows). */
inline void centred_rows(const float *Tm, const float *xy, float *C) {
    const f3 Tu = {Tm[0], Tm[1], Tm[2]}, Tv = {Tm[3], Tm[4], Tm[5]},
             Tw = {Tm[6], Tm[7], Tm[8]};
    const float xs = xy[0], ys = xy[1];
    const f3 kc = {fmaf(xs, Tw.x, -Tu.x), fmaf(xs, Tw.y, -Tu.y), fmaf(xs, Tw.z, -Tu.z)};
    const f3 lc = {fmaf(ys, Tw.x, -Tv.x), fmaf(ys, Tw.y, -Tv.y), fmaf(ys, Tw.z, -Tv.z)};
    const f3 R0 = cross3(kc, lc), nAx = cross3(lc, Tw), nAy = cross3(Tw, kc);
    const float v[9] = {R0.x, R0.y, R0.z, nAx.x, nAx.y, nAx.z, nAy.x, nAy.y, nAy.z};
    for (int k = 0; k < 9; ++k) C[k] = v[k];
}

/* centred_rows of every splat a tile list names. */
static std::vector<float> all_centred_rows(int64_t I, const int32_t *ids, const float *xys,
                                           const float *transmats) {
    int32_t n = 0;
    for (int64_t j = 0; j < I; ++j) n = ids[j] + 1 > n ? ids[j] + 1 : n;
    std::vector<float> C((size_t)n * 9);
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < n; ++g) centred_rows(transmats + 9 * (size_t)g, xys + 2 * (size_t)g, C.data() + 9 * (size_t)g);
    return C;
}

/* One (pixel, splat) evaluation of nd_rasterize_forward_2dgs_kernel
 * (msplat_metal.metal:651-683) on the centred ray; k and l (the reference's
 * per-pixel planes) are kept for the backward's transMat gradients. */
inline bool eval_pair(float px, float py, const float *C, const float *Tm, const float *xy,
                      float opac, PairEval &e) {
    const f3 Tu = {Tm[0], Tm[1], Tm[2]}, Tv = {Tm[3], Tm[4], Tm[5]},
             Tw = {Tm[6], Tm[7], Tm[8]};
    e.k = {fmaf(px, Tw.x, -Tu.x), fmaf(px, Tw.y, -Tu.y), fmaf(px, Tw.z, -Tu.z)};
    e.l = {fmaf(py, Tw.x, -Tv.x), fmaf(py, Tw.y, -Tv.y), fmaf(py, Tw.z, -Tv.z)};
    e.dxs = xy[0] - px;
    e.dys = xy[1] - py;
    e.ray = {fmaf(e.dxs, C[3], fmaf(e.dys, C[6], C[0])), fmaf(e.dxs, C[4], fmaf(e.dys, C[7], C[1])),
             fmaf(e.dxs, C[5], fmaf(e.dys, C[8], C[2]))};
    if (e.ray.z == 0.0f) return false;
    const float inv_z = 1.0f / e.ray.z;
    e.u = e.ray.x * inv_z;
    e.v = e.ray.y * inv_z;
    e.rho3d = fmaf(e.u, e.u, e.v * e.v);
    e.rho2d = FILTER_INV_SQ * fmaf(e.dxs, e.dxs, e.dys * e.dys);
    const float rho = fminf(e.rho3d, e.rho2d);
    e.depth = fmaf(e.u, Tw.x, fmaf(e.v, Tw.y, Tw.z));
    if (e.depth < NEAR_N) return false;
    /* The reference's power > 0 rejection (msplat_metal.metal:676-677) never
     * fires: rho is a minimum of sums of squares (>= 0, +inf or NaN), so
     * -rho / 2 is <= 0, -inf or NaN. */
    e.G = orc_gauss(rho);
    e.alpha = fminf(0.99f, opac * e.G);
    if (e.alpha < 1.0f / 255.0f) return false;
    return true;
}

/* The SSIM window: exp(-(x-5)^2 / (2*1.5^2)) normalised (the table at
 * msplat_metal.metal:2804-2816 holds these values to 12 digits). */
void ssim_window(float w[11]) {
    double g[11], s = 0.0;
    for (int i = 0; i < 11; ++i) {
        double d = i - 5.0;
        g[i] = std::exp(-d * d / (2.0 * 1.5 * 1.5));
        s += g[i];
    }
    for (int i = 0; i < 11; ++i) w[i] = (float)(g[i] / s);
}

/* ssim_blur_horiz_kernel / ssim_blur_vert_kernel (msplat_metal.metal:2847-2903)
 * on a [H,W,3] image, zero padding, taps accumulated k = -5..5 in order. */
void blur_h(int W, int H, const float *in, float *out, const float *w) {
#pragma omp parallel for schedule(static)
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x)
            for (int c = 0; c < 3; ++c) {
                float acc = 0.f;
                for (int k = -5; k <= 5; ++k) {
                    int xs = x + k;
                    if (xs < 0 || xs >= W) continue;
                    acc = fmaf(w[k + 5], in[((size_t)y * W + xs) * 3 + c], acc);
                }
                out[((size_t)y * W + x) * 3 + c] = acc;
            }
}

void blur_v(int W, int H, const float *in, float *out, const float *w) {
#pragma omp parallel for schedule(static)
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x)
            for (int c = 0; c < 3; ++c) {
                float acc = 0.f;
                for (int k = -5; k <= 5; ++k) {
                    int ys = y + k;
                    if (ys < 0 || ys >= H) continue;
                    acc = fmaf(w[k + 5], in[((size_t)ys * W + x) * 3 + c], acc);
                }
                out[((size_t)y * W + x) * 3 + c] = acc;
            }
}

void blur_hv(int W, int H, const float *in, float *out, float *tmp, const float *w) {
    blur_h(W, H, in, tmp, w);
    blur_v(W, H, tmp, out, w);
}

}  // namespace

/* ------------------------------------------------------------------------ */

extern "C" int orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

/* Cephes-style single-precision exp (S. L. Moshier, Cephes Math Library,
 * expf.c): Cody-Waite reduction x = k*ln2 + r with ln2 split as
 * 0.693359375 - 2.12194440e-4, a degree-7 polynomial for e^r on
 * [-ln2/2, ln2/2], then an exact two-step scaling by 2^k. */
extern "C" float orc_expf(float x) {
    if (x != x) return x;
    if (x > 88.72283905206835f) return INFINITY;
    if (x < -103.97208f) return 0.0f;
    float z = rintf(x * 1.44269504088896341f);
    float r = fmaf(z, -0.693359375f, x);
    r = fmaf(z, 2.12194440e-4f, r);
    float r2 = r * r;
    float p = 1.9875691500E-4f;
    p = fmaf(p, r, 1.3981999507E-3f);
    p = fmaf(p, r, 8.3334519073E-3f);
    p = fmaf(p, r, 4.1665795894E-2f);
    p = fmaf(p, r, 1.6666665459E-1f);
    p = fmaf(p, r, 5.0000001201E-1f);
    p = fmaf(p, r2, r);
    p = p + 1.0f;
    int k = (int)z;
    int k1 = k / 2;
    int k2 = k - k1;
    uint32_t b1 = (uint32_t)(k1 + 127) << 23, b2 = (uint32_t)(k2 + 127) << 23;
    float s1, s2;
    memcpy(&s1, &b1, 4);
    memcpy(&s2, &b2, 4);
    return (p * s1) * s2;
}

/* The rasterizer's Gaussian falloff exp(-rho / 2), rho >= 0:
 * t = rho * (-log2(e) / 2) with one rounding (log2(e) as a float, halved
 * exactly), clamped at -124 (NaN becomes -124), z = rint(t), f = t - z
 * (exact), 2^f as the degree-6 Taylor polynomial of e^(f ln 2) on
 * [-1/2, 1/2] (truncation error below 1.2e-7 relative), then ldexp(., z).
 * The same IEEE operations as the kernels' ms_gauss, so both agree bit for
 * bit; within 8 ulp of exp (the rounding of t dominates), never below
 * 4e-38. */
extern "C" float orc_gauss(float rho) {
    const float t = fmaxf(rho * -0.721347510814666748046875f, -124.0f);
    const float z = rintf(t);
    const float f = t - z;
    float p = 1.5403530393381606e-4f;
    p = fmaf(p, f, 1.3333558146428443e-3f);
    p = fmaf(p, f, 9.6181291076284772e-3f);
    p = fmaf(p, f, 5.5504108664821580e-2f);
    p = fmaf(p, f, 2.4022650695910071e-1f);
    p = fmaf(p, f, 6.9314718055994531e-1f);
    p = fmaf(p, f, 1.0f);
    return ldexpf(p, (int)z);
}

extern "C" void orc_gauss_array(int64_t n, const float *rho, float *y) {
    for (int64_t i = 0; i < n; ++i) y[i] = orc_gauss(rho[i]);
}

/* Model::prepareCam (core/src/model.cpp:500-544). */
extern "C" void orc_prepare_cam(const float *d, float fx, float fy, float cx, float cy,
                                int width, int height, OrcCamera *o) {
    float fovX = 2.0f * std::atan(width / (2.0f * fx));
    float fovY = 2.0f * std::atan(height / (2.0f * fy));
    float R[3][3], Rinv[3][3], T[3], Tinv[3];
    for (int i = 0; i < 3; i++) {
        R[i][0] = d[i * 4 + 0];
        R[i][1] = -d[i * 4 + 1];
        R[i][2] = -d[i * 4 + 2];
        T[i] = d[i * 4 + 3];
    }
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) Rinv[i][j] = R[j][i];
    for (int i = 0; i < 3; i++)
        Tinv[i] = -(Rinv[i][0] * T[0] + Rinv[i][1] * T[1] + Rinv[i][2] * T[2]);
    float vm[16] = {Rinv[0][0], Rinv[0][1], Rinv[0][2], Tinv[0],
                    Rinv[1][0], Rinv[1][1], Rinv[1][2], Tinv[1],
                    Rinv[2][0], Rinv[2][1], Rinv[2][2], Tinv[2],
                    0, 0, 0, 1};
    float t_p = 0.001f * std::tan(0.5f * fovY), r_p = 0.001f * std::tan(0.5f * fovX);
    float pm[16] = {0.001f / r_p, 0, 0, 0,
                    0, 0.001f / t_p, 0, 0,
                    0, 0, (1000.0f + 0.001f) / (1000.0f - 0.001f),
                    -1000.0f * 0.001f / (1000.0f - 0.001f),
                    0, 0, 1, 0};
    float pvm[16] = {};
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int k = 0; k < 4; k++) pvm[i * 4 + j] += pm[i * 4 + k] * vm[k * 4 + j];
    memcpy(o->viewmat, vm, sizeof(vm));
    memcpy(o->projmat, pvm, sizeof(pvm));
    o->cam_pos[0] = T[0];
    o->cam_pos[1] = T[1];
    o->cam_pos[2] = T[2];
    o->fx = fx;
    o->fy = fy;
    o->cx = cx;
    o->cy = cy;
    o->width = width;
    o->height = height;
    o->tiles_x = (width + BLOCK - 1) / BLOCK;
    o->tiles_y = (height + BLOCK - 1) / BLOCK;
}

/* project_and_sh_forward_2dgs_kernel (msplat_metal.metal:1413-1521) with
 * compute_transmat_2dgs (:226-295), compute_aabb_2dgs (:302-330),
 * get_tile_bbox (:62-92) and sh_coeffs_to_color (:756-823). */
extern "C" void orc_project_fwd(int n, const float *means, const float *scales,
                                const float *quats, const float *opacities,
                                const float *fdc, const float *frest, int degree,
                                int dtu, const OrcCamera *cam, float glob_scale,
                                float clip_thresh, float *xys, float *depths,
                                int32_t *radii, float *transmats, float *normal_opac,
                                float *colors, int32_t *tiles_hit, int32_t *rect) {
    const float *vm = cam->viewmat, *pm = cam->projmat;
    const int nb = num_sh_bases(degree);
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        radii[i] = 0;
        tiles_hit[i] = 0;
        xys[2 * i] = xys[2 * i + 1] = 0.f;
        depths[i] = 0.f;
        for (int k = 0; k < 9; ++k) transmats[9 * i + k] = 0.f;
        for (int k = 0; k < 4; ++k) normal_opac[4 * i + k] = 0.f;
        for (int k = 0; k < 3; ++k) colors[3 * i + k] = 0.f;
        for (int k = 0; k < 4; ++k) rect[4 * i + k] = 0;

        const float *p = means + 3 * i;
        float pz = vm[8] * p[0] + vm[9] * p[1] + vm[10] * p[2] + vm[11];
        if (pz <= clip_thresh) continue;

        float sx = orc_expf(scales[2 * i]), sy = orc_expf(scales[2 * i + 1]);
        f3 R0, R1, R2;
        quat_to_rotmat(quats + 4 * i, R0, R1, R2);
        const float sxg = sx * glob_scale, syg = sy * glob_scale;
        f3 tu = {R0.x * sxg, R0.y * sxg, R0.z * sxg};
        f3 tv = {R1.x * syg, R1.y * syg, R1.z * syg};
        ClipCols cc = clip_columns(p, tu, tv, pm);
        const float halfW = 0.5f * (float)cam->width, halfH = 0.5f * (float)cam->height;
        const float bx = cam->cx - 0.5f, by = cam->cy - 0.5f;
        f3 cu = {halfW * cc.tu[0] + bx * cc.tu[3], halfH * cc.tu[1] + by * cc.tu[3], cc.tu[3]};
        f3 cv = {halfW * cc.tv[0] + bx * cc.tv[3], halfH * cc.tv[1] + by * cc.tv[3], cc.tv[3]};
        f3 co = {halfW * cc.pc[0] + bx * cc.pc[3], halfH * cc.pc[1] + by * cc.pc[3], cc.pc[3]};
        f3 T0 = {cu.x, cv.x, co.x}, T1 = {cu.y, cv.y, co.y}, T2 = {cu.z, cv.z, co.z};

        /* compute_aabb_2dgs with cutoff 3 */
        const float cutoff = 3.0f;
        f3 t = {cutoff * cutoff, cutoff * cutoff, -1.0f};
        float dd = dot3(t, mul3(T2, T2));
        if (dd == 0.0f) continue;
        float invd = 1.0f / dd;
        f3 f = {invd * t.x, invd * t.y, invd * t.z};
        float cxp = dot3(f, mul3(T0, T2)), cyp = dot3(f, mul3(T1, T2));
        float h0x = cxp * cxp - dot3(f, mul3(T0, T0));
        float h0y = cyp * cyp - dot3(f, mul3(T1, T1));
        float hx = sqrtf(fmaxf(1e-4f, h0x)), hy = sqrtf(fmaxf(1e-4f, h0y));
        float radius = ceilf(fmaxf(fmaxf(hx, hy), cutoff * FILTER_SIZE));

        float tcx = cxp / (float)BLOCK, tcy = cyp / (float)BLOCK;
        float tr = radius / (float)BLOCK;
        int x0 = std::min(std::max(0, f2i(tcx - tr)), cam->tiles_x);
        int x1 = std::min(std::max(0, f2i(tcx + tr + 1)), cam->tiles_x);
        int y0 = std::min(std::max(0, f2i(tcy - tr)), cam->tiles_y);
        int y1 = std::min(std::max(0, f2i(tcy + tr + 1)), cam->tiles_y);
        int area = (x1 - x0) * (y1 - y0);
        if (area <= 0) continue;

        tiles_hit[i] = area;
        depths[i] = pz;
        radii[i] = (int)radius;
        xys[2 * i] = cxp;
        xys[2 * i + 1] = cyp;
        rect[4 * i + 0] = x0;
        rect[4 * i + 1] = y0;
        rect[4 * i + 2] = x1;
        rect[4 * i + 3] = y1;
        float *tm = transmats + 9 * i;
        tm[0] = T0.x; tm[1] = T0.y; tm[2] = T0.z;
        tm[3] = T1.x; tm[4] = T1.y; tm[5] = T1.z;
        tm[6] = T2.x; tm[7] = T2.y; tm[8] = T2.z;
        normal_opac[4 * i + 0] = R2.x;
        normal_opac[4 * i + 1] = R2.y;
        normal_opac[4 * i + 2] = R2.z;
        normal_opac[4 * i + 3] = opacities[i];
        f3 dir = normalize3({p[0] - cam->cam_pos[0], p[1] - cam->cam_pos[1],
                             p[2] - cam->cam_pos[2]});
        sh_eval(dtu, dir, fdc + 3 * i, frest + (size_t)(nb - 1) * 3 * i, colors + 3 * i);
    }
}

extern "C" int64_t orc_count_tiles(int n, const int32_t *radii, const int32_t *rect,
                                   int tiles_x, int tiles_y, int32_t *tile_counts) {
    const int T = tiles_x * tiles_y;
    std::fill(tile_counts, tile_counts + T, 0);
    int64_t total = 0;
    for (int i = 0; i < n; ++i) {
        if (radii[i] <= 0) continue;
        const int32_t *r = rect + 4 * i;
        for (int y = r[1]; y < r[3]; ++y)
            for (int x = r[0]; x < r[2]; ++x) {
                tile_counts[y * tiles_x + x]++;
                ++total;
            }
    }
    return total;
}

extern "C" void orc_bin_sort(int n, const int32_t *radii, const int32_t *rect,
                             const float *depths, int tiles_x, int tiles_y,
                             const int32_t *tile_counts, int32_t *tile_offsets,
                             uint64_t *keys, int32_t *ids) {
    const int T = tiles_x * tiles_y;
    tile_offsets[0] = 0;
    for (int t = 0; t < T; ++t) tile_offsets[t + 1] = tile_offsets[t] + tile_counts[t];
    std::vector<int32_t> cursor(tile_offsets, tile_offsets + T);
    for (int i = 0; i < n; ++i) {
        if (radii[i] <= 0) continue;
        uint32_t db;
        memcpy(&db, depths + i, 4);
        const int32_t *r = rect + 4 * i;
        for (int y = r[1]; y < r[3]; ++y)
            for (int x = r[0]; x < r[2]; ++x)
                keys[cursor[y * tiles_x + x]++] = ((uint64_t)db << 32) | (uint32_t)i;
    }
#pragma omp parallel for schedule(dynamic, 16)
    for (int t = 0; t < T; ++t) {
        std::sort(keys + tile_offsets[t], keys + tile_offsets[t + 1]);
        for (int j = tile_offsets[t]; j < tile_offsets[t + 1]; ++j)
            ids[j] = (int32_t)(keys[j] & 0xFFFFFFFFu);
    }
}

/* nd_rasterize_forward_2dgs_kernel (msplat_metal.metal:553-754). */
extern "C" void orc_raster_fwd(const OrcCamera *cam, const int32_t *tile_offsets,
                               const int32_t *ids, const float *xys,
                               const float *transmats, const float *normal_opac,
                               const float *colors, const float *bg, float *out_img,
                               float *final_Ts, int32_t *final_index, float *out_depth,
                               float *out_normal, float *out_alpha,
                               float *out_median_depth, float *out_distortion,
                               int64_t *pairs_evaluated) {
    const int W = cam->width, H = cam->height, TX = cam->tiles_x;
    const float mscale = FAR_N / (FAR_N - NEAR_N);
    const std::vector<float> crow = all_centred_rows(tile_offsets[TX * cam->tiles_y], ids, xys, transmats);
    int64_t pairs = 0;
#pragma omp parallel for schedule(dynamic, 4) reduction(+ : pairs)
    for (int py_i = 0; py_i < H; ++py_i) {
        for (int px_i = 0; px_i < W; ++px_i) {
            const int tile = (py_i / BLOCK) * TX + (px_i / BLOCK);
            const float px = (float)px_i, py = (float)py_i;
            float T = 1.f, cr = 0.f, cg = 0.f, cb = 0.f, dep = 0.f;
            float nx = 0.f, ny = 0.f, nz = 0.f;
            float M1 = 0.f, M2 = 0.f, distortion = 0.f, median_depth = 0.f;
            int median_contrib = -1, contributor = 0, last_contrib = 0;
            for (int j = tile_offsets[tile]; j < tile_offsets[tile + 1]; ++j) {
                contributor++;
                const int g = ids[j];
                const float *no = normal_opac + 4 * g;
                const float opac = sigmoid(no[3]);
                PairEval e;
                if (!eval_pair(px, py, crow.data() + 9 * (size_t)g, transmats + 9 * g, xys + 2 * g, opac, e)) continue;
                const float next_T = T * (1.0f - e.alpha);
                if (next_T <= 1e-4f) break;
                const float w = e.alpha * T;
                const float A = 1.f - T;
                const float m = mscale * (1.f - NEAR_N / e.depth);
                distortion = fmaf(m * m * A + M2 - 2.f * m * M1, w, distortion);
                M1 = fmaf(m, w, M1);
                M2 = fmaf(m * m, w, M2);
                if (T > 0.5f) {
                    median_depth = e.depth;
                    median_contrib = contributor;
                }
                const float *c = colors + 3 * g;
                cr = fmaf(fmaxf(c[0] + 0.5f, 0.0f), w, cr);
                cg = fmaf(fmaxf(c[1] + 0.5f, 0.0f), w, cg);
                cb = fmaf(fmaxf(c[2] + 0.5f, 0.0f), w, cb);
                dep = fmaf(e.depth, w, dep);
                nx = fmaf(no[0], w, nx);
                ny = fmaf(no[1], w, ny);
                nz = fmaf(no[2], w, nz);
                T = next_T;
                last_contrib = contributor;
            }
            pairs += contributor;
            const size_t pix = (size_t)py_i * W + px_i;
            final_Ts[3 * pix + 0] = T;
            final_Ts[3 * pix + 1] = M1;
            final_Ts[3 * pix + 2] = M2;
            final_index[2 * pix + 0] = last_contrib;
            final_index[2 * pix + 1] = median_contrib;
            out_img[3 * pix + 0] = fmaf(bg[0], T, cr);
            out_img[3 * pix + 1] = fmaf(bg[1], T, cg);
            out_img[3 * pix + 2] = fmaf(bg[2], T, cb);
            out_depth[pix] = dep;
            out_normal[3 * pix + 0] = nx;
            out_normal[3 * pix + 1] = ny;
            out_normal[3 * pix + 2] = nz;
            out_alpha[pix] = 1.f - T;
            out_median_depth[pix] = median_depth;
            out_distortion[pix] = distortion;
        }
    }
    if (pairs_evaluated) *pairs_evaluated = pairs;
}

/* SSIM + L1 (+distortion) loss forward/backward: msplat_metal.metal:2704-3085
 * in the dispatch order of msplat_metal.mm:1077-1212. */
extern "C" double orc_loss_fwd_bwd(int W, int H, const float *img, const float *gt,
                                   const float *distortion, float lambda_l1,
                                   float lambda_dist, float lambda_dssim,
                                   float *dL_dimg, float *dL_ddist, double *ssim_sum_out) {
    const size_t P = (size_t)W * H, E = P * 3;
    const float inv_np = 1.0f / (float)((unsigned)H * (unsigned)W * 3u);
    const float inv_HW = inv_np * 3.0f;
    float w[11];
    ssim_window(w);

    std::vector<float> prod(E), mu1(E), mu2(E), b11(E), b22(E), b12(E), tmp(E);
    blur_hv(W, H, img, mu1.data(), tmp.data(), w);
    blur_hv(W, H, gt, mu2.data(), tmp.data(), w);
    for (size_t i = 0; i < E; ++i) prod[i] = img[i] * img[i];
    blur_hv(W, H, prod.data(), b11.data(), tmp.data(), w);
    for (size_t i = 0; i < E; ++i) prod[i] = gt[i] * gt[i];
    blur_hv(W, H, prod.data(), b22.data(), tmp.data(), w);
    for (size_t i = 0; i < E; ++i) prod[i] = img[i] * gt[i];
    blur_hv(W, H, prod.data(), b12.data(), tmp.data(), w);

    const float C1 = 0.0001f, C2 = 0.0009f;
    const float g = -lambda_dssim * inv_np;
    std::vector<float> gmu1(E), gs1(E), gs12(E);
    double ssim_sum = 0.0;
    for (size_t i = 0; i < E; ++i) {
        float m1 = mu1[i], m2 = mu2[i];
        float m1_sq = m1 * m1, m2_sq = m2 * m2, m1m2 = m1 * m2;
        float s1_sq = b11[i] - m1_sq, s2_sq = b22[i] - m2_sq, s12 = b12[i] - m1m2;
        float A = 2.0f * m1m2 + C1, B = 2.0f * s12 + C2;
        float Cd = m1_sq + m2_sq + C1, Dd = s1_sq + s2_sq + C2;
        float val = (A * B) / (Cd * Dd);
        ssim_sum += (double)val;
        /* ssim_backward_compute_kernel (msplat_metal.metal:2965-3047) */
        float CD = Cd * Dd, AB = A * B;
        float inv_CD = 1.0f / CD, inv_Cd = 1.0f / Cd, inv_Dd = 1.0f / Dd;
        float dmu1 = 2.0f * inv_CD * (m2 * B - m1 * AB * inv_Cd);
        float ds12 = 2.0f * A * inv_CD;
        float ds1 = -AB * inv_CD * inv_Dd;
        float gm = g * dmu1, g12 = g * ds12, g1 = g * ds1;
        gm += g1 * (-2.0f * m1);
        gm += g12 * (-m2);
        gmu1[i] = gm;
        gs1[i] = g1;
        gs12[i] = g12;
    }
    std::vector<float> bgm(E), bg1(E), bg12(E);
    blur_hv(W, H, gmu1.data(), bgm.data(), tmp.data(), w);
    blur_hv(W, H, gs1.data(), bg1.data(), tmp.data(), w);
    blur_hv(W, H, gs12.data(), bg12.data(), tmp.data(), w);

    /* loss_l1_distortion_2dgs_kernel (msplat_metal.metal:2704-2762) */
    double loss = 0.0;
    for (size_t p = 0; p < P; ++p) {
        float local = 0.0f;
        for (int c = 0; c < 3; ++c) {
            float diff = img[3 * p + c] - gt[3 * p + c];
            local += lambda_l1 * fabsf(diff) * inv_np;
            float sgn = (diff > 0.0f) ? 1.0f : ((diff < 0.0f) ? -1.0f : 0.0f);
            dL_dimg[3 * p + c] = lambda_l1 * sgn * inv_np;
        }
        float dist = distortion ? distortion[p] : 0.0f;
        local += lambda_dist * dist * inv_HW;
        if (dL_ddist) dL_ddist[p] = lambda_dist * inv_HW;
        loss += (double)local;
    }
    loss += (double)lambda_dssim * (1.0 - ssim_sum * (double)inv_np);

    /* ssim_backward_accumulate_kernel (msplat_metal.metal:3059-3085) */
    for (size_t i = 0; i < E; ++i) {
        float a = img[i], b = gt[i];
        float contrib = bgm[i] + 2.0f * a * bg1[i] + b * bg12[i];
        dL_dimg[i] += contrib;
    }
    if (ssim_sum_out) *ssim_sum_out = ssim_sum;
    return loss;
}

/* nd_rasterize_backward_2dgs_kernel (msplat_metal.metal:1705-1979). */
extern "C" void orc_raster_bwd(const OrcCamera *cam, int n, const int32_t *tile_offsets,
                               const int32_t *ids, const float *xys,
                               const float *transmats, const float *normal_opac,
                               const float *colors, const float *bg,
                               const float *final_Ts, const int32_t *final_index,
                               const float *dL_dimg, const float *dL_ddepth,
                               const float *dL_daccum, const float *dL_dnormal,
                               const float *dL_dmedian, const float *dL_dreg_map,
                               float *grads, float *grads_abs) {
    const int W = cam->width, H = cam->height, TX = cam->tiles_x, TY = cam->tiles_y;
    const int T_tiles = TX * TY;
    const int64_t I = tile_offsets[T_tiles];
    std::vector<double> acc((size_t)I * 16, 0.0);
    /* grads_abs (nullable): per component the sum of the magnitudes of every
     * summand that went into it, the scale of a floating-point summation's
     * rounding error (test instrumentation; not part of the reference) */
    std::vector<double> acc_abs(grads_abs ? (size_t)I * 16 : 0, 0.0);
    const float mscale = FAR_N / (FAR_N - NEAR_N);
    const std::vector<float> crow = all_centred_rows(I, ids, xys, transmats);

#pragma omp parallel for schedule(dynamic, 1)
    for (int tile = 0; tile < T_tiles; ++tile) {
        const int ty = tile / TX, tx = tile % TX;
        const int start = tile_offsets[tile];
        for (int ly = 0; ly < BLOCK; ++ly)
            for (int lx = 0; lx < BLOCK; ++lx) {
                const int py_i = ty * BLOCK + ly, px_i = tx * BLOCK + lx;
                if (py_i >= H || px_i >= W) continue;
                const size_t pix = (size_t)py_i * W + px_i;
                const float px = (float)px_i, py = (float)py_i;
                const float T_final = final_Ts[3 * pix + 0];
                const float final_D = final_Ts[3 * pix + 1];
                const float final_D2 = final_Ts[3 * pix + 2];
                const float final_A = 1.0f - T_final;
                const int last_contrib = final_index[2 * pix + 0];
                const int median_contrib = final_index[2 * pix + 1];
                const float dpix[3] = {dL_dimg[3 * pix], dL_dimg[3 * pix + 1],
                                       dL_dimg[3 * pix + 2]};
                const float ddepth = dL_ddepth ? dL_ddepth[pix] : 0.f;
                const float daccum = dL_daccum ? dL_daccum[pix] : 0.f;
                const float dn2[3] = {dL_dnormal ? dL_dnormal[3 * pix] : 0.f,
                                      dL_dnormal ? dL_dnormal[3 * pix + 1] : 0.f,
                                      dL_dnormal ? dL_dnormal[3 * pix + 2] : 0.f};
                const float dmed = dL_dmedian ? dL_dmedian[pix] : 0.f;
                const float dreg = dL_dreg_map ? dL_dreg_map[pix] : 0.f;

                float T = T_final;
                float accum_rec[3] = {0, 0, 0}, last_color[3] = {0, 0, 0};
                float last_alpha = 0.f, accum_depth_rec = 0.f, last_depth = 0.f;
                float accum_alpha_rec = 0.f;
                float accum_normal_rec[3] = {0, 0, 0}, last_normal[3] = {0, 0, 0};
                float last_dL_dT = 0.f;
                const float bg_dot = bg[0] * dpix[0] + bg[1] * dpix[1] + bg[2] * dpix[2];

                for (int c = last_contrib - 1; c >= 0; --c) {
                    const int j = start + c;
                    const int g = ids[j];
                    const float *no = normal_opac + 4 * g;
                    const float opa = sigmoid(no[3]);
                    const float *Tm = transmats + 9 * g;
                    PairEval e;
                    if (!eval_pair(px, py, crow.data() + 9 * (size_t)g, Tm, xys + 2 * g, opa, e)) continue;
                    const float alpha = e.alpha, G = e.G;
                    T = T / (1.0f - alpha);
                    const float dchannel_dcolor = alpha * T;
                    float dL_dalpha = 0.0f;
                    double *a = acc.data() + (size_t)j * 16;
                    double *aa = grads_abs ? acc_abs.data() + (size_t)j * 16 : nullptr;
                    const float *crgb = colors + 3 * g;
                    for (int ch = 0; ch < 3; ch++) {
                        const float c_raw = crgb[ch];
                        const float c_used = fmaxf(c_raw + 0.5f, 0.0f);
                        const float mask = (c_raw + 0.5f > 0.0f) ? 1.0f : 0.0f;
                        accum_rec[ch] = last_alpha * last_color[ch] +
                                        (1.f - last_alpha) * accum_rec[ch];
                        last_color[ch] = c_used;
                        dL_dalpha += (c_used - accum_rec[ch]) * dpix[ch];
                        a[13 + ch] += (double)(dchannel_dcolor * dpix[ch] * mask);
                        if (aa) aa[13 + ch] += std::fabs((double)(dchannel_dcolor * dpix[ch] * mask));
                    }
                    float dL_dz = 0.0f, dL_dweight = 0.0f;
                    const float m_d = mscale * (1.0f - NEAR_N / e.depth);
                    const float dmd_dd =
                        (FAR_N * NEAR_N) / ((FAR_N - NEAR_N) * e.depth * e.depth);
                    if (c == median_contrib - 1) dL_dz += dmed;
                    dL_dweight += (final_D2 + m_d * m_d * final_A - 2.0f * m_d * final_D) * dreg;
                    dL_dalpha += dL_dweight - last_dL_dT;
                    last_dL_dT = dL_dweight * alpha + (1.0f - alpha) * last_dL_dT;
                    const float dL_dmd = 2.0f * (T * alpha) * (m_d * final_A - final_D) * dreg;
                    dL_dz += dL_dmd * dmd_dd;
                    accum_depth_rec = last_alpha * last_depth + (1.f - last_alpha) * accum_depth_rec;
                    last_depth = e.depth;
                    dL_dalpha += (e.depth - accum_depth_rec) * ddepth;
                    accum_alpha_rec = last_alpha * 1.0f + (1.f - last_alpha) * accum_alpha_rec;
                    dL_dalpha += (1.0f - accum_alpha_rec) * daccum;
                    for (int ch = 0; ch < 3; ch++) {
                        accum_normal_rec[ch] = last_alpha * last_normal[ch] +
                                               (1.f - last_alpha) * accum_normal_rec[ch];
                        last_normal[ch] = no[ch];
                        dL_dalpha += (no[ch] - accum_normal_rec[ch]) * dn2[ch];
                        a[9 + ch] += (double)(alpha * T * dn2[ch]);
                        if (aa) aa[9 + ch] += std::fabs((double)(alpha * T * dn2[ch]));
                    }
                    dL_dalpha *= T;
                    last_alpha = alpha;
                    dL_dalpha += (-T_final / (1.f - alpha)) * bg_dot;
                    const float dL_dG = opa * dL_dalpha;
                    dL_dz += alpha * T * ddepth;
                    const float Twx = Tm[6], Twy = Tm[7];
                    if (e.rho3d <= e.rho2d) {
                        const float dsx = dL_dG * -G * e.u + dL_dz * Twx;
                        const float dsy = dL_dG * -G * e.v + dL_dz * Twy;
                        const float dsx_pz = dsx / e.ray.z, dsy_pz = dsy / e.ray.z;
                        const f3 dp = {dsx_pz, dsy_pz, -(dsx_pz * e.u + dsy_pz * e.v)};
                        const f3 &k = e.k, &l = e.l;
                        const f3 dk = {l.y * dp.z - l.z * dp.y, l.z * dp.x - l.x * dp.z,
                                       l.x * dp.y - l.y * dp.x};
                        const f3 dl = {dp.y * k.z - dp.z * k.y, dp.z * k.x - dp.x * k.z,
                                       dp.x * k.y - dp.y * k.x};
                        a[0] += (double)(-dk.x);
                        a[1] += (double)(-dk.y);
                        a[2] += (double)(-dk.z);
                        a[3] += (double)(-dl.x);
                        a[4] += (double)(-dl.y);
                        a[5] += (double)(-dl.z);
                        a[6] += (double)(px * dk.x + py * dl.x + dL_dz * e.u);
                        a[7] += (double)(px * dk.y + py * dl.y + dL_dz * e.v);
                        a[8] += (double)(px * dk.z + py * dl.z + dL_dz * 1.0f);
                        if (aa) {
                            /* magnitudes of the parts each summand is formed
                             * from: k = px Tw - Tu, l = py Tw - Tv, dp.z =
                             * -(dp.x u + dp.y v), pushed through the cross
                             * products */
                            const double Tuv[2][3] = {{Tm[0], Tm[1], Tm[2]}, {Tm[3], Tm[4], Tm[5]}};
                            const double Twv[3] = {Tm[6], Tm[7], Tm[8]};
                            double km[3], lm[3];
                            for (int q = 0; q < 3; ++q) {
                                km[q] = std::fabs(px * Twv[q]) + std::fabs(Tuv[0][q]);
                                lm[q] = std::fabs(py * Twv[q]) + std::fabs(Tuv[1][q]);
                            }
                            const double pm[3] = {std::fabs((double)dp.x), std::fabs((double)dp.y),
                                                  std::fabs((double)dsx_pz * e.u) +
                                                      std::fabs((double)dsy_pz * e.v)};
                            const double dkm[3] = {lm[1] * pm[2] + lm[2] * pm[1], lm[2] * pm[0] + lm[0] * pm[2],
                                                   lm[0] * pm[1] + lm[1] * pm[0]};
                            const double dlm[3] = {pm[1] * km[2] + pm[2] * km[1], pm[2] * km[0] + pm[0] * km[2],
                                                   pm[0] * km[1] + pm[1] * km[0]};
                            const double uv1[3] = {e.u, e.v, 1.0};
                            for (int q = 0; q < 3; ++q) {
                                aa[q] += dkm[q];
                                aa[3 + q] += dlm[q];
                                aa[6 + q] += std::fabs(px) * dkm[q] + std::fabs(py) * dlm[q] +
                                             std::fabs(dL_dz * uv1[q]);
                            }
                        }
                    } else {
                        a[6] += (double)(e.u * dL_dz);
                        a[7] += (double)(e.v * dL_dz);
                        a[8] += (double)dL_dz;
                        if (aa) {
                            aa[6] += std::fabs((double)(e.u * dL_dz));
                            aa[7] += std::fabs((double)(e.v * dL_dz));
                            aa[8] += std::fabs((double)dL_dz);
                        }
                    }
                    const float dsig = opa * (1.0f - opa);
                    a[12] += (double)(G * dL_dalpha * dsig);
                    if (aa) aa[12] += std::fabs((double)(G * dL_dalpha * dsig));
                }
            }
    }
    std::vector<double> gsum((size_t)n * 16, 0.0);
    for (int64_t j = 0; j < I; ++j) {
        const double *a = acc.data() + (size_t)j * 16;
        double *o = gsum.data() + (size_t)ids[j] * 16;
        for (int k = 0; k < 16; ++k) o[k] += a[k];
    }
    for (size_t k = 0; k < (size_t)n * 16; ++k) grads[k] = (float)gsum[k];
    if (grads_abs) {
        std::fill(gsum.begin(), gsum.end(), 0.0);
        for (int64_t j = 0; j < I; ++j) {
            const double *a = acc_abs.data() + (size_t)j * 16;
            double *o = gsum.data() + (size_t)ids[j] * 16;
            for (int k = 0; k < 16; ++k) o[k] += a[k];
        }
        for (size_t k = 0; k < (size_t)n * 16; ++k) grads_abs[k] = (float)gsum[k];
    }
}

/* project_and_sh_backward_2dgs_kernel (msplat_metal.metal:2003-2209). */
extern "C" void orc_project_bwd(int n, const float *means, const float *scales,
                                const float *quats, const float *frest, int degree,
                                int dtu, const OrcCamera *cam, float glob_scale,
                                const int32_t *radii, const float *g16, float *dmeans,
                                float *dscales, float *dquats, float *dmean2d,
                                float *dfdc, float *dfrest, float *xys_grad_norm,
                                float *vis_counts, float *max_2d_size, float inv_max_dim) {
    const float *pm = cam->projmat;
    const int nb = num_sh_bases(degree);
    const int K = nb - 1;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        float *dfr = dfrest + (size_t)K * 3 * i;
        for (int k = 0; k < K * 3; ++k) dfr[k] = 0.f;
        if (radii[i] <= 0) {
            for (int k = 0; k < 3; k++) dmeans[3 * i + k] = 0.0f;
            for (int k = 0; k < 2; k++) dscales[2 * i + k] = 0.0f;
            for (int k = 0; k < 4; k++) dquats[4 * i + k] = 0.0f;
            for (int k = 0; k < 2; k++) dmean2d[2 * i + k] = 0.0f;
            for (int k = 0; k < 3; k++) dfdc[3 * i + k] = 0.0f;
            continue;
        }
        const float *p = means + 3 * i;
        const float sx = orc_expf(scales[2 * i]), sy = orc_expf(scales[2 * i + 1]);
        const float *q = quats + 4 * i;
        f3 R0, R1, R2;
        quat_to_rotmat(q, R0, R1, R2);
        const float sxg = sx * glob_scale, syg = sy * glob_scale;
        f3 tu = {R0.x * sxg, R0.y * sxg, R0.z * sxg};
        f3 tv = {R1.x * syg, R1.y * syg, R1.z * syg};
        ClipCols cc = clip_columns(p, tu, tv, pm);
        const float W = (float)cam->width, H = (float)cam->height;
        const float halfW = 0.5f * W, halfH = 0.5f * H;
        const float bx = cam->cx - 0.5f, by = cam->cy - 0.5f;
        const float *g = g16 + 16 * i;
        f3 dcu = {g[0], g[3], g[6]}, dcv = {g[1], g[4], g[7]}, dco = {g[2], g[5], g[8]};
        float du[4] = {halfW * dcu.x, halfH * dcu.y, 0.0f, bx * dcu.x + by * dcu.y + dcu.z};
        float dv[4] = {halfW * dcv.x, halfH * dcv.y, 0.0f, bx * dcv.x + by * dcv.y + dcv.z};
        float dpc[4] = {halfW * dco.x, halfH * dco.y, 0.0f, bx * dco.x + by * dco.y + dco.z};
        f3 gtu, gtv, gp;
        gtu.x = pm[0] * du[0] + pm[4] * du[1] + pm[8] * du[2] + pm[12] * du[3];
        gtu.y = pm[1] * du[0] + pm[5] * du[1] + pm[9] * du[2] + pm[13] * du[3];
        gtu.z = pm[2] * du[0] + pm[6] * du[1] + pm[10] * du[2] + pm[14] * du[3];
        gtv.x = pm[0] * dv[0] + pm[4] * dv[1] + pm[8] * dv[2] + pm[12] * dv[3];
        gtv.y = pm[1] * dv[0] + pm[5] * dv[1] + pm[9] * dv[2] + pm[13] * dv[3];
        gtv.z = pm[2] * dv[0] + pm[6] * dv[1] + pm[10] * dv[2] + pm[14] * dv[3];
        gp.x = pm[0] * dpc[0] + pm[4] * dpc[1] + pm[8] * dpc[2] + pm[12] * dpc[3];
        gp.y = pm[1] * dpc[0] + pm[5] * dpc[1] + pm[9] * dpc[2] + pm[13] * dpc[3];
        gp.z = pm[2] * dpc[0] + pm[6] * dpc[1] + pm[10] * dpc[2] + pm[14] * dpc[3];
        const float dsx = dot3(gtu, R0), dsy = dot3(gtv, R1);
        dscales[2 * i + 0] = dsx * sx * glob_scale;
        dscales[2 * i + 1] = dsy * sy * glob_scale;
        f3 vR[3] = {{gtu.x * sxg, gtu.y * sxg, gtu.z * sxg},
                    {gtv.x * syg, gtv.y * syg, gtv.z * syg},
                    {g[9], g[10], g[11]}};
        quat_to_rotmat_vjp(q, vR, dquats + 4 * i);
        dmeans[3 * i + 0] = gp.x;
        dmeans[3 * i + 1] = gp.y;
        dmeans[3 * i + 2] = gp.z;

        f3 dir_un = {p[0] - cam->cam_pos[0], p[1] - cam->cam_pos[1], p[2] - cam->cam_pos[2]};
        f3 dir = normalize3(dir_un);
        const float *vc = g + 13;
        sh_vjp(dtu, dir, vc, dfdc + 3 * i, dfr);
        if (dtu >= 1) {
            f3 dd = sh_dL_ddir(dtu, dir, frest + (size_t)K * 3 * i, vc);
            f3 dm = dnormvdv(dir_un, dd);
            dmeans[3 * i + 0] += dm.x;
            dmeans[3 * i + 1] += dm.y;
            dmeans[3 * i + 2] += dm.z;
        }
        const float depth_fwd = cc.pc[3];
        const float dmx = g[6] * depth_fwd * 0.5f * W;
        const float dmy = g[7] * depth_fwd * 0.5f * H;
        dmean2d[2 * i + 0] = dmx;
        dmean2d[2 * i + 1] = dmy;
        xys_grad_norm[i] += fabsf(dmx) + fabsf(dmy);
        vis_counts[i] += 1.0f;
        const float r_norm = (float)radii[i] * inv_max_dim;
        if (r_norm > max_2d_size[i]) max_2d_size[i] = r_norm;
    }
}

/* fused_adam_kernel (msplat_metal.metal:1383-1406). */
extern "C" void orc_adam(float *params, const float *grads, float *m_, float *v_, int64_t n,
                         float step_size, float beta1, float beta2, float bc2_sqrt,
                         float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) {
        float g = grads[i];
        float m = fmaf(beta1, m_[i], (1.0f - beta1) * g);
        float v = fmaf(beta2, v_[i], (1.0f - beta2) * g * g);
        params[i] -= step_size * m / (sqrtf(v) / bc2_sqrt + eps);
        m_[i] = m;
        v_[i] = v;
    }
}

/* msplat_densify (msplat_metal.mm:1339-1594): classify (metal:3231-3266),
 * append split (:3271-3361), append dup (:3365-3412), cull (:3417-3456) and
 * stable compaction (:3460-3491), run stage by stage.  SD floats of scale
 * per splat: the kernels' kScaleDim (2 for surfels, 3 for 3D Gaussians,
 * :3253-3255, :3315-3317, :3339-3341). */
static int densify_sd(int SD, int N, int capacity, float grad_thresh, float size_thresh,
                      float screen_thresh, int check_screen, float cull_alpha_thresh,
                      float cull_scale_thresh, float cull_screen_size, int check_huge,
                      const float *xys_grad_norm, const float *vis_counts,
                      const float *max_2d_size, float half_max_dim,
                      float *const params[6], int fr_stride,
                      float *const exp_avg[6], float *const exp_avg_sq[6],
                      const float *rs) {
    if (N > capacity) return -1;
    const int strides[6] = {3, SD, 4, 3, fr_stride, 1};
    float *means = params[0], *scales = params[1], *quats = params[2];
    float *opac = params[5];
    std::vector<int> split(N), dup(N), split_pre(N), dup_pre(N);
    for (int i = 0; i < N; ++i) {
        float vc = vis_counts[i];
        if (vc <= 0.0f) { split[i] = dup[i] = 0; continue; }
        float avg = (xys_grad_norm[i] / vc) * half_max_dim;
        bool high = avg > grad_thresh;
        float ms = orc_expf(scales[(size_t)SD * i]);
        for (int k = 1; k < SD; ++k) ms = fmaxf(ms, orc_expf(scales[(size_t)SD * i + k]));
        bool large = ms > size_thresh;
        bool sp = large;
        if (check_screen && max_2d_size[i] > screen_thresh) sp = true;
        sp = sp && high;
        split[i] = sp ? 1 : 0;
        dup[i] = (!large && high) ? 1 : 0;
    }
    int acc = 0;
    for (int i = 0; i < N; ++i) split_pre[i] = (acc += split[i]);
    acc = 0;
    for (int i = 0; i < N; ++i) dup_pre[i] = (acc += dup[i]);
    const int nS = N > 0 ? split_pre[N - 1] : 0, nD = N > 0 ? dup_pre[N - 1] : 0;
    /* a splat can be both split and dup, so the appended count reaches up
     * to 4N: report the rows needed (negated) before writing anything */
    if ((int64_t)N + 2 * (int64_t)nS + nD > capacity) return -(N + 2 * nS + nD);
    const float log_size_fac = std::log(1.6f);

    auto zero_adam = [&](int dst) {
        for (int gi = 0; gi < 6; ++gi)
            for (int j = 0; j < strides[gi]; ++j) {
                exp_avg[gi][(size_t)dst * strides[gi] + j] = 0.f;
                exp_avg_sq[gi][(size_t)dst * strides[gi] + j] = 0.f;
            }
    };
    for (int i = 0; i < N; ++i) {
        if (!split[i]) continue;
        int ord = split_pre[i] - 1, c0 = N + 2 * ord;
        float qw = quats[i * 4], qx = quats[i * 4 + 1], qy = quats[i * 4 + 2], qz = quats[i * 4 + 3];
        float qlen = sqrtf(qw * qw + qx * qx + qy * qy + qz * qz);
        qw /= qlen; qx /= qlen; qy /= qlen; qz /= qlen;
        float sx = orc_expf(scales[(size_t)i * SD]), sy = orc_expf(scales[(size_t)i * SD + 1]);
        float sz = SD > 2 ? orc_expf(scales[(size_t)i * SD + 2]) : 0.0f;
        for (int k = 0; k < 2; ++k) {
            int child = c0 + k, ri = ord * 2 + k;
            float r0 = rs[ri * 3] * sx, r1 = rs[ri * 3 + 1] * sy, r2 = rs[ri * 3 + 2] * sz;
            float v0 = (1 - 2 * (qy * qy + qz * qz)) * r0 + 2 * (qx * qy - qw * qz) * r1 +
                       2 * (qx * qz + qw * qy) * r2;
            float v1 = 2 * (qx * qy + qw * qz) * r0 + (1 - 2 * (qx * qx + qz * qz)) * r1 +
                       2 * (qy * qz - qw * qx) * r2;
            float v2 = 2 * (qx * qz - qw * qy) * r0 + 2 * (qy * qz + qw * qx) * r1 +
                       (1 - 2 * (qx * qx + qy * qy)) * r2;
            means[child * 3] = means[i * 3] + v0;
            means[child * 3 + 1] = means[i * 3 + 1] + v1;
            means[child * 3 + 2] = means[i * 3 + 2] + v2;
            for (int j = 0; j < SD; ++j) scales[(size_t)child * SD + j] = scales[(size_t)i * SD + j] - log_size_fac;
            for (int gi = 2; gi < 6; ++gi)
                for (int j = 0; j < strides[gi]; ++j)
                    params[gi][(size_t)child * strides[gi] + j] =
                        params[gi][(size_t)i * strides[gi] + j];
            zero_adam(child);
        }
        for (int j = 0; j < SD; ++j) scales[(size_t)i * SD + j] -= log_size_fac;
    }
    for (int i = 0; i < N; ++i) {
        if (!dup[i]) continue;
        int dst = N + 2 * nS + dup_pre[i] - 1;
        for (int gi = 0; gi < 6; ++gi)
            for (int j = 0; j < strides[gi]; ++j)
                params[gi][(size_t)dst * strides[gi] + j] = params[gi][(size_t)i * strides[gi] + j];
        zero_adam(dst);
    }
    const int N_new = N + 2 * nS + nD;
    std::vector<int> keep(N_new);
    for (int i = 0; i < N_new; ++i) {
        float os = 1.0f / (1.0f + orc_expf(-opac[i]));
        bool cull = os < cull_alpha_thresh;
        if (i < N && split[i] != 0) cull = true;
        if (check_huge) {
            float ms = orc_expf(scales[(size_t)i * SD]);
            for (int k = 1; k < SD; ++k) ms = fmaxf(ms, orc_expf(scales[(size_t)i * SD + k]));
            if (ms > cull_scale_thresh) cull = true;
            if (check_screen && i < N && max_2d_size[i] > cull_screen_size) cull = true;
        }
        keep[i] = cull ? 0 : 1;
    }
    int out = 0;
    for (int i = 0; i < N_new; ++i) {
        if (!keep[i]) continue;
        if (out != i) {
            for (int gi = 0; gi < 6; ++gi) {
                const size_t s = strides[gi];
                memmove(params[gi] + out * s, params[gi] + i * s, s * 4);
                memmove(exp_avg[gi] + out * s, exp_avg[gi] + i * s, s * 4);
                memmove(exp_avg_sq[gi] + out * s, exp_avg_sq[gi] + i * s, s * 4);
            }
        }
        ++out;
    }
    return out;
}

extern "C" int orc_densify(int N, int capacity, float grad_thresh, float size_thresh,
                           float screen_thresh, int check_screen, float cull_alpha_thresh,
                           float cull_scale_thresh, float cull_screen_size, int check_huge,
                           const float *xys_grad_norm, const float *vis_counts,
                           const float *max_2d_size, float half_max_dim,
                           float *const params[6], int fr_stride,
                           float *const exp_avg[6], float *const exp_avg_sq[6],
                           const float *rs) {
    return densify_sd(2, N, capacity, grad_thresh, size_thresh, screen_thresh, check_screen, cull_alpha_thresh,
                      cull_scale_thresh, cull_screen_size, check_huge, xys_grad_norm, vis_counts, max_2d_size,
                      half_max_dim, params, fr_stride, exp_avg, exp_avg_sq, rs);
}

extern "C" int orc_densify_3dgs(int N, int capacity, float grad_thresh, float size_thresh,
                                float screen_thresh, int check_screen, float cull_alpha_thresh,
                                float cull_scale_thresh, float cull_screen_size, int check_huge,
                                const float *xys_grad_norm, const float *vis_counts,
                                const float *max_2d_size, float half_max_dim,
                                float *const params[6], int fr_stride,
                                float *const exp_avg[6], float *const exp_avg_sq[6],
                                const float *rs) {
    return densify_sd(3, N, capacity, grad_thresh, size_thresh, screen_thresh, check_screen, cull_alpha_thresh,
                      cull_scale_thresh, cull_screen_size, check_huge, xys_grad_norm, vis_counts, max_2d_size,
                      half_max_dim, params, fr_stride, exp_avg, exp_avg_sq, rs);
}

/* Model::fullIteration (core/src/model.cpp:762-829) + msplat_train_step_2dgs
 * (core/metal/msplat_metal.mm:935-1331) on the CPU. */
extern "C" double orc_train_step(int n, float *means, float *scales, float *quats,
                                 float *opac, float *fdc, float *frest, int degree,
                                 int dtu, const OrcCamera *cam, const float *bg,
                                 const float *gt, float ssim_weight,
                                 float *const exp_avg[6], float *const exp_avg_sq[6],
                                 const float adam_lr[6], int adam_step, float *xys_grad_norm,
                                 float *vis_counts, float *max_2d_size, float *out_img_out,
                                 double *stage_ms, int64_t *num_isect, OrcStepDetail *detail) {
    using clk = std::chrono::steady_clock;
    auto t0 = clk::now();
    auto lap = [&](int s) {
        auto t1 = clk::now();
        if (stage_ms) stage_ms[s] += std::chrono::duration<double, std::milli>(t1 - t0).count();
        t0 = t1;
    };
    const int K = num_sh_bases(degree) - 1;
    const size_t P = (size_t)cam->width * cam->height;
    const int TT = cam->tiles_x * cam->tiles_y;
    std::vector<float> xys(2 * (size_t)n), depths(n), tm(9 * (size_t)n), no(4 * (size_t)n),
        col(3 * (size_t)n);
    std::vector<int32_t> radii(n), hit(n), rect(4 * (size_t)n), counts(TT), offs(TT + 1);
    orc_project_fwd(n, means, scales, quats, opac, fdc, frest, degree, dtu, cam, 1.0f, 0.01f,
                    xys.data(), depths.data(), radii.data(), tm.data(), no.data(), col.data(),
                    hit.data(), rect.data());
    lap(0);
    int64_t I = orc_count_tiles(n, radii.data(), rect.data(), cam->tiles_x, cam->tiles_y,
                                counts.data());
    std::vector<uint64_t> keys(I);
    std::vector<int32_t> ids(I);
    orc_bin_sort(n, radii.data(), rect.data(), depths.data(), cam->tiles_x, cam->tiles_y,
                 counts.data(), offs.data(), keys.data(), ids.data());
    if (num_isect) *num_isect = I;
    lap(1);
    std::vector<float> img(3 * P), fT(3 * P), dep(P), nrm(3 * P), alp(P), med(P), dist(P);
    std::vector<int32_t> fidx(2 * P);
    orc_raster_fwd(cam, offs.data(), ids.data(), xys.data(), tm.data(), no.data(), col.data(),
                   bg, img.data(), fT.data(), fidx.data(), dep.data(), nrm.data(), alp.data(),
                   med.data(), dist.data(), nullptr);
    lap(2);
    std::vector<float> dimg(3 * P), ddist(P);
    double loss = orc_loss_fwd_bwd(cam->width, cam->height, img.data(), gt, dist.data(),
                                   1.0f - ssim_weight, 0.0f, ssim_weight, dimg.data(),
                                   ddist.data(), nullptr);
    lap(3);
    std::vector<float> g16(16 * (size_t)n);
    std::vector<float> g16_abs(detail && detail->want_grads ? 16 * (size_t)n : 0);
    orc_raster_bwd(cam, n, offs.data(), ids.data(), xys.data(), tm.data(), no.data(),
                   col.data(), bg, fT.data(), fidx.data(), dimg.data(), nullptr, nullptr,
                   nullptr, nullptr, ddist.data(), g16.data(),
                   g16_abs.empty() ? nullptr : g16_abs.data());
    lap(4);
    if (detail) {
        auto dup = [](const void *src, size_t bytes) {
            void *d = malloc(bytes ? bytes : 1);
            if (d && bytes) memcpy(d, src, bytes);
            return d;
        };
        detail->num_isect = I;
        detail->tile_offsets = (int32_t *)dup(offs.data(), offs.size() * 4);
        detail->ids = (int32_t *)dup(ids.data(), ids.size() * 4);
        detail->grads16 = detail->want_grads ? (float *)dup(g16.data(), g16.size() * 4) : nullptr;
        detail->grads16_abs = detail->want_grads ? (float *)dup(g16_abs.data(), g16_abs.size() * 4) : nullptr;
    }
    std::vector<float> dm(3 * (size_t)n), ds(2 * (size_t)n), dq(4 * (size_t)n),
        dm2(2 * (size_t)n), ddc(3 * (size_t)n), dfr((size_t)K * 3 * n), dop(n);
    const float inv_max_dim = 1.0f / (float)std::max(cam->width, cam->height);
    orc_project_bwd(n, means, scales, quats, frest, degree, dtu, cam, 1.0f, radii.data(),
                    g16.data(), dm.data(), ds.data(), dq.data(), dm2.data(), ddc.data(),
                    dfr.data(), xys_grad_norm, vis_counts, max_2d_size, inv_max_dim);
    for (int i = 0; i < n; ++i) dop[i] = g16[16 * (size_t)i + 12];
    lap(5);
    const float b1 = 0.9f, b2 = 0.999f, eps = 1e-8f;
    const float bc1 = 1.0f - std::pow(b1, adam_step);
    const float bc2 = 1.0f - std::pow(b2, adam_step);
    const float bc2_sqrt = std::sqrt(bc2);
    float *P6[6] = {means, scales, quats, fdc, frest, opac};
    const float *G6[6] = {dm.data(), ds.data(), dq.data(), ddc.data(), dfr.data(), dop.data()};
    const int64_t n6[6] = {3LL * n, 2LL * n, 4LL * n, 3LL * n, (int64_t)K * 3 * n, n};
    for (int gi = 0; gi < 6; ++gi)
        orc_adam(P6[gi], G6[gi], exp_avg[gi], exp_avg_sq[gi], n6[gi], adam_lr[gi] / bc1, b1,
                 b2, bc2_sqrt, eps);
    lap(6);
    if (out_img_out) memcpy(out_img_out, img.data(), 3 * P * sizeof(float));
    return loss;
}

extern "C" void orc_free(void *p) { free(p); }

/* Test helpers: vectorised exp and the SSIM window. */
extern "C" void orc_expf_array(int64_t n, const float *x, float *y) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) y[i] = orc_expf(x[i]);
}

extern "C" void orc_ssim_window(float *w) { ssim_window(w); }

/* ---- mesh extraction ---------------------------------------------------
 * Expressions are the reference's, left to right, no contraction. */

/* tsdf_integrate_kernel (msplat_metal.metal:2223-2280), one thread's work
 * per voxel, voxels in any order (they are independent). */
void orc_tsdf_integrate(float *grid, int dx, int dy, int dz, const float origin[3],
                        float voxel_size, const float viewmat[16], float fx, float fy,
                        float cx, float cy, int width, int height, float trunc_dist,
                        float alpha_thresh, const float *depth, const float *alpha) {
    const float *m = viewmat;
#pragma omp parallel for schedule(static)
    for (int z = 0; z < dz; ++z)
        for (int y = 0; y < dy; ++y)
            for (int x = 0; x < dx; ++x) {
                /* voxel centre (:2240-2243) */
                const float wx = origin[0] + ((float)x + 0.5f) * voxel_size;
                const float wy = origin[1] + ((float)y + 0.5f) * voxel_size;
                const float wz = origin[2] + ((float)z + 0.5f) * voxel_size;
                const float vx = m[0] * wx + m[1] * wy + m[2] * wz + m[3];
                const float vy = m[4] * wx + m[5] * wy + m[6] * wz + m[7];
                const float vz = m[8] * wx + m[9] * wy + m[10] * wz + m[11];
                if (vz <= 0.01f) continue;
                const float px = vx / vz * fx + cx;
                const float py = vy / vz * fy + cy;
                const int ix = f2i(px), iy = f2i(py);
                if (ix < 0 || ix >= width || iy < 0 || iy >= height) continue;
                const int64_t pid = (int64_t)iy * width + ix;
                const float a = alpha[pid];
                if (a < alpha_thresh) continue;
                const float d = depth[pid];
                if (!std::isfinite(d) || d <= 0.0f) continue;
                float sdf = d - vz;
                if (sdf < -trunc_dist) continue;
                sdf = fminf(fmaxf(sdf, -trunc_dist), trunc_dist); /* Metal clamp */
                float *g = grid + (((int64_t)z * dy + y) * dx + x) * 2;
                const float old_sdf = g[0], old_w = g[1];
                const float new_w = old_w + a;
                g[0] = (old_sdf * old_w + sdf * a) / new_w;
                g[1] = new_w;
            }
}

/* marching_cubes_kernel (msplat_metal.metal:2606-2687). */
int64_t orc_marching_cubes(const float *grid, int dx, int dy, int dz,
                           const float origin[3], float voxel_size,
                           const int8_t *table, int64_t max_triangles, float *out) {
    static const int corner[8][3] = {{0, 0, 0}, {1, 0, 0}, {1, 1, 0}, {0, 1, 0},
                                     {0, 0, 1}, {1, 0, 1}, {1, 1, 1}, {0, 1, 1}};
    static const int edge[12][2] = {{0, 1}, {1, 2}, {2, 3}, {3, 0}, {4, 5}, {5, 6},
                                    {6, 7}, {7, 4}, {0, 4}, {1, 5}, {2, 6}, {3, 7}};
    int64_t count = 0;
    for (int k = 0; k + 1 < dz; ++k)
        for (int j = 0; j + 1 < dy; ++j)
            for (int i = 0; i + 1 < dx; ++i) {
                float sdf[8], wts[8];
                for (int c = 0; c < 8; ++c) {
                    const int64_t idx = (((int64_t)(k + corner[c][2]) * dy + (j + corner[c][1])) * dx +
                                         (i + corner[c][0])) * 2;
                    sdf[c] = grid[idx];
                    wts[c] = grid[idx + 1];
                }
                bool skip = false;
                for (int c = 0; c < 8; ++c)
                    if (wts[c] <= 0.0f) skip = true;
                if (skip) continue;
                int cube = 0;
                for (int c = 0; c < 8; ++c)
                    if (sdf[c] < 0.0f) cube |= 1 << c;
                const int8_t *row = table + cube * 16;
                for (int t = 0; t < 16 && row[t] >= 0; t += 3, ++count) {
                    if (count >= max_triangles) continue;
                    float *dst = out + count * 9;
                    for (int v = 0; v < 3; ++v) {
                        const int e = row[t + v];
                        const int a = edge[e][0], b = edge[e][1];
                        const float s0 = sdf[a], s1 = sdf[b];
                        const float tt = (s1 == s0) ? 0.5f : (-s0 / (s1 - s0));
                        const int ia[3] = {i, j, k};
                        for (int q = 0; q < 3; ++q) {
                            const float p0 = origin[q] + voxel_size * ((float)(ia[q] + corner[a][q]) + 0.5f);
                            const float p1 = origin[q] + voxel_size * ((float)(ia[q] + corner[b][q]) + 0.5f);
                            dst[3 * v + q] = p0 + (p1 - p0) * tt; /* Metal mix */
                        }
                    }
                }
            }
    return count;
}

/* Model::exportPointCloud's pixel loop (model.cpp:580-616). */
int64_t orc_unproject_depth(const float *img, const float *depth, const float *alpha,
                            int width, int height, float fx, float fy, float cx,
                            float cy, const float c2w[16], float alpha_thresh,
                            float *xyz, uint8_t *rgb) {
    const float r00 = c2w[0], r01 = -c2w[1], r02 = -c2w[2];
    const float r10 = c2w[4], r11 = -c2w[5], r12 = -c2w[6];
    const float r20 = c2w[8], r21 = -c2w[9], r22 = -c2w[10];
    const float t0 = c2w[3], t1 = c2w[7], t2 = c2w[11];
    auto u8 = [](float v) { /* clamp(v * 255, 0, 255), NaN -> 0 */
        return (uint8_t)fminf(fmaxf(v * 255.0f, 0.0f), 255.0f);
    };
    int64_t n = 0;
    for (int py = 0; py < height; ++py)
        for (int px = 0; px < width; ++px) {
            const int64_t idx = (int64_t)py * width + px;
            const float a = alpha[idx];
            if (a < alpha_thresh) continue;
            const float d = depth[idx] / a;
            if (!std::isfinite(d) || d <= 0.0f) continue;
            const float xc = ((float)px + 0.5f - cx) * d / fx;
            const float yc = ((float)py + 0.5f - cy) * d / fy;
            const float zc = d;
            xyz[3 * n + 0] = r00 * xc + r01 * yc + r02 * zc + t0;
            xyz[3 * n + 1] = r10 * xc + r11 * yc + r12 * zc + t1;
            xyz[3 * n + 2] = r20 * xc + r21 * yc + r22 * zc + t2;
            rgb[3 * n + 0] = u8(img[3 * idx + 0]);
            rgb[3 * n + 1] = u8(img[3 * idx + 1]);
            rgb[3 * n + 2] = u8(img[3 * idx + 2]);
            ++n;
        }
    return n;
}

/* ---- 3DGS mode ---------------------------------------------------------
 * Projection, compositing and their backward for 3D Gaussians, built on the
 * reference's EWA helpers (scale_rot_to_cov3d msplat_metal.metal:160-176,
 * project_cov3d_ewa :333-378, compute_cov2d_bounds :420-441, project_pix
 * :444-452, and their VJPs :1059-1374), which the 2DGS fork keeps as dead
 * code.  Its 3DGS compositing kernel was removed; the pair rule here is the
 * published 3DGS one (Kerbl et al. 2023) in the fork's blending conventions
 * (alpha = min(0.99, opacity exp(-sigma)), skip below 1/255, stop before T
 * falls to 1e-4), sigma = 0.5 (a dx^2 + c dy^2) + b dx dy with the conic
 * (a, b, c) and d = centre - pixel.  rho = 2 sigma is formed as
 * fmaf(a dx, dx, fmaf(c dy, dy, 2 b dx dy)) and exp(-sigma) = orc_gauss(rho),
 * the arithmetic the kernels use. */
namespace {

/* scale_rot_to_cov3d: M = R diag(glob s), cov = M M^T (upper triangle). */
void cov3d_of(const float s[3], float glob, const float *q, float cov[6], f3 R[3]) {
    quat_to_rotmat(q, R[0], R[1], R[2]);
    const float g0 = glob * s[0], g1 = glob * s[1], g2 = glob * s[2];
    /* rows of M: M[r][c] = R[c][r] * s_c */
    const float M[3][3] = {{R[0].x * g0, R[1].x * g1, R[2].x * g2},
                           {R[0].y * g0, R[1].y * g1, R[2].y * g2},
                           {R[0].z * g0, R[1].z * g1, R[2].z * g2}};
    auto mm = [&](int i, int j) { return M[i][0] * M[j][0] + M[i][1] * M[j][1] + M[i][2] * M[j][2]; };
    cov[0] = mm(0, 0);
    cov[1] = mm(0, 1);
    cov[2] = mm(0, 2);
    cov[3] = mm(1, 1);
    cov[4] = mm(1, 2);
    cov[5] = mm(2, 2);
}

/* The fov-clamped view position of project_cov3d_ewa (:345-347). */
inline void ewa_clamp(float &px, float &py, float pz, float tan_fovx, float tan_fovy) {
    const float lim_x = 1.3f * tan_fovx, lim_y = 1.3f * tan_fovy;
    px = pz * fminf(lim_x, fmaxf(-lim_x, px / pz));
    py = pz * fminf(lim_y, fmaxf(-lim_y, py / pz));
}

/* project_cov3d_ewa (:333-378): cov2d = T V T^T + 0.3 I, T = J W. */
void ewa_cov2d(const float cov[6], const float *vm, float fx, float fy, float tan_fovx, float tan_fovy,
               const float pv[3], float c2[3]) {
    float px = pv[0], py = pv[1];
    const float pz = pv[2];
    ewa_clamp(px, py, pz, tan_fovx, tan_fovy);
    const float rz = 1.f / pz, rz2 = rz * rz;
    const float j00 = fx * rz, j11 = fy * rz;
    const float j20 = -fx * px * rz2, j21 = -fy * py * rz2;
    const f3 t0 = {j00 * vm[0] + j20 * vm[8], j00 * vm[1] + j20 * vm[9], j00 * vm[2] + j20 * vm[10]};
    const f3 t1 = {j11 * vm[4] + j21 * vm[8], j11 * vm[5] + j21 * vm[9], j11 * vm[6] + j21 * vm[10]};
    const float v00 = cov[0], v01 = cov[1], v02 = cov[2], v11 = cov[3], v12 = cov[4], v22 = cov[5];
    const f3 tv0 = {t0.x * v00 + t0.y * v01 + t0.z * v02, t0.x * v01 + t0.y * v11 + t0.z * v12,
                    t0.x * v02 + t0.y * v12 + t0.z * v22};
    const f3 tv1 = {t1.x * v00 + t1.y * v01 + t1.z * v02, t1.x * v01 + t1.y * v11 + t1.z * v12,
                    t1.x * v02 + t1.y * v12 + t1.z * v22};
    c2[0] = dot3(tv0, t0) + 0.3f;
    c2[1] = dot3(tv0, t1);
    c2[2] = dot3(tv1, t1) + 0.3f;
}

/* compute_cov2d_bounds (:420-441). */
bool cov2d_bounds(const float c2[3], float conic[3], float &radius) {
    const float det = c2[0] * c2[2] - c2[1] * c2[1];
    if (det == 0.f) return false;
    const float inv_det = 1.f / det;
    conic[0] = c2[2] * inv_det;
    conic[1] = -c2[1] * inv_det;
    conic[2] = c2[0] * inv_det;
    const float b = 0.5f * (c2[0] + c2[2]);
    const float disc = sqrtf(fmaxf(0.1f, b * b - det));
    radius = ceilf(3.f * sqrtf(b + disc));
    return true;
}

/* project_pix (:444-452) with ndc2pix (:58-60). */
void project_pix(const float *pm, const float *p, int W, int H, float cx, float cy, float xy[2]) {
    const float hx = pm[0] * p[0] + pm[1] * p[1] + pm[2] * p[2] + pm[3];
    const float hy = pm[4] * p[0] + pm[5] * p[1] + pm[6] * p[2] + pm[7];
    const float hw = pm[12] * p[0] + pm[13] * p[1] + pm[14] * p[2] + pm[15];
    const float rw = 1.f / (hw + 1e-6f);
    xy[0] = 0.5f * (float)W * (hx * rw) + cx - 0.5f;
    xy[1] = 0.5f * (float)H * (hy * rw) + cy - 0.5f;
}

/* 2 sigma of a pixel for the conic (a, b, c), d = centre - pixel. */
inline float conic_rho(const float *cn, float dx, float dy) {
    return fmaf(cn[0] * dx, dx, fmaf(cn[2] * dy, dy, 2.f * cn[1] * dx * dy));
}

}  // namespace

/* 3DGS projection + SH forward.  Per splat: xys[2], conics[3], depths,
 * radii (0 = culled), rect (x0, y0, x1, y1), colors (raw SH) and
 * cov2d[3] (nullable). */
extern "C" void orc_project3d_fwd(int n, const float *means, const float *scales, const float *quats,
                                  const float *fdc, const float *frest, int degree, int dtu,
                                  const OrcCamera *cam, float glob_scale, float clip_thresh, float *xys,
                                  float *conics, float *depths, int32_t *radii, int32_t *rect, float *colors,
                                  float *cov2d) {
    const float *vm = cam->viewmat, *pm = cam->projmat;
    const int nb = num_sh_bases(degree);
    const float tan_fovx = 0.5f * (float)cam->width / cam->fx, tan_fovy = 0.5f * (float)cam->height / cam->fy;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        radii[i] = 0;
        depths[i] = 0.f;
        for (int k = 0; k < 2; ++k) xys[2 * i + k] = 0.f;
        for (int k = 0; k < 3; ++k) conics[3 * i + k] = colors[3 * i + k] = 0.f;
        if (cov2d)
            for (int k = 0; k < 3; ++k) cov2d[3 * i + k] = 0.f;
        for (int k = 0; k < 4; ++k) rect[4 * i + k] = 0;
        const float *p = means + 3 * i;
        /* clip_near_plane (:139-150) */
        const float pv[3] = {vm[0] * p[0] + vm[1] * p[1] + vm[2] * p[2] + vm[3],
                             vm[4] * p[0] + vm[5] * p[1] + vm[6] * p[2] + vm[7],
                             vm[8] * p[0] + vm[9] * p[1] + vm[10] * p[2] + vm[11]};
        if (pv[2] <= clip_thresh) continue;
        const float s[3] = {orc_expf(scales[3 * i]), orc_expf(scales[3 * i + 1]), orc_expf(scales[3 * i + 2])};
        float cov[6], c2[3], cn[3], radius;
        f3 R[3];
        cov3d_of(s, glob_scale, quats + 4 * i, cov, R);
        ewa_cov2d(cov, vm, cam->fx, cam->fy, tan_fovx, tan_fovy, pv, c2);
        if (!cov2d_bounds(c2, cn, radius)) continue;
        float xy[2];
        project_pix(pm, p, cam->width, cam->height, cam->cx, cam->cy, xy);
        /* get_tile_bbox (:62-92) */
        const float tcx = xy[0] / (float)BLOCK, tcy = xy[1] / (float)BLOCK, tr = radius / (float)BLOCK;
        const int x0 = std::min(std::max(0, f2i(tcx - tr)), cam->tiles_x);
        const int x1 = std::min(std::max(0, f2i(tcx + tr + 1)), cam->tiles_x);
        const int y0 = std::min(std::max(0, f2i(tcy - tr)), cam->tiles_y);
        const int y1 = std::min(std::max(0, f2i(tcy + tr + 1)), cam->tiles_y);
        if ((x1 - x0) * (y1 - y0) <= 0) continue;
        radii[i] = (int)radius;
        depths[i] = pv[2];
        xys[2 * i] = xy[0];
        xys[2 * i + 1] = xy[1];
        for (int k = 0; k < 3; ++k) conics[3 * i + k] = cn[k];
        if (cov2d)
            for (int k = 0; k < 3; ++k) cov2d[3 * i + k] = c2[k];
        rect[4 * i + 0] = x0;
        rect[4 * i + 1] = y0;
        rect[4 * i + 2] = x1;
        rect[4 * i + 3] = y1;
        const f3 dir = normalize3({p[0] - cam->cam_pos[0], p[1] - cam->cam_pos[1], p[2] - cam->cam_pos[2]});
        sh_eval(dtu, dir, fdc + 3 * i, frest + (size_t)(nb - 1) * 3 * i, colors + 3 * i);
    }
}

/* 3DGS compositing forward: out_img, final_T (T per pixel) and
 * final_index (the last contributor, 1-based list position). */
extern "C" void orc_raster3d_fwd(const OrcCamera *cam, const int32_t *tile_offsets, const int32_t *ids,
                                 const float *xys, const float *conics, const float *colors,
                                 const float *opacities, const float *bg, float *out_img, float *final_T,
                                 int32_t *final_index) {
    const int W = cam->width, H = cam->height, TX = cam->tiles_x;
#pragma omp parallel for schedule(dynamic, 4)
    for (int py_i = 0; py_i < H; ++py_i)
        for (int px_i = 0; px_i < W; ++px_i) {
            const int tile = (py_i / BLOCK) * TX + (px_i / BLOCK);
            const float px = (float)px_i, py = (float)py_i;
            float T = 1.f, cr = 0.f, cg = 0.f, cb = 0.f;
            int contributor = 0, last = 0;
            for (int j = tile_offsets[tile]; j < tile_offsets[tile + 1]; ++j) {
                contributor++;
                const int g = ids[j];
                const float dx = xys[2 * g] - px, dy = xys[2 * g + 1] - py;
                const float rho = conic_rho(conics + 3 * g, dx, dy);
                if (rho < 0.f) continue;
                const float alpha = fminf(0.99f, sigmoid(opacities[g]) * orc_gauss(rho));
                if (alpha < 1.0f / 255.0f) continue;
                const float next_T = T * (1.0f - alpha);
                if (next_T <= 1e-4f) break;
                const float w = alpha * T;
                const float *c = colors + 3 * g;
                cr = fmaf(fmaxf(c[0] + 0.5f, 0.0f), w, cr);
                cg = fmaf(fmaxf(c[1] + 0.5f, 0.0f), w, cg);
                cb = fmaf(fmaxf(c[2] + 0.5f, 0.0f), w, cb);
                T = next_T;
                last = contributor;
            }
            const size_t pix = (size_t)py_i * W + px_i;
            final_T[pix] = T;
            final_index[pix] = last;
            out_img[3 * pix + 0] = fmaf(bg[0], T, cr);
            out_img[3 * pix + 1] = fmaf(bg[1], T, cg);
            out_img[3 * pix + 2] = fmaf(bg[2], T, cb);
        }
}

/* 3DGS compositing backward.  grads is [N,9] = (dL/dxy 2, dL/dconic 3 in
 * the EWA helpers' convention -- the off-diagonal entry is the derivative by
 * one of the two symmetric matrix entries, as cov2d_to_conic_vjp (:1080-1093)
 * expects --, dL/dopacity logit, dL/dcolors 3 (zero where the +0.5 clamp is
 * active)), summed in fp64 in a fixed order; grads_abs (nullable) the sums
 * of the magnitudes of the summands' parts. */
extern "C" void orc_raster3d_bwd(const OrcCamera *cam, int n, const int32_t *tile_offsets, const int32_t *ids,
                                 const float *xys, const float *conics, const float *colors,
                                 const float *opacities, const float *bg, const float *final_T,
                                 const int32_t *final_index, const float *dL_dimg, float *grads,
                                 float *grads_abs) {
    const int W = cam->width, H = cam->height, TX = cam->tiles_x, TY = cam->tiles_y;
    const int T_tiles = TX * TY;
    const int64_t I = tile_offsets[T_tiles];
    std::vector<double> acc((size_t)I * 9, 0.0), acc_abs(grads_abs ? (size_t)I * 9 : 0, 0.0);
#pragma omp parallel for schedule(dynamic, 1)
    for (int tile = 0; tile < T_tiles; ++tile) {
        const int ty = tile / TX, tx = tile % TX;
        const int start = tile_offsets[tile];
        for (int ly = 0; ly < BLOCK; ++ly)
            for (int lx = 0; lx < BLOCK; ++lx) {
                const int py_i = ty * BLOCK + ly, px_i = tx * BLOCK + lx;
                if (py_i >= H || px_i >= W) continue;
                const size_t pix = (size_t)py_i * W + px_i;
                const float px = (float)px_i, py = (float)py_i;
                const float T_final = final_T[pix];
                const float dpix[3] = {dL_dimg[3 * pix], dL_dimg[3 * pix + 1], dL_dimg[3 * pix + 2]};
                const float bg_dot = bg[0] * dpix[0] + bg[1] * dpix[1] + bg[2] * dpix[2];
                float T = T_final, last_alpha = 0.f;
                float accum_rec[3] = {0, 0, 0}, last_color[3] = {0, 0, 0};
                for (int c = final_index[pix] - 1; c >= 0; --c) {
                    const int j = start + c;
                    const int g = ids[j];
                    const float *cn = conics + 3 * g;
                    const float dx = xys[2 * g] - px, dy = xys[2 * g + 1] - py;
                    const float rho = conic_rho(cn, dx, dy);
                    if (rho < 0.f) continue;
                    const float opa = sigmoid(opacities[g]);
                    const float G = orc_gauss(rho);
                    const float alpha = fminf(0.99f, opa * G);
                    if (alpha < 1.0f / 255.0f) continue;
                    T = T / (1.0f - alpha);
                    double *a = acc.data() + (size_t)j * 9;
                    double *aa = grads_abs ? acc_abs.data() + (size_t)j * 9 : nullptr;
                    float dL_dalpha = 0.f;
                    const float *crgb = colors + 3 * g;
                    for (int ch = 0; ch < 3; ++ch) {
                        const float c_raw = crgb[ch];
                        const float c_used = fmaxf(c_raw + 0.5f, 0.0f);
                        const float mask = (c_raw + 0.5f > 0.0f) ? 1.0f : 0.0f;
                        accum_rec[ch] = last_alpha * last_color[ch] + (1.f - last_alpha) * accum_rec[ch];
                        last_color[ch] = c_used;
                        dL_dalpha += (c_used - accum_rec[ch]) * dpix[ch];
                        a[6 + ch] += (double)(alpha * T * dpix[ch] * mask);
                        if (aa) aa[6 + ch] += std::fabs((double)(alpha * T * dpix[ch] * mask));
                    }
                    dL_dalpha *= T;
                    last_alpha = alpha;
                    dL_dalpha += (-T_final / (1.f - alpha)) * bg_dot;
                    /* alpha = opa exp(-sigma): dL/dsigma = -opa G dL/dalpha */
                    const float v_sigma = -opa * G * dL_dalpha;
                    a[0] += (double)(v_sigma * (cn[0] * dx + cn[1] * dy));
                    a[1] += (double)(v_sigma * (cn[1] * dx + cn[2] * dy));
                    a[2] += (double)(0.5f * v_sigma * dx * dx);
                    a[3] += (double)(0.5f * v_sigma * dx * dy);
                    a[4] += (double)(0.5f * v_sigma * dy * dy);
                    const float dsig = opa * (1.0f - opa);
                    a[5] += (double)(G * dL_dalpha * dsig);
                    if (aa) {
                        const double vs = std::fabs((double)v_sigma);
                        aa[0] += vs * (std::fabs((double)cn[0] * dx) + std::fabs((double)cn[1] * dy));
                        aa[1] += vs * (std::fabs((double)cn[1] * dx) + std::fabs((double)cn[2] * dy));
                        aa[2] += 0.5 * vs * dx * dx;
                        aa[3] += 0.5 * vs * std::fabs((double)dx * dy);
                        aa[4] += 0.5 * vs * dy * dy;
                        aa[5] += std::fabs((double)(G * dL_dalpha * dsig));
                    }
                }
            }
    }
    std::vector<double> gsum((size_t)n * 9, 0.0);
    for (int64_t j = 0; j < I; ++j)
        for (int k = 0; k < 9; ++k) gsum[(size_t)ids[j] * 9 + k] += acc[(size_t)j * 9 + k];
    for (size_t k = 0; k < (size_t)n * 9; ++k) grads[k] = (float)gsum[k];
    if (grads_abs) {
        std::fill(gsum.begin(), gsum.end(), 0.0);
        for (int64_t j = 0; j < I; ++j)
            for (int k = 0; k < 9; ++k) gsum[(size_t)ids[j] * 9 + k] += acc_abs[(size_t)j * 9 + k];
        for (size_t k = 0; k < (size_t)n * 9; ++k) grads_abs[k] = (float)gsum[k];
    }
}

/* 3DGS projection + SH backward: grads9 (orc_raster3d_bwd's layout) ->
 * dL/dmeans [N,3], dL/dscales (log) [N,3], dL/dquats [N,4], dL/dfeatures_dc,
 * dL/dfeatures_rest; dmean2d = dL/dxy in NDC units (0.5 W, 0.5 H per pixel),
 * and the densification statistics (|dmean2d| L1 norm, visibility, largest
 * radius / max(W, H)), read-modify-write. */
extern "C" void orc_project3d_bwd(int n, const float *means, const float *scales, const float *quats,
                                  const float *frest, int degree, int dtu, const OrcCamera *cam, float glob_scale,
                                  const int32_t *radii, const float *grads9, float *dmeans, float *dscales,
                                  float *dquats, float *dmean2d, float *dfdc, float *dfrest, float *xys_grad_norm,
                                  float *vis_counts, float *max_2d_size, float inv_max_dim) {
    const float *vm = cam->viewmat, *pm = cam->projmat;
    const int K = num_sh_bases(degree) - 1;
    const float tan_fovx = 0.5f * (float)cam->width / cam->fx, tan_fovy = 0.5f * (float)cam->height / cam->fy;
    const float fx = cam->fx, fy = cam->fy;
#pragma omp parallel for schedule(static)
    for (int i = 0; i < n; ++i) {
        float *dfr = dfrest + (size_t)K * 3 * i;
        for (int k = 0; k < K * 3; ++k) dfr[k] = 0.f;
        for (int k = 0; k < 3; ++k) dmeans[3 * i + k] = dscales[3 * i + k] = dfdc[3 * i + k] = 0.f;
        for (int k = 0; k < 4; ++k) dquats[4 * i + k] = 0.f;
        dmean2d[2 * i] = dmean2d[2 * i + 1] = 0.f;
        if (radii[i] <= 0) continue;
        const float *p = means + 3 * i;
        const float *q = quats + 4 * i;
        const float *g = grads9 + 9 * i;
        const float pv[3] = {vm[0] * p[0] + vm[1] * p[1] + vm[2] * p[2] + vm[3],
                             vm[4] * p[0] + vm[5] * p[1] + vm[6] * p[2] + vm[7],
                             vm[8] * p[0] + vm[9] * p[1] + vm[10] * p[2] + vm[11]};
        const float s[3] = {orc_expf(scales[3 * i]), orc_expf(scales[3 * i + 1]), orc_expf(scales[3 * i + 2])};
        float cov[6], c2[3], cn[3], radius;
        f3 R[3];
        cov3d_of(s, glob_scale, q, cov, R);
        ewa_cov2d(cov, vm, fx, fy, tan_fovx, tan_fovy, pv, c2);
        cov2d_bounds(c2, cn, radius);
        /* cov2d_to_conic_vjp (:1080-1093): v_Sigma = -X G X */
        float vc2[3];
        {
            const float X00 = cn[0], X01 = cn[1], X11 = cn[2];
            const float G00 = g[2], G01 = g[3], G11 = g[4];
            /* XG */
            const float A00 = X00 * G00 + X01 * G01, A01 = X00 * G01 + X01 * G11;
            const float A10 = X01 * G00 + X11 * G01, A11 = X01 * G01 + X11 * G11;
            /* -(XG)X */
            const float S00 = -(A00 * X00 + A01 * X01), S01 = -(A00 * X01 + A01 * X11);
            const float S10 = -(A10 * X00 + A11 * X01), S11 = -(A10 * X01 + A11 * X11);
            vc2[0] = S00;
            vc2[1] = S10 + S01;
            vc2[2] = S11;
        }
        /* project_cov3d_ewa_vjp (:1110-1179) */
        float vcov[6];
        float vmean[3] = {0.f, 0.f, 0.f};
        {
            float px = pv[0], py = pv[1];
            const float pz = pv[2];
            ewa_clamp(px, py, pz, tan_fovx, tan_fovy);
            const float rz = 1.f / pz, rz2 = rz * rz;
            /* T = J W (rows), W = the view rotation (rows of vm) */
            const float Wm[3][3] = {{vm[0], vm[1], vm[2]}, {vm[4], vm[5], vm[6]}, {vm[8], vm[9], vm[10]}};
            const float J[3][3] = {{fx * rz, 0.f, -fx * px * rz2}, {0.f, fy * rz, -fy * py * rz2}, {0.f, 0.f, 0.f}};
            float Tm[3][3];
            for (int r = 0; r < 3; ++r)
                for (int c = 0; c < 3; ++c) Tm[r][c] = J[r][0] * Wm[0][c] + J[r][1] * Wm[1][c] + J[r][2] * Wm[2][c];
            const float V[3][3] = {{cov[0], cov[1], cov[2]}, {cov[1], cov[3], cov[4]}, {cov[2], cov[4], cov[5]}};
            const float vC[3][3] = {{vc2[0], 0.5f * vc2[1], 0.f}, {0.5f * vc2[1], vc2[2], 0.f}, {0.f, 0.f, 0.f}};
            /* v_V = T^T vC T */
            float vCT[3][3], vV[3][3];
            for (int r = 0; r < 3; ++r)
                for (int c = 0; c < 3; ++c) vCT[r][c] = vC[r][0] * Tm[0][c] + vC[r][1] * Tm[1][c] + vC[r][2] * Tm[2][c];
            for (int r = 0; r < 3; ++r)
                for (int c = 0; c < 3; ++c) vV[r][c] = Tm[0][r] * vCT[0][c] + Tm[1][r] * vCT[1][c] + Tm[2][r] * vCT[2][c];
            vcov[0] = vV[0][0];
            vcov[1] = vV[0][1] + vV[1][0];
            vcov[2] = vV[0][2] + vV[2][0];
            vcov[3] = vV[1][1];
            vcov[4] = vV[1][2] + vV[2][1];
            vcov[5] = vV[2][2];
            /* v_T = vC T V^T + vC^T T V = 2 vC T V (vC and V symmetric) */
            float vT[3][3];
            for (int r = 0; r < 3; ++r)
                for (int c = 0; c < 3; ++c) {
                    const float x = vCT[r][0] * V[0][c] + vCT[r][1] * V[1][c] + vCT[r][2] * V[2][c];
                    vT[r][c] = x + x;
                }
            /* v_J = v_T W^T */
            float vJ[3][3];
            for (int r = 0; r < 3; ++r)
                for (int c = 0; c < 3; ++c) vJ[r][c] = vT[r][0] * Wm[c][0] + vT[r][1] * Wm[c][1] + vT[r][2] * Wm[c][2];
            const float fx_rz2 = fx * rz2, fy_rz2 = fy * rz2, rz3 = rz2 * rz;
            /* dJ/d(p_view): J02 = -fx px rz2, J12 = -fy py rz2, J00 = fx rz, J11 = fy rz */
            const float vt[3] = {-fx_rz2 * vJ[0][2], -fy_rz2 * vJ[1][2],
                                 -fx_rz2 * vJ[0][0] + 2.f * fx * px * rz3 * vJ[0][2] - fy_rz2 * vJ[1][1] +
                                     2.f * fy * py * rz3 * vJ[1][2]};
            /* p_view = W p + t: v_mean = W^T v_t */
            for (int k = 0; k < 3; ++k) vmean[k] = Wm[0][k] * vt[0] + Wm[1][k] * vt[1] + Wm[2][k] * vt[2];
        }
        /* scale_rot_to_cov3d_vjp (:1299-1339) */
        {
            const float vV[3][3] = {{vcov[0], 0.5f * vcov[1], 0.5f * vcov[2]},
                                    {0.5f * vcov[1], vcov[3], 0.5f * vcov[4]},
                                    {0.5f * vcov[2], 0.5f * vcov[4], vcov[5]}};
            const float g3[3] = {glob_scale * s[0], glob_scale * s[1], glob_scale * s[2]};
            /* M[r][c] = R[c][r] g_c; v_M = 2 v_V M */
            float M[3][3];
            for (int r = 0; r < 3; ++r) {
                M[r][0] = (r == 0 ? R[0].x : r == 1 ? R[0].y : R[0].z) * g3[0];
                M[r][1] = (r == 0 ? R[1].x : r == 1 ? R[1].y : R[1].z) * g3[1];
                M[r][2] = (r == 0 ? R[2].x : r == 1 ? R[2].y : R[2].z) * g3[2];
            }
            float vM[3][3];
            for (int r = 0; r < 3; ++r)
                for (int c = 0; c < 3; ++c) {
                    const float x = vV[r][0] * M[0][c] + vV[r][1] * M[1][c] + vV[r][2] * M[2][c];
                    vM[r][c] = 2.f * x;
                }
            /* v_S_c = column c of R . column c of v_M; v_R = v_M S */
            f3 vR[3];
            for (int c = 0; c < 3; ++c) {
                const float vs = R[c].x * vM[0][c] + R[c].y * vM[1][c] + R[c].z * vM[2][c];
                dscales[3 * i + c] = vs * glob_scale * s[c];  /* d/d(log scale) */
                vR[c] = {vM[0][c] * g3[c], vM[1][c] * g3[c], vM[2][c] * g3[c]};
            }
            quat_to_rotmat_vjp(q, vR, dquats + 4 * i);
        }
        /* project_pix_vjp (:1059-1077) */
        {
            const float hw = pm[12] * p[0] + pm[13] * p[1] + pm[14] * p[2] + pm[15];
            const float rw = 1.f / (hw + 1e-6f);
            const float hx = pm[0] * p[0] + pm[1] * p[1] + pm[2] * p[2] + pm[3];
            const float hy = pm[4] * p[0] + pm[5] * p[1] + pm[6] * p[2] + pm[7];
            const float vnx = 0.5f * (float)cam->width * g[0], vny = 0.5f * (float)cam->height * g[1];
            /* xy = f(h.xy / h.w): d/dh.x = vnx rw, d/dh.y = vny rw,
             * d/dh.w = -(vnx hx + vny hy) rw^2 */
            const float vhx = vnx * rw, vhy = vny * rw, vhw = -(vnx * hx + vny * hy) * rw * rw;
            for (int k = 0; k < 3; ++k) vmean[k] += pm[k] * vhx + pm[4 + k] * vhy + pm[12 + k] * vhw;
            dmean2d[2 * i] = vnx;
            dmean2d[2 * i + 1] = vny;
        }
        for (int k = 0; k < 3; ++k) dmeans[3 * i + k] = vmean[k];
        /* SH backward (as the 2DGS projection backward) */
        const f3 dir_un = {p[0] - cam->cam_pos[0], p[1] - cam->cam_pos[1], p[2] - cam->cam_pos[2]};
        const f3 dir = normalize3(dir_un);
        const float *vc = g + 6;
        sh_vjp(dtu, dir, vc, dfdc + 3 * i, dfr);
        if (dtu >= 1) {
            const f3 dd = sh_dL_ddir(dtu, dir, frest + (size_t)K * 3 * i, vc);
            const f3 dm = dnormvdv(dir_un, dd);
            dmeans[3 * i + 0] += dm.x;
            dmeans[3 * i + 1] += dm.y;
            dmeans[3 * i + 2] += dm.z;
        }
        xys_grad_norm[i] += fabsf(dmean2d[2 * i]) + fabsf(dmean2d[2 * i + 1]);
        vis_counts[i] += 1.0f;
        const float r_norm = (float)radii[i] * inv_max_dim;
        if (r_norm > max_2d_size[i]) max_2d_size[i] = r_norm;
    }
}
