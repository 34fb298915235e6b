// k_project.hip -- per-gaussian projection + SH forward, projection + SH
// backward (optionally fused with the six Adam updates), and the gathers
// that materialise per-field views of the packed splat records.
#include "kernels.h"
#include "ms_device.h"

using namespace msd;

namespace {

constexpr int kBlock = 256;

// Copies `count` consecutive floats from global memory to LDS with every
// thread's loads of a round (kStageU per thread) in flight together.
constexpr int kStageU = 12;
__device__ __forceinline__ void stage_rows(float *__restrict__ dst, const float *__restrict__ src, int count) {
    for (int e0 = threadIdx.x; e0 < count; e0 += kStageU * kBlock) {
        float v[kStageU];
#pragma unroll
        for (int u = 0; u < kStageU; ++u) {
            const int e = e0 + u * kBlock;
            v[u] = e < count ? src[e] : 0.f;
        }
#pragma unroll
        for (int u = 0; u < kStageU; ++u) {
            const int e = e0 + u * kBlock;
            if (e < count) dst[e] = v[u];
        }
    }
}

// LDS of the projection forwards: half a block's features_rest rows (128 x
// 45 floats), reused to stage the outgoing records (up to 5 float4 per
// thread).  23 KB, so six workgroups share a CU.
constexpr int kStageRows = kBlock / 2;
constexpr int kStageFloats = kStageRows * 45;
static_assert(kStageFloats * 4 >= kBlock * 5 * 16, "record staging fits the SH staging buffer");

// The colour of this thread's splat (sh_coeffs_to_color, sh_eval) with the
// block's features_rest rows staged through s_fr with coalesced loads, half
// the block's rows at a time: threads [0, 128) evaluate from the first half,
// then [128, 256) from the second.  Rows of more than 45 floats (degree 4)
// are read from global memory.  Called by every thread of the block (it
// holds barriers); threads with `active` false only take part in them.
__device__ __forceinline__ void sh_color_staged(const MsplatCamera &cam, int K3, int b0, int cnt,
                                                const float *__restrict__ frest, const float *__restrict__ fdc,
                                                const float p[3], bool active, float *s_fr, float col[3]) {
    const int i = b0 + (int)threadIdx.x;
    const f3 dir = normalize3({p[0] - cam.cam_pos[0], p[1] - cam.cam_pos[1], p[2] - cam.cam_pos[2]});
    const float *dc = fdc + 3 * (size_t)(active ? i : 0);
    if (cam.degrees_to_use <= 0 || K3 > 45) {
        if (active) sh_eval(cam.degrees_to_use, dir, dc, frest + (size_t)K3 * i, col);
        return;
    }
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const int r0 = h * kStageRows, rows = min(kStageRows, cnt - r0);
        if (rows <= 0) break;  // uniform
        if (h) __syncthreads();
        stage_rows(s_fr, frest + (size_t)(b0 + r0) * K3, rows * K3);
        __syncthreads();
        const int t = (int)threadIdx.x - r0;
        if (active && t >= 0 && t < kStageRows) sh_eval(cam.degrees_to_use, dir, dc, s_fr + t * K3, col);
    }
}

// project_and_sh_forward_2dgs_kernel (msplat_metal.metal:1413-1521), with
// the sigmoid of the sort/pack stage (:1684) and the raster's colour clamp
// (:619) folded into the record.  Also sums the visible splats' tile
// rectangle areas, the number of tile intersections the binning will emit
// (one 64-bit atomic per workgroup).
__global__ __launch_bounds__(kBlock) void k_project_fwd(
    MsplatCamera cam, int n, const float *__restrict__ means, const float *__restrict__ scales,
    const float *__restrict__ quats, const float *__restrict__ opac, const float *__restrict__ fdc,
    const float *__restrict__ frest, float4 *__restrict__ rec, float4 *__restrict__ mrec, float *__restrict__ depths,
    int *__restrict__ radii, uint2 *__restrict__ rect, unsigned long long *__restrict__ isect_total,
    float *__restrict__ colors_raw) {
    // The block's features_rest rows (up to 45 floats each) pass through LDS
    // with coalesced loads, half a block's rows at a time (sh_color_staged);
    // the same 23 KB then stage the outgoing records.
    __shared__ float s_fr[kStageFloats];
    const int K3 = (num_sh_bases(cam.degree) - 1) * 3;
    const int b0 = blockIdx.x * kBlock;
    const int cnt = min(kBlock, n - b0);
    // No early return: every thread takes part in the intersection sum.
    const int i = blockIdx.x * kBlock + threadIdx.x;
    const bool valid = i < n;
    const int ii = valid ? i : 0;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    // this splat's record and quadrant-mask record, written out through LDS
    float4 ro[5] = {z4, z4, z4, z4, z4}, mo[3] = {z4, z4, z4};
    const float *vm = cam.viewmat, *pm = cam.projmat;
    const float p[3] = {means[3 * (size_t)ii], means[3 * (size_t)ii + 1], means[3 * (size_t)ii + 2]};
    const float pz = vm[8] * p[0] + vm[9] * p[1] + vm[10] * p[2] + vm[11];

    bool ok = valid && pz > cam.clip_thresh;
    f3 R0, R1, R2;
    float cxp = 0.f, cyp = 0.f, radius = 0.f;
    f3 T0, T1, T2;
    int x0 = 0, y0 = 0, x1 = 0, y1 = 0;
    if (ok) {
        const float sx = ms_expf(scales[2 * (size_t)i]), sy = ms_expf(scales[2 * (size_t)i + 1]);
        const float4 qv = reinterpret_cast<const float4 *>(quats)[i];
        const float q[4] = {qv.x, qv.y, qv.z, qv.w};
        quat_to_rotmat(q, R0, R1, R2);
        const float sxg = sx * cam.glob_scale, syg = sy * cam.glob_scale;
        const f3 tu = {R0.x * sxg, R0.y * sxg, R0.z * sxg};
        const f3 tv = {R1.x * syg, R1.y * syg, R1.z * syg};
        const ClipCols cc = clip_columns(p, tu, tv, pm);
        const float halfW = 0.5f * (float)cam.width, halfH = 0.5f * (float)cam.height;
        const float bx = cam.cx - 0.5f, by = cam.cy - 0.5f;
        const f3 cu = {halfW * cc.tu[0] + bx * cc.tu[3], halfH * cc.tu[1] + by * cc.tu[3], cc.tu[3]};
        const f3 cv = {halfW * cc.tv[0] + bx * cc.tv[3], halfH * cc.tv[1] + by * cc.tv[3], cc.tv[3]};
        const f3 co = {halfW * cc.pc[0] + bx * cc.pc[3], halfH * cc.pc[1] + by * cc.pc[3], cc.pc[3]};
        T0 = {cu.x, cv.x, co.x};
        T1 = {cu.y, cv.y, co.y};
        T2 = {cu.z, cv.z, co.z};
        // compute_aabb_2dgs, cutoff 3 (msplat_metal.metal:302-330)
        const float cutoff = 3.0f;
        const f3 t = {cutoff * cutoff, cutoff * cutoff, -1.0f};
        const float dd = dot3(t, mul3(T2, T2));
        ok = dd != 0.0f;
        if (ok) {
            const float invd = 1.0f / dd;
            const f3 f = {invd * t.x, invd * t.y, invd * t.z};
            cxp = dot3(f, mul3(T0, T2));
            cyp = dot3(f, mul3(T1, T2));
            const float h0x = cxp * cxp - dot3(f, mul3(T0, T0));
            const float h0y = cyp * cyp - dot3(f, mul3(T1, T1));
            const float hx = __builtin_sqrtf(__builtin_fmaxf(1e-4f, h0x));
            const float hy = __builtin_sqrtf(__builtin_fmaxf(1e-4f, h0y));
            radius = __builtin_ceilf(__builtin_fmaxf(__builtin_fmaxf(hx, hy), cutoff * FILTER_SIZE));
            // get_tile_bbox (msplat_metal.metal:62-92)
            const float tcx = cxp / 16.0f, tcy = cyp / 16.0f, tr = radius / 16.0f;
            x0 = min(max(0, f2i(tcx - tr)), cam.tiles_x);
            x1 = min(max(0, f2i(tcx + tr + 1)), cam.tiles_x);
            y0 = min(max(0, f2i(tcy - tr)), cam.tiles_y);
            y1 = min(max(0, f2i(tcy + tr + 1)), cam.tiles_y);
            ok = (x1 - x0) * (y1 - y0) > 0;
        }
    }
    if (!ok) {
        if (valid) {
            radii[i] = 0;
            depths[i] = 0.f;
            rect[i] = make_uint2(0u, 0u);
            if (colors_raw) {
                colors_raw[3 * (size_t)i] = colors_raw[3 * (size_t)i + 1] = colors_raw[3 * (size_t)i + 2] = 0.f;
            }
        }
    }
    float col[3];
    sh_color_staged(cam, K3, b0, cnt, frest, fdc, p, ok, s_fr, col);
    if (ok) {
        const float opa = ms_sigmoid(opac[i]);

        radii[i] = (int)radius;
        depths[i] = pz;
        rect[i] = make_uint2((uint32_t)x0 | ((uint32_t)y0 << 16), (uint32_t)x1 | ((uint32_t)y1 << 16));
        const float4 q0 = make_float4(T0.x, T0.y, T0.z, T1.x), q1 = make_float4(T1.y, T1.z, T2.x, T2.y),
                     q2 = make_float4(T2.z, cxp, cyp, opa);
        // the splat-only part of the rasterizer's quadrant-mask test
        const float tau = splat_reach(opa);
        f3 CR0, CAx, CAy;
        centred_rows(T0, T1, T2, cxp, cyp, CR0, CAx, CAy);
        float lp_r2;
        const MaskRec mr = mask_record(q0, q1, q2, tau, CR0, CAx, CAy, x0, y0, x1, y1, lp_r2);
        ro[0] = q0;
        ro[1] = q1;
        ro[2] = q2;
        ro[3] = make_float4(R2.x, R2.y, R2.z, __builtin_fmaxf(col[0] + 0.5f, 0.0f));
        ro[4] = make_float4(__builtin_fmaxf(col[1] + 0.5f, 0.0f), __builtin_fmaxf(col[2] + 0.5f, 0.0f), tau, lp_r2);
        mo[0] = mr.box;
        mo[1] = mr.e;
        mo[2] = mr.h;
        if (colors_raw) {
            colors_raw[3 * (size_t)i] = col[0];
            colors_raw[3 * (size_t)i + 1] = col[1];
            colors_raw[3 * (size_t)i + 2] = col[2];
        }
    }
    // The block's records leave as contiguous rows: each thread's 5 float4
    // (then its 3 mask float4) go through LDS, and every store instruction
    // writes 1 KB of consecutive float4s.
    {
        float4 *s4 = reinterpret_cast<float4 *>(s_fr);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 5; ++k) s4[5 * threadIdx.x + k] = ro[k];
        __syncthreads();
        float4 *rdst = rec + 5 * (size_t)b0, *mdst = mrec + 3 * (size_t)b0;
        for (int e = threadIdx.x; e < 5 * cnt; e += kBlock) rdst[e] = s4[e];
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 3; ++k) s4[3 * threadIdx.x + k] = mo[k];
        __syncthreads();
        for (int e = threadIdx.x; e < 3 * cnt; e += kBlock) mdst[e] = s4[e];
    }
    // intersections: sum of the rectangle areas over the workgroup
    __shared__ unsigned long long s_area[kBlock / 64];
    unsigned long long area = ok ? (unsigned long long)((x1 - x0) * (y1 - y0)) : 0ull;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) area += __shfl_xor(area, d, 64);
    if ((threadIdx.x & 63) == 0) s_area[threadIdx.x >> 6] = area;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int w = 0; w < kBlock / 64; ++w) t += s_area[w];
        if (t) atomicAdd(isect_total, t);
    }
}

// One Adam step on one element: fused_adam_kernel (msplat_metal.metal:1383-1406).
__device__ __forceinline__ void adam_elem(float *p, float *m_, float *v_, size_t idx, float g, float step,
                                          float b1, float b2, float bc2_sqrt, float eps) {
    const float m = __builtin_fmaf(b1, m_[idx], (1.0f - b1) * g);
    const float v = __builtin_fmaf(b2, v_[idx], (1.0f - b2) * g * g);
    p[idx] -= step * m / (__builtin_sqrtf(v) / bc2_sqrt + eps);
    m_[idx] = m;
    v_[idx] = v;
}

// Adam on the N consecutive elements of one splat's row: all loads first,
// then the updates (adam_elem's operations, element by element), then all
// stores, so the row moves as vector loads and stores.
template <int N>
__device__ __forceinline__ void adam_row(float *p, float *m_, float *v_, size_t base, const float *g, float step,
                                         float b1, float b2, float bc2_sqrt, float eps) {
    float pv[N], mv[N], vv[N];
#pragma unroll
    for (int k = 0; k < N; ++k) pv[k] = p[base + k];
#pragma unroll
    for (int k = 0; k < N; ++k) mv[k] = m_[base + k];
#pragma unroll
    for (int k = 0; k < N; ++k) vv[k] = v_[base + k];
#pragma unroll
    for (int k = 0; k < N; ++k) {
        const float m = __builtin_fmaf(b1, mv[k], (1.0f - b1) * g[k]);
        const float v = __builtin_fmaf(b2, vv[k], (1.0f - b2) * g[k] * g[k]);
        pv[k] -= step * m / (__builtin_sqrtf(v) / bc2_sqrt + eps);
        mv[k] = m;
        vv[k] = v;
    }
#pragma unroll
    for (int k = 0; k < N; ++k) p[base + k] = pv[k];
#pragma unroll
    for (int k = 0; k < N; ++k) m_[base + k] = mv[k];
#pragma unroll
    for (int k = 0; k < N; ++k) v_[base + k] = vv[k];
}

struct AdamDev {
    float *m[6];
    float *v[6];
    float step[6];
    float b1, b2, bc2_sqrt, eps;
    // the launch does nothing when *skip > skip_above (an overflowed blend
    // log: the raster gradients are incomplete and the step is redone)
    const int *skip;
    int skip_above;
};

// Nine transMat gradients from the ray moments the image-only raster
// backward accumulates about the splat centre (xs, ys): S0 = sum dp,
// X = sum (xs - px) dp, Y = sum (ys - py) dp over the pixels (dp = the
// upstream gradient of the pixel's ray).  With Tu' = Tu - xs Tw and
// Tv' = Tv - ys Tw, k = px Tw - Tu = (px - xs) Tw - Tu' and l likewise, so
// the reference's per-pixel terms -l x dp, -dp x k and px (l x dp) +
// py (dp x k) (msplat_metal.metal:1930-1955) sum to the expressions below;
// the (px - xs)(py - ys) terms cancel exactly.  Centring keeps every
// product at the splat's own scale (absolute pixel coordinates would make
// the cross products cancel catastrophically).
__device__ __forceinline__ void moments_to_dT(f3 Tu, f3 Tv, f3 Tw, float xs, float ys, float g[9]) {
    const f3 S0 = {g[0], g[1], g[2]}, X = {g[3], g[4], g[5]}, Y = {g[6], g[7], g[8]};
    const f3 Tu_ = {Tu.x - xs * Tw.x, Tu.y - xs * Tw.y, Tu.z - xs * Tw.z};
    const f3 Tv_ = {Tv.x - ys * Tw.x, Tv.y - ys * Tw.y, Tv.z - ys * Tw.z};
    const f3 a = cross3(Tw, Y), b = cross3(Tv_, S0);
    const f3 c = cross3(X, Tw), d = cross3(S0, Tu_);
    const f3 dU = {a.x + b.x, a.y + b.y, a.z + b.z};
    const f3 dV = {c.x + d.x, c.y + d.y, c.z + d.z};
    const f3 e = cross3(Tv_, X), f = cross3(Tu_, Y);
    g[0] = dU.x;
    g[1] = dU.y;
    g[2] = dU.z;
    g[3] = dV.x;
    g[4] = dV.y;
    g[5] = dV.z;
    g[6] = e.x - f.x - xs * dU.x - ys * dV.x;
    g[7] = e.y - f.y - xs * dU.y - ys * dV.y;
    g[8] = e.z - f.z - xs * dU.z - ys * dV.z;
}

// The image-only raster backward leaves per-splat sums without their
// per-splat factors; this applies them: the nine ray moments times
// -opacity, the opacity sum times the sigmoid's derivative opacity
// (1 - opacity) (msplat_metal.metal:1976), the colour sums masked where the
// colour was clamped at zero (:1873-1880; the record holds the clamped
// colour, positive exactly where the clamp passes the gradient).  Then the
// moments become dL/dtransMat.
__device__ __forceinline__ void finish_image_grads(f3 Tu, f3 Tv, f3 Tw, float4 q2, float4 q3, float4 q4,
                                                   float g[16]) {
    const float opa = q2.w;
#pragma unroll
    for (int k = 0; k < 9; ++k) g[k] *= -opa;
    g[12] *= opa * (1.0f - opa);
    g[13] = q3.w > 0.0f ? g[13] : 0.0f;
    g[14] = q4.x > 0.0f ? g[14] : 0.0f;
    g[15] = q4.y > 0.0f ? g[15] : 0.0f;
    moments_to_dT(Tu, Tv, Tw, q2.y, q2.z, g);
}

// project_and_sh_backward_2dgs_kernel (msplat_metal.metal:2003-2209).
// rec non-null: grads16 holds the image-only raster backward's sums (see
// finish_image_grads), finished here with the transMat rows recomputed from
// the parameters and the rest of the splat's record.
// FUSED: the per-gaussian gradients stay on chip and the six Adam groups
// (model.cpp:806-826) are updated in place, so neither the 58-float gradient
// nor a second pass over the parameters touches HBM.
// The 45-float features_rest rows (parameters, both Adam moments, the SH
// gradient) dominate the traffic; they are moved with coalesced
// element-per-thread loops: the block's rows are staged in LDS for the
// view-direction gradient, and the SH gradient basis[b] * v_color[c] is
// formed per element from per-splat (basis, v_color) kept in LDS.
template <bool FUSED>
__global__ __launch_bounds__(kBlock) void k_project_bwd(
    MsplatCamera cam, int n, float *__restrict__ means, float *__restrict__ scales,
    float *__restrict__ quats, float *__restrict__ opac, float *__restrict__ fdc,
    float *__restrict__ frest, const int *__restrict__ radii, const float *__restrict__ g16,
    float *__restrict__ dmeans, float *__restrict__ dscales, float *__restrict__ dquats,
    float *__restrict__ dmean2d, float *__restrict__ dfdc, float *__restrict__ dfrest,
    float *__restrict__ grad_norm, float *__restrict__ vis, float *__restrict__ max2d, float inv_max_dim,
    AdamDev ad, const float4 *__restrict__ rec) {
    if (ad.skip && *ad.skip > ad.skip_above) return;
    __shared__ float s_basis[kBlock * 24];
    __shared__ float s_vc[kBlock * 3];
    const int nb = num_sh_bases(cam.degree);
    const int K3 = (nb - 1) * 3;
    const int b0 = blockIdx.x * kBlock;
    const int cnt = min(kBlock, n - b0);
    const int sh_deg = cam.degrees_to_use;
    const int i = b0 + threadIdx.x;
    const bool valid = i < n;
    const size_t si = (size_t)(valid ? i : 0);

    float gm[3] = {0.f, 0.f, 0.f}, gs[2] = {0.f, 0.f}, gq[4] = {0.f, 0.f, 0.f, 0.f};
    float gdc[3] = {0.f, 0.f, 0.f}, gm2[2] = {0.f, 0.f};
    float vc[3] = {0.f, 0.f, 0.f};
    float basis[24];
#pragma unroll
    for (int k = 0; k < 24; ++k) basis[k] = 0.f;
    const bool vis_ok = valid && radii[si] > 0;
    float g_opa = 0.f;  // the visible splat's (finished) opacity-logit gradient
    if (vis_ok) {
        const float p[3] = {means[3 * si], means[3 * si + 1], means[3 * si + 2]};
        const float sx = ms_expf(scales[2 * si]), sy = ms_expf(scales[2 * si + 1]);
        const float4 qv = reinterpret_cast<const float4 *>(quats)[si];
        const float q[4] = {qv.x, qv.y, qv.z, qv.w};
        f3 R0, R1, R2;
        quat_to_rotmat(q, R0, R1, R2);
        const float sxg = sx * cam.glob_scale, syg = sy * cam.glob_scale;
        const f3 tu = {R0.x * sxg, R0.y * sxg, R0.z * sxg};
        const f3 tv = {R1.x * syg, R1.y * syg, R1.z * syg};
        const float *pm = cam.projmat;
        const ClipCols cc = clip_columns(p, tu, tv, pm);
        const float W = (float)cam.width, H = (float)cam.height;
        const float halfW = 0.5f * W, halfH = 0.5f * H;
        const float bx = cam.cx - 0.5f, by = cam.cy - 0.5f;
        const float4 *g4 = reinterpret_cast<const float4 *>(g16 + 16 * si);
        const float4 ga = g4[0], gb = g4[1], gc = g4[2], gd = g4[3];
        float g[16] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w,
                       gc.x, gc.y, gc.z, gc.w, gd.x, gd.y, gd.z, gd.w};
        if (rec) {
            // ray moments: the transMat rows as k_project_fwd builds them,
            // the centre from the splat's record
            const f3 cu = {halfW * cc.tu[0] + bx * cc.tu[3], halfH * cc.tu[1] + by * cc.tu[3], cc.tu[3]};
            const f3 cv = {halfW * cc.tv[0] + bx * cc.tv[3], halfH * cc.tv[1] + by * cc.tv[3], cc.tv[3]};
            const f3 co = {halfW * cc.pc[0] + bx * cc.pc[3], halfH * cc.pc[1] + by * cc.pc[3], cc.pc[3]};
            finish_image_grads({cu.x, cv.x, co.x}, {cu.y, cv.y, co.y}, {cu.z, cv.z, co.z}, rec[5 * si + 2],
                               rec[5 * si + 3], rec[5 * si + 4], g);
        }
        const f3 dcu = {g[0], g[3], g[6]}, dcv = {g[1], g[4], g[7]}, dco = {g[2], g[5], g[8]};
        const float du[4] = {halfW * dcu.x, halfH * dcu.y, 0.0f, bx * dcu.x + by * dcu.y + dcu.z};
        const float dv[4] = {halfW * dcv.x, halfH * dcv.y, 0.0f, bx * dcv.x + by * dcv.y + dcv.z};
        const float dpc[4] = {halfW * dco.x, halfH * dco.y, 0.0f, bx * dco.x + by * dco.y + dco.z};
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
        gs[0] = dsx * sx * cam.glob_scale;
        gs[1] = dsy * sy * cam.glob_scale;
        const f3 vR[3] = {{gtu.x * sxg, gtu.y * sxg, gtu.z * sxg},
                          {gtv.x * syg, gtv.y * syg, gtv.z * syg},
                          {g[9], g[10], g[11]}};
        quat_to_rotmat_vjp(q, vR, gq);
        gm[0] = gp.x;
        gm[1] = gp.y;
        gm[2] = gp.z;
        const f3 dir_un = {p[0] - cam.cam_pos[0], p[1] - cam.cam_pos[1], p[2] - cam.cam_pos[2]};
        const f3 dir = normalize3(dir_un);
        g_opa = g[12];
        vc[0] = g[13];
        vc[1] = g[14];
        vc[2] = g[15];
#pragma unroll
        for (int c = 0; c < 3; ++c) gdc[c] = SH_C0 * vc[c];
        sh_vjp_basis(sh_deg, dir, basis);
        if (sh_deg >= 1) {
            const f3 dd = sh_dL_ddir(sh_deg, dir, frest + (size_t)K3 * si, vc);
            const f3 dm = dnormvdv(dir_un, dd);
            gm[0] += dm.x;
            gm[1] += dm.y;
            gm[2] += dm.z;
        }
        const float depth_fwd = cc.pc[3];
        gm2[0] = g[6] * depth_fwd * 0.5f * W;
        gm2[1] = g[7] * depth_fwd * 0.5f * H;
        grad_norm[si] += __builtin_fabsf(gm2[0]) + __builtin_fabsf(gm2[1]);
        vis[si] += 1.0f;
        const float r_norm = (float)radii[si] * inv_max_dim;
        if (r_norm > max2d[si]) max2d[si] = r_norm;
    }
    const int nrest = sh_deg >= 4 ? 24 : sh_deg == 3 ? 15 : sh_deg == 2 ? 8 : sh_deg == 1 ? 3 : 0;
    // dL_dopacity is read for every splat, as the reference's Adam reads the
    // raster's opacity-gradient buffer (zero for culled splats).
    const float gop = vis_ok ? g_opa : valid ? g16[16 * si + 12] : 0.f;
    if (valid) {
        if (!FUSED) {
            for (int k = 0; k < 3; ++k) dmeans[3 * si + k] = gm[k];
            for (int k = 0; k < 2; ++k) dscales[2 * si + k] = gs[k];
            for (int k = 0; k < 4; ++k) dquats[4 * si + k] = gq[k];
            for (int k = 0; k < 2; ++k) dmean2d[2 * si + k] = gm2[k];
            for (int k = 0; k < 3; ++k) dfdc[3 * si + k] = gdc[k];
        } else {
            adam_row<3>(means, ad.m[0], ad.v[0], 3 * si, gm, ad.step[0], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<2>(scales, ad.m[1], ad.v[1], 2 * si, gs, ad.step[1], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<4>(quats, ad.m[2], ad.v[2], 4 * si, gq, ad.step[2], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<3>(fdc, ad.m[3], ad.v[3], 3 * si, gdc, ad.step[3], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<1>(opac, ad.m[5], ad.v[5], si, &gop, ad.step[5], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
        }
    }
    if (K3 == 0) return;
    // features_rest: gradient basis[b] * v_color[c] (sh_coeffs_to_color_vjp,
    // msplat_metal.metal:825-912; zero above degrees_to_use and for culled
    // splats), written or Adam-updated element by element, coalesced.
    for (int k = 0; k < 24; ++k) s_basis[threadIdx.x * 24 + k] = (k < nrest) ? basis[k] : 0.f;
    for (int c = 0; c < 3; ++c) s_vc[threadIdx.x * 3 + c] = vc[c];
    __syncthreads();
    const size_t base = (size_t)b0 * K3;
    const int total = cnt * K3;
    // element e = (splat gl, coefficient k) of the block's rows, advanced
    // by kBlock elements per step without a division
    int gl = (int)threadIdx.x / K3, k = (int)threadIdx.x - gl * K3;
    const int dgl = kBlock / K3, dk = kBlock - dgl * K3;
    constexpr int U = 8;  // elements per thread with loads in flight together
    for (int e0 = threadIdx.x; e0 < total; e0 += U * kBlock) {
        float gr[U], pv[U], mv[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + u * kBlock;
            const bool act = e < total;
            const int b = k / 3, c = k - 3 * b;
            gr[u] = (act && b < nrest) ? s_basis[gl * 24 + b] * s_vc[gl * 3 + c] : 0.f;
            if (FUSED && act) {
                pv[u] = frest[base + e];
                mv[u] = ad.m[4][base + e];
                vv[u] = ad.v[4][base + e];
            }
            gl += dgl;
            k += dk;
            if (k >= K3) {
                k -= K3;
                ++gl;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + u * kBlock;
            if (e >= total) continue;
            if (!FUSED) {
                dfrest[base + e] = gr[u];
            } else {
                // fused_adam_kernel (msplat_metal.metal:1383-1406), as adam_elem
                const float m = __builtin_fmaf(ad.b1, mv[u], (1.0f - ad.b1) * gr[u]);
                const float v = __builtin_fmaf(ad.b2, vv[u], (1.0f - ad.b2) * gr[u] * gr[u]);
                frest[base + e] = pv[u] - ad.step[4] * m / (__builtin_sqrtf(v) / ad.bc2_sqrt + ad.eps);
                ad.m[4][base + e] = m;
                ad.v[4][base + e] = v;
            }
        }
    }
}

// The image-only raster backward's grads16 rows -> the reference's raster
// gradients (finish_image_grads), in place, with the splat records' rows.
__global__ void k_finish_image_grads(int n, const float4 *__restrict__ rec, float *__restrict__ g16) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const float4 *r = rec + 5 * (size_t)i;
    const float4 q0 = r[0], q1 = r[1];
    float4 *g4 = reinterpret_cast<float4 *>(g16 + 16 * (size_t)i);
    float v[16];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 t = g4[k];
        v[4 * k] = t.x;
        v[4 * k + 1] = t.y;
        v[4 * k + 2] = t.z;
        v[4 * k + 3] = t.w;
    }
    finish_image_grads({q0.x, q0.y, q0.z}, {q0.w, q1.x, q1.y}, {q1.z, q1.w, r[2].x}, r[2], r[3], r[4], v);
#pragma unroll
    for (int k = 0; k < 4; ++k) g4[k] = make_float4(v[4 * k], v[4 * k + 1], v[4 * k + 2], v[4 * k + 3]);
}

__global__ void k_gather(const float *__restrict__ src, int src_stride, int src_off, int nf,
                         float *__restrict__ dst, int n) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)n * nf) return;
    const int64_t i = t / nf, k = t - i * nf;
    dst[t] = src[i * src_stride + src_off + k];
}

__global__ void k_tiles_hit(const uint2 *__restrict__ rect, const int *__restrict__ radii, int *__restrict__ out, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint2 r = rect[i];
    const int x0 = r.x & 0xffff, y0 = r.x >> 16, x1 = r.y & 0xffff, y1 = r.y >> 16;
    out[i] = radii[i] > 0 ? (x1 - x0) * (y1 - y0) : 0;
}

// ---- 3DGS mode --------------------------------------------------------
// Projection of 3D Gaussians on the reference's EWA helpers (dead code in
// the 2DGS fork): scale_rot_to_cov3d (msplat_metal.metal:160-176),
// project_cov3d_ewa (:333-378), compute_cov2d_bounds (:420-441),
// project_pix (:444-452) and their VJPs (:1059-1374).  Expressions follow
// the golden model's restatement operation for operation (no contraction),
// so the projection and its backward agree with it bit for bit.
// Record (MSPLAT_REC3_FLOATS = 12): q0 = (x, y, conic a, conic b),
// q1 = (conic c, opacity, 0, 0), q2 = (r, g, b, 0), rgb = max(SH + 0.5, 0);
// the N records are followed by N boxes (xmin, xmax, ymin, ymax) bounding
// the pixels where alpha can reach 1/255, for the quadrant masks.

// M = R diag(glob s), cov = M M^T (upper triangle); R = rotation columns.
__device__ __forceinline__ void cov3d_of(const float s[3], float glob, const float q[4], float cov[6], f3 R[3]) {
    quat_to_rotmat(q, R[0], R[1], R[2]);
    const float g0 = glob * s[0], g1 = glob * s[1], g2 = glob * s[2];
    const float M[3][3] = {{R[0].x * g0, R[1].x * g1, R[2].x * g2},
                           {R[0].y * g0, R[1].y * g1, R[2].y * g2},
                           {R[0].z * g0, R[1].z * g1, R[2].z * g2}};
#define MS_MM(i, j) (M[i][0] * M[j][0] + M[i][1] * M[j][1] + M[i][2] * M[j][2])
    cov[0] = MS_MM(0, 0);
    cov[1] = MS_MM(0, 1);
    cov[2] = MS_MM(0, 2);
    cov[3] = MS_MM(1, 1);
    cov[4] = MS_MM(1, 2);
    cov[5] = MS_MM(2, 2);
#undef MS_MM
}

// the fov-clamped view position of project_cov3d_ewa (:345-347)
__device__ __forceinline__ void ewa_clamp(float &px, float &py, float pz, float tan_fovx, float tan_fovy) {
    const float lim_x = 1.3f * tan_fovx, lim_y = 1.3f * tan_fovy;
    px = pz * __builtin_fminf(lim_x, __builtin_fmaxf(-lim_x, px / pz));
    py = pz * __builtin_fminf(lim_y, __builtin_fmaxf(-lim_y, py / pz));
}

// cov2d = T V T^T + 0.3 I with T = J W (project_cov3d_ewa)
__device__ __forceinline__ void ewa_cov2d(const float cov[6], const float *vm, float fx, float fy, float tan_fovx,
                                          float tan_fovy, const float pv[3], float c2[3]) {
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

// compute_cov2d_bounds: conic = cov2d^-1 and the 3-sigma radius
__device__ __forceinline__ bool cov2d_bounds(const float c2[3], float cn[3], float &radius) {
    const float det = c2[0] * c2[2] - c2[1] * c2[1];
    if (det == 0.f) return false;
    const float inv_det = 1.f / det;
    cn[0] = c2[2] * inv_det;
    cn[1] = -c2[1] * inv_det;
    cn[2] = c2[0] * inv_det;
    const float b = 0.5f * (c2[0] + c2[2]);
    const float disc = __builtin_sqrtf(__builtin_fmaxf(0.1f, b * b - det));
    radius = __builtin_ceilf(3.f * __builtin_sqrtf(b + disc));
    return true;
}

// the view position W p + t
__device__ __forceinline__ void view_pos(const float *vm, const float p[3], float pv[3]) {
    pv[0] = vm[0] * p[0] + vm[1] * p[1] + vm[2] * p[2] + vm[3];
    pv[1] = vm[4] * p[0] + vm[5] * p[1] + vm[6] * p[2] + vm[7];
    pv[2] = vm[8] * p[0] + vm[9] * p[1] + vm[10] * p[2] + vm[11];
}

__global__ __launch_bounds__(kBlock) void k_project3d_fwd(
    MsplatCamera cam, int n, const float *__restrict__ means, const float *__restrict__ scales,
    const float *__restrict__ quats, const float *__restrict__ opac, const float *__restrict__ fdc,
    const float *__restrict__ frest, float4 *__restrict__ rec, float4 *__restrict__ boxes,
    float *__restrict__ depths, int *__restrict__ radii, uint2 *__restrict__ rect,
    unsigned long long *__restrict__ isect_total, float *__restrict__ colors_raw) {
    __shared__ float s_fr[kStageFloats];
    const int K3 = (num_sh_bases(cam.degree) - 1) * 3;
    const int b0 = blockIdx.x * kBlock;
    const int cnt = min(kBlock, n - b0);
    const int i = blockIdx.x * kBlock + threadIdx.x;
    const bool valid = i < n;
    const int ii = valid ? i : 0;
    const float4 z4 = make_float4(0.f, 0.f, 0.f, 0.f);
    float4 ro[3] = {z4, z4, z4}, bo = z4;
    const float *vm = cam.viewmat;
    const float p[3] = {means[3 * (size_t)ii], means[3 * (size_t)ii + 1], means[3 * (size_t)ii + 2]};
    float pv[3];
    view_pos(vm, p, pv);
    // clip_near_plane (:139-150)
    bool ok = valid && !(pv[2] <= cam.clip_thresh);
    float c2[3] = {0.f, 0.f, 0.f}, cn[3] = {0.f, 0.f, 0.f}, radius = 0.f, xy[2] = {0.f, 0.f};
    int x0 = 0, y0 = 0, x1 = 0, y1 = 0;
    if (ok) {
        const float s[3] = {ms_expf(scales[3 * (size_t)i]), ms_expf(scales[3 * (size_t)i + 1]),
                            ms_expf(scales[3 * (size_t)i + 2])};
        const float4 qv = reinterpret_cast<const float4 *>(quats)[i];
        const float q[4] = {qv.x, qv.y, qv.z, qv.w};
        float cov[6];
        f3 R[3];
        cov3d_of(s, cam.glob_scale, q, cov, R);
        const float tan_fovx = 0.5f * (float)cam.width / cam.fx, tan_fovy = 0.5f * (float)cam.height / cam.fy;
        ewa_cov2d(cov, vm, cam.fx, cam.fy, tan_fovx, tan_fovy, pv, c2);
        ok = cov2d_bounds(c2, cn, radius);
        if (ok) {
            // project_pix + ndc2pix (:444-452, :58-60)
            const float *pm = cam.projmat;
            const float hx = pm[0] * p[0] + pm[1] * p[1] + pm[2] * p[2] + pm[3];
            const float hy = pm[4] * p[0] + pm[5] * p[1] + pm[6] * p[2] + pm[7];
            const float hw = pm[12] * p[0] + pm[13] * p[1] + pm[14] * p[2] + pm[15];
            const float rw = 1.f / (hw + 1e-6f);
            xy[0] = 0.5f * (float)cam.width * (hx * rw) + cam.cx - 0.5f;
            xy[1] = 0.5f * (float)cam.height * (hy * rw) + cam.cy - 0.5f;
            // get_tile_bbox (:62-92)
            const float tcx = xy[0] / 16.0f, tcy = xy[1] / 16.0f, tr = radius / 16.0f;
            x0 = min(max(0, f2i(tcx - tr)), cam.tiles_x);
            x1 = min(max(0, f2i(tcx + tr + 1)), cam.tiles_x);
            y0 = min(max(0, f2i(tcy - tr)), cam.tiles_y);
            y1 = min(max(0, f2i(tcy + tr + 1)), cam.tiles_y);
            ok = (x1 - x0) * (y1 - y0) > 0;
        }
    }
    if (!ok) {
        if (valid) {
            radii[i] = 0;
            depths[i] = 0.f;
            rect[i] = make_uint2(0u, 0u);
            if (colors_raw) colors_raw[3 * (size_t)i] = colors_raw[3 * (size_t)i + 1] = colors_raw[3 * (size_t)i + 2] = 0.f;
        }
    }
    float col[3];
    sh_color_staged(cam, K3, b0, cnt, frest, fdc, p, ok, s_fr, col);
    if (ok) {
        const float opa = ms_sigmoid(opac[i]);
        radii[i] = (int)radius;
        depths[i] = pv[2];
        rect[i] = make_uint2((uint32_t)x0 | ((uint32_t)y0 << 16), (uint32_t)x1 | ((uint32_t)y1 << 16));
        ro[0] = make_float4(xy[0], xy[1], cn[0], cn[1]);
        ro[1] = make_float4(cn[2], opa, 0.f, 0.f);
        ro[2] = make_float4(__builtin_fmaxf(col[0] + 0.5f, 0.0f), __builtin_fmaxf(col[1] + 0.5f, 0.0f),
                            __builtin_fmaxf(col[2] + 0.5f, 0.0f), 0.f);
        bo = gauss3_box(xy[0], xy[1], c2, splat_reach(opa));
        if (colors_raw) {
            colors_raw[3 * (size_t)i] = col[0];
            colors_raw[3 * (size_t)i + 1] = col[1];
            colors_raw[3 * (size_t)i + 2] = col[2];
        }
    }
    // records and boxes leave as contiguous rows through LDS
    {
        float4 *s4 = reinterpret_cast<float4 *>(s_fr);
        __syncthreads();
#pragma unroll
        for (int k = 0; k < 3; ++k) s4[3 * threadIdx.x + k] = ro[k];
        s4[3 * kBlock + threadIdx.x] = bo;
        __syncthreads();
        float4 *rdst = rec + 3 * (size_t)b0, *bdst = boxes + (size_t)b0;
        for (int e = threadIdx.x; e < 3 * cnt; e += kBlock) rdst[e] = s4[e];
        for (int e = threadIdx.x; e < cnt; e += kBlock) bdst[e] = s4[3 * kBlock + e];
    }
    __shared__ unsigned long long s_area[kBlock / 64];
    unsigned long long area = ok ? (unsigned long long)((x1 - x0) * (y1 - y0)) : 0ull;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) area += __shfl_xor(area, d, 64);
    if ((threadIdx.x & 63) == 0) s_area[threadIdx.x >> 6] = area;
    __syncthreads();
    if (threadIdx.x == 0) {
        unsigned long long t = 0;
        for (int w = 0; w < kBlock / 64; ++w) t += s_area[w];
        if (t) atomicAdd(isect_total, t);
    }
}

// The 3DGS raster backward's per-splat sums -> the raster gradients
// [dL/dxy 2, dL/dconic 3 (the off-diagonal entry is the derivative by one
// of the two symmetric matrix entries, as cov2d_to_conic_vjp expects),
// dL/dopacity logit, dL/dcolor 3].  The sums, over the pixels the splat
// blends, are of gg = G dL/dalpha times dx^2, dx dy, dy^2, dx, dy and 1
// (d = centre - pixel) and of alpha T dL/dpixel; with v_sigma = -opacity gg
// the per-pixel gradients (dL/dxy = v_sigma conic d, dL/dconic =
// v_sigma / 2 d d^T, dL/dopacity logit = gg opacity (1 - opacity)) are
// linear in them.  Colour sums are masked where the +0.5 clamp is active.
__device__ __forceinline__ void finish3d_grads(const float4 &q0, const float4 &q1, const float4 &q2, float g[16]) {
    const float a = q0.z, b = q0.w, c = q1.x, opa = q1.y;
    const float Sxx = g[0], Sxy = g[1], Syy = g[2], Sx = g[3], Sy = g[4], So = g[5];
    g[0] = -opa * (a * Sx + b * Sy);
    g[1] = -opa * (b * Sx + c * Sy);
    g[2] = -0.5f * opa * Sxx;
    g[3] = -0.5f * opa * Sxy;
    g[4] = -0.5f * opa * Syy;
    g[5] = So * (opa * (1.0f - opa));
    g[6] = q2.x > 0.0f ? g[6] : 0.0f;
    g[7] = q2.y > 0.0f ? g[7] : 0.0f;
    g[8] = q2.z > 0.0f ? g[8] : 0.0f;
}

__global__ void k_finish3d_grads(int n, const float4 *__restrict__ rec, float *__restrict__ g16) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float g[16];
    float4 *g4 = reinterpret_cast<float4 *>(g16 + 16 * (size_t)i);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 v = g4[k];
        g[4 * k] = v.x;
        g[4 * k + 1] = v.y;
        g[4 * k + 2] = v.z;
        g[4 * k + 3] = v.w;
    }
    finish3d_grads(rec[3 * (size_t)i], rec[3 * (size_t)i + 1], rec[3 * (size_t)i + 2], g);
#pragma unroll
    for (int k = 0; k < 4; ++k) g4[k] = make_float4(g[4 * k], g[4 * k + 1], g[4 * k + 2], g[4 * k + 3]);
}

// The 3DGS projection + SH backward: raster gradients (finished here from
// the raster backward's sums when rec is given) -> the parameter
// gradients, through cov2d_to_conic_vjp (:1080-1093), project_cov3d_ewa_vjp
// (:1110-1179), scale_rot_to_cov3d_vjp (:1299-1339) and the derivative of
// the homogeneous projection (project_pix_vjp, :1059-1077, which drops the
// term through w; the exact one here), plus the SH backward.  FUSED applies
// the six Adam updates in place, as k_project_bwd<true>.  dmean2d and the
// densification statistic use dL/dxy in NDC units (0.5 W, 0.5 H per pixel).
template <bool FUSED>
__global__ __launch_bounds__(kBlock) void k_project3d_bwd(
    MsplatCamera cam, int n, float *__restrict__ means, float *__restrict__ scales,
    float *__restrict__ quats, float *__restrict__ opac, float *__restrict__ fdc,
    float *__restrict__ frest, const int *__restrict__ radii, const float *__restrict__ g16,
    float *__restrict__ dmeans, float *__restrict__ dscales, float *__restrict__ dquats,
    float *__restrict__ dmean2d, float *__restrict__ dfdc, float *__restrict__ dfrest,
    float *__restrict__ grad_norm, float *__restrict__ vis, float *__restrict__ max2d, float inv_max_dim,
    AdamDev ad, const float4 *__restrict__ rec) {
    if (ad.skip && *ad.skip > ad.skip_above) return;
    __shared__ float s_basis[kBlock * 24];
    __shared__ float s_vc[kBlock * 3];
    const int nb = num_sh_bases(cam.degree);
    const int K3 = (nb - 1) * 3;
    const int b0 = blockIdx.x * kBlock;
    const int cnt = min(kBlock, n - b0);
    const int sh_deg = cam.degrees_to_use;
    const int i = b0 + threadIdx.x;
    const bool valid = i < n;
    const size_t si = (size_t)(valid ? i : 0);

    float gm[3] = {0.f, 0.f, 0.f}, gs[3] = {0.f, 0.f, 0.f}, gq[4] = {0.f, 0.f, 0.f, 0.f};
    float gdc[3] = {0.f, 0.f, 0.f}, gm2[2] = {0.f, 0.f};
    float vc[3] = {0.f, 0.f, 0.f};
    float basis[24];
#pragma unroll
    for (int k = 0; k < 24; ++k) basis[k] = 0.f;
    const bool vis_ok = valid && radii[si] > 0;
    float g_opa = 0.f;
    if (vis_ok) {
        const float *vm = cam.viewmat, *pm = cam.projmat;
        const float fx = cam.fx, fy = cam.fy;
        const float tan_fovx = 0.5f * (float)cam.width / fx, tan_fovy = 0.5f * (float)cam.height / fy;
        const float p[3] = {means[3 * si], means[3 * si + 1], means[3 * si + 2]};
        const float4 qv = reinterpret_cast<const float4 *>(quats)[si];
        const float q[4] = {qv.x, qv.y, qv.z, qv.w};
        const float4 *g4 = reinterpret_cast<const float4 *>(g16 + 16 * si);
        const float4 ga = g4[0], gb = g4[1], gc = g4[2], gd = g4[3];
        float g[16] = {ga.x, ga.y, ga.z, ga.w, gb.x, gb.y, gb.z, gb.w,
                       gc.x, gc.y, gc.z, gc.w, gd.x, gd.y, gd.z, gd.w};
        if (rec) finish3d_grads(rec[3 * si], rec[3 * si + 1], rec[3 * si + 2], g);
        float pv[3];
        view_pos(vm, p, pv);
        const float s[3] = {ms_expf(scales[3 * si]), ms_expf(scales[3 * si + 1]), ms_expf(scales[3 * si + 2])};
        float cov[6], c2[3], cn[3], radius;
        f3 R[3];
        cov3d_of(s, cam.glob_scale, q, cov, R);
        ewa_cov2d(cov, vm, fx, fy, tan_fovx, tan_fovy, pv, c2);
        cov2d_bounds(c2, cn, radius);
        // cov2d_to_conic_vjp: v_Sigma = -X G X
        float vc2[3];
        {
            const float X00 = cn[0], X01 = cn[1], X11 = cn[2];
            const float G00 = g[2], G01 = g[3], G11 = g[4];
            const float A00 = X00 * G00 + X01 * G01, A01 = X00 * G01 + X01 * G11;
            const float A10 = X01 * G00 + X11 * G01, A11 = X01 * G01 + X11 * G11;
            const float S00 = -(A00 * X00 + A01 * X01), S01 = -(A00 * X01 + A01 * X11);
            const float S10 = -(A10 * X00 + A11 * X01), S11 = -(A10 * X01 + A11 * X11);
            vc2[0] = S00;
            vc2[1] = S10 + S01;
            vc2[2] = S11;
        }
        // project_cov3d_ewa_vjp
        float vcov[6];
        {
            float px = pv[0], py = pv[1];
            const float pz = pv[2];
            ewa_clamp(px, py, pz, tan_fovx, tan_fovy);
            const float rz = 1.f / pz, rz2 = rz * rz;
            const float Wm[3][3] = {{vm[0], vm[1], vm[2]}, {vm[4], vm[5], vm[6]}, {vm[8], vm[9], vm[10]}};
            const float J[3][3] = {{fx * rz, 0.f, -fx * px * rz2}, {0.f, fy * rz, -fy * py * rz2}, {0.f, 0.f, 0.f}};
            float Tm[3][3];
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int c = 0; c < 3; ++c) Tm[r][c] = J[r][0] * Wm[0][c] + J[r][1] * Wm[1][c] + J[r][2] * Wm[2][c];
            const float V[3][3] = {{cov[0], cov[1], cov[2]}, {cov[1], cov[3], cov[4]}, {cov[2], cov[4], cov[5]}};
            const float vC[3][3] = {{vc2[0], 0.5f * vc2[1], 0.f}, {0.5f * vc2[1], vc2[2], 0.f}, {0.f, 0.f, 0.f}};
            float vCT[3][3], vV[3][3];
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int c = 0; c < 3; ++c) vCT[r][c] = vC[r][0] * Tm[0][c] + vC[r][1] * Tm[1][c] + vC[r][2] * Tm[2][c];
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int c = 0; c < 3; ++c) vV[r][c] = Tm[0][r] * vCT[0][c] + Tm[1][r] * vCT[1][c] + Tm[2][r] * vCT[2][c];
            vcov[0] = vV[0][0];
            vcov[1] = vV[0][1] + vV[1][0];
            vcov[2] = vV[0][2] + vV[2][0];
            vcov[3] = vV[1][1];
            vcov[4] = vV[1][2] + vV[2][1];
            vcov[5] = vV[2][2];
            float vT[3][3];
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const float x = vCT[r][0] * V[0][c] + vCT[r][1] * V[1][c] + vCT[r][2] * V[2][c];
                    vT[r][c] = x + x;
                }
            float vJ[3][3];
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int c = 0; c < 3; ++c) vJ[r][c] = vT[r][0] * Wm[c][0] + vT[r][1] * Wm[c][1] + vT[r][2] * Wm[c][2];
            const float fx_rz2 = fx * rz2, fy_rz2 = fy * rz2, rz3 = rz2 * rz;
            const float vt[3] = {-fx_rz2 * vJ[0][2], -fy_rz2 * vJ[1][2],
                                 -fx_rz2 * vJ[0][0] + 2.f * fx * px * rz3 * vJ[0][2] - fy_rz2 * vJ[1][1] +
                                     2.f * fy * py * rz3 * vJ[1][2]};
#pragma unroll
            for (int k = 0; k < 3; ++k) gm[k] = Wm[0][k] * vt[0] + Wm[1][k] * vt[1] + Wm[2][k] * vt[2];
        }
        // scale_rot_to_cov3d_vjp
        {
            const float vV[3][3] = {{vcov[0], 0.5f * vcov[1], 0.5f * vcov[2]},
                                    {0.5f * vcov[1], vcov[3], 0.5f * vcov[4]},
                                    {0.5f * vcov[2], 0.5f * vcov[4], vcov[5]}};
            const float g3[3] = {cam.glob_scale * s[0], cam.glob_scale * s[1], cam.glob_scale * s[2]};
            const float M[3][3] = {{R[0].x * g3[0], R[1].x * g3[1], R[2].x * g3[2]},
                                   {R[0].y * g3[0], R[1].y * g3[1], R[2].y * g3[2]},
                                   {R[0].z * g3[0], R[1].z * g3[1], R[2].z * g3[2]}};
            float vM[3][3];
#pragma unroll
            for (int r = 0; r < 3; ++r)
#pragma unroll
                for (int c = 0; c < 3; ++c) {
                    const float x = vV[r][0] * M[0][c] + vV[r][1] * M[1][c] + vV[r][2] * M[2][c];
                    vM[r][c] = 2.f * x;
                }
            f3 vR[3];
#pragma unroll
            for (int c = 0; c < 3; ++c) {
                const float vs = R[c].x * vM[0][c] + R[c].y * vM[1][c] + R[c].z * vM[2][c];
                gs[c] = vs * cam.glob_scale * s[c];
                vR[c] = {vM[0][c] * g3[c], vM[1][c] * g3[c], vM[2][c] * g3[c]};
            }
            quat_to_rotmat_vjp(q, vR, gq);
        }
        // the homogeneous projection's derivative
        {
            const float hw = pm[12] * p[0] + pm[13] * p[1] + pm[14] * p[2] + pm[15];
            const float rw = 1.f / (hw + 1e-6f);
            const float hx = pm[0] * p[0] + pm[1] * p[1] + pm[2] * p[2] + pm[3];
            const float hy = pm[4] * p[0] + pm[5] * p[1] + pm[6] * p[2] + pm[7];
            const float vnx = 0.5f * (float)cam.width * g[0], vny = 0.5f * (float)cam.height * g[1];
            const float vhx = vnx * rw, vhy = vny * rw, vhw = -(vnx * hx + vny * hy) * rw * rw;
#pragma unroll
            for (int k = 0; k < 3; ++k) gm[k] += pm[k] * vhx + pm[4 + k] * vhy + pm[12 + k] * vhw;
            gm2[0] = vnx;
            gm2[1] = vny;
        }
        const f3 dir_un = {p[0] - cam.cam_pos[0], p[1] - cam.cam_pos[1], p[2] - cam.cam_pos[2]};
        const f3 dir = normalize3(dir_un);
        g_opa = g[5];
        vc[0] = g[6];
        vc[1] = g[7];
        vc[2] = g[8];
#pragma unroll
        for (int c = 0; c < 3; ++c) gdc[c] = SH_C0 * vc[c];
        sh_vjp_basis(sh_deg, dir, basis);
        if (sh_deg >= 1) {
            const f3 dd = sh_dL_ddir(sh_deg, dir, frest + (size_t)K3 * si, vc);
            const f3 dm = dnormvdv(dir_un, dd);
            gm[0] += dm.x;
            gm[1] += dm.y;
            gm[2] += dm.z;
        }
        grad_norm[si] += __builtin_fabsf(gm2[0]) + __builtin_fabsf(gm2[1]);
        vis[si] += 1.0f;
        const float r_norm = (float)radii[si] * inv_max_dim;
        if (r_norm > max2d[si]) max2d[si] = r_norm;
    }
    const int nrest = sh_deg >= 4 ? 24 : sh_deg == 3 ? 15 : sh_deg == 2 ? 8 : sh_deg == 1 ? 3 : 0;
    if (valid) {
        if (!FUSED) {
            for (int k = 0; k < 3; ++k) dmeans[3 * si + k] = gm[k];
            for (int k = 0; k < 3; ++k) dscales[3 * si + k] = gs[k];
            for (int k = 0; k < 4; ++k) dquats[4 * si + k] = gq[k];
            for (int k = 0; k < 2; ++k) dmean2d[2 * si + k] = gm2[k];
            for (int k = 0; k < 3; ++k) dfdc[3 * si + k] = gdc[k];
        } else {
            adam_row<3>(means, ad.m[0], ad.v[0], 3 * si, gm, ad.step[0], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<3>(scales, ad.m[1], ad.v[1], 3 * si, gs, ad.step[1], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<4>(quats, ad.m[2], ad.v[2], 4 * si, gq, ad.step[2], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<3>(fdc, ad.m[3], ad.v[3], 3 * si, gdc, ad.step[3], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
            adam_row<1>(opac, ad.m[5], ad.v[5], si, &g_opa, ad.step[5], ad.b1, ad.b2, ad.bc2_sqrt, ad.eps);
        }
    }
    if (K3 == 0) return;
    for (int k = 0; k < 24; ++k) s_basis[threadIdx.x * 24 + k] = (k < nrest) ? basis[k] : 0.f;
    for (int c = 0; c < 3; ++c) s_vc[threadIdx.x * 3 + c] = vc[c];
    __syncthreads();
    const size_t base = (size_t)b0 * K3;
    const int total = cnt * K3;
    int gl = (int)threadIdx.x / K3, k = (int)threadIdx.x - gl * K3;
    const int dgl = kBlock / K3, dk = kBlock - dgl * K3;
    constexpr int U = 8;
    for (int e0 = threadIdx.x; e0 < total; e0 += U * kBlock) {
        float gr[U], pvv[U], mv[U], vv[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + u * kBlock;
            const bool act = e < total;
            const int b = k / 3, c = k - 3 * b;
            gr[u] = (act && b < nrest) ? s_basis[gl * 24 + b] * s_vc[gl * 3 + c] : 0.f;
            if (FUSED && act) {
                pvv[u] = frest[base + e];
                mv[u] = ad.m[4][base + e];
                vv[u] = ad.v[4][base + e];
            }
            gl += dgl;
            k += dk;
            if (k >= K3) {
                k -= K3;
                ++gl;
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int e = e0 + u * kBlock;
            if (e >= total) continue;
            if (!FUSED) {
                dfrest[base + e] = gr[u];
            } else {
                const float m = __builtin_fmaf(ad.b1, mv[u], (1.0f - ad.b1) * gr[u]);
                const float v = __builtin_fmaf(ad.b2, vv[u], (1.0f - ad.b2) * gr[u] * gr[u]);
                frest[base + e] = pvv[u] - ad.step[4] * m / (__builtin_sqrtf(v) / ad.bc2_sqrt + ad.eps);
                ad.m[4][base + e] = m;
                ad.v[4][base + e] = v;
            }
        }
    }
}

inline unsigned blocks_for(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

}  // namespace

namespace mskern {

void launch_project_fwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, float *rec,
                        float *mrec, float *depths, int *radii, uint32_t *rect, unsigned long long *isect_total,
                        float *colors_raw) {
    if (g.num_points <= 0) return;
    hipLaunchKernelGGL(k_project_fwd, dim3(blocks_for(g.num_points, kBlock)), dim3(kBlock), 0, s, cam,
                       g.num_points, g.means, g.scales, g.quats, g.opacities, g.features_dc, g.features_rest,
                       reinterpret_cast<float4 *>(rec), reinterpret_cast<float4 *>(mrec), depths, radii,
                       reinterpret_cast<uint2 *>(rect), isect_total, colors_raw);
}

void launch_project_bwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, const int *radii,
                        const float *g16, float *dmeans, float *dscales, float *dquats, float *dmean2d,
                        float *dfdc, float *dfrest, float *grad_norm, float *vis, float *max2d,
                        float inv_max_dim, const MsplatAdam *adam, const float *moments_rec, const int *skip_if, int skip_above) {
    if (g.num_points <= 0) return;
    const auto *mrec = reinterpret_cast<const float4 *>(moments_rec);
    AdamDev ad{};
    ad.skip = skip_if;
    ad.skip_above = skip_above;
    if (adam) {
        for (int k = 0; k < 6; ++k) {
            ad.m[k] = adam->exp_avg[k];
            ad.v[k] = adam->exp_avg_sq[k];
            ad.step[k] = adam->step_size[k];
        }
        ad.b1 = adam->beta1;
        ad.b2 = adam->beta2;
        ad.bc2_sqrt = adam->bc2_sqrt;
        ad.eps = adam->eps;
        hipLaunchKernelGGL(k_project_bwd<true>, dim3(blocks_for(g.num_points, kBlock)), dim3(kBlock), 0, s,
                           cam, g.num_points, g.means, g.scales, g.quats, g.opacities, g.features_dc,
                           g.features_rest, radii, g16, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                           grad_norm, vis, max2d, inv_max_dim, ad, mrec);
    } else {
        hipLaunchKernelGGL(k_project_bwd<false>, dim3(blocks_for(g.num_points, kBlock)), dim3(kBlock), 0, s,
                           cam, g.num_points, g.means, g.scales, g.quats, g.opacities, g.features_dc,
                           g.features_rest, radii, g16, dmeans, dscales, dquats, dmean2d, dfdc, dfrest,
                           grad_norm, vis, max2d, inv_max_dim, ad, mrec);
    }
}

void launch_project3d_fwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, float *rec,
                          float *boxes, float *depths, int *radii, uint32_t *rect, unsigned long long *isect_total,
                          float *colors_raw) {
    if (g.num_points <= 0) return;
    hipLaunchKernelGGL(k_project3d_fwd, dim3(blocks_for(g.num_points, kBlock)), dim3(kBlock), 0, s, cam,
                       g.num_points, g.means, g.scales, g.quats, g.opacities, g.features_dc, g.features_rest,
                       reinterpret_cast<float4 *>(rec), reinterpret_cast<float4 *>(boxes), depths, radii,
                       reinterpret_cast<uint2 *>(rect), isect_total, colors_raw);
}

void launch_project3d_bwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, const int *radii,
                          const float *g16, float *dmeans, float *dscales, float *dquats, float *dmean2d,
                          float *dfdc, float *dfrest, float *grad_norm, float *vis, float *max2d,
                          float inv_max_dim, const MsplatAdam *adam, const float *sums_rec, const int *skip_if, int skip_above) {
    if (g.num_points <= 0) return;
    const auto *r4 = reinterpret_cast<const float4 *>(sums_rec);
    AdamDev ad{};
    ad.skip = skip_if;
    ad.skip_above = skip_above;
    if (adam) {
        for (int k = 0; k < 6; ++k) {
            ad.m[k] = adam->exp_avg[k];
            ad.v[k] = adam->exp_avg_sq[k];
            ad.step[k] = adam->step_size[k];
        }
        ad.b1 = adam->beta1;
        ad.b2 = adam->beta2;
        ad.bc2_sqrt = adam->bc2_sqrt;
        ad.eps = adam->eps;
        hipLaunchKernelGGL(k_project3d_bwd<true>, dim3(blocks_for(g.num_points, kBlock)), dim3(kBlock), 0, s,
                           cam, g.num_points, g.means, g.scales, g.quats, g.opacities, g.features_dc,
                           g.features_rest, radii, g16, nullptr, nullptr, nullptr, nullptr, nullptr, nullptr,
                           grad_norm, vis, max2d, inv_max_dim, ad, r4);
    } else {
        hipLaunchKernelGGL(k_project3d_bwd<false>, dim3(blocks_for(g.num_points, kBlock)), dim3(kBlock), 0, s,
                           cam, g.num_points, g.means, g.scales, g.quats, g.opacities, g.features_dc,
                           g.features_rest, radii, g16, dmeans, dscales, dquats, dmean2d, dfdc, dfrest,
                           grad_norm, vis, max2d, inv_max_dim, ad, r4);
    }
}

void launch_finish3d_grads(hipStream_t s, int n, const float *rec, float *g16) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_finish3d_grads, dim3(blocks_for(n, 256)), dim3(256), 0, s, n,
                       reinterpret_cast<const float4 *>(rec), g16);
}

void launch_finish_image_grads(hipStream_t s, int n, const float *rec, float *g16) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_finish_image_grads, dim3(blocks_for(n, 256)), dim3(256), 0, s, n,
                       reinterpret_cast<const float4 *>(rec), g16);
}

void launch_gather(hipStream_t s, const float *src, int src_stride, int src_off, int nf, float *dst, int n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_gather, dim3(blocks_for((int64_t)n * nf, 256)), dim3(256), 0, s, src, src_stride,
                       src_off, nf, dst, n);
}

void launch_tiles_hit(hipStream_t s, const uint32_t *rect, const int *radii, int *out, int n) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_tiles_hit, dim3(blocks_for(n, 256)), dim3(256), 0, s,
                       reinterpret_cast<const uint2 *>(rect), radii, out, n);
}

}  // namespace mskern
