// k_ssim.hip -- SSIM (11-tap Gaussian, sigma 1.5, zero padding) + L1 loss,
// forward and backward.
//
// The reference runs 19 separate dispatches per step over 19 full-image
// scratch buffers (ssim_prep_products, 5+3 separable blur pairs,
// ssim_compute, loss_l1_distortion, ssim_backward_compute/accumulate;
// msplat_metal.metal:2704-3085, msplat_metal.mm:1077-1212).  Because
// dL/dssim_map is a known constant (-lambda / 3HW), the per-pixel SSIM
// partials can be produced in the same pass as the forward statistics, and
// the backward needs nothing else.  Two forms:
//   - k_ssim_stream (images of about 4.7 MP and more, up to the ~89 MP its
//     32-bit offsets allow): one kernel, one wave per (column strip, row
//     segment, channel), carrying each pixel from its inputs to dL/dimg
//     while the wave walks down the strip with the vertical blur windows in
//     registers (see the section below);
//   - the two-pass form for the other images:
//     pass 1 (k_ssim_fwd): per channel, img and gt (+5-pixel halo) -> the 5
//          separable blurs (horizontal, then vertical, as the reference) ->
//          SSIM map, loss partials and the three per-pixel gradient maps
//          (d/dmu1 folded, d/dsigma1^2, d/dsigma12), stored channel-planar;
//     pass 2 (k_ssim_bwd): per channel the three planar maps (+halo) ->
//          adjoint blur (the same symmetric blur) + the L1 gradient; the
//          three channels of a pixel stay in one thread, so dL/dimg is
//          written once, interleaved.
//     Both passes work on 32x32 output tiles one channel at a time (46 / 24
//     KB of LDS) with register blocking: a horizontal work item produces 4
//     adjacent outputs from 14 staged inputs, a vertical one 4 outputs of a
//     column from 14 rows.  Pass 1 loads the three channels of its region at
//     once (each cache line of the interleaved images is fetched once), and
//     both passes walk the tiles in XCD bands (msd::xcd_tile), so a tile's
//     halo is mostly its neighbours' lines, already in the same L2.
// In both forms each output accumulates its taps in ascending order (the
// order of the reference's blur kernels), so they give the same dL/dimg
// bit for bit.
#include "kernels.h"
#include "ms_device.h"

namespace {

constexpr int TS = 32, RAD = 5;   // output tile TS x TS
constexpr int RS = TS + 2 * RAD;  // 42: region rows / columns with halo
constexpr int AST = 48;  // LDS row stride of a staged region
constexpr int BST = 36;  // LDS row stride of horizontal results
constexpr int kThreads = 256;
constexpr int kHItems = RS * (TS / 4);  // 336 horizontal items (row, 4 columns)

// Horizontal work item it -> staged row ry and first column xg.  The two
// 8-lane halves of each 16-lane group take rows r and r + 2, whose starts
// are 2 AST = 96 floats apart (32 banks mod 64), so a group's 16-byte reads
// spread over all banks; rows 40 and 41 pair up in the last group.
// (Measured: LDS bank-conflict cycles 0.22 -> 0.15 of LDS-active in the
// forward, 0.38 -> 0.27 in the backward; kernel times unchanged within 2%.)
__device__ __forceinline__ void h_item(int it, int &ry, int &xg) {
    xg = (it & 7) * 4;
    const int g = it >> 4, h = (it >> 3) & 1, blk = g >> 1, sub = g & 1;
    ry = 4 * blk + 3 < RS ? 4 * blk + sub + 2 * h : 4 * blk + 2 * sub + h;
}

struct Window {
    float w[11];
};

__device__ __forceinline__ double block_sum_d(double v, double *s_red) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    __syncthreads();
    if (lane == 0) s_red[wave] = v;
    __syncthreads();
    double t = 0.0;
    for (int k = 0; k < kThreads / 64; ++k) t += s_red[k];
    return t;
}

constexpr int kStage = (RS * RS + kThreads - 1) / kThreads;  // 7 staged elements per thread

// Loads this thread's kStage elements of the (RS x RS) region around the
// tile of plane `src` (element stride `stride`, offset `off`), zero outside
// the image.  All loads are issued before any is used.
__device__ __forceinline__ void stage_load(const float *__restrict__ src, int W, int H, int x0, int y0, int stride,
                                           int off, float v[kStage]) {
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int k = (int)threadIdx.x + i * kThreads;
        const int ry = k / RS, rx = k - ry * RS;
        const int sy = y0 - RAD + ry, sx = x0 - RAD + rx;
        const bool inb = k < RS * RS && sx >= 0 && sx < W && sy >= 0 && sy < H;
        v[i] = inb ? src[((size_t)sy * W + sx) * stride + off] : 0.f;
    }
}

// All three channels of this thread's kStage pixels of the (RS x RS) region
// of an interleaved RGB image, one 12-byte load per pixel, so that each
// cache line of the region is fetched once for the three channel passes.
__device__ __forceinline__ void stage_load_rgb(const float *__restrict__ src, int W, int H, int x0, int y0,
                                               float v[3][kStage]) {
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int k = (int)threadIdx.x + i * kThreads;
        const int ry = k / RS, rx = k - ry * RS;
        const int sy = y0 - RAD + ry, sx = x0 - RAD + rx;
        const bool inb = k < RS * RS && sx >= 0 && sx < W && sy >= 0 && sy < H;
        const float *p = src + (inb ? ((size_t)sy * W + sx) * 3 : 0);
        v[0][i] = inb ? p[0] : 0.f;
        v[1][i] = inb ? p[1] : 0.f;
        v[2][i] = inb ? p[2] : 0.f;
    }
}

__device__ __forceinline__ void stage_store(float (*dst)[AST], const float v[kStage]) {
#pragma unroll
    for (int i = 0; i < kStage; ++i) {
        const int k = (int)threadIdx.x + i * kThreads;
        if (k < RS * RS) {
            const int ry = k / RS, rx = k - ry * RS;
            dst[ry][rx] = v[i];
        }
    }
}

// 14 consecutive floats of an LDS row starting at a multiple of 4.
__device__ __forceinline__ void lds_row14(const float *p, float v[16]) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const float4 q = reinterpret_cast<const float4 *>(p)[k];
        v[4 * k + 0] = q.x;
        v[4 * k + 1] = q.y;
        v[4 * k + 2] = q.z;
        v[4 * k + 3] = q.w;
    }
}

// At most 168 VGPRs: the LDS allows 3 workgroups per CU, i.e. 3 waves per
// SIMD (the compiler would otherwise use 177 and fit 2).
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(3, 4))) void k_ssim_fwd(int W, int H, const float *__restrict__ img,
                                                       const float *__restrict__ gt, const float *__restrict__ dist,
                                                       float lambda_l1, float lambda_dist, float inv_np, float g,
                                                       Window win, float *__restrict__ gm1,
                                                       float *__restrict__ gs1, float *__restrict__ gs12,
                                                       double *__restrict__ partials) {
    // the window in VGPRs (a VALU instruction that reads an SGPR issues
    // slower; see k_ssim_stream)
    Window wv;
#pragma unroll
    for (int k = 0; k < 11; ++k) asm volatile("v_mov_b32 %0, %1" : "=v"(wv.w[k]) : "s"(win.w[k]));
    __shared__ __align__(16) float s_a[RS][AST];
    __shared__ __align__(16) float s_b[RS][AST];
    __shared__ __align__(16) float s_h[5][RS][BST];
    __shared__ double s_red[kThreads / 64];
    const int tiles_x = (W + TS - 1) / TS, T = tiles_x * ((H + TS - 1) / TS);
    const int tile = msd::xcd_tile(blockIdx.x, T);
    if (tile >= T) return;
    const int x0 = (tile % tiles_x) * TS, y0 = (tile / tiles_x) * TS;
    const size_t plane = (size_t)W * H;
    const float C1 = 0.0001f, C2 = 0.0009f;
    // vertical work item of this thread: column vx, output rows 4 vq .. 4 vq + 3
    const int vx = threadIdx.x & (TS - 1), vq = threadIdx.x >> 5;
    const int gx = x0 + vx;
    double ssim_acc = 0.0;
    float l1[4] = {0.f, 0.f, 0.f, 0.f};
    // the region of both images, all channels, in registers
    float na[3][kStage], nb[3][kStage];
    stage_load_rgb(img, W, H, x0, y0, na);
    stage_load_rgb(gt, W, H, x0, y0, nb);
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        stage_store(s_a, na[c]);
        stage_store(s_b, nb[c]);
        __syncthreads();
        // horizontal pass of ssim_blur_horiz_kernel (msplat_metal.metal:2847-2873)
        for (int it = threadIdx.x; it < kHItems; it += kThreads) {
            int ry, xg;
            h_item(it, ry, xg);
            float a[16], b[16];
            lds_row14(&s_a[ry][xg], a);
            lds_row14(&s_b[ry][xg], b);
            float m1[4] = {0.f, 0.f, 0.f, 0.f}, m2[4] = {0.f, 0.f, 0.f, 0.f}, e11[4] = {0.f, 0.f, 0.f, 0.f},
                  e22[4] = {0.f, 0.f, 0.f, 0.f}, e12[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 11; ++j) {
                const float w = wv.w[j];
#pragma unroll
                for (int o = 0; o < 4; ++o) {
                    const float av = a[o + j], bv = b[o + j];
                    m1[o] = __builtin_fmaf(w, av, m1[o]);
                    m2[o] = __builtin_fmaf(w, bv, m2[o]);
                    e11[o] = __builtin_fmaf(w, av * av, e11[o]);
                    e22[o] = __builtin_fmaf(w, bv * bv, e22[o]);
                    e12[o] = __builtin_fmaf(w, av * bv, e12[o]);
                }
            }
            *reinterpret_cast<float4 *>(&s_h[0][ry][xg]) = make_float4(m1[0], m1[1], m1[2], m1[3]);
            *reinterpret_cast<float4 *>(&s_h[1][ry][xg]) = make_float4(m2[0], m2[1], m2[2], m2[3]);
            *reinterpret_cast<float4 *>(&s_h[2][ry][xg]) = make_float4(e11[0], e11[1], e11[2], e11[3]);
            *reinterpret_cast<float4 *>(&s_h[3][ry][xg]) = make_float4(e22[0], e22[1], e22[2], e22[3]);
            *reinterpret_cast<float4 *>(&s_h[4][ry][xg]) = make_float4(e12[0], e12[1], e12[2], e12[3]);
        }
        __syncthreads();
        // vertical pass + ssim_compute_kernel (:2910-2952) +
        // ssim_backward_compute_kernel (:2965-3047), 4 rows of column vx
        {
            float st[5][4];
#pragma unroll
            for (int s = 0; s < 5; ++s) {
                float col[14];
#pragma unroll
                for (int i = 0; i < 14; ++i) col[i] = s_h[s][4 * vq + i][vx];
#pragma unroll
                for (int o = 0; o < 4; ++o) {
                    float acc = 0.f;
#pragma unroll
                    for (int j = 0; j < 11; ++j) acc = __builtin_fmaf(wv.w[j], col[o + j], acc);
                    st[s][o] = acc;
                }
            }
#pragma unroll
            for (int o = 0; o < 4; ++o) {
                const int gy = y0 + 4 * vq + o;
                const bool live = gx < W && gy < H;
                const float m1 = st[0][o], m2 = st[1][o];
                const float m1_sq = m1 * m1, m2_sq = m2 * m2, m1m2 = m1 * m2;
                const float s1_sq = st[2][o] - m1_sq, s2_sq = st[3][o] - m2_sq, s12 = st[4][o] - m1m2;
                const float A = 2.0f * m1m2 + C1, B = 2.0f * s12 + C2;
                const float Cd = m1_sq + m2_sq + C1, Dd = s1_sq + s2_sq + C2;
                const float CD = Cd * Dd, AB = A * B;
                // the correctly rounded reciprocals (ms_recip, whole-wave);
                // the SSIM value itself is AB * (1 / CD), within an ulp of
                // the quotient (it only enters the loss sum)
                const float inv_CD = msd::ms_recip(CD), inv_Cd = msd::ms_recip(Cd), inv_Dd = msd::ms_recip(Dd);
                if (!live) continue;
                const float val = AB * inv_CD;
                ssim_acc += (double)val;
                const float dmu1 = 2.0f * inv_CD * (m2 * B - m1 * AB * inv_Cd);
                const float ds12 = 2.0f * A * inv_CD;
                const float ds1 = -AB * inv_CD * inv_Dd;
                float gm = g * dmu1;
                const float g12 = g * ds12, g1 = g * ds1;
                gm += g1 * (-2.0f * m1);
                gm += g12 * (-m2);
                const size_t o2 = c * plane + (size_t)gy * W + gx;
                gm1[o2] = gm;
                gs1[o2] = g1;
                gs12[o2] = g12;
                // L1 term of loss_l1_distortion_2dgs_kernel (:2704-2762), channel order
                const float diff = s_a[4 * vq + o + RAD][vx + RAD] - s_b[4 * vq + o + RAD][vx + RAD];
                l1[o] += lambda_l1 * __builtin_fabsf(diff) * inv_np;
            }
        }
        __syncthreads();
    }
    double l1_acc = 0.0;
    const float inv_HW = inv_np * 3.0f;
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        const int gy = y0 + 4 * vq + o;
        if (gx >= W || gy >= H) continue;
        const float dd = dist ? dist[(size_t)gy * W + gx] : 0.0f;
        l1_acc += (double)(l1[o] + lambda_dist * dd * inv_HW);
    }
    const double ts = block_sum_d(ssim_acc, s_red);
    const double tl = block_sum_d(l1_acc, s_red);
    if (threadIdx.x == 0) {
        partials[2 * tile] = ts;
        partials[2 * tile + 1] = tl;
    }
}

// Adjoint blur of the three gradient maps + ssim_backward_accumulate_kernel
// (msplat_metal.metal:3059-3085) + the L1 gradient.  The horizontal results
// are held in registers across a barrier and written over the staged maps,
// so a workgroup needs 24 KB of LDS (six per CU).
constexpr int kHIter = (kHItems + kThreads - 1) / kThreads;  // horizontal items per thread (2)

__global__ __launch_bounds__(kThreads) void k_ssim_bwd(int W, int H, const float *__restrict__ img,
                                                       const float *__restrict__ gt, const float *__restrict__ gm1,
                                                       const float *__restrict__ gs1,
                                                       const float *__restrict__ gs12, float lambda_l1, float inv_np,
                                                       Window win, float *__restrict__ dL_dimg) {
    // staged maps [3][RS][AST]; after the horizontal pass the same memory
    // holds its results [3][RS][BST]
    __shared__ __align__(16) float s_lds[3 * RS * AST];
    float(*s_g)[RS][AST] = reinterpret_cast<float(*)[RS][AST]>(s_lds);
    float(*s_h)[RS][BST] = reinterpret_cast<float(*)[RS][BST]>(s_lds);
    static_assert(BST <= AST, "horizontal results alias the staged maps");
    const int tiles_x = (W + TS - 1) / TS, T = tiles_x * ((H + TS - 1) / TS);
    const int tile = msd::xcd_tile(blockIdx.x, T);
    if (tile >= T) return;
    const int x0 = (tile % tiles_x) * TS, y0 = (tile / tiles_x) * TS;
    const size_t plane = (size_t)W * H;
    const int vx = threadIdx.x & (TS - 1), vq = threadIdx.x >> 5;
    const int gx = x0 + vx;
    float dl[4][3];
    // img / gt of this thread's four pixels, all channels
    float pa[4][3], pb[4][3];
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        const int gy = y0 + 4 * vq + o;
        const bool inb = gx < W && gy < H;
        const size_t p3 = inb ? ((size_t)gy * W + gx) * 3 : 0;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            pa[o][c] = inb ? img[p3 + c] : 0.f;
            pb[o][c] = inb ? gt[p3 + c] : 0.f;
        }
    }
    // the maps of channel c + 1 are loaded into registers while channel c is computed
    float n0[kStage], n1[kStage], n2[kStage];
    stage_load(gm1, W, H, x0, y0, 1, 0, n0);
    stage_load(gs1, W, H, x0, y0, 1, 0, n1);
    stage_load(gs12, W, H, x0, y0, 1, 0, n2);
    for (int c = 0; c < 3; ++c) {
        stage_store(s_g[0], n0);
        stage_store(s_g[1], n1);
        stage_store(s_g[2], n2);
        __syncthreads();
        if (c < 2) {
            const size_t po = (size_t)(c + 1) * plane;
            stage_load(gm1 + po, W, H, x0, y0, 1, 0, n0);
            stage_load(gs1 + po, W, H, x0, y0, 1, 0, n1);
            stage_load(gs12 + po, W, H, x0, y0, 1, 0, n2);
        }
        float hr[kHIter][3][4];
#pragma unroll
        for (int q = 0; q < kHIter; ++q) {
            const int it = (int)threadIdx.x + q * kThreads;
            if (it >= kHItems) continue;
            int ry, xg;
            h_item(it, ry, xg);
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                float v[16];
                lds_row14(&s_g[m][ry][xg], v);
                float h[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 11; ++j)
#pragma unroll
                    for (int o = 0; o < 4; ++o) h[o] = __builtin_fmaf(win.w[j], v[o + j], h[o]);
#pragma unroll
                for (int o = 0; o < 4; ++o) hr[q][m][o] = h[o];
            }
        }
        __syncthreads();
#pragma unroll
        for (int q = 0; q < kHIter; ++q) {
            const int it = (int)threadIdx.x + q * kThreads;
            if (it >= kHItems) continue;
            int ry, xg;
            h_item(it, ry, xg);
#pragma unroll
            for (int m = 0; m < 3; ++m)
                *reinterpret_cast<float4 *>(&s_h[m][ry][xg]) = make_float4(hr[q][m][0], hr[q][m][1], hr[q][m][2],
                                                                           hr[q][m][3]);
        }
        __syncthreads();
        float bl[3][4];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            float col[14];
#pragma unroll
            for (int i = 0; i < 14; ++i) col[i] = s_h[m][4 * vq + i][vx];
#pragma unroll
            for (int o = 0; o < 4; ++o) {
                float acc = 0.f;
#pragma unroll
                for (int j = 0; j < 11; ++j) acc = __builtin_fmaf(win.w[j], col[o + j], acc);
                bl[m][o] = acc;
            }
        }
#pragma unroll
        for (int o = 0; o < 4; ++o) {
            const int gy = y0 + 4 * vq + o;
            dl[o][c] = 0.f;
            if (gx >= W || gy >= H) continue;
            const float a = pa[o][c], b = pb[o][c];
            const float diff = a - b;
            const float sgn = (diff > 0.0f) ? 1.0f : ((diff < 0.0f) ? -1.0f : 0.0f);
            const float contrib = bl[0][o] + 2.0f * a * bl[1][o] + b * bl[2][o];
            dl[o][c] = lambda_l1 * sgn * inv_np + contrib;
        }
        __syncthreads();
    }
#pragma unroll
    for (int o = 0; o < 4; ++o) {
        const int gy = y0 + 4 * vq + o;
        if (gx >= W || gy >= H) continue;
        float *d = dL_dimg + ((size_t)gy * W + gx) * 3;
        d[0] = dl[o][0];
        d[1] = dl[o][1];
        d[2] = dl[o][2];
    }
}

// ---------------------------------------------------------------------------
// One-kernel form (k_ssim_stream): forward statistics, SSIM partials and
// the adjoint blur in one pass.  Because dL/dssim_map is the constant
// -lambda / 3HW, the backward needs nothing but the partial maps, and a
// partial map is needed only 5 pixels around where it is made, so a single
// wave can carry a pixel from its inputs to dL/dimg while it walks down a
// column strip:
//   - one wave per (column strip, row segment, channel); its 64 lanes are
//     the 64 forward columns x0 - 5 .. x0 + 58 of the strip, whose partials
//     the adjoint blur of the 54 output columns x0 .. x0 + 53 needs;
//   - the rows stream through in passes of 4: the horizontal blur of the
//     staged inputs (a lane takes 4 adjacent columns of one row, 14 staged
//     inputs), then per row the vertical blur from a ring of the last 11
//     horizontal results in the lane's registers, the SSIM partials, the
//     horizontal adjoint blur of the partials (staged) and the vertical one
//     from a second register ring; input row i makes the partials of row
//     i - 5 and dL/dimg of row i - 10;
//   - every row's horizontal results are made once (no vertical halo is
//     recomputed except the 20 rows at a segment's start) and the partial
//     maps never leave the CU.
// The ring slot of row i is i mod 11 within an 11-row loop body of passes
// of 4, 4 and 3 rows, so every register index is a compile-time constant.
// Each tap still accumulates in ascending order, as in the two-pass form and
// the reference, so dL/dimg is the same bit for bit.  Inputs are read with
// buffer loads whose out-of-range lanes return 0: rows above or below the
// image and columns outside it (their offsets are pushed past the buffer)
// are the zero padding.
constexpr int kSW = 64;               // forward columns of a strip (= lanes)
constexpr int kSO = kSW - 2 * RAD;    // 54 output columns of a strip
constexpr int kSIn = kSW + 2 * RAD;   // 74 staged input columns
constexpr int kInSt = 80;             // LDS row stride of a staged input row
constexpr int kPtSt = 68;             // LDS row stride of a partials row (reads reach column 65)
constexpr int kRing = 2 * RAD + 1;    // 11 rows of a vertical window = the ring period
constexpr int kPassRows = 4;
constexpr int kLoads = (kPassRows * kSIn + 63) / 64;  // 5 staged inputs per lane per image
constexpr uint32_t kOffPast = 0xC0000000u;  // offset base of a lane whose column is outside the image

struct StreamLds {
    float in[2][kPassRows][kInSt];   // staged img / gt rows of this pass
    float hf[5][kPassRows][kSW];     // horizontal blurs of mu1, mu2, x1^2, x2^2, x1 x2
    float pt[3][kPassRows][kPtSt];   // SSIM partials (d/dmu1 folded, d/dsigma1^2, d/dsigma12)
    float hb[3][kPassRows][kSW];     // horizontal adjoint blurs of the partials
};

struct StreamArgs {
    int W, H, nstrips, seg_rows, units;
    float lambda_l1, lambda_dist, inv_np, inv_HW, g;
};

struct StreamState {
    float hv[5][kRing];             // this lane's column of the last 11 horizontal forward rows
    float gv[3][kRing];             // ... of the last 11 horizontal adjoint rows
    uint32_t ao;                    // byte offset of output column x0 + lane, channel c, at row 0
    float na[kLoads], nb[kLoads];   // the next pass's staged inputs, loaded one pass ahead
    uint32_t lo[kLoads];            // byte offsets of those inputs at input row 0
    int so[kLoads];                 // their LDS slots (row * kInSt + column), -1 if none
    double ssim_acc, l1_acc;
};

__device__ __forceinline__ void stream_load(StreamState &S, __amdgpu_buffer_rsrc_t rimg,
                                            __amdgpu_buffer_rsrc_t rgt, uint32_t row_off) {
#pragma unroll
    for (int m = 0; m < kLoads; ++m) {
        const uint32_t off = S.lo[m] + row_off;
        S.na[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rimg, off, 0, 0));
        S.nb[m] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rgt, off, 0, 0));
    }
}

// One pass of NP input rows starting at input row ib (slots P0 .. P0+NP-1
// of the ring).
template <int P0, int NP>
__device__ __forceinline__ void stream_pass(const StreamArgs &A, const Window &win, StreamLds &L, StreamState &S,
                                            __amdgpu_buffer_rsrc_t rimg, __amdgpu_buffer_rsrc_t rgt, int ib, int x0,
                                            int y0, int y1, int c, const float *__restrict__ dist,
                                            float *__restrict__ dL) {
    const int lane = threadIdx.x;
    const float C1 = 0.0001f, C2 = 0.0009f;
    // img / gt at the output rows of this pass (rows ib - 10 ..): lines this
    // wave read ten rows ago, loaded again (the cache's copy) rather than
    // kept in registers
    float fa[NP], fb[NP];
#pragma unroll
    for (int rr = 0; rr < NP; ++rr) {
        const uint32_t off = S.ao + (uint32_t)(ib + rr - 2 * RAD) * (uint32_t)A.W * 12u;
        fa[rr] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rimg, off, 0, 0));
        fb[rr] = __builtin_bit_cast(float, __builtin_amdgcn_raw_buffer_load_b32(rgt, off, 0, 0));
    }
    // stage this pass's rows, then start loading the next pass's
#pragma unroll
    for (int m = 0; m < kLoads; ++m)
        if (S.so[m] >= 0) {
            (&L.in[0][0][0])[S.so[m]] = S.na[m];
            (&L.in[1][0][0])[S.so[m]] = S.nb[m];
        }
    stream_load(S, rimg, rgt, (uint32_t)(ib + NP) * (uint32_t)A.W * 12u);
    __syncthreads();
    // horizontal pass of ssim_blur_horiz_kernel (msplat_metal.metal:2847-2873):
    // lane (r, q) makes columns 4q .. 4q + 3 of row r
    {
        const int r = lane >> 4, q = lane & 15;
        if (r < NP) {
            float a[16], b[16];
            lds_row14(&L.in[0][r][4 * q], a);
            lds_row14(&L.in[1][r][4 * q], b);
            float m1[4] = {0.f, 0.f, 0.f, 0.f}, m2[4] = {0.f, 0.f, 0.f, 0.f}, e11[4] = {0.f, 0.f, 0.f, 0.f},
                  e22[4] = {0.f, 0.f, 0.f, 0.f}, e12[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int j = 0; j < 11; ++j) {
                const float w = win.w[j];
#pragma unroll
                for (int o = 0; o < 4; ++o) {
                    const float av = a[o + j], bv = b[o + j];
                    m1[o] = __builtin_fmaf(w, av, m1[o]);
                    m2[o] = __builtin_fmaf(w, bv, m2[o]);
                    e11[o] = __builtin_fmaf(w, av * av, e11[o]);
                    e22[o] = __builtin_fmaf(w, bv * bv, e22[o]);
                    e12[o] = __builtin_fmaf(w, av * bv, e12[o]);
                }
            }
            *reinterpret_cast<float4 *>(&L.hf[0][r][4 * q]) = make_float4(m1[0], m1[1], m1[2], m1[3]);
            *reinterpret_cast<float4 *>(&L.hf[1][r][4 * q]) = make_float4(m2[0], m2[1], m2[2], m2[3]);
            *reinterpret_cast<float4 *>(&L.hf[2][r][4 * q]) = make_float4(e11[0], e11[1], e11[2], e11[3]);
            *reinterpret_cast<float4 *>(&L.hf[3][r][4 * q]) = make_float4(e22[0], e22[1], e22[2], e22[3]);
            *reinterpret_cast<float4 *>(&L.hf[4][r][4 * q]) = make_float4(e12[0], e12[1], e12[2], e12[3]);
        }
    }
    __syncthreads();
    // per row: vertical pass + ssim_compute_kernel (:2910-2952) +
    // ssim_backward_compute_kernel (:2965-3047) for row j = i - 5
    const int fx = x0 - RAD + lane;
    const bool fcol = (unsigned)fx < (unsigned)A.W;
    const bool fown = fcol && lane >= RAD && lane < RAD + kSO;
    // the vertical blurs of all NP rows, then their partials side by side
    // (independent chains for the issue to interleave), with one
    // wave-uniform branch for the pass's reciprocals
    float st[NP][5];
#pragma unroll
    for (int rr = 0; rr < NP; ++rr) {
        const int p = P0 + rr;
#pragma unroll
        for (int s = 0; s < 5; ++s) S.hv[s][p] = L.hf[s][rr][lane];
#pragma unroll
        for (int s = 0; s < 5; ++s) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < kRing; ++k) acc = __builtin_fmaf(win.w[k], S.hv[s][(p + 1 + k) % kRing], acc);
            st[rr][s] = acc;
        }
    }
    float A_[NP], B[NP], AB[NP], CD[NP], Cd[NP], Dd[NP], inv_CD[NP], inv_Cd[NP], inv_Dd[NP];
    bool odd = false;
#pragma unroll
    for (int rr = 0; rr < NP; ++rr) {
        const float m1 = st[rr][0], m2 = st[rr][1];
        const float m1_sq = m1 * m1, m2_sq = m2 * m2, m1m2 = m1 * m2;
        const float s1_sq = st[rr][2] - m1_sq, s2_sq = st[rr][3] - m2_sq, s12 = st[rr][4] - m1m2;
        A_[rr] = 2.0f * m1m2 + C1;
        B[rr] = 2.0f * s12 + C2;
        Cd[rr] = m1_sq + m2_sq + C1;
        Dd[rr] = s1_sq + s2_sq + C2;
        CD[rr] = Cd[rr] * Dd[rr];
        AB[rr] = A_[rr] * B[rr];
        // the correctly rounded reciprocals (as msd::ms_recip)
        inv_CD[rr] = msd::ms_rcp_nr(CD[rr]);
        inv_Cd[rr] = msd::ms_rcp_nr(Cd[rr]);
        inv_Dd[rr] = msd::ms_rcp_nr(Dd[rr]);
        odd = odd || !(msd::ms_rcp_nr_exact(CD[rr]) && msd::ms_rcp_nr_exact(Cd[rr]) && msd::ms_rcp_nr_exact(Dd[rr]));
    }
    if (__builtin_amdgcn_ballot_w64(odd)) {
#pragma unroll
        for (int rr = 0; rr < NP; ++rr) {
            float z0 = CD[rr], z1 = Cd[rr], z2 = Dd[rr];
            asm volatile("" : "+v"(z0), "+v"(z1), "+v"(z2));  // keeps the divisions inside the branch
            if (!(msd::ms_rcp_nr_exact(z0) && msd::ms_rcp_nr_exact(z1) && msd::ms_rcp_nr_exact(z2))) {
                inv_CD[rr] = 1.0f / z0;
                inv_Cd[rr] = 1.0f / z1;
                inv_Dd[rr] = 1.0f / z2;
            }
        }
    }
#pragma unroll
    for (int rr = 0; rr < NP; ++rr) {
        const int jrow = ib + rr - RAD;
        const bool live = fcol && (unsigned)jrow < (unsigned)A.H;
        const float m1 = st[rr][0], m2 = st[rr][1];
        const float val = AB[rr] * inv_CD[rr];
        if (fown && jrow >= y0 && jrow < y1) S.ssim_acc += (double)val;
        const float dmu1 = 2.0f * inv_CD[rr] * (m2 * B[rr] - m1 * AB[rr] * inv_Cd[rr]);
        const float ds12 = 2.0f * A_[rr] * inv_CD[rr];
        const float ds1 = -AB[rr] * inv_CD[rr] * inv_Dd[rr];
        float gm = A.g * dmu1;
        const float g12 = A.g * ds12, g1 = A.g * ds1;
        gm += g1 * (-2.0f * m1);
        gm += g12 * (-m2);
        // the partial maps are zero outside the image (the reference's
        // adjoint blur skips those taps)
        L.pt[0][rr][lane] = live ? gm : 0.f;
        L.pt[1][rr][lane] = live ? g1 : 0.f;
        L.pt[2][rr][lane] = live ? g12 : 0.f;
    }
    __syncthreads();
    // horizontal adjoint blur (the same symmetric window): lane (r, q)
    // makes output columns 4q .. 4q + 3 (q < 14) of row r
    {
        const int r = lane >> 4, q = lane & 15;
        if (r < NP && q < (kSO + 3) / 4) {
#pragma unroll
            for (int m = 0; m < 3; ++m) {
                float v[16];
                lds_row14(&L.pt[m][r][4 * q], v);
                float h[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int j = 0; j < 11; ++j)
#pragma unroll
                    for (int o = 0; o < 4; ++o) h[o] = __builtin_fmaf(win.w[j], v[o + j], h[o]);
                *reinterpret_cast<float4 *>(&L.hb[m][r][4 * q]) = make_float4(h[0], h[1], h[2], h[3]);
            }
        }
    }
    __syncthreads();
    // per row: vertical adjoint blur + ssim_backward_accumulate_kernel
    // (:3059-3085) + the L1 gradient and loss of output row o = i - 10
    const int ox = x0 + lane;
    const bool ocol = lane < kSO && ox < A.W;
    float bl[NP][3];
#pragma unroll
    for (int rr = 0; rr < NP; ++rr) {
        const int p = P0 + rr;
#pragma unroll
        for (int m = 0; m < 3; ++m) S.gv[m][p] = L.hb[m][rr][lane];
#pragma unroll
        for (int m = 0; m < 3; ++m) {
            float acc = 0.f;
#pragma unroll
            for (int k = 0; k < kRing; ++k) acc = __builtin_fmaf(win.w[k], S.gv[m][(p + 1 + k) % kRing], acc);
            bl[rr][m] = acc;
        }
    }
#pragma unroll
    for (int rr = 0; rr < NP; ++rr) {
        const int orow = ib + rr - 2 * RAD;
        if (ocol && orow >= y0 && orow < y1) {
            const float a = fa[rr], b = fb[rr];
            const float diff = a - b;
            const float sgn = (diff > 0.0f) ? 1.0f : ((diff < 0.0f) ? -1.0f : 0.0f);
            const float contrib = bl[rr][0] + 2.0f * a * bl[rr][1] + b * bl[rr][2];
            const size_t px = (size_t)orow * A.W + ox;
            dL[px * 3 + c] = A.lambda_l1 * sgn * A.inv_np + contrib;
            // loss_l1_distortion_2dgs_kernel (:2704-2762); the distortion
            // term once per pixel, with channel 0
            double l = (double)(A.lambda_l1 * __builtin_fabsf(diff) * A.inv_np);
            if (dist && c == 0) l += (double)(A.lambda_dist * dist[px] * A.inv_HW);
            S.l1_acc += l;
        }
    }
}

__global__ __launch_bounds__(64) void k_ssim_stream(StreamArgs A, Window win, const float *__restrict__ img,
                                                    const float *__restrict__ gt, const float *__restrict__ dist,
                                                    float *__restrict__ dL, double *__restrict__ partials) {
    __shared__ __align__(16) StreamLds L;
    // units (segment, strip, channel), channel fastest, in 8 XCD bands: the
    // three channel waves of a strip and its neighbouring strips, which
    // read the same input lines, run in one XCD's L2
    const int per = (A.units + 7) >> 3;
    const int u = (int)(blockIdx.x & 7) * per + (int)(blockIdx.x >> 3);
    if (u >= A.units) return;
    const int c = u % 3, ss = u / 3;
    const int strip = ss % A.nstrips, seg = ss / A.nstrips;
    const int x0 = strip * kSO, y0 = seg * A.seg_rows;
    const int y1 = y0 + A.seg_rows < A.H ? y0 + A.seg_rows : A.H;
    const int lane = threadIdx.x;
    // zero the LDS once: the columns past the written ones of the partials
    // and adjoint rows are read (and ignored) by the last lanes
    {
        float *z = &L.in[0][0][0];
        constexpr int n = (int)(sizeof(StreamLds) / sizeof(float));
        for (int k = lane; k < n; k += 64) z[k] = 0.f;
    }
    StreamState S;
#pragma unroll
    for (int k = 0; k < kRing; ++k) {
#pragma unroll
        for (int s = 0; s < 5; ++s) S.hv[s][k] = 0.f;
#pragma unroll
        for (int m = 0; m < 3; ++m) S.gv[m][k] = 0.f;
    }
    S.ssim_acc = 0.0;
    S.l1_acc = 0.0;
    S.ao = (uint32_t)((x0 + lane) * 12 + 4 * c);
#pragma unroll
    for (int m = 0; m < kLoads; ++m) {
        const int k = lane + 64 * m;
        const int r = k / kSIn, col = k - r * kSIn;
        const int x = x0 - 2 * RAD + col;
        const bool ok = k < kPassRows * kSIn;
        S.so[m] = ok ? r * kInSt + col : -1;
        S.lo[m] = ok && (unsigned)x < (unsigned)A.W ? (uint32_t)((r * A.W + x) * 12 + 4 * c) : kOffPast;
    }
    const uint32_t nrec = (uint32_t)A.W * (uint32_t)A.H * 12u;
    const __amdgpu_buffer_rsrc_t rimg = __builtin_amdgcn_make_buffer_rsrc((void *)img, (short)0, nrec, 0x00020000);
    const __amdgpu_buffer_rsrc_t rgt = __builtin_amdgcn_make_buffer_rsrc((void *)gt, (short)0, nrec, 0x00020000);
    // the window in VGPRs: a VALU instruction that reads an SGPR issues at
    // about 60% of the rate of one whose operands are all VGPRs (gfx950,
    // measured on independent FMA chains), and almost every instruction
    // here is a tap of the window
    Window wv;
#pragma unroll
    for (int k = 0; k < 11; ++k) asm volatile("v_mov_b32 %0, %1" : "=v"(wv.w[k]) : "s"(win.w[k]));
    const int ib0 = y0 - 2 * RAD;
    stream_load(S, rimg, rgt, (uint32_t)ib0 * (uint32_t)A.W * 12u);
    const int nbody = (y1 - y0 + 4 * RAD + kRing - 1) / kRing;
    for (int bi = 0; bi < nbody; ++bi) {
        const int ib = ib0 + bi * kRing;
        stream_pass<0, 4>(A, wv, L, S, rimg, rgt, ib, x0, y0, y1, c, dist, dL);
        stream_pass<4, 4>(A, wv, L, S, rimg, rgt, ib + 4, x0, y0, y1, c, dist, dL);
        stream_pass<8, 3>(A, wv, L, S, rimg, rgt, ib + 8, x0, y0, y1, c, dist, dL);
    }
    double ts = S.ssim_acc, tl = S.l1_acc;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        ts += __shfl_xor(ts, d, 64);
        tl += __shfl_xor(tl, d, 64);
    }
    if (lane == 0) {
        partials[2 * u] = ts;
        partials[2 * u + 1] = tl;
    }
}

// Fixed-order fp64 reduction of the per-workgroup partials.
__global__ __launch_bounds__(1024) void k_loss_final(int nblocks, const double *__restrict__ partials,
                                                     float lambda_dssim, float inv_np, double *__restrict__ out) {
    __shared__ double s_s[1024], s_l[1024];
    double s = 0.0, l = 0.0;
    // each thread sums a fixed strided subset, four loads in flight
    for (int b0 = threadIdx.x; b0 < nblocks; b0 += 4 * 1024) {
        double2 v[4];
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            const int b = b0 + u * 1024;
            v[u] = b < nblocks ? reinterpret_cast<const double2 *>(partials)[b] : make_double2(0.0, 0.0);
        }
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            s += v[u].x;
            l += v[u].y;
        }
    }
    s_s[threadIdx.x] = s;
    s_l[threadIdx.x] = l;
    __syncthreads();
    for (int d = 512; d > 0; d >>= 1) {
        if ((int)threadIdx.x < d) {
            s_s[threadIdx.x] += s_s[threadIdx.x + d];
            s_l[threadIdx.x] += s_l[threadIdx.x + d];
        }
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const double ssim_sum = s_s[0];
        out[0] = s_l[0] + (double)lambda_dssim * (1.0 - ssim_sum * (double)inv_np);
        out[1] = ssim_sum;
    }
}

}  // namespace

namespace mskern {

int ssim_num_blocks(int W, int H) { return ((W + TS - 1) / TS) * ((H + TS - 1) / TS); }

static int g_form = 0;
void set_loss_form(int form) { g_form = form; }

// Row segments of the one-kernel form.  Each wave re-makes the 20 rows
// above its segment, so segments are long; the kernel holds 2 waves per
// SIMD (its registers), and it is bound by VALU issue, so the segment count
// is the largest whose waves (segments x strips x 3) all run at once on the
// 1024 SIMDs of an MI355X -- a second, partial round of waves would leave
// most SIMDs idle -- and one segment per 64 rows at most.
constexpr int kStreamWaves = 2048;
// Below this many rows per segment the 20 re-made rows cost more than the
// two-pass form's map round trip (measured: 1297x840 and 1920x1080 frames,
// 60- and 64-row segments, ran 35% and 10% slower streaming).
constexpr int kStreamMinRows = 128;
static void stream_plan(int W, int H, StreamArgs &A) {
    A.nstrips = (W + kSO - 1) / kSO;
    const int per_row = 3 * A.nstrips;
    int nseg = kStreamWaves / per_row;
    const int max_seg = (H + 63) / 64;
    nseg = std::max(1, std::min(nseg, max_seg));
    A.seg_rows = (H + nseg - 1) / nseg;
    nseg = (H + A.seg_rows - 1) / A.seg_rows;
    A.units = nseg * per_row;
}

// The streaming form's offsets (rows -10 .. H + 30 of the 12-byte pixels,
// plus the out-of-image base) must fit in 32 bits.
static bool use_stream(int W, int H) {
    if (g_form == 2 || (int64_t)(H + 32) * W * 12 >= (int64_t(1) << 30)) return false;
    if (g_form == 1) return true;
    StreamArgs A;
    stream_plan(W, H, A);
    return A.seg_rows >= kStreamMinRows;
}

int loss_num_partials(int W, int H) {
    if (!use_stream(W, H)) return ssim_num_blocks(W, H);
    StreamArgs A;
    stream_plan(W, H, A);
    return A.units;
}

bool loss_needs_maps(int W, int H) { return !use_stream(W, H); }

void launch_loss_fwd_bwd(hipStream_t s, int W, int H, const float *img, const float *gt, const float *dist,
                         float lambda_l1, float lambda_dist, float lambda_dssim, const float window[11],
                         float *gm1, float *gs1, float *gs12, double *partials, double *loss_out,
                         float *dL_dimg) {
    const float inv_np = 1.0f / (float)((unsigned)H * (unsigned)W * 3u);
    const float g = -lambda_dssim * inv_np;
    Window win;
    for (int j = 0; j < 11; ++j) win.w[j] = window[j];
    int nparts;
    if (use_stream(W, H)) {
        StreamArgs A;
        stream_plan(W, H, A);
        A.W = W;
        A.H = H;
        A.lambda_l1 = lambda_l1;
        A.lambda_dist = lambda_dist;
        A.inv_np = inv_np;
        A.inv_HW = inv_np * 3.0f;
        A.g = g;
        // one wave per unit, the grid padded to a multiple of the 8 XCDs
        const dim3 grid(((A.units + 7) / 8) * 8);
        hipLaunchKernelGGL(k_ssim_stream, grid, dim3(64), 0, s, A, win, img, gt, dist, dL_dimg, partials);
        nparts = A.units;
    } else {
        // one workgroup per 32x32 tile, the grid padded to a multiple of the 8 XCDs
        const int T = ssim_num_blocks(W, H);
        const dim3 grid(((T + 7) / 8) * 8);
        hipLaunchKernelGGL(k_ssim_fwd, grid, dim3(kThreads), 0, s, W, H, img, gt, dist, lambda_l1, lambda_dist,
                           inv_np, g, win, gm1, gs1, gs12, partials);
        hipLaunchKernelGGL(k_ssim_bwd, grid, dim3(kThreads), 0, s, W, H, img, gt, gm1, gs1, gs12, lambda_l1,
                           inv_np, win, dL_dimg);
        nparts = T;
    }
    hipLaunchKernelGGL(k_loss_final, dim3(1), dim3(1024), 0, s, nparts, partials, lambda_dssim, inv_np, loss_out);
}

}  // namespace mskern
