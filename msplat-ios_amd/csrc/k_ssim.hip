// k_ssim.hip -- SSIM (11-tap Gaussian, sigma 1.5, zero padding) + L1 loss,
// forward and backward, in two LDS-tiled passes.
//
// The reference runs 19 separate dispatches per step over 19 full-image
// scratch buffers (ssim_prep_products, 5+3 separable blur pairs,
// ssim_compute, loss_l1_distortion, ssim_backward_compute/accumulate;
// msplat_metal.metal:2704-3085, msplat_metal.mm:1077-1212).  Because
// dL/dssim_map is a known constant (-lambda / 3HW), the per-pixel SSIM
// partials can be produced in the same pass as the forward statistics:
//   pass 1 (k_ssim_fwd): img, gt (+halo, all three channels in one
//          coalesced sweep of the interleaved rows) -> per channel: 5
//          separable blurs in LDS -> SSIM map, loss partials and the three
//          per-pixel gradient maps (d/dmu1 folded, d/dsigma1^2, d/dsigma12),
//          stored channel-planar so every later access is a contiguous row;
//   pass 2 (k_ssim_bwd): per channel the three planar maps (+halo) ->
//          adjoint blur in LDS; the three channels of a pixel stay in the
//          same thread, so dL/dimg = L1 gradient + blurred SSIM gradient is
//          written once, interleaved.
// HBM traffic per pixel: 24 B in + 36 B out (pass 1), 36 + 24 B in + 12 B
// out (pass 2), plus the halo re-reads of neighbouring tiles.
#include "kernels.h"
#include "ms_device.h"

namespace {

constexpr int TW = 64, TH = 16, RAD = 5;
constexpr int RW = TW + 2 * RAD, RH = TH + 2 * RAD;
constexpr int kThreads = 256;
constexpr int kPix = TH * TW / kThreads;  // output pixels per thread

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

// Loads the (RH x RW) region around the tile of an interleaved [H,W,3]
// image into three planar LDS planes, zero outside the image.
__device__ __forceinline__ void load_region3(const float *__restrict__ src, int W, int H, int x0, int y0,
                                             float (*dst)[RH][RW]) {
    for (int k = threadIdx.x; k < RH * RW * 3; k += kThreads) {
        const int ry = k / (RW * 3), rem = k - ry * (RW * 3);
        const int rx = rem / 3, c = rem - rx * 3;
        const int gy = y0 - RAD + ry, gx = x0 - RAD + rx;
        const bool inb = gx >= 0 && gx < W && gy >= 0 && gy < H;
        dst[c][ry][rx] = inb ? src[((size_t)gy * W + gx) * 3 + c] : 0.f;
    }
}

__global__ __launch_bounds__(kThreads) void k_ssim_fwd(int W, int H, const float *__restrict__ img,
                                                       const float *__restrict__ gt, const float *__restrict__ dist,
                                                       float lambda_l1, float lambda_dist, float inv_np, float g,
                                                       Window win, float *__restrict__ gm1,
                                                       float *__restrict__ gs1, float *__restrict__ gs12,
                                                       double *__restrict__ partials) {
    __shared__ float s_a[3][RH][RW];
    __shared__ float s_b[3][RH][RW];
    __shared__ float s_h[5][RH][TW];
    __shared__ double s_red[kThreads / 64];
    const int x0 = blockIdx.x * TW, y0 = blockIdx.y * TH;
    const size_t plane = (size_t)W * H;
    const float C1 = 0.0001f, C2 = 0.0009f;
    double ssim_acc = 0.0, l1_acc = 0.0;
    load_region3(img, W, H, x0, y0, s_a);
    load_region3(gt, W, H, x0, y0, s_b);
    __syncthreads();
    for (int c = 0; c < 3; ++c) {
        // horizontal pass of ssim_blur_horiz_kernel (msplat_metal.metal:2847-2873)
        for (int k = threadIdx.x; k < RH * TW; k += kThreads) {
            const int ry = k / TW, x = k - ry * TW;
            float m1 = 0.f, m2 = 0.f, e11 = 0.f, e22 = 0.f, e12 = 0.f;
#pragma unroll
            for (int j = 0; j < 11; ++j) {
                const float a = s_a[c][ry][x + j], b = s_b[c][ry][x + j], w = win.w[j];
                m1 = __builtin_fmaf(w, a, m1);
                m2 = __builtin_fmaf(w, b, m2);
                e11 = __builtin_fmaf(w, a * a, e11);
                e22 = __builtin_fmaf(w, b * b, e22);
                e12 = __builtin_fmaf(w, a * b, e12);
            }
            s_h[0][ry][x] = m1;
            s_h[1][ry][x] = m2;
            s_h[2][ry][x] = e11;
            s_h[3][ry][x] = e22;
            s_h[4][ry][x] = e12;
        }
        __syncthreads();
        // vertical pass + ssim_compute_kernel (:2910-2952) +
        // ssim_backward_compute_kernel (:2965-3047)
#pragma unroll
        for (int i = 0; i < kPix; ++i) {
            const int k = threadIdx.x + i * kThreads;
            const int y = k / TW, x = k - y * TW;
            const int gy = y0 + y, gx = x0 + x;
            if (gx >= W || gy >= H) continue;
            float mu1 = 0.f, mu2 = 0.f, b11 = 0.f, b22 = 0.f, b12 = 0.f;
#pragma unroll
            for (int j = 0; j < 11; ++j) {
                const float w = win.w[j];
                mu1 = __builtin_fmaf(w, s_h[0][y + j][x], mu1);
                mu2 = __builtin_fmaf(w, s_h[1][y + j][x], mu2);
                b11 = __builtin_fmaf(w, s_h[2][y + j][x], b11);
                b22 = __builtin_fmaf(w, s_h[3][y + j][x], b22);
                b12 = __builtin_fmaf(w, s_h[4][y + j][x], b12);
            }
            const float m1 = mu1, m2 = mu2;
            const float m1_sq = m1 * m1, m2_sq = m2 * m2, m1m2 = m1 * m2;
            const float s1_sq = b11 - m1_sq, s2_sq = b22 - m2_sq, s12 = b12 - m1m2;
            const float A = 2.0f * m1m2 + C1, B = 2.0f * s12 + C2;
            const float Cd = m1_sq + m2_sq + C1, Dd = s1_sq + s2_sq + C2;
            const float val = (A * B) / (Cd * Dd);
            ssim_acc += (double)val;
            const float CD = Cd * Dd, AB = A * B;
            const float inv_CD = 1.0f / CD, inv_Cd = 1.0f / Cd, inv_Dd = 1.0f / Dd;
            const float dmu1 = 2.0f * inv_CD * (m2 * B - m1 * AB * inv_Cd);
            const float ds12 = 2.0f * A * inv_CD;
            const float ds1 = -AB * inv_CD * inv_Dd;
            float gm = g * dmu1;
            const float g12 = g * ds12, g1 = g * ds1;
            gm += g1 * (-2.0f * m1);
            gm += g12 * (-m2);
            const size_t o = c * plane + (size_t)gy * W + gx;
            gm1[o] = gm;
            gs1[o] = g1;
            gs12[o] = g12;
        }
        __syncthreads();
    }
    // per-pixel L1 + distortion loss of loss_l1_distortion_2dgs_kernel (:2704-2762)
    const float inv_HW = inv_np * 3.0f;
#pragma unroll
    for (int i = 0; i < kPix; ++i) {
        const int k = threadIdx.x + i * kThreads;
        const int y = k / TW, x = k - y * TW;
        const int gy = y0 + y, gx = x0 + x;
        if (gx >= W || gy >= H) continue;
        float local = 0.0f;
        for (int c = 0; c < 3; ++c) {
            const float diff = s_a[c][y + RAD][x + RAD] - s_b[c][y + RAD][x + RAD];
            local += lambda_l1 * __builtin_fabsf(diff) * inv_np;
        }
        const float dd = dist ? dist[(size_t)gy * W + gx] : 0.0f;
        local += lambda_dist * dd * inv_HW;
        l1_acc += (double)local;
    }
    const double ts = block_sum_d(ssim_acc, s_red);
    const double tl = block_sum_d(l1_acc, s_red);
    if (threadIdx.x == 0) {
        const int b = blockIdx.y * gridDim.x + blockIdx.x;
        partials[2 * b] = ts;
        partials[2 * b + 1] = tl;
    }
}

// Adjoint blur of the three gradient maps + ssim_backward_accumulate_kernel
// (msplat_metal.metal:3059-3085) + the L1 gradient.
__global__ __launch_bounds__(kThreads) void k_ssim_bwd(int W, int H, const float *__restrict__ img,
                                                       const float *__restrict__ gt, const float *__restrict__ gm1,
                                                       const float *__restrict__ gs1,
                                                       const float *__restrict__ gs12, float lambda_l1, float inv_np,
                                                       Window win, float *__restrict__ dL_dimg) {
    __shared__ float s_g[3][RH][RW];
    __shared__ float s_h[3][RH][TW];
    const int x0 = blockIdx.x * TW, y0 = blockIdx.y * TH;
    const size_t plane = (size_t)W * H;
    float blur[kPix][3][3];  // [pixel][channel][gm, g1, g12]
    for (int c = 0; c < 3; ++c) {
        const float *m0 = gm1 + c * plane, *m1 = gs1 + c * plane, *m2 = gs12 + c * plane;
        for (int k = threadIdx.x; k < RH * RW; k += kThreads) {
            const int ry = k / RW, rx = k - ry * RW;
            const int gy = y0 - RAD + ry, gx = x0 - RAD + rx;
            const bool inb = gx >= 0 && gx < W && gy >= 0 && gy < H;
            const size_t o = (size_t)gy * W + gx;
            s_g[0][ry][rx] = inb ? m0[o] : 0.f;
            s_g[1][ry][rx] = inb ? m1[o] : 0.f;
            s_g[2][ry][rx] = inb ? m2[o] : 0.f;
        }
        __syncthreads();
        for (int k = threadIdx.x; k < RH * TW; k += kThreads) {
            const int ry = k / TW, x = k - ry * TW;
            float h0 = 0.f, h1 = 0.f, h2 = 0.f;
#pragma unroll
            for (int j = 0; j < 11; ++j) {
                const float w = win.w[j];
                h0 = __builtin_fmaf(w, s_g[0][ry][x + j], h0);
                h1 = __builtin_fmaf(w, s_g[1][ry][x + j], h1);
                h2 = __builtin_fmaf(w, s_g[2][ry][x + j], h2);
            }
            s_h[0][ry][x] = h0;
            s_h[1][ry][x] = h1;
            s_h[2][ry][x] = h2;
        }
        __syncthreads();
#pragma unroll
        for (int i = 0; i < kPix; ++i) {
            const int k = threadIdx.x + i * kThreads;
            const int y = k / TW, x = k - y * TW;
            float bgm = 0.f, bg1 = 0.f, bg12 = 0.f;
#pragma unroll
            for (int j = 0; j < 11; ++j) {
                const float w = win.w[j];
                bgm = __builtin_fmaf(w, s_h[0][y + j][x], bgm);
                bg1 = __builtin_fmaf(w, s_h[1][y + j][x], bg1);
                bg12 = __builtin_fmaf(w, s_h[2][y + j][x], bg12);
            }
            blur[i][c][0] = bgm;
            blur[i][c][1] = bg1;
            blur[i][c][2] = bg12;
        }
        __syncthreads();
    }
#pragma unroll
    for (int i = 0; i < kPix; ++i) {
        const int k = threadIdx.x + i * kThreads;
        const int y = k / TW, x = k - y * TW;
        const int gy = y0 + y, gx = x0 + x;
        if (gx >= W || gy >= H) continue;
        const size_t o = ((size_t)gy * W + gx) * 3;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float a = img[o + c], b = gt[o + c];
            const float diff = a - b;
            const float sgn = (diff > 0.0f) ? 1.0f : ((diff < 0.0f) ? -1.0f : 0.0f);
            const float l1 = lambda_l1 * sgn * inv_np;
            const float contrib = blur[i][c][0] + 2.0f * a * blur[i][c][1] + b * blur[i][c][2];
            dL_dimg[o + c] = l1 + contrib;
        }
    }
}

// Fixed-order fp64 reduction of the per-workgroup partials.
__global__ __launch_bounds__(256) void k_loss_final(int nblocks, const double *__restrict__ partials,
                                                    float lambda_dssim, float inv_np, double *__restrict__ out) {
    __shared__ double s_s[256], s_l[256];
    double s = 0.0, l = 0.0;
    for (int b = threadIdx.x; b < nblocks; b += 256) {
        s += partials[2 * b];
        l += partials[2 * b + 1];
    }
    s_s[threadIdx.x] = s;
    s_l[threadIdx.x] = l;
    __syncthreads();
    for (int d = 128; d > 0; d >>= 1) {
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

int ssim_num_blocks(int W, int H) { return ((W + TW - 1) / TW) * ((H + TH - 1) / TH); }

void launch_loss_fwd_bwd(hipStream_t s, int W, int H, const float *img, const float *gt, const float *dist,
                         float lambda_l1, float lambda_dist, float lambda_dssim, const float window[11],
                         float *gm1, float *gs1, float *gs12, double *partials, double *loss_out,
                         float *dL_dimg) {
    const float inv_np = 1.0f / (float)((unsigned)H * (unsigned)W * 3u);
    const float g = -lambda_dssim * inv_np;
    Window win;
    for (int j = 0; j < 11; ++j) win.w[j] = window[j];
    const dim3 grid((W + TW - 1) / TW, (H + TH - 1) / TH);
    hipLaunchKernelGGL(k_ssim_fwd, grid, dim3(kThreads), 0, s, W, H, img, gt, dist, lambda_l1, lambda_dist, inv_np,
                       g, win, gm1, gs1, gs12, partials);
    hipLaunchKernelGGL(k_ssim_bwd, grid, dim3(kThreads), 0, s, W, H, img, gt, gm1, gs1, gs12, lambda_l1, inv_np,
                       win, dL_dimg);
    hipLaunchKernelGGL(k_loss_final, dim3(1), dim3(256), 0, s, (int)(grid.x * grid.y), partials, lambda_dssim,
                       inv_np, loss_out);
}

}  // namespace mskern
