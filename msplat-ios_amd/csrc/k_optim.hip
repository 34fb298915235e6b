// k_optim.hip -- Adam, a device-wide int32 inclusive scan, and the
// GPU-resident densification cycle (classify -> scan -> append split/dup ->
// cull -> stable compaction of the 18 parameter / optimizer buffers).
#include "kernels.h"
#include "ms_device.h"

using namespace msd;

namespace {

// fused_adam_kernel (msplat_metal.metal:1383-1406).
__global__ __launch_bounds__(256) void k_adam(float *__restrict__ p, const float *__restrict__ g,
                                              float *__restrict__ m_, float *__restrict__ v_, int64_t n,
                                              float step, float b1, float b2, float bc2_sqrt, float eps) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float gi = g[i];
        const float m = __builtin_fmaf(b1, m_[i], (1.0f - b1) * gi);
        const float v = __builtin_fmaf(b2, v_[i], (1.0f - b2) * gi * gi);
        p[i] -= step * m / (__builtin_sqrtf(v) / bc2_sqrt + eps);
        m_[i] = m;
        v_[i] = v;
    }
}

// p[i] = min(p[i], value): the opacity reset of Model::afterTrain
// (model.cpp:290-296), which the reference runs as a host loop on unified
// memory.
__global__ void k_clamp_max(float *__restrict__ p, int64_t n, float value) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256)
        if (p[i] > value) p[i] = value;
}

// RGBA8 of an [n,3] float image: (uint8)(clamp(x, 0, 1) * 255) per channel
// (truncation, the host loop of renderFromPoseToBuffer, msplat_api.mm:207-236)
// and alpha 255, one 4-byte store per pixel.
__global__ void k_rgba8(const float *__restrict__ img, int64_t n, uint32_t *__restrict__ out) {
    for (int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x; i < n; i += (int64_t)gridDim.x * 256) {
        const float *p = img + 3 * i;
        uint32_t v = 0xff000000u;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const float x = __builtin_fminf(__builtin_fmaxf(p[c], 0.0f), 1.0f) * 255.0f;
            v |= (uint32_t)x << (8 * c);
        }
        out[i] = v;
    }
}

// ---- device-wide inclusive scan of int32 (reduce-then-scan) --------------
constexpr int kScanBlock = 256, kScanItems = 4, kScanTile = kScanBlock * kScanItems;

__device__ __forceinline__ int block_incl_scan(int v, int *s_w) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(v, d, 64);
        if (lane >= d) v += o;
    }
    if (lane == 63) s_w[wave] = v;
    __syncthreads();
    int off = 0;
    for (int w = 0; w < wave; ++w) off += s_w[w];
    __syncthreads();
    return v + off;
}

__global__ __launch_bounds__(kScanBlock) void k_scan_local(const int *__restrict__ in, int *__restrict__ out,
                                                           int n, int *__restrict__ totals) {
    __shared__ int s_w[kScanBlock / 64];
    const int base = blockIdx.x * kScanTile + threadIdx.x * kScanItems;
    int v[kScanItems];
    int sum = 0;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        v[k] = (base + k < n) ? in[base + k] : 0;
        sum += v[k];
    }
    const int incl = block_incl_scan(sum, s_w);
    int run = incl - sum;
#pragma unroll
    for (int k = 0; k < kScanItems; ++k) {
        run += v[k];
        if (base + k < n) out[base + k] = run;
    }
    if (threadIdx.x == kScanBlock - 1) totals[blockIdx.x] = incl;
}

__global__ __launch_bounds__(1024) void k_scan_totals(int *__restrict__ totals, int nb) {
    __shared__ int s_w[16];
    const int chunk = (nb + 1023) / 1024;
    const int b = min(nb, (int)threadIdx.x * chunk), e = min(nb, b + chunk);
    int sum = 0;
    for (int i = b; i < e; ++i) sum += totals[i];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) s_w[wave] = incl;
    __syncthreads();
    int off = 0;
    for (int w = 0; w < wave; ++w) off += s_w[w];
    int run = off + incl - sum;  // exclusive offset of this thread's chunk
    for (int i = b; i < e; ++i) {
        const int t = totals[i];
        totals[i] = run;  // becomes the exclusive block offset
        run += t;
    }
}

__global__ __launch_bounds__(kScanBlock) void k_scan_add(int *__restrict__ out, int n, const int *__restrict__ offs) {
    const int base = blockIdx.x * kScanTile + threadIdx.x * kScanItems;
    const int o = offs[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanItems; ++k)
        if (base + k < n) out[base + k] += o;
}

// ---- densification (msplat_metal.metal:3231-3491) ------------------------

// The largest of a splat's SD scales (kScaleDim, :3253-3255).
__device__ __forceinline__ float max_scale(const float *__restrict__ scales, size_t i, int SD) {
    float ms = ms_expf(scales[(size_t)SD * i]);
    for (int k = 1; k < SD; ++k) ms = __builtin_fmaxf(ms, ms_expf(scales[(size_t)SD * i + k]));
    return ms;
}

// densify_classify_kernel (:3231-3266); SD floats of scale per splat.
__global__ void k_classify(int N, int SD, const float *__restrict__ gnorm, const float *__restrict__ vis,
                           const float *__restrict__ scales, const float *__restrict__ max2d, float half_max_dim,
                           float grad_th, float size_th, float screen_th, int check_screen, int *__restrict__ split,
                           int *__restrict__ dup) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const float vc = vis[i];
    if (vc <= 0.0f) {
        split[i] = 0;
        dup[i] = 0;
        return;
    }
    const float avg = (gnorm[i] / vc) * half_max_dim;
    const bool high = avg > grad_th;
    const bool large = max_scale(scales, i, SD) > size_th;
    bool sp = large;
    if (check_screen && max2d[i] > screen_th) sp = true;
    sp = sp && high;
    split[i] = sp ? 1 : 0;
    dup[i] = (!large && high) ? 1 : 0;
}

struct Bufs18 {
    float *b[18];
    int stride[18];
};

__device__ __forceinline__ void zero_adam(const Bufs18 &B, size_t dst) {
    for (int gi = 0; gi < 6; ++gi) {
        const int s = B.stride[gi];
        for (int j = 0; j < s; ++j) {
            B.b[6 + gi][dst * s + j] = 0.f;
            B.b[12 + gi][dst * s + j] = 0.f;
        }
    }
}

// densify_append_split_kernel (:3271-3361): children sampled along the SD
// scale axes (the third is 0 for a surfel, :3315-3317).
__global__ void k_append_split(int N, int SD, const int *__restrict__ split, const int *__restrict__ split_pre,
                               const float *__restrict__ rs, float log_size_fac, Bufs18 B) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N || split[i] == 0) return;
    float *means = B.b[0], *scales = B.b[1], *quats = B.b[2];
    const int ord = split_pre[i] - 1;
    const int c0 = N + 2 * ord;
    float qw = quats[i * 4], qx = quats[i * 4 + 1], qy = quats[i * 4 + 2], qz = quats[i * 4 + 3];
    const float qlen = __builtin_sqrtf(qw * qw + qx * qx + qy * qy + qz * qz);
    qw /= qlen;
    qx /= qlen;
    qy /= qlen;
    qz /= qlen;
    const size_t si = (size_t)i * SD;
    const float sx = ms_expf(scales[si]), sy = ms_expf(scales[si + 1]);
    const float sz = SD > 2 ? ms_expf(scales[si + 2]) : 0.0f;
    for (int k = 0; k < 2; ++k) {
        const size_t child = (size_t)c0 + k;
        const int ri = ord * 2 + k;
        const float r0 = rs[ri * 3] * sx, r1 = rs[ri * 3 + 1] * sy, r2 = rs[ri * 3 + 2] * sz;
        const float v0 = (1 - 2 * (qy * qy + qz * qz)) * r0 + 2 * (qx * qy - qw * qz) * r1 + 2 * (qx * qz + qw * qy) * r2;
        const float v1 = 2 * (qx * qy + qw * qz) * r0 + (1 - 2 * (qx * qx + qz * qz)) * r1 + 2 * (qy * qz - qw * qx) * r2;
        const float v2 = 2 * (qx * qz - qw * qy) * r0 + 2 * (qy * qz + qw * qx) * r1 + (1 - 2 * (qx * qx + qy * qy)) * r2;
        means[child * 3] = means[i * 3] + v0;
        means[child * 3 + 1] = means[i * 3 + 1] + v1;
        means[child * 3 + 2] = means[i * 3 + 2] + v2;
        for (int j = 0; j < SD; ++j) scales[child * SD + j] = scales[si + j] - log_size_fac;
        for (int gi = 2; gi < 6; ++gi) {
            const int s = B.stride[gi];
            for (int j = 0; j < s; ++j) B.b[gi][child * s + j] = B.b[gi][(size_t)i * s + j];
        }
        zero_adam(B, child);
    }
    for (int j = 0; j < SD; ++j) scales[si + j] -= log_size_fac;
}

// densify_append_dup_kernel (:3365-3412)
__global__ void k_append_dup(int N, const int *__restrict__ dup, const int *__restrict__ dup_pre,
                             const int *__restrict__ split_pre, Bufs18 B) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N || dup[i] == 0) return;
    const int nS = N > 0 ? split_pre[N - 1] : 0;
    const size_t dst = (size_t)N + 2 * nS + dup_pre[i] - 1;
    for (int gi = 0; gi < 6; ++gi) {
        const int s = B.stride[gi];
        for (int j = 0; j < s; ++j) B.b[gi][dst * s + j] = B.b[gi][(size_t)i * s + j];
    }
    zero_adam(B, dst);
}

// densify_cull_classify_kernel (:3417-3456)
__global__ void k_cull(int N_old, int worst, int SD, const int *__restrict__ split_pre, const int *__restrict__ dup_pre,
                       const int *__restrict__ split, const float *__restrict__ opac,
                       const float *__restrict__ scales, const float *__restrict__ max2d, float alpha_th,
                       float scale_th, float screen_size, int check_huge, int check_screen,
                       int *__restrict__ keep) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= worst) return;
    const int nS = N_old > 0 ? split_pre[N_old - 1] : 0;
    const int nD = N_old > 0 ? dup_pre[N_old - 1] : 0;
    const int N_new = N_old + 2 * nS + nD;
    if (i >= N_new) {
        keep[i] = 0;
        return;
    }
    const float os = 1.0f / (1.0f + ms_expf(-opac[i]));
    bool cull = os < alpha_th;
    if (i < N_old && split[i] != 0) cull = true;
    if (check_huge) {
        if (max_scale(scales, i, SD) > scale_th) cull = true;
        if (check_screen && i < N_old && max2d[i] > screen_size) cull = true;
    }
    keep[i] = cull ? 0 : 1;
}

// compact_scatter_kernel (:3460-3474) for all 18 buffers in one launch:
// grid.y selects the buffer, grid.x runs over (element, component).
__global__ void k_compact(int worst, const int *__restrict__ keep, const int *__restrict__ keep_pre, Bufs18 src,
                          Bufs18 dst) {
    const int b = blockIdx.y;
    const int s = src.stride[b];
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)worst * s) return;
    const int64_t e = t / s, sub = t - e * s;
    if (keep[e] == 0) return;
    dst.b[b][(int64_t)(keep_pre[e] - 1) * s + sub] = src.b[b][t];
}

// compact_copy_back_kernel (:3478-3491)
__global__ void k_copy_back(int worst, const int *__restrict__ keep_pre, Bufs18 src, Bufs18 dst) {
    const int b = blockIdx.y;
    const int s = src.stride[b];
    const int new_count = keep_pre[worst - 1];
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= (int64_t)new_count * s) return;
    dst.b[b][t] = src.b[b][t];
}

inline unsigned nblk(int64_t n, int b) { return (unsigned)((n + b - 1) / b); }

}  // namespace

namespace mskern {

void launch_adam(hipStream_t s, float *p, const float *g, float *m, float *v, int64_t n, float step, float b1,
                 float b2, float bc2_sqrt, float eps) {
    if (n <= 0) return;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(k_adam, dim3((unsigned)blocks), dim3(256), 0, s, p, g, m, v, n, step, b1, b2, bc2_sqrt, eps);
}

void launch_clamp_max(hipStream_t s, float *p, int64_t n, float value) {
    if (n <= 0) return;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(k_clamp_max, dim3((unsigned)blocks), dim3(256), 0, s, p, n, value);
}

void launch_rgba8(hipStream_t s, const float *img, int64_t n, uint32_t *out) {
    if (n <= 0) return;
    const int64_t blocks = std::min<int64_t>((n + 255) / 256, 65536);
    hipLaunchKernelGGL(k_rgba8, dim3((unsigned)blocks), dim3(256), 0, s, img, n, out);
}

int64_t scan_temp_ints(int64_t n) { return (n + kScanTile - 1) / kScanTile + 1; }

void launch_scan_i32(hipStream_t s, const int *in, int *out, int n, int *temp) {
    if (n <= 0) return;
    const int nb = (n + kScanTile - 1) / kScanTile;
    hipLaunchKernelGGL(k_scan_local, dim3(nb), dim3(kScanBlock), 0, s, in, out, n, temp);
    hipLaunchKernelGGL(k_scan_totals, dim3(1), dim3(1024), 0, s, temp, nb);
    hipLaunchKernelGGL(k_scan_add, dim3(nb), dim3(kScanBlock), 0, s, out, n, temp);
}

void launch_densify_classify(hipStream_t s, const DensifyArgs &a) {
    const int N = a.n;
    hipLaunchKernelGGL(k_classify, dim3(nblk(N, 256)), dim3(256), 0, s, N, a.scale_dim, a.grad_norm, a.vis, a.params[1], a.max2d,
                       a.half_max_dim, a.grad_th, a.size_th, a.screen_th, a.check_screen, a.split, a.dup);
    launch_scan_i32(s, a.split, a.split_pre, N, a.scan_temp);
    launch_scan_i32(s, a.dup, a.dup_pre, N, a.scan_temp);
}

void launch_densify_apply(hipStream_t s, const DensifyArgs &a, int n_new) {
    const int N = a.n, worst = n_new;
    Bufs18 B{}, S{};
    const int strides[6] = {3, a.scale_dim, 4, 3, a.fr_stride, 1};
    for (int gi = 0; gi < 6; ++gi) {
        B.b[gi] = a.params[gi];
        B.b[6 + gi] = a.exp_avg[gi];
        B.b[12 + gi] = a.exp_avg_sq[gi];
        S.b[gi] = a.scratch[gi];
        S.b[6 + gi] = a.scratch[6 + gi];
        S.b[12 + gi] = a.scratch[12 + gi];
        for (int r = 0; r < 3; ++r) {
            B.stride[6 * r + gi] = strides[gi];
            S.stride[6 * r + gi] = strides[gi];
        }
    }
    hipLaunchKernelGGL(k_append_split, dim3(nblk(N, 256)), dim3(256), 0, s, N, a.scale_dim, a.split, a.split_pre, a.random,
                       a.log_size_fac, B);
    hipLaunchKernelGGL(k_append_dup, dim3(nblk(N, 256)), dim3(256), 0, s, N, a.dup, a.dup_pre, a.split_pre, B);
    hipLaunchKernelGGL(k_cull, dim3(nblk(worst, 256)), dim3(256), 0, s, N, worst, a.scale_dim, a.split_pre, a.dup_pre, a.split,
                       a.params[5], a.params[1], a.max2d, a.cull_alpha, a.cull_scale, a.cull_screen, a.check_huge,
                       a.check_screen, a.keep);
    launch_scan_i32(s, a.keep, a.keep_pre, worst, a.scan_temp);
    const int64_t maxs = a.fr_stride > 4 ? a.fr_stride : 4;
    hipLaunchKernelGGL(k_compact, dim3(nblk((int64_t)worst * maxs, 256), 18), dim3(256), 0, s, worst, a.keep,
                       a.keep_pre, B, S);
    hipLaunchKernelGGL(k_copy_back, dim3(nblk((int64_t)worst * maxs, 256), 18), dim3(256), 0, s, worst, a.keep_pre,
                       S, B);
}

}  // namespace mskern
