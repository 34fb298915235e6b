// k_optim.hip -- Adam, a device-wide int32 inclusive scan, and the
// GPU-resident densification cycle (classify -> scans -> keep flags of the
// old and appended rows -> one gather of every surviving row of the 18
// parameter / optimizer buffers into a workspace -> copy back).
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

// Zeroes n float4s, one 16-byte store per thread in a single pass.  It
// clears the raster backward's per-splat gradient rows before each step:
// 192 MB at 3M splats, which hipMemsetAsync wrote at about 2.3 TB/s.
__global__ __launch_bounds__(256) void k_zero16(float4 *__restrict__ p, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (i < n) p[i] = make_float4(0.f, 0.f, 0.f, 0.f);
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

// The rows after the compaction are a stable selection from the virtual
// list [old rows 0..N) ++ [two children per split splat, in split order]
// ++ [one copy per dup splat, in dup order] (msplat_metal.metal:3271-3412
// append these rows, :3417-3491 cull and compact them).  Nothing is
// appended here: every virtual row is a function of its parent's row, so
// k_densify_keep decides each virtual row's fate from the parent alone,
// and k_densify_gather writes each output row once, in output order.

// The split offset of child k of parent i (the rotated, scaled normal
// sample of :3285-3313), in the reference's operation order.
__device__ __forceinline__ float3 split_offset(const float *__restrict__ quats, const float *__restrict__ scales,
                                               const float *__restrict__ rs, int SD, int i, int ri) {
    float qw = quats[(size_t)i * 4], qx = quats[(size_t)i * 4 + 1], qy = quats[(size_t)i * 4 + 2],
          qz = quats[(size_t)i * 4 + 3];
    const float qlen = __builtin_sqrtf(qw * qw + qx * qx + qy * qy + qz * qz);
    qw /= qlen;
    qx /= qlen;
    qy /= qlen;
    qz /= qlen;
    const size_t si = (size_t)i * SD;
    const float sx = ms_expf(scales[si]), sy = ms_expf(scales[si + 1]);
    const float sz = SD > 2 ? ms_expf(scales[si + 2]) : 0.0f;
    const float r0 = rs[(size_t)ri * 3] * sx, r1 = rs[(size_t)ri * 3 + 1] * sy, r2 = rs[(size_t)ri * 3 + 2] * sz;
    float3 v;
    v.x = (1 - 2 * (qy * qy + qz * qz)) * r0 + 2 * (qx * qy - qw * qz) * r1 + 2 * (qx * qz + qw * qy) * r2;
    v.y = 2 * (qx * qy + qw * qz) * r0 + (1 - 2 * (qx * qx + qz * qz)) * r1 + 2 * (qy * qz - qw * qx) * r2;
    v.z = 2 * (qx * qz - qw * qy) * r0 + 2 * (qy * qz + qw * qx) * r1 + (1 - 2 * (qx * qx + qy * qy)) * r2;
    return v;
}

// The reference's cull test (densify_cull_classify_kernel, :3417-3456) for
// a row with opacity logit `opac` and scales `sc` (already reduced by
// log 1.6 where the row is a child or the copy of a split splat).
__device__ __forceinline__ bool culled(float opac, const float *sc, int SD, float alpha_th, float scale_th,
                                       bool check_huge) {
    const float os = 1.0f / (1.0f + ms_expf(-opac));
    bool cull = os < alpha_th;
    if (check_huge) {
        float ms = ms_expf(sc[0]);
        for (int k = 1; k < SD; ++k) ms = __builtin_fmaxf(ms, ms_expf(sc[k]));
        if (ms > scale_th) cull = true;
    }
    return cull;
}

// One thread per old row i: keep[] of row i and of the rows it appends
// (children at N + 2 ord + k, the copy at N + 2 nS + dup ord), and the
// parent of every appended row.  The appended rows carry the parent's
// opacity; a child's scales are the parent's minus log 1.6, and so are a
// copy's when its parent is also split (the reference appends the copy
// after reducing the split parent's scales in place, :3358-3360).
__global__ __launch_bounds__(256) void k_densify_keep(int N, int nS, int SD, const int *__restrict__ split,
                                                      const int *__restrict__ dup,
                                                      const int *__restrict__ split_pre,
                                                      const int *__restrict__ dup_pre, const float *__restrict__ opac,
                                                      const float *__restrict__ scales,
                                                      const float *__restrict__ max2d, float log_size_fac,
                                                      float alpha_th, float scale_th, float screen_size,
                                                      int check_huge, int check_screen, int *__restrict__ keep,
                                                      int *__restrict__ parent) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N) return;
    const float op = opac[i];
    float sc[3], sc_dec[3];
    for (int k = 0; k < SD; ++k) {
        sc[k] = scales[(size_t)i * SD + k];
        sc_dec[k] = sc[k] - log_size_fac;
    }
    const bool sp = split[i] != 0;
    bool cull = sp || culled(op, sc, SD, alpha_th, scale_th, check_huge);
    if (check_huge && check_screen && max2d[i] > screen_size) cull = true;
    keep[i] = cull ? 0 : 1;
    if (sp) {
        const int a = 2 * (split_pre[i] - 1);
        const int kc = culled(op, sc_dec, SD, alpha_th, scale_th, check_huge) ? 0 : 1;
        keep[N + a] = kc;
        keep[N + a + 1] = kc;
        parent[a] = i;
        parent[a + 1] = i;
    }
    if (dup[i]) {
        const int a = 2 * nS + dup_pre[i] - 1;
        keep[N + a] = culled(op, sp ? sc_dec : sc, SD, alpha_th, scale_th, check_huge) ? 0 : 1;
        parent[a] = i;
    }
}

// src_of[output row] = virtual row, from the inclusive scan of keep[].
__global__ __launch_bounds__(256) void k_densify_src(int n_virt, const int *__restrict__ keep,
                                                     const int *__restrict__ keep_pre, int *__restrict__ src_of) {
    const int v = blockIdx.x * blockDim.x + threadIdx.x;
    if (v < n_virt && keep[v]) src_of[keep_pre[v] - 1] = v;
}

// Output rows are written in blocks of kGatherRows rows of one buffer.
constexpr int kGatherRows = 256, kMaxDensBufs = 18;

struct GatherBuf {
    const float *src;  // the caller's buffer (old rows)
    float *dst;        // the compacted rows (workspace)
    int stride;        // floats per row
    uint32_t magic;    // ceil(2^24 / stride): j / stride = (j * magic) >> 24 for j < 2^15
    int group;         // 0 means, 1 scales, 2.. other parameters
    int moment;        // 1 for an Adam moment buffer (appended rows are zero)
    int block0;        // first block of this buffer
};
struct GatherArgs {
    GatherBuf b[kMaxDensBufs];
    int nbuf, N, nS, SD, n_virt;
    float log_size_fac;
    const int *split, *parent, *src_of, *keep_pre;
    const float *quats, *scales, *rs;  // the parent rows of the children
};

// Every output row of every buffer, once: workgroup = (buffer, block of
// kGatherRows output rows), whose floats are contiguous in the output, so
// each store instruction writes 1 KB of consecutive floats; reads follow
// the kept rows, which are contiguous runs of old rows.  An old row is
// copied, an appended row is derived from its parent (moments zero).
__global__ __launch_bounds__(256) void k_densify_gather(GatherArgs g) {
    __shared__ int s_src[kGatherRows];
    int bi = 0;
    while (bi + 1 < g.nbuf && (int)blockIdx.x >= g.b[bi + 1].block0) ++bi;
    const GatherBuf B = g.b[bi];
    const int new_count = g.keep_pre[g.n_virt - 1];
    const int r0 = ((int)blockIdx.x - B.block0) * kGatherRows;
    const int rows = min(kGatherRows, new_count - r0);
    if (rows <= 0) return;
    if ((int)threadIdx.x < rows) s_src[threadIdx.x] = g.src_of[r0 + threadIdx.x];
    __syncthreads();
    const int S = B.stride, total = rows * S;
    const float *__restrict__ src = B.src;
    float *__restrict__ dst = B.dst + (size_t)r0 * S;
    constexpr int U = 4;
    for (int j0 = threadIdx.x; j0 < total; j0 += 256 * U) {
        float out[U];
        int idx[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            const int j = j0 + u * 256;
            idx[u] = j;
            out[u] = 0.0f;
            if (j >= total) continue;
            const int lr = (int)(((uint64_t)(uint32_t)j * B.magic) >> 24);
            const int c = j - lr * S;
            const int v = s_src[lr];
            if (v < g.N) {
                out[u] = src[(size_t)v * S + c];
            } else if (!B.moment) {
                const int a = v - g.N;
                const int p = g.parent[a];
                const float val = src[(size_t)p * S + c];
                const bool child = a < 2 * g.nS;
                if (B.group == 0 && child) {
                    const float3 o = split_offset(g.quats, g.scales, g.rs, g.SD, p, a);
                    out[u] = val + (c == 0 ? o.x : c == 1 ? o.y : o.z);
                } else if (B.group == 1 && (child || g.split[p])) {
                    out[u] = val - g.log_size_fac;
                } else {
                    out[u] = val;
                }
            }
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (idx[u] < total) dst[idx[u]] = out[u];
    }
}

// The compacted rows back into the caller's buffers: the first
// new_count * stride floats of each, in 4096-float blocks.
constexpr int kCopyFloats = 4096;
struct CopyArgs {
    const float *src[kMaxDensBufs];
    float *dst[kMaxDensBufs];
    int stride[kMaxDensBufs], block0[kMaxDensBufs + 1];
    int nbuf, n_virt;
    const int *keep_pre;
};
__global__ __launch_bounds__(256) void k_densify_copy_back(CopyArgs a) {
    int bi = 0;
    while (bi + 1 < a.nbuf && (int)blockIdx.x >= a.block0[bi + 1]) ++bi;
    const int64_t total = (int64_t)a.keep_pre[a.n_virt - 1] * a.stride[bi];
    const int64_t base = (int64_t)((int)blockIdx.x - a.block0[bi]) * kCopyFloats;
    if (base >= total) return;
    const float *__restrict__ s = a.src[bi] + base;
    float *__restrict__ d = a.dst[bi] + base;
    const int n = (int)min<int64_t>(kCopyFloats, total - base);
    constexpr int U = kCopyFloats / 256;
    float v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int j = threadIdx.x + u * 256;
        v[u] = j < n ? s[j] : 0.0f;
    }
#pragma unroll
    for (int u = 0; u < U; ++u) {
        const int j = threadIdx.x + u * 256;
        if (j < n) d[j] = v[u];
    }
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

void launch_zero16(hipStream_t s, float *p, int64_t n_float4) {
    if (n_float4 <= 0) return;
    const int64_t blocks = (n_float4 + 255) / 256;
    hipLaunchKernelGGL(k_zero16, dim3((unsigned)blocks), dim3(256), 0, s, reinterpret_cast<float4 *>(p), n_float4);
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

int64_t densify_workspace_floats(int n_virt, int scale_dim, int fr_stride) {
    // 18 compacted buffers of n_virt rows, each padded to 64 floats
    const int strides[6] = {3, scale_dim, 4, 3, fr_stride, 1};
    int64_t f = 0;
    for (int gi = 0; gi < 6; ++gi) f += 3 * (((int64_t)n_virt * strides[gi] + 63) / 64 * 64);
    return f;
}

void launch_densify_apply(hipStream_t s, const DensifyArgs &a, int nS, int n_virt) {
    const int N = a.n;
    hipLaunchKernelGGL(k_densify_keep, dim3(nblk(N, 256)), dim3(256), 0, s, N, nS, a.scale_dim, a.split, a.dup,
                       a.split_pre, a.dup_pre, a.params[5], a.params[1], a.max2d, a.log_size_fac, a.cull_alpha,
                       a.cull_scale, a.cull_screen, a.check_huge, a.check_screen, a.keep, a.parent);
    launch_scan_i32(s, a.keep, a.keep_pre, n_virt, a.scan_temp);
    hipLaunchKernelGGL(k_densify_src, dim3(nblk(n_virt, 256)), dim3(256), 0, s, n_virt, a.keep, a.keep_pre,
                       a.src_of);
    const int strides[6] = {3, a.scale_dim, 4, 3, a.fr_stride, 1};
    GatherArgs g{};
    CopyArgs c{};
    g.N = N;
    g.nS = nS;
    g.SD = a.scale_dim;
    g.n_virt = n_virt;
    g.log_size_fac = a.log_size_fac;
    g.split = a.split;
    g.parent = a.parent;
    g.src_of = a.src_of;
    g.keep_pre = a.keep_pre;
    g.quats = a.params[2];
    g.scales = a.params[1];
    g.rs = a.random;
    c.n_virt = n_virt;
    c.keep_pre = a.keep_pre;
    const int row_blocks = (int)nblk(n_virt, kGatherRows);
    float *ws = a.workspace;
    int gb = 0, cb = 0, nb = 0;
    for (int gi = 0; gi < 6; ++gi) {
        if (strides[gi] <= 0) continue;
        for (int r = 0; r < 3; ++r) {
            float *buf = r == 0 ? a.params[gi] : r == 1 ? a.exp_avg[gi] : a.exp_avg_sq[gi];
            GatherBuf &B = g.b[nb];
            B.src = buf;
            B.dst = ws;
            B.stride = strides[gi];
            B.magic = (uint32_t)(((1u << 24) + strides[gi] - 1) / strides[gi]);
            B.group = gi;
            B.moment = r != 0;
            B.block0 = gb;
            gb += row_blocks;
            c.src[nb] = ws;
            c.dst[nb] = buf;
            c.stride[nb] = strides[gi];
            c.block0[nb] = cb;
            cb += (int)nblk((int64_t)n_virt * strides[gi], kCopyFloats);
            ws += ((int64_t)n_virt * strides[gi] + 63) / 64 * 64;
            ++nb;
        }
    }
    g.nbuf = c.nbuf = nb;
    c.block0[nb] = cb;
    hipLaunchKernelGGL(k_densify_gather, dim3(gb), dim3(256), 0, s, g);
    hipLaunchKernelGGL(k_densify_copy_back, dim3(cb), dim3(256), 0, s, c);
}

}  // namespace mskern
