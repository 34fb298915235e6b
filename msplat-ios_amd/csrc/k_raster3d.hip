// k_raster3d.hip -- the 3DGS mode's front-to-back compositing forward and
// its backward, on the same machinery as the 2DGS rasterizers (k_raster.hip):
// one 256-thread workgroup per 16x16 tile, each wave an 8x8 quadrant with
// its own slot list of the staged batch (raster_wave.h), and a per-wave
// blend log the backward replays back to front with prefix checkpoints.
//
// The pair rule is the published 3DGS one in the fork's blending
// conventions: with d = centre - pixel and the conic (a, b, c),
// rho = a dx^2 + c dy^2 + 2 b dx dy (= 2 sigma), skipped when negative;
// alpha = min(0.99, opacity exp(-rho / 2)), skipped below 1/255; the pixel
// stops before its transmittance falls to 1e-4 (msplat_metal.metal:663-721
// for the 2DGS pair).  rho and exp are the golden model's operations
// (fmaf(a dx, dx, fmaf(c dy, dy, 2 b dx dy)) and ms_gauss), so images are
// bit-exact with it.
#include "kernels.h"
#include "ms_device.h"
#include "raster_wave.h"

using namespace msd;
using namespace msr;

namespace {

// 2 sigma of a pixel for the conic (a, b, c) in p0.zw / p1.x, centre p0.xy
__device__ __forceinline__ float conic_rho(const float4 &p0, const float4 &p1, float px, float py, float &dx,
                                           float &dy) {
    dx = p0.x - px;
    dy = p0.y - py;
    return __builtin_fmaf(p0.z * dx, dx, __builtin_fmaf(p1.x * dy, dy, 2.f * p0.w * dx * dy));
}

// Stages splat gid (list position pos) in LDS slot threadIdx.x as planes
// 0 = (x, y, a, b), 1 = (c, opacity, pos, gid), 2 = (r, g, b, 0), and
// returns the quadrant mask of its alpha >= 1/255 box for the tile.
__device__ __forceinline__ int load_batch3(const float4 *__restrict__ rec, const float4 *__restrict__ boxes, int gid,
                                           int pos, float4 *s_rec, float sx0, float sy0) {
    const float4 *r = rec + 3 * (size_t)gid;
    const float4 q0 = r[0], q1 = r[1], q2 = r[2];
    s_rec[threadIdx.x] = q0;
    s_rec[kThreads + threadIdx.x] = make_float4(q1.x, q1.y, __int_as_float(pos), __int_as_float(gid));
    s_rec[2 * kThreads + threadIdx.x] = q2;
    return strip_mask(boxes[gid], sx0, sy0);
}

// With LOG, every wave writes its blend log and prefix checkpoints exactly
// as k_raster_fwd<true, ...> does (entries {ballot lo, ballot hi, list
// position, splat id} in 64-entry pool chunks with their checkpoints,
// BlendLog).
// Outputs: out_img and final_Ts[.][0] (the transmittance).
template <bool LOG>
__global__ __launch_bounds__(kThreads) void k_raster3d_fwd(int W, int H, int tiles_x, int T,
                                                           const int *__restrict__ offsets,
                                                           const int *__restrict__ ids,
                                                           const float4 *__restrict__ rec,
                                                           const float4 *__restrict__ boxes,
                                                           const float *__restrict__ bgp, float *__restrict__ out_img,
                                                           float *__restrict__ final_Ts, BlendLog blog) {
    const int tile = xcd_strip_tile(blockIdx.x, tiles_x, T / tiles_x);
    if (tile < 0) return;
    __shared__ float4 s_rec[3 * kThreads];
    __shared__ unsigned char s_list[4][kThreads];
    __shared__ int4 s_cnt[4];
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pxi = tx * 16 + lane_px(wave, lane);
    const int pyi = ty * 16 + lane_py(wave, lane);
    const bool inside = pxi < W && pyi < H;
    float px = (float)pxi, py = (float)pyi;
    asm volatile("" : "+v"(px), "+v"(py));
    const float sx0 = (float)(tx * 16), sy0 = (float)(ty * 16);
    const int start = offsets[tile], end = offsets[tile + 1];
    LogWriter lw;
    lw.tb = LOG ? log_table_base(start, end - start, tile, wave) : 0;
    lw.sp = LOG ? log_subpool(blog, tile, wave) : 0;
    if (LOG && end > start) lw.start(blog, lane);  // an empty list logs nothing
    int nlog = 0;
    uint4 lg_ent = make_uint4(0u, 0u, 0u, 0u);
    const char *s_bytes = reinterpret_cast<const char *>(s_rec);
    float Tr = 1.f, cr = 0.f, cg = 0.f, cb = 0.f;
    uint64_t done_m = __builtin_amdgcn_ballot_w64(!inside);
    for (int b0 = start; b0 < end; b0 += kThreads) {
        if (__syncthreads_and(done_m == ~0ull)) break;
        const int idx = b0 + (int)threadIdx.x;
        const int gid = idx < end ? ids[idx] : 0;
        const int m = idx < end ? load_batch3(rec, boxes, gid, idx - start, s_rec, sx0, sy0) : 0;
        const int n = build_wave_lists(m, s_list, s_cnt);
        // one visit of slot list entry j (a visit after the wave is done
        // changes nothing); two per iteration, as the 2DGS forward
        const auto visit = [&](int j) {
            const int to = 16 * (int)s_list[wave][j];
            const auto plane = [&](int k) {
                return *reinterpret_cast<const float4 *>(s_bytes + k * (kThreads * 16) + to);
            };
            const float4 p0 = plane(0), p1 = plane(1);
            float dx, dy;
            const float rho = conic_rho(p0, p1, px, py, dx, dy);
            const float alpha = __builtin_fminf(0.99f, p1.y * ms_gauss(rho));
            const uint64_t act = __builtin_amdgcn_ballot_w64(!(rho < 0.0f)) &
                                 __builtin_amdgcn_ballot_w64(!(alpha < 1.0f / 255.0f)) & ~done_m;
            const float next_T = Tr * (1.0f - alpha);
            const uint64_t term = act & __builtin_amdgcn_ballot_w64(next_T <= 1e-4f);
            const uint64_t bal = act & ~term;
            done_m |= term;
            const bool blend = __builtin_amdgcn_inverse_ballot_w64(bal);
            const float w = blend ? alpha * Tr : 0.0f;
            const float4 p2 = plane(2);
            cr = __builtin_fmaf(p2.x, w, cr);
            cg = __builtin_fmaf(p2.y, w, cg);
            cb = __builtin_fmaf(p2.z, w, cb);
            Tr = blend ? next_T : Tr;
            if (LOG && bal) {
                const bool mine = __builtin_amdgcn_inverse_ballot_w64(1ull << (nlog & 63));
                lg_ent.x = mine ? (unsigned)bal : lg_ent.x;
                lg_ent.y = mine ? (unsigned)(bal >> 32) : lg_ent.y;
                lg_ent.z = mine ? __float_as_uint(p1.z) : lg_ent.z;
                lg_ent.w = mine ? __float_as_uint(p1.w) : lg_ent.w;
                if ((++nlog & 63) == 0) lw.full(blog, lane, nlog, lg_ent, Tr);
            }
        };
        int j = 0;
        for (; j + 1 < n && done_m != ~0ull; j += 2) {
            visit(j);
            visit(j + 1);
        }
        if (j < n && done_m != ~0ull) visit(j);
    }
    if (LOG) lw.finish(blog, lane, nlog, lg_ent, tile, wave);
    if (!inside) return;
    const size_t pix = (size_t)pyi * W + pxi;
    final_Ts[3 * pix + 0] = Tr;
    out_img[3 * pix + 0] = __builtin_fmaf(bgp[0], Tr, cr);
    out_img[3 * pix + 1] = __builtin_fmaf(bgp[1], Tr, cg);
    out_img[3 * pix + 2] = __builtin_fmaf(bgp[2], Tr, cb);
}

// The 3DGS backward over the forward's blend log (the image-only case: the
// only upstream gradient is dL/dimage).  Each wave replays its log back to
// front in 64-entry chunks, re-anchoring the transmittance at the forward's
// checkpoints and recovering it inside a chunk by T_i = T_{i+1} / (1 -
// alpha_i).  Per (wave, splat) it reduces nine sums over the lanes that
// blended the splat -- gg dx^2, gg dx dy, gg dy^2, gg dx, gg dy, gg with
// gg = G dL/dalpha, and alpha T dL/dpixel -- and adds them to the splat's
// grads16 row (slots 0..8) with one 16-lane atomic; launch_finish3d_grads /
// k_project3d_bwd turn them into the raster gradients (finish3d_grads).
// The sums go to reduction slots 0..4 and 8..11, so three first-stage
// pairs of the reduction are empty and skipped (their scratch rows hold
// zeros).
// The log arrives as separate read-only, non-aliasing pointers (not the
// BlendLog struct) so that the compiler can load the wave-uniform entries
// with scalar loads beside the loop's gradient atomics.
__global__ __launch_bounds__(kThreads) void k_raster3d_bwd(int W, int H, int tiles_x, int T,
                                                           const int *__restrict__ offsets,
                                                           const uint4 *__restrict__ log_ent,
                                                           const float *__restrict__ log_ckpt,
                                                           const int *__restrict__ log_table,
                                                           const int *__restrict__ wave_cnt,
                                                           const int *__restrict__ log_overflow,
                                                           const float4 *__restrict__ rec,
                                                           const float *__restrict__ bgp,
                                                           const float *__restrict__ final_Ts,
                                                           const float *__restrict__ dL_dimg,
                                                           float *__restrict__ grads16) {
    const int tile = xcd_strip_tile(blockIdx.x, tiles_x, T / tiles_x);
    if (tile < 0) return;
    if (*log_overflow) return;  // an incomplete log: the step is redone with a larger pool
    constexpr int kWave = 64;
    __shared__ float4 s_r[4][3][64];
    __shared__ float s_red[4][512];
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int pxi = tx * 16 + lane_px(wave, lane);
    const int pyi = ty * 16 + lane_py(wave, lane);
    const bool inside = pxi < W && pyi < H;
    const float px = (float)pxi, py = (float)pyi;
    const int start = offsets[tile], len = offsets[tile + 1] - start;
    const int nlog = __builtin_amdgcn_readfirstlane(wave_cnt[4 * tile + wave]);
    Red8<0, 0xE0> red8;
    red8.init(&s_red[wave][0], lane);
    red8.zero_skipped();
    const int *__restrict__ chunk_of = log_table + log_table_base(start, len, tile, wave);
    const size_t pix = inside ? (size_t)pyi * W + pxi : 0;
    float T_final = 1.f, dp0 = 0.f, dp1 = 0.f, dp2 = 0.f;
    if (inside) {
        T_final = final_Ts[3 * pix];
        dp0 = dL_dimg[3 * pix];
        dp1 = dL_dimg[3 * pix + 1];
        dp2 = dL_dimg[3 * pix + 2];
    }
    const float bgT = -T_final * (bgp[0] * dp0 + bgp[1] * dp1 + bgp[2] * dp2);
    // the nine sums take five permlane pairs: slots 0..4 hold sums 0..4,
    // slots 8..11 sums 5..8; rows 5..7 are empty and skipped.  (Raw rows
    // save a permlane swap each but add a 256-byte row store per visit:
    // six of them made this kernel 7% slower, its visits being short enough
    // for that LDS traffic to bound it, and one was neutral.)
    const int gi = red8.slot < 8 ? red8.slot : red8.slot - 3;
    float acc_v = 0.f;  // the colour suffix projected on dL/dimage
    const int nchunks = (nlog + kWave - 1) / kWave;
    for (int c = nchunks - 1; c >= 0; --c) {
        const int c0 = c * kWave;
        const int m = min(kWave, nlog - c0);
        const int cid = __builtin_amdgcn_readfirstlane(chunk_of[c]);
        const uint4 *__restrict__ lg = log_ent + 64 * (size_t)cid;
        float Tr = c == nchunks - 1 ? T_final : log_ckpt[64 * (size_t)cid + lane];
        if (lane < m) {
            const uint4 e = lg[lane];
            const float4 *r = rec + 3 * (size_t)e.w;
            s_r[wave][0][lane] = r[0];
            s_r[wave][1][lane] = r[1];
            s_r[wave][2][lane] = r[2];
        }
        wave_lds_sync();
        for (int j = m - 1; j >= 0; --j) {
            const uint4 e = lg[j];
            const bool has = __builtin_amdgcn_inverse_ballot_w64(((uint64_t)e.y << 32) | e.x);
            const float4 p0 = s_r[wave][0][j], p1 = s_r[wave][1][j], p2 = s_r[wave][2][j];
            float dx, dy;
            const float rho = conic_rho(p0, p1, px, py, dx, dy);
            // zero where the lane did not blend: alpha, the transmittance
            // factor, the suffix update and every sum follow
            const float G = has ? __builtin_amdgcn_exp2f(rho * -0.72134752044448170368f) : 0.f;
            const float alpha = __builtin_fminf(0.99f, p1.y * G);
            const float inv_om = __builtin_amdgcn_rcpf(1.0f - alpha);
            Tr *= inv_om;
            const float aT = alpha * Tr;
            const float vv = __builtin_fmaf(dp0, p2.x, __builtin_fmaf(dp1, p2.y, dp2 * p2.z));
            const float dv = vv - acc_v;
            const float dLda = __builtin_fmaf(dv, Tr, bgT * inv_om);
            acc_v = __builtin_fmaf(alpha, dv, acc_v);
            const float gg = dLda * G;
            const float gx = gg * dx, gy = gg * dy;
            float v16[16];
            v16[0] = gx * dx;
            v16[1] = gx * dy;
            v16[2] = gy * dy;
            v16[3] = gx;
            v16[4] = gy;
            v16[8] = gg;
            v16[9] = aT * dp0;
            v16[10] = aT * dp1;
            v16[11] = aT * dp2;
            v16[5] = v16[6] = v16[7] = v16[12] = v16[13] = v16[14] = v16[15] = 0.f;
            const float s = wave_reduce16_lds8(v16, red8);
            if (red8.adds && s != 0.f) unsafeAtomicAdd(&grads16[(size_t)e.w * 16 + gi], s);
        }
        wave_lds_sync();
    }
}

}  // namespace

namespace mskern {

void launch_raster3d_fwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets, const int *ids,
                         const float *rec, const float *boxes, const float *bg, float *out_img, float *final_Ts,
                         const BlendLog *blog) {
    const int T = tiles_x * tiles_y;
    if (T <= 0) return;
    const int grid = xcd_strip_grid(tiles_x, tiles_y);
    const auto *r4 = reinterpret_cast<const float4 *>(rec);
    const auto *b4 = reinterpret_cast<const float4 *>(boxes);
    if (blog)
        hipLaunchKernelGGL(k_raster3d_fwd<true>, dim3(grid), dim3(kThreads), 0, s, W, H, tiles_x, T, offsets, ids,
                           r4, b4, bg, out_img, final_Ts, *blog);
    else
        hipLaunchKernelGGL(k_raster3d_fwd<false>, dim3(grid), dim3(kThreads), 0, s, W, H, tiles_x, T, offsets, ids,
                           r4, b4, bg, out_img, final_Ts, BlendLog{});
}

void launch_raster3d_bwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets,
                         const BlendLog &blog, const float *rec, const float *bg, const float *final_Ts,
                         const float *dL_dimg, float *grads16) {
    const int T = tiles_x * tiles_y;
    if (T <= 0) return;
    const int grid = xcd_strip_grid(tiles_x, tiles_y);
    hipLaunchKernelGGL(k_raster3d_bwd, dim3(grid), dim3(kThreads), 0, s, W, H, tiles_x, T, offsets, blog.ent,
                       blog.ckpt, blog.table, blog.wave_cnt, blog.overflow, reinterpret_cast<const float4 *>(rec), bg,
                       final_Ts, dL_dimg, grads16);
}

}  // namespace mskern
