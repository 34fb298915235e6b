// k_raster.hip -- 2DGS front-to-back compositing forward and its backward.
//
// One 256-thread workgroup (four wave64) per 16x16 tile, one pixel per
// thread: each splat record of the tile list is fetched from HBM once per
// tile (the reference runs four 8x8 threadgroups per tile, each reloading
// the list, msplat_metal.metal:8-10, 576-586).  Records are staged in LDS in
// structure-of-arrays float4 planes so the cooperative load is bank-conflict
// free and the per-pixel loop reads a broadcast.  Each wave owns an 8x8
// quadrant of the tile.  At load time each splat gets a 4-bit mask of the
// quadrants whose pixel centres its alpha >= 1/255 region can reach
// (strip_mask_fine), and the batch is compacted into one ascending slot list
// per wave, so a wave only visits the splats that can touch its quadrant and
// every visited splat is a full evaluation.
#include "kernels.h"
#include "ms_device.h"

using namespace msd;

namespace {

constexpr int kThreads = 256;
constexpr float kMScale = FAR_N / (FAR_N - NEAR_N);

// Stages the record of splat gid in LDS slot threadIdx.x and returns its
// wave-strip mask for the tile whose top-left pixel is (sx0, sy0).
__device__ __forceinline__ int load_batch(const float4 *__restrict__ rec, int gid, float4 *s_rec, float sx0,
                                          float sy0) {
    const float4 *r = rec + 5 * (size_t)gid;
    float4 q[5];
#pragma unroll
    for (int k = 0; k < 5; ++k) {
        q[k] = r[k];
        s_rec[k * kThreads + threadIdx.x] = q[k];
    }
    return strip_mask_fine(q[0], q[1], q[2], q[4].z, sx0, sy0);
}

// Per-wave slot lists of one batch: s_list[w][0..n_w) holds, in ascending
// order, the slots whose mask m has bit w.  Returns n for the calling
// thread's wave.  Called by all threads of the workgroup (two barriers).
__device__ __forceinline__ int build_wave_lists(int m, unsigned char (*s_list)[kThreads], int (*s_cnt)[4]) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;
    int pos[4];
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        const unsigned long long bal = __ballot((m >> w) & 1);
        pos[w] = __popcll(bal & below);
        if (lane == 0) s_cnt[wave][w] = __popcll(bal);
    }
    __syncthreads();
#pragma unroll
    for (int w = 0; w < 4; ++w) {
        if ((m >> w) & 1) {
            int off = pos[w];
            for (int wv = 0; wv < wave; ++wv) off += s_cnt[wv][w];
            s_list[w][off] = (unsigned char)threadIdx.x;
        }
    }
    const int n = s_cnt[0][wave] + s_cnt[1][wave] + s_cnt[2][wave] + s_cnt[3][wave];
    __syncthreads();
    return n;
}

// nd_rasterize_forward_2dgs_kernel (msplat_metal.metal:553-754).
__global__ __launch_bounds__(kThreads) void k_raster_fwd(
    int W, int H, int tiles_x, int T, const int *__restrict__ offsets, const int *__restrict__ ids,
    const float4 *__restrict__ rec, const float *__restrict__ bgp, float *__restrict__ out_img,
    float *__restrict__ final_Ts, int *__restrict__ final_idx, float *__restrict__ out_depth,
    float *__restrict__ out_normal, float *__restrict__ out_alpha, float *__restrict__ out_median,
    float *__restrict__ out_dist, unsigned long long *__restrict__ pair_counter) {
    const int tile = xcd_tile(blockIdx.x, T);
    if (tile >= T) return;
    __shared__ float4 s_rec[5 * kThreads];
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int wave = threadIdx.x >> 6;
    const int pxi = tx * 16 + lane_px(threadIdx.x >> 6, threadIdx.x & 63);
    const int pyi = ty * 16 + lane_py(threadIdx.x >> 6, threadIdx.x & 63);
    const bool inside = pxi < W && pyi < H;
    const float px = (float)pxi, py = (float)pyi;
    const float sx0 = (float)(tx * 16), sy0 = (float)(ty * 16);
    const int start = offsets[tile], end = offsets[tile + 1];
    const float bg0 = bgp[0], bg1 = bgp[1], bg2 = bgp[2];

    float Tr = 1.f, cr = 0.f, cg = 0.f, cb = 0.f, dep = 0.f, nx = 0.f, ny = 0.f, nz = 0.f;
    float M1 = 0.f, M2 = 0.f, dist = 0.f, med = 0.f;
    int med_c = -1, last_c = 0;
    bool done = !inside;

    __shared__ unsigned char s_list[4][kThreads];
    __shared__ int s_cnt[4][4];
    int evals = 0;
    for (int b0 = start; b0 < end; b0 += kThreads) {
        if (__syncthreads_and(done)) break;
        const int idx = b0 + (int)threadIdx.x;
        const int m = idx < end ? load_batch(rec, ids[idx], s_rec, sx0, sy0) : 0;
        const int n = build_wave_lists(m, s_list, s_cnt);
        if (done) continue;
        const int base = b0 - start + 1;  // contributor number of slot 0 (1-based)
        int j = 0;
        for (; j < n; ++j) {
            const int t = s_list[wave][j];
            const float4 q0 = s_rec[t], q1 = s_rec[kThreads + t], q2 = s_rec[2 * kThreads + t];
            PairEval e;
            if (!eval_pair(px, py, q0, q1, q2, e)) continue;
            const float next_T = Tr * (1.0f - e.alpha);
            if (next_T <= 1e-4f) {
                done = true;
                ++j;
                break;
            }
            const float w = e.alpha * Tr;
            const float A = 1.f - Tr;
            const float m_ = kMScale * (1.f - NEAR_N / e.depth);
            dist = __builtin_fmaf(m_ * m_ * A + M2 - 2.f * m_ * M1, w, dist);
            M1 = __builtin_fmaf(m_, w, M1);
            M2 = __builtin_fmaf(m_ * m_, w, M2);
            if (Tr > 0.5f) {
                med = e.depth;
                med_c = base + t;
            }
            const float4 q3 = s_rec[3 * kThreads + t], q4 = s_rec[4 * kThreads + t];
            cr = __builtin_fmaf(q3.w, w, cr);
            cg = __builtin_fmaf(q4.x, w, cg);
            cb = __builtin_fmaf(q4.y, w, cb);
            dep = __builtin_fmaf(e.depth, w, dep);
            nx = __builtin_fmaf(q3.x, w, nx);
            ny = __builtin_fmaf(q3.y, w, ny);
            nz = __builtin_fmaf(q3.z, w, nz);
            Tr = next_T;
            last_c = base + t;
        }
        evals += j;
    }
    if (pair_counter) {
        __shared__ unsigned int s_pairs;
        __syncthreads();
        if (threadIdx.x == 0) s_pairs = 0;
        __syncthreads();
        atomicAdd(&s_pairs, (unsigned)evals);
        __syncthreads();
        if (threadIdx.x == 0) atomicAdd(pair_counter, (unsigned long long)s_pairs);
    }
    if (!inside) return;
    const size_t pix = (size_t)pyi * W + pxi;
    final_Ts[3 * pix + 0] = Tr;
    final_Ts[3 * pix + 1] = M1;
    final_Ts[3 * pix + 2] = M2;
    final_idx[2 * pix + 0] = last_c;
    final_idx[2 * pix + 1] = med_c;
    out_img[3 * pix + 0] = __builtin_fmaf(bg0, Tr, cr);
    out_img[3 * pix + 1] = __builtin_fmaf(bg1, Tr, cg);
    out_img[3 * pix + 2] = __builtin_fmaf(bg2, Tr, cb);
    out_depth[pix] = dep;
    out_normal[3 * pix + 0] = nx;
    out_normal[3 * pix + 1] = ny;
    out_normal[3 * pix + 2] = nz;
    out_alpha[pix] = 1.f - Tr;
    out_median[pix] = med;
    out_dist[pix] = dist;
}

// DPP lane permutations within a 16-lane row (CDNA3/4 dpp_ctrl codes).
constexpr int kDppQuad1032 = 0xB1;   // quad_perm [1,0,3,2]: lane ^ 1
constexpr int kDppQuad2301 = 0x4E;   // quad_perm [2,3,0,1]: lane ^ 2
constexpr int kDppHalfMirror = 0x141;  // lane i of each 8-lane half row <- 7 - i
constexpr int kDppRowMirror = 0x140;   // lane i of each row <- 15 - i

template <int CTRL>
__device__ __forceinline__ float dpp(float x) {
    return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(x), CTRL, 0xF, 0xF, false));
}

// Sum of v[0..15] over the 64 lanes of a wave (a transpose reduction):
// v_permlane32_swap / v_permlane16_swap exchange half-waves / half-rows
// between two value registers, so each of those steps halves the value
// count with one swap and one add per pair and no lane select; two mirror
// DPP steps (partners differ in lane bit 3, then bit 2) and two quad_perm
// DPP adds finish.  Lane l ends with the total of value index
// 8*b5 + 4*b4 + 2*b3 + b2 (b = bits of l); every lane of a quad holds it.
__device__ __forceinline__ float wave_reduce16(float v[16], int lane) {
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        // vdst lanes 32-63 <-> src lanes 0-31: lanes < 32 end with value i,
        // lanes >= 32 with value i + 8
        const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 8]), false,
                                                        false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        // odd rows of vdst <-> even rows of src: lane bit 4 selects i + 4
        const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v[i]), __float_as_uint(v[i + 4]), false,
                                                        false);
        v[i] = __uint_as_float(r[0]) + __uint_as_float(r[1]);
    }
    const bool b3 = lane & 8, b2 = lane & 4;
    {
        const float x0 = v[0] + dpp<kDppRowMirror>(v[0]);
        const float x2 = v[2] + dpp<kDppRowMirror>(v[2]);
        const float x1 = v[1] + dpp<kDppRowMirror>(v[1]);
        const float x3 = v[3] + dpp<kDppRowMirror>(v[3]);
        v[0] = b3 ? x2 : x0;
        v[1] = b3 ? x3 : x1;
    }
    {
        const float x0 = v[0] + dpp<kDppHalfMirror>(v[0]);
        const float x1 = v[1] + dpp<kDppHalfMirror>(v[1]);
        v[0] = b2 ? x1 : x0;
    }
    v[0] += dpp<kDppQuad1032>(v[0]);
    v[0] += dpp<kDppQuad2301>(v[0]);
    return v[0];
}

// nd_rasterize_backward_2dgs_kernel (msplat_metal.metal:1705-1979).
// Back-to-front replay starting at the tile's largest last_contributor (the
// reference starts at the end of the full list).  The skip decisions reuse
// the forward's exact arithmetic (eval_pair); quantities that only scale
// gradients use hardware reciprocals.  Per-splat gradients
// [dL_dtransMat 9, dL_dnormal3D 3, dL_dopacity 1, dL_dcolors 3] are reduced
// across the wave and added with one 16-lane global float atomic (one 64-byte
// line) per (wave, splat); with the strip masks a splat is evaluated by
// about 1.3 of the tile's four waves, so this issues no more atomic requests
// than a per-tile merge in LDS would, without its LDS array, zeroing and
// flush barrier.
// FULL = false is the training step's case: the only upstream gradient is
// dL/dimage (depth, alpha, normal, median-depth and distortion gradients are
// zero), so those terms are compiled out.
template <bool FULL>
__global__ __launch_bounds__(kThreads) void k_raster_bwd(
    int W, int H, int tiles_x, int T, const int *__restrict__ offsets, const int *__restrict__ ids,
    const float4 *__restrict__ rec, const float *__restrict__ bgp, const float *__restrict__ final_Ts,
    const int *__restrict__ final_idx, const float *__restrict__ dL_dimg, const float *__restrict__ dL_ddepth,
    const float *__restrict__ dL_daccum, const float *__restrict__ dL_dnormal,
    const float *__restrict__ dL_dmedian, const float *__restrict__ dL_ddist, float ddist_uniform,
    float *__restrict__ grads16) {
    const int tile = xcd_tile(blockIdx.x, T);
    if (tile >= T) return;
    __shared__ float4 s_rec[5 * kThreads];
    __shared__ unsigned char s_list[4][kThreads];
    __shared__ int s_cnt[4][4];
    __shared__ int s_id[kThreads];
    __shared__ int s_maxlast;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int pxi = tx * 16 + lane_px(threadIdx.x >> 6, threadIdx.x & 63);
    const int pyi = ty * 16 + lane_py(threadIdx.x >> 6, threadIdx.x & 63);
    const bool inside = pxi < W && pyi < H;
    const float px = (float)pxi, py = (float)pyi;
    const float sx0 = (float)(tx * 16), sy0 = (float)(ty * 16);
    const int start = offsets[tile];
    const size_t pix = inside ? (size_t)pyi * W + pxi : 0;

    float T_final = 0.f, final_D = 0.f, final_D2 = 0.f;
    int my_last = 0, med_c = -1;
    float dpix[3] = {0.f, 0.f, 0.f}, dn2[3] = {0.f, 0.f, 0.f};
    float ddepth = 0.f, daccum = 0.f, dmed = 0.f, dreg = 0.f;
    if (inside) {
        T_final = final_Ts[3 * pix];
        my_last = final_idx[2 * pix];
        dpix[0] = dL_dimg[3 * pix];
        dpix[1] = dL_dimg[3 * pix + 1];
        dpix[2] = dL_dimg[3 * pix + 2];
        if (FULL) {
            final_D = final_Ts[3 * pix + 1];
            final_D2 = final_Ts[3 * pix + 2];
            med_c = final_idx[2 * pix + 1];
            if (dL_ddepth) ddepth = dL_ddepth[pix];
            if (dL_daccum) daccum = dL_daccum[pix];
            if (dL_dnormal) {
                dn2[0] = dL_dnormal[3 * pix];
                dn2[1] = dL_dnormal[3 * pix + 1];
                dn2[2] = dL_dnormal[3 * pix + 2];
            }
            if (dL_dmedian) dmed = dL_dmedian[pix];
            dreg = dL_ddist ? dL_ddist[pix] : ddist_uniform;
        }
    }
    const float final_A = 1.0f - T_final;
    const float bg_dot = bgp[0] * dpix[0] + bgp[1] * dpix[1] + bgp[2] * dpix[2];

    if (threadIdx.x == 0) s_maxlast = 0;
    __syncthreads();
    if (my_last > 0) atomicMax(&s_maxlast, my_last);
    __syncthreads();
    const int n_it = s_maxlast;

    float Tr = T_final;
    float accum_rec[3] = {0.f, 0.f, 0.f}, last_color[3] = {0.f, 0.f, 0.f};
    float last_alpha = 0.f, accum_depth_rec = 0.f, last_depth = 0.f, accum_alpha_rec = 0.f;
    float accum_normal_rec[3] = {0.f, 0.f, 0.f}, last_normal[3] = {0.f, 0.f, 0.f};
    float last_dL_dT = 0.f;

    for (int hi = n_it; hi > 0; hi -= kThreads) {
        const int bs = min(kThreads, hi);
        __syncthreads();
        int m = 0;
        if ((int)threadIdx.x < bs) {
            const int gid = ids[start + hi - 1 - (int)threadIdx.x];
            s_id[threadIdx.x] = gid;
            m = load_batch(rec, gid, s_rec, sx0, sy0);
        }
        const int n = build_wave_lists(m, s_list, s_cnt);
        for (int j = 0; j < n; ++j) {
            const int t = s_list[wave][j];
            const int c = hi - 1 - t;
            float v[16];
#pragma unroll
            for (int k = 0; k < 16; ++k) v[k] = 0.f;
            bool has = false;
            if (c < my_last) {
                const float4 q0 = s_rec[t], q1 = s_rec[kThreads + t], q2 = s_rec[2 * kThreads + t];
                PairEval e;
                if (eval_pair(px, py, q0, q1, q2, e)) {
                    has = true;
                    const float4 q3 = s_rec[3 * kThreads + t], q4 = s_rec[4 * kThreads + t];
                    const float alpha = e.alpha, G = e.G, opa = q2.w;
                    const float inv_1ma = __builtin_amdgcn_rcpf(1.0f - alpha);
                    Tr = Tr * inv_1ma;
                    const float aT = alpha * Tr;
                    float dL_dalpha = 0.0f;
                    const float cu[3] = {q3.w, q4.x, q4.y};
#pragma unroll
                    for (int ch = 0; ch < 3; ++ch) {
                        const float mask = cu[ch] > 0.0f ? 1.0f : 0.0f;
                        accum_rec[ch] = last_alpha * last_color[ch] + (1.f - last_alpha) * accum_rec[ch];
                        last_color[ch] = cu[ch];
                        dL_dalpha += (cu[ch] - accum_rec[ch]) * dpix[ch];
                        v[13 + ch] = aT * dpix[ch] * mask;
                    }
                    float dL_dz = 0.0f;
                    if (FULL) {
                        float dL_dweight = 0.0f;
                        const float inv_d = __builtin_amdgcn_rcpf(e.depth);
                        const float m_d = kMScale * (1.0f - NEAR_N * inv_d);
                        const float dmd_dd = (FAR_N * NEAR_N) / (FAR_N - NEAR_N) * inv_d * inv_d;
                        if (c == med_c - 1) dL_dz += dmed;
                        dL_dweight += (final_D2 + m_d * m_d * final_A - 2.0f * m_d * final_D) * dreg;
                        dL_dalpha += dL_dweight - last_dL_dT;
                        last_dL_dT = dL_dweight * alpha + (1.0f - alpha) * last_dL_dT;
                        const float dL_dmd = 2.0f * aT * (m_d * final_A - final_D) * dreg;
                        dL_dz += dL_dmd * dmd_dd;
                        accum_depth_rec = last_alpha * last_depth + (1.f - last_alpha) * accum_depth_rec;
                        last_depth = e.depth;
                        dL_dalpha += (e.depth - accum_depth_rec) * ddepth;
                        accum_alpha_rec = last_alpha * 1.0f + (1.f - last_alpha) * accum_alpha_rec;
                        dL_dalpha += (1.0f - accum_alpha_rec) * daccum;
                        const float nrm[3] = {q3.x, q3.y, q3.z};
#pragma unroll
                        for (int ch = 0; ch < 3; ++ch) {
                            accum_normal_rec[ch] =
                                last_alpha * last_normal[ch] + (1.f - last_alpha) * accum_normal_rec[ch];
                            last_normal[ch] = nrm[ch];
                            dL_dalpha += (nrm[ch] - accum_normal_rec[ch]) * dn2[ch];
                            v[9 + ch] = aT * dn2[ch];
                        }
                        dL_dz += aT * ddepth;
                    }
                    dL_dalpha *= Tr;
                    last_alpha = alpha;
                    dL_dalpha += (-T_final * inv_1ma) * bg_dot;
                    const float dL_dG = opa * dL_dalpha;
                    const float Twx = q1.z, Twy = q1.w;
                    if (e.rho3d <= e.rho2d) {
                        const float dsx = dL_dG * -G * e.u + dL_dz * Twx;
                        const float dsy = dL_dG * -G * e.v + dL_dz * Twy;
                        const float dsx_pz = dsx * e.inv_z, dsy_pz = dsy * e.inv_z;
                        const f3 dp = {dsx_pz, dsy_pz, -(dsx_pz * e.u + dsy_pz * e.v)};
                        const f3 &k = e.k, &l = e.l;
                        const f3 dk = {l.y * dp.z - l.z * dp.y, l.z * dp.x - l.x * dp.z, l.x * dp.y - l.y * dp.x};
                        const f3 dl = {dp.y * k.z - dp.z * k.y, dp.z * k.x - dp.x * k.z, dp.x * k.y - dp.y * k.x};
                        v[0] = -dk.x;
                        v[1] = -dk.y;
                        v[2] = -dk.z;
                        v[3] = -dl.x;
                        v[4] = -dl.y;
                        v[5] = -dl.z;
                        v[6] = px * dk.x + py * dl.x + dL_dz * e.u;
                        v[7] = px * dk.y + py * dl.y + dL_dz * e.v;
                        v[8] = px * dk.z + py * dl.z + dL_dz;
                    } else if (FULL) {
                        v[6] = e.u * dL_dz;
                        v[7] = e.v * dL_dz;
                        v[8] = dL_dz;
                    }
                    v[12] = G * dL_dalpha * (opa * (1.0f - opa));
                }
            }
            if (__any(has)) {
                const float s = wave_reduce16(v, lane);
                if ((lane & 3) == 0) {
                    const int vi = ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 +
                                   ((lane >> 2) & 1);
                    if (s != 0.f) unsafeAtomicAdd(&grads16[(size_t)s_id[t] * 16 + vi], s);
                }
            }
        }
    }
}

}  // namespace

namespace mskern {

void launch_raster_fwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets, const int *ids,
                       const float *rec, const float *bg, float *out_img, float *final_Ts, int *final_idx,
                       float *out_depth, float *out_normal, float *out_alpha, float *out_median, float *out_dist,
                       unsigned long long *pair_counter) {
    const int T = tiles_x * tiles_y;
    const int grid = ((T + 7) / 8) * 8;
    hipLaunchKernelGGL(k_raster_fwd, dim3(grid), dim3(kThreads), 0, s, W, H, tiles_x, T, offsets, ids,
                       reinterpret_cast<const float4 *>(rec), bg, out_img, final_Ts, final_idx, out_depth,
                       out_normal, out_alpha, out_median, out_dist, pair_counter);
}

void launch_raster_bwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets, const int *ids,
                       const float *rec, const float *bg, const float *final_Ts, const int *final_idx,
                       const float *dL_dimg, const float *dL_ddepth, const float *dL_daccum,
                       const float *dL_dnormal, const float *dL_dmedian, const float *dL_ddist,
                       float ddist_uniform, float *grads16) {
    const int T = tiles_x * tiles_y;
    const int grid = ((T + 7) / 8) * 8;
    const bool full = dL_ddepth || dL_daccum || dL_dnormal || dL_dmedian || dL_ddist || ddist_uniform != 0.0f;
    if (full)
        hipLaunchKernelGGL(k_raster_bwd<true>, dim3(grid), dim3(kThreads), 0, s, W, H, tiles_x, T, offsets, ids,
                           reinterpret_cast<const float4 *>(rec), bg, final_Ts, final_idx, dL_dimg, dL_ddepth,
                           dL_daccum, dL_dnormal, dL_dmedian, dL_ddist, ddist_uniform, grads16);
    else
        hipLaunchKernelGGL(k_raster_bwd<false>, dim3(grid), dim3(kThreads), 0, s, W, H, tiles_x, T, offsets, ids,
                           reinterpret_cast<const float4 *>(rec), bg, final_Ts, final_idx, dL_dimg, dL_ddepth,
                           dL_daccum, dL_dnormal, dL_dmedian, dL_ddist, ddist_uniform, grads16);
}

}  // namespace mskern
