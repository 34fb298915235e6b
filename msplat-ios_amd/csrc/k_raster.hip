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
// (quad_mask on the splat's MaskRec, precomputed by the projection), and the
// batch is compacted into one ascending slot list per wave, so a wave only
// visits the splats that can touch its quadrant and every visited splat is
// a full evaluation.
#include "kernels.h"
#include "ms_device.h"
#include "raster_wave.h"

using namespace msd;
using namespace msr;

namespace {

constexpr float kMScale = FAR_N / (FAR_N - NEAR_N);

// Stages splat gid, list position pos, in LDS slot threadIdx.x and returns
// its wave-block mask for the tile whose top-left pixel is (sx0, sy0) (the
// per-tile part of the quadrant-mask test, quad_mask, on the splat's
// MaskRec).  Planes: 0..2 the centred ray rows, centre and opacity
// (eval_pair's p0..p2), 3 = (Tw, pos), 4 = (colour, gid), 5 = (normal, 0)
// when NORMAL.
template <bool NORMAL>
__device__ __forceinline__ int load_batch(const float4 *__restrict__ rec, const float4 *__restrict__ mrec, int gid,
                                          int pos, float4 *s_rec, float sx0, float sy0) {
    const float4 *r = rec + 5 * (size_t)gid;
    const float4 q0 = r[0], q1 = r[1], q2 = r[2], q3 = r[3], q4 = r[4];
    const float4 *mr = mrec + 3 * (size_t)gid;
    const MaskRec m = {mr[0], mr[1], mr[2]};
    const f3 Tw = {q1.z, q1.w, q2.x};
    f3 R0, nAx, nAy;
    centred_rows({q0.x, q0.y, q0.z}, {q0.w, q1.x, q1.y}, Tw, q2.y, q2.z, R0, nAx, nAy);
    s_rec[threadIdx.x] = make_float4(R0.x, R0.y, R0.z, nAx.x);
    s_rec[kThreads + threadIdx.x] = make_float4(nAx.y, nAx.z, nAy.x, nAy.y);
    s_rec[2 * kThreads + threadIdx.x] = make_float4(nAy.z, q2.y, q2.z, q2.w);
    s_rec[3 * kThreads + threadIdx.x] = make_float4(Tw.x, Tw.y, Tw.z, __int_as_float(pos));
    s_rec[4 * kThreads + threadIdx.x] = make_float4(q3.w, q4.x, q4.y, __int_as_float(gid));
    if (NORMAL) s_rec[5 * kThreads + threadIdx.x] = make_float4(q3.x, q3.y, q3.z, 0.f);
    return quad_mask(m, q4.w, q2.y, q2.z, sx0, sy0);
}

// nd_rasterize_forward_2dgs_kernel (msplat_metal.metal:553-754).
// With LOG, every wave also writes its blend log for the backward: one entry
// {ballot low, ballot high, list position, splat id} for each visited list
// entry that at least one of its lanes blended, in visit (front-to-back)
// order, in 64-entry pool chunks (BlendLog); wave_cnt[4 * tile + wave]
// receives the entry count.  Bit l of the ballot is set when lane l's pixel
// blended the splat, so the backward replays exactly the forward's
// decisions.  When a chunk is complete each lane also stores, as the
// chunk's checkpoint, its transmittance before the next log entry (a prefix
// checkpoint).
// COUNT adds the work counters {pairs evaluated, log entries, pairs
// blended, (wave, splat) visits, visit slots} to pair_counter.
// With FULL_OUT = false only what the image-only training step consumes is
// produced: out_img and final_Ts[.][0] (T); the last and median contributor
// indices, the depth, normal, alpha, median and distortion outputs and the
// distortion moments are neither accumulated nor written.  Every
// decision, and so every produced value, is the same as with FULL_OUT.
// 7 waves per SIMD: the LDS of the image-only kernel allows 7 workgroups
// per CU, and at most 72 VGPRs keep all of them resident (the compiler
// would otherwise use more and fit 6; with two visits per iteration it
// spills one value, reloaded once per batch, which costs less than the
// seventh wave saves).
template <bool LOG, bool FULL_OUT, bool COUNT>
__global__ __launch_bounds__(kThreads) __attribute__((amdgpu_waves_per_eu(7, 8))) void k_raster_fwd(
    int W, int H, int tiles_x, int T, const int *__restrict__ offsets, const int *__restrict__ ids,
    const float4 *__restrict__ rec, const float4 *__restrict__ mrec, const float *__restrict__ bgp,
    float *__restrict__ out_img, float *__restrict__ final_Ts, int *__restrict__ final_idx, float *__restrict__ out_depth,
    float *__restrict__ out_normal, float *__restrict__ out_alpha, float *__restrict__ out_median,
    float *__restrict__ out_dist, unsigned long long *__restrict__ pair_counter, BlendLog blog, int deep_len) {
    const int tile = xcd_strip_tile(blockIdx.x, tiles_x, T / tiles_x);
    if (tile < 0) return;
    __shared__ float4 s_rec[(FULL_OUT ? 6 : 5) * kThreads];  // the batch's records (load_batch planes)
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int lane = threadIdx.x & 63;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int pxi = tx * 16 + lane_px(wave, lane);
    const int pyi = ty * 16 + lane_py(wave, lane);
    const bool inside = pxi < W && pyi < H;
    float px = (float)pxi, py = (float)pyi;
    // kept in registers (the compiler would otherwise convert them again on
    // every visit)
    asm volatile("" : "+v"(px), "+v"(py));
    const float sx0 = (float)(tx * 16), sy0 = (float)(ty * 16);
    const int start = offsets[tile], end = offsets[tile + 1];
    if (end - start >= deep_len) return;  // k_raster_deep renders it
    const float bg0 = bgp[0], bg1 = bgp[1], bg2 = bgp[2];
    LogWriter lw;
    lw.tb = LOG ? log_table_base(start, end - start, tile, wave) : 0;
    lw.sp = LOG ? log_subpool(blog, tile, wave) : 0;
    if (LOG && end > start) lw.start(blog, lane);  // an empty list logs nothing
    int nlog = 0;  // wave-uniform
    // the current 64-entry chunk of the wave's log: lane k holds entry k,
    // and a full chunk is written with one coalesced store
    uint4 lg_ent = make_uint4(0u, 0u, 0u, 0u);
    const char *s_bytes = reinterpret_cast<const char *>(s_rec);

    float Tr = 1.f, cr = 0.f, cg = 0.f, cb = 0.f, dep = 0.f, nx = 0.f, ny = 0.f, nz = 0.f;
    float M1 = 0.f, M2 = 0.f, dist = 0.f, med = 0.f;
    int med_c = -1, last_c = 0;
    // the wave's lanes whose pixel is finished (outside the image or
    // terminated); the visit loop keeps every lane decision as a lane mask
    uint64_t done_m = __builtin_amdgcn_ballot_w64(!inside);

    __shared__ unsigned char s_list[4][kThreads];
    __shared__ int4 s_cnt[4];  // s_cnt[wave] = the wave's slot counts per block
    // wave totals of the work counters (scalar: ballot popcounts)
    unsigned evals = 0, blends = 0;
    // COUNT: each wave's visits in the current batch; a batch lasts as long
    // as its busiest wave (the barriers), so it accounts for 4 x max slots
    __shared__ int s_vis[4];
    unsigned visits = 0, slots = 0;
    if (COUNT && threadIdx.x < 4) s_vis[threadIdx.x] = 0;
    for (int b0 = start; b0 < end; b0 += kThreads) {
        if (__syncthreads_and(done_m == ~0ull)) break;
        if (COUNT && threadIdx.x == 0)
            slots += 4u * (unsigned)max(max(s_vis[0], s_vis[1]), max(s_vis[2], s_vis[3]));
        const int idx = b0 + (int)threadIdx.x;
        const int gid = idx < end ? ids[idx] : 0;
        const int m = idx < end ? load_batch<FULL_OUT>(rec, mrec, gid, idx - start, s_rec, sx0, sy0) : 0;
        const int n = build_wave_lists(m, s_list, s_cnt);
        int nv = 0;
        // one visit of slot list entry j; a visit after the wave is done
        // changes nothing (no lane is active, so nothing blends or is logged)
        const auto visit = [&](int j) {
            if (COUNT) nv += done_m != ~0ull;
            const int to = 16 * (int)s_list[wave][j];  // byte offset of the slot in a record plane
            const auto plane = [&](int k) {
                return *reinterpret_cast<const float4 *>(s_bytes + k * (kThreads * 16) + to);
            };
            // predicated: a lane that is done or rejects the pair adds
            // colour * 0 (bit-identical sums) and keeps its state
            if (COUNT) evals += __builtin_popcountll(~done_m);
            const float4 q0 = plane(0), q1 = plane(1), q2 = plane(2), q3 = plane(3);
            PairEval e;
            const uint64_t act = eval_pair(px, py, q0, q1, q2, q3, e) & ~done_m;
            const float next_T = Tr * (1.0f - e.alpha);
            const uint64_t term = act & __builtin_amdgcn_ballot_w64(next_T <= 1e-4f);
            const uint64_t bal = act & ~term;  // the lanes that blend the splat
            done_m |= term;
            const bool blend = __builtin_amdgcn_inverse_ballot_w64(bal);
            const float w = blend ? e.alpha * Tr : 0.0f;
            const float4 q4 = plane(4);
            if (FULL_OUT) {
                // 1-based list position of the splat (the reference's contributor count)
                const int contrib = __float_as_int(q3.w) + 1;
                const float A = 1.f - Tr;
                const float dep_s = blend ? e.depth : 1.0f;  // finite stand-in off the blend
                const float m_ = kMScale * (1.f - NEAR_N / dep_s);
                dist = __builtin_fmaf(m_ * m_ * A + M2 - 2.f * m_ * M1, w, dist);
                M1 = __builtin_fmaf(m_, w, M1);
                M2 = __builtin_fmaf(m_ * m_, w, M2);
                const bool med_now = blend & (Tr > 0.5f);
                med = med_now ? e.depth : med;
                med_c = med_now ? contrib : med_c;
                dep = __builtin_fmaf(dep_s, w, dep);
                const float4 q5 = plane(5);
                nx = __builtin_fmaf(q5.x, w, nx);
                ny = __builtin_fmaf(q5.y, w, ny);
                nz = __builtin_fmaf(q5.z, w, nz);
                last_c = blend ? contrib : last_c;
            }
            cr = __builtin_fmaf(q4.x, w, cr);
            cg = __builtin_fmaf(q4.y, w, cg);
            cb = __builtin_fmaf(q4.z, w, cb);
            Tr = blend ? next_T : Tr;
            if (COUNT) blends += __builtin_popcountll(bal);
            if (LOG && bal) {
                const bool mine = __builtin_amdgcn_inverse_ballot_w64(1ull << (nlog & 63));
                lg_ent.x = mine ? (unsigned)bal : lg_ent.x;
                lg_ent.y = mine ? (unsigned)(bal >> 32) : lg_ent.y;
                lg_ent.z = mine ? __float_as_uint(q3.w) : lg_ent.z;
                lg_ent.w = mine ? __float_as_uint(q4.w) : lg_ent.w;
                // the transmittance before the next logged splat is the
                // current one (a visit no lane blends changes nothing)
                if ((++nlog & 63) == 0) lw.full(blog, lane, nlog, lg_ent, Tr);
            }
        };
        // two visits per iteration: the second's work up to alpha does not
        // depend on the first's blend, so the two can be interleaved
        int j = 0;
        for (; j + 1 < n && done_m != ~0ull; j += 2) {
            visit(j);
            visit(j + 1);
        }
        if (j < n && done_m != ~0ull) visit(j);
        if (COUNT) {
            visits += (unsigned)nv;
            if (lane == 0) s_vis[wave] = nv;
        }
    }
    if (LOG) lw.finish(blog, lane, nlog, lg_ent, tile, wave);  // the last, partial chunk
    if (COUNT) {
        // {pairs evaluated, log entries, pairs blended, visits, visit slots}
        __shared__ unsigned int s_cnt5[5];
        __syncthreads();
        if (threadIdx.x == 0)
            slots += 4u * (unsigned)max(max(s_vis[0], s_vis[1]), max(s_vis[2], s_vis[3]));
        if (threadIdx.x < 5) s_cnt5[threadIdx.x] = 0;
        __syncthreads();
        if (lane == 0) {
            atomicAdd(&s_cnt5[0], evals);
            atomicAdd(&s_cnt5[2], blends);
            atomicAdd(&s_cnt5[1], (unsigned)nlog);
            atomicAdd(&s_cnt5[3], visits);
        }
        if (threadIdx.x == 0) atomicAdd(&s_cnt5[4], slots);
        __syncthreads();
        if (threadIdx.x < 5) atomicAdd(pair_counter + threadIdx.x, (unsigned long long)s_cnt5[threadIdx.x]);
    }
    if (!inside) return;
    const size_t pix = (size_t)pyi * W + pxi;
    final_Ts[3 * pix + 0] = Tr;
    out_img[3 * pix + 0] = __builtin_fmaf(bg0, Tr, cr);
    out_img[3 * pix + 1] = __builtin_fmaf(bg1, Tr, cg);
    out_img[3 * pix + 2] = __builtin_fmaf(bg2, Tr, cb);
    if (!FULL_OUT) return;
    final_idx[2 * pix + 0] = last_c;
    final_Ts[3 * pix + 1] = M1;
    final_Ts[3 * pix + 2] = M2;
    final_idx[2 * pix + 1] = med_c;
    out_depth[pix] = dep;
    out_normal[3 * pix + 0] = nx;
    out_normal[3 * pix + 1] = ny;
    out_normal[3 * pix + 2] = nz;
    out_alpha[pix] = 1.f - Tr;
    out_median[pix] = med;
    out_dist[pix] = dist;
}

// nd_rasterize_backward_2dgs_kernel (msplat_metal.metal:1705-1979) over the
// forward's blend log, with prefix/suffix transmittance.
//
// Each wave replays its blend log back to front in 64-entry chunks.  The
// log's ballots carry the forward's exact blend decisions, so the backward
// needs neither the strip masks nor the forward's correctly rounded ray
// division and exp: u, v, G and alpha only scale gradients and use the
// hardware reciprocal and exp2.  The suffix sums (colour, and in the full
// case depth, alpha, normal and the distortion term) follow the reference's
// back-to-front recurrences (:1846-1916), whose rounding error scales with
// the transmittance.  The transmittance itself is a prefix: at the end of
// every chunk it is re-anchored to the forward's checkpoint (the exact
// product the forward computed), and inside a chunk it is recovered by at
// most 64 divisions T_i = T_{i+1} / (1 - alpha_i); the reference recovers it
// by division over the whole list from T_final (:1858).
// The 16 per-splat gradients [dL_dtransMat 9, dL_dnormal3D 3, dL_dopacity,
// dL_dcolors 3] are reduced across the wave and added with one 16-lane
// global float atomic (one 64-byte line) per (wave, splat).
// FULL = false is the training step's case: the only upstream gradient is
// dL/dimage, so the depth / alpha / normal / median / distortion terms are
// compiled out and the colour suffix is carried as its projection on
// dL/dimage.  Its grads16 rows hold per-splat sums without their per-splat
// factors: the nine ray moments without -opacity, the opacity-logit sum
// without opacity (1 - opacity), the colour sums without the clamp mask;
// finish_image_grads applies them once per splat.
template <bool FULL>
struct BwdLds;
template <>
struct BwdLds<true> {
    float4 r[4][7][64];
    uint4 e[4][64];
};
template <>
struct BwdLds<false> {
    float4 r[4][4][32];
    float red[4][512];
};

// The image-only reduction's slots: 13 non-zero sums in five permlane pairs
// (rows 0, 2, 4, 6, 7) and three raw rows (1, 3, 5), so five permlane swaps
// per visit instead of seven.  Nibble k of kImgGrad is the grads16 index of
// reduction slot k (the unused upper slots of raw rows read 0).
constexpr unsigned kImgRaw = 0x2A;
constexpr unsigned long long kImgGrad = 0xfe0c0308d7654210ull;

template <bool FULL>
__global__ __launch_bounds__(kThreads) void k_raster_bwd(
    int W, int H, int tiles_x, int T, const int *__restrict__ offsets, BlendLog blog, const float4 *__restrict__ rec,
    const float *__restrict__ bgp, const float *__restrict__ final_Ts, const int *__restrict__ final_idx,
    const float *__restrict__ dL_dimg, const float *__restrict__ dL_ddepth, const float *__restrict__ dL_daccum,
    const float *__restrict__ dL_dnormal, const float *__restrict__ dL_dmedian, const float *__restrict__ dL_ddist,
    float ddist_uniform, float *__restrict__ grads16, const int *__restrict__ tile_list, int deep_len) {
    // tile_list: the deep tiles (their own launch); otherwise every other
    // tile, XCD-mapped
    const int tile = tile_list ? tile_list[blockIdx.x] : xcd_strip_tile(blockIdx.x, tiles_x, T / tiles_x);
    if (tile < 0) return;
    if (!tile_list && offsets[tile + 1] - offsets[tile] >= deep_len) return;
    if (overflowed(blog)) return;  // an incomplete log: the step is redone with a larger pool
    constexpr int kWave = 64;
    // per wave: the staged entries' record planes (the image-only path
    // stages 4, the full one 7) and the log entries (full) or the reduction
    // scratch (image-only, wave_reduce16_lds8); 16 KB per workgroup for the
    // image-only kernel
    __shared__ BwdLds<FULL> L;
    auto &s_r = L.r;
    const int lane = threadIdx.x & 63;
    // uniform, so that the log entries of the image-only loop are scalar loads
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int pxi = tx * 16 + lane_px(wave, lane);
    const int pyi = ty * 16 + lane_py(wave, lane);
    const bool inside = pxi < W && pyi < H;
    const float px = (float)pxi, py = (float)pyi;
    const int start = offsets[tile], len = offsets[tile + 1] - start;
    const int nlog = __builtin_amdgcn_readfirstlane(blog.wave_cnt[4 * tile + wave]);
    Red8<kImgRaw> red8;
    if (!FULL) red8.init(reinterpret_cast<float *>(&L) + sizeof(L.r) / sizeof(float) + wave * 512, lane);
    const int *__restrict__ chunk_of = blog.table + log_table_base(start, len, tile, wave);
    const size_t pix = inside ? (size_t)pyi * W + pxi : 0;

    float T_final = 1.f, dp0 = 0.f, dp1 = 0.f, dp2 = 0.f;
    float dn0 = 0.f, dn1 = 0.f, dn2 = 0.f, ddep = 0.f, dacc = 0.f, dmed = 0.f, dreg = 0.f;
    float fD = 0.f, fD2 = 0.f;
    int med_pos = -2;
    if (inside) {
        T_final = final_Ts[3 * pix];
        dp0 = dL_dimg[3 * pix];
        dp1 = dL_dimg[3 * pix + 1];
        dp2 = dL_dimg[3 * pix + 2];
        if (FULL) {
            fD = final_Ts[3 * pix + 1];
            fD2 = final_Ts[3 * pix + 2];
            med_pos = final_idx[2 * pix + 1] - 1;
            if (dL_ddepth) ddep = dL_ddepth[pix];
            if (dL_daccum) dacc = dL_daccum[pix];
            if (dL_dnormal) {
                dn0 = dL_dnormal[3 * pix];
                dn1 = dL_dnormal[3 * pix + 1];
                dn2 = dL_dnormal[3 * pix + 2];
            }
            if (dL_dmedian) dmed = dL_dmedian[pix];
            dreg = dL_ddist ? dL_ddist[pix] : ddist_uniform;
        }
    }
    const float fA = 1.0f - T_final;
    const float bgT = -T_final * (bgp[0] * dp0 + bgp[1] * dp1 + bgp[2] * dp2);
    // lane l of the reduction ends with slot vi (see wave_reduce16), which
    // holds grads16 index gi (image-only: slot red8.slot, its index in
    // kImgGrad; only the lanes red8.adds marks hold a whole sum)
    const int vi = ((lane >> 5) & 1) * 8 + ((lane >> 4) & 1) * 4 + ((lane >> 3) & 1) * 2 + ((lane >> 2) & 1);
    const int gi = FULL ? vi : (int)((kImgGrad >> (4 * red8.slot)) & 15u);
    const bool adds = FULL ? (lane & 3) == 0 : red8.adds;

    // suffix state of the reference's recurrences (image-only: the colour
    // suffix projected on dL/dimage, updated as soon as a splat is done)
    float last_alpha = 0.f, acc_v = 0.f;
    float acc_c[3] = {0.f, 0.f, 0.f}, last_c[3] = {0.f, 0.f, 0.f};
    float acc_d = 0.f, last_d = 0.f, acc_a = 0.f, last_dLdT = 0.f;
    float acc_n[3] = {0.f, 0.f, 0.f}, last_n[3] = {0.f, 0.f, 0.f};

    // entries staged per chunk: 64 (full), 32 (image-only: 16 KB of LDS per
    // workgroup, so that its 52 VGPRs, not LDS, set the waves per SIMD)
    constexpr int kChunk = FULL ? kWave : kWave / 2;
    const int nchunks = (nlog + kChunk - 1) / kChunk;
    float Tr = T_final;
    for (int c = nchunks - 1; c >= 0; --c) {
        const int c0 = c * kChunk;
        const int m = min(kChunk, nlog - c0);
        // transmittance after the chunk's last splat: the final
        // transmittance, the prefix checkpoint of the entry after it when
        // that entry is a multiple of 64, else the value the recurrence of
        // the chunk after it ended with (the same operations in the same
        // order as one 64-entry chunk)
        // the pool chunk holding entries c0 .. c0 + m - 1, and its checkpoint
        const int cid = __builtin_amdgcn_readfirstlane(chunk_of[c0 >> 6]);
        const uint4 *__restrict__ lg = blog.ent + 64 * (size_t)cid + (c0 & 63);
        if (c != nchunks - 1 && ((c0 + kChunk) & (kWave - 1)) == 0) Tr = blog.ckpt[64 * (size_t)cid + lane];
        if (lane < m) {
            const uint4 e = lg[lane];
            const float4 *r = rec + 5 * (size_t)e.w;
            // the forward's centred ray rows (centred_rows), then the colour;
            // the full case adds the raw transMat rows and the normal
            const float4 q0 = r[0], q1 = r[1], q2 = r[2], q3 = r[3], q4 = r[4];
            f3 R0, nAx, nAy;
            centred_rows({q0.x, q0.y, q0.z}, {q0.w, q1.x, q1.y}, {q1.z, q1.w, q2.x}, q2.y, q2.z, R0, nAx, nAy);
            s_r[wave][0][lane] = make_float4(R0.x, R0.y, R0.z, nAx.x);
            s_r[wave][1][lane] = make_float4(nAx.y, nAx.z, nAy.x, nAy.y);
            s_r[wave][2][lane] = make_float4(nAy.z, q2.y, q2.z, q2.w);
            if constexpr (FULL) {
                s_r[wave][3][lane] = q0;
                s_r[wave][4][lane] = q1;
                s_r[wave][5][lane] = make_float4(q2.x, q3.w, q4.x, q4.y);
                s_r[wave][6][lane] = make_float4(q3.x, q3.y, q3.z, 0.f);
            } else {
                s_r[wave][3][lane] = make_float4(q3.w, q4.x, q4.y, 0.f);
            }
            if constexpr (FULL) L.e[wave][lane] = e;
        }
        wave_lds_sync();
        // image-only: the entries' addresses are uniform (scalar loads),
        // each fetched one visit ahead so its latency is not waited on, and
        // an entry's ballot is the lane mask of `has` itself
        uint4 e_next;
        if constexpr (!FULL) e_next = lg[m - 1];
        for (int j = m - 1; j >= 0; --j) {
            uint4 e;
            if constexpr (FULL) {
                e = L.e[wave][j];
            } else {
                e = e_next;
                e_next = lg[max(j - 1, 0)];
            }
            const bool has = FULL ? (((lane < 32 ? e.x : e.y) >> (lane & 31)) & 1u)
                                  : __builtin_amdgcn_inverse_ballot_w64(((uint64_t)e.y << 32) | e.x);
            float v16[16];
            if constexpr (!FULL) {
                const float4 q0 = s_r[wave][0][j], q1 = s_r[wave][1][j], q2 = s_r[wave][2][j];
                const float4 q3 = s_r[wave][3][j];
                const float opa = q2.w;
                const float dxs = q2.y - px, dys = q2.z - py;
                const float rx = __builtin_fmaf(dxs, q0.w, __builtin_fmaf(dys, q1.z, q0.x));
                const float ry = __builtin_fmaf(dxs, q1.x, __builtin_fmaf(dys, q1.w, q0.y));
                const float rz = __builtin_fmaf(dxs, q1.y, __builtin_fmaf(dys, q2.x, q0.z));
                const float inv_z = has ? __builtin_amdgcn_rcpf(rz) : 0.f;
                const float u = rx * inv_z, v = ry * inv_z;
                const float rho3d = __builtin_fmaf(u, u, v * v);
                const float rho2d = FILTER_INV_SQ * __builtin_fmaf(dxs, dxs, dys * dys);
                const bool use3d = rho3d <= rho2d;
                // zero where the lane did not blend: alpha, the transmittance
                // factor, the suffix update and every gradient term follow
                const float G =
                    has ? __builtin_amdgcn_exp2f(__builtin_fminf(rho3d, rho2d) * -0.72134752044448170368f) : 0.f;
                const float alpha = __builtin_fminf(0.99f, opa * G);
                const float inv_om = __builtin_amdgcn_rcpf(1.0f - alpha);
                Tr *= inv_om;  // transmittance before this splat (unchanged where it did not blend)
                const float aT = alpha * Tr;
                const float vv = __builtin_fmaf(dp0, q3.x, __builtin_fmaf(dp1, q3.y, dp2 * q3.z));  // dL/dimage . colour
                // acc_v is the suffix behind this splat.  The reference
                // folds a splat in when the next blended splat is reached
                // (last_alpha / last_color, :1875-1876, :1919); folding it
                // in as soon as it is done uses the same values, and
                // alpha = 0 leaves the suffix unchanged without a select
                const float dv = vv - acc_v;
                const float dLda = __builtin_fmaf(dv, Tr, bgT * inv_om);
                acc_v = __builtin_fmaf(alpha, dv, acc_v);
                const float gg = dLda * G;
                // dL/d(ray), up to the factor -opa, on the 3D branch: the
                // ray-splat point (gg u, gg v) / ray.z pulled back through
                // (u, v) = ray.xy / ray.z; its moments over the wave's pixels
                // about the splat centre (sum dp, sum (xs - px) dp,
                // sum (ys - py) dp) determine the nine transMat gradients
                const float t = (use3d ? gg : 0.f) * inv_z;
                const float dsx = t * u;
                const float dsy = t * v;
                const float dpz = -__builtin_fmaf(dsx, u, dsy * v);
                // reduction slots (kImgRaw, kImgGrad): pairs (0, 8), (2, 10),
                // (4, 12), (6, 14), (7, 15) and raw rows 1, 3, 5; the normal
                // gradients (grads16 9-11) are zero here and take no slot
                v16[0] = dsx;
                v16[8] = dys * dpz;
                v16[1] = dsy;
                v16[2] = dpz;
                v16[10] = dxs * dsx;
                v16[3] = dxs * dsy;
                v16[4] = dxs * dpz;
                v16[12] = gg;
                v16[5] = dys * dsx;
                v16[6] = dys * dsy;
                v16[14] = aT * dp1;
                v16[7] = aT * dp0;
                v16[15] = aT * dp2;
                v16[9] = v16[11] = v16[13] = 0.f;  // raw rows' partners: not read
            } else {
                const float4 c0 = s_r[wave][0][j], c1 = s_r[wave][1][j], c2 = s_r[wave][2][j];
                const float4 q0 = s_r[wave][3][j], q1 = s_r[wave][4][j], q5 = s_r[wave][5][j];
                const float4 q6 = s_r[wave][6][j];
                const float Tux = q0.x, Tuy = q0.y, Tuz = q0.z, Tvx = q0.w, Tvy = q1.x, Tvz = q1.y;
                const float Twx = q1.z, Twy = q1.w, Twz = q5.x;
                const float opa = c2.w;
                // k and l carry the transMat gradients; the ray is the
                // forward's centred one, bit for bit (so ray.z is non-zero
                // wherever the lane blended)
                const f3 k = {__builtin_fmaf(px, Twx, -Tux), __builtin_fmaf(px, Twy, -Tuy),
                              __builtin_fmaf(px, Twz, -Tuz)};
                const f3 l = {__builtin_fmaf(py, Twx, -Tvx), __builtin_fmaf(py, Twy, -Tvy),
                              __builtin_fmaf(py, Twz, -Tvz)};
                const float dxs = c2.y - px, dys = c2.z - py;
                const float rx = __builtin_fmaf(dxs, c0.w, __builtin_fmaf(dys, c1.z, c0.x));
                const float ry = __builtin_fmaf(dxs, c1.x, __builtin_fmaf(dys, c1.w, c0.y));
                const float rz = __builtin_fmaf(dxs, c1.y, __builtin_fmaf(dys, c2.x, c0.z));
                const float inv_z = has ? __builtin_amdgcn_rcpf(rz) : 0.f;
                const float u = rx * inv_z;
                const float v = ry * inv_z;
                const float rho3d = __builtin_fmaf(u, u, v * v);
                const float rho2d = FILTER_INV_SQ * __builtin_fmaf(dxs, dxs, dys * dys);
                const bool use3d = rho3d <= rho2d;
                const float G = __builtin_amdgcn_exp2f(__builtin_fminf(rho3d, rho2d) * -0.72134752044448170368f);
                const float alpha = has ? __builtin_fminf(0.99f, opa * G) : 0.f;
                const float inv_om = __builtin_amdgcn_rcpf(1.0f - alpha);
                Tr *= inv_om;  // transmittance before this splat (unchanged where it did not blend)
                const float aT = alpha * Tr;
                // lanes that did not blend get a finite stand-in (their terms are zeroed)
                const float depth = has ? __builtin_fmaf(u, Twx, __builtin_fmaf(v, Twy, Twz)) : 1.0f;
                const float cu[3] = {q5.y, q5.z, q5.w}, nrm[3] = {q6.x, q6.y, q6.z};
                const float dpix[3] = {dp0, dp1, dp2}, dn[3] = {dn0, dn1, dn2};
                float dL_dalpha = 0.0f;
#pragma unroll
                for (int q = 0; q < 3; ++q) {
                    const float an = last_alpha * last_c[q] + (1.f - last_alpha) * acc_c[q];
                    acc_c[q] = has ? an : acc_c[q];
                    last_c[q] = has ? cu[q] : last_c[q];
                    dL_dalpha += (cu[q] - acc_c[q]) * dpix[q];
                    v16[13 + q] = cu[q] > 0.0f ? aT * dpix[q] : 0.f;
                }
                const float inv_d = __builtin_amdgcn_rcpf(depth);
                const float m_d = kMScale * (1.0f - NEAR_N * inv_d);
                const float dmd_dd = (FAR_N * NEAR_N) / (FAR_N - NEAR_N) * inv_d * inv_d;
                float dL_dz = (has && (int)e.z == med_pos) ? dmed : 0.f;
                const float dL_dweight = (fD2 + m_d * m_d * fA - 2.0f * m_d * fD) * dreg;
                dL_dalpha += dL_dweight - last_dLdT;
                const float ldt = dL_dweight * alpha + (1.0f - alpha) * last_dLdT;
                last_dLdT = has ? ldt : last_dLdT;
                dL_dz += 2.0f * aT * (m_d * fA - fD) * dreg * dmd_dd;
                const float ad = last_alpha * last_d + (1.f - last_alpha) * acc_d;
                acc_d = has ? ad : acc_d;
                last_d = has ? depth : last_d;
                dL_dalpha += (depth - acc_d) * ddep;
                const float aa = last_alpha + (1.f - last_alpha) * acc_a;
                acc_a = has ? aa : acc_a;
                dL_dalpha += (1.0f - acc_a) * dacc;
#pragma unroll
                for (int q = 0; q < 3; ++q) {
                    const float an = last_alpha * last_n[q] + (1.f - last_alpha) * acc_n[q];
                    acc_n[q] = has ? an : acc_n[q];
                    last_n[q] = has ? nrm[q] : last_n[q];
                    dL_dalpha += (nrm[q] - acc_n[q]) * dn[q];
                    v16[9 + q] = aT * dn[q];
                }
                dL_dz += aT * ddep;
                dL_dalpha = __builtin_fmaf(dL_dalpha, Tr, bgT * inv_om);
                last_alpha = has ? alpha : last_alpha;
                dL_dz = has ? dL_dz : 0.f;
                const float dL_dG = has ? opa * dL_dalpha : 0.f;
                // the T rows get gradient only on the 3D branch (selects, not
                // products with zero: u and 1 / ray.z may be huge there)
                const float dsx_pz = use3d ? (-dL_dG * G * u + dL_dz * Twx) * inv_z : 0.f;
                const float dsy_pz = use3d ? (-dL_dG * G * v + dL_dz * Twy) * inv_z : 0.f;
                const float dpz = use3d ? -(dsx_pz * u + dsy_pz * v) : 0.f;
                const f3 dk = {l.y * dpz - l.z * dsy_pz, l.z * dsx_pz - l.x * dpz, l.x * dsy_pz - l.y * dsx_pz};
                const f3 dl = {dsy_pz * k.z - dpz * k.y, dpz * k.x - dsx_pz * k.z, dsx_pz * k.y - dsy_pz * k.x};
                v16[0] = -dk.x;
                v16[1] = -dk.y;
                v16[2] = -dk.z;
                v16[3] = -dl.x;
                v16[4] = -dl.y;
                v16[5] = -dl.z;
                v16[6] = px * dk.x + py * dl.x + dL_dz * u;
                v16[7] = px * dk.y + py * dl.y + dL_dz * v;
                v16[8] = px * dk.z + py * dl.z + dL_dz;
                v16[12] = G * dL_dG * (1.0f - opa);
            }
            const float s = FULL ? wave_reduce16(v16, lane) : wave_reduce16_lds8<kImgRaw>(v16, red8);
            if (adds && s != 0.f) unsafeAtomicAdd(&grads16[(size_t)e.w * 16 + gi], s);
        }
        wave_lds_sync();
    }
}

// ms_rcp_nr against the correctly rounded division for every float of
// exponent field efield (both signs, all 2^23 mantissas); bad counts the
// differences.  One thread per float, 2^24 threads.
__global__ __launch_bounds__(256) void k_check_rcp(uint32_t efield, unsigned long long *__restrict__ bad) {
    const uint32_t i = blockIdx.x * 256u + threadIdx.x;
    const float x = __uint_as_float(((i >> 23) << 31) | (efield << 23) | (i & 0x7fffffu));
    const bool differ = __float_as_uint(ms_rcp_nr(x)) != __float_as_uint(1.0f / x);
    const unsigned long long n = __builtin_popcountll(__builtin_amdgcn_ballot_w64(differ));
    if ((threadIdx.x & 63) == 0 && n) atomicAdd(bad, n);
}


// ---- deep tiles -----------------------------------------------------------
//
// A tile whose list holds thousands of entries (the overflow workload's
// tiles over a dense cluster) is one workgroup's serial walk in
// k_raster_fwd: each of its four waves visits most of the list, and a lone
// wave issues a ~57-instruction visit only every few cycles, so such tiles
// finish long after the rest of the image.  The deep-tile path walks each
// pixel's list independently instead: a wave takes a 2x2 pixel block and 64
// consecutive list entries at a time, one per lane; every lane evaluates
// its entry against each pixel (eval_pair, the same arithmetic on the same
// centred rows), and the entries that pass are blended in list order by a
// scalar loop over the ballot, with the reference's front-to-back
// recurrences.  Each pixel sees the same splats in the same order with the
// same operations as in k_raster_fwd, so every output is bit-identical; a
// deep tile's 256 pixels run on 64 waves instead of 4, on a stream of their
// own beside the per-tile kernel.
//
// For the backward, the training forward also records each pixel's blended
// entries (list position and the transmittance before the blend), and
// k_deep_log turns a quadrant's 64 pixel lists into the wave blend log and
// transmittance checkpoints k_raster_fwd would have written.

// The most splats one pixel can blend: every blend multiplies T by at most
// 1 - 1/255, and blending stops before T reaches 1e-4, so at most
// ln(1e-4) / ln(254/255) = 2344.0 blends (fp32 rounding adds at most one).
constexpr int kDeepMaxBlend = 2368;
// Pixels per wave: a 2x2 block shares each step's record loads and centred
// rows (measured faster than one pixel per wave, whose 4x as many waves
// crowd the SIMDs that run the deepest walks).
constexpr int kDeepPix = 4;
constexpr int kDeepWaves = 256 / kDeepPix;  // waves per deep tile

__device__ __forceinline__ float readlane_f(float v, int l) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), l));
}

// deep_list[0, count) = the tiles whose list holds at least deep_len entries.
__global__ __launch_bounds__(256) void k_deep_tiles(int T, const int *__restrict__ offsets, int deep_len,
                                                    int *__restrict__ deep_list, int *__restrict__ count) {
    const int t = blockIdx.x * 256 + threadIdx.x;
    const bool deep = t < T && offsets[t + 1] - offsets[t] >= deep_len;
    const unsigned long long bal = __ballot(deep);
    if (!bal) return;
    const int lane = threadIdx.x & 63;
    int base = 0;
    if (lane == 0) base = atomicAdd(count, __popcll(bal));
    base = __shfl(base, 0, 64);
    if (deep) deep_list[base + __popcll(bal & ((1ull << lane) - 1ull))] = t;
}

// One wave per (deep tile k, pixel block g of kDeepPix pixels).  With
// LOG, pixel slot k * 256 + 16 y + x (tile-local x, y) receives its blended
// list positions and transmittances before the blend at
// dpos / dtb[slot * kDeepMaxBlend + i] and their count in dcnt[slot].
template <bool LOG, bool FULL_OUT>
__global__ __launch_bounds__(kThreads) void k_raster_deep(
    int W, int H, int tiles_x, int n_deep, const int *__restrict__ deep_list, const int *__restrict__ offsets,
    const int *__restrict__ ids, const float4 *__restrict__ rec, const float *__restrict__ bgp,
    float *__restrict__ out_img, float *__restrict__ final_Ts, int *__restrict__ final_idx,
    float *__restrict__ out_depth, float *__restrict__ out_normal, float *__restrict__ out_alpha,
    float *__restrict__ out_median, float *__restrict__ out_dist, int *__restrict__ dpos, float *__restrict__ dtb,
    int *__restrict__ dcnt) {
    const int lane = threadIdx.x & 63;
    const int item = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    if (item >= n_deep * kDeepWaves) return;
    const int k = item / kDeepWaves, g = item % kDeepWaves;
    const int tile = deep_list[k];
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int start = offsets[tile], end = offsets[tile + 1];
    float px[kDeepPix], py[kDeepPix], Tr[kDeepPix], cr[kDeepPix], cg[kDeepPix], cb[kDeepPix];
    float dep[kDeepPix], nx[kDeepPix], ny[kDeepPix], nz[kDeepPix], M1[kDeepPix], M2[kDeepPix], dist[kDeepPix],
        med[kDeepPix];
    int med_c[kDeepPix], last_c[kDeepPix], nb[kDeepPix], lp[kDeepPix];
    float lt[kDeepPix];
    unsigned done = 0;
    // pixel q of block g (a 2x2 block for 4 pixels per wave)
    const auto local_px = [&](int q) { return kDeepPix == 1 ? (g & 15) : 2 * (g & 7) + (q & 1); };
    const auto local_py = [&](int q) { return kDeepPix == 1 ? (g >> 4) : 2 * (g >> 3) + (q >> 1); };
#pragma unroll
    for (int q = 0; q < kDeepPix; ++q) {
        const int lx = local_px(q), ly = local_py(q);
        const int pxi = tx * 16 + lx, pyi = ty * 16 + ly;
        if (!(pxi < W && pyi < H)) done |= 1u << q;
        px[q] = (float)pxi;
        py[q] = (float)pyi;
        Tr[q] = 1.f;
        cr[q] = cg[q] = cb[q] = 0.f;
        dep[q] = nx[q] = ny[q] = nz[q] = M1[q] = M2[q] = dist[q] = med[q] = 0.f;
        med_c[q] = -1;
        last_c[q] = 0;
        nb[q] = 0;
        lp[q] = 0;
        lt[q] = 0.f;
    }
    const size_t slot0 = (size_t)k * 256;
    auto slot_of = [&](int q) { return slot0 + (size_t)(16 * local_py(q) + local_px(q)); };
    // each step's ids are loaded two steps ahead and its records one step
    // ahead, so the loads overlap the evaluation of the current step
    int gid_n = start + 64 + lane < end ? ids[start + 64 + lane] : 0;
    float4 n0, n1, n2, n3, n4;
    {
        const float4 *r = rec + 5 * (size_t)(start + lane < end ? ids[start + lane] : 0);
        n0 = r[0], n1 = r[1], n2 = r[2], n3 = r[3], n4 = r[4];
    }
    for (int j0 = start; j0 < end && done != (1u << kDeepPix) - 1u; j0 += 64) {
        const int j = j0 + lane;
        const bool valid = j < end;
        const uint64_t valid_m = __builtin_amdgcn_ballot_w64(valid);
        const float4 q0 = n0, q1 = n1, q2 = n2, q3 = n3, q4 = n4;
        if (j0 + 64 < end) {
            const float4 *r = rec + 5 * (size_t)gid_n;
            n0 = r[0], n1 = r[1], n2 = r[2], n3 = r[3], n4 = r[4];
            gid_n = j + 128 < end ? ids[j + 128] : 0;
        }
        const f3 Tw = {q1.z, q1.w, q2.x};
        f3 R0, nAx, nAy;
        centred_rows({q0.x, q0.y, q0.z}, {q0.w, q1.x, q1.y}, Tw, q2.y, q2.z, R0, nAx, nAy);
        // eval_pair's planes, as load_batch stages them
        const float4 p0 = make_float4(R0.x, R0.y, R0.z, nAx.x);
        const float4 p1 = make_float4(nAx.y, nAx.z, nAy.x, nAy.y);
        const float4 p2 = make_float4(nAy.z, q2.y, q2.z, q2.w);
        const float4 p3 = make_float4(Tw.x, Tw.y, Tw.z, 0.f);
#pragma unroll
        for (int q = 0; q < kDeepPix; ++q) {
            if ((done >> q) & 1u) continue;
            PairEval e;
            uint64_t act = eval_pair(px[q], py[q], p0, p1, p2, p3, e) & valid_m;
            while (act) {
                const int l = __builtin_ctzll(act);
                act &= act - 1ull;
                const float a = readlane_f(e.alpha, l);
                const float next_T = Tr[q] * (1.0f - a);
                if (__builtin_amdgcn_ballot_w64(next_T <= 1e-4f)) {
                    done |= 1u << q;
                    break;
                }
                const float w = a * Tr[q];
                const int pos = j0 - start + l;
                if (FULL_OUT) {
                    const int contrib = pos + 1;
                    const float A = 1.f - Tr[q];
                    const float dep_s = readlane_f(e.depth, l);
                    const float m_ = kMScale * (1.f - NEAR_N / dep_s);
                    dist[q] = __builtin_fmaf(m_ * m_ * A + M2[q] - 2.f * m_ * M1[q], w, dist[q]);
                    M1[q] = __builtin_fmaf(m_, w, M1[q]);
                    M2[q] = __builtin_fmaf(m_ * m_, w, M2[q]);
                    if (Tr[q] > 0.5f) {
                        med[q] = dep_s;
                        med_c[q] = contrib;
                    }
                    dep[q] = __builtin_fmaf(dep_s, w, dep[q]);
                    nx[q] = __builtin_fmaf(readlane_f(q3.x, l), w, nx[q]);
                    ny[q] = __builtin_fmaf(readlane_f(q3.y, l), w, ny[q]);
                    nz[q] = __builtin_fmaf(readlane_f(q3.z, l), w, nz[q]);
                    last_c[q] = contrib;
                }
                cr[q] = __builtin_fmaf(readlane_f(q3.w, l), w, cr[q]);
                cg[q] = __builtin_fmaf(readlane_f(q4.x, l), w, cg[q]);
                cb[q] = __builtin_fmaf(readlane_f(q4.y, l), w, cb[q]);
                if (LOG && nb[q] < kDeepMaxBlend) {
                    // entry nb goes to lane nb mod 64; a full chunk is one store
                    const bool mine = lane == (nb[q] & 63);
                    lp[q] = mine ? pos : lp[q];
                    lt[q] = mine ? Tr[q] : lt[q];
                    if ((++nb[q] & 63) == 0) {
                        const size_t o = slot_of(q) * kDeepMaxBlend + (size_t)(nb[q] - 64) + lane;
                        dpos[o] = lp[q];
                        dtb[o] = lt[q];
                    }
                }
                Tr[q] = next_T;
            }
        }
    }
    const float bg0 = bgp[0], bg1 = bgp[1], bg2 = bgp[2];
#pragma unroll
    for (int q = 0; q < kDeepPix; ++q) {
        const int lx = local_px(q), ly = local_py(q);
        const int pxi = tx * 16 + lx, pyi = ty * 16 + ly;
        if (LOG) {
            const size_t o = slot_of(q) * kDeepMaxBlend + (size_t)(nb[q] & ~63) + lane;
            if (lane < (nb[q] & 63)) {
                dpos[o] = lp[q];
                dtb[o] = lt[q];
            }
            if (lane == 0) dcnt[slot_of(q)] = pxi < W && pyi < H ? nb[q] : 0;
        }
        if (lane != 0 || !(pxi < W && pyi < H)) continue;
        const size_t pix = (size_t)pyi * W + pxi;
        final_Ts[3 * pix + 0] = Tr[q];
        out_img[3 * pix + 0] = __builtin_fmaf(bg0, Tr[q], cr[q]);
        out_img[3 * pix + 1] = __builtin_fmaf(bg1, Tr[q], cg[q]);
        out_img[3 * pix + 2] = __builtin_fmaf(bg2, Tr[q], cb[q]);
        if (!FULL_OUT) continue;
        final_idx[2 * pix + 0] = last_c[q];
        final_Ts[3 * pix + 1] = M1[q];
        final_Ts[3 * pix + 2] = M2[q];
        final_idx[2 * pix + 1] = med_c[q];
        out_depth[pix] = dep[q];
        out_normal[3 * pix + 0] = nx[q];
        out_normal[3 * pix + 1] = ny[q];
        out_normal[3 * pix + 2] = nz[q];
        out_alpha[pix] = 1.f - Tr[q];
        out_median[pix] = med[q];
        out_dist[pix] = dist[q];
    }
}

// The blend log of quadrant w of a deep tile from its 64 pixels' lists: the
// entries are the list positions some pixel of the quadrant blended, in
// list order, each with the ballot of those pixels (bit l = pixel
// (lane_px(w, l), lane_py(w, l)), as in k_raster_fwd), and checkpoint c
// (every 64th entry) holds each pixel's transmittance before entry c.  One
// 1024-thread workgroup per (deep tile, quadrant); every pass reads the
// pixel lists in coalesced 64-entry rows (wave v takes pixels v, v + 16, ...),
// in windows of kDeepWin list positions:
//   1. the positions present are marked in an LDS bitmap;
//   2. a block scan of the words' popcounts ranks them;
//   3. the ballots and positions are assembled in LDS for kDeepBal ranks at
//      a time (each pixel's entries of a rank range are a run of its list,
//      taken from a per-pixel cursor) and each entry is written once;
//   4. pixel entry i of rank r_i writes the checkpoints c in (r_{i-1}, r_i]
//      (the transmittance changes only at the pixel's own blends), and
//      after the pixel's last entry the final transmittance fills the rest.
constexpr int kDeepWin = 131072, kDeepWords = kDeepWin / 32, kDeepBal = 2048;
// Log chunks whose pool index the workgroup keeps in LDS (the checkpoint
// pass looks one up per checkpoint and pixel); longer logs read the rest of
// the chunk table from global memory.
constexpr int kDeepTbl = 4096;
constexpr int kLogThreads = 1024, kLogWaves = kLogThreads / 64;
__global__ __launch_bounds__(kLogThreads) void k_deep_log(int W, int H, int tiles_x, int n_deep,
                                                  const int *__restrict__ deep_list, const int *__restrict__ offsets,
                                                  const int *__restrict__ ids, const int *__restrict__ dpos,
                                                  const float *__restrict__ dtb, const int *__restrict__ dcnt,
                                                  const float *__restrict__ final_Ts, BlendLog blog) {
    __shared__ uint32_t s_bits[kDeepWords];
    __shared__ int s_woff[kDeepWords];
    __shared__ uint32_t s_bal[2][kDeepBal];
    __shared__ int s_pos[kDeepBal];
    __shared__ int s_chunk[kDeepTbl];
    __shared__ int s_cnt[64], s_i[64], s_e[64], s_last[64], s_cur[64];
    __shared__ float s_tf[64];
    __shared__ int s_red[kLogWaves];
    __shared__ int s_ok;
    const int item = blockIdx.x;
    if (item >= n_deep * 4) return;
    const int lane = threadIdx.x & 63, wv = threadIdx.x >> 6;
    const int k = item >> 2, w = item & 3;
    const int tile = deep_list[k];
    const int tx = tile % tiles_x, ty = tile / tiles_x;
    const int start = offsets[tile], len = offsets[tile + 1] - start;
    int *__restrict__ chunk_of = blog.table + log_table_base(start, len, tile, w);
    // entry r of the log, and checkpoint c (the chunk of entry c - 1 holds it)
    auto pool_chunk = [&](int q) { return q < kDeepTbl ? s_chunk[q] : chunk_of[q]; };
    auto ent_at = [&](int r) { return blog.ent + 64 * (size_t)pool_chunk(r >> 6) + (r & 63); };
    auto ckpt_at = [&](int c, int p) { return blog.ckpt + 64 * (size_t)pool_chunk((c >> 6) - 1) + p; };
    auto slot_of = [&](int p) { return (size_t)k * 256 + 16 * lane_py(w, p) + lane_px(w, p); };
    if (threadIdx.x < 64) {
        const int p = threadIdx.x;
        const int pxi = tx * 16 + lane_px(w, p), pyi = ty * 16 + lane_py(w, p);
        const bool inside = pxi < W && pyi < H;
        s_cnt[p] = inside ? dcnt[slot_of(p)] : 0;
        s_tf[p] = inside ? final_Ts[3 * ((size_t)pyi * W + pxi)] : 1.0f;
        s_i[p] = 0;
        s_last[p] = -1;
    }
    __syncthreads();
    int nlog = 0;
    for (int P0 = 0;; P0 += kDeepWin) {
        // any pixel entries left?
        int left = 0;
        if (threadIdx.x < 64) left = s_i[threadIdx.x] < s_cnt[threadIdx.x];
        if (!__syncthreads_or(left)) break;
        for (int q = threadIdx.x; q < kDeepWords; q += kLogThreads) s_bits[q] = 0u;
        __syncthreads();
        // 1. mark, and find each pixel's first entry beyond the window
        for (int p = wv; p < 64; p += kLogWaves) {
            const int *__restrict__ P_ = dpos + slot_of(p) * kDeepMaxBlend;
            const int i0 = s_i[p], n = s_cnt[p];
            int e = n;
            for (int i = i0; i < n; i += 64) {
                const int pos = i + lane < n ? P_[i + lane] : INT32_MAX;
                const bool in = pos < P0 + kDeepWin;
                if (in) {
                    const int b = pos - P0;
                    atomicOr(&s_bits[b >> 5], 1u << (b & 31));
                }
                const unsigned long long out = __ballot(!in);
                if (out) {
                    e = i + (int)__builtin_ctzll(out);
                    break;
                }
            }
            if (lane == 0) s_e[p] = e;
        }
        __syncthreads();
        // 2. ranks: block scan of the words' popcounts (4 words per thread)
        constexpr int WPT = kDeepWords / kLogThreads;
        int wsum = 0;
#pragma unroll
        for (int q = 0; q < WPT; ++q) wsum += __popc(s_bits[threadIdx.x * WPT + q]);
        int incl = wsum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
        }
        if (lane == 63) s_red[wv] = incl;
        __syncthreads();
        int woff = incl - wsum, n_w = 0;
        for (int v = 0; v < kLogWaves; ++v) {
            woff += v < wv ? s_red[v] : 0;
            n_w += s_red[v];
        }
        // pool chunks for the window's entries nlog .. nlog + n_w - 1
        if (threadIdx.x == 0) {
            const int have = (nlog + 63) >> 6, need = (nlog + n_w + 63) >> 6;
            int ok = 1;
            if (need > have) {
                const int sp = log_subpool(blog, tile, w), n = need - have;
                const int base = log_resolve(blog, sp, atomicAdd(&blog.counters[sp], n), n);
                ok = base >= 0;
                if (ok)
                    for (int q = have; q < need; ++q) {
                        chunk_of[q] = base + (q - have);
                        if (q < kDeepTbl) s_chunk[q] = base + (q - have);
                    }
            }
            s_ok = ok;
        }
        __syncthreads();
        if (!s_ok) return;  // pool exhausted: the log is incomplete (overflowed)
#pragma unroll
        for (int q = 0; q < WPT; ++q) {
            const int wd = threadIdx.x * WPT + q;
            s_woff[wd] = woff;
            woff += __popc(s_bits[wd]);
        }
        __syncthreads();
        auto rank = [&](int pos) {
            const int b = pos - P0;
            return s_woff[b >> 5] + __popc(s_bits[b >> 5] & ((1u << (b & 31)) - 1u));
        };
        // 3. ballots, kDeepBal ranks at a time.  A pixel's entries are in
        // list order and ranks grow with the position, so the entries of one
        // rank range are a run of its list: each pixel keeps a cursor, and
        // every entry is visited once over all the ranges
        if (threadIdx.x < 64) s_cur[threadIdx.x] = s_i[threadIdx.x];
        for (int R0 = 0; R0 < n_w; R0 += kDeepBal) {
            for (int r = threadIdx.x; r < kDeepBal; r += kLogThreads) {
                s_bal[0][r] = 0u;
                s_bal[1][r] = 0u;
            }
            __syncthreads();
            for (int p = wv; p < 64; p += kLogWaves) {
                const int *__restrict__ P_ = dpos + slot_of(p) * kDeepMaxBlend;
                const int e = s_e[p];
                int i0 = s_cur[p];
                for (; i0 < e; i0 += 64) {
                    const int i = i0 + lane;
                    const int pos = i < e ? P_[i] : 0;
                    const int r = i < e ? rank(pos) - R0 : INT32_MAX;
                    const bool in = r < kDeepBal;
                    if (in) {
                        atomicOr(&s_bal[p >> 5][r], 1u << (p & 31));
                        s_pos[r] = pos;  // every pixel that blended rank r writes the same position
                    }
                    const unsigned long long past = __ballot(!in);
                    if (past) {
                        i0 += (int)__builtin_ctzll(past);  // the first entry of a later range
                        break;
                    }
                }
                if (lane == 0) s_cur[p] = min(i0, e);
            }
            __syncthreads();
            // the range's entries {ballot, list position, gaussian id}, one
            // 16-byte store each (consecutive ranks: consecutive slots)
            for (int r = threadIdx.x; r < min(kDeepBal, n_w - R0); r += kLogThreads) {
                const int pos = s_pos[r];
                *ent_at(nlog + R0 + r) = make_uint4(s_bal[0][r], s_bal[1][r], (unsigned)pos, (unsigned)ids[start + pos]);
            }
            __syncthreads();
        }
        // 4. checkpoints up to each pixel entry
        for (int p = wv; p < 64; p += kLogWaves) {
            const int *__restrict__ P_ = dpos + slot_of(p) * kDeepMaxBlend;
            const float *__restrict__ Tb = dtb + slot_of(p) * kDeepMaxBlend;
            const int e = s_e[p];
            int carry = s_last[p];
            for (int i0 = s_i[p]; i0 < e; i0 += 64) {
                const int i = i0 + lane;
                const int r = i < e ? nlog + rank(P_[i]) : INT32_MAX;
                int rp = __shfl_up(r, 1, 64);
                if (lane == 0) rp = carry;
                if (i < e) {
                    const float tb = Tb[i];
                    for (int c = max(64, (rp + 64) & ~63); c <= r; c += 64) *ckpt_at(c, p) = tb;
                }
                carry = __shfl(r, min(63, e - 1 - i0), 64);
            }
            if (lane == 0) {
                s_last[p] = carry;
                s_i[p] = e;
            }
        }
        nlog += n_w;
        __syncthreads();
    }
    // the final transmittance for the checkpoints after each pixel's last entry
    for (int p = wv; p < 64; p += kLogWaves) {
        const float tf = s_tf[p];
        for (int c = max(64, (s_last[p] + 64) & ~63) + 64 * lane; c <= nlog; c += 64 * 64) *ckpt_at(c, p) = tf;
    }
    if (threadIdx.x == 0) blog.wave_cnt[4 * tile + w] = nlog;
}

}  // namespace

namespace mskern {

void launch_check_rcp(hipStream_t s, int efield, unsigned long long *bad) {
    hipLaunchKernelGGL(k_check_rcp, dim3((1u << 24) / 256), dim3(256), 0, s, (uint32_t)efield, bad);
}

void launch_raster_fwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets, const int *ids,
                       const float *rec, const float *mrec, const float *bg, float *out_img, float *final_Ts, int *final_idx,
                       float *out_depth, float *out_normal, float *out_alpha, float *out_median, float *out_dist,
                       unsigned long long *pair_counter, const BlendLog *blog, bool full_outputs,
                       const DeepTiles &deep) {
    const int T = tiles_x * tiles_y;
    const int grid = xcd_strip_grid(tiles_x, tiles_y);
    const BlendLog lg = blog ? *blog : BlendLog{};
    const int deep_len = deep.n > 0 ? deep.len : INT32_MAX;
    if (deep.n > 0) {
        // the deep tiles on their own stream, beside the per-tile kernel
        // (their walks are the longest; the outputs are disjoint)
        (void)hipEventRecord(deep.fork, s);
        (void)hipStreamWaitEvent(deep.stream, deep.fork, 0);
        hipStream_t sd = deep.stream;
        auto launch_deep = [&](auto kern) {
            hipLaunchKernelGGL(kern, dim3(deep.n * kDeepWaves / 4), dim3(kThreads), 0, sd, W, H, tiles_x, deep.n, deep.list,
                               offsets, ids, reinterpret_cast<const float4 *>(rec), bg, out_img, final_Ts, final_idx,
                               out_depth, out_normal, out_alpha, out_median, out_dist, deep.pos, deep.tb, deep.cnt);
        };
        if (blog)
            full_outputs ? launch_deep(k_raster_deep<true, true>) : launch_deep(k_raster_deep<true, false>);
        else
            full_outputs ? launch_deep(k_raster_deep<false, true>) : launch_deep(k_raster_deep<false, false>);
        const bool defer = blog && deep.defer_log;
        if (defer) (void)hipEventRecord(deep.join, sd);
        if (blog) {
            hipLaunchKernelGGL(k_deep_log, dim3(deep.n * 4), dim3(kLogThreads), 0, sd, W, H, tiles_x, deep.n, deep.list,
                               offsets, ids, deep.pos, deep.tb, deep.cnt, final_Ts, lg);
            (void)hipEventRecord(deep.logged, sd);
        }
        if (!defer) (void)hipEventRecord(deep.join, sd);
    }
    auto launch = [&](auto kern) {
        hipLaunchKernelGGL(kern, dim3(grid), dim3(kThreads), 0, s, W, H, tiles_x, T, offsets, ids,
                           reinterpret_cast<const float4 *>(rec), reinterpret_cast<const float4 *>(mrec), bg,
                           out_img, final_Ts, final_idx, out_depth,
                           out_normal, out_alpha, out_median, out_dist, pair_counter, lg, deep_len);
    };
    // the work counters are a separate instantiation (profiling only)
    if (pair_counter) {
        if (blog)
            full_outputs ? launch(k_raster_fwd<true, true, true>) : launch(k_raster_fwd<true, false, true>);
        else
            full_outputs ? launch(k_raster_fwd<false, true, true>) : launch(k_raster_fwd<false, false, true>);
    } else {
        if (blog)
            full_outputs ? launch(k_raster_fwd<true, true, false>) : launch(k_raster_fwd<true, false, false>);
        else
            full_outputs ? launch(k_raster_fwd<false, true, false>) : launch(k_raster_fwd<false, false, false>);
    }
    if (deep.n > 0) (void)hipStreamWaitEvent(s, deep.join, 0);
}

void launch_deep_tiles(hipStream_t s, int T, const int *offsets, int deep_len, int *deep_list, int *count) {
    hipLaunchKernelGGL(k_deep_tiles, dim3((T + 255) / 256), dim3(256), 0, s, T, offsets, deep_len, deep_list, count);
}

int64_t deep_pixel_entries(int n_deep) { return (int64_t)n_deep * 256 * kDeepMaxBlend; }

bool launch_raster_bwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets,
                       const BlendLog &blog, const float *rec,
                       const float *bg, const float *final_Ts, const int *final_idx, const float *dL_dimg,
                       const float *dL_ddepth, const float *dL_daccum, const float *dL_dnormal,
                       const float *dL_dmedian, const float *dL_ddist, float ddist_uniform, float *grads16,
                       const DeepTiles &deep) {
    const int T = tiles_x * tiles_y;
    const int grid = xcd_strip_grid(tiles_x, tiles_y);
    const bool full = dL_ddepth || dL_daccum || dL_dnormal || dL_dmedian || dL_ddist || ddist_uniform != 0.0f;
    auto launch = [&](hipStream_t st, int blocks, const int *list, int deep_len) {
        if (full)
            hipLaunchKernelGGL(k_raster_bwd<true>, dim3(blocks), dim3(kThreads), 0, st, W, H, tiles_x, T, offsets, blog,
                               reinterpret_cast<const float4 *>(rec), bg, final_Ts, final_idx,
                               dL_dimg, dL_ddepth, dL_daccum, dL_dnormal, dL_dmedian, dL_ddist, ddist_uniform,
                               grads16, list, deep_len);
        else
            hipLaunchKernelGGL(k_raster_bwd<false>, dim3(blocks), dim3(kThreads), 0, st, W, H, tiles_x, T, offsets,
                               blog, reinterpret_cast<const float4 *>(rec), bg, final_Ts, final_idx,
                               dL_dimg, dL_ddepth, dL_daccum, dL_dnormal, dL_dmedian, dL_ddist, ddist_uniform,
                               grads16, list, deep_len);
    };
    if (deep.n > 0) {
        // the deep tiles' long log replays start at once, on their own
        // stream, beside the rest (after the deep tiles' log rebuild, if
        // the forward left it running there: the per-tile launch waits for
        // the rebuild too, so that both launches start together)
        (void)hipStreamWaitEvent(s, deep.logged, 0);
        (void)hipEventRecord(deep.fork, s);
        (void)hipStreamWaitEvent(deep.stream, deep.fork, 0);
        launch(deep.stream, deep.n, deep.list, 0);
        (void)hipEventRecord(deep.join, deep.stream);
        launch(s, grid, nullptr, deep.len);
        (void)hipStreamWaitEvent(s, deep.join, 0);
    } else {
        launch(s, grid, nullptr, INT32_MAX);
    }
    return !full;
}

}  // namespace mskern
