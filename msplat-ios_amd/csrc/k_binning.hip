// k_binning.hip -- tile binning and per-tile depth order, in two levels.
//
// Replaces scatter_to_prealloc_bins_kernel + prefix_sum_kernel +
// bitonic_sort_per_tile_2dgs_kernel (msplat_metal.metal:1557-1690, 3093-3145),
// which preallocate 2048 slots per tile, drop the overflow and sort every
// tile list separately.  Here every intersection is kept and the per-tile
// order is (depth bits, gaussian id), as the reference's keys define it.
//
// Device-scope atomics run at about 28 G/s on this part whether or not they
// collide, so no stage issues one per tile entry:
//   1. k_super_hist: one workgroup per chunk of several thousand splats
//      counts its (splat, 4x4-tile super-tile) pairs in an LDS histogram and
//      writes it as its row of a (workgroup x super-tile) count matrix;
//      k_super_cols turns each column into the workgroups' offsets inside
//      the super-tile and its total, and an exclusive scan of the totals
//      gives the super-tile offsets;
//   2. k_scatter_super: each workgroup places the keys of its chunk at its
//      offsets with LDS atomics -- about 2.5 keys per splat instead of one
//      per tile, with no global atomic and no second count pass;
//   3. k_sort_super: each super-tile counts the entries of its 16 tiles
//      (the tile histogram, no atomics: a super-tile owns its tiles) and
//      sorts its keys in LDS (bitonic, up to 4096 keys), larger lists in
//      4096-key runs merged by k_merge_path; an exclusive scan of the tile
//      counts gives the tile offsets (the layout of the id list the
//      rasterizers read);
//   4. k_emit_tiles: each super-tile's sorted list is filtered, in order,
//      into the id lists of its 16 tiles (wave ballots keep the order), so
//      every tile list comes out sorted without a per-tile sort.
#include "kernels.h"
#include "ms_device.h"

namespace {

constexpr int kSortThreads = 256;
constexpr int kChunk = 4096;  // keys per LDS sort (32 KB of u64)
// Lists longer than this are sorted, counted and emitted chunk-parallel
// (their chunk sorts would otherwise hold one workgroup for longer than the
// rest of the pass); shorter ones stay within their super-tile's workgroup.
constexpr int kHuge = 4 * kChunk;
constexpr int kSuper = 4;     // tiles per super-tile side
static_assert(kHuge == mskern::kSuperHugeList && kChunk == mskern::kSuperSortChunk && kSuper == mskern::kSuperTile,
              "the host sizes the binning buffers with these");

// The merge passes (k_merge_path) take a list of cnt > kChunk keys through
// merge_passes(cnt) passes (L = kChunk, 2 kChunk, ... below cnt), pass p
// reading the key buffer for even p and writing the second buffer, and the
// reverse; merged_keys names where the list ends.
__host__ __device__ __forceinline__ int merge_passes(int cnt) {
    int p = 0;
    for (int64_t L = kChunk; L < cnt; L <<= 1) ++p;
    return p;
}
__device__ __forceinline__ const unsigned long long *merged_keys(int cnt, const unsigned long long *keys,
                                                                  const unsigned long long *keys2) {
    return (merge_passes(cnt) & 1) ? keys2 : keys;
}

// ---- counts -> offsets ------------------------------------------------------
//
// Exclusive scan of a count array (prefix_sum_kernel,
// msplat_metal.metal:3093-3145): local pass over 2048 counts per workgroup,
// block totals, add pass; up to 32768 counts one workgroup does all three
// (k_scan_small).  stats[0] receives the total, stats[1] the largest count
// (stats[1] must be zero on entry).

constexpr int kScanT = 256, kScanI = 8, kScanChunk = kScanT * kScanI;

// Inclusive scan of v over a 256-thread workgroup; *total receives the sum.
__device__ __forceinline__ int block_scan_incl(int v, int *s_w, int *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    __syncthreads();
    if (lane == 63) s_w[wave] = incl;
    __syncthreads();
    int off = 0, tot = 0;
#pragma unroll
    for (int w = 0; w < kScanT / 64; ++w) {
        off += w < wave ? s_w[w] : 0;
        tot += s_w[w];
    }
    *total = tot;
    return off + incl;
}

__global__ __launch_bounds__(kScanT) void k_off_local(int T, const int *__restrict__ counts,
                                                      int *__restrict__ offsets, int *__restrict__ totals,
                                                      int *__restrict__ stats) {
    __shared__ int s_w[kScanT / 64];
    const int base = blockIdx.x * kScanChunk + threadIdx.x * kScanI;
    int v[kScanI], sum = 0, mx = 0;
#pragma unroll
    for (int k = 0; k < kScanI; ++k) {
        v[k] = base + k < T ? counts[base + k] : 0;
        sum += v[k];
        mx = max(mx, v[k]);
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) mx = max(mx, __shfl_xor(mx, d, 64));
    if ((threadIdx.x & 63) == 0 && mx > 0) atomicMax(&stats[1], mx);
    int total;
    int run = block_scan_incl(sum, s_w, &total) - sum;
#pragma unroll
    for (int k = 0; k < kScanI; ++k) {
        if (base + k < T) offsets[base + k] = run;
        run += v[k];
    }
    if (threadIdx.x == 0) totals[blockIdx.x] = total;
}

__global__ __launch_bounds__(1024) void k_off_totals(int nb, int *__restrict__ totals, int *__restrict__ stats) {
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
    int off = 0, all = 0;
    for (int w = 0; w < 16; ++w) {
        off += w < wave ? s_w[w] : 0;
        all += s_w[w];
    }
    int run = off + incl - sum;
    for (int i = b; i < e; ++i) {
        const int t = totals[i];
        totals[i] = run;
        run += t;
    }
    if (threadIdx.x == 0) stats[0] = all;
}

__global__ __launch_bounds__(kScanT) void k_off_add(int T, int *__restrict__ offsets, int *__restrict__ cursor,
                                                    const int *__restrict__ totals, const int *__restrict__ stats) {
    const int base = blockIdx.x * kScanChunk + threadIdx.x * kScanI;
    const int o = totals[blockIdx.x];
#pragma unroll
    for (int k = 0; k < kScanI; ++k)
        if (base + k < T) {
            const int v = offsets[base + k] + o;
            offsets[base + k] = v;
            if (cursor) cursor[base + k] = v;
        }
    if (blockIdx.x == 0 && threadIdx.x == 0) offsets[T] = stats[0];
}

// The same scan in one workgroup of 1024 threads, for counts[] short enough
// that launching three kernels costs more than walking them: 8192 counts
// per round (8 consecutive per thread), the rounds chained by a carry.
constexpr int kScanSmallT = 1024, kScanSmallChunk = kScanSmallT * kScanI;
constexpr int kScanSmallMax = 4 * kScanSmallChunk;  // at most 4 rounds

__global__ __launch_bounds__(kScanSmallT) void k_scan_small(int T, const int *__restrict__ counts,
                                                            int *__restrict__ offsets, int *__restrict__ cursor,
                                                            int *__restrict__ stats) {
    __shared__ int s_w[kScanSmallT / 64];
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    int carry = 0, mx = 0;
    for (int base = 0; base < T; base += kScanSmallChunk) {
        const int i0 = base + (int)threadIdx.x * kScanI;
        int v[kScanI], sum = 0;
#pragma unroll
        for (int k = 0; k < kScanI; ++k) {
            v[k] = i0 + k < T ? counts[i0 + k] : 0;
            sum += v[k];
            mx = max(mx, v[k]);
        }
        int incl = sum;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
        }
        __syncthreads();  // the previous round's reads of s_w are done
        if (lane == 63) s_w[wave] = incl;
        __syncthreads();
        int off = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < kScanSmallT / 64; ++w) {
            off += w < wave ? s_w[w] : 0;
            tot += s_w[w];
        }
        int run = carry + off + incl - sum;
#pragma unroll
        for (int k = 0; k < kScanI; ++k)
            if (i0 + k < T) {
                offsets[i0 + k] = run;
                if (cursor) cursor[i0 + k] = run;
                run += v[k];
            }
        carry += tot;
    }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) mx = max(mx, __shfl_xor(mx, d, 64));
    if (lane == 0 && mx > 0) atomicMax(&stats[1], mx);
    if (threadIdx.x == 0) {
        stats[0] = carry;
        offsets[T] = carry;
    }
}

// ---- super-tile histogram and scatter -------------------------------------
//
// Both kernels give workgroup b the splats [b * chunk, (b + 1) * chunk) and
// count their (splat, super-tile) pairs in an LDS histogram, in windows of
// kHistBins super-tiles.  The rectangles of a wave are enumerated
// cooperatively (wave_expand), so the 64 lanes issue independent LDS atomics
// instead of serial per-lane loops of different lengths.

constexpr int kBinThreads = 1024;
constexpr int kHistBins = 16384;  // super-tiles per LDS window (64 KB)

struct SuperRect {
    int sx0, sy0, sw, sh;  // super-tile rectangle, sw * sh pairs (0 if none)
    uint32_t t0, t1;       // the tile rectangle (x0 | y0 << 16, x1 | y1 << 16)
};

// Keys of the packed layout (fewer than 2^24 splats):
// depth bits << 32 | id << 8 | local rectangle, the splat's tile rectangle
// inside the (sx, sy) super-tile in 8 bits (x0, x1 - 1, y0, y1 - 1 in
// 0..3).  Ids are unique within a super-tile list, so the order is still
// (depth, id), and the sort and the emission read the rectangle from the
// key instead of gathering rect[id].  The wide layout (depth bits << 32 |
// id) gathers it.
constexpr int kPackedMaxSplats = 1 << 24;
__device__ __forceinline__ uint32_t local_rect(uint32_t t0, uint32_t t1, int sx, int sy) {
    const int stx = sx * kSuper, sty = sy * kSuper;
    const int rx0 = max((int)(t0 & 0xffff) - stx, 0), rx1 = min((int)(t1 & 0xffff) - stx, kSuper);
    const int ry0 = max((int)(t0 >> 16) - sty, 0), ry1 = min((int)(t1 >> 16) - sty, kSuper);
    return (uint32_t)(rx0 | ((rx1 - 1) << 2) | (ry0 << 4) | ((ry1 - 1) << 6));
}
// (x0, x1, y0, y1) of a local rectangle, half-open
__device__ __forceinline__ int4 unpack_rect(uint32_t lr) {
    return make_int4(lr & 3, ((lr >> 2) & 3) + 1, (lr >> 4) & 3, ((lr >> 6) & 3) + 1);
}

__device__ __forceinline__ SuperRect super_rect(int i, int n, const int *__restrict__ radii,
                                                const uint2 *__restrict__ rect) {
    SuperRect r{0, 0, 1, 0, 0u, 0u};
    if (i < n && radii[i] > 0) {
        const uint2 q = rect[i];
        r.t0 = q.x;
        r.t1 = q.y;
        const int x0 = q.x & 0xffff, y0 = q.x >> 16, x1 = q.y & 0xffff, y1 = q.y >> 16;
        if (x1 > x0 && y1 > y0) {
            r.sx0 = x0 / kSuper;
            r.sy0 = y0 / kSuper;
            r.sw = (x1 + kSuper - 1) / kSuper - r.sx0;
            r.sh = (y1 + kSuper - 1) / kSuper - r.sy0;
        }
    }
    return r;
}

// fn(bin, splat, local rectangle) for every (splat, super-tile) pair of
// this workgroup's chunk whose super-tile index lies in [w0, w0 + nbin)
// (the local rectangle only with LR).
template <bool LR = false, typename F>
__device__ __forceinline__ void for_pairs(int n, int chunk, int sxn, int w0, int nbin, const int *__restrict__ radii,
                                          const uint2 *__restrict__ rect, F &&fn) {
    const int c0 = blockIdx.x * chunk, c1 = min(n, c0 + chunk);
    for (int base = c0; base < c1; base += kBinThreads) {
        const int i = base + (int)threadIdx.x;
        const SuperRect r = super_rect(i < c1 ? i : n, n, radii, rect);
        msd::wave_expand(r.sw * r.sh, [&](int owner, int k, bool active) {
            const int ow = __shfl(r.sw, owner, 64), ox = __shfl(r.sx0, owner, 64), oy = __shfl(r.sy0, owner, 64);
            const int oi = __shfl(i, owner, 64);
            uint32_t t0 = 0u, t1 = 0u;
            if constexpr (LR) {
                t0 = __shfl(r.t0, owner, 64);
                t1 = __shfl(r.t1, owner, 64);
            }
            if (active) {
                const int ry = k / ow, rx = k - ry * ow;
                const int bin = (oy + ry) * sxn + ox + rx - w0;
                if (bin >= 0 && bin < nbin) fn(bin, oi, LR ? local_rect(t0, t1, ox + rx, oy + ry) : 0u);
            }
        });
    }
}

// Pair counts per (workgroup, super-tile): the LDS histogram of each window
// is written as the workgroup's row of the count matrix cm[blocks][NS].
__global__ __launch_bounds__(kBinThreads) void k_super_hist(int n, int chunk, int sxn, int NS,
                                                            const int *__restrict__ radii,
                                                            const uint2 *__restrict__ rect, int *__restrict__ cm) {
    __shared__ int s_h[kHistBins];
    int *row = cm + (size_t)blockIdx.x * NS;
    for (int w0 = 0; w0 < NS; w0 += kHistBins) {
        const int nbin = min(kHistBins, NS - w0);
        for (int k = threadIdx.x; k < nbin; k += kBinThreads) s_h[k] = 0;
        __syncthreads();
        for_pairs(n, chunk, sxn, w0, nbin, radii, rect, [&](int bin, int, uint32_t) { atomicAdd(&s_h[bin], 1); });
        __syncthreads();
        for (int k = threadIdx.x; k < nbin; k += kBinThreads) row[w0 + k] = s_h[k];
        __syncthreads();
    }
}

// Column pass over the count matrix: super_counts[s] = sum over workgroups
// of cm[g][s], and cm[g][s] becomes the exclusive prefix over g (the offset
// of workgroup g's keys inside super-tile s's list).  64 columns per
// workgroup, 16 waves each over a band of rows.
constexpr int kColW = 64, kColWaves = 16;
__global__ __launch_bounds__(kColW * kColWaves) void k_super_cols(int nb, int NS, int *__restrict__ cm,
                                                                  int *__restrict__ super_counts) {
    __shared__ int s_part[kColWaves][kColW];
    const int lane = threadIdx.x & (kColW - 1), w = threadIdx.x / kColW;
    const int s = blockIdx.x * kColW + lane;
    const int rows = (nb + kColWaves - 1) / kColWaves, r0 = w * rows, r1 = min(nb, r0 + rows);
    int sum = 0;
    if (s < NS)
        for (int r = r0; r < r1; ++r) sum += cm[(size_t)r * NS + s];
    s_part[w][lane] = sum;
    __syncthreads();
    int run = 0;
    for (int k = 0; k < w; ++k) run += s_part[k][lane];
    if (s >= NS) return;
    if (w == kColWaves - 1) super_counts[s] = run + sum;
    for (int r = r0; r < r1; ++r) {
        const int c = cm[(size_t)r * NS + s];
        cm[(size_t)r * NS + s] = run;
        run += c;
    }
}

// One key per (visible splat, super-tile) pair.  Workgroup g's keys of
// super-tile s go to super_offsets[s] + cm[g][s] onwards (the scanned count
// matrix), placed with LDS atomics; the order inside a super-tile list is
// arbitrary, k_sort_super orders it.
template <bool PACKED>
__global__ __launch_bounds__(kBinThreads) void k_scatter_super(int n, int chunk, int sxn, int NS,
                                                               const int *__restrict__ radii,
                                                               const uint2 *__restrict__ rect,
                                                               const float *__restrict__ depths,
                                                               const int *__restrict__ super_offsets,
                                                               const int *__restrict__ cm,
                                                               unsigned long long *__restrict__ keys) {
    __shared__ int s_h[kHistBins];
    const int *row = cm + (size_t)blockIdx.x * NS;
    for (int w0 = 0; w0 < NS; w0 += kHistBins) {
        const int nbin = min(kHistBins, NS - w0);
        for (int k = threadIdx.x; k < nbin; k += kBinThreads) s_h[k] = super_offsets[w0 + k] + row[w0 + k];
        __syncthreads();
        for_pairs<PACKED>(n, chunk, sxn, w0, nbin, radii, rect, [&](int bin, int gid, uint32_t lr) {
            const int pos = atomicAdd(&s_h[bin], 1);
            const uint32_t lo = PACKED ? ((uint32_t)gid << 8) | lr : (uint32_t)gid;
            keys[pos] = ((unsigned long long)__float_as_uint(depths[gid]) << 32) | (unsigned long long)lo;
        });
        __syncthreads();
    }
}

// LDS slot of sort element i: an XOR swizzle of the low five index bits
// with bits 3..7, under which the strided accesses of every blocked pass
// below (group strides 1..2048) are free of bank conflicts for 8-key groups.
__device__ __forceinline__ int sort_slot(int i) { return i ^ ((i >> 3) & 31); }

// M consecutive stages (strides lo << (M - 1), ..., lo) of the bitonic
// merge of block size k over n keys, in registers: every thread takes
// groups of 2^M keys closed under those strides (positions base + q * lo),
// so the M stages need one LDS read and one write per key and no barrier
// between them.  All keys of a group share bit k, hence the direction.
template <int M>
__device__ __forceinline__ void bitonic_pass(unsigned long long *s, int n, int k, int lo) {
    const int groups = n >> M;
    for (int g = threadIdx.x; g < groups; g += kSortThreads) {
        const int base = ((g & ~(lo - 1)) << M) | (g & (lo - 1));
        unsigned long long v[1 << M];
#pragma unroll
        for (int q = 0; q < (1 << M); ++q) v[q] = s[sort_slot(base + q * lo)];
        const bool up = (base & k) == 0;
#pragma unroll
        for (int st = M - 1; st >= 0; --st) {
#pragma unroll
            for (int q = 0; q < (1 << M); ++q) {
                if (q & (1 << st)) continue;
                const unsigned long long x = v[q], y = v[q + (1 << st)];
                const bool sw = (x > y) == up;
                v[q] = sw ? y : x;
                v[q + (1 << st)] = sw ? x : y;
            }
        }
#pragma unroll
        for (int q = 0; q < (1 << M); ++q) s[sort_slot(base + q * lo)] = v[q];
    }
}

// Ascending bitonic sort of `cnt` (2..kChunk) keys in LDS (element i in
// slot sort_slot(i)), padded to a power of two with all-ones keys: the
// stages of each merge go three at a time through registers
// (bitonic_pass), so a 2048-key sort takes 24 barriers instead of 66.
// Block-uniform control flow.
__device__ void lds_bitonic(unsigned long long *s, const unsigned long long *src, int cnt) {
    int n = 2;
    while (n < cnt) n <<= 1;
    for (int i = threadIdx.x; i < n; i += kSortThreads) s[sort_slot(i)] = i < cnt ? src[i] : ~0ull;
    __syncthreads();
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0;) {
            if (j >= 4) {
                bitonic_pass<3>(s, n, k, j >> 2);
                j >>= 3;
            } else if (j == 2) {
                bitonic_pass<2>(s, n, k, 1);
                j = 0;
            } else {
                bitonic_pass<1>(s, n, k, 1);
                j = 0;
            }
            __syncthreads();
        }
    }
}

// The tile counts of a super-tile's entries keys[0, cnt): each entry covers
// the tiles of its rectangle inside the super-tile; s_tc[16] (zeroed by the
// caller) receives the sums.  Block-uniform.
template <bool PACKED>
__device__ __forceinline__ void count_tiles(const unsigned long long *__restrict__ keys, int cnt, int stx, int sty,
                                            const uint2 *__restrict__ rect, int *s_tc) {
    int tc[kSuper * kSuper];
#pragma unroll
    for (int q = 0; q < kSuper * kSuper; ++q) tc[q] = 0;
    for (int e = threadIdx.x; e < cnt; e += kSortThreads) {
        int rx0, rx1, ry0, ry1;
        if constexpr (PACKED) {
            const int4 lr = unpack_rect((uint32_t)keys[e] & 0xffu);
            rx0 = lr.x, rx1 = lr.y, ry0 = lr.z, ry1 = lr.w;
        } else {
            const uint2 r = rect[(uint32_t)(keys[e] & 0xffffffffull)];
            rx0 = max((int)(r.x & 0xffff) - stx, 0), rx1 = min((int)(r.y & 0xffff) - stx, kSuper);
            ry0 = max((int)(r.x >> 16) - sty, 0), ry1 = min((int)(r.y >> 16) - sty, kSuper);
        }
#pragma unroll
        for (int q = 0; q < kSuper * kSuper; ++q) {
            const int lx = q % kSuper, ly = q / kSuper;
            tc[q] += (lx >= rx0 && lx < rx1 && ly >= ry0 && ly < ry1) ? 1 : 0;
        }
    }
#pragma unroll
    for (int q = 0; q < kSuper * kSuper; ++q) {
        int v = tc[q];
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
        if ((threadIdx.x & 63) == 0 && v) atomicAdd(&s_tc[q], v);
    }
    __syncthreads();
}

// Counts the entries of the super-tile's 16 tiles into tile_counts, then
// sorts the super-tile list in place: up to kChunk keys in one LDS sort,
// up to huge_th in kChunk runs queued on big_list for the merge passes.
// Longer lists are only queued, on big_list and huge_list (their tile counts
// zeroed): k_sort_chunks sorts their runs on many workgroups, and after the
// merge k_count_chunks / k_emit_chunks count and emit them chunk by chunk.
// huge_th is kHuge, or kChunk when the frame's long lists go chunk-parallel
// (bin_chunk_parallel: some list exceeds kHuge): every list above kChunk
// then joins the merge and chunk passes instead of holding one workgroup
// for several serial chunk sorts.
template <bool PACKED>
__global__ __launch_bounds__(kSortThreads) void k_sort_super(int tiles_x, int tiles_y, int sxn,
                                                             const int *__restrict__ offsets,
                                                             unsigned long long *__restrict__ keys,
                                                             const uint2 *__restrict__ rect,
                                                             int *__restrict__ tile_counts,
                                                             int *__restrict__ big_list, int *__restrict__ stats,
                                                             int *__restrict__ huge_list,
                                                             int *__restrict__ huge_stats, int huge_th) {
    __shared__ unsigned long long s[kChunk];
    __shared__ int s_tc[kSuper * kSuper];
    const int t = blockIdx.x;
    const int start = offsets[t], end = offsets[t + 1];
    const int cnt = end - start;
    const int stx = (t % sxn) * kSuper, sty = (t / sxn) * kSuper;
    if (threadIdx.x < kSuper * kSuper) s_tc[threadIdx.x] = 0;
    __syncthreads();
    if (cnt <= huge_th) count_tiles<PACKED>(keys + start, cnt, stx, sty, rect, s_tc);
    if (threadIdx.x < kSuper * kSuper) {
        const int tx = stx + (int)threadIdx.x % kSuper, ty = sty + (int)threadIdx.x / kSuper;
        if (tx < tiles_x && ty < tiles_y) tile_counts[ty * tiles_x + tx] = s_tc[threadIdx.x];
    }
    if (cnt > kChunk && threadIdx.x == 0) big_list[atomicAdd(&stats[2], 1)] = t;
    if (cnt > huge_th) {
        if (threadIdx.x == 0) huge_list[atomicAdd(&huge_stats[0], 1)] = t;
        return;
    }
    if (cnt <= 1) return;
    for (int c0 = start; c0 < end; c0 += kChunk) {
        const int c = min(kChunk, end - c0);
        lds_bitonic(s, keys + c0, c);
        for (int i = threadIdx.x; i < c; i += kSortThreads) keys[c0 + i] = s[sort_slot(i)];
        __syncthreads();
    }
}

// Unit numbering of lists of super-tiles: base[b] = the number of
// `unit`-key units (chunks, merge tiles) of lists 0 .. b-1, *total = all of
// them.  Every listed super-tile holds more than `unit` keys, so base is
// strictly increasing.
struct UnitList {
    const int *list, *count;
    int unit;
    int *base, *total;
};
__device__ __forceinline__ void number_units(const int *__restrict__ offsets, const UnitList &u, int *s_w) {
    const int n = *u.count;
    int carry = 0;
    for (int b0 = 0; b0 < n; b0 += 1024) {
        const int b = b0 + (int)threadIdx.x;
        int v = 0;
        if (b < n) {
            const int t = u.list[b];
            v = (offsets[t + 1] - offsets[t] + u.unit - 1) / u.unit;
        }
        const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
        int incl = v;
#pragma unroll
        for (int d = 1; d < 64; d <<= 1) {
            const int o = __shfl_up(incl, d, 64);
            if (lane >= d) incl += o;
        }
        __syncthreads();
        if (lane == 63) s_w[wave] = incl;
        __syncthreads();
        int off = 0, tot = 0;
#pragma unroll
        for (int w = 0; w < 16; ++w) {
            off += w < wave ? s_w[w] : 0;
            tot += s_w[w];
        }
        if (b < n) u.base[b] = carry + off + incl - v;
        carry += tot;
    }
    if (threadIdx.x == 0) *u.total = carry;
}
// One workgroup numbers both: the huge lists' chunks (when a.list is set)
// and the long lists' merge tiles (when b.list is set).
__global__ __launch_bounds__(1024) void k_list_prep(const int *__restrict__ offsets, UnitList a, UnitList b) {
    __shared__ int s_w[16];
    if (a.list) number_units(offsets, a, s_w);
    __syncthreads();
    if (b.list) number_units(offsets, b, s_w);
}

// The list of flattened unit g: the last b with base[b] <= g (base strictly
// increasing from base[0] = 0).  Called with a wave-uniform g.
__device__ __forceinline__ int list_of_unit(const int *__restrict__ base, int n, int g) {
    int lo = 0, hi = n - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (base[mid] <= g)
            lo = mid;
        else
            hi = mid - 1;
    }
    return lo;
}

// Sorts every kChunk run of the huge lists in LDS, one run per workgroup
// iteration: the grid strides over the runs of all the lists (chunk_base
// numbers them), so every run has its own workgroup whatever the lists'
// lengths.
__global__ __launch_bounds__(kSortThreads) void k_sort_chunks(const int *__restrict__ offsets,
                                                              const int *__restrict__ big_list,
                                                              const int *__restrict__ stats,
                                                              const int *__restrict__ chunk_base,
                                                              unsigned long long *__restrict__ keys) {
    __shared__ unsigned long long s[kChunk];
    const int nbig = stats[0], nchunks = stats[1];
    for (int g = blockIdx.x; g < nchunks; g += gridDim.x) {
        const int b = list_of_unit(chunk_base, nbig, g);
        const int t = big_list[b];
        const int start = offsets[t], cnt = offsets[t + 1] - start;
        const int c0 = (g - chunk_base[b]) * kChunk;
        const int c = min(kChunk, cnt - c0);
        lds_bitonic(s, keys + start + c0, c);
        for (int i = threadIdx.x; i < c; i += kSortThreads) keys[start + c0 + i] = s[sort_slot(i)];
        __syncthreads();
    }
}

// Tile counts of every kChunk chunk of the merged huge lists:
// chunk_counts[chunk_base[b] + c][16], summed into tile_counts.
template <bool PACKED>
__global__ __launch_bounds__(kSortThreads) void k_count_chunks(int tiles_x, int tiles_y, int sxn,
                                                               const int *__restrict__ offsets,
                                                               const int *__restrict__ big_list,
                                                               const int *__restrict__ stats,
                                                               const int *__restrict__ chunk_base,
                                                               const unsigned long long *__restrict__ skeys,
                                                               const unsigned long long *__restrict__ keys2,
                                                               const uint2 *__restrict__ rect,
                                                               int *__restrict__ chunk_counts,
                                                               int *__restrict__ tile_counts) {
    __shared__ int s_tc[kSuper * kSuper];
    const int nbig = stats[0], nchunks = stats[1];
    for (int g = blockIdx.x; g < nchunks; g += gridDim.x) {
        const int b = list_of_unit(chunk_base, nbig, g);
        const int t = big_list[b];
        const int start = offsets[t], cnt = offsets[t + 1] - start;
        const int stx = (t % sxn) * kSuper, sty = (t / sxn) * kSuper;
        const int c = g - chunk_base[b];
        const unsigned long long *__restrict__ keys = merged_keys(cnt, skeys, keys2);
        if (threadIdx.x < kSuper * kSuper) s_tc[threadIdx.x] = 0;
        __syncthreads();
        count_tiles<PACKED>(keys + start + c * kChunk, min(kChunk, cnt - c * kChunk), stx, sty, rect, s_tc);
        if (threadIdx.x < kSuper * kSuper) {
            const int v = s_tc[threadIdx.x];
            chunk_counts[(size_t)g * (kSuper * kSuper) + threadIdx.x] = v;
            const int tx = stx + (int)threadIdx.x % kSuper, ty = sty + (int)threadIdx.x / kSuper;
            if (v && tx < tiles_x && ty < tiles_y) atomicAdd(&tile_counts[ty * tiles_x + tx], v);
        }
        __syncthreads();
    }
}

// ---- merge passes over the lists longer than kChunk ------------------------
//
// Runs of L sorted keys are merged pairwise, L = kChunk, 2 kChunk, ... .  A
// pass is a merge path (Odeh et al., "Merge Path -- parallel merging made
// simple", 2012): the merged output of a pair is cut into tiles of kMergeTile
// keys; a workgroup finds where its tile's first and last diagonal cross the
// two runs (one binary search each), stages the tile's keys of both runs in
// LDS with coalesced loads, and each thread merges 8 outputs from its own
// diagonal of the staged keys.  Every key is read and written once per pass
// and the output leaves through LDS in coalesced 2 KB rows.  Keys are unique
// (the id is in the low word), so the merge is a permutation.  A pass skips
// the lists its L already covers: a list of cnt keys takes merge_passes(cnt)
// passes, alternating from the key buffer into the second buffer and back,
// and ends in the buffer merged_keys() names.
constexpr int kMergeTile = 2048, kMergeItems = kMergeTile / 256;


// The number of keys of A among the first d keys of the merge of the
// ascending runs A[0, la) and B[0, lb).
template <typename K>
__device__ __forceinline__ int merge_split(const K *__restrict__ A, int la, const K *__restrict__ B, int lb, int d) {
    int lo = max(0, d - lb), hi = min(d, la);
    while (lo < hi) {
        const int mid = (lo + hi) >> 1;
        if (A[mid] < B[d - mid - 1])
            lo = mid + 1;
        else
            hi = mid;
    }
    return lo;
}

// The grid strides over the merge tiles of all the lists (merge_base
// numbers them), so every tile has its own workgroup whatever the lists'
// lengths.
// merge_split by one wave, 64 probes per step: the predicate A[i] < B[d-1-i]
// holds exactly for i below the split, so each step's ballot narrows the
// range to one of 64 slices and a run of 262k keys takes three steps of
// dependent loads instead of eighteen.  Called by all 64 lanes of a wave;
// returns the split in every lane.
template <typename K>
__device__ __forceinline__ int merge_split_wave(const K *__restrict__ A, int la, const K *__restrict__ B, int lb,
                                                int d) {
    const int lane = threadIdx.x & 63;
    int lo = max(0, d - lb), hi = min(d, la);  // the split lies in [lo, hi]
    while (hi - lo > 64) {
        const int step = (hi - lo + 63) >> 6;
        const int i = lo + lane * step;
        const bool below = i < hi && A[i] < B[d - i - 1];
        const int f = __popcll(__ballot(below));  // probes below the split: lanes 0 .. f - 1
        // split in (lo + (f - 1) step, lo + f step]
        const int nlo = f > 0 ? lo + (f - 1) * step + 1 : lo;
        hi = min(hi, lo + f * step);
        lo = nlo;
    }
    const int i = lo + lane;
    const bool below = i < hi && A[i] < B[d - i - 1];
    return lo + __popcll(__ballot(below));
}

__global__ __launch_bounds__(256) void k_merge_path(int L, const int *__restrict__ offsets,
                                                    const int *__restrict__ big_list, const int *__restrict__ stats,
                                                    const int *__restrict__ merge_base,
                                                    const unsigned long long *__restrict__ src,
                                                    unsigned long long *__restrict__ dst) {
    __shared__ unsigned long long s_k[kMergeTile];
    __shared__ int s_split[2];
    const int nbig = stats[2], ntiles = stats[3];
    for (int g = blockIdx.x; g < ntiles; g += gridDim.x) {
        const int b = list_of_unit(merge_base, nbig, g);
        const int t = big_list[b];
        const int start = offsets[t], cnt = offsets[t + 1] - start;
        if (cnt <= L) continue;  // merged by an earlier pass
        // 2L is a multiple of kMergeTile, so no tile straddles two pairs
        {
            const int o0 = (g - merge_base[b]) * kMergeTile;
            const int pair_base = o0 / (2 * L) * (2 * L);
            const int la = min(L, cnt - pair_base), lb = max(0, min(L, cnt - pair_base - L));
            const unsigned long long *A = src + start + pair_base, *B = A + la;
            const int d0 = o0 - pair_base, d1 = min(d0 + kMergeTile, la + lb);
            if (threadIdx.x < 128) {
                const int w = threadIdx.x >> 6;  // wave 0: the tile's start, wave 1: its end
                const int sp = merge_split_wave(A, la, B, lb, w ? d1 : d0);
                if ((threadIdx.x & 63) == 0) s_split[w] = sp;
            }
            __syncthreads();
            const int a0 = s_split[0], a1 = s_split[1];
            const int na = a1 - a0, n = d1 - d0;
            const int b0 = d0 - a0;
            for (int k = threadIdx.x; k < n; k += 256) s_k[k] = k < na ? A[a0 + k] : B[b0 + k - na];
            __syncthreads();
            const int dd = min(kMergeItems * (int)threadIdx.x, n);
            const int nb = n - na;
            int ia = merge_split(s_k, na, s_k + na, nb, dd), ib = dd - ia;
            unsigned long long out[kMergeItems];
#pragma unroll
            for (int k = 0; k < kMergeItems; ++k) {
                const unsigned long long x = ia < na ? s_k[ia] : ~0ull, y = ib < nb ? s_k[na + ib] : ~0ull;
                const bool take_a = ib >= nb || (ia < na && x < y);
                out[k] = take_a ? x : y;
                ia += take_a ? 1 : 0;
                ib += take_a ? 0 : 1;
            }
            __syncthreads();
#pragma unroll
            for (int k = 0; k < kMergeItems; ++k)
                if (dd + k < n) s_k[dd + k] = out[k];
            __syncthreads();
            for (int k = threadIdx.x; k < n; k += 256) dst[start + o0 + k] = s_k[k];
            __syncthreads();
        }
    }
}

constexpr int kWin = 2048;  // super-list entries staged in LDS per window

// Filters the sorted super-list entries skeys[0, cnt) of the super-tile at
// tile (stx, sty) into the id lists of its tiles: wave w emits the 4 tiles of
// row w; out[lx] is the tile's list position of the first entry (-1 for a
// tile outside the image).  Within a 64-entry chunk a lane's output slot is
// the popcount of the covering lanes below it, so each tile list keeps the
// super-list (depth, id) order.  Block-uniform.
template <bool PACKED>
__device__ __forceinline__ void emit_range(const unsigned long long *__restrict__ skeys, int cnt, int stx, int sty,
                                           const uint2 *__restrict__ rect, int out[kSuper], int *s_gid,
                                           unsigned short *s_rr, int *__restrict__ ids) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;
    for (int w0 = 0; w0 < cnt; w0 += kWin) {
        const int wn = min(kWin, cnt - w0);
        __syncthreads();
        for (int k = threadIdx.x; k < wn; k += 256) {
            const uint32_t lo = (uint32_t)(skeys[w0 + k] & 0xffffffffull);
            int gid, rx0, rx1, ry0, ry1;
            if constexpr (PACKED) {
                gid = (int)(lo >> 8);
                const int4 lr = unpack_rect(lo & 0xffu);
                rx0 = lr.x, rx1 = lr.y, ry0 = lr.z, ry1 = lr.w;
            } else {
                gid = (int)lo;
                const uint2 r = rect[gid];
                const int x0 = r.x & 0xffff, y0 = r.x >> 16, x1 = r.y & 0xffff, y1 = r.y >> 16;
                rx0 = max(x0 - stx, 0), rx1 = min(x1 - stx, kSuper);
                ry0 = max(y0 - sty, 0), ry1 = min(y1 - sty, kSuper);
            }
            s_gid[k] = gid;
            s_rr[k] = (unsigned short)(rx0 | (rx1 << 4) | (ry0 << 8) | (ry1 << 12));
        }
        __syncthreads();
        for (int j = 0; j < wn; j += 64) {
            const int idx = j + lane;
            const int rr = idx < wn ? s_rr[idx] : 0;
            const int lw = wave;
            const bool row_in = ((rr >> 8) & 15) <= lw && lw < ((rr >> 12) & 15);
            const int rx0 = rr & 15, rx1 = (rr >> 4) & 15;
            const int gid = idx < wn ? s_gid[idx] : 0;
#pragma unroll
            for (int lx = 0; lx < kSuper; ++lx) {
                const bool cov = row_in && rx0 <= lx && lx < rx1;
                const unsigned long long bal = __ballot(cov);
                if (cov && out[lx] >= 0) ids[out[lx] + __popcll(bal & below)] = gid;
                if (out[lx] >= 0) out[lx] += __popcll(bal);
            }
        }
    }
}

// Emits each super-tile list of at most huge_th entries into its 16 tile
// lists (longer lists: k_emit_chunks).
template <bool PACKED>
__global__ __launch_bounds__(256) void k_emit_tiles(int tiles_x, int tiles_y, int sxn,
                                                    const int *__restrict__ soffsets,
                                                    const unsigned long long *__restrict__ skeys,
                                                    const unsigned long long *__restrict__ keys2,
                                                    const uint2 *__restrict__ rect,
                                                    const int *__restrict__ toffsets, int *__restrict__ ids,
                                                    int huge_th) {
    __shared__ int s_gid[kWin];
    __shared__ unsigned short s_rr[kWin];
    const int st = blockIdx.x;
    const int stx = (st % sxn) * kSuper, sty = (st / sxn) * kSuper;
    const int start = soffsets[st], cnt = soffsets[st + 1] - start;
    if (cnt > huge_th) return;
    // lists above kChunk went through their merge passes (merged_keys); the
    // shorter ones were sorted in place
    const unsigned long long *__restrict__ keys = cnt > kChunk ? merged_keys(cnt, skeys, keys2) : skeys;
    const int ty = sty + (int)(threadIdx.x >> 6);
    int out[kSuper];
#pragma unroll
    for (int lx = 0; lx < kSuper; ++lx) {
        const int tx = stx + lx;
        out[lx] = (tx < tiles_x && ty < tiles_y) ? toffsets[ty * tiles_x + tx] : -1;
    }
    emit_range<PACKED>(keys + start, cnt, stx, sty, rect, out, s_gid, s_rr, ids);
}

// Emits every kChunk chunk of the huge lists: a chunk's entries start in
// each tile list after those of the chunks before it (chunk_counts).
template <bool PACKED>
__global__ __launch_bounds__(256) void k_emit_chunks(int tiles_x, int tiles_y, int sxn,
                                                     const int *__restrict__ soffsets,
                                                     const int *__restrict__ big_list,
                                                     const int *__restrict__ stats,
                                                     const int *__restrict__ chunk_base,
                                                     const int *__restrict__ chunk_counts,
                                                     const unsigned long long *__restrict__ skeys,
                                                     const unsigned long long *__restrict__ keys2,
                                                     const uint2 *__restrict__ rect,
                                                     const int *__restrict__ toffsets, int *__restrict__ ids) {
    __shared__ int s_gid[kWin];
    __shared__ unsigned short s_rr[kWin];
    const int nbig = stats[0], nchunks = stats[1];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    for (int g = blockIdx.x; g < nchunks; g += gridDim.x) {
        const int b = list_of_unit(chunk_base, nbig, g);
        const int st = big_list[b];
        const int stx = (st % sxn) * kSuper, sty = (st / sxn) * kSuper;
        const int start = soffsets[st], cnt = soffsets[st + 1] - start;
        const int ty = sty + wave;
        const int c = g - chunk_base[b];
        // entries of this wave's four tiles in the chunks before c
        int before[kSuper] = {0, 0, 0, 0};
        for (int k = lane; k < c; k += 64)
#pragma unroll
            for (int lx = 0; lx < kSuper; ++lx)
                before[lx] += chunk_counts[(size_t)(chunk_base[b] + k) * (kSuper * kSuper) + wave * kSuper + lx];
        int out[kSuper];
#pragma unroll
        for (int lx = 0; lx < kSuper; ++lx) {
            int v = before[lx];
#pragma unroll
            for (int d = 32; d > 0; d >>= 1) v += __shfl_xor(v, d, 64);
            const int tx = stx + lx;
            out[lx] = (tx < tiles_x && ty < tiles_y) ? toffsets[ty * tiles_x + tx] + v : -1;
        }
        emit_range<PACKED>(merged_keys(cnt, skeys, keys2) + start + c * kChunk, min(kChunk, cnt - c * kChunk), stx,
                           sty, rect, out, s_gid, s_rr, ids);
    }
}

}  // namespace

namespace mskern {

int64_t tile_scan_temp_ints(int T) { return (T + kScanChunk - 1) / kScanChunk + 1; }

// Exclusive scan of counts[T] into offsets[T + 1] (and cursor[T] if given);
// stats[0] = total, stats[1] = max(stats[1], largest count).
static void launch_scan_counts(hipStream_t s, int T, const int *counts, int *offsets, int *cursor, int *stats,
                               int *temp) {
    if (T <= kScanSmallMax) {
        hipLaunchKernelGGL(k_scan_small, dim3(1), dim3(kScanSmallT), 0, s, T, counts, offsets, cursor, stats);
        return;
    }
    const int nb = (T + kScanChunk - 1) / kScanChunk;
    hipLaunchKernelGGL(k_off_local, dim3(nb), dim3(kScanT), 0, s, T, counts, offsets, temp, stats);
    hipLaunchKernelGGL(k_off_totals, dim3(1), dim3(1024), 0, s, nb, temp, stats);
    hipLaunchKernelGGL(k_off_add, dim3(nb), dim3(kScanT), 0, s, T, offsets, cursor, temp, stats);
}

static void bin_chunks(int n, int *blocks, int *chunk) {
    *blocks = std::max(1, std::min(kBinMaxBlocks, (n + 2047) / 2048));
    *chunk = (n + *blocks - 1) / *blocks;
}

void launch_super_count(hipStream_t s, int n, int tiles_x, int tiles_y, const int *radii, const uint32_t *rect,
                        int *super_counts, int *super_offsets, int *super_cm, int *super_stats, int *temp) {
    const int sxn = (tiles_x + kSuper - 1) / kSuper, syn = (tiles_y + kSuper - 1) / kSuper, NS = sxn * syn;
    int blocks, chunk;
    bin_chunks(n, &blocks, &chunk);
    if (n > 0)
        hipLaunchKernelGGL(k_super_hist, dim3(blocks), dim3(kBinThreads), 0, s, n, chunk, sxn, NS, radii,
                           reinterpret_cast<const uint2 *>(rect), super_cm);
    // with no splats the matrix has no rows and every count is zero
    hipLaunchKernelGGL(k_super_cols, dim3((NS + kColW - 1) / kColW), dim3(kColW * kColWaves), 0, s,
                       n > 0 ? blocks : 0, NS, super_cm, super_counts);
    launch_scan_counts(s, NS, super_counts, super_offsets, nullptr, super_stats, temp);
}

void launch_bin_tiles(hipStream_t s, int n, int tiles_x, int tiles_y, const int *radii, const uint32_t *rect,
                      const float *depths, const int *super_offsets, const int *super_cm, int super_max,
                      uint64_t *super_keys, uint64_t *super_keys_tmp, int *big_list, int *super_stats,
                      int *huge_list, int *huge_stats, int *chunk_base, int *chunk_counts, int *merge_base,
                      int total_keys, int *tile_counts, int *tile_offsets, int *tile_stats, int *tile_temp, int *ids,
                      bool force_wide_keys, const DeepScan *deep) {
    const int sxn = (tiles_x + kSuper - 1) / kSuper, syn = (tiles_y + kSuper - 1) / kSuper, NS = sxn * syn;
    const int T = tiles_x * tiles_y;
    auto *k = reinterpret_cast<unsigned long long *>(super_keys);
    auto *kt = reinterpret_cast<unsigned long long *>(super_keys_tmp);
    const uint2 *r2 = reinterpret_cast<const uint2 *>(rect);
    int blocks, chunk;
    bin_chunks(n, &blocks, &chunk);
    const bool packed = n < kPackedMaxSplats && !force_wide_keys;
    if (n > 0)
        hipLaunchKernelGGL(packed ? k_scatter_super<true> : k_scatter_super<false>, dim3(blocks), dim3(kBinThreads), 0,
                           s, n, chunk, sxn, NS, radii, r2, depths, super_offsets, super_cm, k);
    const bool big = bin_chunk_parallel(super_max, NS);
    const int huge_th = big ? kChunk : kHuge;
    hipLaunchKernelGGL(packed ? k_sort_super<true> : k_sort_super<false>, dim3(NS), dim3(kSortThreads), 0, s, tiles_x,
                       tiles_y, sxn, super_offsets, k, r2, tile_counts, big_list, super_stats, huge_list, huge_stats,
                       huge_th);
    // huge lists: kChunk runs sorted on many workgroups, then merged.  The
    // chunk and merge-tile kernels stride over units numbered across all
    // their lists; their grids cover at most total_keys / unit + NS units
    // (each list rounds up once)
    const int big_grid = (int)std::min<int64_t>(4096, (int64_t)total_keys / kChunk + NS);
    if (super_max > kChunk) {
        const UnitList chunks{huge_list, huge_stats, kChunk, chunk_base, huge_stats + 1};
        const UnitList tiles{big_list, super_stats + 2, kMergeTile, merge_base, super_stats + 3};
        hipLaunchKernelGGL(k_list_prep, dim3(1), dim3(1024), 0, s, super_offsets, big ? chunks : UnitList{}, tiles);
    }
    if (big)
        hipLaunchKernelGGL(k_sort_chunks, dim3(big_grid), dim3(kSortThreads), 0, s, super_offsets, huge_list,
                           huge_stats, chunk_base, k);
    unsigned long long *src = k, *dst = kt;
    const int merge_grid = (int)std::min<int64_t>(8192, (int64_t)total_keys / kMergeTile + NS);
    for (int L = kChunk; L < super_max; L <<= 1) {
        hipLaunchKernelGGL(k_merge_path, dim3(merge_grid), dim3(256), 0, s, L, super_offsets, big_list, super_stats,
                           merge_base, src, dst);
        std::swap(src, dst);
    }
    // each list longer than kChunk ends in the buffer its last pass wrote
    // (merged_keys); the emission reads it there
    if (big)
        hipLaunchKernelGGL(packed ? k_count_chunks<true> : k_count_chunks<false>, dim3(big_grid), dim3(kSortThreads), 0, s,
                           tiles_x, tiles_y, sxn, super_offsets, huge_list, huge_stats, chunk_base, k, kt, r2,
                           chunk_counts, tile_counts);
    launch_scan_counts(s, T, tile_counts, tile_offsets, nullptr, tile_stats, tile_temp);
    if (deep) {
        launch_deep_tiles(s, T, tile_offsets, deep->len, deep->list, deep->count);
        (void)hipMemcpyAsync(deep->host_count, deep->count, sizeof(int), hipMemcpyDeviceToHost, s);
    }
    hipLaunchKernelGGL(packed ? k_emit_tiles<true> : k_emit_tiles<false>, dim3(NS), dim3(256), 0, s, tiles_x, tiles_y,
                       sxn, super_offsets, k, kt, r2, tile_offsets, ids, huge_th);
    if (big)
        hipLaunchKernelGGL(packed ? k_emit_chunks<true> : k_emit_chunks<false>, dim3(big_grid), dim3(256), 0, s, tiles_x,
                           tiles_y, sxn, super_offsets, huge_list, huge_stats, chunk_base, chunk_counts, k, kt, r2,
                           tile_offsets, ids);
}

}  // namespace mskern
