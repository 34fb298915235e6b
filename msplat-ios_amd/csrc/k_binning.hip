// k_binning.hip -- tile binning and per-tile depth order, in two levels.
//
// Replaces scatter_to_prealloc_bins_kernel + prefix_sum_kernel +
// bitonic_sort_per_tile_2dgs_kernel (msplat_metal.metal:1557-1690, 3093-3145),
// which preallocate 2048 slots per tile, drop the overflow and sort every
// tile list separately.  Here every intersection is kept and the per-tile
// order is (depth bits, gaussian id), as the reference's keys define it.
//
//   1. counts: each visible splat adds its tile rectangle, and its rectangle
//      of 4x4-tile super-tiles, to two 2D difference arrays (k_project_fwd);
//      2D prefix sums + exclusive scans give tile offsets (the layout of
//      the id list the rasterizers read) and super-tile offsets;
//   2. k_scatter_super: one (depth bits << 32 | id) key per (splat,
//      super-tile) pair -- about 2.5 per splat instead of one per tile;
//   3. k_sort_super: each super-tile's keys sorted in LDS (bitonic, up to
//      4096 keys), larger lists in 4096-key runs merged by k_merge_pass;
//   4. k_emit_tiles: each super-tile's sorted list is filtered, in order,
//      into the id lists of its 16 tiles (wave ballots keep the order), so
//      every tile list comes out sorted without a per-tile sort.
#include "kernels.h"
#include "ms_device.h"

namespace {

constexpr int kSortThreads = 256;
constexpr int kChunk = 4096;  // keys per LDS sort (32 KB of u64)
constexpr int kSuper = 4;     // tiles per super-tile side

// ---- tile counts and offsets ----------------------------------------------
//
// k_project_fwd records each visible splat's tile rectangle [x0,x1) x [y0,y1)
// as four +-1 corner updates of a (tiles_y + 1) x (tiles_x + 1) difference
// array (4 atomics per splat instead of one per covered tile); the tile
// counts are its 2D inclusive prefix sum.  Then an exclusive scan gives the
// tile offsets (prefix_sum_kernel, msplat_metal.metal:3093-3145), the
// scatter cursors, the intersection total and the largest tile.

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

// Row pass: rows[y][x] = sum over x' <= x of diff[y][x'].
__global__ __launch_bounds__(kScanT) void k_diff_rows(int tx, const int *__restrict__ diff, int *__restrict__ rows,
                                                      int *__restrict__ stats) {
    __shared__ int s_w[kScanT / 64];
    const int y = blockIdx.x;
    const int *d = diff + (size_t)y * (tx + 1);
    int *r = rows + (size_t)y * tx;
    int carry = 0;
    for (int base = 0; base < tx; base += kScanT) {
        const int x = base + (int)threadIdx.x;
        int total;
        const int incl = block_scan_incl(x < tx ? d[x] : 0, s_w, &total);
        if (x < tx) r[x] = carry + incl;
        carry += total;
    }
    if (y == 0 && threadIdx.x == 0) {
        stats[1] = 0;  // largest tile, filled by k_diff_cols
        stats[2] = 0;  // long-list count, filled by k_sort_super
    }
}

// Column pass, in place: counts[y][x] = sum over y' <= y of rows[y'][x].
// 64 columns per workgroup, the rows split in four runs (one per wave).
__global__ __launch_bounds__(kScanT) void k_diff_cols(int tx, int ty, int *__restrict__ counts,
                                                      int *__restrict__ stats) {
    __shared__ int s_part[4][64];
    const int lane = threadIdx.x & 63, g = threadIdx.x >> 6;
    const int col = blockIdx.x * 64 + lane;
    const int run_len = (ty + 3) / 4, y0 = min(ty, g * run_len), y1 = min(ty, y0 + run_len);
    int part = 0;
    if (col < tx)
        for (int y = y0; y < y1; ++y) part += counts[(size_t)y * tx + col];
    s_part[g][lane] = part;
    __syncthreads();
    int run = 0;
    for (int k = 0; k < g; ++k) run += s_part[k][lane];
    int mx = 0;
    if (col < tx)
        for (int y = y0; y < y1; ++y) {
            run += counts[(size_t)y * tx + col];
            counts[(size_t)y * tx + col] = run;
            mx = max(mx, run);
        }
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) mx = max(mx, __shfl_xor(mx, d, 64));
    if (lane == 0) atomicMax(&stats[1], mx);
}

// Exclusive scan of the T tile counts: local pass (2048 counts per
// workgroup), block totals, add pass.
__global__ __launch_bounds__(kScanT) void k_off_local(int T, const int *__restrict__ counts,
                                                      int *__restrict__ offsets, int *__restrict__ totals) {
    __shared__ int s_w[kScanT / 64];
    const int base = blockIdx.x * kScanChunk + threadIdx.x * kScanI;
    int v[kScanI], sum = 0;
#pragma unroll
    for (int k = 0; k < kScanI; ++k) {
        v[k] = base + k < T ? counts[base + k] : 0;
        sum += v[k];
    }
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
            cursor[base + k] = v;
        }
    if (blockIdx.x == 0 && threadIdx.x == 0) offsets[T] = stats[0];
}

// One key per (visible splat, super-tile of its rectangle) at an atomically
// claimed slot of the super-tile's range.  The rectangles of a wave are
// enumerated cooperatively (wave_expand), so the 64 lanes issue independent
// atomics instead of serial per-lane loops.
__global__ __launch_bounds__(256) void k_scatter_super(int n, int sxn, const int *__restrict__ radii,
                                                       const uint2 *__restrict__ rect,
                                                       const float *__restrict__ depths, int *__restrict__ cursor,
                                                       unsigned long long *__restrict__ keys) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const bool vis = i < n && radii[i] > 0;
    const uint2 r = vis ? rect[i] : make_uint2(0u, 0u);
    const int x0 = r.x & 0xffff, y0 = r.x >> 16, x1 = r.y & 0xffff, y1 = r.y >> 16;
    const bool ok = vis && x1 > x0 && y1 > y0;
    const int sx0 = x0 / kSuper, sy0 = y0 / kSuper;
    const int sw = ok ? (x1 + kSuper - 1) / kSuper - sx0 : 1;
    const int sh = ok ? (y1 + kSuper - 1) / kSuper - sy0 : 0;
    const uint32_t dbits = ok ? __float_as_uint(depths[i]) : 0u;
    msd::wave_expand(ok ? sw * sh : 0, [&](int owner, int k, bool active) {
        const int ow = __shfl(sw, owner, 64), ox = __shfl(sx0, owner, 64), oy = __shfl(sy0, owner, 64);
        const uint32_t od = (uint32_t)__shfl((int)dbits, owner, 64);
        const int oi = __shfl(i, owner, 64);
        if (active) {
            const int ry = k / ow;
            const int pos = atomicAdd(&cursor[(oy + ry) * sxn + ox + (k - ry * ow)], 1);
            keys[pos] = ((unsigned long long)od << 32) | (unsigned long long)(uint32_t)oi;
        }
    });
}

// Ascending bitonic sort of `cnt` (<= kChunk) keys in LDS, padded to a power
// of two with all-ones keys.  Block-uniform control flow.
__device__ void lds_bitonic(unsigned long long *s, const unsigned long long *src, int cnt) {
    int n = 1;
    while (n < cnt) n <<= 1;
    for (int i = threadIdx.x; i < n; i += kSortThreads) s[i] = i < cnt ? src[i] : ~0ull;
    __syncthreads();
    for (int k = 2; k <= n; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < (n >> 1); i += kSortThreads) {
                const int pos = 2 * i - (i & (j - 1));
                const int partner = pos | j;
                const bool up = (pos & k) == 0;
                const unsigned long long a = s[pos], b = s[partner];
                if ((a > b) == up) {
                    s[pos] = b;
                    s[partner] = a;
                }
            }
            __syncthreads();
        }
    }
}

// Sorts each super-tile list in place; lists longer than kChunk are sorted
// in kChunk runs and queued on big_list for the merge passes.
__global__ __launch_bounds__(kSortThreads) void k_sort_super(const int *__restrict__ offsets,
                                                             unsigned long long *__restrict__ keys,
                                                             int *__restrict__ big_list, int *__restrict__ stats) {
    __shared__ unsigned long long s[kChunk];
    const int t = blockIdx.x;
    const int start = offsets[t], end = offsets[t + 1];
    const int cnt = end - start;
    if (cnt <= 1) return;
    for (int c0 = start; c0 < end; c0 += kChunk) {
        const int c = min(kChunk, end - c0);
        lds_bitonic(s, keys + c0, c);
        for (int i = threadIdx.x; i < c; i += kSortThreads) keys[c0 + i] = s[i];
        __syncthreads();
    }
    if (cnt > kChunk && threadIdx.x == 0) {
        const int b = atomicAdd(&stats[2], 1);
        big_list[b] = t;
    }
}

// One merge pass over the lists longer than kChunk: runs of length L are
// merged pairwise.  Each key lands at (its index in its run) + (number of
// keys of the partner run that are smaller); keys are unique (the id is in
// the low word), so this is a permutation.
__global__ __launch_bounds__(256) void k_merge_pass(int L, const int *__restrict__ offsets,
                                                    const int *__restrict__ big_list, const int *__restrict__ stats,
                                                    const unsigned long long *__restrict__ src,
                                                    unsigned long long *__restrict__ dst) {
    const int nbig = stats[2];
    for (int b = blockIdx.y; b < nbig; b += gridDim.y) {
        const int t = big_list[b];
        const int start = offsets[t], cnt = offsets[t + 1] - start;
        for (int i = blockIdx.x * 256 + threadIdx.x; i < cnt; i += gridDim.x * 256) {
            const int run = i / L;
            const int rs = run * L;
            const int pair_base = (run & ~1) * L;
            const unsigned long long key = src[start + i];
            int os, olen;
            if (run & 1) {
                os = rs - L;
                olen = L;
            } else {
                os = rs + L;
                olen = max(0, min(L, cnt - os));
            }
            int lo = 0, hi = olen;
            while (lo < hi) {
                const int mid = (lo + hi) >> 1;
                if (src[start + os + mid] < key)
                    lo = mid + 1;
                else
                    hi = mid;
            }
            dst[start + pair_base + (i - rs) + lo] = key;
        }
    }
}

__global__ __launch_bounds__(256) void k_copy_big(const int *__restrict__ offsets, const int *__restrict__ big_list,
                                                  const int *__restrict__ stats,
                                                  const unsigned long long *__restrict__ src,
                                                  unsigned long long *__restrict__ dst) {
    const int nbig = stats[2];
    for (int b = blockIdx.y; b < nbig; b += gridDim.y) {
        const int t = big_list[b];
        const int start = offsets[t], cnt = offsets[t + 1] - start;
        for (int i = blockIdx.x * 256 + threadIdx.x; i < cnt; i += gridDim.x * 256) dst[start + i] = src[start + i];
    }
}

constexpr int kWin = 2048;  // super-list entries staged in LDS per window

// Filters each super-tile's sorted list into the id lists of its 16 tiles.
// Wave w emits the 4 tiles of row w of the super-tile; within a 64-entry
// chunk a lane's output slot is the popcount of the covering lanes below it,
// so each tile list keeps the super-list (depth, id) order.
__global__ __launch_bounds__(256) void k_emit_tiles(int tiles_x, int tiles_y, int sxn,
                                                    const int *__restrict__ soffsets,
                                                    const unsigned long long *__restrict__ skeys,
                                                    const uint2 *__restrict__ rect,
                                                    const int *__restrict__ toffsets, int *__restrict__ ids) {
    __shared__ int s_gid[kWin];
    __shared__ unsigned short s_rr[kWin];
    const int st = blockIdx.x;
    const int stx = (st % sxn) * kSuper, sty = (st / sxn) * kSuper;
    const int start = soffsets[st], cnt = soffsets[st + 1] - start;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const unsigned long long below = (1ull << lane) - 1ull;
    const int ty = sty + wave;
    int out[kSuper], base[kSuper];
#pragma unroll
    for (int lx = 0; lx < kSuper; ++lx) {
        const int tx = stx + lx;
        out[lx] = (tx < tiles_x && ty < tiles_y) ? toffsets[ty * tiles_x + tx] : -1;
        base[lx] = 0;
    }
    for (int w0 = 0; w0 < cnt; w0 += kWin) {
        const int wn = min(kWin, cnt - w0);
        __syncthreads();
        for (int k = threadIdx.x; k < wn; k += 256) {
            const int gid = (int)(uint32_t)(skeys[start + w0 + k] & 0xffffffffull);
            const uint2 r = rect[gid];
            const int x0 = r.x & 0xffff, y0 = r.x >> 16, x1 = r.y & 0xffff, y1 = r.y >> 16;
            const int rx0 = max(x0 - stx, 0), rx1 = min(x1 - stx, kSuper);
            const int ry0 = max(y0 - sty, 0), ry1 = min(y1 - sty, kSuper);
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
                if (cov && out[lx] >= 0) ids[out[lx] + base[lx] + __popcll(bal & below)] = gid;
                base[lx] += __popcll(bal);
            }
        }
    }
}

}  // namespace

namespace mskern {

int64_t tile_scan_temp_ints(int T) { return (T + kScanChunk - 1) / kScanChunk + 1; }

void launch_scan_tiles(hipStream_t s, int tiles_x, int tiles_y, const int *diff, int *counts, int *offsets,
                       int *cursor, int *stats, int *temp) {
    const int T = tiles_x * tiles_y;
    const int nb = (T + kScanChunk - 1) / kScanChunk;
    hipLaunchKernelGGL(k_diff_rows, dim3(tiles_y), dim3(kScanT), 0, s, tiles_x, diff, counts, stats);
    hipLaunchKernelGGL(k_diff_cols, dim3((tiles_x + 63) / 64), dim3(kScanT), 0, s, tiles_x, tiles_y, counts, stats);
    hipLaunchKernelGGL(k_off_local, dim3(nb), dim3(kScanT), 0, s, T, counts, offsets, temp);
    hipLaunchKernelGGL(k_off_totals, dim3(1), dim3(1024), 0, s, nb, temp, stats);
    hipLaunchKernelGGL(k_off_add, dim3(nb), dim3(kScanT), 0, s, T, offsets, cursor, temp, stats);
}

void launch_bin_tiles(hipStream_t s, int n, int tiles_x, int tiles_y, const int *radii, const uint32_t *rect,
                      const float *depths, const int *tile_offsets, const int *super_offsets, int *super_cursor,
                      int super_max, uint64_t *super_keys, uint64_t *super_keys_tmp, int *big_list,
                      int *super_stats, int *ids) {
    const int sxn = (tiles_x + kSuper - 1) / kSuper, syn = (tiles_y + kSuper - 1) / kSuper, NS = sxn * syn;
    auto *k = reinterpret_cast<unsigned long long *>(super_keys);
    auto *kt = reinterpret_cast<unsigned long long *>(super_keys_tmp);
    const uint2 *r2 = reinterpret_cast<const uint2 *>(rect);
    if (n > 0)
        hipLaunchKernelGGL(k_scatter_super, dim3((n + 255) / 256), dim3(256), 0, s, n, sxn, radii, r2, depths,
                           super_cursor, k);
    hipLaunchKernelGGL(k_sort_super, dim3(NS), dim3(kSortThreads), 0, s, super_offsets, k, big_list, super_stats);
    unsigned long long *src = k, *dst = kt;
    for (int L = kChunk; L < super_max; L <<= 1) {
        hipLaunchKernelGGL(k_merge_pass, dim3(64, 64), dim3(256), 0, s, L, super_offsets, big_list, super_stats, src,
                           dst);
        std::swap(src, dst);
    }
    // the merged lists of long super-tiles end in src; copy them back so
    // every list is in super_keys for the emission
    if (src != k)
        hipLaunchKernelGGL(k_copy_big, dim3(64, 64), dim3(256), 0, s, super_offsets, big_list, super_stats, src, k);
    hipLaunchKernelGGL(k_emit_tiles, dim3(NS), dim3(256), 0, s, tiles_x, tiles_y, sxn, super_offsets, k, r2,
                       tile_offsets, ids);
}

}  // namespace mskern
