// k_binning.hip -- tile binning (count -> scan -> scatter) and the per-tile
// depth sort: an LDS bitonic sort for tiles of up to 2048 intersections and
// a global merge path (2048-key LDS runs merged by ranking) for larger tiles.
//
// Replaces scatter_to_prealloc_bins_kernel + prefix_sum_kernel +
// bitonic_sort_per_tile_2dgs_kernel (msplat_metal.metal:1557-1690, 3093-3145),
// which preallocate 2048 slots per tile and drop the overflow.  Here every
// intersection is kept and the per-tile order is (depth bits, gaussian id).
#include "kernels.h"
#include "ms_device.h"

namespace {

constexpr int kSortThreads = 256;
constexpr int kChunk = 2048;  // keys per LDS sort (16 KB of u64)

// Exclusive scan of the per-tile counts by one 1024-thread workgroup; also
// seeds the scatter cursors and records the total and the largest tile.
__global__ __launch_bounds__(1024) void k_scan_tiles(int T, const int *__restrict__ counts,
                                                     int *__restrict__ offsets, int *__restrict__ cursor,
                                                     int *__restrict__ stats) {
    __shared__ int s_sum[16];
    __shared__ int s_max[16];
    const int tid = threadIdx.x;
    const int chunk = (T + 1023) / 1024;
    const int b = min(T, tid * chunk), e = min(T, b + chunk);
    int sum = 0, mx = 0;
    for (int i = b; i < e; ++i) {
        const int c = counts[i];
        sum += c;
        mx = max(mx, c);
    }
    // wave64 inclusive scan
    const int lane = tid & 63, wave = tid >> 6;
    int incl = sum;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const int o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    int wmax = mx;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) wmax = max(wmax, __shfl_xor(wmax, d, 64));
    if (lane == 63) s_sum[wave] = incl;
    if (lane == 0) s_max[wave] = wmax;
    __syncthreads();
    int wave_off = 0, total = 0, gmax = 0;
    for (int w = 0; w < 16; ++w) {
        if (w < wave) wave_off += s_sum[w];
        total += s_sum[w];
        gmax = max(gmax, s_max[w]);
    }
    int run = wave_off + incl - sum;
    for (int i = b; i < e; ++i) {
        offsets[i] = run;
        cursor[i] = run;
        run += counts[i];
    }
    if (tid == 0) {
        offsets[T] = total;
        stats[0] = total;
        stats[1] = gmax;
        stats[2] = 0;  // big-tile list length, filled by k_sort_tiles
    }
}

// Scatter: every visible gaussian appends (depth bits << 32 | id) to each
// tile of its rectangle at an atomically claimed slot of that tile's range.
// The rectangles of a wave are enumerated cooperatively (wave_expand), so
// the 64 lanes issue independent atomics instead of serial per-lane loops.
__global__ __launch_bounds__(256) void k_scatter(int n, int tiles_x, const int *__restrict__ radii,
                                                 const uint2 *__restrict__ rect, const float *__restrict__ depths,
                                                 int *__restrict__ cursor, unsigned long long *__restrict__ keys) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    const bool ok = i < n && radii[i] > 0;
    const uint2 r = ok ? rect[i] : make_uint2(0u, 0u);
    const int x0 = r.x & 0xffff, y0 = r.x >> 16, x1 = r.y & 0xffff, y1 = r.y >> 16;
    const int w = ok ? x1 - x0 : 1;
    const uint32_t dbits = ok ? __float_as_uint(depths[i]) : 0u;
    msd::wave_expand(ok ? (x1 - x0) * (y1 - y0) : 0, [&](int owner, int k, bool active) {
        const int ow = __shfl(w, owner, 64), ox = __shfl(x0, owner, 64), oy = __shfl(y0, owner, 64);
        const uint32_t od = (uint32_t)__shfl((int)dbits, owner, 64);
        const int oi = __shfl(i, owner, 64);
        if (active) {
            const int ty = k / ow;
            const int pos = atomicAdd(&cursor[(oy + ty) * tiles_x + ox + (k - ty * ow)], 1);
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

__global__ __launch_bounds__(kSortThreads) void k_sort_tiles(const int *__restrict__ offsets,
                                                             unsigned long long *__restrict__ keys,
                                                             int *__restrict__ ids, int *__restrict__ big_list,
                                                             int *__restrict__ stats) {
    __shared__ unsigned long long s[kChunk];
    const int t = blockIdx.x;
    const int start = offsets[t], end = offsets[t + 1];
    const int cnt = end - start;
    if (cnt <= 0) return;
    if (cnt <= kChunk) {
        lds_bitonic(s, keys + start, cnt);
        for (int i = threadIdx.x; i < cnt; i += kSortThreads) ids[start + i] = (int)(uint32_t)(s[i] & 0xffffffffull);
        return;
    }
    for (int c0 = start; c0 < end; c0 += kChunk) {
        const int c = min(kChunk, end - c0);
        lds_bitonic(s, keys + c0, c);
        for (int i = threadIdx.x; i < c; i += kSortThreads) keys[c0 + i] = s[i];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const int b = atomicAdd(&stats[2], 1);
        big_list[b] = t;
    }
}

// One merge pass over the tiles larger than kChunk: runs of length L are
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

__global__ __launch_bounds__(256) void k_big_ids(const int *__restrict__ offsets, const int *__restrict__ big_list,
                                                 const int *__restrict__ stats,
                                                 const unsigned long long *__restrict__ src, int *__restrict__ ids) {
    const int nbig = stats[2];
    for (int b = blockIdx.y; b < nbig; b += gridDim.y) {
        const int t = big_list[b];
        const int start = offsets[t], cnt = offsets[t + 1] - start;
        for (int i = blockIdx.x * 256 + threadIdx.x; i < cnt; i += gridDim.x * 256)
            ids[start + i] = (int)(uint32_t)(src[start + i] & 0xffffffffull);
    }
}

}  // namespace

namespace mskern {

void launch_scan_tiles(hipStream_t s, int T, const int *counts, int *offsets, int *cursor, int *stats) {
    hipLaunchKernelGGL(k_scan_tiles, dim3(1), dim3(1024), 0, s, T, counts, offsets, cursor, stats);
}

void launch_scatter(hipStream_t s, int n, int tiles_x, const int *radii, const uint32_t *rect,
                    const float *depths, int *cursor, uint64_t *keys) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_scatter, dim3((n + 255) / 256), dim3(256), 0, s, n, tiles_x, radii,
                       reinterpret_cast<const uint2 *>(rect), depths, cursor,
                       reinterpret_cast<unsigned long long *>(keys));
}

uint64_t *launch_sort_tiles(hipStream_t s, int T, int max_count, const int *offsets, uint64_t *keys,
                            uint64_t *keys_tmp, int *ids, int *big_list, int *stats) {
    auto *k = reinterpret_cast<unsigned long long *>(keys);
    auto *kt = reinterpret_cast<unsigned long long *>(keys_tmp);
    hipLaunchKernelGGL(k_sort_tiles, dim3(T), dim3(kSortThreads), 0, s, offsets, k, ids, big_list, stats);
    if (max_count <= kChunk) return keys;
    unsigned long long *src = k, *dst = kt;
    for (int L = kChunk; L < max_count; L <<= 1) {
        hipLaunchKernelGGL(k_merge_pass, dim3(64, 64), dim3(256), 0, s, L, offsets, big_list, stats, src, dst);
        std::swap(src, dst);
    }
    hipLaunchKernelGGL(k_big_ids, dim3(64, 64), dim3(256), 0, s, offsets, big_list, stats, src, ids);
    return reinterpret_cast<uint64_t *>(src);
}

}  // namespace mskern
