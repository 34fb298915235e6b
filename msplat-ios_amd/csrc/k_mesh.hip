// k_mesh.hip -- mesh extraction on the GPU: TSDF fusion of rendered depth
// maps (tsdf_integrate_kernel, core/metal/msplat_metal.metal:2223-2280),
// marching cubes (marching_cubes_kernel, :2606-2687) and the depth
// unprojection of Model::exportPointCloud (core/src/model.cpp:565-640).
//
// All three are HBM-bound streams over a voxel grid or an image.  The
// reference appends triangles through an atomic counter (arrival order);
// here marching cubes and the unprojection are two-pass compactions
// (classify + count per 4096-element chunk, scan of the chunk counts, emit
// at the scanned offsets), so the output order is the element order and
// identical from run to run.  Arithmetic is the reference's expressions
// evaluated left to right with no contraction (the build uses
// -ffp-contract=off).
#include <hip/hip_runtime.h>

#include <cstring>

#include "kernels.h"
#include "mc_table.h"
#include "ms_device.h"

namespace mskern {
namespace {

constexpr int kThreads = 256;
constexpr int kPerThread = kMeshChunk / kThreads;  // 16 consecutive elements per thread
static_assert(kPerThread == 16, "the emit passes load 16 case bytes as one uint4");

__constant__ mcgen::McTable c_mc = mcgen::make_mc_table();

struct McGeom {
    int8_t corner[8][3];
    int8_t edge[12][2];
};
constexpr McGeom make_geom() {
    McGeom g{};
    for (int c = 0; c < 8; ++c)
        for (int k = 0; k < 3; ++k) g.corner[c][k] = (int8_t)mcgen::kCorner[c][k];
    for (int e = 0; e < 12; ++e)
        for (int k = 0; k < 2; ++k) g.edge[e][k] = (int8_t)mcgen::kEdge[e][k];
    return g;
}
__constant__ McGeom c_geom = make_geom();

// Exclusive scan over the 256 threads of a workgroup; *total = the sum.
// lds holds 4 values; the trailing barrier lets the caller reuse it.
__device__ __forceinline__ uint32_t block_excl_scan(uint32_t v, uint32_t *lds, uint32_t *total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    uint32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) lds[wave] = incl;
    __syncthreads();
    uint32_t base = 0, sum = 0;
#pragma unroll
    for (int w = 0; w < kThreads / 64; ++w) {
        const uint32_t x = lds[w];
        base += w < wave ? x : 0u;
        sum += x;
    }
    __syncthreads();
    *total = sum;
    return base + incl - v;
}

// ---- TSDF fusion --------------------------------------------------------
// A voxel-view pair reads the view's depth and alpha only where the pixel
// passes the reference's pixel tests (alpha >= threshold, depth finite and
// positive, msplat_metal.metal:2259-2265); a first pass packs that test into
// one bit per pixel, so the pairs that land on background -- most of them
// -- touch only an L2-resident bitmask instead of the alpha map.

// One wave per 64-pixel run of a row (blockIdx.y = view).
__global__ __launch_bounds__(kThreads) void k_tsdf_masks(const TsdfViewDev *__restrict__ views, float athr) {
    const TsdfViewDev &D = views[blockIdx.y];
    const int W = D.v.width, H = D.v.height;
    const int segs = (W + 63) >> 6;
    const int64_t wv = (int64_t)blockIdx.x * (kThreads / 64) + (threadIdx.x >> 6);
    if (wv >= (int64_t)segs * H) return;  // uniform over the wave
    const int row = (int)(wv / segs), seg = (int)(wv % segs);
    const int px = seg * 64 + (threadIdx.x & 63);
    bool pass = false;
    if (px < W) {
        const int64_t pid = (int64_t)row * W + px;
        const float a = D.v.alpha_dev[pid];
        const float d = D.v.depth_dev[pid];
        pass = !(a < athr) && __builtin_isfinite(d) && d > 0.0f;
    }
    const unsigned long long bits = __ballot(pass);
    if ((threadIdx.x & 63) == 0) {
        uint32_t *w = D.mask + (int64_t)row * D.words_per_row + 2 * seg;
        w[0] = (uint32_t)bits;
        w[1] = (uint32_t)(bits >> 32);
    }
}

// One thread per voxel; a workgroup owns an 8 x 8 x 4 brick and each wave a
// 4 x 4 x 4 sub-brick, so a wave's voxels project to a compact patch of
// every view rather than a long image-space line, and bricks go to the
// XCDs in contiguous bands (msd::xcd_tile), so neighbouring bricks, whose
// patches overlap, share an L2.  Every voxel folds the views in order with
// the reference kernel's update, reads the voxel on its first update and
// writes it once at the end (untouched voxels are neither read nor written,
// as in the reference).
constexpr int kBrickX = 8, kBrickY = 8, kBrickZ = 4;

__global__ __launch_bounds__(kThreads) void k_tsdf_integrate(float2 *__restrict__ grid, int nx, int ny, int nz,
                                                             int bx, int by, int nbricks, float ox, float oy,
                                                             float oz, float vs,
                                                             const TsdfViewDev *__restrict__ views, int nviews,
                                                             float trunc) {
    const int brick = msd::xcd_tile(blockIdx.x, nbricks);
    if (brick >= nbricks) return;
    const int b_x = brick % bx, b_y = (brick / bx) % by, b_z = brick / (bx * by);
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int x = b_x * kBrickX + (wave & 1) * 4 + (lane & 3);
    const int y = b_y * kBrickY + (wave >> 1) * 4 + ((lane >> 2) & 3);
    const int z = b_z * kBrickZ + (lane >> 4);
    if (x >= nx || y >= ny || z >= nz) return;
    const int64_t vid = ((int64_t)z * ny + y) * nx + x;
    // voxel centre (msplat_metal.metal:2240-2243)
    const float wx = ox + ((float)x + 0.5f) * vs;
    const float wy = oy + ((float)y + 0.5f) * vs;
    const float wz = oz + ((float)z + 0.5f) * vs;
    float2 cur = make_float2(0.f, 0.f);
    bool have = false;
    for (int k = 0; k < nviews; ++k) {
        const TsdfViewDev &D = views[k];
        const float *m = D.v.viewmat;
        // world -> view (:2246-2249)
        const float vx = m[0] * wx + m[1] * wy + m[2] * wz + m[3];
        const float vy = m[4] * wx + m[5] * wy + m[6] * wz + m[7];
        const float vz = m[8] * wx + m[9] * wy + m[10] * wz + m[11];
        if (vz <= 0.01f) continue;
        // pinhole projection (:2252-2256)
        const float px = vx / vz * D.v.fx + D.v.cx;
        const float py = vy / vz * D.v.fy + D.v.cy;
        const int ix = msd::f2i(px), iy = msd::f2i(py);
        if (ix < 0 || ix >= D.v.width || iy < 0 || iy >= D.v.height) continue;
        // the pixel tests (:2259-2265), from the mask
        if (!((D.mask[(int64_t)iy * D.words_per_row + (ix >> 5)] >> (ix & 31)) & 1u)) continue;
        const int64_t pid = (int64_t)iy * D.v.width + ix;
        const float a = D.v.alpha_dev[pid];
        const float depth = D.v.depth_dev[pid];
        // truncated SDF and weighted running mean (:2267-2279)
        float sdf = depth - vz;
        if (sdf < -trunc) continue;
        sdf = __builtin_fminf(__builtin_fmaxf(sdf, -trunc), trunc);
        if (!have) {
            cur = grid[vid];
            have = true;
        }
        const float nw = cur.y + a;
        cur.x = (cur.x * cur.y + sdf * a) / nw;
        cur.y = nw;
    }
    if (have) grid[vid] = cur;
}

// ---- marching cubes -----------------------------------------------------
// case of the cell whose corner 0 is voxel b; 0 when a corner's weight is
// <= 0 (:2628-2631)
__device__ __forceinline__ uint32_t cell_case(const float2 *__restrict__ grid, int64_t b, int nx, int64_t nxy) {
    uint32_t m = 0;
    bool skip = false;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
        const float2 v = grid[b + c_geom.corner[q][0] + c_geom.corner[q][1] * (int64_t)nx + c_geom.corner[q][2] * nxy];
        skip |= v.y <= 0.0f;
        m |= (v.x < 0.0f ? 1u : 0u) << q;
    }
    return skip ? 0u : m;
}

// Cell c (x fastest) spans voxels (i..i+1, j..j+1, k..k+1).  Chunk b holds
// cells b*4096 .. +4095; here lane t takes cells b*4096 + 256r + t, so each
// load instruction of a wave reads 64 consecutive voxels, and the chunks
// go to the XCDs in contiguous bands (the cells of neighbouring rows and
// slices share voxels).  The emit pass gives each thread 16 consecutive
// cells instead (one 16-byte load of their case bytes, one scan).
__global__ __launch_bounds__(kThreads) void k_mc_classify(const float2 *__restrict__ grid, int nx, int ny,
                                                          int64_t ncells, int64_t nchunks,
                                                          uint8_t *__restrict__ cases,
                                                          uint32_t *__restrict__ chunk_tris) {
    __shared__ uint32_t lds[kThreads / 64];
    const int64_t chunk = msd::xcd_tile(blockIdx.x, (int)nchunks);
    if (chunk >= nchunks) return;
    const int64_t nxy = (int64_t)nx * ny;
    const int cx = nx - 1, cy = ny - 1;
    uint32_t tris = 0;
    for (int r = 0; r < kPerThread; ++r) {
        const int64_t c = chunk * kMeshChunk + r * kThreads + threadIdx.x;
        uint32_t m = 0;
        if (c < ncells) {
            const int i = (int)(c % cx);
            const int64_t q = c / cx;
            const int j = (int)(q % cy), k = (int)(q / cy);
            m = cell_case(grid, ((int64_t)k * ny + j) * nx + i, nx, nxy);
            tris += c_mc.ntri[m];
        }
        cases[c] = (uint8_t)m;  // the case buffer covers whole chunks
    }
    uint32_t total;
    (void)block_excl_scan(tris, lds, &total);
    if (threadIdx.x == 0) chunk_tris[chunk] = total;
}

// Exclusive scan of n chunk counts into off[0..n] (off[n] = total) by one
// workgroup of 1024 threads, each owning a contiguous run of counts.
__global__ __launch_bounds__(1024) void k_chunk_scan(const uint32_t *__restrict__ counts, int64_t n,
                                                     uint64_t *__restrict__ off) {
    __shared__ unsigned long long lds[16];
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int64_t per = (n + 1023) / 1024;
    const int64_t a = (int64_t)t * per, e = a + per < n ? a + per : n;
    unsigned long long s = 0;
    for (int64_t q = a; q < e; ++q) s += counts[q];
    unsigned long long incl = s;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const unsigned long long o = __shfl_up(incl, d, 64);
        if (lane >= d) incl += o;
    }
    if (lane == 63) lds[wave] = incl;
    __syncthreads();
    unsigned long long base = 0;
    for (int w = 0; w < wave; ++w) base += lds[w];
    base += incl - s;
    for (int64_t q = a; q < e; ++q) {
        off[q] = base;
        base += counts[q];
    }
    if (t == 1023) {
        unsigned long long tot = 0;
        for (int w = 0; w < 16; ++w) tot += lds[w];
        off[n] = tot;
    }
}

// Emit: each thread counts the triangles of its 16 consecutive cells (one
// 16-byte load of their case bytes); one block scan gives every cell's
// triangle offset and its slot in an LDS list of the chunk's surface cells;
// the threads then take the listed cells in turn, so the few surface cells
// of a chunk spread over all lanes instead of serialising in the lanes
// that own them.
__global__ __launch_bounds__(kThreads) void k_mc_emit(const float2 *__restrict__ grid, int nx, int ny,
                                                      int64_t ncells, float ox, float oy, float oz, float vs,
                                                      const uint8_t *__restrict__ cases,
                                                      const uint64_t *__restrict__ chunk_off, int64_t max_tris,
                                                      float *__restrict__ out) {
    __shared__ uint32_t lds[kThreads / 64];
    __shared__ uint32_t s_cell[kMeshChunk];  // (cell in chunk) << 8 | case
    __shared__ uint16_t s_tri[kMeshChunk];   // first triangle of the cell, in the chunk
    const int64_t base = (int64_t)blockIdx.x * kMeshChunk;
    const int64_t c0 = base + (int64_t)threadIdx.x * kPerThread;
    uint32_t packed[4] = {0u, 0u, 0u, 0u};
    uint32_t tris = 0, cells = 0;
    if (c0 < ncells) {
        const uint4 p = *reinterpret_cast<const uint4 *>(cases + c0);
        packed[0] = p.x;
        packed[1] = p.y;
        packed[2] = p.z;
        packed[3] = p.w;
#pragma unroll
        for (int q = 0; q < kPerThread; ++q) {
            const uint32_t nt = c_mc.ntri[(packed[q >> 2] >> (8 * (q & 3))) & 255u];
            tris += nt;
            cells += nt ? 1u : 0u;
        }
    }
    // triangles (< 20481) in the high half, surface cells (<= 4096) in the low
    uint32_t total;
    const uint32_t pre = block_excl_scan(tris << 16 | cells, lds, &total);
    const uint32_t ncell = total & 0xffffu;
    if (ncell == 0) return;  // uniform over the workgroup
    uint32_t tp = pre >> 16, cp = pre & 0xffffu;
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
        const uint32_t m = (packed[q >> 2] >> (8 * (q & 3))) & 255u;
        const uint32_t nt = c_mc.ntri[m];
        if (nt == 0) continue;
        s_cell[cp] = (uint32_t)(threadIdx.x * kPerThread + q) << 8 | m;
        s_tri[cp] = (uint16_t)tp;
        ++cp;
        tp += nt;
    }
    __syncthreads();
    const uint64_t chunk_first = chunk_off[blockIdx.x];
    const int64_t nxy = (int64_t)nx * ny;
    const int cx = nx - 1, cy = ny - 1;
    for (uint32_t e = threadIdx.x; e < ncell; e += kThreads) {
        const uint32_t cm = s_cell[e];
        const uint32_t m = cm & 255u;
        uint64_t o = chunk_first + s_tri[e];
        if ((int64_t)o >= max_tris) continue;
        const int64_t c = base + (cm >> 8);
        const int i = (int)(c % cx);
        const int64_t r = c / cx;
        const int j = (int)(r % cy), k = (int)(r / cy);
        const int64_t b = ((int64_t)k * ny + j) * nx + i;
        float sv[8];
#pragma unroll
        for (int cn = 0; cn < 8; ++cn)
            sv[cn] = grid[b + c_geom.corner[cn][0] + c_geom.corner[cn][1] * (int64_t)nx +
                          c_geom.corner[cn][2] * nxy].x;
        const int nt = c_mc.ntri[m];
        for (int t = 0; t < nt && (int64_t)o < max_tris; ++t, ++o) {
            float *dst = out + o * 9;
            for (int v = 0; v < 3; ++v) {
                const int ed = c_mc.tri[m][3 * t + v];
                const int a = c_geom.edge[ed][0], bb = c_geom.edge[ed][1];
                const float s0 = sv[a], s1 = sv[bb];
                // edge interpolation (:2644-2661)
                const float tt = (s1 == s0) ? 0.5f : (-s0 / (s1 - s0));
                const float p0x = ox + vs * ((float)(i + c_geom.corner[a][0]) + 0.5f);
                const float p0y = oy + vs * ((float)(j + c_geom.corner[a][1]) + 0.5f);
                const float p0z = oz + vs * ((float)(k + c_geom.corner[a][2]) + 0.5f);
                const float p1x = ox + vs * ((float)(i + c_geom.corner[bb][0]) + 0.5f);
                const float p1y = oy + vs * ((float)(j + c_geom.corner[bb][1]) + 0.5f);
                const float p1z = oz + vs * ((float)(k + c_geom.corner[bb][2]) + 0.5f);
                dst[3 * v + 0] = p0x + (p1x - p0x) * tt;
                dst[3 * v + 1] = p0y + (p1y - p0y) * tt;
                dst[3 * v + 2] = p0z + (p1z - p0z) * tt;
            }
        }
    }
}

// ---- depth unprojection -------------------------------------------------
struct UnprojArgs {
    const float *img, *depth, *alpha;
    int W;
    int64_t npix;
    float fx, fy, cx, cy, thr;
    float r[9], t[3];  // camToWorld rotation with columns 1, 2 negated; translation
};

// the pixel test of model.cpp:592-596; d = depth / alpha
__device__ __forceinline__ bool unproj_valid(const UnprojArgs &A, int64_t p, float *d) {
    const float a = A.alpha[p];
    if (a < A.thr) return false;
    *d = A.depth[p] / a;
    return __builtin_isfinite(*d) && *d > 0.0f;
}

__global__ __launch_bounds__(kThreads) void k_unproject_count(UnprojArgs A, uint32_t *__restrict__ chunk_pts) {
    __shared__ uint32_t lds[kThreads / 64];
    const int64_t p0 = (int64_t)blockIdx.x * kMeshChunk + (int64_t)threadIdx.x * kPerThread;
    uint32_t cnt = 0;
    for (int q = 0; q < kPerThread; ++q) {
        float d;
        if (p0 + q < A.npix && unproj_valid(A, p0 + q, &d)) ++cnt;
    }
    uint32_t total;
    (void)block_excl_scan(cnt, lds, &total);
    if (threadIdx.x == 0) chunk_pts[blockIdx.x] = total;
}

__device__ __forceinline__ uint8_t to_u8(float x) {
    return (uint8_t)__builtin_fminf(__builtin_fmaxf(x * 255.0f, 0.0f), 255.0f);
}

__global__ __launch_bounds__(kThreads) void k_unproject_emit(UnprojArgs A, const uint64_t *__restrict__ chunk_off,
                                                             float *__restrict__ xyz, uint8_t *__restrict__ rgb) {
    __shared__ uint32_t lds[kThreads / 64];
    const int64_t p0 = (int64_t)blockIdx.x * kMeshChunk + (int64_t)threadIdx.x * kPerThread;
    uint32_t valid = 0, cnt = 0;
    float dv[kPerThread];
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
        dv[q] = 0.f;
        if (p0 + q < A.npix && unproj_valid(A, p0 + q, &dv[q])) {
            valid |= 1u << q;
            ++cnt;
        }
    }
    uint32_t total;
    int64_t o = (int64_t)(chunk_off[blockIdx.x] + block_excl_scan(cnt, lds, &total));
#pragma unroll
    for (int q = 0; q < kPerThread; ++q) {
        if (!(valid >> q & 1u)) continue;
        const int64_t p = p0 + q;
        const int px = (int)(p % A.W), py = (int)(p / A.W);
        const float d = dv[q];
        // OpenCV camera ray through the pixel centre (model.cpp:599-602)
        const float xc = ((float)px + 0.5f - A.cx) * d / A.fx;
        const float yc = ((float)py + 0.5f - A.cy) * d / A.fy;
        const float zc = d;
        // camera -> world (:604-607)
        xyz[3 * o + 0] = A.r[0] * xc + A.r[1] * yc + A.r[2] * zc + A.t[0];
        xyz[3 * o + 1] = A.r[3] * xc + A.r[4] * yc + A.r[5] * zc + A.t[1];
        xyz[3 * o + 2] = A.r[6] * xc + A.r[7] * yc + A.r[8] * zc + A.t[2];
        rgb[3 * o + 0] = to_u8(A.img[3 * p + 0]);
        rgb[3 * o + 1] = to_u8(A.img[3 * p + 1]);
        rgb[3 * o + 2] = to_u8(A.img[3 * p + 2]);
        ++o;
    }
}

}  // namespace

void mc_table_host(int8_t *tri) {
    static constexpr mcgen::McTable t = mcgen::make_mc_table();
    std::memcpy(tri, &t.tri[0][0], sizeof(t.tri));
}

void launch_tsdf_masks(hipStream_t s, const TsdfViewDev *views_dev, int nviews, int64_t max_segs, float athr) {
    const dim3 g((unsigned)((max_segs + kThreads / 64 - 1) / (kThreads / 64)), (unsigned)nviews);
    k_tsdf_masks<<<g, kThreads, 0, s>>>(views_dev, athr);
}

void launch_tsdf_integrate(hipStream_t s, float *grid, int nx, int ny, int nz, const float origin[3], float vs,
                           const TsdfViewDev *views_dev, int nviews, float trunc) {
    const int bx = (nx + kBrickX - 1) / kBrickX, by = (ny + kBrickY - 1) / kBrickY, bz = (nz + kBrickZ - 1) / kBrickZ;
    const int nb = bx * by * bz;
    k_tsdf_integrate<<<(unsigned)(8 * ((nb + 7) / 8)), kThreads, 0, s>>>(
        reinterpret_cast<float2 *>(grid), nx, ny, nz, bx, by, nb, origin[0], origin[1], origin[2], vs, views_dev,
        nviews, trunc);
}

void launch_mc_classify(hipStream_t s, const float *grid, int nx, int ny, int nz, uint8_t *cases,
                        uint32_t *chunk_tris) {
    const int64_t nc = mc_num_cells(nx, ny, nz), nch = mesh_chunks(nc);
    k_mc_classify<<<(unsigned)(8 * ((nch + 7) / 8)), kThreads, 0, s>>>(reinterpret_cast<const float2 *>(grid), nx,
                                                                        ny, nc, nch, cases, chunk_tris);
}

void launch_chunk_scan(hipStream_t s, const uint32_t *counts, int64_t n, uint64_t *off) {
    k_chunk_scan<<<1, 1024, 0, s>>>(counts, n, off);
}

void launch_mc_emit(hipStream_t s, const float *grid, int nx, int ny, int nz, const float origin[3], float vs,
                    const uint8_t *cases, const uint64_t *chunk_off, int64_t max_tris, float *out) {
    const int64_t nc = mc_num_cells(nx, ny, nz);
    k_mc_emit<<<(unsigned)mesh_chunks(nc), kThreads, 0, s>>>(reinterpret_cast<const float2 *>(grid), nx, ny, nc,
                                                              origin[0], origin[1], origin[2], vs, cases,
                                                              chunk_off, max_tris, out);
}

static UnprojArgs unproj_args(const float *img, const float *depth, const float *alpha, int W, int H, float fx,
                              float fy, float cx, float cy, const float c2w[16], float thr) {
    UnprojArgs A;
    A.img = img;
    A.depth = depth;
    A.alpha = alpha;
    A.W = W;
    A.npix = (int64_t)W * H;
    A.fx = fx;
    A.fy = fy;
    A.cx = cx;
    A.cy = cy;
    A.thr = thr;
    for (int r = 0; r < 3; ++r) {
        A.r[3 * r + 0] = c2w[4 * r + 0];
        A.r[3 * r + 1] = -c2w[4 * r + 1];
        A.r[3 * r + 2] = -c2w[4 * r + 2];
        A.t[r] = c2w[4 * r + 3];
    }
    return A;
}

void launch_unproject_count(hipStream_t s, const float *img, const float *depth, const float *alpha, int W, int H,
                            float fx, float fy, float cx, float cy, const float c2w[16], float thr,
                            uint32_t *chunk_pts) {
    const UnprojArgs A = unproj_args(img, depth, alpha, W, H, fx, fy, cx, cy, c2w, thr);
    k_unproject_count<<<(unsigned)mesh_chunks(A.npix), kThreads, 0, s>>>(A, chunk_pts);
}

void launch_unproject_emit(hipStream_t s, const float *img, const float *depth, const float *alpha, int W, int H,
                           float fx, float fy, float cx, float cy, const float c2w[16], float thr,
                           const uint64_t *chunk_off, float *xyz, uint8_t *rgb) {
    const UnprojArgs A = unproj_args(img, depth, alpha, W, H, fx, fy, cx, cy, c2w, thr);
    k_unproject_emit<<<(unsigned)mesh_chunks(A.npix), kThreads, 0, s>>>(A, chunk_off, xyz, rgb);
}

}  // namespace mskern
