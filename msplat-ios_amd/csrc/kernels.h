// kernels.h -- host-side launchers of the gfx950 kernels (one translation
// unit per kernel family; the engine calls these on its stream).
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <algorithm>

#include "msplat_engine.h"
#include "raster_wave.h"

namespace mskern {

// k_project.hip
// isect_total (64-bit, zeroed by the caller) receives the number of tile
// intersections, the sum of the visible splats' tile-rectangle areas.
// mrec receives the per-splat part of the rasterizer's quadrant-mask test
// (msd::MaskRec, 12 floats per splat), read by launch_raster_fwd.
void launch_project_fwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, float *rec,
                        float *mrec, float *depths, int *radii, uint32_t *rect, unsigned long long *isect_total,
                        float *colors_raw);
// moments_rec (the forward's splat records) non-null: g16 holds the
// image-only raster backward's sums (ray moments and unscaled per-splat
// sums), finished inside the kernel.
void launch_project_bwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, const int *radii,
                        const float *g16, float *dmeans, float *dscales, float *dquats, float *dmean2d,
                        float *dfdc, float *dfrest, float *grad_norm, float *vis, float *max2d,
                        float inv_max_dim, const MsplatAdam *adam, const float *moments_rec,
                        const int *skip_if = nullptr, int skip_above = 0);
// The image-only raster backward's g16 rows -> the reference's raster
// gradients (dL/dtransMat, dL/dopacity logit, dL/dcolors), in place.
void launch_finish_image_grads(hipStream_t s, int n, const float *rec, float *g16);
void launch_gather(hipStream_t s, const float *src, int src_stride, int src_off, int nf, float *dst, int n);
// 3DGS mode.  rec: N records of kRec3Floats, then N quadrant-mask boxes
// (4 floats); scales are [N,3].  sums_rec non-null: g16 holds the 3DGS
// raster backward's per-splat sums, finished inside the kernel.
constexpr int kRec3Floats = 12;
void launch_project3d_fwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, float *rec,
                          float *boxes, float *depths, int *radii, uint32_t *rect, unsigned long long *isect_total,
                          float *colors_raw);
void launch_project3d_bwd(hipStream_t s, const MsplatCamera &cam, const MsplatGaussians &g, const int *radii,
                          const float *g16, float *dmeans, float *dscales, float *dquats, float *dmean2d,
                          float *dfdc, float *dfrest, float *grad_norm, float *vis, float *max2d,
                          float inv_max_dim, const MsplatAdam *adam, const float *sums_rec,
                          const int *skip_if = nullptr, int skip_above = 0);
// The 3DGS raster backward's sums -> the raster gradients [dxy 2, dconic 3,
// dopacity logit, dcolor 3] (the first 9 of each 16-float row), in place.
void launch_finish3d_grads(hipStream_t s, int n, const float *rec, float *g16);
void launch_tiles_hit(hipStream_t s, const uint32_t *rect, const int *radii, int *out, int n);

// k_binning.hip
// Super-tiles are 4x4 tiles: sxn = ceil(tiles_x / 4), syn = ceil(tiles_y / 4),
// NS = sxn * syn.  Scan temporaries: tile_scan_temp_ints(count) ints.
int64_t tile_scan_temp_ints(int T);
// (splat, super-tile) pair counts -> super_counts[NS], super_offsets[NS + 1];
// super_stats = {pairs, largest list, long-list count}, zero on entry.
// super_cm (kBinMaxBlocks x NS ints) receives the per-(workgroup,
// super-tile) key offsets that launch_bin_tiles places the keys at.
void launch_super_count(hipStream_t s, int n, int tiles_x, int tiles_y, const int *radii, const uint32_t *rect,
                        int *super_counts, int *super_offsets, int *super_cm, int *super_stats, int *temp);
constexpr int kBinMaxBlocks = 256;
// Scatter, per-super-tile sort, tile counts and offsets (tile_offsets[T + 1],
// tile_stats = {intersections, largest tile}, zero on entry) and the
// per-tile sorted gaussian ids.  When super_max > 4096 the long lists need
// super_keys_tmp (the size of super_keys) and merge_base[NS], and
// super_stats[3] receives their merge-tile count; when
// bin_chunk_parallel(super_max, NS) huge_list[NS], huge_stats[2] (zero on
// entry), chunk_base[NS] and chunk_counts[big_chunk_ints(total, NS)].
// total_keys = the pair count (super_stats[0]).
// The deep-tile scan launch_bin_tiles queues once the tile offsets exist
// (before the emission kernels): the tiles with at least `len` entries into
// `list`, their number into *count, copied to *host_count.
struct DeepScan {
    int len = 0;
    int *list = nullptr, *count = nullptr, *host_count = nullptr;
};
void launch_bin_tiles(hipStream_t s, int n, int tiles_x, int tiles_y, const int *radii, const uint32_t *rect,
                      const float *depths, const int *super_offsets, const int *super_cm, int super_max,
                      uint64_t *super_keys, uint64_t *super_keys_tmp, int *big_list, int *super_stats,
                      int *huge_list, int *huge_stats, int *chunk_base, int *chunk_counts, int *merge_base,
                      int total_keys, int *tile_counts, int *tile_offsets, int *tile_stats, int *tile_temp, int *ids,
                      bool force_wide_keys, const DeepScan *deep = nullptr);
constexpr int kSuperHugeList = 4 * 4096;
// Whether the super-tile lists above 4096 keys are sorted, counted and
// emitted chunk-parallel (k_sort_chunks, k_count_chunks, k_emit_chunks):
// when some list exceeds kSuperHugeList, which a workgroup would otherwise
// hold for several serial chunk sorts.  (Also taking that path for frames
// with few super-tiles, e.g. 294 at 1297x840, measured 1-3% slower steps:
// its extra launches cost more than the serial sorts of lists of <= 16k.)
inline bool bin_chunk_parallel(int super_max, int /*num_super*/) { return super_max > kSuperHugeList; }
// Ints of chunk_counts: 16 per 4096-key chunk of the long lists, at most
// total / 4096 + NS chunks.
inline int64_t big_chunk_ints(int64_t total_keys, int NS) { return (total_keys / 4096 + NS) * 16; }
constexpr int kSuperTile = 4;
constexpr int kSuperSortChunk = 4096;

// k_raster.hip
// blog (msr::BlendLog: a pool of 64-entry chunks of 16-byte entries with
// their 64-float checkpoints, the per-wave chunk table of
// msr::log_table_ints(I, T) ints, the per-wave counts [4T] and the chunk
// counter) receives the per-wave blend log and transmittance checkpoints the
// backward replays; pass nullptr for render-only frames.  full_outputs =
// false produces only out_img and final_Ts[.][0] (what the image-only
// training step consumes).
// Deep tiles (lists of at least len entries) are rendered pixel by pixel
// (k_raster_deep) instead of by one workgroup; list[0, n) are their tile
// indices (launch_deep_tiles), and with a blend log pos / tb / cnt hold
// their pixels' blended entries (deep_pixel_entries(n) ints / floats, and
// n * 256 counts), from which their wave logs are built.
struct DeepTiles {
    int n = 0, len = 0;
    const int *list = nullptr;
    int *pos = nullptr;
    float *tb = nullptr;
    int *cnt = nullptr;
    // the deep tiles run on `stream` between `fork` (recorded on the
    // caller's stream) and `join` (waited on by the caller's stream); with
    // defer_log the forward's `join` follows the deep tiles' outputs only
    // and their blend logs (k_deep_log) are rebuilt after it on `stream`,
    // where the raster backward's deep part follows them (the caller's
    // stream reaches them through the backward's `join`).  `logged` is
    // recorded on `stream` after every log rebuild; the backward's per-tile
    // part waits for it, so the rebuild's large workgroups are not starved
    // of CUs by the per-tile launch (which would delay the deep part behind
    // the whole per-tile backward)
    hipStream_t stream = nullptr;
    hipEvent_t fork = nullptr, join = nullptr, logged = nullptr;
    bool defer_log = false;
};
void launch_deep_tiles(hipStream_t s, int T, const int *offsets, int deep_len, int *deep_list, int *count);
int64_t deep_pixel_entries(int n_deep);
void launch_raster_fwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets, const int *ids,
                       const float *rec, const float *mrec, const float *bg, float *out_img, float *final_Ts, int *final_idx,
                       float *out_depth, float *out_normal, float *out_alpha, float *out_median, float *out_dist,
                       unsigned long long *pair_counter, const msr::BlendLog *blog, bool full_outputs,
                       const DeepTiles &deep);
// Returns true when the image-only kernel ran: grads16 then holds its sums
// (launch_finish_image_grads / launch_project_bwd finish them).
bool launch_raster_bwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets,
                       const msr::BlendLog &blog, const float *rec,
                       const float *bg, const float *final_Ts, const int *final_idx, const float *dL_dimg,
                       const float *dL_ddepth, const float *dL_daccum, const float *dL_dnormal,
                       const float *dL_dmedian, const float *dL_ddist, float ddist_uniform, float *grads16,
                       const DeepTiles &deep);
constexpr int kBlendLogEntryBytes = 16;

// k_raster3d.hip (3DGS mode): rec = the 3DGS records (kRec3Floats each),
// boxes = their quadrant-mask boxes.  blend_log / t_ckpt / wave_cnt as for
// launch_raster_fwd (nullptr: render only).  The backward adds the per-splat
// sums to grads16 (launch_finish3d_grads finishes them).
void launch_raster3d_fwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets, const int *ids,
                         const float *rec, const float *boxes, const float *bg, float *out_img, float *final_Ts,
                         const msr::BlendLog *blog);
void launch_raster3d_bwd(hipStream_t s, int W, int H, int tiles_x, int tiles_y, const int *offsets,
                         const msr::BlendLog &blog, const float *rec, const float *bg, const float *final_Ts,
                         const float *dL_dimg, float *grads16);
// Adds to *bad the number of floats of exponent field efield (1..254, both
// signs, every mantissa) where the rasterizer's fast reciprocal differs from
// the correctly rounded 1 / x.
void launch_check_rcp(hipStream_t s, int efield, unsigned long long *bad);

// k_ssim.hip
void launch_rgba8(hipStream_t s, const float *img, int64_t n, uint32_t *out);
int ssim_num_blocks(int W, int H);
// Loss partials (16 bytes each) that launch_loss_fwd_bwd writes, and whether
// it uses the three gradient maps gm1 / gs1 / gs12 (the two-pass form, for
// images too large for the one-kernel form's 32-bit offsets).
int loss_num_partials(int W, int H);
bool loss_needs_maps(int W, int H);
void set_loss_form(int form);  // 0: by size, 1: streaming, 2: two-pass (self-test hook)
void launch_loss_fwd_bwd(hipStream_t s, int W, int H, const float *img, const float *gt, const float *dist,
                         float lambda_l1, float lambda_dist, float lambda_dssim, const float window[11],
                         float *gm1, float *gs1, float *gs12, double *partials, double *loss_out,
                         float *dL_dimg);

// k_optim.hip
void launch_adam(hipStream_t s, float *p, const float *g, float *m, float *v, int64_t n, float step, float b1,
                 float b2, float bc2_sqrt, float eps);
void launch_clamp_max(hipStream_t s, float *p, int64_t n, float value);
// p[0, 4 * n_float4) = 0; p 16-byte aligned.
void launch_zero16(hipStream_t s, float *p, int64_t n_float4);
int64_t scan_temp_ints(int64_t n);
void launch_scan_i32(hipStream_t s, const int *in, int *out, int n, int *temp);

struct DensifyArgs {
    int n, fr_stride;
    int scale_dim;  // floats of scale per splat: 2 (surfels) or 3 (3D Gaussians)
    float grad_th, size_th, screen_th;
    int check_screen;
    float cull_alpha, cull_scale, cull_screen;
    int check_huge;
    const float *grad_norm, *vis, *max2d;
    float half_max_dim, log_size_fac;
    float *params[6], *exp_avg[6], *exp_avg_sq[6];
    float *workspace;  // densify_workspace_floats(n_virt, scale_dim, fr_stride) floats
    const float *random;
    int *split, *dup, *split_pre, *dup_pre, *scan_temp;
    int *keep, *keep_pre, *src_of;  // n_virt entries each
    int *parent;                    // n_virt - n entries
};
// Classification and the split / dup prefix counts (the count after
// appending is N + 2 * split_pre[N-1] + dup_pre[N-1]; a splat can be both).
void launch_densify_classify(hipStream_t s, const DensifyArgs &a);
// Keep flags of the old and appended rows, the gather of every surviving
// row into the workspace and its copy back into the caller's buffers.
// n_virt = n + 2 nS + nD (the count after appending) must fit the buffers'
// capacity; the new count is keep_pre[n_virt - 1].  Strides up to 127.
int64_t densify_workspace_floats(int n_virt, int scale_dim, int fr_stride);
void launch_densify_apply(hipStream_t s, const DensifyArgs &a, int nS, int n_virt);

// k_mesh.hip
// The compaction passes work on chunks of kMeshChunk cells / pixels: one
// uint32 count per chunk, scanned into mesh_chunks(n) + 1 uint64 offsets.
// The marching-cubes case bytes need mesh_chunks(cells) * kMeshChunk bytes.
constexpr int kMeshChunk = 4096;
inline int64_t mesh_chunks(int64_t n) { return (n + kMeshChunk - 1) / kMeshChunk; }
inline int64_t mc_num_cells(int nx, int ny, int nz) {
    return nx < 2 || ny < 2 || nz < 2 ? 0 : (int64_t)(nx - 1) * (ny - 1) * (nz - 1);
}
void mc_table_host(int8_t *tri);  // 256 x 16
// A view as the TSDF kernels read it: the caller's record plus its pass
// mask, 1 bit per pixel (alpha >= threshold, depth finite and positive),
// row-major, tsdf_mask_words(W) 32-bit words per row.
struct TsdfViewDev {
    MsplatTsdfView v;
    uint32_t *mask;
    int32_t words_per_row;
    int32_t pad_;
};
inline int tsdf_mask_words(int W) { return ((W + 63) / 64) * 2; }
// Builds every view's mask; max_segs = the largest H * ceil(W / 64).
void launch_tsdf_masks(hipStream_t s, const TsdfViewDev *views_dev, int nviews, int64_t max_segs, float athr);
void launch_tsdf_integrate(hipStream_t s, float *grid, int nx, int ny, int nz, const float origin[3], float vs,
                           const TsdfViewDev *views_dev, int nviews, float trunc);
void launch_mc_classify(hipStream_t s, const float *grid, int nx, int ny, int nz, uint8_t *cases,
                        uint32_t *chunk_tris);
void launch_chunk_scan(hipStream_t s, const uint32_t *counts, int64_t n, uint64_t *off);
void launch_mc_emit(hipStream_t s, const float *grid, int nx, int ny, int nz, const float origin[3], float vs,
                    const uint8_t *cases, const uint64_t *chunk_off, int64_t max_tris, float *out);
void launch_unproject_count(hipStream_t s, const float *img, const float *depth, const float *alpha, int W, int H,
                            float fx, float fy, float cx, float cy, const float c2w[16], float thr,
                            uint32_t *chunk_pts);
void launch_unproject_emit(hipStream_t s, const float *img, const float *depth, const float *alpha, int W, int H,
                           float fx, float fy, float cx, float cy, const float c2w[16], float thr,
                           const uint64_t *chunk_off, float *xyz, uint8_t *rgb);

}  // namespace mskern
