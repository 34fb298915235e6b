/*
 * golden.h -- CPU golden model (the oracle) of the msplat 2DGS training step.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is a scalar C++ restatement of the
 * reference's Metal kernels (core/metal/msplat_metal.metal) and their host
 * orchestration (core/metal/msplat_metal.mm, core/src/model.cpp).  It is
 * linked only by tests/, by __graft_entry__.smoke() and by bench.py's
 * cpu_baseline leg, always as the checker -- never by the product library.
 *
 * Arithmetic contract shared with the HIP kernels (so results can be compared
 * bit-for-bit where no float atomics are involved):
 *   - compiled with -ffp-contract=off; every fused multiply-add is an explicit
 *     fmaf() call;
 *   - '/' and sqrtf are IEEE correctly rounded; rsqrt is written 1/sqrtf;
 *   - exp is orc_expf (Cephes-style polynomial with Cody-Waite reduction),
 *     not libm, and the rasterizer's Gaussian falloff is orc_gauss
 *     (exp2 reduction + degree-6 polynomial + ldexp), so host and device
 *     agree exactly;
 *   - float->int truncation saturates (orc_f2i) instead of invoking UB.
 *
 * Deviations from the fork that the golden model takes deliberately (each is
 * the documented, deterministic intent of the fork's code):
 *   1. tiles are never truncated at 2048 entries (msplat_metal.metal:1581-1586
 *      drops an atomic-order-dependent subset);
 *   2. per-gaussian gradient sums are accumulated in fp64 in a fixed order
 *      (the fork uses float atomics, msplat_metal.metal:1879-1976);
 *   3. the rasterizer backward recomputes (u,v) with the forward's arithmetic
 *      (ray * (1/ray.z), msplat_metal.metal:680-682) so that it replays exactly
 *      the forward's skip decisions (the fork divides, :1826);
 *   4. densify compaction uses the 2-float scale stride (kScaleDim) for the
 *      scales buffer and its Adam state (msplat_metal.mm:1365 passes 3);
 *   5. split random samples are supplied by the caller (host generated).
 */
#ifndef MSPLAT_GOLDEN_H
#define MSPLAT_GOLDEN_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Camera set-up of Model::prepareCam (core/src/model.cpp:500-544). */
typedef struct {
    float viewmat[16];   /* world -> camera (OpenCV), row-major */
    float projmat[16];   /* world -> clip  (P * V), row-major  */
    float cam_pos[3];
    float fx, fy, cx, cy;
    int width, height;
    int tiles_x, tiles_y;
} OrcCamera;

void  orc_prepare_cam(const float cam_to_world[16], float fx, float fy,
                      float cx, float cy, int width, int height, OrcCamera *out);

float orc_expf(float x);
void  orc_expf_array(int64_t n, const float *x, float *y);
float orc_gauss(float rho);
void  orc_gauss_array(int64_t n, const float *rho, float *y);
void  orc_ssim_window(float w[11]);
int   orc_num_threads(void);

/* project_and_sh_forward_2dgs_kernel (msplat_metal.metal:1413-1521).
 * Culled gaussians get radii = 0 and zeros in every other output.
 * normal_opac = (normal.xyz, raw opacity logit); colors are raw SH output.
 * rect = (x0, y0, x1, y1) tile rectangle, x1/y1 exclusive. */
void orc_project_fwd(int n, const float *means, const float *scales,
                     const float *quats, const float *opacities,
                     const float *features_dc, const float *features_rest,
                     int degree, int degrees_to_use, const OrcCamera *cam,
                     float glob_scale, float clip_thresh,
                     float *xys, float *depths, int32_t *radii,
                     float *transmats, float *normal_opac, float *colors,
                     int32_t *tiles_hit, int32_t *rect);

/* Binning: per-tile intersection counts; returns the total I. */
int64_t orc_count_tiles(int n, const int32_t *radii, const int32_t *rect,
                        int tiles_x, int tiles_y, int32_t *tile_counts);
/* Per-tile lists sorted by key (float_bits(depth) << 32 | gaussian id),
 * i.e. scatter_to_prealloc_bins_kernel + prefix_sum_kernel +
 * bitonic_sort_per_tile_2dgs_kernel (msplat_metal.metal:1557-1690, 3093-3145)
 * without the 2048-entry truncation.  tile_offsets has tiles+1 entries
 * (exclusive scan); tile_bins (start,end) is tile_offsets[t], tile_offsets[t+1]. */
void orc_bin_sort(int n, const int32_t *radii, const int32_t *rect,
                  const float *depths, int tiles_x, int tiles_y,
                  const int32_t *tile_counts, int32_t *tile_offsets,
                  uint64_t *keys, int32_t *ids);

/* nd_rasterize_forward_2dgs_kernel (msplat_metal.metal:553-754). */
void orc_raster_fwd(const OrcCamera *cam, const int32_t *tile_offsets,
                    const int32_t *ids, const float *xys,
                    const float *transmats, const float *normal_opac,
                    const float *colors, const float *background,
                    float *out_img, float *final_Ts, int32_t *final_index,
                    float *out_depth, float *out_normal, float *out_alpha,
                    float *out_median_depth, float *out_distortion,
                    int64_t *pairs_evaluated);

/* SSIM (11-tap, sigma 1.5, zero pad) + L1 (+ distortion) loss forward and
 * backward: ssim_* kernels, loss_l1_distortion_2dgs_kernel and
 * ssim_backward_* (msplat_metal.metal:2704-3085) in the order of
 * msplat_metal.mm:1077-1212.  dL_dimg is overwritten; the return value is the
 * scalar loss (fp64 sum); *ssim_sum receives the fp64 sum of the SSIM map. */
double orc_loss_fwd_bwd(int width, int height, const float *img,
                        const float *gt, const float *distortion,
                        float lambda_l1, float lambda_dist,
                        float lambda_dssim, float *dL_dimg,
                        float *dL_ddistortion, double *ssim_sum);

/* nd_rasterize_backward_2dgs_kernel (msplat_metal.metal:1705-1979).
 * grads is [N,16] = (dL_dtransMat[9], dL_dnormal3D[3], dL_dopacity_logit,
 * dL_dcolors[3]), accumulated in fp64 in a fixed order and stored as float.
 * grads_abs (nullable, [N,16]) receives per component the sum of the
 * magnitudes of its summands: the scale of a float summation's error. */
void orc_raster_bwd(const OrcCamera *cam, int n, const int32_t *tile_offsets,
                    const int32_t *ids, const float *xys,
                    const float *transmats, const float *normal_opac,
                    const float *colors, const float *background,
                    const float *final_Ts, const int32_t *final_index,
                    const float *dL_dimg, const float *dL_ddepth,
                    const float *dL_dalpha, const float *dL_dnormal,
                    const float *dL_dmedian, const float *dL_ddistortion,
                    float *grads, float *grads_abs);

/* project_and_sh_backward_2dgs_kernel (msplat_metal.metal:2003-2209).
 * grads16 is the [N,16] raster-gradient record above.  xys_grad_norm,
 * vis_counts and max_2d_size are read-modify-write. */
void orc_project_bwd(int n, const float *means, const float *scales,
                     const float *quats, const float *features_rest,
                     int degree, int degrees_to_use, const OrcCamera *cam,
                     float glob_scale, const int32_t *radii,
                     const float *grads16, float *dL_dmeans,
                     float *dL_dscales, float *dL_dquats,
                     float *dL_dmean2d, float *dL_dfeatures_dc,
                     float *dL_dfeatures_rest, float *xys_grad_norm,
                     float *vis_counts, float *max_2d_size,
                     float inv_max_dim);

/* fused_adam_kernel (msplat_metal.metal:1383-1406). */
void orc_adam(float *params, const float *grads, float *exp_avg,
              float *exp_avg_sq, int64_t n, float step_size, float beta1,
              float beta2, float bc2_sqrt, float eps);

/* GPU densification of msplat_densify (msplat_metal.mm:1339-1594) with the
 * kernels of msplat_metal.metal:3231-3491.  Buffers are capacity-sized
 * backing buffers: params[6] = means(3), scales(2), quats(4), features_dc(3),
 * features_rest(fr_stride), opacities(1); exp_avg[6] / exp_avg_sq[6] the same
 * strides.  random_samples is [2N,3].  Returns the new gaussian count, or
 * minus the rows needed (nothing modified) when the appended count exceeds
 * capacity. */
int orc_densify(int n, int capacity, float grad_thresh, float size_thresh,
                float screen_thresh, int check_screen,
                float cull_alpha_thresh, float cull_scale_thresh,
                float cull_screen_size, int check_huge,
                const float *xys_grad_norm, const float *vis_counts,
                const float *max_2d_size, float half_max_dim,
                float *const params[6], int fr_stride,
                float *const exp_avg[6], float *const exp_avg_sq[6],
                const float *random_samples);
/* The same with 3 scales per splat (the 3DGS mode): scales stride 3, split
 * children sampled along all three axes. */
int orc_densify_3dgs(int n, int capacity, float grad_thresh, float size_thresh,
                     float screen_thresh, int check_screen,
                     float cull_alpha_thresh, float cull_scale_thresh,
                     float cull_screen_size, int check_huge,
                     const float *xys_grad_norm, const float *vis_counts,
                     const float *max_2d_size, float half_max_dim,
                     float *const params[6], int fr_stride,
                     float *const exp_avg[6], float *const exp_avg_sq[6],
                     const float *random_samples);

/* Optional intermediate results of orc_train_step, for comparing a whole
 * step stage by stage (test instrumentation): arrays are malloc'd by the
 * golden model and released with orc_free.  want_grads also fills grads16
 * and grads16_abs (see orc_raster_bwd). */
typedef struct {
    int want_grads;
    int64_t num_isect;
    int32_t *tile_offsets; /* [T+1] */
    int32_t *ids;          /* [I]   */
    float *grads16;        /* [N,16] */
    float *grads16_abs;    /* [N,16] */
} OrcStepDetail;

/* Timing helper for the CPU baseline: one full training step (forward,
 * SSIM+L1, backward, six Adam groups) in place on the given parameters.
 * adam_lr[6], bc1, bc2 as Model::fullIteration (model.cpp:767-826).
 * stage_ms (optional, 8 entries) receives per-stage wall times. */
double orc_train_step(int n, float *means, float *scales, float *quats,
                      float *opacities, float *features_dc,
                      float *features_rest, int degree, int degrees_to_use,
                      const OrcCamera *cam, const float *background,
                      const float *gt, float ssim_weight,
                      float *const exp_avg[6], float *const exp_avg_sq[6],
                      const float adam_lr[6], int adam_step,
                      float *xys_grad_norm, float *vis_counts,
                      float *max_2d_size, float *out_img, double *stage_ms,
                      int64_t *num_intersections, OrcStepDetail *detail);

/* Frees an array the golden model handed out (OrcStepDetail). */
void orc_free(void *p);

/* tsdf_integrate_kernel (msplat_metal.metal:2223-2280): folds one depth
 * view into the [dz, dy, dx, 2] (sdf, weight) grid in place. */
void orc_tsdf_integrate(float *grid, int dx, int dy, int dz, const float origin[3],
                        float voxel_size, const float viewmat[16], float fx, float fy,
                        float cx, float cy, int width, int height, float trunc_dist,
                        float alpha_thresh, const float *depth, const float *alpha);

/* marching_cubes_kernel (msplat_metal.metal:2606-2687) with the case table
 * `table` (256 x 16 edge indices, -1 terminated), cells visited in linear
 * order (x fastest); the first max_triangles triangles are written to out
 * (9 floats each).  Returns the number of triangles the grid produces. */
int64_t orc_marching_cubes(const float *grid, int dx, int dy, int dz,
                           const float origin[3], float voxel_size,
                           const int8_t *table, int64_t max_triangles, float *out);

/* The unprojection loop of Model::exportPointCloud (model.cpp:580-616) for
 * one view: xyz [H*W,3], rgb [H*W,3]; returns the number of points. */
int64_t orc_unproject_depth(const float *img, const float *depth, const float *alpha,
                            int width, int height, float fx, float fy, float cx,
                            float cy, const float cam_to_world[16], float alpha_thresh,
                            float *xyz, uint8_t *rgb);

#ifdef __cplusplus
}
#endif

#endif
