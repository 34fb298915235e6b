/*
 * msplat_engine.h -- C-ABI launch layer of the MI355X (gfx950) engine.
 *
 * This is the boundary between the C++ host (MTensor / Model / Trainer, the
 * public C API in msplat_c_api.h) and the hand-written HIP kernels.  It
 * replaces the reference's internal engine interface
 * core/metal/bindings.h:7-158 (plain C++ functions taking MTensor&) with
 * extern "C" entry points that take plain device pointers and sizes, so a
 * cgo / ctypes / JNI caller can bind it directly.
 *
 * Conventions
 *  - All pointers named *_dev are device pointers (hipMalloc memory, e.g.
 *    from msplat_hip_alloc).  Host pointers are named *_host.
 *  - Every entry point returns 0 on success and a negative MSPLAT_E_* code
 *    on failure; msplat_hip_last_error() gives the message.  No C++
 *    exception crosses this boundary.
 *  - All work runs in order on the engine's single HIP stream (the
 *    reference's serial dispatch queue, msplat_metal.mm:182,732).  Entry
 *    points are asynchronous unless documented otherwise.
 *  - One engine per process (the reference's g_tcache,
 *    msplat_metal.mm:538): intermediate buffers are cached and reused.
 */
#ifndef MSPLAT_ENGINE_H
#define MSPLAT_ENGINE_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSPLAT_OK 0
#define MSPLAT_E_HIP (-1)       /* a HIP runtime call failed            */
#define MSPLAT_E_ARG (-2)       /* invalid argument / shape             */
#define MSPLAT_E_NOMEM (-3)     /* device allocation failed             */
#define MSPLAT_E_NODEV (-4)     /* no usable gfx950 device              */
#define MSPLAT_E_CAPACITY (-5)  /* caller-provided capacity too small   */

#define MSPLAT_TILE 16          /* BLOCK_X / BLOCK_Y, core/include/msplat.hpp:4-5 */
/* Per-gaussian splat record, 5 x float4: (Tu.xyz, Tv.x), (Tv.yz, Tw.xy),
 * (Tw.z, x, y, sigmoid(opacity)), (normal.xyz, r), (g, b, tau, lp_r2);
 * rgb = max(SH + 0.5, 0), tau = the largest rho at which alpha can still
 * reach 1/255 (-1 if never), lp_r2 = squared radius of its low-pass disc as
 * the quadrant masks use it. */
#define MSPLAT_REC_FLOATS 20
#define MSPLAT_GRAD_FLOATS 16   /* per-gaussian raster-gradient record       */

/* Camera + projection set-up: the arguments of msplat_train_step_2dgs /
 * msplat_render (bindings.h:47-62, 145-155) that Model::prepareCam
 * (core/src/model.cpp:500-544) computes. */
typedef struct {
    float viewmat[16];   /* world -> camera, row-major                   */
    float projmat[16];   /* world -> clip (P*V), row-major               */
    float cam_pos[3];
    float fx, fy, cx, cy;
    int32_t width, height;
    int32_t tiles_x, tiles_y;
    float glob_scale;    /* 1.0 in Model (model.cpp:550,782)             */
    float clip_thresh;   /* 0.01 in Model                                */
    int32_t degree;      /* SH degree of the features_rest layout        */
    int32_t degrees_to_use;
} MsplatCamera;

/* The six parameter groups (Model::means ... opacities, model.hpp:81-86)
 * as device pointers: means[N,3], scales[N,2] (log), quats[N,4] (w,x,y,z),
 * opacities[N] (logit), features_dc[N,3], features_rest[N,K,3]. */
typedef struct {
    int32_t num_points;
    float *means;
    float *scales;
    float *quats;
    float *opacities;
    float *features_dc;
    float *features_rest;
} MsplatGaussians;

/* Adam state and step sizes for the six groups (model.cpp:806-826). */
typedef struct {
    float *exp_avg[6];
    float *exp_avg_sq[6];
    float step_size[6];  /* lr[g] / (1 - beta1^t)                        */
    float beta1, beta2;
    float bc2_sqrt;      /* sqrt(1 - beta2^t)                            */
    float eps;
} MsplatAdam;

/* Model::prepareCam (core/src/model.cpp:500-544) without the downscale:
 * viewmat = inverse of camToWorld after negating its columns 1 and 2
 * (OpenGL -> OpenCV), projmat = P(fovX, fovY, near 0.001, far 1000) * V,
 * cam_pos = translation, tiles = ceil(W/16) x ceil(H/16).  Host only. */
int msplat_hip_prepare_camera(const float cam_to_world[16], float fx, float fy,
                              float cx, float cy, int width, int height,
                              int degree, int degrees_to_use,
                              MsplatCamera *out);

/* ---- context, memory, stream (bindings.h:7-25) -------------------------- */

/* Creates the engine (device 0, one stream).  Idempotent.  Replaces the
 * lazily created MetalContext (msplat_metal.mm:287-293). */
int msplat_hip_init(void);
/* Releases every cached buffer: cleanup_msplat_metal (bindings.h:8). */
void msplat_hip_cleanup(void);
const char *msplat_hip_last_error(void);
/* Device name / gfx arch of the engine's device into buf. */
int msplat_hip_device_name(char *buf, int len);

/* gpu_empty / gpu_zeros (bindings.h:17-18). */
void *msplat_hip_alloc(size_t bytes);
int msplat_hip_free(void *ptr_dev);
int msplat_hip_memset(void *ptr_dev, int value, size_t bytes);
int msplat_hip_upload(void *dst_dev, const void *src_host, size_t bytes);
int msplat_hip_download(void *dst_host, const void *src_dev, size_t bytes);
int msplat_hip_copy(void *dst_dev, const void *src_dev, size_t bytes);
/* msplat_commit (bindings.h:21): work is already queued; returns at once. */
int msplat_hip_commit(void);
/* msplat_gpu_sync (bindings.h:24): waits for the engine stream. */
int msplat_hip_sync(void);

/* ---- the training step and render path ---------------------------------- */

/* msplat_train_step_2dgs (bindings.h:47-62): projection + SH, tile binning,
 * per-tile depth sort, rasterize forward, SSIM + L1 loss forward/backward,
 * rasterize backward, projection + SH backward.  Synchronous (reads the
 * loss back, like msplat_metal.mm:1328-1330).
 *  - gt_dev is the [H,W,3] target image;
 *  - xys_grad_norm/vis_counts/max_2d_size are [N] densify statistics,
 *    read-modify-write (model.cpp:771-775);
 *  - adam == NULL: per-group gradients are written to the engine cache
 *    (msplat_hip_last) for msplat_hip_fused_adam, as the reference does;
 *  - adam != NULL: the six Adam updates are fused into the projection
 *    backward and applied to g in place (no gradient tensors are written).
 *  *loss_host receives the scalar loss; *num_isect_host (nullable) the
 *  tile-intersection count. */
int msplat_hip_train_step(const MsplatCamera *cam, const MsplatGaussians *g,
                          const float *background_dev, const float *gt_dev,
                          float lambda_l1, float lambda_dist,
                          float lambda_dssim, float *xys_grad_norm_dev,
                          float *vis_counts_dev, float *max_2d_size_dev,
                          float inv_max_dim, const MsplatAdam *adam,
                          float *loss_host, int64_t *num_isect_host);

/* msplat_render (bindings.h:145-155): forward only; outputs in the cache
 * (MSPLAT_LAST_OUT_IMG etc.).  Asynchronous apart from one mid-pipeline
 * read of the intersection count. */
int msplat_hip_render(const MsplatCamera *cam, const MsplatGaussians *g,
                      const float *background_dev, int64_t *num_isect_host);

/* The RGBA8 conversion of Trainer::renderFromPoseToBuffer
 * (core/src/msplat_api.mm:207-236, a host loop there): (uint8)(clamp(x, 0,
 * 1) * 255) per channel, truncating, alpha 255, computed on the GPU from the
 * [num_pixels,3] image img_dev; the 4-byte pixels are copied to rgba_host.
 * Synchronous. */
int msplat_hip_image_to_rgba8(const float *img_dev, int64_t num_pixels,
                              uint8_t *rgba_host);

/* msplat_fused_adam (bindings.h:135-140): one Adam step on n floats. */
int msplat_hip_fused_adam(float *params_dev, const float *grads_dev,
                          float *exp_avg_dev, float *exp_avg_sq_dev,
                          int64_t n, float step_size, float beta1,
                          float beta2, float bc2_sqrt, float eps);

/* msplat_densify (bindings.h:143-158): classify, append split/dup children,
 * cull, stable compaction of the 18 capacity-sized buffers.  params[6],
 * exp_avg[6], exp_avg_sq[6] are the backing buffers (strides 3, 2, 4, 3,
 * fr_stride, 1); random_samples_dev is [2N,3].  Synchronous; returns the
 * new count in *new_count_host.  The count after appending is N + 2 * splits
 * + dups, up to 4N (a splat small in the world but wide on screen is both
 * split and duplicated); when it exceeds capacity nothing is modified,
 * *new_count_host receives the rows needed and MSPLAT_E_CAPACITY is
 * returned, so the caller can grow the buffers and call again (the
 * reference assumes 3N, msplat_metal.mm:1358, and overruns). */
int msplat_hip_densify(int n, int capacity, float grad_thresh,
                       float size_thresh, float screen_thresh,
                       int check_screen, float cull_alpha_thresh,
                       float cull_scale_thresh, float cull_screen_size,
                       int check_huge, const float *xys_grad_norm_dev,
                       const float *vis_counts_dev,
                       const float *max_2d_size_dev, float half_max_dim,
                       float *const params_dev[6], int fr_stride,
                       float *const exp_avg_dev[6],
                       float *const exp_avg_sq_dev[6],
                       const float *random_samples_dev, int *new_count_host);

/* p[i] = min(p[i], value) on n floats: the opacity reset of Model::afterTrain
 * (core/src/model.cpp:290-296), a host loop on unified memory there. */
int msplat_hip_clamp_max(float *p_dev, int64_t n, float value);

/* ---- stage entry points (each one kernel of the step) -------------------- */

/* ssim_* + loss_l1_distortion_2dgs + ssim_backward_* kernels
 * (msplat_metal.metal:2704-3085) fused into two passes.  dL_dimg_dev
 * [H,W,3] is overwritten; distortion_dev may be NULL when lambda_dist == 0.
 * Synchronous (reads the loss). */
int msplat_hip_loss_fwd_bwd(int width, int height, const float *img_dev,
                            const float *gt_dev, const float *distortion_dev,
                            float lambda_l1, float lambda_dist,
                            float lambda_dssim, float *dL_dimg_dev,
                            double *loss_host, double *ssim_sum_host);

/* msplat_hip_loss_fwd_bwd without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (tight
 * serving loops, harnesses that forbid hipMalloc).  It is not capturable
 * in a HIP graph: it reads the loss back into pinned host memory and
 * synchronises the engine stream.  The scratch it needs lives in a fixed device array of the
 * library (about 77 MB per GPU, held until the process ends): images up to
 * 2^21 pixels (e.g. 2048x1024, 1920x1080); larger ones return
 * MSPLAT_E_CAPACITY.  msplat_hip_init must have run (this call does no
 * set-up).  Results are bit-identical to msplat_hip_loss_fwd_bwd.  Every
 * call on a GPU shares that GPU's scratch: calls are serialised by the
 * engine's lock and stream, and anything that ran these kernels
 * concurrently on that array would race.  Synchronous. */
int msplat_hip_loss_fwd_bwd_noalloc(int width, int height, const float *img_dev,
                                    const float *gt_dev,
                                    const float *distortion_dev,
                                    float lambda_l1, float lambda_dist,
                                    float lambda_dssim, float *dL_dimg_dev,
                                    double *loss_host, double *ssim_sum_host);

/* nd_rasterize_backward_2dgs (msplat_metal.metal:1705-1979) on the forward
 * state of the most recent render / train step.  Per-pixel upstream
 * gradients [H,W,{3,1}] may be NULL (zero).  grads16_dev [N,16] is
 * accumulated into (caller zeroes it): dL_dtransMat[9], dL_dnormal3D[3],
 * dL_dopacity (logit), dL_dcolors[3]. */
int msplat_hip_raster_bwd(const float *dL_dimg_dev, const float *dL_ddepth_dev,
                          const float *dL_dalpha_dev,
                          const float *dL_dnormal_dev,
                          const float *dL_dmedian_dev,
                          const float *dL_ddistortion_dev, float *grads16_dev);

/* project_and_sh_backward_2dgs (msplat_metal.metal:2003-2209) on explicit
 * inputs (radii from the forward, grads16 from the raster backward).
 * Outputs [N,3],[N,2],[N,4],[N,2],[N,3],[N,K,3] are overwritten; the three
 * densify statistics are read-modify-write. */
int msplat_hip_project_bwd(const MsplatCamera *cam, const MsplatGaussians *g,
                           const int32_t *radii_dev, const float *grads16_dev,
                           float *dL_dmeans_dev, float *dL_dscales_dev,
                           float *dL_dquats_dev, float *dL_dmean2d_dev,
                           float *dL_dfeatures_dc_dev,
                           float *dL_dfeatures_rest_dev,
                           float *xys_grad_norm_dev, float *vis_counts_dev,
                           float *max_2d_size_dev, float inv_max_dim);

/* The projection backward above with the six Adam updates fused in
 * (Model::fullIteration's Adam loop, core/src/model.cpp:806-826, applied in
 * registers): g's parameters and adam's moments are updated in place and no
 * gradient tensor is written.  Bit-identical to msplat_hip_project_bwd
 * followed by msplat_hip_fused_adam on each group. */
int msplat_hip_project_bwd_adam(const MsplatCamera *cam,
                                const MsplatGaussians *g,
                                const int32_t *radii_dev,
                                const float *grads16_dev,
                                float *xys_grad_norm_dev,
                                float *vis_counts_dev, float *max_2d_size_dev,
                                float inv_max_dim, const MsplatAdam *adam);

/* ---- cached buffers (the msplat_last_* accessors, bindings.h:36-42,
 *      bindings.h:103-130) ------------------------------------------------ */
enum {
    MSPLAT_LAST_XYS = 0,          /* [N,2]  f32 (materialised)           */
    MSPLAT_LAST_DEPTHS,           /* [N]    f32                          */
    MSPLAT_LAST_RADII,            /* [N]    i32                          */
    MSPLAT_LAST_NUM_TILES_HIT,    /* [N]    i32 (materialised)           */
    MSPLAT_LAST_TRANSMATS,        /* [N,9]  f32 (materialised)           */
    MSPLAT_LAST_COLORS_USED,      /* [N,3]  f32 max(raw+0.5,0) (mat.)    */
    MSPLAT_LAST_OPACITY_SIGMOID,  /* [N]    f32 (materialised)           */
    MSPLAT_LAST_NORMALS,          /* [N,3]  f32 (materialised)           */
    MSPLAT_LAST_RECORDS,          /* [N,20] f32 splat records            */
    MSPLAT_LAST_TILE_OFFSETS,     /* [T+1]  i32                          */
    MSPLAT_LAST_GAUSSIAN_IDS,     /* [I]    i32 sorted per tile          */
    MSPLAT_LAST_OUT_IMG,          /* [H,W,3] f32                         */
    MSPLAT_LAST_FINAL_TS,         /* [H,W,3] f32 (T, M1, M2)             */
    MSPLAT_LAST_FINAL_IDX,        /* [H,W,2] i32 (last, median)          */
    MSPLAT_LAST_OUT_DEPTH,        /* [H,W]  f32                          */
    MSPLAT_LAST_OUT_NORMAL,       /* [H,W,3] f32                         */
    MSPLAT_LAST_OUT_ALPHA,        /* [H,W]  f32                          */
    MSPLAT_LAST_OUT_MEDIAN_DEPTH, /* [H,W]  f32                          */
    MSPLAT_LAST_OUT_DISTORTION,   /* [H,W]  f32                          */
    MSPLAT_LAST_DL_DOUT_IMG,      /* [H,W,3] f32                         */
    MSPLAT_LAST_GRADS16,          /* [N,16] f32 raster gradients         */
    MSPLAT_LAST_DL_DTRANSMAT,     /* [N,9]  f32 (materialised)           */
    MSPLAT_LAST_DL_DNORMAL3D,     /* [N,3]  f32 (materialised)           */
    MSPLAT_LAST_DL_DOPACITY,      /* [N]    f32 (materialised)           */
    MSPLAT_LAST_DL_DCOLORS,       /* [N,3]  f32 (materialised)           */
    MSPLAT_LAST_DL_DMEAN3D,       /* [N,3]  f32 (unfused step only)      */
    MSPLAT_LAST_DL_DSCALE,        /* [N,2]                               */
    MSPLAT_LAST_DL_DQUAT,         /* [N,4]                               */
    MSPLAT_LAST_DL_DMEAN2D,       /* [N,2]                               */
    MSPLAT_LAST_DL_DFEATURES_DC,  /* [N,3]                               */
    MSPLAT_LAST_DL_DFEATURES_REST,/* [N,K,3]                             */
    MSPLAT_LAST_BLEND_LOG,        /* [C,64,4] u32 blend-log pool chunks  */
    MSPLAT_LAST_BLEND_CKPT,       /* [C,64] f32 their checkpoints        */
    MSPLAT_LAST_WAVE_COUNTS,      /* [T,4]  i32 entries per wave log     */
    MSPLAT_LAST_BLEND_CHUNKS,     /* i32 per-wave chunk tables           */
    MSPLAT_LAST_COUNT
};
/* Returns the device pointer and element count of a cached buffer (NULL /
 * 0 if it does not exist yet).  Materialised entries are gathered from the
 * packed records on each call (asynchronously, on the engine stream).  The
 * raster gradients (GRADS16, DL_DTRANSMAT, DL_DNORMAL3D, DL_DOPACITY,
 * DL_DCOLORS) are those of the most recent train step and exist until the
 * next forward.  BLEND_LOG / BLEND_CKPT / WAVE_COUNTS / BLEND_CHUNKS are
 * the rasterizer's per-wave blend logs in a pool of C chunks of 64 entries
 * {ballot low, ballot high, list position, gaussian id}: wave w of tile t
 * (list offset s, length n) has WAVE_COUNTS[4t + w] entries, its entries
 * 64k .. 64k + 63 in chunk BLEND_CHUNKS[(4 s + w n) / 64 + 4t + w + k],
 * whose 64 checkpoint floats are each lane's transmittance before entry
 * 64 (k + 1).  They exist once the training forward or a backward's replay
 * ran on the current tile lists (a test accessor, no counterpart in the
 * reference). */
int msplat_hip_last(int which, void **ptr_dev, int64_t *numel);

/* Per-kernel timings of the most recent train step / render, in ms, from
 * HIP events recorded on the engine stream when MSPLAT_TIMING_EVENTS is set
 * (the PROFILE_GPU hooks of msplat_metal.mm:20-23).  names receives up to
 * max entries of static strings.  MSPLAT_TIMING_PAIRS additionally counts
 * the (pixel, gaussian) pairs the forward rasterizer evaluates, which costs
 * one atomic per wave and tile. */
enum { MSPLAT_TIMING_EVENTS = 1, MSPLAT_TIMING_PAIRS = 2 };
int msplat_hip_enable_timing(int flags);
int msplat_hip_stage_times(const char **names, float *ms, int max);
/* Pair counter of the most recent forward run with MSPLAT_TIMING_PAIRS. */
int64_t msplat_hip_last_pairs_evaluated(void);
/* Counters of the same forward: out[0] = (pixel, gaussian) pairs evaluated,
 * out[1] = blend-log entries (visits of a wave in which at least one pixel
 * blended the gaussian; 0 for a forward without the log), out[2] =
 * (pixel, gaussian) pairs blended, out[3] = (wave, gaussian) visits,
 * out[4] = visit slots (per 256-entry batch, four times the largest wave's
 * visit count: the visits the batch's barriers allow for); all zero after
 * a 3DGS forward.  No counterpart in the reference: it measures the
 * rasterizers' work. */
int msplat_hip_last_raster_counts(int64_t out[5]);
/* Self-check of the rasterizer's arithmetic: *mismatches receives the
 * number of floats with exponent field efield_lo..efield_hi (1..254, both
 * signs, every mantissa) where the fast reciprocal it uses for 1 / ray.z
 * (hardware reciprocal + one Newton step) differs from the correctly rounded
 * division.  Zero is required for efield 1..252 (|x| in [2^-126, 2^126));
 * the rasterizer divides outside that range.  msplat_hip_init runs it over
 * [1, 2) and fails on a mismatch.  No counterpart in the reference. */
int msplat_hip_check_fast_rcp(int efield_lo, int efield_hi, int64_t *mismatches);
/* Binning self-test hook.  Below 2^24 gaussians the per-super-tile sort keys
 * carry each gaussian's rectangle inside the super-tile (depth bits << 32 |
 * id << 8 | rectangle); from 2^24 on they are depth bits << 32 | id and the
 * rectangle is gathered.  on != 0 forces the wide layout at any size, so the
 * tests can check it against the golden model on small scenes; the tile
 * lists are the same either way.  No counterpart in the reference. */
int msplat_hip_set_wide_keys(int on);
/* Rasterizer self-test hook.  Tiles whose list holds at least len entries
 * are rendered pixel by pixel, each 2x2 pixel block on its own wave, instead
 * of by one workgroup per tile; the outputs, blend log and checkpoints are
 * the same either way.  A small len sends ordinary tiles down that path, so
 * the tests can check it on small scenes; len <= 0 restores the default
 * (lists of at least 4096 entries and 4x the frame's mean list).  No
 * counterpart in the reference. */
int msplat_hip_set_deep_tile_len(int len);
/* Loss self-test hook.  The SSIM + L1 loss has two forms with the same
 * dL/dimage bit for bit: one streaming kernel, used for images of about
 * 4.7 MP and more (row segments of at least 128 rows) whose byte offsets fit
 * in 32 bits (up to ~89 MP), and two tiled passes through three gradient
 * maps otherwise.  form 1 forces the streaming form wherever it fits, form
 * 2 the two-pass form, 0 restores the choice by size, so the tests can
 * check both against the golden model on small images.  No counterpart in
 * the reference. */
int msplat_hip_set_loss_form(int form);
/* Blend-log pool self-test hook.  A frame's pool holds `chunks` chunks of
 * 64 entries instead of the size estimated from its intersection count, or
 * more once an overflow grew it: a step whose log overflows the pool
 * changes nothing and is redone after the pool doubles (up to a size no log
 * overflows), so a tiny pool exercises that path with the same results.
 * Drops the grown size; chunks <= 0 restores the estimate.  No counterpart
 * in the reference. */
int msplat_hip_set_log_pool_chunks(int chunks);
/* Blend-log pool counters: out[0] = chunks in the current frame's pool,
 * out[1] = chunks the last forward that logged claimed (0 once the log is
 * stale), out[2] = overflowed logs (steps and replays redone) since init,
 * out[3] = the most chunks the frame's logs could take, out[4] = device
 * bytes the pool's buffers hold (chunks, checkpoints, chunk tables,
 * counts).  A frame's pool holds 1.25 times the largest share of a static
 * estimate (one chunk per 96 intersections plus one per wave) that a log
 * claimed so far, or more after an overflow.  Waits for the engine stream.
 * No counterpart in the reference. */
int msplat_hip_log_pool_stats(int64_t out[5]);

/* ---- 3DGS mode ------------------------------------------------------------
 * 3D Gaussians (scales [N,3], log) projected with the reference's EWA
 * helpers (scale_rot_to_cov3d, project_cov3d_ewa, compute_cov2d_bounds,
 * project_pix: core/metal/msplat_metal.metal:152-459, VJPs :1059-1374,
 * dead code in the 2DGS fork) and composited with the 3DGS pair rule in the
 * fork's blending conventions.  The fork removed its 3DGS step
 * (msplat_train_step, bindings.h:140); these are its replacement.  The
 * binning, the loss and the densification statistics are the 2DGS path's.
 * Outputs: MSPLAT_LAST_OUT_IMG and MSPLAT_LAST_FINAL_TS (first component);
 * after a train step, MSPLAT_LAST_GRADS16 holds per splat [dL/dxy 2,
 * dL/dconic 3, dL/dopacity logit, dL/dcolor 3] in its first 9 floats.
 * Gaussians carry MsplatGaussians' layouts except scales [N,3]. */
int msplat_hip_render_3dgs(const MsplatCamera *cam, const MsplatGaussians *g, const float *background_dev,
                           int64_t *num_isect_host);
/* One 3DGS training step: forward with the blend log, SSIM + L1 (no
 * distortion term), backward, projection backward; adam non-null fuses
 * the six Adam updates (scales [N,3]), NULL leaves the parameter gradients
 * in the MSPLAT_LAST_DL_* buffers (DL_DSCALE [N,3]). */
int msplat_hip_train_step_3dgs(const MsplatCamera *cam, const MsplatGaussians *g, const float *background_dev,
                               const float *gt_dev, float lambda_l1, float lambda_dssim, float *xys_grad_norm_dev,
                               float *vis_counts_dev, float *max_2d_size_dev, float inv_max_dim,
                               const MsplatAdam *adam, float *loss_host, int64_t *num_isect_host);
/* msplat_hip_densify for 3D Gaussians: the reference's densify kernels at
 * kScaleDim = 3 (msplat_metal.metal:3253-3255, :3315-3317, :3339-3341):
 * scales stride 3, the largest of three scales classifies and culls, split
 * children are sampled along all three axes.  Same arguments, capacity
 * contract and results otherwise. */
int msplat_hip_densify_3dgs(int n, int capacity, float grad_thresh,
                            float size_thresh, float screen_thresh,
                            int check_screen, float cull_alpha_thresh,
                            float cull_scale_thresh, float cull_screen_size,
                            int check_huge, const float *xys_grad_norm_dev,
                            const float *vis_counts_dev,
                            const float *max_2d_size_dev, float half_max_dim,
                            float *const params_dev[6], int fr_stride,
                            float *const exp_avg_dev[6],
                            float *const exp_avg_sq_dev[6],
                            const float *random_samples_dev, int *new_count_host);

/* ---- mesh extraction: TSDF fusion, marching cubes, depth unprojection ----
 * The voxel grid is [Dz, Dy, Dx, 2] f32 (sdf, weight) in HBM, voxel (x, y, z)
 * centred at origin + voxel_size * (index + 0.5) (Model::VoxelGrid,
 * core/include/model.hpp:51-56). */

/* One depth view of msplat_hip_tsdf_integrate: the per-camera inputs of
 * tsdf_integrate_kernel (core/metal/msplat_metal.metal:2223-2234). */
typedef struct {
    float viewmat[16];       /* world -> camera (OpenCV), row-major         */
    float fx, fy, cx, cy;    /* intrinsics at the depth map's resolution    */
    int32_t width, height;   /* of the depth and alpha maps                 */
    const float *depth_dev;  /* [H,W] surface depth (median depth)          */
    const float *alpha_dev;  /* [H,W] accumulated alpha                     */
} MsplatTsdfView;

/* msplat_tsdf_integrate (bindings.h:82-93, msplat_metal.mm:836-881) for
 * num_views views at once: every voxel folds the views in array order,
 * which is what num_views successive single-view calls (the reference's
 * loop, model.cpp:723-757) compute, reading and writing the grid once.
 * views is host memory.  Synchronous: the call returns when the grid is
 * updated (the next call rewrites the engine's copies of the view records
 * and pass masks), so the depth / alpha maps may be released after it. */
int msplat_hip_tsdf_integrate(float *grid_dev, int dx, int dy, int dz, const float origin[3],
                              float voxel_size, const MsplatTsdfView *views, int num_views,
                              float trunc_dist, float alpha_thresh);

/* msplat_marching_cubes (bindings.h:66-77, msplat_metal.mm:790-834): one
 * triangle list (9 floats per triangle, world space, non-indexed) from the
 * grid; cells with a corner of weight <= 0 are skipped.  Triangles come in
 * cell order (x fastest, then y, then z), each cell's in case-table order,
 * so the output is deterministic; the first max_triangles of them are
 * written to tris_dev [max_triangles, 9].  *num_triangles = the number
 * written (the reference's return value), *num_emitted (optional) = the
 * number the grid produces.  Synchronous. */
int msplat_hip_marching_cubes(const float *grid_dev, int dx, int dy, int dz, const float origin[3],
                              float voxel_size, int64_t max_triangles, float *tris_dev,
                              int64_t *num_triangles, int64_t *num_emitted);

/* The case table msplat_hip_marching_cubes uses (256 rows of 16 edge
 * indices, 3 per triangle, -1 terminated; edges and corners numbered as
 * msplat_metal.metal:2594-2604), generated from the corner signs; host
 * only, no device needed. */
int msplat_hip_mc_table(int8_t tri[256 * 16]);

/* The unprojection of Model::exportPointCloud (core/src/model.cpp:565-640,
 * a host loop there) for one rendered view: every pixel with alpha >=
 * alpha_thresh and finite positive depth / alpha gives one world-space
 * point (the OpenCV ray through the pixel centre, rotated by camToWorld
 * with columns 1 and 2 negated) and its colour (uint8)(clamp(rgb * 255, 0,
 * 255)).  Points come in pixel order (row-major).  xyz_dev [H*W, 3] and
 * rgb_dev [H*W, 3] have room for every pixel; *num_points = points written.
 * Synchronous. */
int msplat_hip_unproject_depth(const float *img_dev, const float *depth_dev, const float *alpha_dev,
                               int width, int height, float fx, float fy, float cx, float cy,
                               const float cam_to_world[16], float alpha_thresh, float *xyz_dev,
                               uint8_t *rgb_dev, int64_t *num_points);

#ifdef __cplusplus
}
#endif

#endif
