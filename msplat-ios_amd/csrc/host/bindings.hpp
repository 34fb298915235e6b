// bindings.hpp -- the engine interface the C++ Model programs against, with
// the names and argument meaning of the reference's core/metal/bindings.h
// (lines 7-158), implemented over the C-ABI launch layer (msplat_engine.h).
// viewmat / projmat may be host or device MTensors (4x4, row-major).
#pragma once

#include <tuple>
#include <vector>

#include "mtensor.hpp"

// bindings.h:7-25
void cleanup_msplat_metal();
MTensor gpu_zeros(std::vector<int64_t> shape, DType dtype);
MTensor gpu_empty(std::vector<int64_t> shape, DType dtype);
void msplat_commit();
void msplat_gpu_sync();
void msplat_enable_gpu_timing(bool enable);
void msplat_drain_gpu_times(std::vector<double> &out);

// bindings.h:36-42, 103-130
MTensor msplat_last_out_depth();
MTensor msplat_last_out_normal();
MTensor msplat_last_out_alpha();
MTensor msplat_last_out_median_depth();
MTensor msplat_last_out_distortion();
MTensor msplat_last_dL_dmean3D();
MTensor msplat_last_dL_dscale();
MTensor msplat_last_dL_dquat();
MTensor msplat_last_dL_dopacity();
MTensor msplat_last_dL_dfeatures_dc();
MTensor msplat_last_dL_dfeatures_rest();
MTensor msplat_last_dL_dmean2D();
MTensor msplat_last_radii();
MTensor msplat_last_dL_dcolors();
MTensor msplat_last_dL_dtransMat();
MTensor msplat_last_dL_dnormal3D();
MTensor msplat_last_out_img();
MTensor msplat_last_dL_dout_img();
MTensor msplat_last_final_idx();
MTensor msplat_last_final_Ts();
MTensor msplat_last_xys();
MTensor msplat_last_depths();
MTensor msplat_last_num_tiles_hit();

// bindings.h:47-62
std::tuple<MTensor, float> msplat_train_step_2dgs(
    int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats, MTensor &viewmat,
    MTensor &projmat, float fx, float fy, float cx, float cy, unsigned img_height, unsigned img_width,
    const std::tuple<int, int, int> tile_bounds, float clip_thresh, unsigned degree, unsigned degrees_to_use,
    float cam_pos[3], MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background,
    MTensor &gt, int features_rest_bases, float lambda_l1, float lambda_dist, float lambda_dssim,
    MTensor &xys_grad_norm, MTensor &vis_counts, MTensor &max_2d_size, float inv_max_dim);

// The same step with the six Adam updates fused into the projection
// backward (no counterpart in bindings.h; Model::fullIteration uses it).
std::tuple<MTensor, float> msplat_train_step_2dgs_adam(
    int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats, MTensor &viewmat,
    MTensor &projmat, float fx, float fy, float cx, float cy, unsigned img_height, unsigned img_width,
    const std::tuple<int, int, int> tile_bounds, float clip_thresh, unsigned degree, unsigned degrees_to_use,
    float cam_pos[3], MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background,
    MTensor &gt, int features_rest_bases, float lambda_l1, float lambda_dist, float lambda_dssim,
    MTensor &xys_grad_norm, MTensor &vis_counts, MTensor &max_2d_size, float inv_max_dim, MTensor exp_avg[6],
    MTensor exp_avg_sq[6], const float step_size[6], float beta1, float beta2, float bc2_sqrt, float eps);

// bindings.h:135-140
void msplat_fused_adam(MTensor &params, MTensor &grads, MTensor &exp_avg, MTensor &exp_avg_sq, uint32_t n,
                       float step_size, float beta1, float beta2, float bc2_sqrt, float eps);

// bindings.h:145-155
MTensor msplat_render(int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats,
                      MTensor &viewmat, MTensor &projmat, float fx, float fy, float cx, float cy,
                      unsigned img_height, unsigned img_width, const std::tuple<int, int, int> tile_bounds,
                      float clip_thresh, unsigned degree, unsigned degrees_to_use, float cam_pos[3],
                      MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background);

// The 3DGS mode (scales [N,3]; no counterpart in the fork, whose 3DGS step
// was removed, bindings.h:140): the render and the fused train step, with
// the arguments of msplat_render and msplat_train_step_2dgs_adam (no
// distortion weight).
MTensor msplat_render_3dgs(int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats,
                           MTensor &viewmat, MTensor &projmat, float fx, float fy, float cx, float cy,
                           unsigned img_height, unsigned img_width, const std::tuple<int, int, int> tile_bounds,
                           float clip_thresh, unsigned degree, unsigned degrees_to_use, float cam_pos[3],
                           MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background);
std::tuple<MTensor, float> msplat_train_step_3dgs_adam(
    int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats, MTensor &viewmat,
    MTensor &projmat, float fx, float fy, float cx, float cy, unsigned img_height, unsigned img_width,
    const std::tuple<int, int, int> tile_bounds, float clip_thresh, unsigned degree, unsigned degrees_to_use,
    float cam_pos[3], MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background,
    MTensor &gt, int features_rest_bases, float lambda_l1, float lambda_dssim, MTensor &xys_grad_norm,
    MTensor &vis_counts, MTensor &max_2d_size, float inv_max_dim, MTensor exp_avg[6], MTensor exp_avg_sq[6],
    const float step_size[6], float beta1, float beta2, float bc2_sqrt, float eps);

// bindings.h:143-158.  The flag / prefix / block / scratch tensors of the
// reference are accepted for signature compatibility; the engine keeps its
// own scratch.  The scale stride follows scales_buf's shape (the reference's
// kScaleDim): 2 for surfels, 3 for the 3DGS mode's Gaussians.
int msplat_densify(int N, int buf_capacity, float grad_thresh, float size_thresh, float screen_thresh,
                   int check_screen, float cull_alpha_thresh, float cull_scale_thresh, float cull_screen_size,
                   int check_huge, MTensor &xys_grad_norm, MTensor &vis_counts, MTensor &max_2d_size,
                   float half_max_dim, MTensor &means_buf, MTensor &scales_buf, MTensor &quats_buf,
                   MTensor &featuresDc_buf, MTensor &featuresRest_buf, MTensor &opacities_buf, int fr_stride,
                   MTensor adam_exp_avg_buf[], MTensor adam_exp_avg_sq_buf[], MTensor &split_flag,
                   MTensor &dup_flag, MTensor &split_prefix, MTensor &dup_prefix, MTensor &keep_flag,
                   MTensor &keep_prefix, MTensor &block_totals, MTensor &compact_scratch,
                   MTensor &random_samples);

// bindings.h:66-77: marching cubes on a device [Dz, Dy, Dx, 2] (sdf, weight)
// grid; `triangles` receives 9 floats per triangle (host), in cell order.
// Returns the number of triangles written (at most maxTriangles).
int64_t msplat_marching_cubes(MTensor &grid, int Dx, int Dy, int Dz, float origin_x, float origin_y, float origin_z,
                              float voxelSize, int maxTriangles, std::vector<float> &triangles);

// bindings.h:79-93: fold one rendered depth + alpha map into the grid.
void msplat_tsdf_integrate(MTensor &grid, int Dx, int Dy, int Dz, float origin_x, float origin_y, float origin_z,
                           float voxelSize, MTensor &viewmat, float fx, float fy, float cx, float cy, uint32_t imgW,
                           uint32_t imgH, float truncDist, float alphaThresh, MTensor &depthMap, MTensor &alphaMap);
