// bindings.cpp -- C++ engine interface over the C-ABI launch layer.
#include "bindings.hpp"

#include <algorithm>
#include <cstdint>
#include <cstring>
#include <stdexcept>
#include <string>

namespace {

void check(int rc) {
    if (rc != MSPLAT_OK) throw std::runtime_error(std::string("msplat engine: ") + msplat_hip_last_error());
}

void host_copy16(MTensor &m, float out[16]) {
    if (m.numel() != 16) throw std::invalid_argument("view/projection matrix must have 16 elements");
    if (m.isGpu())
        m.copy_to_host(out);
    else
        std::memcpy(out, m.data_ptr(), 16 * sizeof(float));
}

MsplatCamera make_camera(MTensor &viewmat, MTensor &projmat, float fx, float fy, float cx, float cy,
                         unsigned H, unsigned W, const std::tuple<int, int, int> &tb, float clip_thresh,
                         float glob_scale, unsigned degree, unsigned dtu, const float cam_pos[3]) {
    MsplatCamera c{};
    host_copy16(viewmat, c.viewmat);
    host_copy16(projmat, c.projmat);
    for (int i = 0; i < 3; ++i) c.cam_pos[i] = cam_pos[i];
    c.fx = fx;
    c.fy = fy;
    c.cx = cx;
    c.cy = cy;
    c.width = (int32_t)W;
    c.height = (int32_t)H;
    c.tiles_x = std::get<0>(tb);
    c.tiles_y = std::get<1>(tb);
    c.glob_scale = glob_scale;
    c.clip_thresh = clip_thresh;
    c.degree = (int32_t)degree;
    c.degrees_to_use = (int32_t)dtu;
    return c;
}

MsplatGaussians make_gaussians(int n, MTensor &m, MTensor &s, MTensor &q, MTensor &o, MTensor &dc, MTensor &fr) {
    MsplatGaussians g{};
    g.num_points = n;
    g.means = m.data<float>();
    g.scales = s.data<float>();
    g.quats = q.data<float>();
    g.opacities = o.data<float>();
    g.features_dc = dc.data<float>();
    g.features_rest = fr.defined() ? fr.data<float>() : nullptr;
    return g;
}

MTensor last(int which, std::vector<int64_t> shape, DType dt) {
    void *p = nullptr;
    int64_t n = 0;
    check(msplat_hip_last(which, &p, &n));
    if (!p) return MTensor();
    int64_t want = 1;
    for (auto d : shape) want *= d;
    if (want != n) shape = {n};
    return MTensor::wrap_device(p, shape, dt);
}

int g_n = 0, g_H = 0, g_W = 0, g_K = 0;

}  // namespace

void cleanup_msplat_metal() { msplat_hip_cleanup(); }
MTensor gpu_empty(std::vector<int64_t> shape, DType dtype) { return MTensor::device(std::move(shape), dtype); }
MTensor gpu_zeros(std::vector<int64_t> shape, DType dtype) {
    MTensor t = MTensor::device(std::move(shape), dtype);
    t.zero();
    return t;
}
void msplat_commit() { check(msplat_hip_commit()); }
void msplat_gpu_sync() { check(msplat_hip_sync()); }
void msplat_enable_gpu_timing(bool enable) { check(msplat_hip_enable_timing(enable ? 1 : 0)); }
void msplat_drain_gpu_times(std::vector<double> &out) {
    const char *names[16];
    float ms[16];
    int k = msplat_hip_stage_times(names, ms, 16);
    double tot = 0.0;
    for (int i = 0; i < k; ++i) tot += ms[i];
    if (k) out.push_back(tot);
}

MTensor msplat_last_out_depth() { return last(MSPLAT_LAST_OUT_DEPTH, {g_H, g_W}, DType::Float32); }
MTensor msplat_last_out_normal() { return last(MSPLAT_LAST_OUT_NORMAL, {g_H, g_W, 3}, DType::Float32); }
MTensor msplat_last_out_alpha() { return last(MSPLAT_LAST_OUT_ALPHA, {g_H, g_W}, DType::Float32); }
MTensor msplat_last_out_median_depth() { return last(MSPLAT_LAST_OUT_MEDIAN_DEPTH, {g_H, g_W}, DType::Float32); }
MTensor msplat_last_out_distortion() { return last(MSPLAT_LAST_OUT_DISTORTION, {g_H, g_W}, DType::Float32); }
MTensor msplat_last_dL_dmean3D() { return last(MSPLAT_LAST_DL_DMEAN3D, {g_n, 3}, DType::Float32); }
MTensor msplat_last_dL_dscale() { return last(MSPLAT_LAST_DL_DSCALE, {g_n, 2}, DType::Float32); }
MTensor msplat_last_dL_dquat() { return last(MSPLAT_LAST_DL_DQUAT, {g_n, 4}, DType::Float32); }
MTensor msplat_last_dL_dopacity() { return last(MSPLAT_LAST_DL_DOPACITY, {g_n, 1}, DType::Float32); }
MTensor msplat_last_dL_dfeatures_dc() { return last(MSPLAT_LAST_DL_DFEATURES_DC, {g_n, 3}, DType::Float32); }
MTensor msplat_last_dL_dfeatures_rest() {
    return last(MSPLAT_LAST_DL_DFEATURES_REST, {g_n, g_K, 3}, DType::Float32);
}
MTensor msplat_last_dL_dmean2D() { return last(MSPLAT_LAST_DL_DMEAN2D, {g_n, 2}, DType::Float32); }
MTensor msplat_last_radii() { return last(MSPLAT_LAST_RADII, {g_n}, DType::Int32); }
MTensor msplat_last_dL_dcolors() { return last(MSPLAT_LAST_DL_DCOLORS, {g_n, 3}, DType::Float32); }
MTensor msplat_last_dL_dtransMat() { return last(MSPLAT_LAST_DL_DTRANSMAT, {g_n, 9}, DType::Float32); }
MTensor msplat_last_dL_dnormal3D() { return last(MSPLAT_LAST_DL_DNORMAL3D, {g_n, 3}, DType::Float32); }
MTensor msplat_last_out_img() { return last(MSPLAT_LAST_OUT_IMG, {g_H, g_W, 3}, DType::Float32); }
MTensor msplat_last_dL_dout_img() { return last(MSPLAT_LAST_DL_DOUT_IMG, {g_H, g_W, 3}, DType::Float32); }
MTensor msplat_last_final_idx() { return last(MSPLAT_LAST_FINAL_IDX, {g_H, g_W, 2}, DType::Int32); }
MTensor msplat_last_final_Ts() { return last(MSPLAT_LAST_FINAL_TS, {g_H, g_W, 3}, DType::Float32); }
MTensor msplat_last_xys() { return last(MSPLAT_LAST_XYS, {g_n, 2}, DType::Float32); }
MTensor msplat_last_depths() { return last(MSPLAT_LAST_DEPTHS, {g_n}, DType::Float32); }
MTensor msplat_last_num_tiles_hit() { return last(MSPLAT_LAST_NUM_TILES_HIT, {g_n}, DType::Int32); }

static std::tuple<MTensor, float> train_step_impl(
    int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats, MTensor &viewmat,
    MTensor &projmat, float fx, float fy, float cx, float cy, unsigned H, unsigned W,
    const std::tuple<int, int, int> tb, float clip_thresh, unsigned degree, unsigned dtu, float cam_pos[3],
    MTensor &fdc, MTensor &frest, MTensor &opac, MTensor &bg, MTensor &gt, int frBases, float l1, float ldist,
    float ldssim, MTensor &gnorm, MTensor &vis, MTensor &max2d, float inv_max_dim, const MsplatAdam *adam) {
    MsplatCamera cam = make_camera(viewmat, projmat, fx, fy, cx, cy, H, W, tb, clip_thresh, glob_scale, degree, dtu,
                                   cam_pos);
    MsplatGaussians g = make_gaussians(num_points, means3d, scales, quats, opac, fdc, frest);
    float loss = 0.f;
    check(msplat_hip_train_step(&cam, &g, bg.data<float>(), gt.data<float>(), l1, ldist, ldssim,
                                gnorm.data<float>(), vis.data<float>(), max2d.data<float>(), inv_max_dim, adam, &loss,
                                nullptr));
    g_n = num_points;
    g_H = (int)H;
    g_W = (int)W;
    g_K = frBases;
    return {msplat_last_radii(), loss};
}

std::tuple<MTensor, float> msplat_train_step_2dgs(
    int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats, MTensor &viewmat,
    MTensor &projmat, float fx, float fy, float cx, float cy, unsigned img_height, unsigned img_width,
    const std::tuple<int, int, int> tile_bounds, float clip_thresh, unsigned degree, unsigned degrees_to_use,
    float cam_pos[3], MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background,
    MTensor &gt, int features_rest_bases, float lambda_l1, float lambda_dist, float lambda_dssim,
    MTensor &xys_grad_norm, MTensor &vis_counts, MTensor &max_2d_size, float inv_max_dim) {
    return train_step_impl(num_points, means3d, scales, glob_scale, quats, viewmat, projmat, fx, fy, cx, cy,
                           img_height, img_width, tile_bounds, clip_thresh, degree, degrees_to_use, cam_pos,
                           features_dc, features_rest, opacities, background, gt, features_rest_bases, lambda_l1,
                           lambda_dist, lambda_dssim, xys_grad_norm, vis_counts, max_2d_size, inv_max_dim, nullptr);
}

std::tuple<MTensor, float> msplat_train_step_2dgs_adam(
    int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats, MTensor &viewmat,
    MTensor &projmat, float fx, float fy, float cx, float cy, unsigned img_height, unsigned img_width,
    const std::tuple<int, int, int> tile_bounds, float clip_thresh, unsigned degree, unsigned degrees_to_use,
    float cam_pos[3], MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background,
    MTensor &gt, int features_rest_bases, float lambda_l1, float lambda_dist, float lambda_dssim,
    MTensor &xys_grad_norm, MTensor &vis_counts, MTensor &max_2d_size, float inv_max_dim, MTensor exp_avg[6],
    MTensor exp_avg_sq[6], const float step_size[6], float beta1, float beta2, float bc2_sqrt, float eps) {
    MsplatAdam a{};
    for (int k = 0; k < 6; ++k) {
        a.exp_avg[k] = exp_avg[k].data<float>();
        a.exp_avg_sq[k] = exp_avg_sq[k].data<float>();
        a.step_size[k] = step_size[k];
    }
    a.beta1 = beta1;
    a.beta2 = beta2;
    a.bc2_sqrt = bc2_sqrt;
    a.eps = eps;
    return train_step_impl(num_points, means3d, scales, glob_scale, quats, viewmat, projmat, fx, fy, cx, cy,
                           img_height, img_width, tile_bounds, clip_thresh, degree, degrees_to_use, cam_pos,
                           features_dc, features_rest, opacities, background, gt, features_rest_bases, lambda_l1,
                           lambda_dist, lambda_dssim, xys_grad_norm, vis_counts, max_2d_size, inv_max_dim, &a);
}

void msplat_fused_adam(MTensor &params, MTensor &grads, MTensor &exp_avg, MTensor &exp_avg_sq, uint32_t n,
                       float step_size, float beta1, float beta2, float bc2_sqrt, float eps) {
    check(msplat_hip_fused_adam(params.data<float>(), grads.data<float>(), exp_avg.data<float>(),
                                exp_avg_sq.data<float>(), (int64_t)n, step_size, beta1, beta2, bc2_sqrt, eps));
}

MTensor msplat_render(int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats,
                      MTensor &viewmat, MTensor &projmat, float fx, float fy, float cx, float cy,
                      unsigned img_height, unsigned img_width, const std::tuple<int, int, int> tile_bounds,
                      float clip_thresh, unsigned degree, unsigned degrees_to_use, float cam_pos[3],
                      MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background) {
    MsplatCamera cam = make_camera(viewmat, projmat, fx, fy, cx, cy, img_height, img_width, tile_bounds,
                                   clip_thresh, glob_scale, degree, degrees_to_use, cam_pos);
    MsplatGaussians g = make_gaussians(num_points, means3d, scales, quats, opacities, features_dc, features_rest);
    check(msplat_hip_render(&cam, &g, background.data<float>(), nullptr));
    g_n = num_points;
    g_H = (int)img_height;
    g_W = (int)img_width;
    return msplat_last_out_img();
}

MTensor msplat_render_3dgs(int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats,
                           MTensor &viewmat, MTensor &projmat, float fx, float fy, float cx, float cy,
                           unsigned img_height, unsigned img_width, const std::tuple<int, int, int> tile_bounds,
                           float clip_thresh, unsigned degree, unsigned degrees_to_use, float cam_pos[3],
                           MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background) {
    MsplatCamera cam = make_camera(viewmat, projmat, fx, fy, cx, cy, img_height, img_width, tile_bounds,
                                   clip_thresh, glob_scale, degree, degrees_to_use, cam_pos);
    MsplatGaussians g = make_gaussians(num_points, means3d, scales, quats, opacities, features_dc, features_rest);
    check(msplat_hip_render_3dgs(&cam, &g, background.data<float>(), nullptr));
    g_n = num_points;
    g_H = (int)img_height;
    g_W = (int)img_width;
    return msplat_last_out_img();
}

std::tuple<MTensor, float> msplat_train_step_3dgs_adam(
    int num_points, MTensor &means3d, MTensor &scales, float glob_scale, MTensor &quats, MTensor &viewmat,
    MTensor &projmat, float fx, float fy, float cx, float cy, unsigned img_height, unsigned img_width,
    const std::tuple<int, int, int> tile_bounds, float clip_thresh, unsigned degree, unsigned degrees_to_use,
    float cam_pos[3], MTensor &features_dc, MTensor &features_rest, MTensor &opacities, MTensor &background,
    MTensor &gt, int features_rest_bases, float lambda_l1, float lambda_dssim, MTensor &xys_grad_norm,
    MTensor &vis_counts, MTensor &max_2d_size, float inv_max_dim, MTensor exp_avg[6], MTensor exp_avg_sq[6],
    const float step_size[6], float beta1, float beta2, float bc2_sqrt, float eps) {
    MsplatAdam a{};
    for (int k = 0; k < 6; ++k) {
        a.exp_avg[k] = exp_avg[k].data<float>();
        a.exp_avg_sq[k] = exp_avg_sq[k].data<float>();
        a.step_size[k] = step_size[k];
    }
    a.beta1 = beta1;
    a.beta2 = beta2;
    a.bc2_sqrt = bc2_sqrt;
    a.eps = eps;
    MsplatCamera cam = make_camera(viewmat, projmat, fx, fy, cx, cy, img_height, img_width, tile_bounds,
                                   clip_thresh, glob_scale, degree, degrees_to_use, cam_pos);
    MsplatGaussians g = make_gaussians(num_points, means3d, scales, quats, opacities, features_dc, features_rest);
    float loss = 0.f;
    check(msplat_hip_train_step_3dgs(&cam, &g, background.data<float>(), gt.data<float>(), lambda_l1, lambda_dssim,
                                     xys_grad_norm.data<float>(), vis_counts.data<float>(), max_2d_size.data<float>(),
                                     inv_max_dim, &a, &loss, nullptr));
    g_n = num_points;
    g_H = (int)img_height;
    g_W = (int)img_width;
    g_K = features_rest_bases;
    return {msplat_last_radii(), loss};
}

int msplat_densify(int N, int buf_capacity, float grad_thresh, float size_thresh, float screen_thresh,
                   int check_screen, float cull_alpha_thresh, float cull_scale_thresh, float cull_screen_size,
                   int check_huge, MTensor &xys_grad_norm, MTensor &vis_counts, MTensor &max_2d_size,
                   float half_max_dim, MTensor &means_buf, MTensor &scales_buf, MTensor &quats_buf,
                   MTensor &featuresDc_buf, MTensor &featuresRest_buf, MTensor &opacities_buf, int fr_stride,
                   MTensor adam_exp_avg_buf[], MTensor adam_exp_avg_sq_buf[], MTensor &, MTensor &, MTensor &,
                   MTensor &, MTensor &, MTensor &, MTensor &, MTensor &, MTensor &random_samples) {
    float *params[6] = {means_buf.data<float>(), scales_buf.data<float>(), quats_buf.data<float>(),
                        featuresDc_buf.data<float>(), featuresRest_buf.data<float>(), opacities_buf.data<float>()};
    float *m[6], *v[6];
    for (int k = 0; k < 6; ++k) {
        m[k] = adam_exp_avg_buf[k].data<float>();
        v[k] = adam_exp_avg_sq_buf[k].data<float>();
    }
    int new_count = 0;
    const int sd = scales_buf.ndim() == 2 ? (int)scales_buf.size(1) : 2;
    if (sd != 2 && sd != 3) throw std::invalid_argument("densify: scales_buf must be [capacity, 2] or [capacity, 3]");
    const int rc = (sd == 3 ? msplat_hip_densify_3dgs : msplat_hip_densify)(N, buf_capacity, grad_thresh, size_thresh, screen_thresh, check_screen,
                                      cull_alpha_thresh, cull_scale_thresh, cull_screen_size, check_huge,
                                      xys_grad_norm.data<float>(), vis_counts.data<float>(),
                                      max_2d_size.data<float>(), half_max_dim, params, fr_stride, m, v,
                                      random_samples.data<float>(), &new_count);
    // the buffers are too small for the appended splats: nothing was
    // modified; the negated row count tells the caller what to grow to
    if (rc == MSPLAT_E_CAPACITY) return -new_count;
    check(rc);
    return new_count;
}

int64_t msplat_marching_cubes(MTensor &grid, int Dx, int Dy, int Dz, float origin_x, float origin_y, float origin_z,
                              float voxelSize, int maxTriangles, std::vector<float> &triangles) {
    if (!grid.isGpu() || grid.numel() != (int64_t)Dx * Dy * Dz * 2)
        throw std::invalid_argument("marching cubes: grid must be a device [Dz, Dy, Dx, 2] tensor");
    const float origin[3] = {origin_x, origin_y, origin_z};
    const int64_t cap = std::max(maxTriangles, 0);
    MTensor out = MTensor::device({std::max<int64_t>(cap, 1), 9}, DType::Float32);
    int64_t written = 0;
    check(msplat_hip_marching_cubes(grid.data<float>(), Dx, Dy, Dz, origin, voxelSize, cap, out.data<float>(),
                                    &written, nullptr));
    triangles.resize((size_t)written * 9);
    if (written > 0) check(msplat_hip_download(triangles.data(), out.data_ptr(), (size_t)written * 36));
    return written;
}

void msplat_tsdf_integrate(MTensor &grid, int Dx, int Dy, int Dz, float origin_x, float origin_y, float origin_z,
                           float voxelSize, MTensor &viewmat, float fx, float fy, float cx, float cy, uint32_t imgW,
                           uint32_t imgH, float truncDist, float alphaThresh, MTensor &depthMap, MTensor &alphaMap) {
    if (!grid.isGpu() || grid.numel() != (int64_t)Dx * Dy * Dz * 2)
        throw std::invalid_argument("TSDF: grid must be a device [Dz, Dy, Dx, 2] tensor");
    if (!depthMap.isGpu() || !alphaMap.isGpu() || depthMap.numel() < (int64_t)imgW * imgH ||
        alphaMap.numel() < (int64_t)imgW * imgH)
        throw std::invalid_argument("TSDF: depth / alpha must be device [H, W] maps");
    MsplatTsdfView v{};
    host_copy16(viewmat, v.viewmat);
    v.fx = fx;
    v.fy = fy;
    v.cx = cx;
    v.cy = cy;
    v.width = (int32_t)imgW;
    v.height = (int32_t)imgH;
    v.depth_dev = depthMap.data<float>();
    v.alpha_dev = alphaMap.data<float>();
    const float origin[3] = {origin_x, origin_y, origin_z};
    check(msplat_hip_tsdf_integrate(grid.data<float>(), Dx, Dy, Dz, origin, voxelSize, &v, 1, truncDist,
                                    alphaThresh));
}
