// model.cpp -- Model: initialisation from a point cloud, Adam groups,
// capacity management, the densification schedule and checkpoints
// (core/src/model.cpp:45-498, 762-829 of the reference).
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>
#include <iostream>
#include <random>
#include <stdexcept>

void check_copy(MTensor &dst, const MTensor &src);

namespace {

constexpr double kC0 = 0.28209479177387814;
constexpr uint32_t kCkptMagic = 0x4C50534D;  // "MSPL"
constexpr uint32_t kCkptVersion = 1;

MTensor upload(std::vector<int64_t> shape, const float *src) {
    MTensor t = MTensor::device(std::move(shape), DType::Float32);
    t.copy_from_host(src, t.nbytes());
    return t;
}

// Backing buffer of `cap` rows holding `src` in its first rows, zero after.
MTensor backing(const MTensor &src, int cap) {
    std::vector<int64_t> shape = src.shape();
    shape[0] = cap;
    MTensor buf = gpu_zeros(shape, DType::Float32);
    if (src.nbytes()) check_copy(buf, src);
    return buf;
}

}  // namespace

int numShBases(int degree) {
    switch (degree) {
        case 0: return 1;
        case 1: return 4;
        case 2: return 9;
        case 3: return 16;
        default: return 25;
    }
}

Model::Model(const InputData &inputData, int numCameras, int numDownscales, int resolutionSchedule, int shDegree,
             int shDegreeInterval, int refineEvery, int warmupLength, int resetAlphaEvery, float densifyGradThresh,
             float densifySizeThresh, int stopScreenSizeAt, float splitScreenSize, int maxSteps, bool keepCrs,
             const float *bgColor, int scaleDim)
    : scaleDim(scaleDim),
      numCameras(numCameras),
      numDownscales(numDownscales),
      resolutionSchedule(resolutionSchedule),
      shDegree(shDegree),
      shDegreeInterval(shDegreeInterval),
      refineEvery(refineEvery),
      warmupLength(warmupLength),
      resetAlphaEvery(resetAlphaEvery),
      stopSplitAt(maxSteps - 500),
      densifyGradThresh(densifyGradThresh),
      densifySizeThresh(densifySizeThresh),
      stopScreenSizeAt(stopScreenSizeAt),
      splitScreenSize(splitScreenSize),
      maxSteps(maxSteps),
      keepCrs(keepCrs) {
    if (shDegree < 0 || shDegree > 4) throw std::invalid_argument("sh_degree must be in [0, 4]");
    if (scaleDim != 2 && scaleDim != 3) throw std::invalid_argument("scaleDim must be 2 (2DGS) or 3 (3DGS)");
    if (refineEvery <= 0 || resetAlphaEvery <= 0 || shDegreeInterval <= 0 || resolutionSchedule <= 0)
        throw std::invalid_argument("refine_every, reset_alpha_every, sh_degree_interval and resolution_schedule "
                                    "must be positive");
    const int64_t n = inputData.points.count;
    if ((int64_t)inputData.points.xyz.size() < 3 * n || (int64_t)inputData.points.rgb.size() < 3 * n)
        throw std::invalid_argument("point cloud arrays are shorter than its count");
    scale = inputData.scale;
    std::memcpy(translation, inputData.translation, sizeof(translation));

    means = upload({n, 3}, inputData.points.xyz.data());
    {
        const std::vector<float> d = knnMeanDistance(inputData.points.xyz.data(), n, 3);
        std::vector<float> s((size_t)n * scaleDim);
        for (int64_t i = 0; i < n; ++i)
            for (int k = 0; k < scaleDim; ++k) s[i * scaleDim + k] = std::log(d[i]);
        scales = upload({n, (int64_t)scaleDim}, s.data());
    }
    {
        // uniformly random rotations (model.cpp:79-93)
        std::mt19937 rng(42);
        std::uniform_real_distribution<float> uni(0.0f, 1.0f);
        std::vector<float> q((size_t)n * 4);
        for (int64_t i = 0; i < n; ++i) {
            const float u = uni(rng), v = uni(rng), w = uni(rng);
            q[4 * i + 0] = std::sqrt(1 - u) * std::sin(2 * M_PI * v);
            q[4 * i + 1] = std::sqrt(1 - u) * std::cos(2 * M_PI * v);
            q[4 * i + 2] = std::sqrt(u) * std::sin(2 * M_PI * w);
            q[4 * i + 3] = std::sqrt(u) * std::cos(2 * M_PI * w);
        }
        quats = upload({n, 4}, q.data());
    }
    const int dimSh = numShBases(shDegree);
    {
        std::vector<float> dc((size_t)n * 3);
        for (int64_t i = 0; i < 3 * n; ++i) dc[i] = (float)((inputData.points.rgb[i] / 255.0 - 0.5) / kC0);
        featuresDc = upload({n, 3}, dc.data());
        featuresRest = gpu_zeros({n, (int64_t)(dimSh - 1), 3}, DType::Float32);
    }
    {
        std::vector<float> o((size_t)n, std::log(0.1f / 0.9f));
        opacities = upload({n, 1}, o.data());
    }
    static const float kDefaultBg[3] = {0.6130f, 0.0101f, 0.3984f};
    backgroundColor = upload({3}, bgColor ? bgColor : kDefaultBg);
    setupOptimizers();
}

void check_copy(MTensor &dst, const MTensor &src) {
    if (src.nbytes() > dst.nbytes()) throw std::runtime_error("copy exceeds destination");
    if (!src.nbytes()) return;
    if (src.isGpu()) {
        if (msplat_hip_copy(dst.data_ptr(), src.data_ptr(), src.nbytes()) != MSPLAT_OK)
            throw std::runtime_error(std::string("msplat engine: ") + msplat_hip_last_error());
    } else {
        dst.copy_from_host(src.data_ptr(), src.nbytes());
    }
}

void Model::setupOptimizers() {
    releaseOptimizers();
    num_active = (int)means.size(0);
    buf_capacity = std::max(num_active * 4, 16);
    means_buf = backing(means, buf_capacity);
    scales_buf = backing(scales, buf_capacity);
    quats_buf = backing(quats, buf_capacity);
    featuresDc_buf = backing(featuresDc, buf_capacity);
    featuresRest_buf = backing(featuresRest, buf_capacity);
    opacities_buf = backing(opacities, buf_capacity);
    static constexpr float kLrInit[N_ADAM_GROUPS] = {0.00016f, 0.005f, 0.001f, 0.0025f, 0.000125f, 0.05f};
    const MTensor *params[N_ADAM_GROUPS] = {&means, &scales, &quats, &featuresDc, &featuresRest, &opacities};
    for (int g = 0; g < N_ADAM_GROUPS; ++g) {
        std::vector<int64_t> shape = params[g]->shape();
        shape[0] = buf_capacity;
        adam_exp_avg_buf[g] = gpu_zeros(shape, DType::Float32);
        adam_exp_avg_sq_buf[g] = gpu_zeros(shape, DType::Float32);
        adam_lr[g] = kLrInit[g];
    }
    adam_step_count = 0;
    means_lr_init = 0.00016f;
    means_lr_final = 0.0000016f;
    densify_random_samples = gpu_zeros({(int64_t)buf_capacity, 3}, DType::Float32);
    refreshViews();
}

void Model::releaseOptimizers() {
    for (int g = 0; g < N_ADAM_GROUPS; ++g) {
        adam_exp_avg[g].reset();
        adam_exp_avg_sq[g].reset();
        adam_exp_avg_buf[g].reset();
        adam_exp_avg_sq_buf[g].reset();
    }
    means_buf.reset();
    scales_buf.reset();
    quats_buf.reset();
    featuresDc_buf.reset();
    featuresRest_buf.reset();
    opacities_buf.reset();
    densify_random_samples.reset();
}

// Log-linear decay of the means learning rate over maxSteps
// (model.cpp:183-186).
void Model::schedulersStep(int step) {
    const float t = std::clamp((float)step / (float)maxSteps, 0.f, 1.f);
    adam_lr[0] = std::exp(std::log(means_lr_init) * (1.f - t) + std::log(means_lr_final) * t);
}

void Model::refreshViews() {
    means = means_buf.view(num_active);
    scales = scales_buf.view(num_active);
    quats = quats_buf.view(num_active);
    featuresDc = featuresDc_buf.view(num_active);
    featuresRest = featuresRest_buf.view(num_active);
    opacities = opacities_buf.view(num_active);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) {
        adam_exp_avg[g] = adam_exp_avg_buf[g].view(num_active);
        adam_exp_avg_sq[g] = adam_exp_avg_sq_buf[g].view(num_active);
    }
}

// Grows every backing buffer to max(needed, 2 x capacity) rows, keeping
// the first num_active rows (model.cpp:201-233).
void Model::ensureCapacity(int needed) {
    if (needed <= buf_capacity) return;
    const int cap = std::max(needed, buf_capacity * 2);
    auto grow = [&](MTensor &buf) {
        std::vector<int64_t> shape = buf.shape();
        shape[0] = cap;
        MTensor nb = gpu_zeros(shape, DType::Float32);
        MTensor live = buf.view(num_active);
        check_copy(nb, live);
        buf = nb;
    };
    grow(means_buf);
    grow(scales_buf);
    grow(quats_buf);
    grow(featuresDc_buf);
    grow(featuresRest_buf);
    grow(opacities_buf);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) {
        grow(adam_exp_avg_buf[g]);
        grow(adam_exp_avg_sq_buf[g]);
    }
    densify_random_samples = gpu_zeros({(int64_t)cap, 3}, DType::Float32);
    buf_capacity = cap;
    refreshViews();
}

int Model::getDownscaleFactor(int step) {
    const int remaining = numDownscales - step / resolutionSchedule;
    return 1 << std::max(remaining, 0);
}

void Model::allocStats(int n) {
    xysGradNorm = gpu_zeros({(int64_t)n}, DType::Float32);
    visCounts = gpu_zeros({(int64_t)n}, DType::Float32);
    max2DSize = gpu_zeros({(int64_t)n}, DType::Float32);
}

// Densify / prune / opacity-reset schedule (model.cpp:240-306).
void Model::afterTrain(int step) {
    if (!radii.defined()) return;
    if (!(step % refineEvery == 0 && step > warmupLength)) return;
    const int resetInterval = resetAlphaEvery * refineEvery;
    const bool capacityOk = num_active < maxSplats;
    const bool doDensification =
        step < stopSplitAt && step % resetInterval > numCameras + refineEvery && capacityOk;
    if (doDensification && xysGradNorm.defined()) {
        const int before = num_active;
        ensureCapacity(3 * num_active);
        {
            // normal samples of the split offsets, drawn on the host from
            // mt19937(step) as the reference does (model.cpp:258-263)
            std::mt19937 rng(step);
            std::normal_distribution<float> nd(0.0f, 1.0f);
            std::vector<float> r((size_t)2 * num_active * 3);
            for (auto &x : r) x = nd(rng);
            densify_random_samples.copy_from_host(r.data(), r.size() * sizeof(float));
        }
        const float half_max_dim = 0.5f * (float)std::max(lastWidth, lastHeight);
        const int check_screen = step < stopScreenSizeAt ? 1 : 0;
        const bool checkHuge = step > refineEvery * resetAlphaEvery;
        MTensor unused;
        auto densify = [&] {
            const int fr_stride = (int)featuresRest_buf.stride0();
            return msplat_densify(num_active, buf_capacity, densifyGradThresh, densifySizeThresh, splitScreenSize,
                                  check_screen, cullAlphaThresh, 0.5f, 0.15f, checkHuge ? 1 : 0, xysGradNorm,
                                  visCounts, max2DSize, half_max_dim, means_buf, scales_buf, quats_buf,
                                  featuresDc_buf, featuresRest_buf, opacities_buf, fr_stride, adam_exp_avg_buf,
                                  adam_exp_avg_sq_buf, unused, unused, unused, unused, unused, unused, unused,
                                  unused, densify_random_samples);
        };
        int nc = densify();
        if (nc < 0) {
            // splats both split and duplicated need more than 3N rows:
            // nothing was modified, grow to the reported count and redo
            ensureCapacity(-nc);
            nc = densify();
        }
        num_active = nc;
        refreshViews();
        std::cout << "Densified: " << before << " -> " << num_active << " gaussians" << std::endl;
    }
    if (step < stopSplitAt && step % resetInterval == refineEvery) {
        // opacity reset to logit(0.2) (model.cpp:290-300)
        constexpr float kResetLogit = -1.3862943611198906f;
        if (msplat_hip_clamp_max(opacities.data<float>(), opacities.numel(), kResetLogit) != MSPLAT_OK)
            throw std::runtime_error(std::string("msplat engine: ") + msplat_hip_last_error());
        adam_exp_avg[5].zero();
        adam_exp_avg_sq[5].zero();
        std::fprintf(stderr, "Opacity reset at step %d\n", step);
    }
    xysGradNorm.reset();
    visCounts.reset();
    max2DSize.reset();
}

Model::CamSetup Model::prepareCam(Camera &cam, int step) {
    const float sf = (float)getDownscaleFactor(step);
    CamSetup s;
    s.fx = cam.fx / sf;
    s.fy = cam.fy / sf;
    s.cx = cam.cx / sf;
    s.cy = cam.cy / sf;
    s.height = (int)(cam.height / sf);
    s.width = (int)(cam.width / sf);
    s.degreesToUse = std::min(step / shDegreeInterval, shDegree);
    const int b = (int)featuresRest.size(-2) + 1;
    s.degree = b <= 1 ? 0 : b <= 4 ? 1 : b <= 9 ? 2 : b <= 16 ? 3 : 4;
    s.degreesToUse = std::min(s.degreesToUse, s.degree);
    MsplatCamera mc;
    if (msplat_hip_prepare_camera(cam.camToWorld, s.fx, s.fy, s.cx, s.cy, s.width, s.height, s.degree,
                                  s.degreesToUse, &mc) != MSPLAT_OK)
        throw std::runtime_error(std::string("msplat engine: ") + msplat_hip_last_error());
    s.tileBounds = std::make_tuple(mc.tiles_x, mc.tiles_y, 1);
    for (int k = 0; k < 3; ++k) s.cam_pos[k] = mc.cam_pos[k];
    s.viewMat = MTensor({4, 4}, DType::Float32);
    s.projViewMat = MTensor({4, 4}, DType::Float32);
    std::memcpy(s.viewMat.data_ptr(), mc.viewmat, sizeof(mc.viewmat));
    std::memcpy(s.projViewMat.data_ptr(), mc.projmat, sizeof(mc.projmat));
    return s;
}

float Model::fullIteration(Camera &cam, int step, MTensor &gt, float ssimWeight) {
    CamSetup s = prepareCam(cam, step);
    if (gt.ndim() != 3 || gt.size(0) != s.height || gt.size(1) != s.width || gt.size(2) != 3 || !gt.isGpu())
        throw std::invalid_argument("ground-truth image must be a device [H,W,3] tensor matching the camera");
    lastHeight = s.height;
    lastWidth = s.width;
    const int n = (int)means.size(0);
    ++adam_step_count;
    // bias corrections as the reference computes them: pow in double,
    // rounded to float (model.cpp:767-768)
    const float bc1 = 1.0f - std::pow(adam_beta1, adam_step_count);
    const float bc2 = 1.0f - std::pow(adam_beta2, adam_step_count);
    if (!xysGradNorm.defined() || xysGradNorm.numel() != n) allocStats(n);
    const float invMaxDim = 1.0f / (float)std::max(s.width, s.height);
    float step_size[N_ADAM_GROUPS];
    for (int g = 0; g < N_ADAM_GROUPS; ++g) step_size[g] = adam_lr[g] / bc1;
    auto out = scaleDim == 3
                   ? msplat_train_step_3dgs_adam(
                         n, means, scales, 1.0f, quats, s.viewMat, s.projViewMat, s.fx, s.fy, s.cx, s.cy,
                         (unsigned)s.height, (unsigned)s.width, s.tileBounds, 0.01f, (unsigned)s.degree,
                         (unsigned)s.degreesToUse, s.cam_pos, featuresDc, featuresRest, opacities, backgroundColor, gt,
                         (int)featuresRest.size(-2), 1.0f - ssimWeight, ssimWeight, xysGradNorm, visCounts,
                         max2DSize, invMaxDim, adam_exp_avg, adam_exp_avg_sq, step_size, adam_beta1, adam_beta2,
                         std::sqrt(bc2), adam_eps)
                   : msplat_train_step_2dgs_adam(
                         n, means, scales, 1.0f, quats, s.viewMat, s.projViewMat, s.fx, s.fy, s.cx, s.cy,
                         (unsigned)s.height, (unsigned)s.width, s.tileBounds, 0.01f, (unsigned)s.degree,
                         (unsigned)s.degreesToUse, s.cam_pos, featuresDc, featuresRest, opacities, backgroundColor, gt,
                         (int)featuresRest.size(-2), 1.0f - ssimWeight, 0.0f, ssimWeight, xysGradNorm, visCounts,
                         max2DSize, invMaxDim, adam_exp_avg, adam_exp_avg_sq, step_size, adam_beta1, adam_beta2,
                         std::sqrt(bc2), adam_eps);
    radii = std::get<0>(out);
    return std::get<1>(out);
}

MTensor Model::render(Camera &cam, int step) {
    CamSetup s = prepareCam(cam, step);
    auto fn = scaleDim == 3 ? msplat_render_3dgs : msplat_render;
    return fn((int)means.size(0), means, scales, 1.0f, quats, s.viewMat, s.projViewMat, s.fx, s.fy, s.cx, s.cy,
              (unsigned)s.height, (unsigned)s.width, s.tileBounds, 0.01f, (unsigned)s.degree,
              (unsigned)s.degreesToUse, s.cam_pos, featuresDc, featuresRest, opacities, backgroundColor);
}

// ---- checkpoints (model.cpp:343-498): little-endian, magic "MSPL",
// version 1, then step, count, SH degree and Adam step (u32), the six
// learning rates and the means schedule (f32), then 18 tensors (6 params,
// 6 first moments, 6 second moments), each as ndim (u32), shape (i64 x
// ndim), byte count (u64), data.

namespace {

void write_tensor(std::ofstream &f, const MTensor &t) {
    const uint32_t nd = (uint32_t)t.ndim();
    f.write((const char *)&nd, 4);
    for (int i = 0; i < (int)nd; ++i) {
        const int64_t s = t.size(i);
        f.write((const char *)&s, 8);
    }
    const uint64_t bytes = t.nbytes();
    f.write((const char *)&bytes, 8);
    std::vector<uint8_t> host(bytes);
    t.copy_to_host(host.data());
    f.write((const char *)host.data(), (std::streamsize)bytes);
}

MTensor read_tensor(std::ifstream &f) {
    uint32_t nd = 0;
    f.read((char *)&nd, 4);
    if (!f || nd == 0 || nd > 8) throw std::runtime_error("checkpoint: corrupt tensor header");
    std::vector<int64_t> shape(nd);
    for (auto &s : shape) f.read((char *)&s, 8);
    uint64_t bytes = 0;
    f.read((char *)&bytes, 8);
    int64_t numel = 1;
    for (auto s : shape) {
        if (s < 0) throw std::runtime_error("checkpoint: negative dimension");
        numel *= s;
    }
    if (!f || bytes != (uint64_t)numel * 4) throw std::runtime_error("checkpoint: tensor size mismatch");
    std::vector<float> host((size_t)numel);
    f.read((char *)host.data(), (std::streamsize)bytes);
    if (!f) throw std::runtime_error("checkpoint: truncated tensor data");
    MTensor t = MTensor::device(shape, DType::Float32);
    t.copy_from_host(host.data(), bytes);
    return t;
}

}  // namespace

void Model::saveCheckpoint(const std::string &filename, int step) {
    msplat_gpu_sync();
    std::ofstream f(filename, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open checkpoint file for writing: " + filename);
    f.write((const char *)&kCkptMagic, 4);
    f.write((const char *)&kCkptVersion, 4);
    const uint32_t head[4] = {(uint32_t)step, (uint32_t)num_active, (uint32_t)shDegree, (uint32_t)adam_step_count};
    f.write((const char *)head, sizeof(head));
    f.write((const char *)adam_lr, sizeof(adam_lr));
    f.write((const char *)&means_lr_init, 4);
    f.write((const char *)&means_lr_final, 4);
    for (const MTensor *t : {&means, &scales, &quats, &featuresDc, &featuresRest, &opacities}) write_tensor(f, *t);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) write_tensor(f, adam_exp_avg[g]);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) write_tensor(f, adam_exp_avg_sq[g]);
    if (!f) throw std::runtime_error("Failed writing checkpoint: " + filename);
    std::cout << "Checkpoint saved: " << filename << " (step " << step << ", " << num_active << " gaussians)"
              << std::endl;
}

int Model::loadCheckpoint(const std::string &filename) {
    std::ifstream f(filename, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open checkpoint file: " + filename);
    uint32_t magic = 0, version = 0;
    f.read((char *)&magic, 4);
    f.read((char *)&version, 4);
    if (magic != kCkptMagic) throw std::runtime_error("Not a valid msplat checkpoint file");
    if (version != kCkptVersion) throw std::runtime_error("Unsupported checkpoint version: " + std::to_string(version));
    uint32_t head[4];
    f.read((char *)head, sizeof(head));
    float lr[N_ADAM_GROUPS], lr0 = 0, lr1 = 0;
    f.read((char *)lr, sizeof(lr));
    f.read((char *)&lr0, 4);
    f.read((char *)&lr1, 4);
    if (!f) throw std::runtime_error("checkpoint: truncated header");
    MTensor p[6], m[6], v[6];
    for (auto &t : p) t = read_tensor(f);
    for (auto &t : m) t = read_tensor(f);
    for (auto &t : v) t = read_tensor(f);
    const int64_t n = head[1];
    for (int g = 0; g < 6; ++g)
        if (p[g].size(0) != n || m[g].shape() != p[g].shape() || v[g].shape() != p[g].shape())
            throw std::runtime_error("checkpoint: inconsistent tensor shapes");
    if (p[1].ndim() != 2 || p[1].size(1) != scaleDim)
        throw std::runtime_error("checkpoint: scales must be [N," + std::to_string(scaleDim) + "] for this model");
    releaseOptimizers();
    means = p[0];
    scales = p[1];
    quats = p[2];
    featuresDc = p[3];
    featuresRest = p[4];
    opacities = p[5];
    num_active = (int)n;
    buf_capacity = std::max(num_active * 4, 16);
    means_buf = backing(means, buf_capacity);
    scales_buf = backing(scales, buf_capacity);
    quats_buf = backing(quats, buf_capacity);
    featuresDc_buf = backing(featuresDc, buf_capacity);
    featuresRest_buf = backing(featuresRest, buf_capacity);
    opacities_buf = backing(opacities, buf_capacity);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) {
        adam_exp_avg_buf[g] = backing(m[g], buf_capacity);
        adam_exp_avg_sq_buf[g] = backing(v[g], buf_capacity);
        adam_lr[g] = lr[g];
    }
    shDegree = (int)head[2];
    adam_step_count = (int)head[3];
    means_lr_init = lr0;
    means_lr_final = lr1;
    densify_random_samples = gpu_zeros({(int64_t)buf_capacity, 3}, DType::Float32);
    xysGradNorm.reset();
    visCounts.reset();
    max2DSize.reset();
    radii.reset();
    refreshViews();
    std::cout << "Checkpoint loaded: " << filename << " (step " << head[0] << ", " << num_active << " gaussians)"
              << std::endl;
    return (int)head[0];
}

// ---- point cloud, TSDF fusion, mesh (model.cpp:565-757) ----

namespace {

void engine_check(int rc) {
    if (rc != MSPLAT_OK) throw std::runtime_error(std::string("msplat engine: ") + msplat_hip_last_error());
}

}  // namespace

int64_t Model::exportPointCloud(std::vector<Camera> &cameras, int step, float alphaThresh,
                                const std::string &outPath) {
    if (scaleDim != 2) throw std::runtime_error("point cloud export needs the 2DGS mode's depth");
    std::vector<float> xyz;
    std::vector<uint8_t> rgb;
    MTensor xyzDev, rgbDev;
    for (auto &cam : cameras) {
        const CamSetup s = prepareCam(cam, step);
        MTensor img = render(cam, step);
        MTensor depth = msplat_last_out_depth();  // alpha-weighted depth sum
        MTensor alpha = msplat_last_out_alpha();
        const int64_t np = (int64_t)s.width * s.height;
        if (!xyzDev.defined() || xyzDev.numel() < np * 3) {
            xyzDev = MTensor::device({std::max<int64_t>(np, 1), 3}, DType::Float32);
            rgbDev = MTensor::device({std::max<int64_t>(np, 1), 3}, DType::UInt8);
        }
        int64_t n = 0;
        engine_check(msplat_hip_unproject_depth(img.data<float>(), depth.data<float>(), alpha.data<float>(), s.width,
                                                s.height, s.fx, s.fy, s.cx, s.cy, cam.camToWorld, alphaThresh,
                                                xyzDev.data<float>(), rgbDev.data<uint8_t>(), &n));
        const size_t off = xyz.size() / 3;
        xyz.resize((off + n) * 3);
        rgb.resize((off + n) * 3);
        if (n > 0) {
            engine_check(msplat_hip_download(xyz.data() + off * 3, xyzDev.data_ptr(), (size_t)n * 12));
            engine_check(msplat_hip_download(rgb.data() + off * 3, rgbDev.data_ptr(), (size_t)n * 3));
        }
    }
    const int64_t N = (int64_t)(xyz.size() / 3);
    std::ofstream out(outPath, std::ios::binary);
    if (!out.is_open()) throw std::runtime_error("Cannot open " + outPath);
    out << "ply\nformat binary_little_endian 1.0\n";
    out << "comment msplat 2c.0 point cloud (unprojected depth, " << cameras.size() << " views)\n";
    out << "element vertex " << N << "\n";
    out << "property float x\nproperty float y\nproperty float z\n";
    out << "property uchar red\nproperty uchar green\nproperty uchar blue\n";
    out << "end_header\n";
    std::vector<char> body((size_t)N * 15);
    for (int64_t i = 0; i < N; ++i) {
        std::memcpy(&body[(size_t)i * 15], &xyz[(size_t)i * 3], 12);
        std::memcpy(&body[(size_t)i * 15 + 12], &rgb[(size_t)i * 3], 3);
    }
    out.write(body.data(), (std::streamsize)body.size());
    return N;
}

Model::VoxelGrid Model::makeVoxelGrid(const std::vector<Camera> &cameras, float voxelSize, float boundRadius,
                                      int memoryCapMB) const {
    if (cameras.empty()) throw std::runtime_error("makeVoxelGrid: no cameras");
    if (!(voxelSize > 0.0f) || !(boundRadius > 0.0f))
        throw std::invalid_argument("makeVoxelGrid: voxelSize and boundRadius must be positive");
    VoxelGrid g;
    g.origin[0] = g.origin[1] = g.origin[2] = -boundRadius;
    const float dimf = std::ceil(2.0f * boundRadius / voxelSize);
    if (!(dimf <= 65535.0f)) throw std::runtime_error("makeVoxelGrid: grid of more than 65535 voxels per axis");
    const int dim = (int)dimf;
    g.dims[0] = g.dims[1] = g.dims[2] = dim;
    g.voxelSize = voxelSize;
    const int64_t bytes = (int64_t)dim * dim * dim * 2 * 4;
    if (bytes > (int64_t)memoryCapMB * 1024 * 1024)
        throw std::runtime_error("makeVoxelGrid: " + std::to_string(bytes / (1024 * 1024)) + " MB exceeds " +
                                 std::to_string(memoryCapMB) + " MB cap (dim=" + std::to_string(dim) +
                                 ", voxelSize=" + std::to_string(voxelSize) + "m). " +
                                 "Increase voxelSize or decrease boundRadius.");
    g.data = gpu_zeros({dim, dim, dim, 2}, DType::Float32);
    return g;
}

void Model::integrateTSDF(VoxelGrid &grid, std::vector<Camera> &cameras, int step, float truncDist,
                          float alphaThresh) {
    if (scaleDim != 2) throw std::runtime_error("TSDF fusion needs the 2DGS mode's median depth");
    // Each camera's median depth (the surface depth, where T crosses 0.5)
    // and alpha are staged in HBM; a batch of views is then folded into the
    // grid in one pass, every voxel applying the views in camera order --
    // the values the reference's one dispatch per camera produces.
    constexpr size_t kStageFloats = size_t(1) << 28;  // 1 GiB of staged maps per pass
    MTensor stage;
    size_t used = 0;
    std::vector<MsplatTsdfView> views;
    auto flush = [&] {
        if (!views.empty())
            engine_check(msplat_hip_tsdf_integrate(grid.data.data<float>(), grid.dims[0], grid.dims[1], grid.dims[2],
                                                   grid.origin, grid.voxelSize, views.data(), (int)views.size(),
                                                   truncDist, alphaThresh));
        views.clear();
        used = 0;
    };
    for (auto &cam : cameras) {
        const CamSetup s = prepareCam(cam, step);
        render(cam, step);
        MTensor depth = msplat_last_out_median_depth();
        MTensor alpha = msplat_last_out_alpha();
        const size_t np = (size_t)s.width * s.height;
        if (used + 2 * np > (size_t)stage.numel()) {
            flush();
            if (2 * np > (size_t)stage.numel())
                stage = MTensor::device({(int64_t)std::max(kStageFloats, 2 * np)}, DType::Float32);
        }
        float *d = stage.data<float>() + used;
        engine_check(msplat_hip_copy(d, depth.data_ptr(), np * 4));
        engine_check(msplat_hip_copy(d + np, alpha.data_ptr(), np * 4));
        used += 2 * np;
        MsplatTsdfView v{};
        std::memcpy(v.viewmat, s.viewMat.data_ptr(), sizeof(v.viewmat));
        v.fx = s.fx;
        v.fy = s.fy;
        v.cx = s.cx;
        v.cy = s.cy;
        v.width = s.width;
        v.height = s.height;
        v.depth_dev = d;
        v.alpha_dev = d + np;
        views.push_back(v);
    }
    flush();
    msplat_gpu_sync();
}

int64_t Model::extractMesh(const VoxelGrid &grid, const std::string &outPath, int maxTriangles) {
    std::vector<float> tris;
    const int64_t nTri = msplat_marching_cubes(const_cast<MTensor &>(grid.data), grid.dims[0], grid.dims[1],
                                               grid.dims[2], grid.origin[0], grid.origin[1], grid.origin[2],
                                               grid.voxelSize, maxTriangles, tris);
    std::ofstream out(outPath, std::ios::binary);
    if (!out.is_open()) throw std::runtime_error("Cannot open " + outPath);
    out << "ply\nformat binary_little_endian 1.0\n";
    out << "comment msplat 2c.3 Marching Cubes mesh (non-indexed)\n";
    out << "element vertex " << nTri * 3 << "\n";
    out << "property float x\nproperty float y\nproperty float z\n";
    out << "element face " << nTri << "\n";
    out << "property list uchar int vertex_indices\n";
    out << "end_header\n";
    out.write(reinterpret_cast<const char *>(tris.data()), (std::streamsize)(nTri * 9 * sizeof(float)));
    // each triangle owns its three vertices: faces (3, 3i, 3i+1, 3i+2)
    std::vector<char> faces((size_t)nTri * 13);
    for (int64_t i = 0; i < nTri; ++i) {
        char *f = &faces[(size_t)i * 13];
        f[0] = 3;
        for (int k = 0; k < 3; ++k) {
            const int32_t idx = (int32_t)(i * 3 + k);
            std::memcpy(f + 1 + 4 * k, &idx, 4);
        }
    }
    out.write(faces.data(), (std::streamsize)faces.size());
    return nTri;
}
