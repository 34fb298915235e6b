// msplat_api.cpp -- Dataset / Trainer (C++ API, include/msplat_api.hpp)
// and the C ABI over them (include/msplat_c_api.h), following
// core/src/msplat_api.mm:1-407 of the reference: camera shuffling with
// mt19937(42), step = fullIteration + schedulersStep + afterTrain, test
// evaluation with host-side PSNR / SSIM / L1, renders copied to malloc'd
// buffers the caller frees.
#include "msplat_api.hpp"

#include <algorithm>
#include <chrono>
#include <cstring>
#include <numeric>
#include <random>
#include <stdexcept>
#include <string>

#include "msplat_c_api.h"
#include "model.hpp"
#include "msplat_engine.h"

namespace msplat {

struct Dataset::Impl {
    InputData data;
    std::vector<Camera> trainCams;
    std::vector<Camera> testCams;

    void split(bool evalMode, int testEvery) {
        if (evalMode) {
            auto s = data.splitTrainTest(testEvery);
            trainCams = std::get<0>(s);
            testCams = std::get<1>(s);
        } else {
            trainCams = std::get<0>(data.getCameras(false));
        }
        if (trainCams.empty()) throw std::runtime_error("dataset has no training cameras");
    }
};

Dataset::Dataset(const std::string &path, float downscaleFactor, bool evalMode, int testEvery)
    : impl(std::make_unique<Impl>()) {
    impl->data = inputDataFromX(path);
    for (auto &cam : impl->data.cameras) cam.loadImage(downscaleFactor);
    impl->split(evalMode, testEvery);
}

Dataset::Dataset(const std::vector<CameraImage> &cameras, const float *xyz, const uint8_t *rgb, int64_t numPoints,
                 bool evalMode, int testEvery)
    : impl(std::make_unique<Impl>()) {
    if (cameras.empty()) throw std::invalid_argument("no cameras");
    for (size_t i = 0; i < cameras.size(); ++i) {
        const CameraImage &ci = cameras[i];
        if (ci.width <= 0 || ci.height <= 0 || !ci.rgb || !(ci.fx > 0) || !(ci.fy > 0))
            throw std::invalid_argument("camera " + std::to_string(i) + ": invalid size, intrinsics or image");
        Camera c;
        c.width = ci.width;
        c.height = ci.height;
        c.fx = ci.fx;
        c.fy = ci.fy;
        c.cx = ci.cx;
        c.cy = ci.cy;
        std::memcpy(c.camToWorld, ci.camToWorld, sizeof(c.camToWorld));
        c.filePath = "memory:" + std::to_string(i);
        c.image.width = ci.width;
        c.image.height = ci.height;
        c.image.data.assign(ci.rgb, ci.rgb + (size_t)ci.width * ci.height * 3);
        impl->data.cameras.push_back(std::move(c));
    }
    if (numPoints > 0) {
        if (!xyz || !rgb) throw std::invalid_argument("point arrays are null");
        impl->data.points.xyz.assign(xyz, xyz + numPoints * 3);
        impl->data.points.rgb.assign(rgb, rgb + numPoints * 3);
        impl->data.points.count = numPoints;
    } else {
        initializeRandomPointsCameraAware(impl->data, 100000, 0.35f);
    }
    impl->split(evalMode, testEvery);
}

Dataset::~Dataset() = default;
Dataset::Dataset(Dataset &&) noexcept = default;
Dataset &Dataset::operator=(Dataset &&) noexcept = default;

int Dataset::numTrain() const { return (int)impl->trainCams.size(); }
int Dataset::numTest() const { return (int)impl->testCams.size(); }
void Dataset::cameraPose(int index, float camToWorld[16]) const {
    if (index >= 0 && index < (int)impl->trainCams.size())
        std::memcpy(camToWorld, impl->trainCams[index].camToWorld, 16 * sizeof(float));
}
void *Dataset::_handle() const { return impl.get(); }

struct Trainer::Impl {
    std::unique_ptr<Model> model;
    Config config;
    Dataset::Impl *ds = nullptr;
    int currentStep = 0;
    std::vector<size_t> camIndices;
    size_t camIterPos = 0;
    std::mt19937 rng{42};

    void shuffleCameras() {
        std::shuffle(camIndices.begin(), camIndices.end(), rng);
        camIterPos = 0;
    }
    size_t nextCamera() {
        if (camIterPos >= camIndices.size()) shuffleCameras();
        return camIndices[camIterPos++];
    }
    PixelBuffer renderCam(Camera &cam) {
        MTensor rgb = model->render(cam, currentStep);
        const int h = (int)rgb.size(0), w = (int)rgb.size(1);
        float *buf = (float *)std::malloc((size_t)h * w * 3 * sizeof(float));
        if (!buf) throw std::bad_alloc();
        rgb.copy_to_host(buf);
        return PixelBuffer(buf, w, h);
    }
    // The intrinsics of the reference camera at a new pose.  Only those
    // fields are taken: the camera's image, pyramid and GPU image cache stay
    // behind (copying them cost a full-resolution image per frame).
    Camera poseCamera(const float camToWorld[16], int ref) {
        const Camera &src = ds->trainCams.at(ref);
        Camera cam;
        cam.width = src.width;
        cam.height = src.height;
        cam.fx = src.fx;
        cam.fy = src.fy;
        cam.cx = src.cx;
        cam.cy = src.cy;
        cam.k1 = src.k1;
        cam.k2 = src.k2;
        cam.k3 = src.k3;
        cam.p1 = src.p1;
        cam.p2 = src.p2;
        std::memcpy(cam.camToWorld, camToWorld, 16 * sizeof(float));
        return cam;
    }
};

Trainer::Trainer(Dataset &dataset, const Config &config) : Trainer(dataset, config, Primitive::Surfel2D) {}

Trainer::Trainer(Dataset &dataset, const Config &config, Primitive primitive) : impl(std::make_unique<Impl>()) {
    impl->config = config;
    impl->ds = static_cast<Dataset::Impl *>(dataset._handle());
    impl->model = std::make_unique<Model>(
        impl->ds->data, (int)impl->ds->trainCams.size(), config.numDownscales, config.resolutionSchedule,
        config.shDegree, config.shDegreeInterval, config.refineEvery, config.warmupLength, config.resetAlphaEvery,
        config.densifyGradThresh, config.densifySizeThresh, config.stopScreenSizeAt, config.splitScreenSize,
        config.iterations, config.keepCrs, config.bgColor, primitive == Primitive::Gaussian3D ? 3 : 2);
    impl->camIndices.resize(impl->ds->trainCams.size());
    std::iota(impl->camIndices.begin(), impl->camIndices.end(), 0);
    impl->shuffleCameras();
}

Trainer::~Trainer() = default;

Stats Trainer::step() {
    Impl &I = *impl;
    ++I.currentStep;
    Camera &cam = I.ds->trainCams[I.nextCamera()];
    MTensor &gt = cam.getGPUImage(I.model->getDownscaleFactor(I.currentStep));
    const auto t0 = std::chrono::steady_clock::now();
    const float loss = I.model->fullIteration(cam, I.currentStep, gt, I.config.ssimWeight);
    I.model->schedulersStep(I.currentStep);
    I.model->afterTrain(I.currentStep);
    msplat_commit();
    const auto t1 = std::chrono::steady_clock::now();
    Stats s;
    s.iteration = I.currentStep;
    s.splatCount = (int)I.model->means.size(0);
    s.msPerStep = std::chrono::duration<float, std::milli>(t1 - t0).count();
    s.loss = loss;
    return s;
}

void Trainer::train(int) {
    while (impl->currentStep < impl->config.iterations) step();
}

EvalMetrics Trainer::evaluate() {
    auto &test = impl->ds->testCams;
    if (test.empty()) return {};
    double sp = 0, ss = 0, sl = 0;
    const int ds = impl->model->getDownscaleFactor(impl->config.iterations);
    for (auto &cam : test) {
        MTensor rgb = impl->model->render(cam, impl->config.iterations).cpu();
        MTensor gt = cam.getGPUImage(ds).cpu();
        sp += psnr(rgb, gt);
        ss += ssim_eval(rgb, gt);
        sl += l1_loss(rgb, gt);
    }
    const int n = (int)test.size();
    EvalMetrics m;
    m.psnr = (float)(sp / n);
    m.ssim = (float)(ss / n);
    m.l1 = (float)(sl / n);
    m.numTest = n;
    m.numGaussians = (int)impl->model->means.size(0);
    return m;
}

PixelBuffer Trainer::render(int cameraIndex, bool useTest) {
    auto &cams = useTest ? impl->ds->testCams : impl->ds->trainCams;
    if (cameraIndex < 0 || cameraIndex >= (int)cams.size()) return {};
    return impl->renderCam(cams[cameraIndex]);
}

PixelBuffer Trainer::renderFromPose(const float camToWorld[16], int refCameraIndex) {
    if (refCameraIndex < 0 || refCameraIndex >= (int)impl->ds->trainCams.size()) return {};
    Camera cam = impl->poseCamera(camToWorld, refCameraIndex);
    return impl->renderCam(cam);
}

void Trainer::renderFromPoseToBuffer(const float camToWorld[16], int refCameraIndex, uint8_t *outRGBA, int *outWidth,
                                     int *outHeight) {
    if (refCameraIndex < 0 || refCameraIndex >= (int)impl->ds->trainCams.size()) {
        *outWidth = 0;
        *outHeight = 0;
        return;
    }
    Camera cam = impl->poseCamera(camToWorld, refCameraIndex);
    MTensor rgb = impl->model->render(cam, impl->currentStep);
    *outWidth = (int)rgb.size(1);
    *outHeight = (int)rgb.size(0);
    if (!outRGBA) return;
    // converted on the GPU: 4 bytes per pixel cross PCIe instead of 12
    const int rc = msplat_hip_image_to_rgba8(static_cast<const float *>(rgb.data_ptr()),
                                             (int64_t)rgb.size(0) * rgb.size(1), outRGBA);
    if (rc != MSPLAT_OK) throw std::runtime_error(std::string("rgba8 conversion: ") + msplat_hip_last_error());
}

void Trainer::exportPly(const std::string &path) { impl->model->savePly(path, impl->currentStep); }
void Trainer::exportSplat(const std::string &path) { impl->model->saveSplat(path); }

int64_t Trainer::extractMesh(const std::string &path, float voxelSize, float boundRadius, float alphaThresh,
                             float truncMultiplier) {
    // msplat_api.mm:242-250
    auto grid = impl->model->makeVoxelGrid(impl->ds->trainCams, voxelSize, boundRadius);
    const float truncDist = truncMultiplier * voxelSize;
    impl->model->integrateTSDF(grid, impl->ds->trainCams, impl->currentStep, truncDist, alphaThresh);
    return impl->model->extractMesh(grid, path);
}

int64_t Trainer::exportPointCloud(const std::string &path, float alphaThresh) {
    return impl->model->exportPointCloud(impl->ds->trainCams, impl->currentStep, alphaThresh, path);
}

void Trainer::saveCheckpoint(const std::string &path) { impl->model->saveCheckpoint(path, impl->currentStep); }

int Trainer::loadCheckpoint(const std::string &path) {
    impl->currentStep = impl->model->loadCheckpoint(path);
    impl->shuffleCameras();
    return impl->currentStep;
}

int Trainer::splatCount() const { return (int)impl->model->means.size(0); }
int Trainer::iteration() const { return impl->currentStep; }
Primitive Trainer::primitive() const {
    return impl->model->scaleDim == 3 ? Primitive::Gaussian3D : Primitive::Surfel2D;
}

int Trainer::loadPly(const std::string &path) {
    impl->currentStep = impl->model->loadPly(path);
    impl->shuffleCameras();
    return impl->currentStep;
}

void Trainer::setMaxSplats(int maxSplats) { impl->model->maxSplats = maxSplats; }
void Trainer::setCullAlphaThresh(float thresh) { impl->model->cullAlphaThresh = thresh; }

void sync() { msplat_gpu_sync(); }
void cleanup() { cleanup_msplat_metal(); }

}  // namespace msplat

// ---------------------------------------------------------------- C ABI --

namespace {

thread_local std::string g_err;

template <typename R, typename F>
R guarded(R fail, F &&f) {
    try {
        g_err.clear();
        return f();
    } catch (const std::exception &e) {
        g_err = e.what();
    } catch (...) {
        g_err = "unknown error";
    }
    return fail;
}

msplat::Config config_from_c(const MsplatConfig &c) {
    msplat::Config k;
    k.iterations = c.iterations;
    k.shDegree = c.shDegree;
    k.shDegreeInterval = c.shDegreeInterval;
    k.ssimWeight = c.ssimWeight;
    k.numDownscales = c.numDownscales;
    k.resolutionSchedule = c.resolutionSchedule;
    k.refineEvery = c.refineEvery;
    k.warmupLength = c.warmupLength;
    k.resetAlphaEvery = c.resetAlphaEvery;
    k.densifyGradThresh = c.densifyGradThresh;
    k.densifySizeThresh = c.densifySizeThresh;
    k.stopScreenSizeAt = c.stopScreenSizeAt;
    k.splitScreenSize = c.splitScreenSize;
    k.keepCrs = c.keepCrs;
    k.downscaleFactor = c.downscaleFactor;
    std::memcpy(k.bgColor, c.bgColor, sizeof(k.bgColor));
    return k;
}

msplat::Dataset *D(MsplatDataset d) {
    if (!d) throw std::invalid_argument("null dataset handle");
    return static_cast<msplat::Dataset *>(d);
}
msplat::Trainer *T(MsplatTrainer t) {
    if (!t) throw std::invalid_argument("null trainer handle");
    return static_cast<msplat::Trainer *>(t);
}
MsplatPixelBuffer release(msplat::PixelBuffer &&b) {
    MsplatPixelBuffer r{b.data, b.width, b.height};
    b.data = nullptr;
    return r;
}

}  // namespace

extern "C" {

MsplatDataset msplat_dataset_create(const char *path, float downscaleFactor, bool evalMode, int testEvery) {
    return guarded<MsplatDataset>(nullptr, [&]() -> MsplatDataset {
        if (!path) throw std::invalid_argument("null path");
        return new msplat::Dataset(std::string(path), downscaleFactor, evalMode, testEvery);
    });
}

MsplatDataset msplat_dataset_create_from_memory(const MsplatCameraImage *cameras, int numCameras, const float *xyz,
                                                const uint8_t *rgb, int64_t numPoints, bool evalMode, int testEvery) {
    return guarded<MsplatDataset>(nullptr, [&]() -> MsplatDataset {
        if (!cameras || numCameras <= 0) throw std::invalid_argument("no cameras");
        std::vector<msplat::CameraImage> cams((size_t)numCameras);
        for (int i = 0; i < numCameras; ++i) {
            const MsplatCameraImage &c = cameras[i];
            cams[i].width = c.width;
            cams[i].height = c.height;
            cams[i].fx = c.fx;
            cams[i].fy = c.fy;
            cams[i].cx = c.cx;
            cams[i].cy = c.cy;
            std::memcpy(cams[i].camToWorld, c.camToWorld, sizeof(c.camToWorld));
            cams[i].rgb = c.rgb;
        }
        return new msplat::Dataset(cams, xyz, rgb, numPoints, evalMode, testEvery);
    });
}

void msplat_dataset_destroy(MsplatDataset ds) { delete static_cast<msplat::Dataset *>(ds); }
int msplat_dataset_num_train(MsplatDataset ds) {
    return guarded(0, [&] { return D(ds)->numTrain(); });
}
int msplat_dataset_num_test(MsplatDataset ds) {
    return guarded(0, [&] { return D(ds)->numTest(); });
}
void msplat_dataset_camera_pose(MsplatDataset ds, int cameraIndex, float camToWorld[16]) {
    guarded(0, [&] {
        D(ds)->cameraPose(cameraIndex, camToWorld);
        return 0;
    });
}

MsplatTrainer msplat_trainer_create(MsplatDataset ds, MsplatConfig config) {
    return guarded<MsplatTrainer>(nullptr, [&]() -> MsplatTrainer {
        return new msplat::Trainer(*D(ds), config_from_c(config));
    });
}
MsplatTrainer msplat_trainer_create_3dgs(MsplatDataset ds, MsplatConfig config) {
    return guarded<MsplatTrainer>(nullptr, [&]() -> MsplatTrainer {
        return new msplat::Trainer(*D(ds), config_from_c(config), msplat::Primitive::Gaussian3D);
    });
}
void msplat_trainer_destroy(MsplatTrainer t) { delete static_cast<msplat::Trainer *>(t); }

MsplatStats msplat_trainer_step(MsplatTrainer t) {
    return guarded(MsplatStats{0, 0, 0.f, 0.f}, [&] {
        const msplat::Stats s = T(t)->step();
        return MsplatStats{s.iteration, s.splatCount, s.msPerStep, s.loss};
    });
}
void msplat_trainer_train(MsplatTrainer t) {
    guarded(0, [&] {
        T(t)->train(0);
        return 0;
    });
}
MsplatEvalMetrics msplat_trainer_evaluate(MsplatTrainer t) {
    return guarded(MsplatEvalMetrics{0.f, 0.f, 0.f, 0, 0}, [&] {
        const msplat::EvalMetrics m = T(t)->evaluate();
        return MsplatEvalMetrics{m.psnr, m.ssim, m.l1, m.numTest, m.numGaussians};
    });
}
MsplatPixelBuffer msplat_trainer_render(MsplatTrainer t, int cameraIndex, bool useTest) {
    return guarded(MsplatPixelBuffer{nullptr, 0, 0}, [&] { return release(T(t)->render(cameraIndex, useTest)); });
}
MsplatPixelBuffer msplat_trainer_render_pose(MsplatTrainer t, const float camToWorld[16], int refCameraIndex) {
    return guarded(MsplatPixelBuffer{nullptr, 0, 0},
                   [&] { return release(T(t)->renderFromPose(camToWorld, refCameraIndex)); });
}
void msplat_trainer_render_pose_to_buffer(MsplatTrainer t, const float camToWorld[16], int refCameraIndex,
                                          uint8_t *outRGBA, int *outWidth, int *outHeight) {
    const int ok = guarded(0, [&] {
        T(t)->renderFromPoseToBuffer(camToWorld, refCameraIndex, outRGBA, outWidth, outHeight);
        return 1;
    });
    if (!ok) {
        if (outWidth) *outWidth = 0;
        if (outHeight) *outHeight = 0;
    }
}
void msplat_trainer_export_ply(MsplatTrainer t, const char *path) {
    guarded(0, [&] {
        T(t)->exportPly(path ? path : "");
        return 0;
    });
}
void msplat_trainer_export_splat(MsplatTrainer t, const char *path) {
    guarded(0, [&] {
        T(t)->exportSplat(path ? path : "");
        return 0;
    });
}
int64_t msplat_trainer_extract_mesh(MsplatTrainer t, const char *path, float voxelSize, float boundRadius,
                                    float alphaThresh, float truncMultiplier) {
    return guarded((int64_t)-1, [&] {
        return T(t)->extractMesh(path ? path : "", voxelSize, boundRadius, alphaThresh, truncMultiplier);
    });
}
void msplat_trainer_save_checkpoint(MsplatTrainer t, const char *path) {
    guarded(0, [&] {
        T(t)->saveCheckpoint(path ? path : "");
        return 0;
    });
}
int msplat_trainer_load_checkpoint(MsplatTrainer t, const char *path) {
    return guarded(-1, [&] { return T(t)->loadCheckpoint(path ? path : ""); });
}
int msplat_trainer_splat_count(MsplatTrainer t) {
    return guarded(0, [&] { return T(t)->splatCount(); });
}
int msplat_trainer_iteration(MsplatTrainer t) {
    return guarded(0, [&] { return T(t)->iteration(); });
}
int msplat_trainer_load_ply(MsplatTrainer t, const char *path) {
    return guarded(-1, [&] { return T(t)->loadPly(path ? path : ""); });
}
void msplat_trainer_set_max_splats(MsplatTrainer t, int maxSplats) {
    guarded(0, [&] {
        T(t)->setMaxSplats(maxSplats);
        return 0;
    });
}
void msplat_trainer_set_cull_alpha(MsplatTrainer t, float thresh) {
    guarded(0, [&] {
        T(t)->setCullAlphaThresh(thresh);
        return 0;
    });
}

void msplat_set_metallib_path(const char *) {}
void msplat_sync(void) {
    guarded(0, [] {
        msplat::sync();
        return 0;
    });
}
void msplat_cleanup(void) { msplat::cleanup(); }
const char *msplat_last_error(void) { return g_err.c_str(); }

}  // extern "C"
