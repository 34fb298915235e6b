// msplat_api.hpp -- C++ API of the trainer (Config, Stats, EvalMetrics,
// PixelBuffer, Dataset, Trainer, sync, cleanup), with the names, defaults
// and semantics of the reference's core/include/msplat_api.hpp:12-172.
// Implementation: msplat-ios_amd/csrc/host/msplat_api.cpp over the HIP
// engine.  Errors are reported by std::runtime_error / std::invalid_argument.
#pragma once

#include <cstdint>
#include <cstdlib>
#include <memory>
#include <string>
#include <vector>

namespace msplat {

struct Config {
    int iterations = 30000;
    int shDegree = 3;
    int shDegreeInterval = 1000;
    float ssimWeight = 0.2f;
    int numDownscales = 2;
    int resolutionSchedule = 3000;
    int refineEvery = 100;
    int warmupLength = 500;
    int resetAlphaEvery = 30;
    float densifyGradThresh = 0.0002f;
    float densifySizeThresh = 0.01f;
    int stopScreenSizeAt = 4000;
    float splitScreenSize = 0.05f;
    bool keepCrs = false;
    float downscaleFactor = 1.0f;
    float bgColor[3] = {0.6130f, 0.0101f, 0.3984f};
};

struct Stats {
    int iteration = 0;
    int splatCount = 0;
    float msPerStep = 0.0f;
    float loss = 0.0f;
};

struct EvalMetrics {
    float psnr = 0.0f;
    float ssim = 0.0f;
    float l1 = 0.0f;
    int numTest = 0;
    int numGaussians = 0;
};

// Rendered RGB float32 HWC image; owns `data` (released with free()).
struct PixelBuffer {
    float *data = nullptr;
    int width = 0;
    int height = 0;

    PixelBuffer() = default;
    PixelBuffer(float *d, int w, int h) : data(d), width(w), height(h) {}
    PixelBuffer(const PixelBuffer &) = delete;
    PixelBuffer &operator=(const PixelBuffer &) = delete;
    PixelBuffer(PixelBuffer &&o) noexcept : data(o.data), width(o.width), height(o.height) { o.data = nullptr; }
    PixelBuffer &operator=(PixelBuffer &&o) noexcept {
        if (this != &o) {
            std::free(data);
            data = o.data;
            width = o.width;
            height = o.height;
            o.data = nullptr;
        }
        return *this;
    }
    ~PixelBuffer() { std::free(data); }
};

// A camera with its image, for datasets assembled in memory (no
// counterpart in the reference, whose datasets always come from disk).
struct CameraImage {
    int width = 0, height = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0;
    float camToWorld[16] = {};  // row-major, OpenGL axes
    const float *rgb = nullptr; // [height, width, 3] float32 in [0,1], copied
};

class Dataset {
public:
    // COLMAP / Nerfstudio / Polycam directory (auto-detected).
    Dataset(const std::string &path, float downscaleFactor, bool evalMode, int testEvery);
    // In-memory cameras + images and an initial point cloud (xyz float32
    // [n,3], rgb uint8 [n,3]; n = 0 seeds 100k random points).  No
    // counterpart in the reference.
    Dataset(const std::vector<CameraImage> &cameras, const float *xyz, const uint8_t *rgb, int64_t numPoints,
            bool evalMode, int testEvery);
    ~Dataset();
    Dataset(const Dataset &) = delete;
    Dataset &operator=(const Dataset &) = delete;
    Dataset(Dataset &&) noexcept;
    Dataset &operator=(Dataset &&) noexcept;

    int numTrain() const;
    int numTest() const;
    void cameraPose(int index, float camToWorld[16]) const;
    void *_handle() const;

    struct Impl;

private:
    std::unique_ptr<Impl> impl;
};

// The splat primitive a Trainer optimises (an extension: the reference
// trains surfels only).
enum class Primitive {
    Surfel2D,    // 2DGS (the reference's step)
    Gaussian3D,  // 3DGS: three scales, EWA projection, no depth outputs
};

class Trainer {
public:
    // The dataset must outlive the trainer.
    Trainer(Dataset &dataset, const Config &config);
    Trainer(Dataset &dataset, const Config &config, Primitive primitive);
    ~Trainer();
    Trainer(const Trainer &) = delete;
    Trainer &operator=(const Trainer &) = delete;

    Stats step();
    void train(int callbackEvery);
    EvalMetrics evaluate();
    PixelBuffer render(int cameraIndex, bool useTest);
    PixelBuffer renderFromPose(const float camToWorld[16], int refCameraIndex);
    // RGBA8 (truncating (uint8)(clamp(x, 0, 1) * 255), alpha 255) into
    // outRGBA (width * height * 4 bytes); outRGBA == nullptr only reports
    // the size.
    void renderFromPoseToBuffer(const float camToWorld[16], int refCameraIndex, uint8_t *outRGBA, int *outWidth,
                                int *outHeight);
    void exportPly(const std::string &path);
    // TSDF fusion of every training camera's render into a cube of side
    // 2 * boundRadius around the origin (voxels of voxelSize, truncation
    // truncMultiplier voxels), then marching cubes -> non-indexed triangle
    // PLY at path; returns the triangle count (msplat_api.hpp:138-148).
    int64_t extractMesh(const std::string &path, float voxelSize = 0.004f, float boundRadius = 0.3f,
                        float alphaThresh = 0.5f, float truncMultiplier = 4.0f);
    void exportSplat(const std::string &path);
    // The unprojected depth of every training camera as a coloured PLY
    // point cloud (Model::exportPointCloud, driven by the reference CLI's
    // --export-point-cloud, cli/msplat.cpp:285-291); returns the point count.
    int64_t exportPointCloud(const std::string &path, float alphaThresh = 0.5f);
    void saveCheckpoint(const std::string &path);
    int loadCheckpoint(const std::string &path);
    int splatCount() const;
    int iteration() const;

    // Extensions (no counterpart in the reference): the densification cap
    // (250000 there, model.cpp:249) and the cull opacity threshold (0.1,
    // model.cpp:273).
    void setMaxSplats(int maxSplats);
    void setCullAlphaThresh(float thresh);
    // Replaces the scene with a Gaussian PLY (the reference CLI's --resume,
    // Model::loadPly, core/src/model.cpp:329-340; 3-scale rows keep their
    // first two scales) and resets the optimiser; the iteration becomes the
    // step recorded in the file.  Returns it.
    int loadPly(const std::string &path);
    Primitive primitive() const;

private:
    struct Impl;
    std::unique_ptr<Impl> impl;
};

void sync();
void cleanup();

}  // namespace msplat
