// model.hpp -- the trainable 2DGS scene: parameters, Adam state, the
// densification policy and checkpoint / PLY / .splat I/O, with the member
// names and behaviour of the reference's Model (core/include/model.hpp:30-149,
// core/src/model.cpp).  All per-splat tensors live in HBM in capacity-sized
// backing buffers; the six parameter tensors and the twelve Adam moments
// are views of their first num_active rows (model.cpp:188-199).
#pragma once

#include <string>
#include <tuple>
#include <vector>

#include "bindings.hpp"
#include "input_data.hpp"

int numShBases(int degree);
// Metrics on host tensors of equal shape (model.cpp:26-43, ssim.cpp:64-123).
float psnr(const MTensor &rendered, const MTensor &gt);
float l1_loss(const MTensor &rendered, const MTensor &gt);
float ssim_eval(const MTensor &rendered, const MTensor &gt, int windowSize = 11, float sigma = 1.5f);

// Scales per splat: kScaleDim = 2 (2DGS surfel, model.hpp:20).  A Model
// built with scaleDim 3 trains 3D Gaussians (the 3DGS mode).
constexpr int kScaleDim = 2;

// Mean distance of every point to its k nearest neighbours (the initial
// splat scale, kdtree_tensor.hpp:30-42), by a uniform-grid search.
std::vector<float> knnMeanDistance(const float *xyz, int64_t n, int k = 3);

struct Model {
    Model(const InputData &inputData, int numCameras, int numDownscales, int resolutionSchedule, int shDegree,
          int shDegreeInterval, int refineEvery, int warmupLength, int resetAlphaEvery, float densifyGradThresh,
          float densifySizeThresh, int stopScreenSizeAt, float splitScreenSize, int maxSteps, bool keepCrs,
          const float *bgColor = nullptr, int scaleDim = kScaleDim);
    ~Model() { releaseOptimizers(); }
    Model(const Model &) = delete;
    Model &operator=(const Model &) = delete;

    void setupOptimizers();
    void releaseOptimizers();
    void schedulersStep(int step);
    int getDownscaleFactor(int step);
    void afterTrain(int step);
    void save(const std::string &filename, int step);
    void savePly(const std::string &filename, int step);
    void saveSplat(const std::string &filename);
    int loadPly(const std::string &filename);
    void saveCheckpoint(const std::string &filename, int step);
    int loadCheckpoint(const std::string &filename);

    struct CamSetup {
        float fx, fy, cx, cy;
        int height, width, degree, degreesToUse;
        std::tuple<int, int, int> tileBounds;
        float cam_pos[3];
        MTensor viewMat, projViewMat;  // host 4x4, row-major
    };
    CamSetup prepareCam(Camera &cam, int step);
    // One training step on camera `cam` against `gt` ([H,W,3] device):
    // forward, SSIM + L1, backward and the six Adam updates (fused into the
    // projection backward).  Returns the loss (model.cpp:762-829).
    float fullIteration(Camera &cam, int step, MTensor &gt, float ssimWeight);
    // Rendered image [H,W,3] (device view of the engine's output buffer,
    // valid until the next render or step).
    MTensor render(Camera &cam, int step);

    // Point cloud, TSDF fusion and mesh extraction (model.hpp:42-77,
    // model.cpp:565-757).  Every pixel with alpha >= alphaThresh of every
    // camera's render becomes one (x, y, z, r, g, b) PLY vertex; returns the
    // number written.
    int64_t exportPointCloud(std::vector<Camera> &cameras, int step, float alphaThresh, const std::string &outPath);
    // A [Dz, Dy, Dx, 2] f32 (sdf, weight) grid in HBM, zero-initialised by
    // makeVoxelGrid.
    struct VoxelGrid {
        float origin[3];  // world position of voxel (0, 0, 0)'s corner
        int dims[3];      // (Dx, Dy, Dz)
        float voxelSize;
        MTensor data;
    };
    // A cube of side 2 * boundRadius centred on the world origin, voxels of
    // voxelSize; throws if it would exceed memoryCapMB.
    VoxelGrid makeVoxelGrid(const std::vector<Camera> &cameras, float voxelSize, float boundRadius,
                            int memoryCapMB = 512) const;
    // Fold every camera's rendered median depth (weighted by its alpha) into
    // the grid, truncated at +-truncDist.
    void integrateTSDF(VoxelGrid &grid, std::vector<Camera> &cameras, int step, float truncDist, float alphaThresh);
    // Marching cubes on the grid -> non-indexed triangle PLY; returns the
    // number of triangles written (at most maxTriangles).
    int64_t extractMesh(const VoxelGrid &grid, const std::string &outPath, int maxTriangles = 4'000'000);

    MTensor means, scales, quats, featuresDc, featuresRest, opacities;
    // 2: surfels (the reference's 2DGS step); 3: 3D Gaussians projected with
    // the EWA helpers (render / train step / densify of the 3DGS mode).  The
    // 3DGS mode renders image and transmittance only, so the point cloud and
    // mesh exports, which need depth, are 2DGS-only.
    int scaleDim = kScaleDim;

    static constexpr int N_ADAM_GROUPS = 6;
    MTensor adam_exp_avg[N_ADAM_GROUPS];
    MTensor adam_exp_avg_sq[N_ADAM_GROUPS];
    int adam_step_count = 0;
    float adam_lr[N_ADAM_GROUPS] = {};
    float adam_beta1 = 0.9f, adam_beta2 = 0.999f, adam_eps = 1e-8f;
    float means_lr_init = 0, means_lr_final = 0;

    MTensor means_buf, scales_buf, quats_buf, featuresDc_buf, featuresRest_buf, opacities_buf;
    MTensor adam_exp_avg_buf[N_ADAM_GROUPS], adam_exp_avg_sq_buf[N_ADAM_GROUPS];
    int num_active = 0, buf_capacity = 0;
    void refreshViews();
    void ensureCapacity(int needed);

    MTensor densify_random_samples;  // device [capacity, 3]: the split offsets' normal samples

    MTensor radii;
    int lastHeight = 0;
    int lastWidth = 0;

    MTensor xysGradNorm, visCounts, max2DSize;
    MTensor backgroundColor;  // device [3]

    int numCameras;
    int numDownscales;
    int resolutionSchedule;
    int shDegree;
    int shDegreeInterval;
    int refineEvery;
    int warmupLength;
    int resetAlphaEvery;
    int stopSplitAt;
    float densifyGradThresh;
    float densifySizeThresh;
    int stopScreenSizeAt;
    float splitScreenSize;
    int maxSteps;
    bool keepCrs;
    // Densification stops growing the model at this many splats
    // (kMaxSplats = 250000 in model.cpp:249); settable for larger scenes.
    int maxSplats = 250000;
    // Densification cull threshold on sigmoid(opacity) (0.1 in model.cpp:273).
    float cullAlphaThresh = 0.1f;

    float scale;
    float translation[3] = {};

private:
    void allocStats(int n);
};
