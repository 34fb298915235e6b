// input_data.hpp -- cameras, images and the initial point cloud of a scene,
// with the reference's type and member names (core/include/input_data.hpp:
// Image, Camera, Points, InputData).
//
// Camera images live in host memory as float32 RGB [0,1] HWC; the
// training target of a camera at a given downscale factor is uploaded to
// HBM once and cached (getGPUImage), as the reference caches its Metal
// buffers (input_data.cpp:74-84).
#pragma once

#include <cstdint>
#include <map>
#include <string>
#include <tuple>
#include <vector>

#include "mtensor.hpp"

struct Image {
    std::vector<float> data;  // width * height * 3, RGB in [0,1]
    int width = 0, height = 0;

    bool empty() const { return data.empty(); }
    float *ptr() { return data.data(); }
    const float *ptr() const { return data.data(); }
};

struct Camera {
    int width = 0, height = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0;
    float k1 = 0, k2 = 0, k3 = 0, p1 = 0, p2 = 0;
    float camToWorld[16] = {};  // 4x4 row-major camera-to-world, OpenGL axes (Y up, Z back)
    std::string filePath;

    Image image;
    std::map<int, Image> imagePyramids;
    std::map<int, MTensor> mtensorImageCache;

    // Decodes filePath (unless an image is already attached), rescales the
    // intrinsics to the decoded size, applies the dataset downscale factor
    // (box filter) and undistorts (input_data.cpp:17-52).
    void loadImage(float downscaleFactor);
    // Box-filtered pyramid level (input_data.cpp:54-64).
    Image getImage(int downscaleFactor);
    // Device copy of getImage(downscaleFactor), cached (input_data.cpp:66-72).
    MTensor &getGPUImage(int downscaleFactor);
    bool hasDistortion() const { return k1 != 0 || k2 != 0 || k3 != 0 || p1 != 0 || p2 != 0; }
};

struct Points {
    std::vector<float> xyz;    // count * 3
    std::vector<uint8_t> rgb;  // count * 3
    int64_t count = 0;
};

struct InputData {
    std::vector<Camera> cameras;
    float scale = 1.0f;
    float translation[3] = {};
    Points points;

    // All cameras (validate = false), or all but one validation camera
    // (input_data.cpp:163-183).
    std::tuple<std::vector<Camera>, Camera *> getCameras(bool validate, const std::string &valImage = "random");
    // Cameras 0, testEvery, 2 testEvery, ... are held out for testing
    // (input_data.cpp:185-195).
    std::tuple<std::vector<Camera>, std::vector<Camera>> splitTrainTest(int testEvery);
};

// Loaders: COLMAP (sparse/0 binary or text), Nerfstudio (transforms.json)
// and Polycam (cameras/*.json), auto-detected from the directory layout
// (input_data.cpp:300-340).  Images are PNG (8/16-bit, any colour type) or
// binary PPM/PGM.
InputData inputDataFromX(const std::string &path, const std::string &colmapImagePath = "");

// Scene normalisation: subtract the mean camera position, scale so the
// largest coordinate is 1 (input_data.cpp:124-175).
void autoScaleAndCenter(InputData &data);

// The face-capture normalisation (input_data.cpp:82-110): the origin moves
// to the point faceDistance in front of the first camera and every camera
// position and point is scaled by scaleFactor about it.  The Nerfstudio
// loader applies it instead of autoScaleAndCenter when the environment sets
// MSPLAT_FACE_DISTANCE > 0 (MSPLAT_SCALE_FACTOR, default 10;
// load_nerfstudio.cpp:135-146).
void faceCenteredTransform(InputData &data, float faceDistance, float scaleFactor);

// Fallback initialisation without a point cloud: uniform points in
// [-extent, extent]^3 with random colours (input_data.cpp:351-369).
void initializeRandomPoints(InputData &data, int64_t numPoints = 100000, float extent = 1.3f);
// Fallback used by the loaders: points in a ball of radiusFrac x (mean
// camera distance) about the origin, near-black colours
// (input_data.cpp:371-420).
void initializeRandomPointsCameraAware(InputData &data, int64_t numPoints = 100000, float radiusFrac = 0.35f);

// Image utilities (core/src/loaders/image_io.cpp).
Image imreadRGB(const std::string &path);
Image resizeArea(const Image &src, int dstW, int dstH);
void imwriteRGB(const std::string &path, const Image &img);  // binary PPM

struct UndistortResult {
    Image image;
    float fx, fy, cx, cy;
    int width, height;
};
UndistortResult undistortImage(const Image &src, float fx, float fy, float cx, float cy, float k1, float k2,
                               float p1, float p2, float k3);

// Point cloud readers.
Points readPly(const std::string &path);
Points readColmapPoints(const std::string &path);
