// input_data.cpp -- camera image handling, train/test split, scene
// normalisation and random point initialisation
// (core/src/input_data.cpp:17-252, 351-420 of the reference).
#include "input_data.hpp"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <iostream>
#include <random>
#include <stdexcept>

void Camera::loadImage(float downscaleFactor) {
    Image raw = image.empty() ? imreadRGB(filePath) : image;
    if (raw.empty()) return;
    // metadata size differs from the decoded image: rescale the intrinsics
    if (width > 0 && height > 0 && (raw.width != width || raw.height != height)) {
        const float sx = (float)raw.width / (float)width, sy = (float)raw.height / (float)height;
        fx *= sx;
        fy *= sy;
        cx *= sx;
        cy *= sy;
        width = raw.width;
        height = raw.height;
    } else if (width == 0 || height == 0) {
        width = raw.width;
        height = raw.height;
    }
    if (downscaleFactor > 1.0f) {
        const int nw = (int)(width / downscaleFactor), nh = (int)(height / downscaleFactor);
        raw = resizeArea(raw, nw, nh);
        const float s = 1.0f / downscaleFactor;
        fx *= s;
        fy *= s;
        cx *= s;
        cy *= s;
        width = nw;
        height = nh;
    }
    if (hasDistortion()) {
        UndistortResult u = undistortImage(raw, fx, fy, cx, cy, k1, k2, p1, p2, k3);
        raw = std::move(u.image);
        fx = u.fx;
        fy = u.fy;
        cx = u.cx;
        cy = u.cy;
        width = u.width;
        height = u.height;
        k1 = k2 = k3 = p1 = p2 = 0;
    }
    image = std::move(raw);
    imagePyramids.clear();
    mtensorImageCache.clear();
}

Image Camera::getImage(int downscaleFactor) {
    if (downscaleFactor <= 1) return image;
    auto it = imagePyramids.find(downscaleFactor);
    if (it != imagePyramids.end()) return it->second;
    Image scaled = resizeArea(image, image.width / downscaleFactor, image.height / downscaleFactor);
    imagePyramids[downscaleFactor] = scaled;
    return scaled;
}

MTensor &Camera::getGPUImage(int downscaleFactor) {
    auto it = mtensorImageCache.find(downscaleFactor);
    if (it != mtensorImageCache.end()) return it->second;
    Image img = getImage(downscaleFactor);
    if (img.empty()) throw std::runtime_error("camera has no image: " + filePath);
    MTensor t = MTensor::device({img.height, img.width, 3}, DType::Float32);
    t.copy_from_host(img.ptr(), img.data.size() * sizeof(float));
    return mtensorImageCache[downscaleFactor] = t;
}

std::tuple<std::vector<Camera>, Camera *> InputData::getCameras(bool validate, const std::string &valImage) {
    if (!validate || cameras.empty()) return {cameras, nullptr};
    int val = -1;
    if (valImage == "random") {
        std::mt19937 rng(42);
        val = (int)(rng() % cameras.size());
    } else {
        for (int i = 0; i < (int)cameras.size(); ++i)
            if (cameras[i].filePath.find(valImage) != std::string::npos) {
                val = i;
                break;
            }
    }
    if (val < 0) val = 0;
    std::vector<Camera> train;
    for (int i = 0; i < (int)cameras.size(); ++i)
        if (i != val) train.push_back(cameras[i]);
    return {train, &cameras[val]};
}

std::tuple<std::vector<Camera>, std::vector<Camera>> InputData::splitTrainTest(int testEvery) {
    if (testEvery <= 0) throw std::invalid_argument("test_every must be positive");
    std::vector<Camera> train, test;
    for (int i = 0; i < (int)cameras.size(); ++i) (i % testEvery == 0 ? test : train).push_back(cameras[i]);
    return {train, test};
}

void autoScaleAndCenter(InputData &data) {
    if (data.cameras.empty()) return;
    float mean[3] = {0.f, 0.f, 0.f};
    for (auto &c : data.cameras)
        for (int k = 0; k < 3; ++k) mean[k] += c.camToWorld[4 * k + 3];
    const int n = (int)data.cameras.size();
    for (int k = 0; k < 3; ++k) {
        mean[k] /= n;
        data.translation[k] = mean[k];
    }
    float max_abs = 0.f;
    for (auto &c : data.cameras)
        for (int k = 0; k < 3; ++k) {
            c.camToWorld[4 * k + 3] -= mean[k];
            max_abs = std::max(max_abs, std::abs(c.camToWorld[4 * k + 3]));
        }
    data.scale = max_abs > 0 ? 1.0f / max_abs : 1.0f;
    for (auto &c : data.cameras)
        for (int k = 0; k < 3; ++k) c.camToWorld[4 * k + 3] *= data.scale;
    for (int64_t i = 0; i < data.points.count; ++i)
        for (int k = 0; k < 3; ++k) data.points.xyz[3 * i + k] = (data.points.xyz[3 * i + k] - mean[k]) * data.scale;
}

void faceCenteredTransform(InputData &data, float faceDistance, float scaleFactor) {
    if (data.cameras.empty()) return;
    // the point faceDistance in front of the first camera (its -Z axis in
    // the OpenGL convention): M0 (0, 0, -d, 1)
    const float *M0 = data.cameras.front().camToWorld;
    float face[3];
    for (int k = 0; k < 3; ++k) face[k] = M0[4 * k + 2] * (-faceDistance) + M0[4 * k + 3];
    for (int k = 0; k < 3; ++k) data.translation[k] = face[k];
    data.scale = scaleFactor;
    for (auto &c : data.cameras)
        for (int k = 0; k < 3; ++k) c.camToWorld[4 * k + 3] = (c.camToWorld[4 * k + 3] - face[k]) * scaleFactor;
    for (int64_t i = 0; i < data.points.count; ++i)
        for (int k = 0; k < 3; ++k) data.points.xyz[3 * i + k] = (data.points.xyz[3 * i + k] - face[k]) * scaleFactor;
}

void initializeRandomPoints(InputData &data, int64_t numPoints, float extent) {
    std::mt19937 rng(42);
    std::uniform_real_distribution<float> dxyz(-extent, extent);
    std::uniform_int_distribution<int> drgb(0, 255);
    data.points.xyz.resize(numPoints * 3);
    data.points.rgb.resize(numPoints * 3);
    for (int64_t i = 0; i < numPoints; ++i) {
        for (int k = 0; k < 3; ++k) data.points.xyz[3 * i + k] = dxyz(rng);
        for (int k = 0; k < 3; ++k) data.points.rgb[3 * i + k] = (uint8_t)drgb(rng);
    }
    data.points.count = numPoints;
}

void initializeRandomPointsCameraAware(InputData &data, int64_t numPoints, float radiusFrac) {
    if (data.cameras.empty()) {
        initializeRandomPoints(data, numPoints, 1.3f);
        return;
    }
    float mean_dist = 0.f;
    for (const auto &c : data.cameras) {
        const float x = c.camToWorld[3], y = c.camToWorld[7], z = c.camToWorld[11];
        mean_dist += std::sqrt(x * x + y * y + z * z);
    }
    mean_dist /= (float)data.cameras.size();
    const float radius = std::max(mean_dist * radiusFrac, 0.05f);
    std::mt19937 rng(42);
    std::normal_distribution<float> dn(0.0f, 1.0f);
    std::uniform_real_distribution<float> du(0.0f, 1.0f);
    std::uniform_int_distribution<int> drgb(0, 1);
    data.points.xyz.resize(numPoints * 3);
    data.points.rgb.resize(numPoints * 3);
    for (int64_t i = 0; i < numPoints; ++i) {
        const float gx = dn(rng), gy = dn(rng), gz = dn(rng);
        const float inv = 1.0f / std::sqrt(gx * gx + gy * gy + gz * gz + 1e-12f);
        const float r = radius * std::cbrt(du(rng));
        data.points.xyz[3 * i + 0] = gx * inv * r;
        data.points.xyz[3 * i + 1] = gy * inv * r;
        data.points.xyz[3 * i + 2] = gz * inv * r;
        for (int k = 0; k < 3; ++k) data.points.rgb[3 * i + k] = (uint8_t)drgb(rng);
    }
    data.points.count = numPoints;
}

Image resizeArea(const Image &src, int dstW, int dstH) {
    if (dstW <= 0 || dstH <= 0) throw std::invalid_argument("resizeArea: empty target size");
    Image dst;
    dst.width = dstW;
    dst.height = dstH;
    dst.data.assign((size_t)dstW * dstH * 3, 0.0f);
    const float sx = (float)src.width / dstW, sy = (float)src.height / dstH;
    for (int dy = 0; dy < dstH; ++dy) {
        const float y0 = dy * sy, y1 = (dy + 1) * sy;
        const int iy0 = (int)y0, iy1 = std::min((int)std::ceil(y1), src.height);
        for (int dx = 0; dx < dstW; ++dx) {
            const float x0 = dx * sx, x1 = (dx + 1) * sx;
            const int ix0 = (int)x0, ix1 = std::min((int)std::ceil(x1), src.width);
            float acc[3] = {0.f, 0.f, 0.f}, area = 0.f;
            for (int iy = iy0; iy < iy1; ++iy) {
                const float wy = std::min((float)(iy + 1), y1) - std::max((float)iy, y0);
                for (int ix = ix0; ix < ix1; ++ix) {
                    const float a = (std::min((float)(ix + 1), x1) - std::max((float)ix, x0)) * wy;
                    const float *p = &src.data[((size_t)iy * src.width + ix) * 3];
                    for (int c = 0; c < 3; ++c) acc[c] += p[c] * a;
                    area += a;
                }
            }
            float *o = &dst.data[((size_t)dy * dstW + dx) * 3];
            const float inv = 1.0f / area;
            for (int c = 0; c < 3; ++c) o[c] = acc[c] * inv;
        }
    }
    return dst;
}
