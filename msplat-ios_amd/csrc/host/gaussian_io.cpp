// gaussian_io.cpp -- trained-scene export / import: the Gaussian PLY
// layout shared with the 3DGS tooling and the 32-byte .splat viewer format
// (core/src/loaders/save_gaussians.cpp of the reference).
//
// PLY vertex row: x y z, nx ny nz (zero), f_dc_0..2, f_rest_0..3K-1 (the
// [K,3] SH rest coefficients written channel-major), opacity (logit),
// scale_0..S-1 (log), rot_0..3 (w x y z), all float32 little-endian.
// .splat row: position (3 f32), linear scale (3 f32, the missing third axis
// of a surfel written as 1e-5), RGBA (4 u8, SH DC colour and sigmoid
// opacity), rotation (4 u8, q * 128 + 128), sorted by decreasing
// scale x opacity.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <filesystem>
#include <fstream>
#include <numeric>
#include <stdexcept>
#include <string>

#include "model.hpp"

namespace {

constexpr double kC0 = 0.28209479177387814;

std::vector<float> host_copy(const MTensor &t) {
    std::vector<float> v((size_t)t.numel());
    t.copy_to_host(v.data());
    return v;
}

}  // namespace

void Model::save(const std::string &filename, int step) {
    const std::string ext = std::filesystem::path(filename).extension().string();
    if (ext == ".splat")
        saveSplat(filename);
    else
        savePly(filename, step);
    std::fprintf(stderr, "Saved %s\n", filename.c_str());
}

void Model::savePly(const std::string &filename, int step) {
    msplat_gpu_sync();
    const int64_t n = means.size(0);
    const int nfr = (int)featuresRest.size(-2), ns = (int)scales.size(1);
    const auto m = host_copy(means), s = host_copy(scales), q = host_copy(quats);
    const auto dc = host_copy(featuresDc), fr = host_copy(featuresRest), op = host_copy(opacities);
    std::ofstream o(filename, std::ios::binary);
    if (!o) throw std::runtime_error("Cannot open PLY for writing: " + filename);
    o << "ply\nformat binary_little_endian 1.0\n";
    o << "comment msplat v" << step << "\n";
    o << "element vertex " << n << "\n";
    o << "property float x\nproperty float y\nproperty float z\n";
    o << "property float nx\nproperty float ny\nproperty float nz\n";
    for (int i = 0; i < 3; ++i) o << "property float f_dc_" << i << "\n";
    for (int i = 0; i < 3 * nfr; ++i) o << "property float f_rest_" << i << "\n";
    o << "property float opacity\n";
    for (int i = 0; i < ns; ++i) o << "property float scale_" << i << "\n";
    o << "property float rot_0\nproperty float rot_1\nproperty float rot_2\nproperty float rot_3\n";
    o << "end_header\n";
    std::vector<float> row(3 + 3 + 3 + 3 * nfr + 1 + ns + 4);
    for (int64_t i = 0; i < n; ++i) {
        size_t c = 0;
        for (int j = 0; j < 3; ++j) row[c++] = keepCrs ? m[3 * i + j] / scale + translation[j] : m[3 * i + j];
        for (int j = 0; j < 3; ++j) row[c++] = 0.0f;
        for (int j = 0; j < 3; ++j) row[c++] = dc[3 * i + j];
        for (int ch = 0; ch < 3; ++ch)
            for (int b = 0; b < nfr; ++b) row[c++] = fr[(size_t)i * nfr * 3 + b * 3 + ch];
        row[c++] = op[i];
        for (int j = 0; j < ns; ++j)
            row[c++] = keepCrs ? std::log(std::exp(s[i * ns + j]) / scale) : s[i * ns + j];
        for (int j = 0; j < 4; ++j) row[c++] = q[4 * i + j];
        o.write((const char *)row.data(), (std::streamsize)(row.size() * sizeof(float)));
    }
    if (!o) throw std::runtime_error("Failed writing PLY: " + filename);
}

void Model::saveSplat(const std::string &filename) {
    msplat_gpu_sync();
    const int64_t n = means.size(0);
    const int ns = (int)scales.size(1);
    const auto m = host_copy(means), s = host_copy(scales), q = host_copy(quats);
    const auto dc = host_copy(featuresDc), op = host_copy(opacities);
    std::vector<float> key((size_t)n);
    for (int64_t i = 0; i < n; ++i) {
        float sz = 0.0f;
        for (int j = 0; j < ns; ++j) sz += std::exp(s[i * ns + j]);
        if (keepCrs) sz /= scale;
        key[i] = sz / (1.0f + std::exp(-op[i]));
    }
    std::vector<int64_t> idx((size_t)n);
    std::iota(idx.begin(), idx.end(), 0);
    std::stable_sort(idx.begin(), idx.end(), [&](int64_t a, int64_t b) { return key[a] > key[b]; });
    std::ofstream o(filename, std::ios::binary);
    if (!o) throw std::runtime_error("Cannot open .splat for writing: " + filename);
    for (int64_t i : idx) {
        float pos[3], sc[3] = {0.0f, 0.0f, 0.0f};
        for (int j = 0; j < 3; ++j) pos[j] = keepCrs ? m[3 * i + j] / scale + translation[j] : m[3 * i + j];
        for (int j = 0; j < ns && j < 3; ++j) sc[j] = keepCrs ? std::exp(s[i * ns + j]) / scale : std::exp(s[i * ns + j]);
        if (ns < 3) sc[2] = 1e-5f;
        uint8_t rgba[4], rot[4];
        for (int j = 0; j < 3; ++j)
            rgba[j] = (uint8_t)std::clamp(((double)dc[3 * i + j] * kC0 + 0.5) * 255.0, 0.0, 255.0);
        const float sig = 1.0f / (1.0f + std::exp(-op[i]));
        rgba[3] = (uint8_t)std::clamp(sig * 255.0f, 0.0f, 255.0f);
        for (int j = 0; j < 4; ++j) rot[j] = (uint8_t)std::clamp(q[4 * i + j] * 128.0f + 128.0f, 0.0f, 255.0f);
        o.write((const char *)pos, 12);
        o.write((const char *)sc, 12);
        o.write((const char *)rgba, 4);
        o.write((const char *)rot, 4);
    }
    if (!o) throw std::runtime_error("Failed writing .splat: " + filename);
}

// Reads a Gaussian PLY written by savePly (or 3DGS tooling with the same
// property order) into a model of scaleDim scales: a 2DGS model keeps the
// first two of a 3-scale row; a 3DGS model gives a 2-scale row a third
// scale equal to the smaller of its two.  Replaces the scene and resets the
// optimiser (model.cpp:319-330).
int Model::loadPly(const std::string &filename) {
    msplat_gpu_sync();
    std::ifstream f(filename, std::ios::binary);
    if (!f) throw std::runtime_error("Cannot open PLY file: " + filename);
    std::string line;
    std::getline(f, line);
    if (line.rfind("ply", 0) != 0) throw std::runtime_error("Not a PLY file: " + filename);
    int64_t n = 0;
    int step = 0, ndc = 0, nfr = 0, ns = 0, nprops = 0;
    bool binary_le = false;
    while (std::getline(f, line)) {
        if (!line.empty() && line.back() == '\r') line.pop_back();
        if (line == "end_header") break;
        if (line.rfind("format binary_little_endian", 0) == 0) binary_le = true;
        for (const char *pre : {"comment Generated by msplat at iteration ", "comment msplat v"})
            if (line.rfind(pre, 0) == 0) step = std::atoi(line.c_str() + std::strlen(pre));
        if (line.rfind("element vertex ", 0) == 0) n = std::atoll(line.c_str() + 15);
        if (line.rfind("property ", 0) == 0) {
            if (line.rfind("property float ", 0) != 0) throw std::runtime_error("PLY: only float properties");
            ++nprops;
        }
        if (line.rfind("property float f_dc_", 0) == 0) ++ndc;
        if (line.rfind("property float f_rest_", 0) == 0) ++nfr;
        if (line.rfind("property float scale_", 0) == 0) ++ns;
    }
    if (!binary_le) throw std::runtime_error("PLY: only binary_little_endian is supported");
    if (n <= 0) throw std::runtime_error("PLY has no vertices");
    if (ndc != 3 || nfr % 3 != 0 || (ns != 2 && ns != 3) || nprops != 3 + 3 + ndc + nfr + 1 + ns + 4)
        throw std::runtime_error("PLY: unexpected Gaussian property layout");
    const int bases = nfr / 3;
    std::vector<float> row((size_t)nprops);
    const int sd = scaleDim;
    std::vector<float> m(3 * n), dc(3 * n), fr((size_t)n * nfr), op(n), s((size_t)sd * n), q(4 * n);
    for (int64_t i = 0; i < n; ++i) {
        f.read((char *)row.data(), (std::streamsize)(row.size() * sizeof(float)));
        if (!f) throw std::runtime_error("PLY: truncated vertex data");
        size_t c = 0;
        for (int j = 0; j < 3; ++j) m[3 * i + j] = row[c++];
        c += 3;
        for (int j = 0; j < 3; ++j) dc[3 * i + j] = row[c++];
        for (int ch = 0; ch < 3; ++ch)
            for (int b = 0; b < bases; ++b) fr[(size_t)i * nfr + b * 3 + ch] = row[c++];
        op[i] = row[c++];
        for (int j = 0; j < ns; ++j) {
            if (j < sd) s[(size_t)sd * i + j] = row[c];
            ++c;
        }
        if (ns < sd) s[(size_t)sd * i + 2] = std::min(s[(size_t)sd * i], s[(size_t)sd * i + 1]);
        for (int j = 0; j < 4; ++j) q[4 * i + j] = row[c++];
    }
    if (keepCrs) {
        for (int64_t i = 0; i < n; ++i)
            for (int j = 0; j < 3; ++j) m[3 * i + j] = (m[3 * i + j] - translation[j]) * scale;
        for (auto &v : s) v = std::log(scale * std::exp(v));
    }
    auto up = [](std::vector<int64_t> shape, const std::vector<float> &v) {
        MTensor t = MTensor::device(std::move(shape), DType::Float32);
        t.copy_from_host(v.data(), v.size() * sizeof(float));
        return t;
    };
    means = up({n, 3}, m);
    scales = up({n, (int64_t)sd}, s);
    quats = up({n, 4}, q);
    featuresDc = up({n, 3}, dc);
    featuresRest = up({n, (int64_t)bases, 3}, fr);
    opacities = up({n, 1}, op);
    int deg = 0;
    while (numShBases(deg) < bases + 1 && deg < 4) ++deg;
    shDegree = deg;
    setupOptimizers();
    xysGradNorm.reset();
    visCounts.reset();
    max2DSize.reset();
    radii.reset();
    return step;
}
