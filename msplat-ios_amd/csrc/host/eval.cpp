// eval.cpp -- host-side image metrics for Trainer::evaluate: PSNR, L1 and
// SSIM with an 11-tap Gaussian window (sigma 1.5) and clamp-to-edge
// padding (model.cpp:26-43 and ssim.cpp:64-123 of the reference; the
// training loss pads with zeros instead, a difference the reference has
// too).  Inputs are host tensors [H,W,C] of equal shape.
#include <cmath>
#include <stdexcept>
#include <vector>

#include "model.hpp"

namespace {

void check_pair(const MTensor &a, const MTensor &b) {
    if (a.isGpu() || b.isGpu()) throw std::invalid_argument("metrics take host tensors");
    if (a.shape() != b.shape()) throw std::invalid_argument("metric inputs differ in shape");
}

void blur_clamped(const float *in, float *out, float *tmp, int H, int W, const float *k, int ks) {
    const int pad = ks / 2;
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            float s = 0;
            for (int j = 0; j < ks; ++j) {
                const int sx = std::min(std::max(x + j - pad, 0), W - 1);
                s += in[y * W + sx] * k[j];
            }
            tmp[y * W + x] = s;
        }
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            float s = 0;
            for (int j = 0; j < ks; ++j) {
                const int sy = std::min(std::max(y + j - pad, 0), H - 1);
                s += tmp[sy * W + x] * k[j];
            }
            out[y * W + x] = s;
        }
}

}  // namespace

float psnr(const MTensor &rendered, const MTensor &gt) {
    check_pair(rendered, gt);
    const int64_t n = rendered.numel();
    const float *r = rendered.data<float>(), *g = gt.data<float>();
    double mse = 0;
    for (int64_t i = 0; i < n; ++i) {
        const double d = r[i] - g[i];
        mse += d * d;
    }
    mse /= (double)n;
    return 10.0f * std::log10(1.0 / mse);
}

float l1_loss(const MTensor &rendered, const MTensor &gt) {
    check_pair(rendered, gt);
    const int64_t n = rendered.numel();
    const float *r = rendered.data<float>(), *g = gt.data<float>();
    double s = 0;
    for (int64_t i = 0; i < n; ++i) s += std::abs(r[i] - g[i]);
    return (float)(s / (double)n);
}

float ssim_eval(const MTensor &rendered, const MTensor &gt, int windowSize, float sigma) {
    check_pair(rendered, gt);
    if (rendered.ndim() != 3) throw std::invalid_argument("ssim_eval takes [H,W,C] images");
    const int H = (int)rendered.size(0), W = (int)rendered.size(1), C = (int)rendered.size(2), HW = H * W;
    std::vector<float> k(windowSize);
    float ks = 0;
    for (int i = 0; i < windowSize; ++i) {
        const float x = (float)(i - windowSize / 2);
        k[i] = std::exp(-(x * x) / (2.0f * sigma * sigma));
        ks += k[i];
    }
    for (auto &v : k) v /= ks;
    const float *r = rendered.data<float>(), *g = gt.data<float>();
    std::vector<float> a(HW), b(HW), aa(HW), bb(HW), ab(HW), m1(HW), m2(HW), s11(HW), s22(HW), s12(HW), tmp(HW);
    const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
    double sum = 0;
    int64_t count = 0;
    for (int c = 0; c < C; ++c) {
        for (int i = 0; i < HW; ++i) {
            a[i] = r[i * C + c];
            b[i] = g[i * C + c];
            aa[i] = a[i] * a[i];
            bb[i] = b[i] * b[i];
            ab[i] = a[i] * b[i];
        }
        blur_clamped(a.data(), m1.data(), tmp.data(), H, W, k.data(), windowSize);
        blur_clamped(b.data(), m2.data(), tmp.data(), H, W, k.data(), windowSize);
        blur_clamped(aa.data(), s11.data(), tmp.data(), H, W, k.data(), windowSize);
        blur_clamped(bb.data(), s22.data(), tmp.data(), H, W, k.data(), windowSize);
        blur_clamped(ab.data(), s12.data(), tmp.data(), H, W, k.data(), windowSize);
        for (int i = 0; i < HW; ++i) {
            const float mm1 = m1[i] * m1[i], mm2 = m2[i] * m2[i], mm12 = m1[i] * m2[i];
            const float num = (2.0f * mm12 + C1) * (2.0f * (s12[i] - mm12) + C2);
            const float den = (mm1 + mm2 + C1) * ((s11[i] - mm1) + (s22[i] - mm2) + C2);
            sum += num / den;
            ++count;
        }
    }
    return (float)(sum / (double)count);
}
