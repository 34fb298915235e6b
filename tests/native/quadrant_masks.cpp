// Test helper (CPU only): checks that the rasterizer's quadrant masks
// (msd::mask_record per splat and msd::quad_mask per tile, compiled here for
// the host from the product header)
// are conservative.  For every visible splat and every tile its screen box
// meets, every pixel whose alpha reaches 1/255 in fp64 (with a 1e-4 relative
// margin, far above the fp32 evaluation's rounding) must lie in a quadrant
// whose mask bit is set.  The fp64 evaluation restates
// nd_rasterize_forward_2dgs_kernel's pair test (msplat_metal.metal:651-683).
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <vector>

#include "ms_device.h"

using namespace msd;

namespace {

// splat_reach (the kernels' tau) with the host's logf
float reach(float opa) {
    const float a = 255.0f * opa;
    if (!(a >= 0.999f)) return -1.0f;
    const float t = std::fmax(2.0f * std::log(a), 0.0f);
    return t * 1.0001f + 1e-3f;
}

}  // namespace

// transmats [n,9] (Tu, Tv, Tw), xys [n,2], normal_opac [n,4] (opacity logit
// in column 3), radii [n], rect [n,4] (the tiles x0, y0, x1, y1 the splat is
// binned into, half-open).  Every (tile, splat) pair the rasterizer sees is
// checked.  Returns the number of (pixel, splat) pairs that pass in fp64 but
// whose quadrant bit is clear; out[0] = pairs checked, out[1] = tiles whose
// box mask is set, out[2] = tiles whose fine mask is set, out[3] = quadrant
// bits set by the box mask, out[4] = by the fine mask.  tau_scale (1 in the
// real check) scales the reach the masks are computed from: below 1 it
// plants a too-tight mask, which the check must report.
extern "C" int64_t qm_check(int n, const float *transmats, const float *xys, const float *normal_opac,
                            const int32_t *radii, const int32_t *rect, int W, int H, float tau_scale,
                            int64_t out[5]) {
    const int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
    int64_t misses = 0, checked = 0, box_tiles = 0, fine_tiles = 0, box_bits = 0, fine_bits = 0;
    for (int g = 0; g < n; ++g) {
        if (radii[g] <= 0) continue;
        const float *T = transmats + 9 * (size_t)g;
        const float xs = xys[2 * g], ys = xys[2 * g + 1];
        const float opa = 1.0f / (1.0f + std::exp(-normal_opac[4 * g + 3]));
        const float4 q0 = make_float4(T[0], T[1], T[2], T[3]);
        const float4 q1 = make_float4(T[4], T[5], T[6], T[7]);
        const float4 q2 = make_float4(T[8], xs, ys, opa);
        const float tau = reach(opa) * tau_scale;
        if (tau < 0.0f) continue;
        f3 R0, nAx, nAy;
        centred_rows({T[0], T[1], T[2]}, {T[3], T[4], T[5]}, {T[6], T[7], T[8]}, xs, ys, R0, nAx, nAy);
        const int *rc = rect + 4 * (size_t)g;
        const int tx0 = std::max(0, rc[0]), ty0 = std::max(0, rc[1]);
        const int tx1 = std::min(tiles_x, rc[2]) - 1, ty1 = std::min(tiles_y, rc[3]) - 1;
        // the projection's per-splat part, over the splat's tile rectangle
        float lp_r2;
        const MaskRec mr = mask_record(q0, q1, q2, tau, R0, nAx, nAy, tx0, ty0, tx1 + 1, ty1 + 1, lp_r2);
        const float4 box = mr.box;
        const double Tu[3] = {T[0], T[1], T[2]}, Tv[3] = {T[3], T[4], T[5]}, Tw[3] = {T[6], T[7], T[8]};
        for (int ty = ty0; ty <= ty1; ++ty)
            for (int tx = tx0; tx <= tx1; ++tx) {
                const float sx0 = (float)(tx * 16), sy0 = (float)(ty * 16);
                const int mbox = strip_mask(box, sx0, sy0);
                const int m = quad_mask(mr, lp_r2, xs, ys, sx0, sy0);
                box_tiles += mbox != 0;
                fine_tiles += m != 0;
                box_bits += __builtin_popcount(mbox);
                fine_bits += __builtin_popcount(m);
                for (int w = 0; w < 4; ++w)
                    for (int l = 0; l < 64; ++l) {
                        const int pxi = tx * 16 + lane_px(w, l), pyi = ty * 16 + lane_py(w, l);
                        if (pxi >= W || pyi >= H) continue;
                        const double px = pxi, py = pyi;
                        const double k[3] = {px * Tw[0] - Tu[0], px * Tw[1] - Tu[1], px * Tw[2] - Tu[2]};
                        const double lv[3] = {py * Tw[0] - Tv[0], py * Tw[1] - Tv[1], py * Tw[2] - Tv[2]};
                        const double rx = k[1] * lv[2] - k[2] * lv[1];
                        const double ry = k[2] * lv[0] - k[0] * lv[2];
                        const double rz = k[0] * lv[1] - k[1] * lv[0];
                        if (rz == 0.0) continue;
                        const double u = rx / rz, v = ry / rz;
                        const double dx = xs - px, dy = ys - py;
                        const double rho = std::fmin(u * u + v * v, 2.0 * (dx * dx + dy * dy));
                        const double depth = u * Tw[0] + v * Tw[1] + Tw[2];
                        const double alpha = std::fmin(0.99, opa * std::exp(-0.5 * rho));
                        ++checked;
                        if (depth >= 0.2 * (1.0 - 1e-6) && alpha >= (1.0 / 255.0) * (1.0 - 1e-4) && !((m >> w) & 1))
                            ++misses;
                    }
            }
    }
    out[0] = checked;
    out[1] = box_tiles;
    out[2] = fine_tiles;
    out[3] = box_bits;
    out[4] = fine_bits;
    return misses;
}

// The 3DGS mode's masks (msd::gauss3_box per splat, msd::strip_mask per
// tile).  xys [n,2], conics [n,3] (a, b, c), cov2d [n,3] (xx, xy, yy),
// opacity logits [n], radii [n], rect [n,4] as qm_check.  A pixel passes
// when alpha = min(0.99, opacity exp(-rho / 2)) reaches 1/255 for some rho
// within the fp32 evaluation's rounding of rho = a dx^2 + c dy^2 + 2 b dx dy
// (fp64, from the fp32 conic; 6 units of roundoff of the sum of the terms'
// magnitudes, above the five roundings of the fp32 evaluation).
// Returns the passing pixels whose quadrant bit is clear; out as qm_check
// (out[2] = out[1], out[4] = out[3]: there is no finer mask).
extern "C" int64_t qm3_check(int n, const float *xys, const float *conics, const float *cov2d,
                             const float *opac_logit, const int32_t *radii, const int32_t *rect, int W, int H,
                             float tau_scale, int64_t out[5]) {
    const int tiles_x = (W + 15) / 16, tiles_y = (H + 15) / 16;
    int64_t misses = 0, checked = 0, box_tiles = 0, box_bits = 0;
    const double ulp = std::ldexp(1.0, -24);
    for (int g = 0; g < n; ++g) {
        if (radii[g] <= 0) continue;
        const float xs = xys[2 * g], ys = xys[2 * g + 1];
        const float opa = 1.0f / (1.0f + std::exp(-opac_logit[g]));
        const float tau = reach(opa) * tau_scale;
        const float4 box = gauss3_box(xs, ys, cov2d + 3 * (size_t)g, tau);
        const double a = conics[3 * g], b = conics[3 * g + 1], c = conics[3 * g + 2];
        const int *rc = rect + 4 * (size_t)g;
        const int tx0 = std::max(0, rc[0]), ty0 = std::max(0, rc[1]);
        const int tx1 = std::min(tiles_x, rc[2]) - 1, ty1 = std::min(tiles_y, rc[3]) - 1;
        for (int ty = ty0; ty <= ty1; ++ty)
            for (int tx = tx0; tx <= tx1; ++tx) {
                const int m = strip_mask(box, (float)(tx * 16), (float)(ty * 16));
                box_tiles += m != 0;
                box_bits += __builtin_popcount(m);
                for (int w = 0; w < 4; ++w)
                    for (int l = 0; l < 64; ++l) {
                        const int pxi = tx * 16 + lane_px(w, l), pyi = ty * 16 + lane_py(w, l);
                        if (pxi >= W || pyi >= H) continue;
                        const double dx = (double)(xs - (float)pxi), dy = (double)(ys - (float)pyi);
                        const double t1 = a * dx * dx, t2 = c * dy * dy, t3 = 2.0 * b * dx * dy;
                        const double rho = t1 + t2 + t3;
                        const double err = 6.0 * ulp * (std::fabs(t1) + std::fabs(t2) + std::fabs(t3));
                        const double alpha = std::fmin(0.99, opa * std::exp(-0.5 * std::fmax(rho - err, 0.0)));
                        ++checked;
                        if (alpha >= (1.0 / 255.0) * (1.0 - 1e-6) && !((m >> w) & 1)) ++misses;
                    }
            }
    }
    out[0] = checked;
    out[1] = out[2] = box_tiles;
    out[3] = out[4] = box_bits;
    return misses;
}

// The rasterizers' workgroup -> tile order (msd::xcd_strip_tile): the
// number of tiles of a tx x ty grid that the xcd_strip_grid(tx, ty)
// workgroups do not cover exactly once (0 for a bijection), or -1 when a
// workgroup maps outside the grid.
extern "C" int64_t tile_order_check(int tx, int ty) {
    const int T = tx * ty, G = xcd_strip_grid(tx, ty);
    std::vector<int> hits(T, 0);
    for (int b = 0; b < G; ++b) {
        const int t = xcd_strip_tile(b, tx, ty);
        if (t < -1 || t >= T) return -1;
        if (t >= 0) ++hits[t];
    }
    int64_t bad = 0;
    for (int t = 0; t < T; ++t) bad += hits[t] != 1;
    return bad;
}
