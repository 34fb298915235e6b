// knn.cpp -- mean distance of each point to its k nearest neighbours, the
// initial splat scale of Model (kdtree_tensor.hpp:30-42 of the reference,
// which queries a nanoflann KD-tree for k + 1 = 4 points including the
// point itself).  Uniform-grid search: points are bucketed into cubic
// cells of about two points each and every query scans shells of cells
// outwards until the next shell cannot hold a closer point.
#include <algorithm>
#include <cmath>
#include <cstdint>
#include <limits>
#include <vector>

#include "model.hpp"

std::vector<float> knnMeanDistance(const float *xyz, int64_t n, int k) {
    std::vector<float> out((size_t)std::max<int64_t>(n, 0), 0.01f);
    if (n < 2) return out;
    k = (int)std::min<int64_t>(k, n - 1);
    float lo[3], hi[3];
    for (int d = 0; d < 3; ++d) lo[d] = hi[d] = xyz[d];
    for (int64_t i = 1; i < n; ++i)
        for (int d = 0; d < 3; ++d) {
            lo[d] = std::min(lo[d], xyz[3 * i + d]);
            hi[d] = std::max(hi[d], xyz[3 * i + d]);
        }
    double ext[3], vol = 1.0;
    for (int d = 0; d < 3; ++d) {
        ext[d] = std::max((double)hi[d] - lo[d], 1e-9);
        vol *= ext[d];
    }
    double cell = std::cbrt(vol * 2.0 / (double)n);
    int dim[3];
    for (int d = 0; d < 3; ++d) {
        cell = std::max(cell, ext[d] / 1024.0);  // at most 1024 cells per axis
    }
    for (int d = 0; d < 3; ++d) dim[d] = std::max(1, (int)std::ceil(ext[d] / cell));
    const int64_t ncell = (int64_t)dim[0] * dim[1] * dim[2];
    auto cell_of = [&](const float *p, int c[3]) {
        for (int d = 0; d < 3; ++d) c[d] = std::min(dim[d] - 1, std::max(0, (int)((p[d] - lo[d]) / cell)));
    };
    // counting sort of point ids by cell
    std::vector<int64_t> start(ncell + 1, 0);
    std::vector<int64_t> cid((size_t)n);
    for (int64_t i = 0; i < n; ++i) {
        int c[3];
        cell_of(xyz + 3 * i, c);
        cid[i] = ((int64_t)c[2] * dim[1] + c[1]) * dim[0] + c[0];
        ++start[cid[i] + 1];
    }
    for (int64_t c = 0; c < ncell; ++c) start[c + 1] += start[c];
    std::vector<int64_t> order((size_t)n), fill(start.begin(), start.end() - 1);
    for (int64_t i = 0; i < n; ++i) order[fill[cid[i]]++] = i;

#pragma omp parallel for schedule(dynamic, 256)
    for (int64_t i = 0; i < n; ++i) {
        const float *p = xyz + 3 * i;
        int c[3];
        cell_of(p, c);
        float best[8];
        for (int j = 0; j < k; ++j) best[j] = std::numeric_limits<float>::infinity();
        for (int r = 0;; ++r) {
            for (int z = c[2] - r; z <= c[2] + r; ++z) {
                if (z < 0 || z >= dim[2]) continue;
                for (int y = c[1] - r; y <= c[1] + r; ++y) {
                    if (y < 0 || y >= dim[1]) continue;
                    for (int x = c[0] - r; x <= c[0] + r; ++x) {
                        if (x < 0 || x >= dim[0]) continue;
                        if (std::max({std::abs(x - c[0]), std::abs(y - c[1]), std::abs(z - c[2])}) != r) continue;
                        const int64_t cc = ((int64_t)z * dim[1] + y) * dim[0] + x;
                        for (int64_t t = start[cc]; t < start[cc + 1]; ++t) {
                            const int64_t j = order[t];
                            if (j == i) continue;
                            const float dx = xyz[3 * j] - p[0], dy = xyz[3 * j + 1] - p[1], dz = xyz[3 * j + 2] - p[2];
                            const float d2 = dx * dx + dy * dy + dz * dz;
                            if (d2 < best[k - 1]) {
                                int m = k - 1;
                                while (m > 0 && best[m - 1] > d2) {
                                    best[m] = best[m - 1];
                                    --m;
                                }
                                best[m] = d2;
                            }
                        }
                    }
                }
            }
            // every point outside shells 0..r is at least r * cell away
            const double reach = (double)r * cell;
            const bool covered = r >= std::max({dim[0], dim[1], dim[2]});
            if (covered || (best[k - 1] < std::numeric_limits<float>::infinity() && reach * reach >= best[k - 1])) break;
        }
        float sum = 0.f;
        for (int j = 0; j < k; ++j) sum += std::sqrt(best[j]);
        // coincident points would give log(0); keep the scale finite
        out[i] = std::max(sum / k, 1e-7f);
    }
    return out;
}
