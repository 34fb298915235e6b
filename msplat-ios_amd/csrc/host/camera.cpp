// camera.cpp -- the camera set-up of Model::prepareCam
// (core/src/model.cpp:500-544), shared by the C++ Model and C-ABI callers.
#include <cmath>
#include <cstring>

#include "msplat_engine.h"

extern "C" int msplat_hip_prepare_camera(const float *d, float fx, float fy, float cx, float cy, int width,
                                         int height, int degree, int degrees_to_use, MsplatCamera *o) {
    if (!d || !o || width <= 0 || height <= 0 || fx <= 0.f || fy <= 0.f) return MSPLAT_E_ARG;
    const float fovX = 2.0f * std::atan(width / (2.0f * fx));
    const float fovY = 2.0f * std::atan(height / (2.0f * fy));
    float R[3][3], Rinv[3][3], T[3], Tinv[3];
    for (int i = 0; i < 3; i++) {
        R[i][0] = d[i * 4 + 0];
        R[i][1] = -d[i * 4 + 1];
        R[i][2] = -d[i * 4 + 2];
        T[i] = d[i * 4 + 3];
    }
    for (int i = 0; i < 3; i++)
        for (int j = 0; j < 3; j++) Rinv[i][j] = R[j][i];
    for (int i = 0; i < 3; i++) Tinv[i] = -(Rinv[i][0] * T[0] + Rinv[i][1] * T[1] + Rinv[i][2] * T[2]);
    const float vm[16] = {Rinv[0][0], Rinv[0][1], Rinv[0][2], Tinv[0], Rinv[1][0], Rinv[1][1], Rinv[1][2], Tinv[1],
                          Rinv[2][0], Rinv[2][1], Rinv[2][2], Tinv[2], 0,          0,          0,          1};
    const float t_p = 0.001f * std::tan(0.5f * fovY), r_p = 0.001f * std::tan(0.5f * fovX);
    const float pm[16] = {0.001f / r_p, 0, 0, 0, 0, 0.001f / t_p, 0, 0,
                          0, 0, (1000.0f + 0.001f) / (1000.0f - 0.001f), -1000.0f * 0.001f / (1000.0f - 0.001f),
                          0, 0, 1, 0};
    float pvm[16] = {};
    for (int i = 0; i < 4; i++)
        for (int j = 0; j < 4; j++)
            for (int k = 0; k < 4; k++) pvm[i * 4 + j] += pm[i * 4 + k] * vm[k * 4 + j];
    std::memcpy(o->viewmat, vm, sizeof(vm));
    std::memcpy(o->projmat, pvm, sizeof(pvm));
    o->cam_pos[0] = T[0];
    o->cam_pos[1] = T[1];
    o->cam_pos[2] = T[2];
    o->fx = fx;
    o->fy = fy;
    o->cx = cx;
    o->cy = cy;
    o->width = width;
    o->height = height;
    o->tiles_x = (width + MSPLAT_TILE - 1) / MSPLAT_TILE;
    o->tiles_y = (height + MSPLAT_TILE - 1) / MSPLAT_TILE;
    o->glob_scale = 1.0f;
    o->clip_thresh = 0.01f;
    o->degree = degree;
    o->degrees_to_use = degrees_to_use;
    return MSPLAT_OK;
}
