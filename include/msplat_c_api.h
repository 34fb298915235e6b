/* msplat_c_api.h -- the trainer's C ABI: opaque Dataset / Trainer handles
 * and free functions, declared exactly as the reference's
 * core/include/msplat_c_api.h:16-127 (same names, struct layouts, defaults
 * and ownership rules), implemented over the HIP engine in
 * msplat-ios_amd/csrc/host/msplat_api.cpp and exported by
 * libmsplat_hip.so.
 *
 * Differences a caller can observe:
 *  - no exception crosses this boundary: a failing create returns NULL,
 *    other calls return zeroed results / -1 and record the message for
 *    msplat_last_error();
 *  - msplat_set_metallib_path is accepted and ignored (the GPU code is
 *    linked into the library);
 *  - msplat_trainer_extract_mesh returns the triangle count, or -1 with
 *    msplat_last_error() set.
 * Threading: one trainer per process, as the reference (one engine
 * context and buffer cache). */
#ifndef MSPLAT_C_API_H
#define MSPLAT_C_API_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* msplat_c_api.h:16-33 */
typedef struct {
    int iterations;
    int shDegree;
    int shDegreeInterval;
    float ssimWeight;
    int numDownscales;
    int resolutionSchedule;
    int refineEvery;
    int warmupLength;
    int resetAlphaEvery;
    float densifyGradThresh;
    float densifySizeThresh;
    int stopScreenSizeAt;
    float splitScreenSize;
    bool keepCrs;
    float downscaleFactor;
    float bgColor[3];
} MsplatConfig;

/* msplat_c_api.h:35-54 */
static inline MsplatConfig msplat_default_config(void) {
    MsplatConfig c;
    c.iterations = 30000;
    c.shDegree = 3;
    c.shDegreeInterval = 1000;
    c.ssimWeight = 0.2f;
    c.numDownscales = 2;
    c.resolutionSchedule = 3000;
    c.refineEvery = 100;
    c.warmupLength = 500;
    c.resetAlphaEvery = 30;
    c.densifyGradThresh = 0.0002f;
    c.densifySizeThresh = 0.01f;
    c.stopScreenSizeAt = 4000;
    c.splitScreenSize = 0.05f;
    c.keepCrs = false;
    c.downscaleFactor = 1.0f;
    c.bgColor[0] = 0.6130f;
    c.bgColor[1] = 0.0101f;
    c.bgColor[2] = 0.3984f;
    return c;
}

/* msplat_c_api.h:58-72 */
typedef struct {
    int iteration;
    int splatCount;
    float msPerStep;
    float loss;
} MsplatStats;

typedef struct {
    float psnr;
    float ssim;
    float l1;
    int numTest;
    int numGaussians;
} MsplatEvalMetrics;

/* msplat_c_api.h:75-79: RGB float32 HWC; the caller must free() data. */
typedef struct {
    float *data;
    int width;
    int height;
} MsplatPixelBuffer;

typedef void *MsplatDataset;
typedef void *MsplatTrainer;

/* msplat_c_api.h:83-88 */
MsplatDataset msplat_dataset_create(const char *path, float downscaleFactor, bool evalMode, int testEvery);
void msplat_dataset_destroy(MsplatDataset ds);
int msplat_dataset_num_train(MsplatDataset ds);
int msplat_dataset_num_test(MsplatDataset ds);

/* msplat_c_api.h:92-122 */
MsplatTrainer msplat_trainer_create(MsplatDataset ds, MsplatConfig config);
void msplat_trainer_destroy(MsplatTrainer t);
MsplatStats msplat_trainer_step(MsplatTrainer t);
void msplat_trainer_train(MsplatTrainer t);
MsplatEvalMetrics msplat_trainer_evaluate(MsplatTrainer t);
MsplatPixelBuffer msplat_trainer_render(MsplatTrainer t, int cameraIndex, bool useTest);
MsplatPixelBuffer msplat_trainer_render_pose(MsplatTrainer t, const float camToWorld[16], int refCameraIndex);
void msplat_trainer_render_pose_to_buffer(MsplatTrainer t, const float camToWorld[16], int refCameraIndex,
                                          uint8_t *outRGBA, int *outWidth, int *outHeight);
void msplat_trainer_export_ply(MsplatTrainer t, const char *path);
void msplat_trainer_export_splat(MsplatTrainer t, const char *path);
int64_t msplat_trainer_extract_mesh(MsplatTrainer t, const char *path, float voxelSize, float boundRadius,
                                    float alphaThresh, float truncMultiplier);
void msplat_trainer_save_checkpoint(MsplatTrainer t, const char *path);
int msplat_trainer_load_checkpoint(MsplatTrainer t, const char *path);
int msplat_trainer_splat_count(MsplatTrainer t);
int msplat_trainer_iteration(MsplatTrainer t);
void msplat_dataset_camera_pose(MsplatDataset ds, int cameraIndex, float camToWorld[16]);

/* msplat_c_api.h:124-127 */
void msplat_set_metallib_path(const char *path);
void msplat_sync(void);
void msplat_cleanup(void);

/* ---- extensions (no counterpart in the reference) ----------------------- */

/* A camera and its image for in-memory datasets: callers that decode or
 * synthesise images themselves (rgb: [height, width, 3] float32 in [0,1],
 * copied). */
typedef struct {
    int width, height;
    float fx, fy, cx, cy;
    float camToWorld[16];
    const float *rgb;
} MsplatCameraImage;

/* Dataset from memory: cameras + images and an initial point cloud (xyz
 * float32 [n,3], rgb uint8 [n,3]; numPoints = 0 seeds random points). */
MsplatDataset msplat_dataset_create_from_memory(const MsplatCameraImage *cameras, int numCameras,
                                                const float *xyz, const uint8_t *rgb, int64_t numPoints,
                                                bool evalMode, int testEvery);
/* Message of the most recent failure in this thread ("" if none). */
const char *msplat_last_error(void);
/* Densification cap (250000 by default, as the reference) and cull
 * threshold on sigmoid(opacity) (0.1 by default). */
void msplat_trainer_set_max_splats(MsplatTrainer t, int maxSplats);
void msplat_trainer_set_cull_alpha(MsplatTrainer t, float thresh);
/* Scene from a Gaussian PLY, resuming at the step the file records: the
 * reference CLI's --resume (Model::loadPly, core/src/model.cpp:329-340,
 * cli/msplat.cpp:259).  Returns that step, or -1 (msplat_last_error). */
int msplat_trainer_load_ply(MsplatTrainer t, const char *path);
/* A trainer of 3D Gaussians (the 3DGS mode: three scales per splat, EWA
 * projection, the 3DGS compositing rule), with the arguments of
 * msplat_trainer_create.  Every other call applies to it unchanged, except
 * msplat_trainer_extract_mesh, which needs depth and returns -1.  PLY and
 * .splat exports carry three scales. */
MsplatTrainer msplat_trainer_create_3dgs(MsplatDataset ds, MsplatConfig config);

#ifdef __cplusplus
}
#endif

#endif /* MSPLAT_C_API_H */
