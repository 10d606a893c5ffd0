/*
 * msplat_c_api.h — the reference's C API (core/include/msplat_c_api.h) over
 * the MI355X backend (libmsplat_hip.so).
 *
 * Every declaration below has the reference's name, return type and
 * parameter list, so a Swift or C caller built against the reference's
 * header links against this library and behaves the same; the types
 * (MsplatConfig, MsplatStats, MsplatEvalMetrics, MsplatPixelBuffer and the
 * two opaque handles) have the reference's layouts.  Cited per declaration
 * (msplat_c_api.h line numbers of the reference).
 *
 * Backend differences, none visible in the prototypes:
 *  - the device context is created on the first call that needs it (GPU 0),
 *    as the reference creates its Metal context lazily; msplat_cleanup
 *    releases it;
 *  - the dataset's images are decoded by the library's PNG and JPEG
 *    decoders, or by a decoder the application registers with
 *    msplat_set_image_decoder (msplat_trainer.h) for other formats (the
 *    reference decodes through CoreGraphics, which has no counterpart here);
 *  - failures that the reference reports by exception or by an empty result
 *    give the same empty result here (NULL handle, zero-sized buffer,
 *    negative count) and leave a message in msplat_trainer_last_error().
 */
#ifndef MSPLAT_C_API_H
#define MSPLAT_C_API_H

#include <stdbool.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Training configuration (msplat_c_api.h:16-33). */
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

/* The reference's defaults (msplat_c_api.h:35-54). */
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

/* Per-step statistics (msplat_c_api.h:58-62). */
typedef struct {
    int iteration;
    int splatCount;
    float msPerStep;
} MsplatStats;

/* Evaluation over the held-out cameras (msplat_c_api.h:64-70). */
typedef struct {
    float psnr;
    float ssim;
    float l1;
    int numTest;
    int numGaussians;
} MsplatEvalMetrics;

/* An RGB float32 HWC image in malloc'ed host memory, which the caller
 * free()s (msplat_c_api.h:74-78). */
typedef struct {
    float* data;
    int width;
    int height;
} MsplatPixelBuffer;

/* Dataset (msplat_c_api.h:82-88): a COLMAP reconstruction under path, each
 * camera's image decoded, downscaled by downscaleFactor (> 1: area resize,
 * intrinsics scaled) and undistorted, as Camera::loadImage does; with
 * evalMode every testEvery-th camera (0, testEvery, ...) is held out for
 * evaluation.  NULL on failure. */
typedef void* MsplatDataset;

MsplatDataset msplat_dataset_create(const char* path, float downscaleFactor,
                                    bool evalMode, int testEvery);
void msplat_dataset_destroy(MsplatDataset ds);
int msplat_dataset_num_train(MsplatDataset ds);
int msplat_dataset_num_test(MsplatDataset ds);

/* Trainer (msplat_c_api.h:92-113): gaussians initialised from the dataset's
 * point cloud, trained on its training cameras in a shuffled order. */
typedef void* MsplatTrainer;

MsplatTrainer msplat_trainer_create(MsplatDataset ds, MsplatConfig config);
void msplat_trainer_destroy(MsplatTrainer t);

MsplatStats msplat_trainer_step(MsplatTrainer t);
/* Steps until config.iterations. */
void msplat_trainer_train(MsplatTrainer t);
/* PSNR / SSIM / L1 over the test cameras at the final iteration's
 * resolution; all zero without test cameras. */
MsplatEvalMetrics msplat_trainer_evaluate(MsplatTrainer t);
/* Render training (useTest false) or test camera cameraIndex at the current
 * step's resolution; zero-sized for an index out of range. */
MsplatPixelBuffer msplat_trainer_render(MsplatTrainer t, int cameraIndex, bool useTest);
/* Render a camera-to-world pose (row-major 4x4, OpenGL) with the intrinsics
 * of training camera refCameraIndex. */
MsplatPixelBuffer msplat_trainer_render_pose(MsplatTrainer t, const float camToWorld[16],
                                             int refCameraIndex);
/* The same as RGBA8 into outRGBA (width * height * 4 bytes): call with
 * outRGBA NULL for the size; 0 x 0 for an index out of range. */
void msplat_trainer_render_pose_to_buffer(MsplatTrainer t, const float camToWorld[16],
                                          int refCameraIndex, uint8_t* outRGBA,
                                          int* outWidth, int* outHeight);
void msplat_trainer_export_ply(MsplatTrainer t, const char* path);
void msplat_trainer_export_splat(MsplatTrainer t, const char* path);
void msplat_trainer_save_checkpoint(MsplatTrainer t, const char* path);
/* Returns the restored step. */
int msplat_trainer_load_checkpoint(MsplatTrainer t, const char* path);
int msplat_trainer_splat_count(MsplatTrainer t);
int msplat_trainer_iteration(MsplatTrainer t);
/* Pose of training camera cameraIndex (left unchanged when out of range). */
void msplat_dataset_camera_pose(MsplatDataset ds, int cameraIndex, float camToWorld[16]);

/* Lifecycle (msplat_c_api.h:119-121).  There is no metallib here (the kernels
 * are part of the library): the path is accepted and ignored.  msplat_sync
 * waits for all queued GPU work; msplat_cleanup releases the device context
 * and its caches. */
void msplat_set_metallib_path(const char* path);
void msplat_sync(void);
void msplat_cleanup(void);

#ifdef __cplusplus
}
#endif

#endif
