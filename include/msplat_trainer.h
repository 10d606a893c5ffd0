/*
 * msplat_trainer.h — the host-side trainer's C API beyond the reference's
 * (libmsplat_hip.so).
 *
 * include/msplat_c_api.h holds the reference's C API with its exact
 * prototypes (core/include/msplat_c_api.h: MsplatConfig, MsplatStats,
 * MsplatEvalMetrics, MsplatPixelBuffer, the dataset and trainer calls); this
 * header adds what the MI355X build offers next to it: a trainer built from
 * gaussian arrays, cameras and target images already in memory (host or
 * device), evaluation on caller-supplied images, render into a device buffer,
 * the lower-level COLMAP reader, PLY resume and scene-file writers, the
 * camera set-up, an image-decoder hook and error messages.
 */
#ifndef MSPLAT_TRAINER_H
#define MSPLAT_TRAINER_H

#include <stdint.h>

#include "msplat_c_api.h"

#ifdef __cplusplus
extern "C" {
#endif

/* MsplatConfig (msplat_c_api.h:16-33) without the dataset-only fields
 * (keepCrs, downscaleFactor), plus the cull thresholds model.cpp:263
 * hard-codes, the camera order and its seed. */
typedef struct MsplatTrainerConfig {
    int32_t iterations;
    int32_t shDegree;
    int32_t shDegreeInterval;   /* <= 0: all bands from the first step */
    float ssimWeight;
    int32_t numDownscales;
    int32_t resolutionSchedule;
    int32_t refineEvery;
    int32_t warmupLength;
    int32_t resetAlphaEvery;
    float densifyGradThresh;
    float densifySizeThresh;
    int32_t stopScreenSizeAt;
    float splitScreenSize;
    float bgColor[3];
    float cullAlphaThresh;      /* model.cpp:263: 0.1 */
    float cullScaleThresh;      /* 0.5 */
    float cullScreenSize;       /* 0.15 */
    int32_t shuffleCameras;     /* 1: std::shuffle with mt19937(seed) per epoch (bindings.cpp:127-137) */
    uint32_t seed;              /* 42 in the reference */
} MsplatTrainerConfig;

static inline MsplatTrainerConfig msplat_trainer_default_config(void) {
    MsplatTrainerConfig c;
    c.iterations = 30000; c.shDegree = 3; c.shDegreeInterval = 1000; c.ssimWeight = 0.2f;
    c.numDownscales = 2; c.resolutionSchedule = 3000; c.refineEvery = 100; c.warmupLength = 500;
    c.resetAlphaEvery = 30; c.densifyGradThresh = 0.0002f; c.densifySizeThresh = 0.01f;
    c.stopScreenSizeAt = 4000; c.splitScreenSize = 0.05f;
    c.bgColor[0] = 0.6130f; c.bgColor[1] = 0.0101f; c.bgColor[2] = 0.3984f;
    c.cullAlphaThresh = 0.1f; c.cullScaleThresh = 0.5f; c.cullScreenSize = 0.15f;
    c.shuffleCameras = 1; c.seed = 42;
    return c;
}

/* A pinhole training camera (input_data.hpp:20-38); camToWorld is a
 * row-major 4x4 OpenGL pose. */
typedef struct MsplatTrainerCamera {
    int32_t width, height;
    float fx, fy, cx, cy;
    float camToWorld[16];
} MsplatTrainerCamera;

/* Model::CamSetup plus the matrices prepareCam caches (model.hpp:33-38,
 * model.cpp:490-534): viewmat = [R^T | -R^T T] of the OpenCV-flipped pose,
 * projmat = P V (near 0.001, far 1000), both row-major. */
typedef struct MsplatCamSetup {
    float fx, fy, cx, cy;
    int32_t width, height;
    float viewmat[16];
    float projmat[16];
    float cam_pos[3];
    int32_t tile_bounds[3];
} MsplatCamSetup;

/* prepareCam for one camera at an integer downscale factor (host only, no
 * device work).  Returns 0 or a negative code. */
int32_t msplat_prepare_cam(const MsplatTrainerCamera* cam, int32_t downscale, MsplatCamSetup* out);

/* Builds a trainer from arrays (the reference builds one from a dataset,
 * msplat_trainer_create in msplat_c_api.h).  params[6] = means[N,3], scales[N,3] (log), quats[N,4]
 * (w,x,y,z), f_dc[N,3], f_rest[N,(shDegree+1)^2-1,3], opacities[N] (logits);
 * targets[i] is the full-resolution [H,W,3] image of cameras[i] (images for
 * downscaled steps are box-filtered from it once, on the host).
 * on_device: 1 if params and targets are device pointers.  Returns NULL on
 * error (message in msplat_trainer_last_error). */
MsplatTrainer msplat_trainer_create_from_arrays(const MsplatTrainerConfig* config, int64_t n,
                                                const float* const params[6], int32_t n_cameras,
                                                const MsplatTrainerCamera* cameras,
                                                const float* const* targets, int32_t on_device);
/* Message of the latest failed call of this API or of msplat_c_api.h ("" if
 * the latest call succeeded). */
const char* msplat_trainer_last_error(void);

/* Loss of the most recent step known to have completed (wait = 0) or of
 * the latest step (wait = 1). */
float msplat_trainer_last_loss(MsplatTrainer t, int32_t wait);

/* msplat_trainer_render_pose rendered straight into a caller-provided
 * device buffer of H*W*3 floats (no copy, no synchronisation; outDevice
 * NULL: size only): the display-loop form of renderFromPoseToBuffer. */
int32_t msplat_trainer_render_pose_device(MsplatTrainer t, const float camToWorld[16],
                                          int32_t refCameraIndex, float* outDevice,
                                          int32_t* outWidth, int32_t* outHeight);

/* Evaluation on caller-supplied cameras and full-resolution images (images
 * on the device when on_device != 0), as msplat_trainer_evaluate does for a
 * dataset's test cameras (Trainer::evaluate, msplat_api.mm:138-166): each
 * camera is rendered at the final iteration's resolution, its image is
 * box-filtered to that size, and PSNR / SSIM (11 taps, sigma 1.5) / L1 are
 * averaged over the cameras (msplat_hip_image_metrics).  numTest = 0 on
 * error. */
MsplatEvalMetrics msplat_trainer_evaluate_images(MsplatTrainer t, int32_t n_test,
                                                 const MsplatTrainerCamera* cameras,
                                                 const float* const* images, int32_t on_device);

/* Resume from an exported PLY (the CLI's --resume, cli/msplat.cpp:132;
 * Model::loadPly, model.cpp:319-330): replaces the gaussians, restarts the
 * optimiser and returns the step recorded in the file (0 if none) or a
 * negative code.  The iteration counter is left to the caller, as there. */
int32_t msplat_trainer_load_ply(MsplatTrainer t, const char* path);

/* Dataset normalisation the scene files undo (export) or apply (load) when
 * keep != 0: world = stored / scale + translation (keepCrs,
 * loaders.hpp:38-43).  Identity by default. */
int32_t msplat_trainer_set_crs(MsplatTrainer t, float scale, const float translation[3],
                               int32_t keep);

/* Host-memory scene files (no GPU call): the writers and the reader behind
 * the trainer's exports, for parameter arrays already in host memory
 * (params[6] as for msplat_trainer_create_from_arrays; opacities [n]).  read: call with
 * params == NULL for *n and *rest_bases, then with six buffers of those
 * sizes.  0 or a negative code (message in msplat_trainer_last_error). */
int32_t msplat_scene_write_ply(const char* path, int64_t n, int32_t rest_bases,
                               const float* const params[6], float crs_scale,
                               const float crs_translation[3], int32_t keep_crs, int32_t step);
int32_t msplat_scene_write_splat(const char* path, int64_t n, int32_t rest_bases,
                                 const float* const params[6], float crs_scale,
                                 const float crs_translation[3], int32_t keep_crs);
int32_t msplat_scene_read_ply(const char* path, float crs_scale, const float crs_translation[3],
                              int32_t keep_crs, int64_t* n, int32_t* rest_bases, int32_t* step,
                              float* const params[6]);

/* A COLMAP reconstruction without its images (the reader under
 * msplat_dataset_create; loadColmap, load_colmap.cpp:121-164):
 * cameras.bin / images.bin / points3D.bin (or points3D.ply) under path or
 * path/sparse/0, cameras sorted by image name, OpenGL camera-to-world poses,
 * then autoScaleAndCenter (input_data.cpp:79-125).  image_dir NULL:
 * path/images if present, else path.  Each camera carries its image path; the
 * caller decodes and supplies pixels to msplat_trainer_create_from_arrays.
 * Every camera counts as a training camera.  Released with
 * msplat_dataset_destroy.  NULL on error. */
MsplatDataset msplat_dataset_open_colmap(const char* path, const char* image_dir);
int32_t msplat_dataset_num_cameras(MsplatDataset ds);
/* Camera i: intrinsics and pose (cam), distortion k1 k2 p1 p2 (nullable),
 * image path (nullable; valid while ds lives). */
int32_t msplat_dataset_camera(MsplatDataset ds, int32_t i, MsplatTrainerCamera* cam,
                              float distortion[4], const char** image_path);
int64_t msplat_dataset_num_points(MsplatDataset ds);
/* Normalised points [n,3] and colours [n,3] (either nullable). */
int32_t msplat_dataset_points(MsplatDataset ds, float* xyz, uint8_t* rgb);
/* world = normalised / scale + translation. */
int32_t msplat_dataset_normalisation(MsplatDataset ds, float* scale, float translation[3]);
/* Initial gaussians of the point cloud into six host buffers sized for
 * num_points (Model::Model, model.cpp:59-110): the nearest-neighbour scales
 * run on the GPU (msplat_hip_knn_mean_dist). */
int32_t msplat_dataset_init_gaussians(MsplatDataset ds, int32_t sh_degree, float* const params[6]);

/* Device pointer and row count of parameter group g (0..5) or of its Adam
 * moments (which = 0 params, 1 exp_avg, 2 exp_avg_sq); the first
 * splat_count rows are active.  Valid until the next step. */
int32_t msplat_trainer_group(MsplatTrainer t, int32_t g, int32_t which, float** devPtr,
                             int64_t* rows, int64_t* rowFloats);

/* Image decoding for msplat_dataset_create: a function that decodes the
 * file at path into a malloc'ed float32 RGB HWC buffer in [0, 1] (*rgb, which
 * the library free()s) of *width x *height pixels and returns 0, or returns
 * nonzero if it cannot.  PNG and JPEG files are decoded by the library
 * itself; other formats need a registered decoder, which, when set, decodes
 * every file.  NULL removes it. */
typedef int (*MsplatImageDecoder)(const char* path, float** rgb, int* width, int* height);
void msplat_set_image_decoder(MsplatImageDecoder decoder);

/* An image file decoded as msplat_dataset_create decodes it (the registered
 * decoder, else the built-in decoders, each channel byte / 255 as imreadRGB,
 * image_io.cpp:12-50: PNG of colour types grey, RGB, palette, grey + alpha
 * and RGBA at 1-16 bits, not interlaced, 16-bit samples by their high byte,
 * transparency (alpha or tRNS) drawn over black; JPEG baseline, extended
 * sequential or progressive with Huffman coding, grey or three components,
 * any sampling factors, the samples libjpeg's default decoding gives): a
 * malloc'ed float32 RGB HWC buffer in *rgb that the caller free()s.  Host
 * only.  0 or a negative code (message in msplat_trainer_last_error). */
int32_t msplat_image_read(const char* path, float** rgb, int32_t* width, int32_t* height);

#ifdef __cplusplus
}
#endif
#endif
