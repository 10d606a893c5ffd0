/*
 * msplat_hip.h — C ABI of the MI355X (gfx950) splatting hot path.
 *
 * This is the drop-in for msplat's backend boundary
 * /root/reference/core/metal/bindings.h: every entry point below replaces one
 * declaration there (cited per function).  Plain pointers and sizes only;
 * per-gaussian arrays are device pointers in the reference's row-major AoS
 * layouts:
 *   means[N,3]  scales[N,3] (log)  quats[N,4] (w,x,y,z)
 *   features_dc[N,3]  features_rest[N,K-1,3]  opacities[N] (logits)
 *   images [H,W,3] fp32.
 * Camera matrices and the background colour are passed by value (host).
 *
 * Errors: every function returns MSPLAT_OK (0) or a negative code;
 * msplat_hip_last_error() returns a message for the last failure.
 * Threading: one context per process, not reentrant (as bindings.h).  All GPU
 * work is issued in order on one HIP stream (the context's own stream, or the
 * caller's via msplat_hip_set_stream).
 */
#ifndef MSPLAT_HIP_H
#define MSPLAT_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define MSPLAT_OK 0
#define MSPLAT_ERR_ARG (-1)
#define MSPLAT_ERR_HIP (-2)
#define MSPLAT_ERR_NOINIT (-3)
#define MSPLAT_ERR_NOMEM (-4)

/* Everything msplat_render takes (bindings.h:37-46). */
typedef struct MsplatRenderArgs {
    int32_t num_points;
    const float* means3d;
    const float* scales;
    float glob_scale;
    const float* quats;
    float viewmat[16];
    float projmat[16];
    float fx, fy, cx, cy;
    uint32_t img_height, img_width;
    int32_t tile_bounds[3];
    float clip_thresh;
    uint32_t degree;
    uint32_t degrees_to_use;
    float cam_pos[3];
    const float* features_dc;
    const float* features_rest;
    const float* opacities;
    float background[3];
} MsplatRenderArgs;

/* Everything msplat_train_step takes (bindings.h:50-67).  The six Adam
 * groups are means, scales, quats, features_dc, features_rest, opacities;
 * adam_params[g] must alias the matching render pointer.  The three
 * v_*_out pointers are optional device outputs of the projection backward
 * (NULL: not written). */
typedef struct MsplatTrainArgs {
    MsplatRenderArgs r;
    const float* gt;
    float ssim_weight;
    float loss_inv_n;
    int32_t features_rest_bases;
    int32_t num_adam_groups;
    float* adam_params[6];
    float* adam_exp_avg[6];
    float* adam_exp_avg_sq[6];
    float adam_step_sizes[6];
    float adam_bc2_sqrts[6];
    float adam_beta1, adam_beta2, adam_eps;
    float* vis_counts;
    float* xys_grad_norm;
    float* max_2d_size;
    float inv_max_dim;
    float* v_mean3d_out;
    float* v_scale_out;
    float* v_quat_out;
} MsplatTrainArgs;

/* Everything msplat_densify takes (bindings.h:69-84) except the nine scratch
 * tensors, which the library owns.  random_samples: device [2N,3] standard
 * normals, or NULL to draw them on the GPU from seed. */
typedef struct MsplatDensifyArgs {
    int32_t N;
    int32_t buf_capacity;
    float grad_thresh, size_thresh, screen_thresh;
    int32_t check_screen;
    float cull_alpha_thresh, cull_scale_thresh, cull_screen_size;
    int32_t check_huge;
    const float* xys_grad_norm;
    const float* vis_counts;
    const float* max_2d_size;
    float half_max_dim;
    float* bufs[6];            /* means, scales, quats, f_dc, f_rest, opacities */
    int32_t fr_stride;
    float* adam_exp_avg_buf[6];
    float* adam_exp_avg_sq_buf[6];
    const float* random_samples;
    uint64_t seed;
} MsplatDensifyArgs;

/* Context (replaces the lazily created MetalContext, msplat_metal.mm:173-288,
 * and cleanup_msplat_metal, bindings.h:8). */
int msplat_hip_init(int device);
int msplat_hip_shutdown(void);
const char* msplat_hip_last_error(void);
int msplat_hip_set_stream(void* hip_stream);   /* NULL: back to the context's own stream */
void* msplat_hip_get_stream(void);

/* Memory (gpu_empty / gpu_zeros, bindings.h:18-19).  Copies are ordered on
 * the context stream; d2h returns after the data has arrived. */
int msplat_hip_alloc(void** ptr, size_t bytes);
int msplat_hip_free(void* ptr);
int msplat_hip_memset(void* ptr, int value, size_t bytes);
int msplat_hip_memcpy_h2d(void* dst, const void* src, size_t bytes);
int msplat_hip_memcpy_d2h(void* dst, const void* src, size_t bytes);
int msplat_hip_memcpy_d2d(void* dst, const void* src, size_t bytes);
/* Coherent host memory mapped into the device's address space at the same
 * address: the host writes and reads it through the pointer with no copy or
 * stream wait, kernels read it directly (the reference's MTensor storage is
 * such shared memory, metal_tensor.hpp:48-50, MTLResourceStorageModeShared).
 * The host layer backs tensors of at most 256 bytes (camera matrices,
 * background colour) with it.  Accesses race with kernels still running
 * that use it, as on the reference's shared buffers. */
int msplat_hip_alloc_mapped(void** ptr, size_t bytes);
int msplat_hip_free_mapped(void* ptr);

/* msplat_commit (bindings.h:22): flush; a no-op on HIP (work is issued eagerly).
 * msplat_gpu_sync (bindings.h:25): wait for all work on the stream. */
int msplat_hip_commit(void);
int msplat_hip_sync(void);

/* msplat_render (bindings.h:37-46).  The rasteriser writes the image
 * [H,W,3] straight to out_img (device; the context's own image buffer is
 * then left as it was); NULL writes it to the context's own buffer, readable
 * with msplat_hip_copy_intermediate("out_img"). */
int msplat_hip_render(const MsplatRenderArgs* a, float* out_img);

/* msplat_train_step (bindings.h:50-67).  radii_out: optional device [N];
 * loss_out: optional host float — when given the call waits for the step
 * and returns sum(pixel loss)/(H*W) (the reference reads it unsynchronised,
 * msplat_metal.mm:1328). */
int msplat_hip_train_step(const MsplatTrainArgs* a, int32_t* radii_out, float* loss_out);

/* Loss value (sum of per-pixel losses / (H W)) of the most recent train step
 * called with loss_out == NULL.  wait == 0 returns the value of the latest
 * step known to have finished without waiting (NaN if none) — the reference
 * likewise reads its loss buffer without waiting (msplat_metal.mm:1328);
 * wait != 0 first waits for the latest step. */
int msplat_hip_last_loss(float* loss, int wait);

/* msplat_densify (bindings.h:69-84).  Waits for the result and returns the
 * new gaussian count in *new_count. */
int msplat_hip_densify(const MsplatDensifyArgs* a, int32_t* new_count);

/* Fill dst[n] with standard normals from a counter-based generator
 * (the reference fills random_samples with mt19937 on the host,
 * model.cpp:248-253). */
int msplat_hip_randn(float* dst, int64_t n, uint64_t seed);

/* p[i] = min(p[i], hi) for i < n on the context stream: the opacity reset of
 * afterTrain (model.cpp:280-287 clamps the logits on the host). */
int msplat_hip_clamp_max(float* p, int64_t n, float hi);

/* RGBA8 display image of an fp32 RGB render: for each of n_pixels pixels
 * (device img[n,3] -> device rgba[n,4], 4-byte aligned) each channel is
 * clamped to [0, 1], multiplied by 255 and truncated to a byte; alpha is 255.
 * The conversion of Trainer::renderFromPoseToBuffer (msplat_api.mm:230-238,
 * done there on the CPU), on the context stream. */
int msplat_hip_image_to_rgba8(const float* img, int64_t n_pixels, uint8_t* rgba);

/* Area resize of a device [src_h, src_w, 3] fp32 image into device
 * [dst_h, dst_w, 3]: each output pixel is the overlap-weighted mean of the
 * source pixels its footprint covers (resizeArea, image_io.cpp:91-138; used
 * by Camera::getImage and Camera::loadImage, input_data.cpp:17-65), equal bit
 * for bit to the reference's CPU loop.  On the context stream. */
int msplat_hip_resize_area(const float* src, int32_t src_w, int32_t src_h, float* dst,
                           int32_t dst_w, int32_t dst_h);

/* Undistortion of a Brown-Conrady camera image (undistortImage,
 * image_io.cpp:203-330).  intrinsics = {fx, fy, cx, cy}, distortion =
 * {k1, k2, p1, p2, k3}.  msplat_undistort_roi (host only, no device needed)
 * gives the crop rectangle roi = {x, y, w, h} of the undistorted image that
 * has no empty border; the reference's camera then has cx - x, cy - y and
 * size w x h.  msplat_hip_undistort writes that rectangle of the undistorted
 * device [height, width, 3] image into device dst [roi h, roi w, 3] (forward
 * distortion of each output pixel, bilinear sampling with edge clamping), on
 * the context stream. */
int msplat_undistort_roi(int32_t width, int32_t height, const float intrinsics[4],
                         const float distortion[5], int32_t roi[4]);
int msplat_hip_undistort(const float* src, int32_t width, int32_t height, const float intrinsics[4],
                         const float distortion[5], const int32_t roi[4], float* dst);

/* Evaluation metrics of a render against its target (device [H,W,3] fp32
 * images): PSNR = 10 log10(1 / MSE) and mean |r - g| as psnr / l1_loss
 * (model.cpp:25-40) compute them, and SSIM averaged over pixels and channels
 * as ssim_eval (ssim.cpp:61-123) does, with a window_size-tap Gaussian
 * (odd, <= 11; the reference's default 11) of width sigma (default 1.5) and
 * borders clamped to the edge pixel.  Sums are fp64, as there.  Waits for the
 * result. */
typedef struct MsplatImageMetrics {
    float psnr, ssim, l1;
} MsplatImageMetrics;
int msplat_hip_image_metrics(const float* img, const float* gt, int32_t height, int32_t width,
                             int32_t window_size, float sigma, MsplatImageMetrics* out);

/* msplat_hip_image_metrics without any allocation.  No counterpart in the
 * reference: it is for callers that cannot allocate device memory (code under
 * HIP graph capture, tight serving or evaluation loops, harnesses that forbid
 * hipMalloc).  Same arguments, kernels and results as
 * msplat_hip_image_metrics; the per-workgroup partial sums live in a
 * fixed 1.5 MiB device workspace inside the library (one per GPU, held until
 * the process ends) instead of the context's grow-only buffers.  Images are
 * limited to 65536 metric tiles of 64x16 pixels (e.g. 8192x8192); larger ones
 * return MSPLAT_ERR_ARG.  All calls on one GPU share that workspace: calls
 * that overlap on one GPU (from several threads or streams) race. */
int msplat_hip_image_metrics_noalloc(const float* img, const float* gt, int32_t height,
                                     int32_t width, int32_t window_size, float sigma,
                                     MsplatImageMetrics* out);

/* Initial gaussian scale of every point of a cloud: the mean distance to its
 * three nearest other points (device xyz[n,3] -> device mean_dist[n]),
 * exactly as the reference's nanoflann kd-tree query gives it
 * (PointsTensor::scales, kdtree_tensor.hpp:26-40; Model::Model takes its log,
 * model.cpp:63-73).  n >= 4.  Reads the points back once for their bounding
 * box; the result is ready when the stream is. */
int msplat_hip_knn_mean_dist(const float* xyz, int64_t n, float* mean_dist);

/* Per-stage GPU timing (msplat_enable_gpu_timing / msplat_drain_stage_times,
 * bindings.h:28-33).  When enabled every stage of every render / train /
 * densify call is bracketed by HIP events on the context stream (no extra
 * synchronisation).  drain waits for the stream, then returns for each stage
 * i the summed milliseconds ms[i] and the number of timed instances
 * counts[i] since the last drain (or enable), its name, and the number of
 * calls timed.  Stage names are the reference profiler's
 * (msplat_metal.mm:30-34), with ".part" where a stage runs as two kernels:
 * proj_sh_fwd, prefix_sort_pack.depth_sort, prefix_sort_pack.tile_lists,
 * rast_fwd, loss_fwd_bwd, rast_bwd, proj_sh_bwd_adam.sh_rest,
 * proj_sh_bwd_adam.dense, and densify (one msplat_hip_densify call).  The
 * reference's blit_zero is part of proj_sh_fwd here and its grad_stats part
 * of proj_sh_bwd_adam.dense. */
int msplat_hip_enable_stage_timing(int enable);
/* Bracket only the stages whose bit (1 << stage index, in the order drain
 * names them) is set; the default is every stage.  Each event leaves the GPU
 * idle for a few microseconds between the kernels it separates, so a
 * throughput run times just the stages it reports.  No counterpart in the
 * reference (its timing is per command-buffer encoder). */
int msplat_hip_set_stage_timing_mask(uint32_t mask);
int msplat_hip_drain_stage_times(double* ms, int64_t* counts, const char** names, int max_stages,
                                 int* n_stages, int64_t* n_calls);

/* The bracketed GPU milliseconds of each timed call since the last drain (or
 * enable), in call order: the sum of its stages' intervals, all stages with
 * the default mask (msplat_drain_gpu_times, bindings.h:29-30, which the
 * reference fills per command buffer).  Waits for the stream; fills up to
 * max_calls values (the context keeps the latest 65536) and clears them. */
int msplat_hip_drain_call_times(double* ms, int max_calls, int* n_calls);

/* While stage timing is enabled the rasteriser also counts, on the GPU,
 * counts[0] (pixel, entry) pairs composited by the forward, counts[1] pairs
 * that carry a gradient in the backward, and counts[2] / counts[3] the
 * entries evaluated per 64-pixel wave in the forward / backward (each one
 * wave-wide step), summed over the timed calls.  The forward counts only
 * while its stage (rast_fwd) is in the stage mask and the backward only
 * while rast_bwd is (other calls run kernels without the counting).  drain
 * returns them (zeros when timing is off) and restarts the sums.  Part of
 * the profiler interface above; the reference has no counterpart. */
int msplat_hip_drain_raster_counters(int64_t counts[4]);

/* Copy a named intermediate of the last render / train step to host memory.
 * Names: xys, depths, radii, conics, colors, aabb, num_tiles_hit,
 * tile_bins, gaussian_ids, final_Ts, final_index, out_img, v_rendered,
 * v_xy, v_conic, v_rgb, v_opacity, meta, tile_done (after a train step, for
 * each tile of more than 16 depth chunks: 1 if every pixel's running
 * transmittance was exactly 0 after its first 16 chunks, so that its later
 * chunks were not rasterised).  *nbytes is set to the size; pass dst == NULL
 * to query it. */
int msplat_hip_copy_intermediate(const char* name, void* dst, size_t* nbytes);

/* Algorithmic rasteriser work of the last render / train step, counted on the
 * GPU per (pixel, entry) pair in the order of the reference's per-pixel loops
 * (no culling): counts[0..2] forward pairs tested / with sigma in [0, 5.55) /
 * composited; counts[3..5] backward pairs tested / in range / carrying a
 * gradient (meaningful after a train step).  Measurement aid with no
 * counterpart in the reference; it changes no state. */
int msplat_hip_raster_work(int64_t counts[6]);

#ifdef __cplusplus
}
#endif
#endif
