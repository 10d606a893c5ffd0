/*
 * oracle.h — CPU restatement of msplat's per-step splatting hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the parity checker for the HIP
 * path in msplat_amd/.  Only tests/, __graft_entry__.smoke() and bench.py's
 * cpu_baseline leg may load it, and only as the checker / CPU baseline; the
 * product never links, loads or calls it.
 *
 * Every function restates the algorithm of /root/reference/core/metal/
 * msplat_metal.metal (kernels) and msplat_metal.mm (stage order), citing the
 * lines it follows.  Arithmetic is IEEE fp32 with no contraction
 * (-ffp-contract=off); an fma is used exactly where the reference writes one.
 * exp() is the Cody–Waite / Taylor exp defined in oracle.cpp (the reference's
 * Metal exp is closed); it is pinned against libm by the CPU tests.
 *
 * Array layouts are the reference's row-major AoS layouts:
 *   means[N,3] scales[N,3] (log) quats[N,4] (w,x,y,z) f_dc[N,3]
 *   f_rest[N,K-1,3] opacities[N] (logits); images [H,W,3].
 */
#ifndef MSPLAT_ORACLE_H
#define MSPLAT_ORACLE_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* One camera + render configuration (everything msplat_render takes that is
 * not a per-gaussian array; bindings.h:37-46). */
typedef struct OrcCamera {
    float viewmat[16];     /* row-major world->camera */
    float projmat[16];     /* row-major P*V (model.cpp:511-513) */
    float fx, fy, cx, cy;
    int32_t width, height;
    float cam_pos[3];
    float clip_thresh;     /* 0.01 (model.cpp:541) */
    float glob_scale;      /* 1.0 */
    int32_t degree;        /* SH degree of the stored coefficients */
    int32_t degrees_to_use;
    float background[3];
} OrcCamera;

/* Adam hyper-parameters for one step (model.cpp:558-571, model.hpp:55). */
typedef struct OrcAdam {
    float step_size[6];    /* lr_g / (1 - beta1^t) */
    float bc2_sqrt[6];     /* sqrt(1 - beta2^t) */
    float beta1, beta2, eps;
} OrcAdam;

uint32_t orc_version(void);
int32_t orc_num_threads(void);
/* Summed wall milliseconds per train stage of the orc_train_step calls since
 * the last call (blit_zero, proj_sh_fwd, prefix_sort_pack, rast_fwd,
 * loss_fwd_bwd, rast_bwd, proj_sh_bwd_adam, grad_stats; the names of the
 * reference profiler, msplat_metal.mm:30-34) and the number of steps; resets
 * the sums. */
void orc_stage_times(double ms[8], int64_t* steps);

/* ---- scalar building blocks (exported for the closed-form tests) ---- */
float orc_expf(float x);
void orc_expf_n(int64_t n, const float* x, float* y);
float orc_expf_raster(float x);            /* exp of the rasteriser's -sigma */
void orc_expf_raster_n(int64_t n, const float* x, float* y);
void orc_sh_consts(float out[25]);         /* C0, C1, C2[5], C3[7], C4[9], pad */
void orc_gauss1d(float out[11]);
void orc_quat_to_rotmat(const float q[4], float R_rowmajor[9]);
void orc_cov3d(const float scale[3], float glob_scale, const float q[4], float cov[6]);
void orc_sh_eval(int degree, const float dir[3], const float* dc, const float* rest,
                 float color[3]);

/* ---- a1: project_and_sh_forward (.metal:1695-1787) ---- */
void orc_project_forward(const OrcCamera* cam, int32_t N,
                         const float* means, const float* scales, const float* quats,
                         const float* f_dc, const float* f_rest,
                         float* xys, float* depths, int32_t* radii, float* conics,
                         int32_t* num_tiles_hit, float* colors, float* aabb);

/* Tile rectangle of one gaussian (get_tile_bbox, .metal:72-87). */
void orc_tile_rect(const OrcCamera* cam, const float xy[2], const float aabb[2],
                   int32_t rect[4] /* xmin, ymin, xmax, ymax (exclusive) */);

/* ---- a2/a3/a4: per-tile counts, offsets, depth sort (.metal:2025-2138, 2312-2364) ----
 * tile_bins[T,2] = (start, end); gaussian_ids[start:end] sorted by
 * (depth_bits << 32 | gid).  Per-tile counts are uncapped (no 2048 drop).
 * Returns the number of intersections, or -1 if it exceeds cap. */
int64_t orc_bin_sort(const OrcCamera* cam, int32_t N, const float* xys, const float* depths,
                     const int32_t* radii, const float* aabb, int64_t cap,
                     int32_t* tile_counts, int32_t* tile_bins, int32_t* gaussian_ids);

/* Number of depth chunks a tile with n entries is rasterised in (one = the
 * monolithic kernel).  Reference selector .mm:873-889 plus no-truncation. */
int32_t orc_tile_chunks(int32_t n, int32_t num_tiles);

/* ---- a5/a6/a8/a9: rasterize forward (+ optional backward) ----
 * Forward: nd_rasterize_forward (.metal:472-585) for single-chunk tiles,
 * rasterize_forward_chunked + merge (.metal:2633-2799) otherwise.
 * If v_out != NULL also runs the backward (.metal:898-1099, 2804-3031) and
 * writes v_xy[N,2], v_conic[N,3], v_rgb[N,3], v_opacity[N] (overwritten). */
void orc_rasterize(const OrcCamera* cam, int32_t N,
                   const float* xys, const float* conics, const float* colors,
                   const float* opacity_logits,
                   const int32_t* tile_bins, const int32_t* gaussian_ids,
                   float* final_Ts, int32_t* final_index, float* out_img,
                   const float* v_out,
                   float* v_xy, float* v_conic, float* v_rgb, float* v_opacity);

/* Work of the last orc_rasterize call: forward (pairs tested, sigma in
 * range, composited), backward (pairs tested, sigma in range, with
 * gradient).  Counts are per (pixel, entry) pair, algorithmic (no lockstep
 * overshoot).  The backward counts are zero when it did not run. */
void orc_raster_counts(int64_t out[6]);

/* ---- a7: separable SSIM + L1, training semantics (.metal:3053-3115, 3226-3313, 3396-3464) ----
 * Returns the loss sum over pixels (divide by H*W for msplat's loss value). */
double orc_ssim_loss(int32_t H, int32_t W, const float* img, const float* gt,
                     float ssim_weight, float inv_n, float* v_rendered,
                     float* h_buf /* [H,W,15] or NULL */, float* deriv_buf /* [H,W,15] or NULL */);

/* ---- a10: projection backward, gradients only (.metal:1813-1910) ----
 * For radii > 0 writes v_mean3d, v_scale (w.r.t. log scale), v_quat; zeros elsewhere. */
void orc_project_backward(const OrcCamera* cam, int32_t N,
                          const float* means, const float* scales, const float* quats,
                          const int32_t* radii, const float* conics,
                          const float* v_xy, const float* v_conic,
                          float* v_mean3d, float* v_scale, float* v_quat);

/* Bound on |GPU - oracle| of each gaussian's projection backward outputs
 * err_out[N,10] = (v_mean3d 3, v_scale 3, v_quat 4), absolute, by running
 * error analysis of the oracle's formulas evaluated on these inputs: the
 * inputs' own bounds err_xy[N,2] / err_conic[N,3] (NULL = exact inputs)
 * propagated, plus 4 x each operation's rounding (the GPU kernel's hardware
 * reciprocal / square root round to about 1 ulp).  Zeros for radii <= 0. */
void orc_project_backward_err(const OrcCamera* cam, int32_t N,
                              const float* means, const float* scales, const float* quats,
                              const int32_t* radii, const float* conics,
                              const float* v_xy, const float* v_conic,
                              const float* err_xy, const float* err_conic, float* err_out);

/* SH colour backward (sh_coeffs_to_color_vjp semantics, .metal:656-743 / 1924-1985):
 * for radii > 0 writes v_dc[N,3], v_rest[N,K-1,3] (zeros for unused bands). */
void orc_sh_backward(const OrcCamera* cam, int32_t N, const float* means,
                     const int32_t* radii, const float* v_rgb,
                     float* v_dc, float* v_rest);

/* ---- a11: fused_adam (.metal:1666-1689) ---- */
void orc_adam(int64_t n, float* param, const float* grad, float* m, float* v,
              float step_size, float beta1, float beta2, float bc2_sqrt, float eps);

/* ---- a12: accumulate_grad_stats (.metal:1643-1664) ---- */
void orc_grad_stats(int32_t N, const int32_t* radii, const float* v_xy,
                    float* vis, float* gnorm, float* max2d, float inv_max_dim);

/* ---- a13: one full train step (msplat_train_step, .mm:771-1330) ----
 * Updates params and Adam state in place (params[g], m[g], v[g] for the six
 * groups means, scales, quats, f_dc, f_rest, opacities) and the grad stats.
 * Optional outputs (may be NULL): out_img [H,W,3], radii [N],
 * v_xy/v_conic/v_rgb/v_opacity (raster gradients), v_mean3d/v_scale/v_quat.
 * Returns the loss value (sum / (H*W)), or NaN on capacity overflow. */
typedef struct OrcTrainOut {
    float* out_img; int32_t* radii;
    float* v_xy; float* v_conic; float* v_rgb; float* v_opacity;
    float* v_mean3d; float* v_scale; float* v_quat;
    float* v_rendered;
    /* Error bounds of the gradients (all optional).  mag_raster / err_raster
     * [N,9] for v_xy (2), v_conic (3), v_rgb (3), v_opacity (1): the sum of
     * the magnitudes of the terms each gradient is summed from, and a
     * first-order bound on |GPU - oracle| from the two evaluations'
     * arithmetic (running error analysis; absolute).  grad / grad_mag /
     * grad_err [6]: the gradient each Adam group is updated with (means,
     * scales, quats, f_dc, f_rest, opacities; zero where Adam leaves the
     * element as it is), its magnitude and its bound, shaped like the group. */
    float* mag_raster; float* err_raster;
    float* grad[6]; float* grad_mag[6]; float* grad_err[6];
} OrcTrainOut;

float orc_train_step(const OrcCamera* cam, int32_t N, int32_t rest_bases,
                     float* const params[6], float* const m[6], float* const v[6],
                     const OrcAdam* adam, const float* gt, float ssim_weight,
                     float* vis, float* gnorm, float* max2d,
                     const OrcTrainOut* out);

/* ---- render only (msplat_render / forward_pipeline(compute_loss=false)) ---- */
int orc_render(const OrcCamera* cam, int32_t N, const float* means, const float* scales,
               const float* quats, const float* f_dc, const float* f_rest,
               const float* opacity_logits, float* out_img,
               float* final_Ts, int32_t* final_index);

/* ---- a14: densify (msplat_densify .mm:1337-1592, kernels .metal:3475-3729) ----
 * Operates in place on the 6 parameter buffers and 12 Adam buffers of
 * capacity >= 3N.  random_samples holds 2N*3 standard normals (row-major,
 * sample (ord*2+k) for split ordinal ord and child k).  Returns the new N. */
typedef struct OrcDensifyArgs {
    int32_t N;
    float grad_thresh, size_thresh, screen_thresh; int32_t check_screen;
    float cull_alpha_thresh, cull_scale_thresh, cull_screen_size; int32_t check_huge;
    float half_max_dim;
    int32_t fr_stride;
} OrcDensifyArgs;

int32_t orc_densify(const OrcDensifyArgs* a, const float* xys_grad_norm,
                    const float* vis_counts, const float* max_2d_size,
                    float* const bufs[6], float* const m[6], float* const v[6],
                    const float* random_samples,
                    int32_t* split_flag_out, int32_t* dup_flag_out, int32_t* keep_flag_out);

/* ---- next to the path: evaluation metrics and the RGBA8 display image ----
 * psnr / l1_loss (model.cpp:25-40) and ssim_eval (ssim.cpp:61-123) of an
 * [H,W,3] render against its target: out[0] = PSNR, out[1] = SSIM with a
 * window_size-tap Gaussian of width sigma and edge-clamped borders,
 * out[2] = mean |r - g|.  rgba8: renderFromPoseToBuffer's conversion
 * (msplat_api.mm:230-238). */
void orc_image_metrics(int32_t H, int32_t W, const float* img, const float* gt,
                       int32_t window_size, float sigma, float out[3]);
void orc_image_to_rgba8(int64_t n_pixels, const float* img, uint8_t* rgba);

/* Initial scales of a point cloud (PointsTensor::scales,
 * kdtree_tensor.hpp:26-40): for each of n points the mean of sqrt of the
 * 2nd..4th smallest squared distances to all points (itself first), squared
 * distances summed per axis in fp32 like nanoflann's L2_Simple_Adaptor.
 * Brute force, O(n^2). */
void orc_knn_mean_dist(int64_t n, const float* xyz, float* out);

/* Target images.  resize_area (image_io.cpp:91-138): the overlap-weighted
 * box resample of an [sh,sw,3] image to [dh,dw,3].  undistort_roi /
 * undistort (image_io.cpp:140-330): the crop rectangle {x, y, w, h} of a
 * Brown-Conrady image (intr = fx fy cx cy, dist = k1 k2 p1 p2 k3) and the
 * undistorted image cropped to it (dst holds roi w x h x 3 floats; at most
 * w x h x 3). */
void orc_resize_area(int32_t sw, int32_t sh, const float* src, int32_t dw, int32_t dh, float* dst);
void orc_undistort_roi(int32_t w, int32_t h, const float intr[4], const float dist[5], int32_t roi[4]);
void orc_undistort(int32_t w, int32_t h, const float* src, const float intr[4], const float dist[5],
                   int32_t roi[4], float* dst);

#ifdef __cplusplus
}
#endif
#endif
