// bindings.hpp — the reference's backend interface (core/metal/bindings.h)
// over the C ABI of include/msplat_hip.h, in namespace msplat.  Every
// function of bindings.h is here with its parameter list and return value
// (bindings.h:8-84), so Model code written against bindings.h compiles
// against this header; MTensor here holds HIP device memory, and the camera
// matrices and background that bindings.h passes as MTensors are read back to
// the host (64 + 64 + 12 bytes per call).  Next to them, the forms this
// build's own Model uses: the same calls with the matrices and background as
// host float arrays, a render into a caller's buffer, and a densify without
// the scratch tensors (the library owns its scratch).
#pragma once

#include <tuple>
#include <vector>

#include "mtensor.hpp"

namespace msplat {

// cleanup_msplat_metal (bindings.h:8): releases the context and its caches.
void cleanup_msplat();
void cleanup_msplat_metal();

// msplat_device (bindings.h:11-15): the backend's device handle; here the
// context's HIP stream (hipStream_t), the handle HIP code orders its own work
// against, or NULL before the context exists.
void* msplat_device();

// gpu_zeros / gpu_empty (bindings.h:18-19).
MTensor gpu_zeros(std::vector<int64_t> shape, DType dtype);
MTensor gpu_empty(std::vector<int64_t> shape, DType dtype);

// msplat_commit / msplat_gpu_sync (bindings.h:22-25).
void msplat_commit();
void msplat_gpu_sync();

// Stage timing (bindings.h:28-33).  msplat_drain_gpu_times gives each timed
// call's bracketed GPU milliseconds.
void msplat_enable_gpu_timing(bool enable);
void msplat_drain_gpu_times(std::vector<double>& out);
void msplat_drain_stage_times(std::vector<double> stage_times[], int max_stages, int& n_stages,
                              const char** stage_names);

// msplat_render (bindings.h:37-46).  viewmat / projmat are 4x4 row-major host
// matrices here (the reference keeps them in shared GPU buffers).  Returns
// the (H, W, 3) image, which stays valid until the next render.
MTensor msplat_render(int num_points, MTensor& means3d, MTensor& scales, float glob_scale,
                      MTensor& quats, const float viewmat[16], const float projmat[16], float fx,
                      float fy, float cx, float cy, unsigned img_height, unsigned img_width,
                      const std::tuple<int, int, int> tile_bounds, float clip_thresh,
                      unsigned degree, unsigned degrees_to_use, const float cam_pos[3],
                      MTensor& features_dc, MTensor& features_rest, MTensor& opacities,
                      const float background[3]);
// The same render written straight into a caller's device buffer of
// img_height * img_width * 3 floats (no copy through the cached image).
void msplat_render_to(float* out, int num_points, MTensor& means3d, MTensor& scales,
                      float glob_scale, MTensor& quats, const float viewmat[16],
                      const float projmat[16], float fx, float fy, float cx, float cy,
                      unsigned img_height, unsigned img_width,
                      const std::tuple<int, int, int> tile_bounds, float clip_thresh,
                      unsigned degree, unsigned degrees_to_use, const float cam_pos[3],
                      MTensor& features_dc, MTensor& features_rest, MTensor& opacities,
                      const float background[3]);

// msplat_train_step (bindings.h:50-67): fused forward + loss + backward +
// Adam + grad stats.  Returns (radii [N], loss value).  window2d is not
// needed (the kernels carry the separable taps).
std::tuple<MTensor, float> msplat_train_step(
    int num_points, MTensor& means3d, MTensor& scales, float glob_scale, MTensor& quats,
    const float viewmat[16], const float projmat[16], float fx, float fy, float cx, float cy,
    unsigned img_height, unsigned img_width, const std::tuple<int, int, int> tile_bounds,
    float clip_thresh, unsigned degree, unsigned degrees_to_use, const float cam_pos[3],
    MTensor& features_dc, MTensor& features_rest, MTensor& opacities, const float background[3],
    MTensor& gt, float ssim_weight, float loss_inv_n, int features_rest_bases,
    int num_adam_groups, MTensor adam_params[], MTensor adam_exp_avg[],
    MTensor adam_exp_avg_sq[], float adam_step_sizes[], float adam_bc2_sqrts[],
    float adam_beta1, float adam_beta2, float adam_eps, MTensor& vis_counts,
    MTensor& xys_grad_norm, MTensor& max_2d_size, float inv_max_dim);

// bindings.h:37-46 exactly: viewmat, projmat [4,4] and background [3] as
// tensors.
MTensor msplat_render(int num_points, MTensor& means3d, MTensor& scales, float glob_scale,
                      MTensor& quats, MTensor& viewmat, MTensor& projmat, float fx, float fy,
                      float cx, float cy, unsigned img_height, unsigned img_width,
                      const std::tuple<int, int, int> tile_bounds, float clip_thresh,
                      unsigned degree, unsigned degrees_to_use, float cam_pos[3],
                      MTensor& features_dc, MTensor& features_rest, MTensor& opacities,
                      MTensor& background);

// bindings.h:50-67 exactly (window2d is accepted and unused, as by the
// reference's separable SSIM kernels, msplat_metal.mm:1002-1025).
std::tuple<MTensor, float> msplat_train_step(
    int num_points, MTensor& means3d, MTensor& scales, float glob_scale, MTensor& quats,
    MTensor& viewmat, MTensor& projmat, float fx, float fy, float cx, float cy,
    unsigned img_height, unsigned img_width, const std::tuple<int, int, int> tile_bounds,
    float clip_thresh, unsigned degree, unsigned degrees_to_use, float cam_pos[3],
    MTensor& features_dc, MTensor& features_rest, MTensor& opacities, MTensor& background,
    MTensor& gt, MTensor& window2d, float ssim_weight, float loss_inv_n, int features_rest_bases,
    int num_adam_groups, MTensor adam_params[], MTensor adam_exp_avg[],
    MTensor adam_exp_avg_sq[], float adam_step_sizes[], float adam_bc2_sqrts[],
    float adam_beta1, float adam_beta2, float adam_eps, MTensor& vis_counts,
    MTensor& xys_grad_norm, MTensor& max_2d_size, float inv_max_dim);

// bindings.h:69-84 exactly: the eight flag / prefix / total / scratch
// tensors are accepted and unused (the library sizes its own), and
// random_samples ([2N,3] normals, as the reference's Model fills them) is
// required.
int msplat_densify(int N, int buf_capacity, float grad_thresh, float size_thresh,
                   float screen_thresh, int check_screen, float cull_alpha_thresh,
                   float cull_scale_thresh, float cull_screen_size, int check_huge,
                   MTensor& xys_grad_norm, MTensor& vis_counts, MTensor& max_2d_size,
                   float half_max_dim, MTensor& means_buf, MTensor& scales_buf,
                   MTensor& quats_buf, MTensor& featuresDc_buf, MTensor& featuresRest_buf,
                   MTensor& opacities_buf, int fr_stride, MTensor adam_exp_avg_buf[],
                   MTensor adam_exp_avg_sq_buf[], MTensor& split_flag, MTensor& dup_flag,
                   MTensor& split_prefix, MTensor& dup_prefix, MTensor& keep_flag,
                   MTensor& keep_prefix, MTensor& block_totals, MTensor& compact_scratch,
                   MTensor& random_samples);

// msplat_densify (bindings.h:69-84).  The flag / prefix / scratch buffers of
// the reference are internal to the library; random_samples may be an
// undefined tensor, in which case the library draws them from `seed`.
int msplat_densify(int N, int buf_capacity, float grad_thresh, float size_thresh,
                   float screen_thresh, int check_screen, float cull_alpha_thresh,
                   float cull_scale_thresh, float cull_screen_size, int check_huge,
                   MTensor& xys_grad_norm, MTensor& vis_counts, MTensor& max_2d_size,
                   float half_max_dim, MTensor& means_buf, MTensor& scales_buf,
                   MTensor& quats_buf, MTensor& featuresDc_buf, MTensor& featuresRest_buf,
                   MTensor& opacities_buf, int fr_stride, MTensor adam_exp_avg_buf[],
                   MTensor adam_exp_avg_sq_buf[], MTensor& random_samples, uint64_t seed);

}  // namespace msplat
