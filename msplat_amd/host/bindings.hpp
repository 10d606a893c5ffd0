// bindings.hpp — the reference's backend interface (core/metal/bindings.h)
// with the same functions, parameter lists and return values, implemented
// over the C ABI of include/msplat_hip.h.  Model code written against
// bindings.h compiles against this header unchanged apart from the MTensor
// type, which here holds HIP device memory.
#pragma once

#include <tuple>
#include <vector>

#include "mtensor.hpp"

namespace msplat {

// cleanup_msplat_metal (bindings.h:8): releases the context and its caches.
void cleanup_msplat();

// gpu_zeros / gpu_empty (bindings.h:18-19).
MTensor gpu_zeros(std::vector<int64_t> shape, DType dtype);
MTensor gpu_empty(std::vector<int64_t> shape, DType dtype);

// msplat_commit / msplat_gpu_sync (bindings.h:22-25).
void msplat_commit();
void msplat_gpu_sync();

// Stage timing (bindings.h:28-33).
void msplat_enable_gpu_timing(bool enable);
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
