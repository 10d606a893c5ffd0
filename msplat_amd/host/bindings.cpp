// bindings.cpp — bindings.h-shaped functions over the C ABI.
#include "bindings.hpp"

#include <cstring>
#include <stdexcept>
#include <string>

namespace msplat {

namespace {

MTensor g_out_img;   // the render output, reused like the reference's g_tcache.out_img
MTensor g_radii;

void fill_render(MsplatRenderArgs& a, int num_points, MTensor& means3d, MTensor& scales,
                 float glob_scale, MTensor& quats, const float viewmat[16],
                 const float projmat[16], float fx, float fy, float cx, float cy,
                 unsigned img_height, unsigned img_width, const std::tuple<int, int, int>& tb,
                 float clip_thresh, unsigned degree, unsigned degrees_to_use,
                 const float cam_pos[3], MTensor& features_dc, MTensor& features_rest,
                 MTensor& opacities, const float background[3]) {
    std::memset(&a, 0, sizeof(a));
    a.num_points = num_points;
    a.means3d = means3d.data<float>();
    a.scales = scales.data<float>();
    a.glob_scale = glob_scale;
    a.quats = quats.data<float>();
    std::memcpy(a.viewmat, viewmat, sizeof(a.viewmat));
    std::memcpy(a.projmat, projmat, sizeof(a.projmat));
    a.fx = fx; a.fy = fy; a.cx = cx; a.cy = cy;
    a.img_height = img_height;
    a.img_width = img_width;
    a.tile_bounds[0] = std::get<0>(tb);
    a.tile_bounds[1] = std::get<1>(tb);
    a.tile_bounds[2] = std::get<2>(tb);
    a.clip_thresh = clip_thresh;
    a.degree = degree;
    a.degrees_to_use = degrees_to_use;
    for (int i = 0; i < 3; ++i) { a.cam_pos[i] = cam_pos[i]; a.background[i] = background[i]; }
    a.features_dc = features_dc.data<float>();
    a.features_rest = features_rest.defined() ? features_rest.data<float>() : nullptr;
    a.opacities = opacities.data<float>();
}

}  // namespace

void cleanup_msplat() {
    g_out_img.reset();
    g_radii.reset();
    msplat_hip_shutdown();
}

void cleanup_msplat_metal() { cleanup_msplat(); }

void* msplat_device() { return msplat_hip_get_stream(); }

void msplat_drain_gpu_times(std::vector<double>& out) {
    std::vector<double> ms(1 << 16);
    int n = 0;
    check(msplat_hip_drain_call_times(ms.data(), (int)ms.size(), &n), "drain gpu times");
    out.insert(out.end(), ms.begin(), ms.begin() + n);
}

MTensor gpu_zeros(std::vector<int64_t> shape, DType dtype) { return MTensor::zeros(std::move(shape), dtype); }
MTensor gpu_empty(std::vector<int64_t> shape, DType dtype) { return MTensor::empty(std::move(shape), dtype); }

void msplat_commit() { check(msplat_hip_commit(), "commit"); }
void msplat_gpu_sync() { check(msplat_hip_sync(), "sync"); }

void msplat_enable_gpu_timing(bool enable) { check(msplat_hip_enable_stage_timing(enable ? 1 : 0), "timing"); }

void msplat_drain_stage_times(std::vector<double> stage_times[], int max_stages, int& n_stages,
                              const char** stage_names) {
    std::vector<double> ms(max_stages);
    std::vector<int64_t> cnt(max_stages);
    int64_t calls = 0;
    check(msplat_hip_drain_stage_times(ms.data(), cnt.data(), stage_names, max_stages, &n_stages, &calls),
          "drain stage times");
    for (int i = 0; i < n_stages; ++i) {
        stage_times[i].clear();
        if (cnt[i]) stage_times[i].push_back(ms[i]);
    }
}

MTensor msplat_render(int num_points, MTensor& means3d, MTensor& scales, float glob_scale,
                      MTensor& quats, const float viewmat[16], const float projmat[16], float fx,
                      float fy, float cx, float cy, unsigned img_height, unsigned img_width,
                      const std::tuple<int, int, int> tile_bounds, float clip_thresh,
                      unsigned degree, unsigned degrees_to_use, const float cam_pos[3],
                      MTensor& features_dc, MTensor& features_rest, MTensor& opacities,
                      const float background[3]) {
    MsplatRenderArgs a;
    fill_render(a, num_points, means3d, scales, glob_scale, quats, viewmat, projmat, fx, fy, cx, cy,
                img_height, img_width, tile_bounds, clip_thresh, degree, degrees_to_use, cam_pos,
                features_dc, features_rest, opacities, background);
    const int64_t need = (int64_t)img_height * img_width * 3;
    if (!g_out_img.defined() || g_out_img.numel() != need)
        g_out_img = MTensor::empty({(int64_t)img_height, (int64_t)img_width, 3}, DType::Float32);
    check(msplat_hip_render(&a, g_out_img.data<float>()), "msplat_render");
    return g_out_img;
}

void msplat_render_to(float* out, int num_points, MTensor& means3d, MTensor& scales,
                      float glob_scale, MTensor& quats, const float viewmat[16],
                      const float projmat[16], float fx, float fy, float cx, float cy,
                      unsigned img_height, unsigned img_width,
                      const std::tuple<int, int, int> tile_bounds, float clip_thresh,
                      unsigned degree, unsigned degrees_to_use, const float cam_pos[3],
                      MTensor& features_dc, MTensor& features_rest, MTensor& opacities,
                      const float background[3]) {
    MsplatRenderArgs a;
    fill_render(a, num_points, means3d, scales, glob_scale, quats, viewmat, projmat, fx, fy, cx, cy,
                img_height, img_width, tile_bounds, clip_thresh, degree, degrees_to_use, cam_pos,
                features_dc, features_rest, opacities, background);
    check(msplat_hip_render(&a, out), "msplat_render");
}

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
    MTensor& xys_grad_norm, MTensor& max_2d_size, float inv_max_dim) {
    MsplatTrainArgs t;
    std::memset(&t, 0, sizeof(t));
    fill_render(t.r, num_points, means3d, scales, glob_scale, quats, viewmat, projmat, fx, fy, cx, cy,
                img_height, img_width, tile_bounds, clip_thresh, degree, degrees_to_use, cam_pos,
                features_dc, features_rest, opacities, background);
    t.gt = gt.data<float>();
    t.ssim_weight = ssim_weight;
    t.loss_inv_n = loss_inv_n;
    t.features_rest_bases = features_rest_bases;
    t.num_adam_groups = num_adam_groups;
    for (int g = 0; g < num_adam_groups && g < 6; ++g) {
        t.adam_params[g] = adam_params[g].data<float>();
        t.adam_exp_avg[g] = adam_exp_avg[g].data<float>();
        t.adam_exp_avg_sq[g] = adam_exp_avg_sq[g].data<float>();
        t.adam_step_sizes[g] = adam_step_sizes[g];
        t.adam_bc2_sqrts[g] = adam_bc2_sqrts[g];
    }
    t.adam_beta1 = adam_beta1;
    t.adam_beta2 = adam_beta2;
    t.adam_eps = adam_eps;
    t.vis_counts = vis_counts.data<float>();
    t.xys_grad_norm = xys_grad_norm.data<float>();
    t.max_2d_size = max_2d_size.data<float>();
    t.inv_max_dim = inv_max_dim;
    if (!g_radii.defined() || g_radii.size(0) < num_points)
        g_radii = MTensor::empty({(int64_t)num_points * 5 / 4 + 16}, DType::Int32);
    // The loss returned is that of the latest completed step, read without
    // waiting for this one, like the reference's read of loss_sum right after
    // committing the command buffer (msplat_metal.mm:1326): a synchronous read
    // here would drain the stream every step and leave the GPU waiting for
    // the host to launch the next one.
    check(msplat_hip_train_step(&t, g_radii.data<int32_t>(), nullptr), "msplat_train_step");
    float loss = 0.f;
    check(msplat_hip_last_loss(&loss, 0), "msplat_train_step");
    return {g_radii.view(num_points), loss};
}

namespace {
// A camera matrix or colour held in a tensor, as host values.  gpu_empty /
// gpu_zeros back such small tensors with mapped host memory, which the
// caller writes on the host as the reference's Model writes its shared
// buffers (model.cpp:113-115, prepareCam): it is read here directly, with no
// copy and no wait for the stream.  A larger, device-resident tensor is
// copied back (which waits for the stream).
template <int K>
void host_floats(const MTensor& t, float (&dst)[K], const char* what) {
    if (!t.defined() || t.numel() < K) throw std::runtime_error(std::string(what) + ": too few elements");
    if (t.mapped()) std::memcpy(dst, t.data<float>(), sizeof(dst));
    else t.copy_to_host(dst, sizeof(dst));
}
}  // namespace

MTensor msplat_render(int num_points, MTensor& means3d, MTensor& scales, float glob_scale,
                      MTensor& quats, MTensor& viewmat, MTensor& projmat, float fx, float fy,
                      float cx, float cy, unsigned img_height, unsigned img_width,
                      const std::tuple<int, int, int> tile_bounds, float clip_thresh,
                      unsigned degree, unsigned degrees_to_use, float cam_pos[3],
                      MTensor& features_dc, MTensor& features_rest, MTensor& opacities,
                      MTensor& background) {
    float vm[16], pm[16], bg[3];
    host_floats(viewmat, vm, "viewmat");
    host_floats(projmat, pm, "projmat");
    host_floats(background, bg, "background");
    return msplat_render(num_points, means3d, scales, glob_scale, quats, vm, pm, fx, fy, cx, cy,
                         img_height, img_width, tile_bounds, clip_thresh, degree, degrees_to_use,
                         cam_pos, features_dc, features_rest, opacities, bg);
}

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
    MTensor& xys_grad_norm, MTensor& max_2d_size, float inv_max_dim) {
    (void)window2d;
    float vm[16], pm[16], bg[3];
    host_floats(viewmat, vm, "viewmat");
    host_floats(projmat, pm, "projmat");
    host_floats(background, bg, "background");
    return msplat_train_step(num_points, means3d, scales, glob_scale, quats, vm, pm, fx, fy, cx, cy,
                             img_height, img_width, tile_bounds, clip_thresh, degree, degrees_to_use,
                             cam_pos, features_dc, features_rest, opacities, bg, gt, ssim_weight,
                             loss_inv_n, features_rest_bases, num_adam_groups, adam_params,
                             adam_exp_avg, adam_exp_avg_sq, adam_step_sizes, adam_bc2_sqrts,
                             adam_beta1, adam_beta2, adam_eps, vis_counts, xys_grad_norm,
                             max_2d_size, inv_max_dim);
}

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
                   MTensor& random_samples) {
    (void)split_flag; (void)dup_flag; (void)split_prefix; (void)dup_prefix;
    (void)keep_flag; (void)keep_prefix; (void)block_totals; (void)compact_scratch;
    if (!random_samples.defined()) throw std::runtime_error("msplat_densify: random_samples is required");
    return msplat_densify(N, buf_capacity, grad_thresh, size_thresh, screen_thresh, check_screen,
                          cull_alpha_thresh, cull_scale_thresh, cull_screen_size, check_huge,
                          xys_grad_norm, vis_counts, max_2d_size, half_max_dim, means_buf,
                          scales_buf, quats_buf, featuresDc_buf, featuresRest_buf, opacities_buf,
                          fr_stride, adam_exp_avg_buf, adam_exp_avg_sq_buf, random_samples,
                          (uint64_t)0);
}

int msplat_densify(int N, int buf_capacity, float grad_thresh, float size_thresh,
                   float screen_thresh, int check_screen, float cull_alpha_thresh,
                   float cull_scale_thresh, float cull_screen_size, int check_huge,
                   MTensor& xys_grad_norm, MTensor& vis_counts, MTensor& max_2d_size,
                   float half_max_dim, MTensor& means_buf, MTensor& scales_buf,
                   MTensor& quats_buf, MTensor& featuresDc_buf, MTensor& featuresRest_buf,
                   MTensor& opacities_buf, int fr_stride, MTensor adam_exp_avg_buf[],
                   MTensor adam_exp_avg_sq_buf[], MTensor& random_samples, uint64_t seed) {
    MsplatDensifyArgs a;
    std::memset(&a, 0, sizeof(a));
    a.N = N;
    a.buf_capacity = buf_capacity;
    a.grad_thresh = grad_thresh;
    a.size_thresh = size_thresh;
    a.screen_thresh = screen_thresh;
    a.check_screen = check_screen;
    a.cull_alpha_thresh = cull_alpha_thresh;
    a.cull_scale_thresh = cull_scale_thresh;
    a.cull_screen_size = cull_screen_size;
    a.check_huge = check_huge;
    a.xys_grad_norm = xys_grad_norm.data<float>();
    a.vis_counts = vis_counts.data<float>();
    a.max_2d_size = max_2d_size.data<float>();
    a.half_max_dim = half_max_dim;
    MTensor* bufs[6] = {&means_buf, &scales_buf, &quats_buf, &featuresDc_buf, &featuresRest_buf,
                        &opacities_buf};
    for (int g = 0; g < 6; ++g) {
        a.bufs[g] = bufs[g]->defined() ? bufs[g]->data<float>() : nullptr;
        a.adam_exp_avg_buf[g] = adam_exp_avg_buf[g].data<float>();
        a.adam_exp_avg_sq_buf[g] = adam_exp_avg_sq_buf[g].data<float>();
    }
    a.fr_stride = fr_stride;
    a.random_samples = random_samples.defined() ? random_samples.data<float>() : nullptr;
    a.seed = seed;
    int32_t out = 0;
    check(msplat_hip_densify(&a, &out), "msplat_densify");
    return out;
}

}  // namespace msplat
