// trainer.cpp — GaussianTrainer (python/bindings.cpp:101-280) and the C API
// of include/msplat_trainer.h.
#include "../../include/msplat_trainer.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <map>
#include <memory>
#include <numeric>
#include <random>
#include <string>
#include <vector>

#include "dataset.hpp"
#include "model.hpp"

namespace msplat {

namespace {

std::string g_err;

// Camera::getImage (input_data.cpp:54-65): the image at 1/ds resolution,
// (W / ds) x (H / ds) by the reference's area resize, on the GPU.
MTensor downscaled(const MTensor& full, int W, int H, int ds) {
    const int w2 = W / ds, h2 = H / ds;
    if (w2 <= 0 || h2 <= 0) throw std::runtime_error("image too small for the downscale factor");
    MTensor t = gpu_empty({h2, w2, 3}, DType::Float32);
    check(msplat_hip_resize_area(full.data<float>(), W, H, t.data<float>(), w2, h2), "resize");
    return t;
}

}  // namespace

class GaussianTrainer {
public:
    GaussianTrainer(const MsplatTrainerConfig& c, int64_t n, const float* const params[6],
                    int n_cams, const MsplatTrainerCamera* cams, const float* const* targets,
                    bool on_device)
        : cfg(c), rng(c.seed) {
        if (n_cams <= 0) throw std::runtime_error("at least one camera is needed");
        ModelConfig mc;
        mc.iterations = c.iterations;
        mc.shDegree = c.shDegree;
        mc.shDegreeInterval = c.shDegreeInterval;
        mc.ssimWeight = c.ssimWeight;
        mc.numDownscales = c.numDownscales;
        mc.resolutionSchedule = c.resolutionSchedule;
        mc.refineEvery = c.refineEvery;
        mc.warmupLength = c.warmupLength;
        mc.resetAlphaEvery = c.resetAlphaEvery;
        mc.densifyGradThresh = c.densifyGradThresh;
        mc.densifySizeThresh = c.densifySizeThresh;
        mc.stopScreenSizeAt = c.stopScreenSizeAt;
        mc.splitScreenSize = c.splitScreenSize;
        mc.cullAlphaThresh = c.cullAlphaThresh;
        mc.cullScaleThresh = c.cullScaleThresh;
        mc.cullScreenSize = c.cullScreenSize;
        for (int i = 0; i < 3; ++i) mc.bgColor[i] = c.bgColor[i];
        model = std::make_unique<Model>(mc, n_cams, n, params, on_device);
        cameras.resize(n_cams);
        gpu_images.resize(n_cams);
        for (int i = 0; i < n_cams; ++i) {
            Camera& k = cameras[i];
            k.width = cams[i].width; k.height = cams[i].height;
            k.fx = cams[i].fx; k.fy = cams[i].fy; k.cx = cams[i].cx; k.cy = cams[i].cy;
            std::memcpy(k.camToWorld, cams[i].camToWorld, sizeof(k.camToWorld));
            if (!targets || !targets[i]) throw std::runtime_error("missing target image");
            MTensor t = gpu_empty({k.height, k.width, 3}, DType::Float32);
            if (on_device) t.copy_from_device(targets[i], t.nbytes());
            else t.copy_from_host(targets[i], t.nbytes());
            gpu_images[i][1] = t;
        }
        cam_indices.resize(n_cams);
        std::iota(cam_indices.begin(), cam_indices.end(), (size_t)0);
        shuffle_cameras();
    }

    MsplatStats step() {   // bindings.cpp:144-167
        current_step++;
        const size_t ci = next_camera();
        Camera& cam = cameras[ci];
        MTensor& gt = gpu_image(ci, model->getDownscaleFactor(current_step));
        const auto t0 = std::chrono::high_resolution_clock::now();
        model->fullIteration(cam, current_step, gt);
        model->schedulersStep(current_step);
        model->afterTrain(current_step);
        msplat_commit();
        const auto t1 = std::chrono::high_resolution_clock::now();
        MsplatStats s;
        s.iteration = current_step;
        s.splatCount = (int32_t)model->numActive();
        s.msPerStep = std::chrono::duration_cast<std::chrono::microseconds>(t1 - t0).count() / 1000.0f;
        return s;
    }

    // render_from_pose (bindings.cpp:236-259): intrinsics of the reference
    // camera, the given pose, the current step's resolution and SH degree.
    MTensor render_pose(const float camToWorld[16], int ref) {
        if (ref < 0 || ref >= (int)cameras.size()) throw std::runtime_error("ref_cam_idx out of range");
        Camera cam = cameras[ref];
        std::memcpy(cam.camToWorld, camToWorld, sizeof(cam.camToWorld));
        cam.cached = false;
        return model->render(cam, current_step);
    }

    // Trainer::evaluate (msplat_api.mm:138-166): render at the final
    // iteration's resolution against the target box-filtered to it.
    MsplatEvalMetrics evaluate(int n, const MsplatTrainerCamera* cams, const float* const* images,
                               bool on_device) {
        if (n <= 0 || !cams || !images) throw std::runtime_error("no test cameras");
        const int ds = model->getDownscaleFactor(cfg.iterations);
        double sp = 0.0, ss = 0.0, sl = 0.0;
        for (int i = 0; i < n; ++i) {
            Camera cam;
            cam.width = cams[i].width; cam.height = cams[i].height;
            cam.fx = cams[i].fx; cam.fy = cams[i].fy; cam.cx = cams[i].cx; cam.cy = cams[i].cy;
            std::memcpy(cam.camToWorld, cams[i].camToWorld, sizeof(cam.camToWorld));
            if (!images[i]) throw std::runtime_error("missing test image");
            MTensor gt = gpu_empty({cam.height, cam.width, 3}, DType::Float32);
            if (on_device) gt.copy_from_device(images[i], gt.nbytes());
            else gt.copy_from_host(images[i], gt.nbytes());
            if (ds > 1) gt = downscaled(gt, cam.width, cam.height, ds);
            const int h2 = (int)gt.size(0), w2 = (int)gt.size(1);
            MTensor img = model->render(cam, cfg.iterations);
            if (img.size(0) != h2 || img.size(1) != w2)
                throw std::runtime_error("render and target sizes differ");
            MsplatImageMetrics m;
            check(msplat_hip_image_metrics(img.data<float>(), gt.data<float>(), h2, w2, 11, 1.5f, &m),
                  "image metrics");
            sp += m.psnr;
            ss += m.ssim;
            sl += m.l1;
        }
        MsplatEvalMetrics out;
        out.psnr = (float)(sp / n);
        out.ssim = (float)(ss / n);
        out.l1 = (float)(sl / n);
        out.numTest = n;
        out.numGaussians = (int32_t)model->numActive();
        return out;
    }

    int load_checkpoint(const std::string& path) {   // Trainer::loadCheckpoint (msplat_api.mm:252-257)
        current_step = model->loadCheckpoint(path);
        shuffle_cameras();
        return current_step;
    }

    // The same into a caller's device buffer (dst NULL: size only).
    void render_pose_to(const float camToWorld[16], int ref, float* dst, int& w, int& h) {
        if (ref < 0 || ref >= (int)cameras.size()) throw std::runtime_error("ref_cam_idx out of range");
        Camera cam = cameras[ref];
        std::memcpy(cam.camToWorld, camToWorld, sizeof(cam.camToWorld));
        cam.cached = false;
        model->renderTo(cam, current_step, dst, w, h);
    }

    MTensor render_camera(int i) {
        if (i < 0 || i >= (int)cameras.size()) throw std::runtime_error("camera index out of range");
        return model->render(cameras[i], current_step);
    }

    MsplatTrainerConfig cfg;
    std::unique_ptr<Model> model;
    int current_step = 0;

private:
    void shuffle_cameras() {
        if (cfg.shuffleCameras) std::shuffle(cam_indices.begin(), cam_indices.end(), rng);
        cam_iter_pos = 0;
    }
    size_t next_camera() {
        if (cam_iter_pos >= cam_indices.size()) shuffle_cameras();
        return cam_indices[cam_iter_pos++];
    }
    // Camera::getGPUImage (input_data.cpp:67-76): per-factor cache.
    MTensor& gpu_image(size_t ci, int ds) {
        auto& cache = gpu_images[ci];
        auto it = cache.find(ds);
        if (it != cache.end()) return it->second;
        const Camera& k = cameras[ci];
        MTensor t = downscaled(cache.at(1), k.width, k.height, ds);
        return cache[ds] = t;
    }

    std::vector<Camera> cameras;
    std::vector<std::map<int, MTensor>> gpu_images;
    std::vector<size_t> cam_indices;
    size_t cam_iter_pos = 0;
    std::mt19937 rng;
};

}  // namespace msplat

using msplat::GaussianTrainer;

namespace {

template <typename F>
auto guarded(F&& f, decltype(f()) on_error) -> decltype(f()) {
    try {
        return f();
    } catch (const std::exception& e) {
        msplat::g_err = e.what();
        return on_error;
    }
}

GaussianTrainer* T(MsplatTrainer t) { return static_cast<GaussianTrainer*>(t); }

MsplatPixelBuffer to_host(const msplat::MTensor& img) {
    MsplatPixelBuffer b{nullptr, 0, 0};
    b.height = (int32_t)img.size(0);
    b.width = (int32_t)img.size(1);
    b.data = static_cast<float*>(std::malloc(img.nbytes()));
    if (!b.data) throw std::runtime_error("out of host memory");
    img.copy_to_host(b.data, img.nbytes());
    return b;
}

}  // namespace

extern "C" {

MsplatTrainer msplat_trainer_create(const MsplatTrainerConfig* config, int64_t n,
                                    const float* const params[6], int32_t n_cameras,
                                    const MsplatTrainerCamera* cameras,
                                    const float* const* targets, int32_t on_device) {
    return guarded([&]() -> MsplatTrainer {
        if (!config || !params || !cameras || !targets) throw std::runtime_error("null argument");
        return new GaussianTrainer(*config, n, params, n_cameras, cameras, targets, on_device != 0);
    }, nullptr);
}

void msplat_trainer_destroy(MsplatTrainer t) { delete T(t); }

const char* msplat_trainer_last_error(void) { return msplat::g_err.c_str(); }

MsplatStats msplat_trainer_step(MsplatTrainer t) {
    MsplatStats bad{-1, -1, 0.f};
    if (!t) return bad;
    return guarded([&]() { return T(t)->step(); }, bad);
}

float msplat_trainer_last_loss(MsplatTrainer t, int32_t wait) {
    if (!t) return NAN;
    float v = NAN;
    if (msplat_hip_last_loss(&v, wait) != MSPLAT_OK) return NAN;
    return v;
}

MsplatPixelBuffer msplat_trainer_render(MsplatTrainer t, int32_t cameraIndex) {
    MsplatPixelBuffer empty{nullptr, 0, 0};
    if (!t) return empty;
    return guarded([&]() { return to_host(T(t)->render_camera(cameraIndex)); }, empty);
}

MsplatPixelBuffer msplat_trainer_render_pose(MsplatTrainer t, const float camToWorld[16],
                                             int32_t refCameraIndex) {
    MsplatPixelBuffer empty{nullptr, 0, 0};
    if (!t || !camToWorld) return empty;
    return guarded([&]() { return to_host(T(t)->render_pose(camToWorld, refCameraIndex)); }, empty);
}

int32_t msplat_trainer_render_pose_to_buffer(MsplatTrainer t, const float camToWorld[16],
                                             int32_t refCameraIndex, uint8_t* outRGBA,
                                             int32_t* outWidth, int32_t* outHeight) {
    if (!t || !camToWorld) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        msplat::MTensor img = T(t)->render_pose(camToWorld, refCameraIndex);
        const int h = (int)img.size(0), w = (int)img.size(1);
        if (outWidth) *outWidth = w;
        if (outHeight) *outHeight = h;
        if (!outRGBA) return MSPLAT_OK;
        const int64_t n = (int64_t)w * h;
        msplat::MTensor rgba = msplat::gpu_empty({n}, msplat::DType::Int32);   // 4 bytes per pixel
        msplat::check(msplat_hip_image_to_rgba8(img.data<float>(), n, rgba.data<uint8_t>()), "rgba8");
        rgba.copy_to_host(outRGBA, (size_t)n * 4);
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_render_pose_device(MsplatTrainer t, const float camToWorld[16],
                                          int32_t refCameraIndex, float* outDevice,
                                          int32_t* outWidth, int32_t* outHeight) {
    if (!t || !camToWorld) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        int w = 0, h = 0;
        T(t)->render_pose_to(camToWorld, refCameraIndex, outDevice, w, h);
        if (outWidth) *outWidth = (int32_t)w;
        if (outHeight) *outHeight = (int32_t)h;
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_prepare_cam(const MsplatTrainerCamera* cam, int32_t downscale, MsplatCamSetup* out) {
    if (!cam || !out || downscale < 1) return MSPLAT_ERR_ARG;
    msplat::Camera k;
    k.width = cam->width; k.height = cam->height;
    k.fx = cam->fx; k.fy = cam->fy; k.cx = cam->cx; k.cy = cam->cy;
    std::memcpy(k.camToWorld, cam->camToWorld, sizeof(k.camToWorld));
    int w = 0, h = 0;
    msplat::prepare_camera(k, (float)downscale, out->fx, out->fy, out->cx, out->cy, w, h);
    out->width = w;
    out->height = h;
    std::memcpy(out->viewmat, k.cachedViewMat, sizeof(out->viewmat));
    std::memcpy(out->projmat, k.cachedProjViewMat, sizeof(out->projmat));
    for (int i = 0; i < 3; ++i) out->cam_pos[i] = k.cachedCamPos[i];
    out->tile_bounds[0] = (w + msplat::TILE - 1) / msplat::TILE;
    out->tile_bounds[1] = (h + msplat::TILE - 1) / msplat::TILE;
    out->tile_bounds[2] = 1;
    return MSPLAT_OK;
}

MsplatEvalMetrics msplat_trainer_evaluate(MsplatTrainer t, int32_t n_test,
                                          const MsplatTrainerCamera* cameras,
                                          const float* const* images, int32_t on_device) {
    MsplatEvalMetrics bad{0.f, 0.f, 0.f, 0, 0};
    if (!t) return bad;
    return guarded([&]() { return T(t)->evaluate(n_test, cameras, images, on_device != 0); }, bad);
}

int32_t msplat_trainer_export_ply(MsplatTrainer t, const char* path) {
    if (!t || !path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        T(t)->model->savePly(path, T(t)->current_step);
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_export_splat(MsplatTrainer t, const char* path) {
    if (!t || !path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        T(t)->model->saveSplat(path);
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_save_checkpoint(MsplatTrainer t, const char* path) {
    if (!t || !path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        T(t)->model->saveCheckpoint(path, T(t)->current_step);
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_load_checkpoint(MsplatTrainer t, const char* path) {
    if (!t || !path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t { return T(t)->load_checkpoint(path); }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_load_ply(MsplatTrainer t, const char* path) {
    if (!t || !path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t { return T(t)->model->loadPly(path); }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_set_crs(MsplatTrainer t, float scale, const float translation[3],
                               int32_t keep) {
    if (!t || !translation || !(scale > 0.f)) return MSPLAT_ERR_ARG;
    msplat::Crs& c = T(t)->model->crs;
    c.scale = scale;
    for (int i = 0; i < 3; ++i) c.translation[i] = translation[i];
    c.keep = keep != 0;
    return MSPLAT_OK;
}

namespace {
msplat::HostGaussians host_gaussians(int64_t n, int32_t rest_bases, const float* const params[6]) {
    if (n < 0 || rest_bases < 0 || !params) throw std::runtime_error("bad scene arguments");
    const size_t per[6] = {3, 3, 4, 3, (size_t)rest_bases * 3, 1};
    for (int g = 0; g < 6; ++g)
        if (!params[g] && (per[g] > 0 && n > 0)) throw std::runtime_error("null parameter array");
    msplat::HostGaussians h;
    h.n = n;
    h.rest_bases = rest_bases;
    std::vector<float>* dst[6] = {&h.means, &h.scales, &h.quats, &h.f_dc, &h.f_rest, &h.opacities};
    for (int g = 0; g < 6; ++g)
        dst[g]->assign(params[g], params[g] + (size_t)n * per[g]);
    return h;
}
msplat::Crs make_crs(float scale, const float translation[3], int32_t keep) {
    msplat::Crs c;
    if (keep) {
        if (!(scale > 0.f) || !translation) throw std::runtime_error("bad coordinate normalisation");
        c.scale = scale;
        for (int i = 0; i < 3; ++i) c.translation[i] = translation[i];
    }
    c.keep = keep != 0;
    return c;
}
}  // namespace

int32_t msplat_scene_write_ply(const char* path, int64_t n, int32_t rest_bases,
                               const float* const params[6], float crs_scale,
                               const float crs_translation[3], int32_t keep_crs, int32_t step) {
    if (!path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        msplat::save_gaussian_ply(path, host_gaussians(n, rest_bases, params),
                                  make_crs(crs_scale, crs_translation, keep_crs), step);
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_scene_write_splat(const char* path, int64_t n, int32_t rest_bases,
                                 const float* const params[6], float crs_scale,
                                 const float crs_translation[3], int32_t keep_crs) {
    if (!path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        msplat::save_gaussian_splat(path, host_gaussians(n, rest_bases, params),
                                    make_crs(crs_scale, crs_translation, keep_crs));
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_scene_read_ply(const char* path, float crs_scale, const float crs_translation[3],
                              int32_t keep_crs, int64_t* n, int32_t* rest_bases, int32_t* step,
                              float* const params[6]) {
    if (!path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        int st = 0;
        msplat::HostGaussians g =
            msplat::load_gaussian_ply(path, make_crs(crs_scale, crs_translation, keep_crs), &st);
        if (n) *n = g.n;
        if (rest_bases) *rest_bases = g.rest_bases;
        if (step) *step = st;
        if (params) {
            const std::vector<float>* src[6] = {&g.means, &g.scales, &g.quats,
                                                &g.f_dc, &g.f_rest, &g.opacities};
            for (int k = 0; k < 6; ++k) {
                if (!params[k]) throw std::runtime_error("null parameter buffer");
                std::memcpy(params[k], src[k]->data(), src[k]->size() * sizeof(float));
            }
        }
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

MsplatDataset msplat_dataset_create(const char* path, const char* image_dir) {
    if (!path) return nullptr;
    return guarded([&]() -> MsplatDataset {
        return new msplat::Dataset(msplat::load_colmap(path, image_dir ? image_dir : ""));
    }, nullptr);
}

void msplat_dataset_destroy(MsplatDataset ds) { delete static_cast<msplat::Dataset*>(ds); }

namespace {
msplat::Dataset* D(MsplatDataset ds) { return static_cast<msplat::Dataset*>(ds); }
const msplat::DatasetCamera& dcam(MsplatDataset ds, int32_t i) {
    if (!ds || i < 0 || i >= (int32_t)D(ds)->cameras.size())
        throw std::runtime_error("camera index out of range");
    return D(ds)->cameras[i];
}
}  // namespace

int32_t msplat_dataset_num_cameras(MsplatDataset ds) {
    return ds ? (int32_t)D(ds)->cameras.size() : -1;
}

int32_t msplat_dataset_camera(MsplatDataset ds, int32_t i, MsplatTrainerCamera* cam,
                              float distortion[4], const char** image_path) {
    return guarded([&]() -> int32_t {
        const msplat::DatasetCamera& c = dcam(ds, i);
        if (cam) {
            cam->width = c.width; cam->height = c.height;
            cam->fx = c.fx; cam->fy = c.fy; cam->cx = c.cx; cam->cy = c.cy;
            std::memcpy(cam->camToWorld, c.camToWorld, sizeof(c.camToWorld));
        }
        if (distortion) {
            distortion[0] = c.k1; distortion[1] = c.k2; distortion[2] = c.p1; distortion[3] = c.p2;
        }
        if (image_path) *image_path = c.filePath.c_str();
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_dataset_camera_pose(MsplatDataset ds, int32_t i, float camToWorld[16]) {
    if (!camToWorld) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        std::memcpy(camToWorld, dcam(ds, i).camToWorld, 16 * sizeof(float));
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int64_t msplat_dataset_num_points(MsplatDataset ds) {
    return ds ? (int64_t)(D(ds)->xyz.size() / 3) : -1;
}

int32_t msplat_dataset_points(MsplatDataset ds, float* xyz, uint8_t* rgb) {
    if (!ds) return MSPLAT_ERR_ARG;
    if (xyz) std::memcpy(xyz, D(ds)->xyz.data(), D(ds)->xyz.size() * sizeof(float));
    if (rgb) std::memcpy(rgb, D(ds)->rgb.data(), D(ds)->rgb.size());
    return MSPLAT_OK;
}

int32_t msplat_dataset_normalisation(MsplatDataset ds, float* scale, float translation[3]) {
    if (!ds) return MSPLAT_ERR_ARG;
    if (scale) *scale = D(ds)->scale;
    if (translation)
        for (int k = 0; k < 3; ++k) translation[k] = D(ds)->translation[k];
    return MSPLAT_OK;
}

int32_t msplat_dataset_init_gaussians(MsplatDataset ds, int32_t sh_degree, float* const params[6]) {
    if (!ds || !params) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        msplat::HostGaussians g = msplat::init_gaussians(D(ds)->xyz, D(ds)->rgb, sh_degree);
        const std::vector<float>* src[6] = {&g.means, &g.scales, &g.quats,
                                            &g.f_dc, &g.f_rest, &g.opacities};
        for (int k = 0; k < 6; ++k) {
            if (!params[k]) throw std::runtime_error("null parameter buffer");
            std::memcpy(params[k], src[k]->data(), src[k]->size() * sizeof(float));
        }
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_splat_count(MsplatTrainer t) { return t ? (int32_t)T(t)->model->numActive() : -1; }

int32_t msplat_trainer_iteration(MsplatTrainer t) { return t ? T(t)->current_step : -1; }

int32_t msplat_trainer_group(MsplatTrainer t, int32_t g, int32_t which, float** devPtr,
                             int64_t* rows, int64_t* rowFloats) {
    if (!t) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        msplat::MTensor m = T(t)->model->group(g, which);
        if (devPtr) *devPtr = m.data<float>();
        if (rows) *rows = m.size(0);
        if (rowFloats) *rowFloats = m.stride0();
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

}  // extern "C"
