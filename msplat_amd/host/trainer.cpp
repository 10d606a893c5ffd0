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

#include "model.hpp"

namespace msplat {

namespace {

std::string g_err;

// Box filter by an integer factor d over the floor(W/d) x floor(H/d) grid:
// the area resampling of Camera::getImage (input_data.cpp:54-65) for image
// sizes divisible by d.
std::vector<float> box_downscale(const std::vector<float>& img, int W, int H, int d, int& w2,
                                 int& h2) {
    w2 = W / d;
    h2 = H / d;
    std::vector<float> out((size_t)w2 * h2 * 3, 0.f);
    const float inv = 1.f / (float)(d * d);
    for (int y = 0; y < h2; ++y)
        for (int x = 0; x < w2; ++x)
            for (int c = 0; c < 3; ++c) {
                float acc = 0.f;
                for (int dy = 0; dy < d; ++dy)
                    for (int dx = 0; dx < d; ++dx)
                        acc += img[((size_t)(y * d + dy) * W + (x * d + dx)) * 3 + c];
                out[((size_t)y * w2 + x) * 3 + c] = acc * inv;
            }
    return out;
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
        MTensor& full = cache.at(1);
        std::vector<float> host((size_t)full.numel());
        full.copy_to_host(host.data(), full.nbytes());
        int w2, h2;
        std::vector<float> small = box_downscale(host, k.width, k.height, ds, w2, h2);
        MTensor t = gpu_empty({h2, w2, 3}, DType::Float32);
        t.copy_from_host(small.data(), small.size() * sizeof(float));
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
        std::vector<float> host((size_t)img.numel());
        img.copy_to_host(host.data(), img.nbytes());
        for (size_t p = 0; p < (size_t)w * h; ++p) {
            for (int c = 0; c < 3; ++c) {
                const float v = std::min(std::max(host[3 * p + c], 0.f), 1.f);
                outRGBA[4 * p + c] = (uint8_t)std::lround(v * 255.f);
            }
            outRGBA[4 * p + 3] = 255;
        }
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int32_t msplat_trainer_render_pose_device(MsplatTrainer t, const float camToWorld[16],
                                          int32_t refCameraIndex, float* outDevice,
                                          int32_t* outWidth, int32_t* outHeight) {
    if (!t || !camToWorld) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        msplat::MTensor img = T(t)->render_pose(camToWorld, refCameraIndex);
        if (outWidth) *outWidth = (int32_t)img.size(1);
        if (outHeight) *outHeight = (int32_t)img.size(0);
        if (outDevice) msplat::check(msplat_hip_memcpy_d2d(outDevice, img.data_ptr(), img.nbytes()), "copy");
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
