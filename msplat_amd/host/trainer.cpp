// trainer.cpp — GaussianTrainer (python/bindings.cpp:101-280; Trainer,
// msplat_api.mm:54-278), the reference's C API of include/msplat_c_api.h
// (msplat_api.mm:280-390) and the additions of include/msplat_trainer.h.
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
#include "jpeg_decode.hpp"
#include "png_decode.hpp"

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
        std::vector<Camera> cs(n);
        std::vector<MTensor> gts(n);
        for (int i = 0; i < n; ++i) {
            Camera& cam = cs[i];
            cam.width = cams[i].width; cam.height = cams[i].height;
            cam.fx = cams[i].fx; cam.fy = cams[i].fy; cam.cx = cams[i].cx; cam.cy = cams[i].cy;
            std::memcpy(cam.camToWorld, cams[i].camToWorld, sizeof(cam.camToWorld));
            if (!images[i]) throw std::runtime_error("missing test image");
            gts[i] = gpu_empty({cam.height, cam.width, 3}, DType::Float32);
            if (on_device) gts[i].copy_from_device(images[i], gts[i].nbytes());
            else gts[i].copy_from_host(images[i], gts[i].nbytes());
        }
        return evaluate_cameras(cs, gts);
    }

    // The held-out cameras of the dataset the trainer was built from.
    void set_test(std::vector<Camera> cams, std::vector<MTensor> images) {
        test_cameras = std::move(cams);
        test_images = std::move(images);
    }

    // Trainer::evaluate over the held-out cameras; all zero without any.
    MsplatEvalMetrics evaluate_test() {
        if (test_cameras.empty()) return MsplatEvalMetrics{0.f, 0.f, 0.f, 0, 0};
        return evaluate_cameras(test_cameras, test_images);
    }

    MsplatEvalMetrics evaluate_cameras(std::vector<Camera> cams, const std::vector<MTensor>& images) {
        const int n = (int)cams.size();
        const int ds = model->getDownscaleFactor(cfg.iterations);
        double sp = 0.0, ss = 0.0, sl = 0.0;
        for (int i = 0; i < n; ++i) {
            Camera& cam = cams[i];
            MTensor gt = images[i];
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

    // Trainer::render (msplat_api.mm:168-186): a training or held-out camera
    // at the current step's resolution; an empty tensor when out of range.
    MTensor render_camera(int i, bool use_test) {
        std::vector<Camera>& cs = use_test ? test_cameras : cameras;
        if (i < 0 || i >= (int)cs.size()) return MTensor();
        return model->render(cs[i], current_step);
    }

    int num_cameras() const { return (int)cameras.size(); }

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
    std::vector<Camera> test_cameras;
    std::vector<MTensor> test_images;
    std::vector<std::map<int, MTensor>> gpu_images;
    std::vector<size_t> cam_indices;
    size_t cam_iter_pos = 0;
    std::mt19937 rng;
};

}  // namespace msplat

using msplat::GaussianTrainer;

namespace {

// Clears the last error, runs f and turns an exception into on_error with
// its message kept for msplat_trainer_last_error.
template <typename F>
auto guarded(F&& f, decltype(f()) on_error) -> decltype(f()) {
    msplat::g_err.clear();
    try {
        return f();
    } catch (const std::exception& e) {
        msplat::g_err = e.what();
        return on_error;
    }
}

// Runs f for a call without a result (the reference's void functions).
template <typename F>
void guarded_void(F&& f) {
    msplat::g_err.clear();
    try {
        f();
    } catch (const std::exception& e) {
        msplat::g_err = e.what();
    }
}

GaussianTrainer* T(MsplatTrainer t) { return static_cast<GaussianTrainer*>(t); }

MsplatPixelBuffer to_host(const msplat::MTensor& img) {
    MsplatPixelBuffer b{nullptr, 0, 0};
    if (img.dim() == 0) return b;
    b.height = (int)img.size(0);
    b.width = (int)img.size(1);
    b.data = static_cast<float*>(std::malloc(img.nbytes()));
    if (!b.data) throw std::runtime_error("out of host memory");
    img.copy_to_host(b.data, img.nbytes());
    return b;
}

// A dataset handle: the COLMAP reconstruction and, when built by
// msplat_dataset_create, each camera's prepared image on the GPU and the
// train / test split (Dataset::Impl, msplat_api.mm:20-46).
struct CDataset {
    msplat::Dataset data;
    bool with_images = false;
    std::vector<msplat::Camera> train_cams, test_cams;
    std::vector<msplat::MTensor> train_imgs, test_imgs;
};

CDataset* D(MsplatDataset ds) { return static_cast<CDataset*>(ds); }

MsplatImageDecoder g_decoder = nullptr;

// The device context, created on first use on GPU 0 (as the reference
// creates its Metal context on first use).
void ensure_device() {
    if (msplat_hip_init(0) == MSPLAT_OK) return;
    if (std::strstr(msplat_hip_last_error(), "already initialised")) return;   // on another GPU
    throw std::runtime_error(std::string("device initialisation failed: ") + msplat_hip_last_error());
}

// imreadRGB (image_io.cpp:12-50): a registered decoder, else the library's
// PNG or JPEG decoder by the file's signature.
msplat::DecodedImage read_image(const std::string& path) {
    if (g_decoder) {
        float* rgb = nullptr;
        int w = 0, h = 0;
        if (g_decoder(path.c_str(), &rgb, &w, &h) != 0 || !rgb || w <= 0 || h <= 0) {
            std::free(rgb);
            throw std::runtime_error("the registered image decoder failed on " + path);
        }
        msplat::DecodedImage img;
        img.width = w;
        img.height = h;
        img.rgb.assign(rgb, rgb + (size_t)w * h * 3);
        std::free(rgb);
        return img;
    }
    if (msplat::is_png_file(path)) return msplat::decode_png(path);
    if (msplat::is_jpeg_file(path)) return msplat::decode_jpeg(path);
    throw std::runtime_error(path + ": neither PNG nor JPEG; register a decoder for this format "
                                    "with msplat_set_image_decoder");
}

// Camera::loadImage (input_data.cpp:17-52) on the GPU: intrinsics rescaled
// when the file's size differs from the camera's, the optional load-time
// downscale by an area resize, then the undistortion of a distorted camera
// (crop to the valid rectangle); fp32 intrinsics arithmetic as there.
msplat::MTensor load_camera_image(const msplat::DatasetCamera& dc, float downscale, msplat::Camera& cam) {
    using msplat::MTensor;
    const msplat::DecodedImage raw = read_image(dc.filePath);
    MTensor img = msplat::gpu_empty({raw.height, raw.width, 3}, msplat::DType::Float32);
    img.copy_from_host(raw.rgb.data(), img.nbytes());
    float fx = dc.fx, fy = dc.fy, cx = dc.cx, cy = dc.cy;
    int width = dc.width, height = dc.height;
    if (width > 0 && height > 0 && (raw.width != width || raw.height != height)) {
        const float sx = (float)raw.width / (float)width, sy = (float)raw.height / (float)height;
        fx *= sx; fy *= sy; cx *= sx; cy *= sy;
        width = raw.width;
        height = raw.height;
    } else if (width == 0 || height == 0) {
        width = raw.width;
        height = raw.height;
    }
    if (downscale > 1.0f) {
        const int nw = (int)(width / downscale), nh = (int)(height / downscale);
        if (nw <= 0 || nh <= 0) throw std::runtime_error("downscale factor too large for " + dc.filePath);
        MTensor small = msplat::gpu_empty({nh, nw, 3}, msplat::DType::Float32);
        msplat::check(msplat_hip_resize_area(img.data<float>(), width, height, small.data<float>(), nw, nh),
                      "resize");
        img = small;
        const float sc = 1.0f / downscale;
        fx *= sc; fy *= sc; cx *= sc; cy *= sc;
        width = nw;
        height = nh;
    }
    if (dc.k1 != 0.f || dc.k2 != 0.f || dc.p1 != 0.f || dc.p2 != 0.f) {
        const float intr[4] = {fx, fy, cx, cy};
        const float dist[5] = {dc.k1, dc.k2, dc.p1, dc.p2, 0.f};
        int32_t roi[4];
        msplat::check(msplat_undistort_roi(width, height, intr, dist, roi), "undistortion rectangle");
        MTensor out = msplat::gpu_empty({roi[3], roi[2], 3}, msplat::DType::Float32);
        msplat::check(msplat_hip_undistort(img.data<float>(), width, height, intr, dist, roi,
                                           out.data<float>()),
                      "undistort");
        img = out;
        cx -= (float)roi[0];
        cy -= (float)roi[1];
        width = roi[2];
        height = roi[3];
    }
    cam.width = width;
    cam.height = height;
    cam.fx = fx; cam.fy = fy; cam.cx = cx; cam.cy = cy;
    std::memcpy(cam.camToWorld, dc.camToWorld, sizeof(cam.camToWorld));
    cam.cached = false;
    return img;
}

MsplatTrainerCamera c_camera(const msplat::Camera& k) {
    MsplatTrainerCamera c;
    c.width = k.width; c.height = k.height;
    c.fx = k.fx; c.fy = k.fy; c.cx = k.cx; c.cy = k.cy;
    std::memcpy(c.camToWorld, k.camToWorld, sizeof(c.camToWorld));
    return c;
}

const msplat::DatasetCamera& dcam(MsplatDataset ds, int32_t i) {
    if (!ds || i < 0 || i >= (int32_t)D(ds)->data.cameras.size())
        throw std::runtime_error("camera index out of range");
    return D(ds)->data.cameras[i];
}

}  // namespace

extern "C" {

MsplatTrainer msplat_trainer_create_from_arrays(const MsplatTrainerConfig* config, int64_t n,
                                                const float* const params[6], int32_t n_cameras,
                                                const MsplatTrainerCamera* cameras,
                                                const float* const* targets, int32_t on_device) {
    return guarded([&]() -> MsplatTrainer {
        if (!config || !params || !cameras || !targets) throw std::runtime_error("null argument");
        return new GaussianTrainer(*config, n, params, n_cameras, cameras, targets, on_device != 0);
    }, nullptr);
}

// msplat_trainer_create (msplat_c_api.h:94; msplat_api.mm:322-327 and
// Trainer::Trainer, msplat_api.mm:76-98): gaussians from the point cloud, the
// training cameras and their images, the held-out ones kept for evaluation.
MsplatTrainer msplat_trainer_create(MsplatDataset ds, MsplatConfig config) {
    return guarded([&]() -> MsplatTrainer {
        if (!ds) throw std::runtime_error("null dataset");
        CDataset* d = D(ds);
        if (!d->with_images)
            throw std::runtime_error("the dataset has no images (open it with msplat_dataset_create)");
        if (d->train_cams.empty()) throw std::runtime_error("the dataset has no training cameras");
        ensure_device();
        MsplatTrainerConfig c = msplat_trainer_default_config();
        c.iterations = config.iterations;
        c.shDegree = config.shDegree;
        c.shDegreeInterval = config.shDegreeInterval;
        c.ssimWeight = config.ssimWeight;
        c.numDownscales = config.numDownscales;
        c.resolutionSchedule = config.resolutionSchedule;
        c.refineEvery = config.refineEvery;
        c.warmupLength = config.warmupLength;
        c.resetAlphaEvery = config.resetAlphaEvery;
        c.densifyGradThresh = config.densifyGradThresh;
        c.densifySizeThresh = config.densifySizeThresh;
        c.stopScreenSizeAt = config.stopScreenSizeAt;
        c.splitScreenSize = config.splitScreenSize;
        for (int k = 0; k < 3; ++k) c.bgColor[k] = config.bgColor[k];
        // The initial gaussians go to the device first: the trainer takes
        // parameters and images from the same memory space, and the images
        // are already on the device.
        msplat::HostGaussians g = msplat::init_gaussians(d->data.xyz, d->data.rgb, config.shDegree);
        const std::vector<float>* host[6] = {&g.means, &g.scales, &g.quats,
                                             &g.f_dc, &g.f_rest, &g.opacities};
        msplat::MTensor dev[6];
        const float* params[6];
        for (int k = 0; k < 6; ++k) {
            dev[k] = msplat::gpu_empty({(int64_t)std::max<size_t>(host[k]->size(), 1)},
                                       msplat::DType::Float32);
            if (!host[k]->empty()) dev[k].copy_from_host(host[k]->data(), host[k]->size() * sizeof(float));
            params[k] = dev[k].data<float>();
        }
        std::vector<MsplatTrainerCamera> cams;
        std::vector<const float*> imgs;
        for (size_t i = 0; i < d->train_cams.size(); ++i) {
            cams.push_back(c_camera(d->train_cams[i]));
            imgs.push_back(d->train_imgs[i].data<float>());
        }
        std::unique_ptr<GaussianTrainer> tr(new GaussianTrainer(
            c, g.n, params, (int)cams.size(), cams.data(), imgs.data(), true));
        tr->set_test(d->test_cams, d->test_imgs);
        msplat::Crs& crs = tr->model->crs;
        crs.scale = d->data.scale;
        for (int k = 0; k < 3; ++k) crs.translation[k] = d->data.translation[k];
        crs.keep = config.keepCrs;
        return tr.release();
    }, nullptr);
}

void msplat_trainer_destroy(MsplatTrainer t) { delete T(t); }

const char* msplat_trainer_last_error(void) { return msplat::g_err.c_str(); }

MsplatStats msplat_trainer_step(MsplatTrainer t) {
    MsplatStats bad{-1, -1, 0.f};
    if (!t) return bad;
    return guarded([&]() { return T(t)->step(); }, bad);
}

// Trainer::train (msplat_api.mm:130-136).
void msplat_trainer_train(MsplatTrainer t) {
    if (!t) return;
    guarded_void([&]() {
        while (T(t)->current_step < T(t)->cfg.iterations) T(t)->step();
    });
}

float msplat_trainer_last_loss(MsplatTrainer t, int32_t wait) {
    if (!t) return NAN;
    float v = NAN;
    if (msplat_hip_last_loss(&v, wait) != MSPLAT_OK) return NAN;
    return v;
}

MsplatPixelBuffer msplat_trainer_render(MsplatTrainer t, int cameraIndex, bool useTest) {
    MsplatPixelBuffer empty{nullptr, 0, 0};
    if (!t) return empty;
    return guarded([&]() { return to_host(T(t)->render_camera(cameraIndex, useTest)); }, empty);
}

MsplatPixelBuffer msplat_trainer_render_pose(MsplatTrainer t, const float camToWorld[16],
                                             int refCameraIndex) {
    MsplatPixelBuffer empty{nullptr, 0, 0};
    if (!t || !camToWorld) return empty;
    if (refCameraIndex < 0 || refCameraIndex >= T(t)->num_cameras()) return empty;
    return guarded([&]() { return to_host(T(t)->render_pose(camToWorld, refCameraIndex)); }, empty);
}

// Trainer::renderFromPoseToBuffer (msplat_api.mm:207-238): the RGBA8
// conversion runs on the GPU and 4 bytes per pixel are copied.
void msplat_trainer_render_pose_to_buffer(MsplatTrainer t, const float camToWorld[16],
                                          int refCameraIndex, uint8_t* outRGBA, int* outWidth,
                                          int* outHeight) {
    if (!t || !camToWorld || refCameraIndex < 0 || refCameraIndex >= T(t)->num_cameras()) {
        if (outWidth) *outWidth = 0;
        if (outHeight) *outHeight = 0;
        return;
    }
    guarded_void([&]() {
        msplat::MTensor img = T(t)->render_pose(camToWorld, refCameraIndex);
        const int h = (int)img.size(0), w = (int)img.size(1);
        if (outWidth) *outWidth = w;
        if (outHeight) *outHeight = h;
        if (!outRGBA) return;
        const int64_t n = (int64_t)w * h;
        msplat::MTensor rgba = msplat::gpu_empty({n}, msplat::DType::Int32);   // 4 bytes per pixel
        msplat::check(msplat_hip_image_to_rgba8(img.data<float>(), n, rgba.data<uint8_t>()), "rgba8");
        rgba.copy_to_host(outRGBA, (size_t)n * 4);
    });
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

MsplatEvalMetrics msplat_trainer_evaluate_images(MsplatTrainer t, int32_t n_test,
                                                 const MsplatTrainerCamera* cameras,
                                                 const float* const* images, int32_t on_device) {
    MsplatEvalMetrics bad{0.f, 0.f, 0.f, 0, 0};
    if (!t) return bad;
    return guarded([&]() { return T(t)->evaluate(n_test, cameras, images, on_device != 0); }, bad);
}

MsplatEvalMetrics msplat_trainer_evaluate(MsplatTrainer t) {
    MsplatEvalMetrics bad{0.f, 0.f, 0.f, 0, 0};
    if (!t) return bad;
    return guarded([&]() { return T(t)->evaluate_test(); }, bad);
}

void msplat_trainer_export_ply(MsplatTrainer t, const char* path) {
    if (!t || !path) return;
    guarded_void([&]() { T(t)->model->savePly(path, T(t)->current_step); });
}

void msplat_trainer_export_splat(MsplatTrainer t, const char* path) {
    if (!t || !path) return;
    guarded_void([&]() { T(t)->model->saveSplat(path); });
}

void msplat_trainer_save_checkpoint(MsplatTrainer t, const char* path) {
    if (!t || !path) return;
    guarded_void([&]() { T(t)->model->saveCheckpoint(path, T(t)->current_step); });
}

int msplat_trainer_load_checkpoint(MsplatTrainer t, const char* path) {
    if (!t || !path) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int { return T(t)->load_checkpoint(path); }, (int)MSPLAT_ERR_ARG);
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

MsplatDataset msplat_dataset_open_colmap(const char* path, const char* image_dir) {
    if (!path) return nullptr;
    return guarded([&]() -> MsplatDataset {
        std::unique_ptr<CDataset> d(new CDataset);
        d->data = msplat::load_colmap(path, image_dir ? image_dir : "");
        for (const msplat::DatasetCamera& dc : d->data.cameras) {
            msplat::Camera k;
            k.width = dc.width; k.height = dc.height;
            k.fx = dc.fx; k.fy = dc.fy; k.cx = dc.cx; k.cy = dc.cy;
            std::memcpy(k.camToWorld, dc.camToWorld, sizeof(k.camToWorld));
            d->train_cams.push_back(k);
        }
        return d.release();
    }, nullptr);
}

// msplat_dataset_create (msplat_c_api.h:84-85; Dataset::Dataset,
// msplat_api.mm:27-46): the COLMAP reconstruction, every camera's image
// prepared on the GPU, then the split (InputData::splitTrainTest,
// input_data.cpp:152-161: cameras 0, testEvery, 2 testEvery, ... are held out).
MsplatDataset msplat_dataset_create(const char* path, float downscaleFactor, bool evalMode,
                                    int testEvery) {
    if (!path) return nullptr;
    return guarded([&]() -> MsplatDataset {
        if (evalMode && testEvery <= 0) throw std::runtime_error("testEvery must be positive");
        std::unique_ptr<CDataset> d(new CDataset);
        d->data = msplat::load_colmap(path, "");
        ensure_device();
        d->with_images = true;
        for (size_t i = 0; i < d->data.cameras.size(); ++i) {
            msplat::Camera k;
            msplat::MTensor img = load_camera_image(d->data.cameras[i], downscaleFactor, k);
            const bool test = evalMode && (int)(i % (size_t)testEvery) == 0;
            (test ? d->test_cams : d->train_cams).push_back(k);
            (test ? d->test_imgs : d->train_imgs).push_back(img);
        }
        return d.release();
    }, nullptr);
}

void msplat_dataset_destroy(MsplatDataset ds) { delete D(ds); }

int msplat_dataset_num_train(MsplatDataset ds) { return ds ? (int)D(ds)->train_cams.size() : -1; }

int msplat_dataset_num_test(MsplatDataset ds) { return ds ? (int)D(ds)->test_cams.size() : -1; }

// Dataset::cameraPose (msplat_api.mm:50-53): training camera cameraIndex.
void msplat_dataset_camera_pose(MsplatDataset ds, int cameraIndex, float camToWorld[16]) {
    if (!ds || !camToWorld || cameraIndex < 0 || cameraIndex >= (int)D(ds)->train_cams.size()) return;
    std::memcpy(camToWorld, D(ds)->train_cams[cameraIndex].camToWorld, 16 * sizeof(float));
}

int32_t msplat_dataset_num_cameras(MsplatDataset ds) {
    return ds ? (int32_t)D(ds)->data.cameras.size() : -1;
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

int64_t msplat_dataset_num_points(MsplatDataset ds) {
    return ds ? (int64_t)(D(ds)->data.xyz.size() / 3) : -1;
}

int32_t msplat_dataset_points(MsplatDataset ds, float* xyz, uint8_t* rgb) {
    if (!ds) return MSPLAT_ERR_ARG;
    if (xyz) std::memcpy(xyz, D(ds)->data.xyz.data(), D(ds)->data.xyz.size() * sizeof(float));
    if (rgb) std::memcpy(rgb, D(ds)->data.rgb.data(), D(ds)->data.rgb.size());
    return MSPLAT_OK;
}

int32_t msplat_dataset_normalisation(MsplatDataset ds, float* scale, float translation[3]) {
    if (!ds) return MSPLAT_ERR_ARG;
    if (scale) *scale = D(ds)->data.scale;
    if (translation)
        for (int k = 0; k < 3; ++k) translation[k] = D(ds)->data.translation[k];
    return MSPLAT_OK;
}

int32_t msplat_dataset_init_gaussians(MsplatDataset ds, int32_t sh_degree, float* const params[6]) {
    if (!ds || !params) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        msplat::HostGaussians g = msplat::init_gaussians(D(ds)->data.xyz, D(ds)->data.rgb, sh_degree);
        const std::vector<float>* src[6] = {&g.means, &g.scales, &g.quats,
                                            &g.f_dc, &g.f_rest, &g.opacities};
        for (int k = 0; k < 6; ++k) {
            if (!params[k]) throw std::runtime_error("null parameter buffer");
            std::memcpy(params[k], src[k]->data(), src[k]->size() * sizeof(float));
        }
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

int msplat_trainer_splat_count(MsplatTrainer t) { return t ? (int)T(t)->model->numActive() : -1; }

int msplat_trainer_iteration(MsplatTrainer t) { return t ? T(t)->current_step : -1; }

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

void msplat_set_image_decoder(MsplatImageDecoder decoder) { g_decoder = decoder; }

int32_t msplat_image_read(const char* path, float** rgb, int32_t* width, int32_t* height) {
    if (!path || !rgb || !width || !height) return MSPLAT_ERR_ARG;
    return guarded([&]() -> int32_t {
        const msplat::DecodedImage img = read_image(path);
        float* out = static_cast<float*>(std::malloc(img.rgb.size() * sizeof(float)));
        if (!out) throw std::runtime_error("out of host memory");
        std::memcpy(out, img.rgb.data(), img.rgb.size() * sizeof(float));
        *rgb = out;
        *width = img.width;
        *height = img.height;
        return MSPLAT_OK;
    }, (int32_t)MSPLAT_ERR_ARG);
}

// Lifecycle (msplat_c_api.h:119-121; msplat_api.mm:275-278, 388-389).
void msplat_set_metallib_path(const char* path) { (void)path; }

void msplat_sync(void) { (void)msplat_hip_sync(); }

void msplat_cleanup(void) { (void)msplat_hip_shutdown(); }

}  // extern "C"
