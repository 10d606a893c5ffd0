// model.cpp — Model: parameters, optimiser state, camera set-up, train step
// and refinement policy over the HIP backend (core/src/model.cpp).
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>
#include <fstream>

namespace msplat {

Model::Model(const ModelConfig& cfg, int numCameras_, int64_t n, const float* const params[6],
             bool paramsOnDevice)
    : cfg_(cfg), numCameras(numCameras_), stopSplitAt(cfg.iterations / 2) {
    if (n <= 0) throw std::runtime_error("Model needs at least one gaussian");
    if (cfg.shDegree < 0 || cfg.shDegree > 4) throw std::runtime_error("SH degree must be 0..4");
    num_active = n;
    setupOptimizers(params, paramsOnDevice);
}

// model.cpp:119-164: buffers of 4x the initial count, zeroed Adam moments and
// the per-group learning rates.
void Model::setupOptimizers(const float* const params[6], bool onDevice) {
    buf_capacity = num_active * 4;
    const int64_t K1 = (int64_t)(cfg_.shDegree + 1) * (cfg_.shDegree + 1) - 1;
    const std::vector<int64_t> tail[6] = {{3}, {3}, {4}, {3}, {K1, 3}, {1}};
    MTensor* bufs[6] = {&means_buf, &scales_buf, &quats_buf, &featuresDc_buf, &featuresRest_buf,
                        &opacities_buf};
    static constexpr float lr_init[N_ADAM_GROUPS] = {0.00016f, 0.005f, 0.001f,
                                                     0.0025f, 0.000125f, 0.05f};
    for (int g = 0; g < 6; ++g) {
        std::vector<int64_t> shape{buf_capacity};
        shape.insert(shape.end(), tail[g].begin(), tail[g].end());
        *bufs[g] = gpu_zeros(shape, DType::Float32);
        const size_t bytes = (size_t)num_active * bufs[g]->stride0() * sizeof(float);
        if (bytes && params[g]) {
            if (onDevice) bufs[g]->copy_from_device(params[g], bytes);
            else bufs[g]->copy_from_host(params[g], bytes);
        }
        adam_exp_avg_buf[g] = gpu_zeros(shape, DType::Float32);
        adam_exp_avg_sq_buf[g] = gpu_zeros(shape, DType::Float32);
        adam_lr[g] = lr_init[g];
    }
    allocStats();
    adam_step_count = 0;
    refreshViews();
}

void Model::allocStats() {
    for (auto& s : stats_buf) s = gpu_zeros({buf_capacity}, DType::Float32);
}

void Model::refreshViews() {
    means = means_buf.view(num_active);
    scales = scales_buf.view(num_active);
    quats = quats_buf.view(num_active);
    featuresDc = featuresDc_buf.view(num_active);
    featuresRest = featuresRest_buf.view(num_active);
    opacities = opacities_buf.view(num_active);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) {
        adam_exp_avg[g] = adam_exp_avg_buf[g].view(num_active);
        adam_exp_avg_sq[g] = adam_exp_avg_sq_buf[g].view(num_active);
    }
    visCounts = stats_buf[0].view(num_active);
    xysGradNorm = stats_buf[1].view(num_active);
    max2DSize = stats_buf[2].view(num_active);
}

// model.cpp:197-228: grow every buffer to max(needed, 2 x capacity), keeping
// the active rows.
void Model::ensureCapacity(int64_t needed) {
    if (needed <= buf_capacity) return;
    const int64_t new_cap = std::max(needed, buf_capacity * 2);
    auto grow = [&](MTensor& buf) {
        std::vector<int64_t> shape = buf.shape();
        shape[0] = new_cap;
        MTensor nb = gpu_zeros(shape, DType::Float32);
        nb.copy_from_device(buf.data_ptr(), (size_t)num_active * buf.stride0() * sizeof(float));
        buf = nb;
    };
    grow(means_buf); grow(scales_buf); grow(quats_buf);
    grow(featuresDc_buf); grow(featuresRest_buf); grow(opacities_buf);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) {
        grow(adam_exp_avg_buf[g]);
        grow(adam_exp_avg_sq_buf[g]);
    }
    for (auto& s : stats_buf) grow(s);
    buf_capacity = new_cap;
    refreshViews();
}

void Model::schedulersStep(int step) {   // model.cpp:179-182
    const float t = std::clamp((float)step / (float)cfg_.iterations, 0.f, 1.f);
    adam_lr[0] = std::exp(std::log(means_lr_init) * (1.f - t) + std::log(means_lr_final) * t);
}

int Model::getDownscaleFactor(int step) const {   // model.cpp:230-233
    const int remaining = cfg_.numDownscales - step / cfg_.resolutionSchedule;
    return 1 << std::max(remaining, 0);
}

int Model::degreesToUse(int step) const {
    if (cfg_.shDegreeInterval <= 0) return cfg_.shDegree;
    return std::min(step / cfg_.shDegreeInterval, cfg_.shDegree);
}

int Model::shDegreeStored() const { return cfg_.shDegree; }

MTensor Model::group(int g, int which) const {
    if (g < 0 || g >= N_ADAM_GROUPS || which < 0 || which > 2)
        throw std::runtime_error("group index out of range");
    if (which == 1) return adam_exp_avg[g];
    if (which == 2) return adam_exp_avg_sq[g];
    const MTensor* p[6] = {&means, &scales, &quats, &featuresDc, &featuresRest, &opacities};
    return *p[g];
}

// model.cpp:490-519, in fp32 step by step.
void prepare_camera(Camera& cam, float sf, float& fx, float& fy, float& cx, float& cy,
                    int& width, int& height) {
    fx = cam.fx / sf; fy = cam.fy / sf;
    cx = cam.cx / sf; cy = cam.cy / sf;
    height = static_cast<int>(cam.height / sf);
    width = static_cast<int>(cam.width / sf);
    const float fovX = 2.0f * std::atan(width / (2.0f * fx));
    const float fovY = 2.0f * std::atan(height / (2.0f * fy));
    if (cam.cached && cam.cachedFovX == fovX && cam.cachedFovY == fovY) return;
    const float* d = cam.camToWorld;
    float R[3][3], Rinv[3][3], T[3], Tinv[3];
    for (int i = 0; i < 3; ++i) {
        R[i][0] = d[i * 4 + 0]; R[i][1] = -d[i * 4 + 1]; R[i][2] = -d[i * 4 + 2];
        T[i] = d[i * 4 + 3];
    }
    for (int i = 0; i < 3; ++i)
        for (int j = 0; j < 3; ++j) Rinv[i][j] = R[j][i];
    for (int i = 0; i < 3; ++i) Tinv[i] = -(Rinv[i][0] * T[0] + Rinv[i][1] * T[1] + Rinv[i][2] * T[2]);
    const float vm[16] = {Rinv[0][0], Rinv[0][1], Rinv[0][2], Tinv[0],
                          Rinv[1][0], Rinv[1][1], Rinv[1][2], Tinv[1],
                          Rinv[2][0], Rinv[2][1], Rinv[2][2], Tinv[2],
                          0, 0, 0, 1};
    const float t_p = 0.001f * std::tan(0.5f * fovY), r_p = 0.001f * std::tan(0.5f * fovX);
    const float pm[16] = {0.001f / r_p, 0, 0, 0,
                          0, 0.001f / t_p, 0, 0,
                          0, 0, (1000.0f + 0.001f) / (1000.0f - 0.001f), -1000.0f * 0.001f / (1000.0f - 0.001f),
                          0, 0, 1, 0};
    float pvm[16] = {};
    for (int i = 0; i < 4; ++i)
        for (int j = 0; j < 4; ++j)
            for (int k = 0; k < 4; ++k) {
                const float prod = pm[i * 4 + k] * vm[k * 4 + j];
                pvm[i * 4 + j] = pvm[i * 4 + j] + prod;
            }
    std::memcpy(cam.cachedViewMat, vm, sizeof(vm));
    std::memcpy(cam.cachedProjViewMat, pvm, sizeof(pvm));
    for (int i = 0; i < 3; ++i) cam.cachedCamPos[i] = T[i];
    cam.cachedFovX = fovX;
    cam.cachedFovY = fovY;
    cam.cached = true;
}

// model.cpp:490-534.
Model::CamSetup Model::prepareCam(Camera& cam, int step) {
    CamSetup s;
    prepare_camera(cam, (float)getDownscaleFactor(step), s.fx, s.fy, s.cx, s.cy, s.width, s.height);
    s.degree = (unsigned)cfg_.shDegree;
    s.degreesToUse = (unsigned)degreesToUse(step);
    s.tileBounds = std::make_tuple((s.width + TILE - 1) / TILE, (s.height + TILE - 1) / TILE, 1);
    for (int i = 0; i < 3; ++i) s.cam_pos[i] = cam.cachedCamPos[i];
    return s;
}

// model.cpp:546-597.
void Model::fullIteration(Camera& cam, int step, MTensor& gt) {
    CamSetup s = prepareCam(cam, step);
    lastHeight = s.height;
    lastWidth = s.width;
    if (gt.numel() != (int64_t)s.height * s.width * 3)
        throw std::runtime_error("target image size does not match the camera");
    const int numPoints = (int)num_active;
    adam_step_count++;
    // std::pow(float, int) promotes to double (as in the reference)
    const float bc1 = 1.0f - std::pow(adam_beta1, adam_step_count);
    const float bc2 = 1.0f - std::pow(adam_beta2, adam_step_count);
    MTensor adam_p[N_ADAM_GROUPS] = {means, scales, quats, featuresDc, featuresRest, opacities};
    float ss[N_ADAM_GROUPS], bc2s[N_ADAM_GROUPS];
    for (int i = 0; i < N_ADAM_GROUPS; ++i) {
        ss[i] = adam_lr[i] / bc1;
        bc2s[i] = std::sqrt(bc2);
    }
    const float invMaxDim = 1.0f / static_cast<float>(std::max(lastHeight, lastWidth));
    const float lossInvN = 1.0f / (float)(s.height * s.width * 3);
    auto [r, loss] = msplat_train_step(
        numPoints, means, scales, 1.0f, quats, cam.cachedViewMat, cam.cachedProjViewMat, s.fx,
        s.fy, s.cx, s.cy, s.height, s.width, s.tileBounds, 0.01f, s.degree, s.degreesToUse,
        s.cam_pos, featuresDc, featuresRest, opacities, cfg_.bgColor, gt, cfg_.ssimWeight,
        lossInvN, (int)featuresRest.size(-2), N_ADAM_GROUPS, adam_p, adam_exp_avg,
        adam_exp_avg_sq, ss, bc2s, adam_beta1, adam_beta2, adam_eps, visCounts, xysGradNorm,
        max2DSize, invMaxDim);
    radii = r;
    last_loss = loss;
}

// model.cpp:236-296.
void Model::afterTrain(int step) {
    if (!radii.defined()) return;
    if (!(step % cfg_.refineEvery == 0 && step > cfg_.warmupLength)) return;
    const int resetInterval = cfg_.resetAlphaEvery * cfg_.refineEvery;
    const bool doDensification =
        step < stopSplitAt && step % resetInterval > numCameras + cfg_.refineEvery;
    if (doDensification) {
        ensureCapacity(3 * num_active);   // worst case: every gaussian splits
        const float half_max_dim = 0.5f * (float)std::max(lastWidth, lastHeight);
        const int check_screen = step < cfg_.stopScreenSizeAt ? 1 : 0;
        const bool checkHuge = step > cfg_.refineEvery * cfg_.resetAlphaEvery;
        const int fr_stride = (int)featuresRest_buf.stride0();
        const int new_count = msplat_densify(
            (int)num_active, (int)buf_capacity, cfg_.densifyGradThresh, cfg_.densifySizeThresh,
            cfg_.splitScreenSize, check_screen, cfg_.cullAlphaThresh, cfg_.cullScaleThresh,
            cfg_.cullScreenSize, checkHuge ? 1 : 0, xysGradNorm, visCounts, max2DSize,
            half_max_dim, means_buf, scales_buf, quats_buf, featuresDc_buf, featuresRest_buf,
            opacities_buf, fr_stride, adam_exp_avg_buf, adam_exp_avg_sq_buf, no_samples,
            (uint64_t)step);
        num_active = new_count;
        refreshViews();
    }
    if (step < stopSplitAt && step % resetInterval == cfg_.refineEvery) {
        constexpr float resetLogit = -1.3862943611198906f;   // logit(0.2)
        check(msplat_hip_clamp_max(opacities.data<float>(), opacities.numel(), resetLogit),
              "opacity reset");
        adam_exp_avg[5].zero();
        adam_exp_avg_sq[5].zero();
    }
    visCounts.zero();
    xysGradNorm.zero();
    max2DSize.zero();
}

MTensor Model::render(Camera& cam, int step) {   // model.cpp:536-544
    CamSetup s = prepareCam(cam, step);
    return msplat_render((int)num_active, means, scales, 1.0f, quats, cam.cachedViewMat,
                         cam.cachedProjViewMat, s.fx, s.fy, s.cx, s.cy, s.height, s.width,
                         s.tileBounds, 0.01f, s.degree, s.degreesToUse, s.cam_pos, featuresDc,
                         featuresRest, opacities, cfg_.bgColor);
}

void Model::renderTo(Camera& cam, int step, float* dst, int& width, int& height) {
    CamSetup s = prepareCam(cam, step);
    width = s.width;
    height = s.height;
    if (!dst) return;
    msplat_render_to(dst, (int)num_active, means, scales, 1.0f, quats, cam.cachedViewMat,
                     cam.cachedProjViewMat, s.fx, s.fy, s.cx, s.cy, s.height, s.width,
                     s.tileBounds, 0.01f, s.degree, s.degreesToUse, s.cam_pos, featuresDc,
                     featuresRest, opacities, cfg_.bgColor);
}

// ---- scene files and checkpoints ----

HostGaussians Model::toHost() const {
    msplat_gpu_sync();
    HostGaussians g;
    g.n = num_active;
    g.rest_bases = (int)(featuresRest.stride0() / 3);
    auto get = [](const MTensor& t, std::vector<float>& dst) {
        dst.resize((size_t)t.numel());
        t.copy_to_host(dst.data(), dst.size() * sizeof(float));
    };
    get(means, g.means);
    get(scales, g.scales);
    get(quats, g.quats);
    get(featuresDc, g.f_dc);
    get(featuresRest, g.f_rest);
    get(opacities, g.opacities);
    return g;
}

void Model::save(const std::string& filename, int step) {   // model.cpp:298-305
    const size_t dot = filename.rfind('.');
    if (dot != std::string::npos && filename.substr(dot) == ".splat") saveSplat(filename);
    else savePly(filename, step);
}

void Model::savePly(const std::string& filename, int step) {
    save_gaussian_ply(filename, toHost(), crs, step);
}

void Model::saveSplat(const std::string& filename) { save_gaussian_splat(filename, toHost(), crs); }

int Model::loadPly(const std::string& filename) {   // model.cpp:319-330
    int step = 0;
    HostGaussians g = load_gaussian_ply(filename, crs, &step);
    const int K1 = (cfg_.shDegree + 1) * (cfg_.shDegree + 1) - 1;
    if (g.rest_bases != K1)
        throw std::runtime_error("PLY has " + std::to_string(g.rest_bases) +
                                 " higher-order SH bases, the model's degree needs " +
                                 std::to_string(K1));
    num_active = g.n;
    const float* params[6] = {g.means.data(), g.scales.data(), g.quats.data(),
                              g.f_dc.data(), g.f_rest.data(), g.opacities.data()};
    setupOptimizers(params, false);
    return step;
}

namespace {

constexpr uint32_t CKPT_MAGIC = 0x4C50534D;   // "MSPL"
constexpr uint32_t CKPT_VERSION = 1;

template <typename T>
void put(std::ofstream& f, const T& v) { f.write(reinterpret_cast<const char*>(&v), sizeof(T)); }
template <typename T>
T take(std::ifstream& f) {
    T v{};
    f.read(reinterpret_cast<char*>(&v), sizeof(T));
    if (!f) throw std::runtime_error("checkpoint is truncated");
    return v;
}

// writeTensor (model.cpp:336-346): ndim, int64 shape, byte count, data.
void write_tensor(std::ofstream& f, const MTensor& t) {
    put<uint32_t>(f, (uint32_t)t.dim());
    for (int64_t d = 0; d < t.dim(); ++d) put<int64_t>(f, t.size((int)d));
    const uint64_t bytes = t.nbytes();
    put<uint64_t>(f, bytes);
    std::vector<char> host(bytes);
    t.copy_to_host(host.data(), bytes);
    f.write(host.data(), (std::streamsize)bytes);
}

struct HostTensor {
    std::vector<int64_t> shape;
    std::vector<float> data;
};

HostTensor read_tensor(std::ifstream& f) {   // readTensor (model.cpp:348-359)
    HostTensor t;
    const uint32_t ndim = take<uint32_t>(f);
    if (ndim == 0 || ndim > 8) throw std::runtime_error("checkpoint tensor has a bad rank");
    int64_t numel = 1;
    for (uint32_t i = 0; i < ndim; ++i) {
        t.shape.push_back(take<int64_t>(f));
        if (t.shape.back() < 0) throw std::runtime_error("checkpoint tensor has a bad shape");
        numel *= t.shape.back();
    }
    const uint64_t bytes = take<uint64_t>(f);
    if (bytes != (uint64_t)numel * 4) throw std::runtime_error("checkpoint tensor size mismatch");
    t.data.resize((size_t)numel);
    f.read(reinterpret_cast<char*>(t.data.data()), (std::streamsize)bytes);
    if (!f) throw std::runtime_error("checkpoint is truncated");
    return t;
}

}  // namespace

void Model::saveCheckpoint(const std::string& filename, int step) {   // model.cpp:361-399
    msplat_gpu_sync();
    std::ofstream f(filename, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open checkpoint file for writing: " + filename);
    put(f, CKPT_MAGIC);
    put(f, CKPT_VERSION);
    put<uint32_t>(f, (uint32_t)step);
    put<uint32_t>(f, (uint32_t)num_active);
    put<uint32_t>(f, (uint32_t)cfg_.shDegree);
    put<uint32_t>(f, (uint32_t)adam_step_count);
    f.write(reinterpret_cast<const char*>(adam_lr), sizeof(adam_lr));
    put(f, means_lr_init);
    put(f, means_lr_final);
    const MTensor* p[6] = {&means, &scales, &quats, &featuresDc, &featuresRest, &opacities};
    for (const MTensor* t : p) write_tensor(f, *t);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) write_tensor(f, adam_exp_avg[g]);
    for (int g = 0; g < N_ADAM_GROUPS; ++g) write_tensor(f, adam_exp_avg_sq[g]);
    if (!f) throw std::runtime_error("write failed: " + filename);
}

int Model::loadCheckpoint(const std::string& filename) {   // model.cpp:401-488
    std::ifstream f(filename, std::ios::binary);
    if (!f.is_open()) throw std::runtime_error("Cannot open checkpoint file: " + filename);
    if (take<uint32_t>(f) != CKPT_MAGIC) throw std::runtime_error("Not a valid msplat checkpoint file");
    const uint32_t version = take<uint32_t>(f);
    if (version != CKPT_VERSION)
        throw std::runtime_error("Unsupported checkpoint version: " + std::to_string(version));
    const uint32_t step = take<uint32_t>(f);
    const uint32_t n = take<uint32_t>(f);
    const uint32_t deg = take<uint32_t>(f);
    const uint32_t adam_steps = take<uint32_t>(f);
    float lr[N_ADAM_GROUPS];
    for (float& v : lr) v = take<float>(f);
    const float lr_init = take<float>(f), lr_final = take<float>(f);
    if ((int)deg != cfg_.shDegree)
        throw std::runtime_error("checkpoint SH degree " + std::to_string(deg) +
                                 " differs from the model's " + std::to_string(cfg_.shDegree));
    if (n == 0) throw std::runtime_error("checkpoint holds no gaussians");
    HostTensor t[3 * N_ADAM_GROUPS];
    for (auto& x : t) x = read_tensor(f);
    const int64_t K1 = (int64_t)(cfg_.shDegree + 1) * (cfg_.shDegree + 1) - 1;
    const std::vector<int64_t> tail[6] = {{3}, {3}, {4}, {3}, {K1, 3}, {1}};
    for (int k = 0; k < 3 * N_ADAM_GROUPS; ++k) {
        std::vector<int64_t> want{(int64_t)n};
        want.insert(want.end(), tail[k % 6].begin(), tail[k % 6].end());
        if (t[k].shape != want) throw std::runtime_error("checkpoint tensor has an unexpected shape");
    }
    // Fresh backing buffers of 4x the count holding the loaded rows.
    num_active = n;
    buf_capacity = 4 * (int64_t)n;
    MTensor* bufs[6] = {&means_buf, &scales_buf, &quats_buf, &featuresDc_buf, &featuresRest_buf,
                        &opacities_buf};
    for (int g = 0; g < 6; ++g) {
        std::vector<int64_t> shape{buf_capacity};
        shape.insert(shape.end(), tail[g].begin(), tail[g].end());
        MTensor* dst[3] = {bufs[g], &adam_exp_avg_buf[g], &adam_exp_avg_sq_buf[g]};
        const HostTensor* src[3] = {&t[g], &t[6 + g], &t[12 + g]};
        for (int k = 0; k < 3; ++k) {
            *dst[k] = gpu_zeros(shape, DType::Float32);
            dst[k]->copy_from_host(src[k]->data.data(), src[k]->data.size() * sizeof(float));
        }
    }
    allocStats();
    std::memcpy(adam_lr, lr, sizeof(adam_lr));
    means_lr_init = lr_init;
    means_lr_final = lr_final;
    adam_step_count = (int)adam_steps;
    refreshViews();
    return (int)step;
}

}  // namespace msplat
