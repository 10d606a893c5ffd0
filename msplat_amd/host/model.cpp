// model.cpp — Model: parameters, optimiser state, camera set-up, train step
// and refinement policy over the HIP backend (core/src/model.cpp).
#include "model.hpp"

#include <algorithm>
#include <cmath>
#include <cstdio>
#include <cstring>

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
    for (auto& s : stats_buf) s = gpu_zeros({buf_capacity}, DType::Float32);
    adam_step_count = 0;
    refreshViews();
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

}  // namespace msplat
