// model.hpp — the gaussian model and its training step on the host side.
//
// Mirrors the reference's Model (core/include/model.hpp:12-100,
// core/src/model.cpp): six parameter views over 4x-capacity buffers, Adam
// moments per group, the LR table and means schedule, prepareCam,
// fullIteration, afterTrain (densify / opacity reset policy) and render, all
// calling the backend through bindings.hpp.  Initialisation from a dataset
// (KNN scales, point clouds), checkpoints and export are not part of this
// layer: a model is built from given parameter arrays.
#pragma once

#include <cstdint>
#include <tuple>
#include <vector>

#include "bindings.hpp"
#include "gaussian_io.hpp"

namespace msplat {

constexpr int N_ADAM_GROUPS = 6;
constexpr int TILE = 16;

// Camera (core/include/input_data.hpp:20-38): intrinsics, an OpenGL
// camera-to-world pose (row-major 4x4) and the matrices prepareCam caches.
struct Camera {
    int width = 0, height = 0;
    float fx = 0, fy = 0, cx = 0, cy = 0;
    float camToWorld[16] = {1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1, 0, 0, 0, 0, 1};
    // prepareCam cache (model.cpp:499-519)
    bool cached = false;
    float cachedViewMat[16] = {};
    float cachedProjViewMat[16] = {};
    float cachedCamPos[3] = {};
    float cachedFovX = 0, cachedFovY = 0;
};

// Training options (python/bindings.cpp:25-46 TrainingConfig), plus the cull
// thresholds that model.cpp:263 hard-codes as 0.1 / 0.5 / 0.15.
struct ModelConfig {
    int iterations = 30000;
    int shDegree = 3;
    int shDegreeInterval = 1000;   // <= 0: all bands from the first step
    float ssimWeight = 0.2f;
    int numDownscales = 2;
    int resolutionSchedule = 3000;
    int refineEvery = 100;
    int warmupLength = 500;
    int resetAlphaEvery = 30;
    float densifyGradThresh = 0.0002f;
    float densifySizeThresh = 0.01f;
    int stopScreenSizeAt = 4000;
    float splitScreenSize = 0.05f;
    float cullAlphaThresh = 0.1f;
    float cullScaleThresh = 0.5f;
    float cullScreenSize = 0.15f;
    float bgColor[3] = {0.6130f, 0.0101f, 0.3984f};
};

// prepareCam's camera part (model.cpp:490-519) at downscale factor sf: fills
// the camera's cached view / projection matrices and position, returns the
// scaled intrinsics and size in fx, fy, cx, cy, width, height.
void prepare_camera(Camera& cam, float sf, float& fx, float& fy, float& cx, float& cy,
                    int& width, int& height);

class Model {
public:
    // Model::CamSetup (model.hpp:33-38).
    struct CamSetup {
        float fx, fy, cx, cy;
        int height, width;
        unsigned degree, degreesToUse;
        std::tuple<int, int, int> tileBounds;
        float cam_pos[3];
    };

    // params: means[N,3], scales[N,3] (log), quats[N,4] (w,x,y,z), f_dc[N,3],
    // f_rest[N,K-1,3], opacities[N] (logits) as device or host pointers.
    Model(const ModelConfig& cfg, int numCameras, int64_t n, const float* const params[6],
          bool paramsOnDevice);

    CamSetup prepareCam(Camera& cam, int step);
    void fullIteration(Camera& cam, int step, MTensor& gt);
    void schedulersStep(int step);
    void afterTrain(int step);
    MTensor render(Camera& cam, int step);
    // render into a caller's device buffer; returns the image size
    void renderTo(Camera& cam, int step, float* dst, int& width, int& height);

    int getDownscaleFactor(int step) const;
    int degreesToUse(int step) const;
    int shDegreeStored() const;
    int64_t numActive() const { return num_active; }
    // Active rows of parameter group g (which = 0), or of its first / second
    // Adam moment (which = 1 / 2).
    MTensor group(int g, int which) const;
    int bufCapacity() const { return buf_capacity; }
    float lastLoss() const { return last_loss; }

    // Scene files (model.cpp:298-330): PLY or .splat by extension, and a
    // PLY import that replaces the gaussians and restarts the optimiser;
    // loadPly returns the iteration recorded in the file (0 if none).
    void save(const std::string& filename, int step);
    void savePly(const std::string& filename, int step);
    void saveSplat(const std::string& filename);
    int loadPly(const std::string& filename);
    // Checkpoint (model.cpp:333-488), the reference's byte format: "MSPL"
    // magic, version 1, step, gaussian count, SH degree, Adam step count,
    // learning rates, then the six parameter tensors and the twelve Adam
    // moment tensors (ndim, shape, byte count, data).  loadCheckpoint
    // returns the saved step.
    void saveCheckpoint(const std::string& filename, int step);
    int loadCheckpoint(const std::string& filename);
    // Active gaussians copied to host memory.
    HostGaussians toHost() const;
    // Dataset normalisation applied by the scene files when crs.keep is set
    // (identity by default: a model built from given arrays).
    Crs crs;

    // parameter / moment views of the active rows
    MTensor means, scales, quats, featuresDc, featuresRest, opacities;
    MTensor adam_exp_avg[N_ADAM_GROUPS], adam_exp_avg_sq[N_ADAM_GROUPS];
    MTensor xysGradNorm, visCounts, max2DSize;
    MTensor radii;
    float adam_lr[N_ADAM_GROUPS];
    int adam_step_count = 0;

private:
    void setupOptimizers(const float* const params[6], bool onDevice);
    void allocStats();
    void refreshViews();
    void ensureCapacity(int64_t needed);

    ModelConfig cfg_;
    int numCameras;
    int stopSplitAt;
    int64_t num_active = 0;
    int64_t buf_capacity = 0;
    int lastHeight = 0, lastWidth = 0;
    float last_loss = 0.f;
    float adam_beta1 = 0.9f, adam_beta2 = 0.999f, adam_eps = 1e-8f;
    float means_lr_init = 0.00016f, means_lr_final = 0.0000016f;
    MTensor means_buf, scales_buf, quats_buf, featuresDc_buf, featuresRest_buf, opacities_buf;
    MTensor adam_exp_avg_buf[N_ADAM_GROUPS], adam_exp_avg_sq_buf[N_ADAM_GROUPS];
    MTensor stats_buf[3];   // visCounts, xysGradNorm, max2DSize backing buffers
    MTensor no_samples;     // densify draws its normals on the GPU
};

}  // namespace msplat
