// eval.hip — the two image steps either side of a render: the RGBA8 display
// conversion and the evaluation metrics (PSNR, L1, SSIM) of a render against
// its target.
//
// RGBA8: Trainer::renderFromPoseToBuffer (msplat_api.mm:230-238) converts on
// the CPU: each channel min(max(v, 0), 1) * 255 truncated to a byte, alpha
// 255.  Here one thread per pixel writes its four bytes as one 32-bit store,
// so only 4 bytes per pixel cross to the host instead of 12.
//
// Metrics: psnr / l1_loss (model.cpp:25-40) and ssim_eval (ssim.cpp:61-123).
// SSIM blurs five maps per channel (x, y, x^2, y^2, xy) with a separable
// window_size-tap Gaussian whose borders clamp to the edge pixel
// (gaussianBlur, ssim.cpp:26-59), then averages
//   (2 mu_x mu_y + C1)(2 s_xy + C2) / ((mu_x^2 + mu_y^2 + C1)(s_x^2 + s_y^2 + C2))
// over pixels and channels, C1 = 0.01^2, C2 = 0.03^2.  One 256-thread
// workgroup per 64x16 output tile stages the tile plus a 5-pixel clamped
// halo of both images in LDS, one channel at a time, takes the horizontal
// sums into LDS and the vertical sums from there.  Every per-pixel float is
// formed with the reference's operations in its order (horizontal pass
// first, taps summed from the first, products rounded before weighting), so
// per-pixel SSIM terms equal the CPU's; the sums over pixels are fp64 like
// the reference's, folded per workgroup and then over workgroups in a fixed
// order.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

__global__ __launch_bounds__(256) void k_to_rgba8(const float* __restrict__ img, int64_t n,
                                                  uint32_t* __restrict__ rgba) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= n) return;
    uint32_t word = 0xFF000000u;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float v = fminf(fmaxf(img[3 * p + c], 0.f), 1.f) * 255.f;
        word |= (uint32_t)(uint8_t)v << (8 * c);
    }
    rgba[p] = word;
}

constexpr int EV_R = 5;                  // largest window radius (11 taps)
constexpr int EV_TW = 64, EV_TH = 16;    // output tile
constexpr int EV_IW = EV_TW + 2 * EV_R, EV_IH = EV_TH + 2 * EV_R;

// Double sum over the 256 threads of a block, fixed order (sh: 256 doubles).
__device__ __forceinline__ double block_sum_f64(double v, double* sh) {
    sh[threadIdx.x] = v;
    __syncthreads();
    for (int s = 128; s > 0; s >>= 1) {
        if ((int)threadIdx.x < s) sh[threadIdx.x] += sh[threadIdx.x + s];
        __syncthreads();
    }
    const double t = sh[0];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(256) void k_eval_tiles(const float* __restrict__ img,
                                                    const float* __restrict__ gt, int W, int H,
                                                    EvalWindow win, double* __restrict__ part) {
    __shared__ float s_r[EV_IH][EV_IW];
    __shared__ float s_g[EV_IH][EV_IW];
    __shared__ float s_h[5][EV_IH][EV_TW];
    __shared__ double s_red[256];
    const int x0 = blockIdx.x * EV_TW, y0 = blockIdx.y * EV_TH;
    const int tid = threadIdx.x;
    // taps k = 0..ws-1 read offsets d = k - pad from the staged centre
    const int off = EV_R - win.pad;
    const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
    double ssim_sum = 0.0, sq_sum = 0.0, abs_sum = 0.0;
    for (int c = 0; c < 3; ++c) {
        __syncthreads();
        for (int i = tid; i < EV_IH * EV_IW; i += 256) {
            const int r = i / EV_IW, col = i - r * EV_IW;
            const int sy = min(max(y0 - EV_R + r, 0), H - 1);
            const int sx = min(max(x0 - EV_R + col, 0), W - 1);
            const size_t s = 3 * ((size_t)sy * W + sx) + c;
            s_r[r][col] = img[s];
            s_g[r][col] = gt[s];
        }
        __syncthreads();
        for (int i = tid; i < EV_IH * EV_TW; i += 256) {
            const int r = i / EV_TW, ox = i - r * EV_TW;
            float a = 0.f, b = 0.f, aa = 0.f, bb = 0.f, ab = 0.f;
            for (int k = 0; k < win.ws; ++k) {
                const float rv = s_r[r][ox + off + k], gv = s_g[r][ox + off + k], wk = win.w[k];
                const float rr = rv * rv, gg = gv * gv, rg = rv * gv;
                a += rv * wk;
                b += gv * wk;
                aa += rr * wk;
                bb += gg * wk;
                ab += rg * wk;
            }
            s_h[0][r][ox] = a;
            s_h[1][r][ox] = b;
            s_h[2][r][ox] = aa;
            s_h[3][r][ox] = bb;
            s_h[4][r][ox] = ab;
        }
        __syncthreads();
        for (int i = tid; i < EV_TH * EV_TW; i += 256) {
            const int oy = i / EV_TW, ox = i - oy * EV_TW;
            if (y0 + oy >= H || x0 + ox >= W) continue;
            float mu1 = 0.f, mu2 = 0.f, s11 = 0.f, s22 = 0.f, s12 = 0.f;
            for (int k = 0; k < win.ws; ++k) {
                const int r = oy + off + k;
                const float wk = win.w[k];
                mu1 += s_h[0][r][ox] * wk;
                mu2 += s_h[1][r][ox] * wk;
                s11 += s_h[2][r][ox] * wk;
                s22 += s_h[3][r][ox] * wk;
                s12 += s_h[4][r][ox] * wk;
            }
            const float m1sq = mu1 * mu1, m2sq = mu2 * mu2, m12 = mu1 * mu2;
            const float sig1sq = s11 - m1sq, sig2sq = s22 - m2sq, sig12 = s12 - m12;
            const float num = (2.0f * m12 + C1) * (2.0f * sig12 + C2);
            const float den = (m1sq + m2sq + C1) * (sig1sq + sig2sq + C2);
            ssim_sum += (double)(num / den);
            const float d = s_r[oy + EV_R][ox + EV_R] - s_g[oy + EV_R][ox + EV_R];
            sq_sum += (double)d * (double)d;
            abs_sum += (double)fabsf(d);
        }
    }
    const size_t b = (size_t)blockIdx.y * gridDim.x + blockIdx.x;
    const double t0 = block_sum_f64(ssim_sum, s_red);
    const double t1 = block_sum_f64(sq_sum, s_red);
    const double t2 = block_sum_f64(abs_sum, s_red);
    if (tid == 0) {
        part[3 * b + 0] = t0;
        part[3 * b + 1] = t1;
        part[3 * b + 2] = t2;
    }
}

// Sum of the nb workgroup partials (3 each), fixed order, into out[3].
__global__ __launch_bounds__(256) void k_eval_fold(const double* __restrict__ part, int nb,
                                                   double* __restrict__ out) {
    __shared__ double s_red[256];
    double v[3] = {0.0, 0.0, 0.0};
    for (int b = threadIdx.x; b < nb; b += 256)
#pragma unroll
        for (int k = 0; k < 3; ++k) v[k] += part[3 * (size_t)b + k];
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        const double t = block_sum_f64(v[k], s_red);
        if (threadIdx.x == 0) out[k] = t;
    }
}

}  // namespace

int64_t eval_partial_count(int H, int W) {
    return (int64_t)((W + EV_TW - 1) / EV_TW) * ((H + EV_TH - 1) / EV_TH);
}

void launch_to_rgba8(hipStream_t s, const float* img, int64_t n, uint32_t* rgba) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_to_rgba8, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, img, n,
                       rgba);
}

void launch_image_metrics(hipStream_t s, const float* img, const float* gt, int H, int W,
                          const EvalWindow& win, double* part, double* out3) {
    const dim3 grid((W + EV_TW - 1) / EV_TW, (H + EV_TH - 1) / EV_TH);
    hipLaunchKernelGGL(k_eval_tiles, grid, dim3(256), 0, s, img, gt, W, H, win, part);
    hipLaunchKernelGGL(k_eval_fold, dim3(1), dim3(256), 0, s, (const double*)part,
                       (int)(grid.x * grid.y), out3);
}

}  // namespace msp
