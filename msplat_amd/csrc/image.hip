// image.hip — the target-image steps of dataset ingest, on the GPU.
//
// Area resize (resizeArea, image_io.cpp:91-138): output pixel (dx, dy) of a
// dstW x dstH image covers the source rectangle [dx*sx, (dx+1)*sx) x
// [dy*sy, (dy+1)*sy), sx = srcW / dstW, sy = srcH / dstH (fp32).  Every source
// pixel it touches is weighted by its overlap wx * wy; the result is the
// weighted sum times 1 / (sum of weights).  The reference loops over output
// pixels on the CPU; here one thread per output pixel runs the same loop,
// rows outer and columns inner, with the same fp32 operations in the same
// order (no contraction), so the output matches the CPU bit for bit.
// Camera::getImage (input_data.cpp:54-65) builds the training pyramid with it
// (integer factors) and Camera::loadImage (input_data.cpp:17-38) the load-time
// downscale (fractional factors).
//
// Undistortion (undistortImage, image_io.cpp:140-330, Brown-Conrady k1 k2 p1
// p2 k3): the host finds the crop rectangle from 4 x 200 boundary points,
// each undistorted by 20 fixed-point iterations (undistort_roi below, the
// reference's own steps); the kernel then, for each pixel of that rectangle
// only, applies the forward distortion to its normalised coordinates and
// samples the source bilinearly with edge clamping.  The reference remaps the
// whole image and copies the rectangle out; remapping only the rectangle
// gives the same pixels.
#include <algorithm>
#include <cmath>

#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

__global__ __launch_bounds__(256) void k_resize_area(const float* __restrict__ src, int sw, int sh,
                                                     float* __restrict__ dst, int dw, int dh,
                                                     float scale_x, float scale_y) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= (int64_t)dw * dh) return;
    const int dx = (int)(p % dw), dy = (int)(p / dw);
    const float y0 = (float)dy * scale_y, y1 = (float)(dy + 1) * scale_y;
    const float x0 = (float)dx * scale_x, x1 = (float)(dx + 1) * scale_x;
    const int iy0 = (int)y0, iy1 = min((int)ceilf(y1), sh);
    const int ix0 = (int)x0, ix1 = min((int)ceilf(x1), sw);
    float s0 = 0.f, s1 = 0.f, s2 = 0.f, total = 0.f;
    for (int iy = iy0; iy < iy1; ++iy) {
        const float wy = fminf((float)(iy + 1), y1) - fmaxf((float)iy, y0);
        const float* row = src + ((int64_t)iy * sw) * 3;
        for (int ix = ix0; ix < ix1; ++ix) {
            const float wx = fminf((float)(ix + 1), x1) - fmaxf((float)ix, x0);
            const float area = wx * wy;
            const float* q = row + 3 * ix;
            s0 += q[0] * area;
            s1 += q[1] * area;
            s2 += q[2] * area;
            total += area;
        }
    }
    const float inv = 1.f / total;
    float* o = dst + 3 * p;
    o[0] = s0 * inv;
    o[1] = s1 * inv;
    o[2] = s2 * inv;
}

// Source index of a sample coordinate: floor, then clamped into the image.
// Values beyond the int range (where the reference's conversion is
// undefined) clamp the same way as values just outside the image.
__device__ __forceinline__ int clamp_floor(float v, int n) {
    const float f = floorf(v);
    if (!(f > -1.f)) return -1;     // also NaN
    if (f > (float)n) return n;
    return (int)f;
}

__global__ __launch_bounds__(256) void k_undistort(const float* __restrict__ src, int w, int h,
                                                   UndistortParams u, float* __restrict__ dst) {
    const int64_t p = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (p >= (int64_t)u.roi_w * u.roi_h) return;
    const int ox = u.roi_x + (int)(p % u.roi_w), oy = u.roi_y + (int)(p / u.roi_w);
    // distortPoint (image_io.cpp:143-153) of the normalised pixel
    const float x = ((float)ox - u.cx) / u.fx;
    const float y = ((float)oy - u.cy) / u.fy;
    const float r2 = x * x + y * y;
    const float r4 = r2 * r2;
    const float r6 = r4 * r2;
    const float radial = 1.0f + u.k1 * r2 + u.k2 * r4 + u.k3 * r6;
    const float xd = x * radial + 2.0f * u.p1 * x * y + u.p2 * (r2 + 2.0f * x * x);
    const float yd = y * radial + u.p1 * (r2 + 2.0f * y * y) + 2.0f * u.p2 * x * y;
    const float sx = xd * u.fx + u.cx;
    const float sy = yd * u.fy + u.cy;
    // bilinearSample (image_io.cpp:174-201)
    const int bx = clamp_floor(sx, w), by = clamp_floor(sy, h);
    const int x0 = min(max(bx, 0), w - 1), x1 = min(max(bx + 1, 0), w - 1);
    const int y0 = min(max(by, 0), h - 1), y1 = min(max(by + 1, 0), h - 1);
    const float fx = sx - floorf(sx);
    const float fy = sy - floorf(sy);
    const float* p00 = src + ((int64_t)y0 * w + x0) * 3;
    const float* p10 = src + ((int64_t)y0 * w + x1) * 3;
    const float* p01 = src + ((int64_t)y1 * w + x0) * 3;
    const float* p11 = src + ((int64_t)y1 * w + x1) * 3;
    float* o = dst + 3 * p;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float top = p00[c] * (1.0f - fx) + p10[c] * fx;
        const float bottom = p01[c] * (1.0f - fx) + p11[c] * fx;
        o[c] = top * (1.0f - fy) + bottom * fy;
    }
}

// undistortPoint (image_io.cpp:156-171): 20 fixed-point iterations.
void undistort_point(float xd, float yd, const UndistortParams& u, float& xu, float& yu) {
    xu = xd;
    yu = yd;
    for (int i = 0; i < 20; i++) {
        const float r2 = xu * xu + yu * yu;
        const float r4 = r2 * r2;
        const float r6 = r4 * r2;
        const float radial = 1.0f + u.k1 * r2 + u.k2 * r4 + u.k3 * r6;
        const float dx = 2.0f * u.p1 * xu * yu + u.p2 * (r2 + 2.0f * xu * xu);
        const float dy = u.p1 * (r2 + 2.0f * yu * yu) + 2.0f * u.p2 * xu * yu;
        xu = (xd - dx) / radial;
        yu = (yd - dy) / radial;
    }
}

}  // namespace

void undistort_roi(int w, int h, UndistortParams& u) {
    // The inner rectangle of the undistorted image borders (image_io.cpp:244-282),
    // 200 samples per edge at t = i / 199 of the width / height.
    float top_max = -1e9f, bottom_min = 1e9f, left_max = -1e9f, right_min = 1e9f;
    const int n = 200;
    for (int i = 0; i < n; i++) {
        const float t = (float)i / (float)(n - 1);
        float xu, yu;
        undistort_point((t * (float)w - u.cx) / u.fx, (0.0f - u.cy) / u.fy, u, xu, yu);
        top_max = std::max(top_max, yu * u.fy + u.cy);
        undistort_point((t * (float)w - u.cx) / u.fx, ((float)(h - 1) - u.cy) / u.fy, u, xu, yu);
        bottom_min = std::min(bottom_min, yu * u.fy + u.cy);
        undistort_point((0.0f - u.cx) / u.fx, (t * (float)h - u.cy) / u.fy, u, xu, yu);
        left_max = std::max(left_max, xu * u.fx + u.cx);
        undistort_point(((float)(w - 1) - u.cx) / u.fx, (t * (float)h - u.cy) / u.fy, u, xu, yu);
        right_min = std::min(right_min, xu * u.fx + u.cx);
    }
    // (float -> int of a value outside the int range is clamped first)
    auto to_int = [](float v) {
        if (!(v > -2.0e9f)) return -2000000000;
        if (v > 2.0e9f) return 2000000000;
        return (int)v;
    };
    int rx = std::max(0, to_int(std::ceil(left_max)));
    int ry = std::max(0, to_int(std::ceil(top_max)));
    int rw = std::min(w, to_int(std::floor(right_min))) - rx;
    int rh = std::min(h, to_int(std::floor(bottom_min))) - ry;
    if (rw <= 0 || rh <= 0) { rx = 0; ry = 0; rw = w; rh = h; }
    u.roi_x = rx; u.roi_y = ry; u.roi_w = rw; u.roi_h = rh;
}

void launch_resize_area(hipStream_t s, const float* src, int sw, int sh, float* dst, int dw,
                        int dh) {
    const int64_t n = (int64_t)dw * dh;
    if (n <= 0) return;
    const float scale_x = (float)sw / (float)dw, scale_y = (float)sh / (float)dh;
    hipLaunchKernelGGL(k_resize_area, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, sw,
                       sh, dst, dw, dh, scale_x, scale_y);
}

void launch_undistort(hipStream_t s, const float* src, int w, int h, const UndistortParams& u,
                      float* dst) {
    const int64_t n = (int64_t)u.roi_w * u.roi_h;
    if (n <= 0) return;
    hipLaunchKernelGGL(k_undistort, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, s, src, w, h,
                       u, dst);
}

}  // namespace msp
