// oracle.cpp — CPU restatement of msplat's splatting hot path.
//
// TEST INFRASTRUCTURE ONLY: the parity checker and CPU baseline for the HIP
// path.  Nothing in msplat_amd/ links or loads it.  Built with
// -ffp-contract=off so every a*b+c rounds twice unless written as fmaf(), the
// way the reference writes fma() (msplat_metal.metal).
//
// Functions and the reference lines they restate:
//   oexp                    exp() call sites (.metal:1736, 2133 ...); own
//                           Cody–Waite + Taylor exp, pinned vs libm in tests
//   oexp_raster             exp() of the rasteriser (.metal:555, 1032); own
//                           Remez-fitted exp, pinned vs libm in tests
//   quat_to_rotmat          .metal:111-131
//   scale_rot_to_cov3d      .metal:175-188
//   project_cov3d_ewa       .metal:241-281
//   compute_cov2d_bounds    .metal:283-305
//   project_pix / ndc2pix   .metal:308-317, 53-55
//   get_bbox/get_tile_bbox  .metal:57-87
//   sh_coeffs_to_color      .metal:587-654
//   project_and_sh_forward  .metal:1695-1787
//   scatter/prefix/bitonic  .metal:2025-2138, 2312-2364 (uncapped tiles)
//   rasterize forward       .metal:472-585; chunked + merge .metal:2633-2799
//   rasterize backward      .metal:898-1099; prefix/suffix + chunked .metal:2804-3031
//   SSIM (training path)    .metal:3041-3045, 3053-3115, 3226-3313, 3396-3464
//   projection backward     .metal:1216-1234, 1253-1264, 1339-1407, 1409-1452,
//                           1498-1531, 1813-1910
//   SH backward + Adam      .metal:1791-1800, 1912-1985
//   fused_adam              .metal:1666-1689
//   accumulate_grad_stats   .metal:1643-1664
//   train step order        msplat_metal.mm:1141-1330
//   densify                 .metal:3475-3729, msplat_metal.mm:1337-1592
//   image metrics           model.cpp:25-40, ssim.cpp:26-123
//   rgba8                   msplat_api.mm:230-238
//   knn mean distance       kdtree_tensor.hpp:26-40 (brute force)
//   resize_area             image_io.cpp:91-138
//   undistort (+ roi)       image_io.cpp:140-330

#include "oracle.h"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdint>
#include <cstring>
#include <limits>
#include <vector>
#ifdef _OPENMP
#include <omp.h>
#endif

namespace {

constexpr int BLOCK = 16;          // msplat.hpp:4-5
constexpr int CHUNK = 512;         // .metal:2616
// Largest tile rasterised in one piece outside chunk mode.  The reference's
// monolithic kernel bins at most MAX_TILE_ELEMS = 2048 entries per tile
// (.metal:2021) and drops the rest; here tiles of up to 8192 entries are
// rasterised in one piece, uncapped (the reference's monolithic result
// wherever it keeps every entry), and larger ones in 512-entry chunks.
constexpr int MONO_MAX = 8192;
constexpr int CHUNK_MODE_TILES = 400;  // .mm:876

// SH constants (.metal:14-39).
constexpr float SH_C0 = 0.28209479177387814f;
constexpr float SH_C1 = 0.4886025119029199f;
constexpr float SH_C2[5] = {1.0925484305920792f, -1.0925484305920792f, 0.31539156525252005f,
                            -1.0925484305920792f, 0.5462742152960396f};
constexpr float SH_C3[7] = {-0.5900435899266435f, 2.890611442640554f, -0.4570457994644658f,
                            0.3731763325901154f, -0.4570457994644658f, 1.445305721320277f,
                            -0.5900435899266435f};
constexpr float SH_C4[9] = {2.5033429417967046f, -1.7701307697799304f, 0.9461746957575601f,
                            -0.6690465435572892f, 0.10578554691520431f, -0.6690465435572892f,
                            0.47308734787878004f, -1.7701307697799304f, 0.6258357354491761f};

// GAUSS_1D (.metal:3041-3045).
constexpr float GAUSS_1D[11] = {0.0010283801f, 0.0075987581f, 0.0360007721f, 0.1093606895f,
                                0.2130055377f, 0.2660117249f, 0.2130055377f, 0.1093606895f,
                                0.0360007721f, 0.0075987581f, 0.0010283801f};
constexpr float SSIM_C1 = 0.0001f;   // .metal:2448
constexpr float SSIM_C2 = 0.0009f;   // .metal:2449

inline float bits_to_float(uint32_t u) { float f; std::memcpy(&f, &u, 4); return f; }
inline uint32_t float_to_bits(float f) { uint32_t u; std::memcpy(&u, &f, 4); return u; }

// exp(x): Cody–Waite reduction x = k*ln2 + r (|r| <= ln2/2, ln2 split in a
// 16-bit head and a tail), degree-7 Taylor polynomial in Horner form with
// fmaf, then scaling by 2^k through the exponent field.  Inputs below -87 give
// 0 (no subnormal results), above 88 give +inf, NaN propagates.
inline float oexp(float x) {
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.0f) return std::numeric_limits<float>::infinity();
    const float k = std::nearbyint(x * 1.44269504f);
    float r = std::fma(k, -0.693145751953125f, x);
    r = std::fma(k, -1.42860682e-6f, r);
    float p = 1.98412698e-4f;
    p = std::fma(p, r, 1.38888889e-3f);
    p = std::fma(p, r, 8.33333333e-3f);
    p = std::fma(p, r, 4.16666667e-2f);
    p = std::fma(p, r, 1.66666667e-1f);
    p = std::fma(p, r, 0.5f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    const int ki = (int)k;
    return p * bits_to_float((uint32_t)(ki + 127) << 23);
}

// exp(x) of the rasteriser's -sigma (.metal:555, 1032), x in (-5.55, 0]:
// k = rint(x log2 e), r = x - k ln2 with one fma, a degree-6 polynomial with
// coefficients from a Remez exchange for least relative error of e^r on
// [-ln2/2, ln2/2] (rounded to float), then ldexp.  Within 1.02 ulp of exp
// over [-5.6, 0] (pinned vs libm in tests).  The exponent is clamped before
// the conversion so that every input has a defined result; NaN propagates.
inline float oexp_raster(float x) {
    const float k = std::nearbyint(x * 0x1.715476p+0f);
    const float r = std::fma(k, -0x1.62e430p-1f, x);
    float p = 0x1.6ab980p-10f;
    p = std::fma(p, r, 0x1.126d0cp-7f);
    p = std::fma(p, r, 0x1.55589ap-5f);
    p = std::fma(p, r, 0x1.55540ap-3f);
    p = std::fma(p, r, 0x1.fffffap-2f);
    p = std::fma(p, r, 1.0f);
    p = std::fma(p, r, 1.0f);
    return std::ldexp(p, (int)std::fmin(std::fmax(k, -256.f), 256.f));
}

// The rasteriser's range early-out (.metal:551, 1029, 2718, 2976: skip when
// sigma < 0 || sigma >= 5.55), as the HIP kernels evaluate it: sigma's bits
// clamped with one unsigned min to those of 5.55f, so that sigma in
// [+0, 5.55) keeps its value and everything else (negative, -0, >= 5.55,
// +inf, NaN) becomes 5.55, where alpha = min(0.999, o exp(-5.55)) <=
// 0.0038875 < 1/255 for every opacity o in [0, 1] and the alpha test rejects
// the pair.  Returns whether the pair goes on to the alpha test, and the
// sigma it uses there.  This equals the reference's test for every sigma
// but -0 and NaN (rejected here), which only a degenerate conic produces,
// and for every opacity but NaN (whose alpha is 0.999 either way).
inline bool sigma_in(float sigma, float opac, float* s_used) {
    uint32_t b;
    std::memcpy(&b, &sigma, 4);
    if (b < 0x40B1999Au) {   // 0x40B1999A = 5.55f
        *s_used = sigma;
        return true;
    }
    *s_used = 5.55f;
    return opac != opac;     // a NaN opacity makes alpha 0.999 even here
}

// float -> int with the operand clamped to [-2^30, 2^30] first, so every
// input (inf and NaN included) has one defined result on every target.
inline int f2i(float v) { return (int)std::fmin(std::fmax(v, -1073741824.f), 1073741824.f); }

inline float sigmoid(float o) { return 1.f / (1.f + oexp(-o)); }   // .metal:2133
inline float clampf(float v, float lo, float hi) { return std::fmin(std::fmax(v, lo), hi); }

// Running error analysis (Wilkinson; Higham, "Accuracy and Stability of
// Numerical Algorithms", 2nd ed., section 3.3).  An RE carries a value v and
// a first-order bound e on the absolute error of a float computation of v,
// in units of u = 2^-24.  Every operation adds its own rounding (|result|)
// to the errors its operands carry, scaled by the partial derivatives:
//   e(a +- b) = e(a) + e(b) + |a +- b|
//   e(a * b)  = e(a) |b| + |a| e(b) + |a b|
//   e(a / b)  = (e(a) + |a / b| e(b)) / |b| + |a / b|
//   e(sqrt a) = e(a) / (2 sqrt a) + sqrt a
// The backward helpers below are templates over the scalar type: S = float
// is the oracle itself (the same float operations as before), S = RE
// evaluates the same expression graph for its error bound.
constexpr double kU = 1.0 / 16777216.0;   // u = 2^-24, the fp32 unit roundoff

struct RE {
    double v = 0.0, e = 0.0;
    RE() = default;
    RE(float x) : v(x), e(0.0) {}          // exact operand
    RE(double x, double err) : v(x), e(err) {}
};
inline RE operator+(RE a, RE b) { const double v = a.v + b.v; return RE(v, a.e + b.e + std::fabs(v)); }
inline RE operator-(RE a, RE b) { const double v = a.v - b.v; return RE(v, a.e + b.e + std::fabs(v)); }
inline RE operator-(RE a) { return RE(-a.v, a.e); }
inline RE operator*(RE a, RE b) {
    const double v = a.v * b.v;
    return RE(v, a.e * std::fabs(b.v) + std::fabs(a.v) * b.e + std::fabs(v));
}
inline RE operator/(RE a, RE b) {
    const double v = a.v / b.v;
    return RE(v, (a.e + std::fabs(v) * b.e) / std::fabs(b.v) + std::fabs(v));
}
inline RE& operator+=(RE& a, RE b) { a = a + b; return a; }
inline float msqrt(float x) { return std::sqrt(x); }
inline RE msqrt(RE a) {
    const double v = std::sqrt(a.v);
    return RE(v, (v > 0.0 ? a.e / (2.0 * v) : 0.0) + v);
}
inline float mfmin(float a, float b) { return std::fmin(a, b); }
inline float mfmax(float a, float b) { return std::fmax(a, b); }
inline RE mfmin(RE a, RE b) { return RE(std::fmin(a.v, b.v), std::fmax(a.e, b.e)); }
inline RE mfmax(RE a, RE b) { return RE(std::fmax(a.v, b.v), std::fmax(a.e, b.e)); }

template <class S> struct V3 { S x, y, z; };
// Column-major 3x3 (m[col][row]) like Metal's float3x3.
template <class S> struct Mat3 { S m[3][3]; };
using F3 = V3<float>;
using M3 = Mat3<float>;

template <class S>
inline V3<S> mat_vec(const Mat3<S>& A, V3<S> v) {   // A * v = A[0]*v.x + A[1]*v.y + A[2]*v.z
    V3<S> r;
    r.x = A.m[0][0] * v.x + A.m[1][0] * v.y + A.m[2][0] * v.z;
    r.y = A.m[0][1] * v.x + A.m[1][1] * v.y + A.m[2][1] * v.z;
    r.z = A.m[0][2] * v.x + A.m[1][2] * v.y + A.m[2][2] * v.z;
    return r;
}
template <class S>
inline Mat3<S> mat_mul(const Mat3<S>& A, const Mat3<S>& B) {
    Mat3<S> C;
    for (int j = 0; j < 3; ++j) {
        V3<S> col = mat_vec(A, V3<S>{B.m[j][0], B.m[j][1], B.m[j][2]});
        C.m[j][0] = col.x; C.m[j][1] = col.y; C.m[j][2] = col.z;
    }
    return C;
}
template <class S>
inline Mat3<S> transpose(const Mat3<S>& A) {
    Mat3<S> T;
    for (int i = 0; i < 3; ++i) for (int j = 0; j < 3; ++j) T.m[i][j] = A.m[j][i];
    return T;
}
template <class S>
inline Mat3<S> mat_add(const Mat3<S>& A, const Mat3<S>& B) {
    Mat3<S> C;
    for (int i = 0; i < 3; ++i) for (int j = 0; j < 3; ++j) C.m[i][j] = A.m[i][j] + B.m[i][j];
    return C;
}
template <class S>
inline S dot3(V3<S> a, V3<S> b) { return a.x * b.x + a.y * b.y + a.z * b.z; }

// .metal:111-131.  quat stored (w,x,y,z); 1/sqrt stands in for rsqrt.
template <class S>
inline Mat3<S> quat_to_rotmat(const S* q) {
    const S s = S(1.f) / msqrt(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
    const S w = q[0] * s, x = q[1] * s, y = q[2] * s, z = q[3] * s;
    Mat3<S> R;
    R.m[0][0] = 1.f - 2.f * (y * y + z * z);
    R.m[0][1] = 2.f * (x * y + w * z);
    R.m[0][2] = 2.f * (x * z - w * y);
    R.m[1][0] = 2.f * (x * y - w * z);
    R.m[1][1] = 1.f - 2.f * (x * x + z * z);
    R.m[1][2] = 2.f * (y * z + w * x);
    R.m[2][0] = 2.f * (x * z + w * y);
    R.m[2][1] = 2.f * (y * z - w * x);
    R.m[2][2] = 1.f - 2.f * (x * x + y * y);
    return R;
}

// .metal:175-188: cov = (R S)(R S)^T, upper triangle.  M[j] = R[j] * s_j.
template <class S>
inline void scale_rot_to_cov3d(const S* s3, float glob, const S* q, S* cov) {
    const Mat3<S> R = quat_to_rotmat(q);
    const S sv[3] = {glob * s3[0], glob * s3[1], glob * s3[2]};
    Mat3<S> M;
    for (int j = 0; j < 3; ++j) for (int i = 0; i < 3; ++i) M.m[j][i] = R.m[j][i] * sv[j];
    auto t = [&](int i, int j) {   // tmp[j][i] = sum_k M[k][i] * M[k][j]
        return M.m[0][i] * M.m[0][j] + M.m[1][i] * M.m[1][j] + M.m[2][i] * M.m[2][j];
    };
    cov[0] = t(0, 0); cov[1] = t(1, 0); cov[2] = t(2, 0);
    cov[3] = t(1, 1); cov[4] = t(2, 1); cov[5] = t(2, 2);
}

// .metal:90-108.
template <class S>
inline V3<S> transform_4x3(const float* m, V3<S> p) {
    return V3<S>{m[0] * p.x + m[1] * p.y + m[2] * p.z + m[3],
                 m[4] * p.x + m[5] * p.y + m[6] * p.z + m[7],
                 m[8] * p.x + m[9] * p.y + m[10] * p.z + m[11]};
}

// .metal:241-281.
inline F3 project_cov3d_ewa(const float* cov3d, const float* vm, float fx, float fy,
                            float tan_fovx, float tan_fovy, F3 pv) {
    const float lim_x = 1.3f * tan_fovx, lim_y = 1.3f * tan_fovy;
    pv.x = pv.z * std::fmin(lim_x, std::fmax(-lim_x, pv.x / pv.z));
    pv.y = pv.z * std::fmin(lim_y, std::fmax(-lim_y, pv.y / pv.z));
    const float rz = 1.f / pv.z, rz2 = rz * rz;
    const float j00 = fx * rz, j11 = fy * rz;
    const float j20 = -fx * pv.x * rz2, j21 = -fy * pv.y * rz2;
    const F3 mr0{vm[0], vm[1], vm[2]}, mr1{vm[4], vm[5], vm[6]}, mr2{vm[8], vm[9], vm[10]};
    const F3 t0{j00 * mr0.x + j20 * mr2.x, j00 * mr0.y + j20 * mr2.y, j00 * mr0.z + j20 * mr2.z};
    const F3 t1{j11 * mr1.x + j21 * mr2.x, j11 * mr1.y + j21 * mr2.y, j11 * mr1.z + j21 * mr2.z};
    const float v00 = cov3d[0], v01 = cov3d[1], v02 = cov3d[2];
    const float v11 = cov3d[3], v12 = cov3d[4], v22 = cov3d[5];
    const F3 tv0{t0.x * v00 + t0.y * v01 + t0.z * v02, t0.x * v01 + t0.y * v11 + t0.z * v12,
                 t0.x * v02 + t0.y * v12 + t0.z * v22};
    const F3 tv1{t1.x * v00 + t1.y * v01 + t1.z * v02, t1.x * v01 + t1.y * v11 + t1.z * v12,
                 t1.x * v02 + t1.y * v12 + t1.z * v22};
    return F3{dot3(tv0, t0) + 0.3f, dot3(tv0, t1), dot3(tv1, t1) + 0.3f};
}

// .metal:283-305.
inline bool compute_cov2d_bounds(F3 c, F3& conic, float& radius) {
    const float det = c.x * c.z - c.y * c.y;
    if (det == 0.f) return false;
    const float inv_det = 1.f / det;
    conic.x = c.z * inv_det;
    conic.y = -c.y * inv_det;
    conic.z = c.x * inv_det;
    const float b = 0.5f * (c.x + c.z);
    const float disc = std::sqrt(std::fmax(0.1f, b * b - det));
    radius = std::ceil(3.f * std::sqrt(b + disc));
    return true;
}

// .metal:53-55, 308-317 (the 0.5 of ndc2pix is fp32 in Metal).
inline void project_pix(const float* m, F3 p, int W, int H, float cx, float cy, float* out) {
    const float hx = m[0] * p.x + m[1] * p.y + m[2] * p.z + m[3];
    const float hy = m[4] * p.x + m[5] * p.y + m[6] * p.z + m[7];
    const float hw = m[12] * p.x + m[13] * p.y + m[14] * p.z + m[15];
    const float rw = 1.f / (hw + 1e-6f);
    const float px = hx * rw, py = hy * rw;
    out[0] = 0.5f * (float)W * px + cx - 0.5f;
    out[1] = 0.5f * (float)H * py + cy - 0.5f;
}

// .metal:57-87.
inline void tile_bbox(const float* xy, const float* ext, int tbx, int tby, int* r) {
    const float tcx = xy[0] / (float)BLOCK, tcy = xy[1] / (float)BLOCK;
    const float trx = ext[0] / (float)BLOCK, try_ = ext[1] / (float)BLOCK;
    r[0] = std::min(std::max(0, f2i(tcx - trx)), tbx);
    r[2] = std::min(std::max(0, f2i(tcx + trx + 1)), tbx);
    r[1] = std::min(std::max(0, f2i(tcy - try_)), tby);
    r[3] = std::min(std::max(0, f2i(tcy + try_ + 1)), tby);
}

// SH basis values for bands 1..degree (.metal:602-652), written in the order
// of the rest coefficients.  Returns the number of rest bases filled.
template <class S>
inline int sh_rest_basis(int degree, V3<S> d, S* out) {
    if (degree < 1) return 0;
    const S x = d.x, y = d.y, z = d.z;
    const S xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
    out[0] = -SH_C1 * y; out[1] = SH_C1 * z; out[2] = -SH_C1 * x;
    if (degree < 2) return 3;
    out[3] = SH_C2[0] * xy;
    out[4] = SH_C2[1] * yz;
    out[5] = SH_C2[2] * (2.f * zz - xx - yy);
    out[6] = SH_C2[3] * xz;
    out[7] = SH_C2[4] * (xx - yy);
    if (degree < 3) return 8;
    out[8] = SH_C3[0] * y * (3.f * xx - yy);
    out[9] = SH_C3[1] * xy * z;
    out[10] = SH_C3[2] * y * (4.f * zz - xx - yy);
    out[11] = SH_C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy);
    out[12] = SH_C3[4] * x * (4.f * zz - xx - yy);
    out[13] = SH_C3[5] * z * (xx - yy);
    out[14] = SH_C3[6] * x * (xx - 3.f * yy);
    if (degree < 4) return 15;
    out[15] = SH_C4[0] * xy * (xx - yy);
    out[16] = SH_C4[1] * yz * (3.f * xx - yy);
    out[17] = SH_C4[2] * xy * (7.f * zz - 1.f);
    out[18] = SH_C4[3] * yz * (7.f * zz - 3.f);
    out[19] = SH_C4[4] * (zz * (35.f * zz - 30.f) + 3.f);
    out[20] = SH_C4[5] * xz * (7.f * zz - 3.f);
    out[21] = SH_C4[6] * (xx - yy) * (7.f * zz - 1.f);
    out[22] = SH_C4[7] * xz * (xx - 3.f * yy);
    out[23] = SH_C4[8] * (xx * (xx - 3.f * yy) - yy * (3.f * xx - yy));
    return 24;
}

// .metal:587-654.  The forward groups the basis terms of one band into one
// parenthesised sum (band 1: -y*r0 + z*r1 - x*r2, then times SH_C1).
inline void sh_coeffs_to_color(int degree, F3 d, const float* dc, const float* rest, float* col) {
    for (int c = 0; c < 3; ++c) col[c] = SH_C0 * dc[c];
    if (degree < 1) return;
    const float x = d.x, y = d.y, z = d.z;
    const float xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
    for (int c = 0; c < 3; ++c) {
        const float* r = rest + c;   // r[3*b] = coefficient b, channel c
        col[c] += SH_C1 * (-y * r[0] + z * r[3] - x * r[6]);
        if (degree < 2) continue;
        col[c] += (SH_C2[0] * xy * r[9] + SH_C2[1] * yz * r[12] +
                   SH_C2[2] * (2.f * zz - xx - yy) * r[15] + SH_C2[3] * xz * r[18] +
                   SH_C2[4] * (xx - yy) * r[21]);
        if (degree < 3) continue;
        col[c] += (SH_C3[0] * y * (3.f * xx - yy) * r[24] + SH_C3[1] * xy * z * r[27] +
                   SH_C3[2] * y * (4.f * zz - xx - yy) * r[30] +
                   SH_C3[3] * z * (2.f * zz - 3.f * xx - 3.f * yy) * r[33] +
                   SH_C3[4] * x * (4.f * zz - xx - yy) * r[36] +
                   SH_C3[5] * z * (xx - yy) * r[39] + SH_C3[6] * x * (xx - 3.f * yy) * r[42]);
        if (degree < 4) continue;
        col[c] += (SH_C4[0] * xy * (xx - yy) * r[45] + SH_C4[1] * yz * (3.f * xx - yy) * r[48] +
                   SH_C4[2] * xy * (7.f * zz - 1.f) * r[51] +
                   SH_C4[3] * yz * (7.f * zz - 3.f) * r[54] +
                   SH_C4[4] * (zz * (35.f * zz - 30.f) + 3.f) * r[57] +
                   SH_C4[5] * xz * (7.f * zz - 3.f) * r[60] +
                   SH_C4[6] * (xx - yy) * (7.f * zz - 1.f) * r[63] +
                   SH_C4[7] * xz * (xx - 3.f * yy) * r[66] +
                   SH_C4[8] * (xx * (xx - 3.f * yy) - yy * (3.f * xx - yy)) * r[69]);
    }
}

inline int num_sh_bases(int degree) {   // .metal:41-51
    return degree == 0 ? 1 : degree == 1 ? 4 : degree == 2 ? 9 : degree == 3 ? 16 : 25;
}

// normalize(p - cam_pos) (.metal:1780): v * (1/sqrt(dot(v, v))).
inline F3 view_dir(const float* p, const float* cam) {
    const F3 v{p[0] - cam[0], p[1] - cam[1], p[2] - cam[2]};
    const float inv = 1.f / std::sqrt(v.x * v.x + v.y * v.y + v.z * v.z);
    return F3{v.x * inv, v.y * inv, v.z * inv};
}

inline int tiles_x(const OrcCamera* c) { return (c->width + BLOCK - 1) / BLOCK; }
inline int tiles_y(const OrcCamera* c) { return (c->height + BLOCK - 1) / BLOCK; }

// ---------------- backward helpers ----------------

// .metal:1216-1234: only the x/y rows through a fixed 1/w (the w row is dropped).
template <class S>
inline V3<S> project_pix_vjp(const float* m, V3<S> p, int W, int H, const S* v_xy) {
    const S hw = m[12] * p.x + m[13] * p.y + m[14] * p.z + m[15];
    const S rw = S(1.f) / (hw + 1e-6f);
    const S vnx = 0.5f * (float)W * v_xy[0], vny = 0.5f * (float)H * v_xy[1];
    const S vpx = vnx * rw, vpy = vny * rw, vpz = 0.f;
    return V3<S>{m[0] * vpx + m[4] * vpy + m[8] * vpz,
                 m[1] * vpx + m[5] * vpy + m[9] * vpz,
                 m[2] * vpx + m[6] * vpy + m[10] * vpz};
}

// .metal:1253-1264: v_Sigma = -X G X (2x2 symmetric), off-diagonal summed.
template <class S>
inline void cov2d_to_conic_vjp(const S* conic, const S* v_conic, S* v_cov2d) {
    const S X[2][2] = {{conic[0], conic[1]}, {conic[1], conic[2]}};   // [col][row]
    const S G[2][2] = {{v_conic[0], v_conic[1]}, {v_conic[1], v_conic[2]}};
    S nX[2][2];
    for (int i = 0; i < 2; ++i) for (int j = 0; j < 2; ++j) nX[i][j] = -1.f * X[i][j];
    auto mul = [](const S A[2][2], const S B[2][2], S C[2][2]) {
        for (int j = 0; j < 2; ++j)
            for (int i = 0; i < 2; ++i) C[j][i] = A[0][i] * B[j][0] + A[1][i] * B[j][1];
    };
    S T1[2][2], Sm[2][2];
    mul(nX, G, T1);
    mul(T1, X, Sm);
    v_cov2d[0] = Sm[0][0];
    v_cov2d[1] = Sm[1][0] + Sm[0][1];
    v_cov2d[2] = Sm[1][1];
}

// .metal:1339-1407.
template <class S>
inline void project_cov3d_ewa_vjp(const S* cov3d, const float* vm, float fx, float fy,
                                  float tan_fovx, float tan_fovy, const S* v_cov2d,
                                  V3<S>& v_mean, S* v_cov3d, V3<S> pv) {
    const float lim_x = 1.3f * tan_fovx, lim_y = 1.3f * tan_fovy;
    pv.x = pv.z * mfmin(S(lim_x), mfmax(S(-lim_x), pv.x / pv.z));
    pv.y = pv.z * mfmin(S(lim_y), mfmax(S(-lim_y), pv.y / pv.z));
    const S rz = S(1.f) / pv.z, rz2 = rz * rz;
    Mat3<S> W;   // columns (vm0,vm4,vm8), (vm1,vm5,vm9), (vm2,vm6,vm10)
    W.m[0][0] = vm[0]; W.m[0][1] = vm[4]; W.m[0][2] = vm[8];
    W.m[1][0] = vm[1]; W.m[1][1] = vm[5]; W.m[1][2] = vm[9];
    W.m[2][0] = vm[2]; W.m[2][1] = vm[6]; W.m[2][2] = vm[10];
    Mat3<S> J;
    J.m[0][0] = fx * rz; J.m[0][1] = 0.f; J.m[0][2] = 0.f;
    J.m[1][0] = 0.f; J.m[1][1] = fy * rz; J.m[1][2] = 0.f;
    J.m[2][0] = -fx * pv.x * rz2; J.m[2][1] = -fy * pv.y * rz2; J.m[2][2] = 0.f;
    Mat3<S> V;
    V.m[0][0] = cov3d[0]; V.m[0][1] = cov3d[1]; V.m[0][2] = cov3d[2];
    V.m[1][0] = cov3d[1]; V.m[1][1] = cov3d[3]; V.m[1][2] = cov3d[4];
    V.m[2][0] = cov3d[2]; V.m[2][1] = cov3d[4]; V.m[2][2] = cov3d[5];
    Mat3<S> vc;
    vc.m[0][0] = v_cov2d[0]; vc.m[0][1] = 0.5f * v_cov2d[1]; vc.m[0][2] = 0.f;
    vc.m[1][0] = 0.5f * v_cov2d[1]; vc.m[1][1] = v_cov2d[2]; vc.m[1][2] = 0.f;
    vc.m[2][0] = 0.f; vc.m[2][1] = 0.f; vc.m[2][2] = 0.f;
    const Mat3<S> T = mat_mul(J, W);
    const Mat3<S> Tt = transpose(T), Vt = transpose(V);
    const Mat3<S> vV = mat_mul(mat_mul(Tt, vc), T);
    const Mat3<S> vT = mat_add(mat_mul(mat_mul(vc, T), Vt), mat_mul(mat_mul(transpose(vc), T), V));
    v_cov3d[0] = vV.m[0][0];
    v_cov3d[1] = vV.m[0][1] + vV.m[1][0];
    v_cov3d[2] = vV.m[0][2] + vV.m[2][0];
    v_cov3d[3] = vV.m[1][1];
    v_cov3d[4] = vV.m[1][2] + vV.m[2][1];
    v_cov3d[5] = vV.m[2][2];
    const Mat3<S> vJ = mat_mul(vT, transpose(W));
    const S fx_rz2 = fx * rz2, fy_rz2 = fy * rz2, rz3 = rz2 * rz;
    const V3<S> vt{-fx_rz2 * vJ.m[2][0], -fy_rz2 * vJ.m[2][1],
                   -fx_rz2 * vJ.m[0][0] + 2.f * fx * pv.x * rz3 * vJ.m[2][0] -
                       fy_rz2 * vJ.m[1][1] + 2.f * fy * pv.y * rz3 * vJ.m[2][1]};
    v_mean.x += dot3(vt, V3<S>{W.m[0][0], W.m[0][1], W.m[0][2]});
    v_mean.y += dot3(vt, V3<S>{W.m[1][0], W.m[1][1], W.m[1][2]});
    v_mean.z += dot3(vt, V3<S>{W.m[2][0], W.m[2][1], W.m[2][2]});
}

// .metal:1409-1452 (derivative w.r.t. the normalised components).
template <class S>
inline void quat_to_rotmat_vjp(const S* q, const Mat3<S>& vR, S* out) {
    const S s = S(1.f) / msqrt(q[3] * q[3] + q[0] * q[0] + q[1] * q[1] + q[2] * q[2]);
    const S w = q[0] * s, x = q[1] * s, y = q[2] * s, z = q[3] * s;
    const auto& R = vR.m;
    out[0] = 2.f * (x * (R[1][2] - R[2][1]) + y * (R[2][0] - R[0][2]) + z * (R[0][1] - R[1][0]));
    out[1] = 2.f * (-2.f * x * (R[1][1] + R[2][2]) + y * (R[0][1] + R[1][0]) +
                    z * (R[0][2] + R[2][0]) + w * (R[1][2] - R[2][1]));
    out[2] = 2.f * (x * (R[0][1] + R[1][0]) - 2.f * y * (R[0][0] + R[2][2]) +
                    z * (R[1][2] + R[2][1]) + w * (R[2][0] - R[0][2]));
    out[3] = 2.f * (x * (R[0][2] + R[2][0]) + y * (R[1][2] + R[2][1]) -
                    2.f * z * (R[0][0] + R[1][1]) + w * (R[0][1] - R[1][0]));
}

// .metal:1498-1531.
template <class S>
inline void scale_rot_to_cov3d_vjp(const S* s3, float glob, const S* q,
                                   const S* v_cov3d, S* v_scale, S* v_quat) {
    Mat3<S> vV;
    vV.m[0][0] = v_cov3d[0]; vV.m[0][1] = 0.5f * v_cov3d[1]; vV.m[0][2] = 0.5f * v_cov3d[2];
    vV.m[1][0] = 0.5f * v_cov3d[1]; vV.m[1][1] = v_cov3d[3]; vV.m[1][2] = 0.5f * v_cov3d[4];
    vV.m[2][0] = 0.5f * v_cov3d[2]; vV.m[2][1] = 0.5f * v_cov3d[4]; vV.m[2][2] = v_cov3d[5];
    const Mat3<S> R = quat_to_rotmat(q);
    Mat3<S> Sc{};
    Sc.m[0][0] = glob * s3[0]; Sc.m[1][1] = glob * s3[1]; Sc.m[2][2] = glob * s3[2];
    const Mat3<S> M = mat_mul(R, Sc);
    Mat3<S> vM = mat_mul(vV, M);
    for (int i = 0; i < 3; ++i) for (int j = 0; j < 3; ++j) vM.m[i][j] = 2.f * vM.m[i][j];
    for (int i = 0; i < 3; ++i)
        v_scale[i] = dot3(V3<S>{R.m[i][0], R.m[i][1], R.m[i][2]}, V3<S>{vM.m[i][0], vM.m[i][1], vM.m[i][2]});
    const Mat3<S> vR = mat_mul(vM, Sc);
    quat_to_rotmat_vjp(q, vR, v_quat);
}

// .metal:1791-1800.
inline void adam_elem(float& p, float& m, float& v, float g, float step, float b1, float b2,
                      float bc2, float eps) {
    const float mn = std::fma(b1, m, (1.0f - b1) * g);
    const float vn = std::fma(b2, v, (1.0f - b2) * g * g);
    p -= step * mn / (std::sqrt(vn) / bc2 + eps);
    m = mn;
    v = vn;
}

// ---------------- rasterization core ----------------

struct Entry { float x, y, a, b, c, o, r, g, bl; int id; };

// Work counters of the last orc_rasterize call: (pixel, entry) pairs tested,
// pairs with sigma in [0, 5.55), pairs that composite (forward) or carry a
// gradient (backward).  Used only to state the algorithmic work of a step.
struct Counts { int64_t e = 0, r = 0, s = 0; };
Counts g_fwd_counts, g_bwd_counts;

// Forward over entries [s, e) for one pixel with local transmittance start 1
// (.metal:510-572 / 2691-2731).  Returns T; fills C and last.
inline float raster_pixel_fwd(const Entry* ent, int s, int e, float px, float py, float* C,
                              int* last, Counts* cnt) {
    float T = 1.f;
    C[0] = C[1] = C[2] = 0.f;
    int lc = s - 1;
    for (int i = s; i < e; ++i) {
        const Entry& en = ent[i];
        ++cnt->e;
        const float dx = en.x - px, dy = en.y - py;
        const float sigma = std::fma(0.5f, std::fma(en.a, dx * dx, en.c * dy * dy), en.b * dx * dy);
        if (!(sigma < 0.f || sigma >= 5.55f)) ++cnt->r;
        float su;
        if (!sigma_in(sigma, en.o, &su)) continue;
        const float alpha = std::fmin(0.999f, en.o * oexp_raster(-su));
        if (alpha < 1.f / 255.f) continue;
        const float next_T = T * (1.f - alpha);
        if (next_T <= 1e-4f) { lc = i - 1; break; }
        ++cnt->s;
        const float vis = alpha * T;
        const float rgb[3] = {std::fmax(en.r + 0.5f, 0.f), std::fmax(en.g + 0.5f, 0.f),
                              std::fmax(en.bl + 0.5f, 0.f)};
        for (int c = 0; c < 3; ++c) C[c] = std::fma(rgb[c], vis, C[c]);
        T = next_T;
        lc = i;
    }
    *last = lc;
    return T;
}

// Optional error-bound accumulators of the raster backward, per entry:
// mag[i*9+q] = sum over the entry's pairs of the magnitude of gradient term q
// (the term with every signed quantity replaced by the sum of the absolute
// values it is formed from), err[i*9+q] = the same weighted by the term's
// two-sided relative error bound in units of u (below), quad[i] = bit set of
// the tile's 8x8 quadrants with at least one pair carrying a gradient.
struct BwdBounds { float* mag; float* err; uint8_t* quad; };

// Backward over entries [s, bin_final] for one pixel, back to front
// (.metal:1015-1096 / 2963-3028).  Accumulates per-entry gradients into acc[i*9..].
//
// Error bounds (bb != NULL).  The GPU kernel evaluates the same pairs with
// the same alpha (bit-identical forward) but its own arithmetic: the
// transmittance is recovered with a hardware reciprocal (1 ulp) instead of a
// division, the colour behind is carried as E = sum_k v_out_k B_k + sum_k
// v_out_k T_final bg_k instead of per channel, and v_xy / v_conic come from
// moments of v_sigma (sum v dx, sum v dy, ...) formed with the conic once per
// gaussian.  At the d-th pair with a gradient of a pixel's walk (d = 1 at the
// walk's first), first-order bounds on the relative difference of the two
// evaluations, in units of u = 2^-24:
//   T:     7 d   (1 - alpha rounded once, reciprocal 2 + division 1, product
//                 1 + 1, accumulated over the walk from the exact T_final)
//   fac = alpha T:             7 d + 2
//   E, or v_out . B:           8 d + 6 relative to E_mag = sum_k |v_out_k|
//                              (B_k + |T_final bg_k|), B_k >= 0
//   v_alpha:                   8 d + 15 relative to
//                              mva = T sum_k r_k |v_out_k| + ra E_mag
//   v_sigma = -alpha v_alpha:  8 d + 17
//   the nine terms:            <= 8 d + 24 relative to their magnitudes
//                              (v_sigma mag alpha mva times |a dx| + |b dy|,
//                              dx^2 / 2 ..., fac |v_out_k|, |1 - o|)
// so err accumulates (8 d + 24) x magnitude; the per-gaussian summation of
// the terms adds (n_w + 10) x the gaussian's total magnitude (done by the
// caller): a tree of at most 10 levels inside a wave plus n_w float atomics,
// one per 8x8 quadrant and entry with a gradient.
inline void raster_pixel_bwd(const Entry* ent, int s, int bin_final, float px, float py,
                             float T, const float* buf0, float T_final, const float* bg,
                             const float* v_out, double* acc, int acc_base, Counts* cnt,
                             const BwdBounds* bb = nullptr, int quad = 0) {
    float buffer[3] = {buf0[0], buf0[1], buf0[2]};
    const float Tfb[3] = {T_final * bg[0], T_final * bg[1], T_final * bg[2]};
    const double tb_mag = std::fabs((double)Tfb[0] * v_out[0]) + std::fabs((double)Tfb[1] * v_out[1]) +
                          std::fabs((double)Tfb[2] * v_out[2]);
    int d = 0;
    for (int i = bin_final; i >= s; --i) {
        const Entry& en = ent[i];
        ++cnt->e;
        const float opac = en.o;
        const float dx = en.x - px, dy = en.y - py;
        const float sigma = std::fma(0.5f, std::fma(en.a, dx * dx, en.c * dy * dy), en.b * dx * dy);
        if (!(sigma < 0.f || sigma >= 5.55f)) ++cnt->r;
        float su;
        if (!sigma_in(sigma, opac, &su)) continue;
        const float vis = oexp_raster(-su);
        const float alpha = std::fmin(0.999f, opac * vis);
        if (alpha < 1.f / 255.f) continue;
        if (!(alpha < 0.999f)) continue;
        ++cnt->s;
        const float ra = 1.f / (1.f - alpha);
        T *= ra;
        const float fac = alpha * T;
        const float rawc[3] = {en.r, en.g, en.bl};
        float v_alpha = 0.f;
        float t3[3];
        for (int c = 0; c < 3; ++c) {
            const float rgb = std::fmax(rawc[c] + 0.5f, 0.f);
            t3[c] = std::fma(rgb, T, std::fma(-buffer[c], ra, -ra * Tfb[c]));
        }
        v_alpha += t3[0] * v_out[0] + t3[1] * v_out[1] + t3[2] * v_out[2];
        for (int c = 0; c < 3; ++c) {
            const float rgb = std::fmax(rawc[c] + 0.5f, 0.f);
            buffer[c] = std::fma(rgb, fac, buffer[c]);
        }
        const float v_sigma = -alpha * v_alpha;
        if (bb) {
            ++d;
            // buffer[] already holds this pair's colour: the magnitude uses the
            // colour behind it, as v_alpha does
            double rv = 0.0, eb = tb_mag;
            for (int c = 0; c < 3; ++c) {
                const double rgb = std::fmax(rawc[c] + 0.5f, 0.f);
                rv += rgb * std::fabs(v_out[c]);
                eb += std::fabs(v_out[c]) * std::fmax(0.0, (double)buffer[c] - rgb * fac);
            }
            const double mva = (double)T * rv + (double)ra * eb;
            const double vsm = (double)alpha * mva;
            const double adx = std::fabs(dx), ady = std::fabs(dy);
            double tm[9];
            tm[0] = vsm * (std::fabs(en.a) * adx + std::fabs(en.b) * ady);
            tm[1] = vsm * (std::fabs(en.b) * adx + std::fabs(en.c) * ady);
            tm[2] = 0.5 * vsm * adx * adx;
            tm[3] = 0.5 * vsm * adx * ady;
            tm[4] = 0.5 * vsm * ady * ady;
            for (int c = 0; c < 3; ++c)
                tm[5 + c] = rawc[c] + 0.5f >= 0.f ? (double)fac * std::fabs(v_out[c]) : 0.0;
            tm[8] = vsm * std::fabs(1.0 - (double)opac);
            const double w = 8.0 * d + 24.0;
            float* bm = bb->mag + (size_t)(i - acc_base) * 9;
            float* be = bb->err + (size_t)(i - acc_base) * 9;
            for (int q = 0; q < 9; ++q) {
                bm[q] += (float)tm[q];
                be[q] += (float)(w * tm[q]);
            }
            bb->quad[i - acc_base] |= (uint8_t)(1u << quad);
        }
        double* a = acc + (size_t)(i - acc_base) * 9;
        // v_xy (2), v_conic (3), v_rgb (3), v_opacity (1)
        a[0] += v_sigma * std::fma(en.a, dx, en.b * dy);
        a[1] += v_sigma * std::fma(en.b, dx, en.c * dy);
        const float hv = 0.5f * v_sigma;
        a[2] += hv * (dx * dx);
        a[3] += hv * (dx * dy);
        a[4] += hv * (dy * dy);
        for (int c = 0; c < 3; ++c)
            if (rawc[c] + 0.5f >= 0.f) a[5 + c] += fac * v_out[c];
        a[8] += -v_sigma * (1.f - opac);
    }
}

}  // namespace

// ======================================================================
// Per-stage wall time of orc_train_step, under the reference profiler's
// train stage names (msplat_metal.mm:30-34): blit_zero, proj_sh_fwd,
// prefix_sort_pack, rast_fwd, loss_fwd_bwd, rast_bwd, proj_sh_bwd_adam,
// grad_stats (blit_zero stays 0: the buffers are zeroed as they are made).
double g_stage_ms[8] = {};
int64_t g_stage_steps = 0;
struct StageClock {
    std::chrono::steady_clock::time_point t = std::chrono::steady_clock::now();
    void lap(int stage) {
        const auto now = std::chrono::steady_clock::now();
        g_stage_ms[stage] += std::chrono::duration<double, std::milli>(now - t).count();
        t = now;
    }
    ~StageClock() { ++g_stage_steps; }
};

extern "C" {

uint32_t orc_version(void) { return 1; }

void orc_stage_times(double ms[8], int64_t* steps) {
    for (int i = 0; i < 8; ++i) { ms[i] = g_stage_ms[i]; g_stage_ms[i] = 0.0; }
    if (steps) *steps = g_stage_steps;
    g_stage_steps = 0;
}

int32_t orc_num_threads(void) {
#ifdef _OPENMP
    return omp_get_max_threads();
#else
    return 1;
#endif
}

float orc_expf(float x) { return oexp(x); }
float orc_expf_raster(float x) { return oexp_raster(x); }
void orc_expf_raster_n(int64_t n, const float* x, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = oexp_raster(x[i]);
}
void orc_expf_n(int64_t n, const float* x, float* y) {
    for (int64_t i = 0; i < n; ++i) y[i] = oexp(x[i]);
}

void orc_raster_counts(int64_t out[6]) {
    out[0] = g_fwd_counts.e; out[1] = g_fwd_counts.r; out[2] = g_fwd_counts.s;
    out[3] = g_bwd_counts.e; out[4] = g_bwd_counts.r; out[5] = g_bwd_counts.s;
}

void orc_sh_consts(float out[25]) {
    out[0] = SH_C0; out[1] = SH_C1;
    for (int i = 0; i < 5; ++i) out[2 + i] = SH_C2[i];
    for (int i = 0; i < 7; ++i) out[7 + i] = SH_C3[i];
    for (int i = 0; i < 9; ++i) out[14 + i] = SH_C4[i];
    out[23] = out[24] = 0.f;
}

void orc_gauss1d(float out[11]) { for (int i = 0; i < 11; ++i) out[i] = GAUSS_1D[i]; }

void orc_quat_to_rotmat(const float q[4], float R[9]) {
    const M3 M = quat_to_rotmat(q);
    for (int r = 0; r < 3; ++r) for (int c = 0; c < 3; ++c) R[r * 3 + c] = M.m[c][r];
}

void orc_cov3d(const float scale[3], float glob, const float q[4], float cov[6]) {
    scale_rot_to_cov3d(scale, glob, q, cov);
}

void orc_sh_eval(int degree, const float dir[3], const float* dc, const float* rest, float color[3]) {
    sh_coeffs_to_color(degree, F3{dir[0], dir[1], dir[2]}, dc, rest, color);
}

void orc_tile_rect(const OrcCamera* cam, const float xy[2], const float ext[2], int32_t rect[4]) {
    int r[4];
    tile_bbox(xy, ext, tiles_x(cam), tiles_y(cam), r);
    for (int i = 0; i < 4; ++i) rect[i] = r[i];
}

// .metal:1695-1787.  Culled gaussians get radii = num_tiles_hit = 0 and their
// other outputs are left untouched (as in the reference).
void orc_project_forward(const OrcCamera* cam, int32_t N, const float* means,
                         const float* scales, const float* quats, const float* f_dc,
                         const float* f_rest, float* xys, float* depths, int32_t* radii,
                         float* conics, int32_t* num_tiles_hit, float* colors, float* aabb) {
    const int W = cam->width, H = cam->height;
    const int tbx = tiles_x(cam), tby = tiles_y(cam);
    const int rest_per = (num_sh_bases(cam->degree) - 1) * 3;
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < N; ++g) {
        radii[g] = 0;
        num_tiles_hit[g] = 0;
        const F3 pw{means[3 * g], means[3 * g + 1], means[3 * g + 2]};
        const F3 pv = transform_4x3(cam->viewmat, pw);
        if (pv.z <= cam->clip_thresh) continue;
        const float sc[3] = {oexp(scales[3 * g]), oexp(scales[3 * g + 1]), oexp(scales[3 * g + 2])};
        float cov3d[6];
        scale_rot_to_cov3d(sc, cam->glob_scale, quats + 4 * g, cov3d);
        const float tan_fovx = 0.5f * (float)W / cam->fx;
        const float tan_fovy = 0.5f * (float)H / cam->fy;
        const F3 cov2d = project_cov3d_ewa(cov3d, cam->viewmat, cam->fx, cam->fy, tan_fovx,
                                           tan_fovy, pv);
        F3 conic;
        float radius;
        if (!compute_cov2d_bounds(cov2d, conic, radius)) continue;
        conics[3 * g] = conic.x; conics[3 * g + 1] = conic.y; conics[3 * g + 2] = conic.z;
        float center[2];
        project_pix(cam->projmat, pw, W, H, cam->cx, cam->cy, center);
        const float ext[2] = {std::ceil(3.0f * std::sqrt(cov2d.x)), std::ceil(3.0f * std::sqrt(cov2d.z))};
        int r[4];
        tile_bbox(center, ext, tbx, tby, r);
        const int area = (r[2] - r[0]) * (r[3] - r[1]);
        if (area <= 0) continue;
        num_tiles_hit[g] = area;
        depths[g] = pv.z;
        radii[g] = f2i(radius);
        xys[2 * g] = center[0]; xys[2 * g + 1] = center[1];
        aabb[2 * g] = ext[0]; aabb[2 * g + 1] = ext[1];
        const F3 dir = view_dir(means + 3 * g, cam->cam_pos);
        sh_coeffs_to_color(std::min(cam->degrees_to_use, cam->degree), dir, f_dc + 3 * g, f_rest + (size_t)rest_per * g,
                           colors + 3 * g);
    }
}

int64_t orc_bin_sort(const OrcCamera* cam, int32_t N, const float* xys, const float* depths,
                     const int32_t* radii, const float* aabb, int64_t cap,
                     int32_t* tile_counts, int32_t* tile_bins, int32_t* gaussian_ids) {
    const int tbx = tiles_x(cam), tby = tiles_y(cam), T = tbx * tby;
    // Per-tile key lists (scatter_to_prealloc_bins without the 2048 cap).
    std::vector<std::vector<uint64_t>> bins(T);
    for (int32_t g = 0; g < N; ++g) {
        if (radii[g] <= 0) continue;
        int r[4];
        tile_bbox(xys + 2 * g, aabb + 2 * g, tbx, tby, r);
        const uint64_t key = ((uint64_t)float_to_bits(depths[g]) << 32) | (uint64_t)(uint32_t)g;
        for (int ty = r[1]; ty < r[3]; ++ty)
            for (int tx = r[0]; tx < r[2]; ++tx) bins[(size_t)ty * tbx + tx].push_back(key);
    }
    // prefix_sum_kernel: inclusive scan of counts gives each tile's end.
    int64_t total = 0;
    for (int t = 0; t < T; ++t) {
        const int64_t cnt = (int64_t)bins[t].size();
        if (tile_counts) tile_counts[t] = (int32_t)cnt;
        tile_bins[2 * t] = (int32_t)total;
        total += cnt;
        tile_bins[2 * t + 1] = (int32_t)total;
    }
    if (total > cap) return -1;
    // bitonic_sort_per_tile: ascending (depth_bits, gid).
#pragma omp parallel for schedule(dynamic, 16)
    for (int t = 0; t < T; ++t) {
        std::vector<uint64_t>& b = bins[t];
        std::sort(b.begin(), b.end());
        const int s = tile_bins[2 * t];
        for (size_t i = 0; i < b.size(); ++i) gaussian_ids[s + i] = (int32_t)(b[i] & 0xFFFFFFFFu);
    }
    return total;
}

int32_t orc_tile_chunks(int32_t n, int32_t num_tiles) {
    if (n <= 0) return 1;
    const bool chunk_mode = num_tiles < CHUNK_MODE_TILES;
    if (chunk_mode || n > MONO_MAX) return (n + CHUNK - 1) / CHUNK;
    return 1;
}

}  // extern "C"

namespace {

// orc_rasterize, plus (mag9 / err9 != NULL, backward only) the per-gaussian
// magnitudes and error bounds of the nine raster gradients (BwdBounds):
// mag9[g*9+q] = sum of the term magnitudes, err9[g*9+q] = the two-sided bound
// on |GPU - oracle| in units of u = 2^-24, both in the order v_xy (2),
// v_conic (3), v_rgb (3), v_opacity (1).
void rasterize_impl(const OrcCamera* cam, int32_t N, const float* xys, const float* conics,
                    const float* colors, const float* opacity_logits, const int32_t* tile_bins,
                    const int32_t* gaussian_ids, float* final_Ts, int32_t* final_index,
                    float* out_img, const float* v_out, float* v_xy, float* v_conic,
                    float* v_rgb, float* v_opacity, double* mag9, double* err9) {
    const int W = cam->width, H = cam->height;
    const int tbx = tiles_x(cam), tby = tiles_y(cam), T = tbx * tby;
    const int64_t I = tile_bins[2 * (T - 1) + 1];
    const float* bg = cam->background;

    // Packed entries (bitonic_sort_per_tile pack, .metal:2128-2137).
    std::vector<Entry> ent((size_t)I);
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < I; ++i) {
        const int g = gaussian_ids[i];
        Entry& e = ent[i];
        e.x = xys[2 * g]; e.y = xys[2 * g + 1];
        e.a = conics[3 * g]; e.b = conics[3 * g + 1]; e.c = conics[3 * g + 2];
        e.o = sigmoid(opacity_logits[g]);
        e.r = colors[3 * g]; e.g = colors[3 * g + 1]; e.bl = colors[3 * g + 2];
        e.id = g;
    }
    std::vector<double> acc;
    if (v_out) acc.assign((size_t)I * 9, 0.0);
    std::vector<float> bmag, berr;
    std::vector<uint8_t> bquad;
    BwdBounds bbs{nullptr, nullptr, nullptr};
    const BwdBounds* bb = nullptr;
    if (v_out && mag9 && err9) {
        bmag.assign((size_t)I * 9, 0.f);
        berr.assign((size_t)I * 9, 0.f);
        bquad.assign((size_t)I, 0);
        bbs = BwdBounds{bmag.data(), berr.data(), bquad.data()};
        bb = &bbs;
    }
    int64_t fe = 0, fr = 0, fs = 0, be = 0, br = 0, bs = 0;

#pragma omp parallel for schedule(dynamic, 4) reduction(+ : fe, fr, fs, be, br, bs)
    for (int t = 0; t < T; ++t) {
        Counts cf, cbk;
        const int s = tile_bins[2 * t], e = tile_bins[2 * t + 1], n = e - s;
        const int K = orc_tile_chunks(n, T);
        const int tx0 = (t % tbx) * BLOCK, ty0 = (t / tbx) * BLOCK;
        std::vector<float> cT(K), cC(3 * K), pT(K), aC(3 * K);
        std::vector<int> cidx(K);
        for (int ly = 0; ly < BLOCK; ++ly) {
            for (int lx = 0; lx < BLOCK; ++lx) {
                const int i = ty0 + ly, j = tx0 + lx;
                if (i >= H || j >= W) continue;
                const float px = (float)j, py = (float)i;
                const size_t pix = (size_t)i * W + j;
                float Tfin, Cfin[3];
                int last;
                if (K == 1) {
                    Tfin = raster_pixel_fwd(ent.data(), s, e, px, py, Cfin, &last, &cf);
                } else {
                    for (int k = 0; k < K; ++k) {
                        const int cs = s + k * CHUNK, ce = std::min(s + (k + 1) * CHUNK, e);
                        cT[k] = raster_pixel_fwd(ent.data(), cs, ce, px, py, &cC[3 * k], &cidx[k], &cf);
                    }
                    // rasterize_forward_merge_kernel (.metal:2764-2799)
                    float Tr = 1.f, Cr[3] = {0.f, 0.f, 0.f};
                    int li = -1, cutoff = K;
                    for (int k = 0; k < K; ++k) {
                        const int ck = cidx[k];
                        if (ck < 0 && k > 0) break;
                        for (int c = 0; c < 3; ++c) Cr[c] = std::fma(cC[3 * k + c], Tr, Cr[c]);
                        Tr *= cT[k];
                        if (ck >= 0) li = ck;
                        if (Tr <= 1e-4f) { cutoff = k + 1; break; }
                    }
                    for (int k = cutoff; k < K; ++k) cidx[k] = -1;
                    Tfin = Tr;
                    Cfin[0] = Cr[0]; Cfin[1] = Cr[1]; Cfin[2] = Cr[2];
                    last = li;
                }
                final_Ts[pix] = Tfin;
                final_index[pix] = last;
                for (int c = 0; c < 3; ++c) out_img[3 * pix + c] = clampf(std::fma(bg[c], Tfin, Cfin[c]), 0.f, 1.f);

                if (!v_out) continue;
                const float* vo = v_out + 3 * pix;
                const int quad = ((ly >> 3) << 1) | (lx >> 3);   // the 8x8 quadrant (one GPU wave)
                if (K == 1) {
                    const float zero[3] = {0.f, 0.f, 0.f};
                    raster_pixel_bwd(ent.data(), s, last, px, py, Tfin, zero, Tfin, bg, vo,
                                     acc.data(), 0, &cbk, bb, quad);
                } else {
                    // compute_chunk_prefix_suffix_kernel (.metal:2820-2839)
                    float p = 1.f;
                    for (int k = 0; k < K; ++k) { pT[k] = p; p *= cT[k]; }
                    float a3[3] = {0.f, 0.f, 0.f};
                    for (int k = K - 1; k >= 0; --k) {
                        for (int c = 0; c < 3; ++c) aC[3 * k + c] = a3[c];
                        for (int c = 0; c < 3; ++c) a3[c] += pT[k] * cC[3 * k + c];
                    }
                    // rasterize_backward_chunked_kernel (.metal:2884-3028)
                    for (int k = 0; k < K; ++k) {
                        const int cs = s + k * CHUNK, ce = std::min(s + (k + 1) * CHUNK, e);
                        const int bf = cidx[k];
                        if (cs >= ce || bf < cs) continue;
                        raster_pixel_bwd(ent.data(), cs, std::min(bf, ce - 1), px, py,
                                         pT[k] * cT[k], &aC[3 * k], Tfin, bg, vo, acc.data(), 0, &cbk,
                                         bb, quad);
                    }
                }
            }
        }
        fe += cf.e; fr += cf.r; fs += cf.s;
        be += cbk.e; br += cbk.r; bs += cbk.s;
    }
    g_fwd_counts.e = fe; g_fwd_counts.r = fr; g_fwd_counts.s = fs;
    g_bwd_counts.e = be; g_bwd_counts.r = br; g_bwd_counts.s = bs;
    if (!v_out) return;
    // Fixed-order reduction of per-entry gradients into per-gaussian gradients.
    std::vector<double> g9((size_t)N * 9, 0.0);
    for (int64_t i = 0; i < I; ++i) {
        const int g = ent[i].id;
        for (int q = 0; q < 9; ++q) g9[(size_t)g * 9 + q] += acc[(size_t)i * 9 + q];
    }
    for (int32_t g = 0; g < N; ++g) {
        const double* a = &g9[(size_t)g * 9];
        v_xy[2 * g] = (float)a[0]; v_xy[2 * g + 1] = (float)a[1];
        v_conic[3 * g] = (float)a[2]; v_conic[3 * g + 1] = (float)a[3]; v_conic[3 * g + 2] = (float)a[4];
        v_rgb[3 * g] = (float)a[5]; v_rgb[3 * g + 1] = (float)a[6]; v_rgb[3 * g + 2] = (float)a[7];
        v_opacity[g] = (float)a[8];
    }
    if (!bb) return;
    std::fill(mag9, mag9 + (size_t)N * 9, 0.0);
    std::fill(err9, err9 + (size_t)N * 9, 0.0);
    std::vector<int32_t> nw((size_t)N, 0);
    for (int64_t i = 0; i < I; ++i) {
        const int g = ent[i].id;
        nw[g] += __builtin_popcount(bquad[i]);
        for (int q = 0; q < 9; ++q) {
            mag9[(size_t)g * 9 + q] += bmag[(size_t)i * 9 + q];
            err9[(size_t)g * 9 + q] += berr[(size_t)i * 9 + q];
        }
    }
    for (int32_t g = 0; g < N; ++g)
        for (int q = 0; q < 9; ++q) err9[(size_t)g * 9 + q] += (nw[g] + 10.0) * mag9[(size_t)g * 9 + q];
}

}  // namespace

extern "C" {

void orc_rasterize(const OrcCamera* cam, int32_t N, const float* xys, const float* conics,
                   const float* colors, const float* opacity_logits, const int32_t* tile_bins,
                   const int32_t* gaussian_ids, float* final_Ts, int32_t* final_index,
                   float* out_img, const float* v_out, float* v_xy, float* v_conic,
                   float* v_rgb, float* v_opacity) {
    rasterize_impl(cam, N, xys, conics, colors, opacity_logits, tile_bins, gaussian_ids, final_Ts,
                   final_index, out_img, v_out, v_xy, v_conic, v_rgb, v_opacity, nullptr, nullptr);
}

double orc_ssim_loss(int32_t H, int32_t W, const float* img, const float* gt, float w_ssim,
                     float inv_n, float* v_rendered, float* h_buf_out, float* deriv_out) {
    const size_t P = (size_t)H * W;
    // ssim_h_fwd (.metal:3094-3114): horizontal zero-padded sums.
    std::vector<float> hb(P * 15);
#pragma omp parallel for schedule(static)
    for (int y = 0; y < H; ++y) {
        for (int x = 0; x < W; ++x) {
            for (int c = 0; c < 3; ++c) {
                float mx = 0, my = 0, sx = 0, sy = 0, cxy = 0;
                for (int d = 0; d < 11; ++d) {
                    const int xx = x - 5 + d;
                    float gv = 0.f, rv = 0.f;
                    if (xx >= 0 && xx < W) {
                        gv = gt[((size_t)y * W + xx) * 3 + c];
                        rv = img[((size_t)y * W + xx) * 3 + c];
                    }
                    // one fma per window term, (w gv) gv as a product then an
                    // fma: the reference's w * gv * gv with the sum contracted
                    // as its fast-math Metal build may do (and the kernels do)
                    const float w = GAUSS_1D[d];
                    const float wg = w * gv, wr = w * rv;
                    mx = std::fma(w, gv, mx); my = std::fma(w, rv, my);
                    sx = std::fma(wg, gv, sx); sy = std::fma(wr, rv, sy);
                    cxy = std::fma(wg, rv, cxy);
                }
                float* o = &hb[((size_t)y * W + x) * 15 + c * 5];
                o[0] = mx; o[1] = my; o[2] = sx; o[3] = sy; o[4] = cxy;
            }
        }
    }
    if (h_buf_out) std::memcpy(h_buf_out, hb.data(), P * 15 * sizeof(float));

    // ssim_fused_v_fwd_h_bwd (.metal:3243-3300).  Derivative fields exist for
    // centre columns x in [-5, W+5): outside the image the stats are zero.
    const int WE = W + 10;
    std::vector<float> F((size_t)H * WE * 9);   // [y][x+5][c*3 + f]
    std::vector<double> row_loss(H, 0.0);
#pragma omp parallel for schedule(static)
    for (int y = 0; y < H; ++y) {
        double rl = 0.0;
        for (int xe = 0; xe < WE; ++xe) {
            const int x = xe - 5;
            float ssim_sum = 0.f, l1_sum = 0.f;
            for (int c = 0; c < 3; ++c) {
                float mx = 0, my = 0, sx = 0, sy = 0, cxy = 0;
                for (int k = 0; k < 11; ++k) {
                    const int yy = y - 5 + k;
                    float h[5] = {0, 0, 0, 0, 0};
                    if (x >= 0 && x < W && yy >= 0 && yy < H)
                        for (int f = 0; f < 5; ++f) h[f] = hb[((size_t)yy * W + x) * 15 + c * 5 + f];
                    const float w = GAUSS_1D[k];
                    mx = std::fma(w, h[0], mx); my = std::fma(w, h[1], my);
                    sx = std::fma(w, h[2], sx); sy = std::fma(w, h[3], sy);
                    cxy = std::fma(w, h[4], cxy);
                }
                const float sxs = sx - mx * mx, sys = sy - my * my, sxy = cxy - mx * my;
                const float A = 2.0f * mx * my + SSIM_C1, B = 2.0f * sxy + SSIM_C2;
                const float Cd = mx * mx + my * my + SSIM_C1, D = sxs + sys + SSIM_C2;
                const float iCD = 1.0f / (Cd * D);
                const float dmu = 2.0f * B * (mx * Cd - A * my) / (Cd * Cd * D);
                const float dsyq = -A * B * iCD / D, dsxy = 2.0f * A * iCD;
                float* f = &F[((size_t)y * WE + xe) * 9 + c * 3];
                f[0] = dmu - 2.0f * my * dsyq - mx * dsxy;
                f[1] = 2.0f * dsyq;
                f[2] = dsxy;
                if (x >= 0 && x < W) {
                    ssim_sum += (A * B) / (Cd * D);
                    l1_sum += std::fabs(gt[((size_t)y * W + x) * 3 + c] - img[((size_t)y * W + x) * 3 + c]);
                }
            }
            if (x >= 0 && x < W)
                rl += (double)(w_ssim * (1.0f - ssim_sum / 3.0f) + (1.0f - w_ssim) * l1_sum / 3.0f);
        }
        row_loss[y] = rl;
    }
    // H-backward: mirrored window over centre columns x-5 .. x+5.
    std::vector<float> D((size_t)P * 9);
#pragma omp parallel for schedule(static)
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x)
            for (int c = 0; c < 3; ++c) {
                float h1 = 0, h2 = 0, h3 = 0;
                for (int d = 0; d < 11; ++d) {
                    const float w = GAUSS_1D[10 - d];
                    const float* f = &F[((size_t)y * WE + (x + d)) * 9 + c * 3];
                    h1 = std::fma(w, f[0], h1); h2 = std::fma(w, f[1], h2); h3 = std::fma(w, f[2], h3);
                }
                float* o = &D[((size_t)y * W + x) * 9 + c * 3];
                o[0] = h1; o[1] = h2; o[2] = h3;
            }
    if (deriv_out) {
        for (size_t p = 0; p < P; ++p)
            for (int c = 0; c < 3; ++c) {
                deriv_out[p * 15 + c * 5 + 0] = D[p * 9 + c * 3 + 0];
                deriv_out[p * 15 + c * 5 + 1] = D[p * 9 + c * 3 + 1];
                deriv_out[p * 15 + c * 5 + 2] = D[p * 9 + c * 3 + 2];
                deriv_out[p * 15 + c * 5 + 3] = 0.f;
                deriv_out[p * 15 + c * 5 + 4] = 0.f;
            }
    }
    // ssim_v_bwd (.metal:3443-3463): vertical mirrored window, rows outside are zero.
    if (v_rendered) {
#pragma omp parallel for schedule(static)
        for (int y = 0; y < H; ++y)
            for (int x = 0; x < W; ++x)
                for (int c = 0; c < 3; ++c) {
                    float f1 = 0, f2 = 0, f3 = 0;
                    for (int d = 0; d < 11; ++d) {
                        const int yy = y - 5 + d;
                        float a = 0, b = 0, cc = 0;
                        if (yy >= 0 && yy < H) {
                            const float* o = &D[((size_t)yy * W + x) * 9 + c * 3];
                            a = o[0]; b = o[1]; cc = o[2];
                        }
                        const float w = GAUSS_1D[10 - d];
                        f1 = std::fma(w, a, f1); f2 = std::fma(w, b, f2); f3 = std::fma(w, cc, f3);
                    }
                    const size_t q = ((size_t)y * W + x) * 3 + c;
                    const float r = img[q], g = gt[q];
                    const float v_ssim = f1 + r * f2 + g * f3;
                    const float v_l1 = (g > r) ? -1.0f : ((g < r) ? 1.0f : 0.0f);
                    v_rendered[q] = inv_n * (-w_ssim * v_ssim + (1.0f - w_ssim) * v_l1);
                }
    }
    double total = 0.0;
    for (int y = 0; y < H; ++y) total += row_loss[y];
    return total;
}

}  // extern "C"

namespace {

// One gaussian of the projection backward (.metal:1813-1910): mean, the
// exponentiated scales es, quaternion, conic and the raster gradients in;
// v_mean3d, v_scale (w.r.t. the log scale) and v_quat out.
template <class S>
inline void project_backward_one(const OrcCamera* cam, const S* mean, const S* es, const S* q,
                                 const S* conic, const S* v_xy, const S* v_conic, S* v_mean3d,
                                 S* v_scale, S* v_quat) {
    const int W = cam->width, H = cam->height;
    const float fx = cam->fx, fy = cam->fy;
    const float tan_fovx = 0.5f * (float)W / fx, tan_fovy = 0.5f * (float)H / fy;
    const V3<S> pw{mean[0], mean[1], mean[2]};
    V3<S> vm = project_pix_vjp(cam->projmat, pw, W, H, v_xy);
    const float v_z = 0.f;   // v_depth is zero-filled and never written (.mm:1168)
    vm.x = vm.x + cam->viewmat[8] * v_z;
    vm.y = vm.y + cam->viewmat[9] * v_z;
    vm.z = vm.z + cam->viewmat[10] * v_z;
    S v_cov2d[3];
    cov2d_to_conic_vjp(conic, v_conic, v_cov2d);
    S cov3d[6];
    scale_rot_to_cov3d(es, cam->glob_scale, q, cov3d);
    const V3<S> pv = transform_4x3(cam->viewmat, pw);
    S v_cov3d[6];
    project_cov3d_ewa_vjp(cov3d, cam->viewmat, fx, fy, tan_fovx, tan_fovy, v_cov2d, vm, v_cov3d, pv);
    S vs[3], vq[4];
    scale_rot_to_cov3d_vjp(es, cam->glob_scale, q, v_cov3d, vs, vq);
    v_mean3d[0] = vm.x; v_mean3d[1] = vm.y; v_mean3d[2] = vm.z;
    for (int k = 0; k < 3; ++k) v_scale[k] = vs[k] * es[k];
    for (int k = 0; k < 4; ++k) v_quat[k] = vq[k];
}

// Error bounds of the projection backward of gaussian g, by running error
// analysis of project_backward_one (RE).  The inputs (mean, scale, quat,
// conic) are exact: the projection forward is bit-identical on both sides.
// The raster gradients v_xy / v_conic come with magnitudes a_* (sums of
// |contribution|) and two-sided error bounds e_* (in units of u).  Outputs,
// per component of v_mean3d (3), v_scale (3), v_quat (4):
//   a_out = propagation of a_in + the rounding of every operation once
//           (first-order error of one float evaluation whose inputs err by a_in);
//   e_out = propagation of e_in + 4 x the operations' own rounding: the
//           oracle rounds each operation once (u), the GPU kernel up to 3 u
//           (hardware reciprocal and square root of about 1 ulp = 2 u, and
//           x * rcp(z) in place of x / z: 2 u + u).
inline void project_backward_bounds(const OrcCamera* cam, const float* mean, const float* es_f,
                                    const float* q_f, const float* conic_f, const float* vxy,
                                    const float* vconic, const double* a_xy, const double* a_conic,
                                    const double* e_xy, const double* e_conic, double* a_out,
                                    double* e_out) {
    RE m[3], es[3], q[4], cn[3];
    for (int k = 0; k < 3; ++k) { m[k] = RE(mean[k]); es[k] = RE(es_f[k]); cn[k] = RE(conic_f[k]); }
    for (int k = 0; k < 4; ++k) q[k] = RE(q_f[k]);
    auto run = [&](const double* exy, const double* ecn, double* out) {
        RE vx[2] = {RE((double)vxy[0], exy ? exy[0] : 0.0), RE((double)vxy[1], exy ? exy[1] : 0.0)};
        RE vc[3];
        for (int k = 0; k < 3; ++k) vc[k] = RE((double)vconic[k], ecn ? ecn[k] : 0.0);
        RE om[3], os[3], oq[4];
        project_backward_one(cam, m, es, q, cn, vx, vc, om, os, oq);
        for (int k = 0; k < 3; ++k) { out[k] = om[k].e; out[3 + k] = os[k].e; }
        for (int k = 0; k < 4; ++k) out[6 + k] = oq[k].e;
    };
    double ops[10], prop_a[10], prop_e[10];
    run(nullptr, nullptr, ops);
    run(a_xy, a_conic, prop_a);
    run(e_xy, e_conic, prop_e);
    for (int k = 0; k < 10; ++k) {
        a_out[k] = prop_a[k];
        e_out[k] = (prop_e[k] - ops[k]) + 4.0 * ops[k];
    }
}

}  // namespace

extern "C" {

void orc_project_backward_err(const OrcCamera* cam, int32_t N, const float* means,
                              const float* scales, const float* quats, const int32_t* radii,
                              const float* conics, const float* v_xy, const float* v_conic,
                              const float* err_xy, const float* err_conic, float* err_out) {
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < N; ++g) {
        float* o = err_out + (size_t)g * 10;
        if (radii[g] <= 0) {
            for (int k = 0; k < 10; ++k) o[k] = 0.f;
            continue;
        }
        const float es[3] = {oexp(scales[3 * g]), oexp(scales[3 * g + 1]), oexp(scales[3 * g + 2])};
        double ex[2] = {0.0, 0.0}, ec[3] = {0.0, 0.0, 0.0}, pa[10], pe[10];
        for (int k = 0; k < 2; ++k) ex[k] = err_xy ? err_xy[2 * (size_t)g + k] / kU : 0.0;
        for (int k = 0; k < 3; ++k) ec[k] = err_conic ? err_conic[3 * (size_t)g + k] / kU : 0.0;
        project_backward_bounds(cam, means + 3 * g, es, quats + 4 * g, conics + 3 * g, v_xy + 2 * g,
                                v_conic + 3 * g, ex, ec, ex, ec, pa, pe);
        for (int k = 0; k < 10; ++k) o[k] = (float)(pe[k] * kU);
    }
}

void orc_project_backward(const OrcCamera* cam, int32_t N, const float* means,
                          const float* scales, const float* quats, const int32_t* radii,
                          const float* conics, const float* v_xy, const float* v_conic,
                          float* v_mean3d, float* v_scale, float* v_quat) {
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < N; ++g) {
        if (radii[g] <= 0) {
            for (int k = 0; k < 3; ++k) { v_mean3d[3 * g + k] = 0.f; v_scale[3 * g + k] = 0.f; }
            for (int k = 0; k < 4; ++k) v_quat[4 * g + k] = 0.f;
            continue;
        }
        const float es[3] = {oexp(scales[3 * g]), oexp(scales[3 * g + 1]), oexp(scales[3 * g + 2])};
        project_backward_one(cam, means + 3 * g, es, quats + 4 * g, conics + 3 * g, v_xy + 2 * g,
                             v_conic + 3 * g, v_mean3d + 3 * g, v_scale + 3 * g, v_quat + 4 * g);
    }
}

void orc_sh_backward(const OrcCamera* cam, int32_t N, const float* means, const int32_t* radii,
                     const float* v_rgb, float* v_dc, float* v_rest) {
    const int nb = num_sh_bases(cam->degree) - 1;
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < N; ++g) {
        float* vr = v_rest + (size_t)g * nb * 3;
        for (int i = 0; i < nb * 3; ++i) vr[i] = 0.f;
        for (int c = 0; c < 3; ++c) v_dc[3 * g + c] = 0.f;
        if (radii[g] <= 0) continue;
        for (int c = 0; c < 3; ++c) v_dc[3 * g + c] = SH_C0 * v_rgb[3 * g + c];
        const F3 dir = view_dir(means + 3 * g, cam->cam_pos);
        float basis[24];
        const int nbu = std::min(sh_rest_basis(std::min(cam->degrees_to_use, 3), dir, basis), nb);
        for (int b = 0; b < nbu; ++b)
            for (int c = 0; c < 3; ++c) vr[b * 3 + c] = basis[b] * v_rgb[3 * g + c];
    }
}

void orc_adam(int64_t n, float* p, const float* g, float* m, float* v, float step,
              float b1, float b2, float bc2, float eps) {
#pragma omp parallel for schedule(static)
    for (int64_t i = 0; i < n; ++i) adam_elem(p[i], m[i], v[i], g[i], step, b1, b2, bc2, eps);
}

void orc_grad_stats(int32_t N, const int32_t* radii, const float* v_xy, float* vis,
                    float* gnorm, float* max2d, float inv_max_dim) {
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < N; ++g) {
        if (radii[g] <= 0) continue;
        vis[g] += 1.0f;
        const float gx = v_xy[2 * g], gy = v_xy[2 * g + 1];
        gnorm[g] += std::sqrt(gx * gx + gy * gy);
        const float r = (float)radii[g] * inv_max_dim;
        max2d[g] = std::fmax(max2d[g], r);
    }
}

}  // extern "C"

namespace {

// Gradients fed to Adam and their bounds (OrcTrainOut.grad / grad_mag /
// grad_err), from the raster gradients' magnitudes and bounds (units of u):
// means / scales / quats through the running error analysis of the
// projection backward, opacity as the raster's, f_dc = SH_C0 v_rgb and
// f_rest = basis_b(dir) v_rgb (the basis evaluated in RE from the exact view
// direction; each product adds its own rounding, counted 3 x in the
// two-sided bound).  The raster outputs: mag_raster = magnitudes, err_raster
// = absolute bounds.  pb holds means [N,3], scales [N,3], quats [N,4] as the
// step read them.
void train_step_bounds(const OrcCamera* cam, int32_t N, int32_t rest_bases, const float* pb,
                       const int32_t* radii, const float* conics, const float* v_xy,
                       const float* v_conic, const float* v_rgb, const float* v_op,
                       const float* v_mean, const float* v_scale, const float* v_quat,
                       const double* mag9, const double* err9, const OrcTrainOut* out) {
    const float* means = pb;
    const float* scales = pb + (size_t)N * 3;
    const float* quats = pb + (size_t)N * 6;
    const int rp = rest_bases * 3;
    const int dtu = std::min(cam->degrees_to_use, 3);
    const int64_t numel[6] = {3LL * N, 3LL * N, 4LL * N, 3LL * N, (int64_t)rp * N, (int64_t)N};
    for (int gi = 0; gi < 6; ++gi) {
        if (out->grad[gi]) std::fill(out->grad[gi], out->grad[gi] + numel[gi], 0.f);
        if (out->grad_mag[gi]) std::fill(out->grad_mag[gi], out->grad_mag[gi] + numel[gi], 0.f);
        if (out->grad_err[gi]) std::fill(out->grad_err[gi], out->grad_err[gi] + numel[gi], 0.f);
    }
    auto put = [&](int gi, size_t i, float g, double mag, double err_u) {
        if (out->grad[gi]) out->grad[gi][i] = g;
        if (out->grad_mag[gi]) out->grad_mag[gi][i] = (float)mag;
        if (out->grad_err[gi]) out->grad_err[gi][i] = (float)(err_u * kU);
    };
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < N; ++g) {
        const double* a = mag9 + (size_t)g * 9;
        const double* e = err9 + (size_t)g * 9;
        if (out->mag_raster)
            for (int q = 0; q < 9; ++q) out->mag_raster[(size_t)g * 9 + q] = (float)a[q];
        if (out->err_raster)
            for (int q = 0; q < 9; ++q) out->err_raster[(size_t)g * 9 + q] = (float)(e[q] * kU);
        // opacity: the raster's own (dense: every gaussian)
        put(5, g, v_op[g], a[8], e[8]);
        if (radii[g] <= 0) {   // zero gradients, exactly, on both sides
            continue;
        }
        const float es[3] = {oexp(scales[3 * g]), oexp(scales[3 * g + 1]), oexp(scales[3 * g + 2])};
        double pa[10], pe[10];
        project_backward_bounds(cam, means + 3 * g, es, quats + 4 * g, conics + 3 * g, v_xy + 2 * g,
                                v_conic + 3 * g, a, a + 2, e, e + 2, pa, pe);
        for (int k = 0; k < 3; ++k) put(0, 3 * (size_t)g + k, v_mean[3 * g + k], pa[k], pe[k]);
        for (int k = 0; k < 3; ++k) put(1, 3 * (size_t)g + k, v_scale[3 * g + k], pa[3 + k], pe[3 + k]);
        for (int k = 0; k < 4; ++k) put(2, 4 * (size_t)g + k, v_quat[4 * g + k], pa[6 + k], pe[6 + k]);
        for (int c = 0; c < 3; ++c) {
            const float gr = SH_C0 * v_rgb[3 * g + c];
            const double ag = std::fabs((double)gr);
            put(3, 3 * (size_t)g + c, gr, SH_C0 * a[5 + c] + ag, SH_C0 * e[5 + c] + 3.0 * ag);
        }
        if (dtu < 1) continue;
        const F3 dir = view_dir(means + 3 * g, cam->cam_pos);
        float basis[24];
        RE rb[24];
        const int nb = std::min(sh_rest_basis(dtu, dir, basis), rest_bases);
        sh_rest_basis(dtu, V3<RE>{RE(dir.x), RE(dir.y), RE(dir.z)}, rb);
        for (int b = 0; b < nb; ++b)
            for (int c = 0; c < 3; ++c) {
                const float gr = basis[b] * v_rgb[3 * g + c];
                const double ag = std::fabs((double)gr), vr = std::fabs((double)v_rgb[3 * g + c]);
                const double bm = std::fabs(rb[b].v);
                put(4, (size_t)rp * g + b * 3 + c, gr, bm * a[5 + c] + rb[b].e * vr + ag,
                    bm * e[5 + c] + 3.0 * rb[b].e * vr + 3.0 * ag);
            }
    }
}

}  // namespace

extern "C" {

float orc_train_step(const OrcCamera* cam, int32_t N, int32_t rest_bases,
                     float* const params[6], float* const m[6], float* const v[6],
                     const OrcAdam* ad, const float* gt, float ssim_weight, float* vis,
                     float* gnorm, float* max2d, const OrcTrainOut* out) {
    const int W = cam->width, H = cam->height, T = tiles_x(cam) * tiles_y(cam);
    const size_t P = (size_t)H * W;
    const int rp = rest_bases * 3;
    // the bounds of the projection backward need the parameters it read
    std::vector<float> params_before;
    if (out && (out->mag_raster || out->err_raster || out->grad[0])) {
        params_before.resize((size_t)N * 10);
        std::memcpy(params_before.data(), params[0], (size_t)N * 12);
        std::memcpy(params_before.data() + (size_t)N * 3, params[1], (size_t)N * 12);
        std::memcpy(params_before.data() + (size_t)N * 6, params[2], (size_t)N * 16);
    }
    StageClock clk;
    std::vector<float> xys(2 * (size_t)N, 0.f), depths(N, 0.f), conics(3 * (size_t)N, 0.f),
        colors(3 * (size_t)N, 0.f), aabb(2 * (size_t)N, 0.f);
    std::vector<int32_t> radii(N), nth(N);
    orc_project_forward(cam, N, params[0], params[1], params[2], params[3], params[4], xys.data(),
                        depths.data(), radii.data(), conics.data(), nth.data(), colors.data(),
                        aabb.data());
    clk.lap(1);   // proj_sh_fwd
    int64_t cap = 0;
    for (int32_t g = 0; g < N; ++g) cap += nth[g];
    std::vector<int32_t> tile_bins(2 * (size_t)T), ids((size_t)std::max<int64_t>(cap, 1));
    if (orc_bin_sort(cam, N, xys.data(), depths.data(), radii.data(), aabb.data(), cap, nullptr,
                     tile_bins.data(), ids.data()) < 0)
        return std::numeric_limits<float>::quiet_NaN();
    clk.lap(2);   // prefix_sort_pack
    std::vector<float> Ts(P), img(P * 3), v_rendered(P * 3);
    std::vector<int32_t> fidx(P);
    // Forward first (image needed by the loss), backward after the loss.
    orc_rasterize(cam, N, xys.data(), conics.data(), colors.data(), params[5], tile_bins.data(),
                  ids.data(), Ts.data(), fidx.data(), img.data(), nullptr, nullptr, nullptr,
                  nullptr, nullptr);
    clk.lap(3);   // rast_fwd
    const float inv_n = 1.0f / (float)(H * W * 3);
    const double loss_sum = orc_ssim_loss(H, W, img.data(), gt, ssim_weight, inv_n,
                                          v_rendered.data(), nullptr, nullptr);
    clk.lap(4);   // loss_fwd_bwd
    std::vector<float> v_xy(2 * (size_t)N), v_conic(3 * (size_t)N), v_rgb(3 * (size_t)N), v_op(N);
    const bool bounds = out && (out->mag_raster || out->err_raster || out->grad[0]);
    std::vector<double> mag9, err9;
    if (bounds) {
        mag9.assign((size_t)N * 9, 0.0);
        err9.assign((size_t)N * 9, 0.0);
    }
    rasterize_impl(cam, N, xys.data(), conics.data(), colors.data(), params[5], tile_bins.data(),
                   ids.data(), Ts.data(), fidx.data(), img.data(), v_rendered.data(), v_xy.data(),
                   v_conic.data(), v_rgb.data(), v_op.data(), bounds ? mag9.data() : nullptr,
                   bounds ? err9.data() : nullptr);
    clk.lap(5);   // rast_bwd (the backward call recomputes each pixel's forward)
    std::vector<float> v_mean(3 * (size_t)N), v_scale(3 * (size_t)N), v_quat(4 * (size_t)N);
    orc_project_backward(cam, N, params[0], params[1], params[2], radii.data(), conics.data(),
                         v_xy.data(), v_conic.data(), v_mean.data(), v_scale.data(), v_quat.data());
    // Fused SH backward + Adam for groups 3 and 4: visible gaussians only,
    // rest bands up to degrees_to_use (.metal:1912-1985).
    const int dtu = std::min(cam->degrees_to_use, 3);
#pragma omp parallel for schedule(static)
    for (int32_t g = 0; g < N; ++g) {
        if (radii[g] <= 0) continue;
        for (int c = 0; c < 3; ++c) {
            const size_t i = 3 * (size_t)g + c;
            adam_elem(params[3][i], m[3][i], v[3][i], SH_C0 * v_rgb[3 * g + c], ad->step_size[3],
                      ad->beta1, ad->beta2, ad->bc2_sqrt[3], ad->eps);
        }
        if (dtu < 1) continue;
        const F3 dir = view_dir(params[0] + 3 * g, cam->cam_pos);
        float basis[24];
        const int nb = std::min(sh_rest_basis(dtu, dir, basis), rest_bases);
        for (int b = 0; b < nb; ++b)
            for (int c = 0; c < 3; ++c) {
                const size_t i = (size_t)rp * g + b * 3 + c;
                adam_elem(params[4][i], m[4][i], v[4][i], basis[b] * v_rgb[3 * g + c],
                          ad->step_size[4], ad->beta1, ad->beta2, ad->bc2_sqrt[4], ad->eps);
            }
    }
    // Dense Adam for groups 0, 1, 2, 5 (.mm:1117-1138).
    const float* grads[6] = {v_mean.data(), v_scale.data(), v_quat.data(), nullptr, nullptr, v_op.data()};
    const int64_t numel[6] = {3LL * N, 3LL * N, 4LL * N, 0, 0, (int64_t)N};
    for (int gi : {0, 1, 2, 5})
        orc_adam(numel[gi], params[gi], grads[gi], m[gi], v[gi], ad->step_size[gi], ad->beta1,
                 ad->beta2, ad->bc2_sqrt[gi], ad->eps);
    clk.lap(6);   // proj_sh_bwd_adam
    orc_grad_stats(N, radii.data(), v_xy.data(), vis, gnorm, max2d,
                   1.0f / (float)std::max(H, W));
    clk.lap(7);   // grad_stats
    if (bounds)
        train_step_bounds(cam, N, rest_bases, params_before.data(), radii.data(), conics.data(),
                          v_xy.data(), v_conic.data(), v_rgb.data(), v_op.data(), v_mean.data(),
                          v_scale.data(), v_quat.data(), mag9.data(), err9.data(), out);
    if (out) {
        if (out->out_img) std::memcpy(out->out_img, img.data(), P * 3 * sizeof(float));
        if (out->radii) std::memcpy(out->radii, radii.data(), (size_t)N * 4);
        if (out->v_xy) std::memcpy(out->v_xy, v_xy.data(), (size_t)N * 8);
        if (out->v_conic) std::memcpy(out->v_conic, v_conic.data(), (size_t)N * 12);
        if (out->v_rgb) std::memcpy(out->v_rgb, v_rgb.data(), (size_t)N * 12);
        if (out->v_opacity) std::memcpy(out->v_opacity, v_op.data(), (size_t)N * 4);
        if (out->v_mean3d) std::memcpy(out->v_mean3d, v_mean.data(), (size_t)N * 12);
        if (out->v_scale) std::memcpy(out->v_scale, v_scale.data(), (size_t)N * 12);
        if (out->v_quat) std::memcpy(out->v_quat, v_quat.data(), (size_t)N * 16);
        if (out->v_rendered) std::memcpy(out->v_rendered, v_rendered.data(), P * 12);
    }
    return (float)(loss_sum / (double)(H * W));
}

int orc_render(const OrcCamera* cam, int32_t N, const float* means, const float* scales,
               const float* quats, const float* f_dc, const float* f_rest,
               const float* opacity_logits, float* out_img, float* final_Ts,
               int32_t* final_index) {
    const int W = cam->width, H = cam->height, T = tiles_x(cam) * tiles_y(cam);
    const size_t P = (size_t)H * W;
    std::vector<float> xys(2 * (size_t)N, 0.f), depths(N, 0.f), conics(3 * (size_t)N, 0.f),
        colors(3 * (size_t)N, 0.f), aabb(2 * (size_t)N, 0.f);
    std::vector<int32_t> radii(N), nth(N);
    orc_project_forward(cam, N, means, scales, quats, f_dc, f_rest, xys.data(), depths.data(),
                        radii.data(), conics.data(), nth.data(), colors.data(), aabb.data());
    int64_t cap = 0;
    for (int32_t g = 0; g < N; ++g) cap += nth[g];
    std::vector<int32_t> tile_bins(2 * (size_t)T), ids((size_t)std::max<int64_t>(cap, 1));
    if (orc_bin_sort(cam, N, xys.data(), depths.data(), radii.data(), aabb.data(), cap, nullptr,
                     tile_bins.data(), ids.data()) < 0)
        return -1;
    std::vector<float> Ts(P);
    std::vector<int32_t> fidx(P);
    orc_rasterize(cam, N, xys.data(), conics.data(), colors.data(), opacity_logits,
                  tile_bins.data(), ids.data(), final_Ts ? final_Ts : Ts.data(),
                  final_index ? final_index : fidx.data(), out_img, nullptr, nullptr, nullptr,
                  nullptr, nullptr);
    return 0;
}

int32_t orc_densify(const OrcDensifyArgs* a, const float* gnorm, const float* vis,
                    const float* max2d, float* const bufs[6], float* const m[6],
                    float* const v[6], const float* rnd, int32_t* split_out, int32_t* dup_out,
                    int32_t* keep_out) {
    const int N = a->N, fr = a->fr_stride;
    const int strides[6] = {3, 3, 4, 3, fr, 1};
    std::vector<int32_t> split(N), dup(N);
    // densify_classify_kernel (.metal:3490-3508)
    for (int i = 0; i < N; ++i) {
        const float vc = vis[i];
        if (vc <= 0.0f) { split[i] = 0; dup[i] = 0; continue; }
        const float avg = (gnorm[i] / vc) * a->half_max_dim;
        const bool high = avg > a->grad_thresh;
        const float* s = bufs[1] + 3 * (size_t)i;
        const float mx = std::fmax(std::fmax(oexp(s[0]), oexp(s[1])), oexp(s[2]));
        const bool large = mx > a->size_thresh;
        bool do_split = large;
        if (a->check_screen && max2d[i] > a->screen_thresh) do_split = true;
        do_split = do_split && high;
        split[i] = do_split ? 1 : 0;
        dup[i] = (!large && high) ? 1 : 0;
    }
    // Inclusive scans (block_reduce + block_scan_propagate).
    std::vector<int32_t> sp(N), dp(N);
    int32_t acc = 0;
    for (int i = 0; i < N; ++i) { acc += split[i]; sp[i] = acc; }
    acc = 0;
    for (int i = 0; i < N; ++i) { acc += dup[i]; dp[i] = acc; }
    const int nS = N > 0 ? sp[N - 1] : 0, nD = N > 0 ? dp[N - 1] : 0;
    const float lsf = std::log(1.6f);
    // densify_append_split_kernel (.metal:3541-3599)
    for (int i = 0; i < N; ++i) {
        if (!split[i]) continue;
        const int ord = sp[i] - 1;
        const float* q = bufs[2] + 4 * (size_t)i;
        float qw = q[0], qx = q[1], qy = q[2], qz = q[3];
        const float ql = std::sqrt(qw * qw + qx * qx + qy * qy + qz * qz);
        qw /= ql; qx /= ql; qy /= ql; qz /= ql;
        float* sc = bufs[1];
        const float sx = oexp(sc[3 * i]), sy = oexp(sc[3 * i + 1]), sz = oexp(sc[3 * i + 2]);
        for (int k = 0; k < 2; ++k) {
            const int ch = N + 2 * ord + k, ri = ord * 2 + k;
            const float r0 = rnd[3 * ri] * sx, r1 = rnd[3 * ri + 1] * sy, r2 = rnd[3 * ri + 2] * sz;
            const float v0 = (1 - 2 * (qy * qy + qz * qz)) * r0 + 2 * (qx * qy - qw * qz) * r1 + 2 * (qx * qz + qw * qy) * r2;
            const float v1 = 2 * (qx * qy + qw * qz) * r0 + (1 - 2 * (qx * qx + qz * qz)) * r1 + 2 * (qy * qz - qw * qx) * r2;
            const float v2 = 2 * (qx * qz - qw * qy) * r0 + 2 * (qy * qz + qw * qx) * r1 + (1 - 2 * (qx * qx + qy * qy)) * r2;
            float* mb = bufs[0];
            mb[3 * ch] = mb[3 * i] + v0; mb[3 * ch + 1] = mb[3 * i + 1] + v1; mb[3 * ch + 2] = mb[3 * i + 2] + v2;
            for (int j = 0; j < 3; ++j) sc[3 * ch + j] = sc[3 * i + j] - lsf;
            for (int j = 0; j < 4; ++j) bufs[2][4 * ch + j] = bufs[2][4 * i + j];
            for (int j = 0; j < 3; ++j) bufs[3][3 * ch + j] = bufs[3][3 * i + j];
            for (int j = 0; j < fr; ++j) bufs[4][(size_t)fr * ch + j] = bufs[4][(size_t)fr * i + j];
            bufs[5][ch] = bufs[5][i];
            for (int gi = 0; gi < 6; ++gi)
                for (int j = 0; j < strides[gi]; ++j) {
                    m[gi][(size_t)strides[gi] * ch + j] = 0.f;
                    v[gi][(size_t)strides[gi] * ch + j] = 0.f;
                }
        }
        for (int j = 0; j < 3; ++j) sc[3 * i + j] -= lsf;
    }
    // densify_append_dup_kernel (.metal:3630-3650)
    for (int i = 0; i < N; ++i) {
        if (!dup[i]) continue;
        const int dst = N + 2 * nS + dp[i] - 1;
        for (int gi = 0; gi < 6; ++gi)
            for (int j = 0; j < strides[gi]; ++j) {
                bufs[gi][(size_t)strides[gi] * dst + j] = bufs[gi][(size_t)strides[gi] * i + j];
                m[gi][(size_t)strides[gi] * dst + j] = 0.f;
                v[gi][(size_t)strides[gi] * dst + j] = 0.f;
            }
    }
    // densify_cull_classify_kernel (.metal:3672-3693) over the grown set.
    const int Nn = N + 2 * nS + nD;
    std::vector<int32_t> keep(Nn);
    for (int i = 0; i < Nn; ++i) {
        const float os = 1.0f / (1.0f + oexp(-bufs[5][i]));
        bool cull = os < a->cull_alpha_thresh;
        if (i < N && split[i] != 0) cull = true;
        if (a->check_huge) {
            const float* s = bufs[1] + 3 * (size_t)i;
            const float mx = std::fmax(std::fmax(oexp(s[0]), oexp(s[1])), oexp(s[2]));
            if (mx > a->cull_scale_thresh) cull = true;
            if (a->check_screen && i < N && max2d[i] > a->cull_screen_size) cull = true;
        }
        keep[i] = cull ? 0 : 1;
    }
    // Stable compaction of all 18 buffers (compact_scatter / copy_back).
    int out = 0;
    for (int i = 0; i < Nn; ++i) {
        if (!keep[i]) continue;
        if (out != i) {
            for (int gi = 0; gi < 6; ++gi) {
                const size_t st = (size_t)strides[gi];
                std::memmove(bufs[gi] + st * out, bufs[gi] + st * i, st * 4);
                std::memmove(m[gi] + st * out, m[gi] + st * i, st * 4);
                std::memmove(v[gi] + st * out, v[gi] + st * i, st * 4);
            }
        }
        ++out;
    }
    if (split_out) std::memcpy(split_out, split.data(), (size_t)N * 4);
    if (dup_out) std::memcpy(dup_out, dup.data(), (size_t)N * 4);
    if (keep_out) std::memcpy(keep_out, keep.data(), (size_t)Nn * 4);
    return out;
}

// ---- evaluation metrics (model.cpp:25-40, ssim.cpp:26-123) ----

namespace {
// gaussianBlur (ssim.cpp:26-59): horizontal pass into tmp, then vertical,
// taps summed from the first, borders clamped.
void blur_clamped(const float* in, float* out, float* tmp, int H, int W, const float* k, int ks) {
    const int pad = ks / 2;
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            float sum = 0.f;
            for (int i = 0; i < ks; ++i) {
                const int sx = std::min(std::max(x + i - pad, 0), W - 1);
                sum += in[(size_t)y * W + sx] * k[i];
            }
            tmp[(size_t)y * W + x] = sum;
        }
    for (int y = 0; y < H; ++y)
        for (int x = 0; x < W; ++x) {
            float sum = 0.f;
            for (int i = 0; i < ks; ++i) {
                const int sy = std::min(std::max(y + i - pad, 0), H - 1);
                sum += tmp[(size_t)sy * W + x] * k[i];
            }
            out[(size_t)y * W + x] = sum;
        }
}
}  // namespace

void orc_image_metrics(int32_t H, int32_t W, const float* img, const float* gt,
                       int32_t window_size, float sigma, float out[3]) {
    const int64_t n = (int64_t)H * W * 3;
    // psnr (model.cpp:25-32): fp64 mean of the squared fp32 differences
    double mse = 0.0, l1 = 0.0;
    for (int64_t i = 0; i < n; ++i) {
        const double d = img[i] - gt[i];
        mse += d * d;
        l1 += std::fabs(img[i] - gt[i]);
    }
    mse /= (double)n;
    out[0] = (float)(10.0f * std::log10(1.0 / mse));
    out[2] = (float)(l1 / (double)n);
    // ssim_eval (ssim.cpp:61-123)
    std::vector<float> k(window_size);
    float ksum = 0.f;
    for (int i = 0; i < window_size; ++i) {
        const float x = (float)(i - window_size / 2);
        k[i] = std::exp(-(x * x) / (2.0f * sigma * sigma));
        ksum += k[i];
    }
    for (int i = 0; i < window_size; ++i) k[i] /= ksum;
    const size_t HW = (size_t)H * W;
    std::vector<float> r(HW), g(HW), rr(HW), gg(HW), rg(HW), mu1(HW), mu2(HW), s11(HW), s22(HW),
        s12(HW), tmp(HW);
    const float C1 = 0.01f * 0.01f, C2 = 0.03f * 0.03f;
    double sum = 0.0;
    int64_t count = 0;
    for (int c = 0; c < 3; ++c) {
        for (size_t i = 0; i < HW; ++i) {
            r[i] = img[3 * i + c];
            g[i] = gt[3 * i + c];
            rr[i] = r[i] * r[i];
            gg[i] = g[i] * g[i];
            rg[i] = r[i] * g[i];
        }
        blur_clamped(r.data(), mu1.data(), tmp.data(), H, W, k.data(), window_size);
        blur_clamped(g.data(), mu2.data(), tmp.data(), H, W, k.data(), window_size);
        blur_clamped(rr.data(), s11.data(), tmp.data(), H, W, k.data(), window_size);
        blur_clamped(gg.data(), s22.data(), tmp.data(), H, W, k.data(), window_size);
        blur_clamped(rg.data(), s12.data(), tmp.data(), H, W, k.data(), window_size);
        for (size_t i = 0; i < HW; ++i) {
            const float m1sq = mu1[i] * mu1[i], m2sq = mu2[i] * mu2[i], m12 = mu1[i] * mu2[i];
            const float sig1sq = s11[i] - m1sq, sig2sq = s22[i] - m2sq, sig12 = s12[i] - m12;
            const float num = (2.0f * m12 + C1) * (2.0f * sig12 + C2);
            const float den = (m1sq + m2sq + C1) * (sig1sq + sig2sq + C2);
            sum += num / den;
            ++count;
        }
    }
    out[1] = (float)(sum / (double)count);
}

void orc_image_to_rgba8(int64_t n_pixels, const float* img, uint8_t* rgba) {
    for (int64_t p = 0; p < n_pixels; ++p) {
        for (int c = 0; c < 3; ++c)
            rgba[4 * p + c] = (uint8_t)(std::fmin(std::fmax(img[3 * p + c], 0.f), 1.f) * 255.f);
        rgba[4 * p + 3] = 255;
    }
}

void orc_knn_mean_dist(int64_t n, const float* xyz, float* out) {
#pragma omp parallel for schedule(dynamic, 64)
    for (int64_t i = 0; i < n; ++i) {
        float b[4] = {INFINITY, INFINITY, INFINITY, INFINITY};
        for (int64_t j = 0; j < n; ++j) {
            float d = 0.f;
            for (int k = 0; k < 3; ++k) {
                const float diff = xyz[3 * i + k] - xyz[3 * j + k];
                d += diff * diff;
            }
            if (d < b[3]) {   // insertion into the four smallest, ascending
                int p = 3;
                while (p > 0 && d < b[p - 1]) { b[p] = b[p - 1]; --p; }
                b[p] = d;
            }
        }
        float sum = 0.f;
        for (int j = 1; j < 4; ++j) sum += std::sqrt(b[j]);
        out[i] = sum / 3;
    }
}


// ---- target images: area resize and undistortion ----

void orc_resize_area(int32_t sw, int32_t sh, const float* src, int32_t dw, int32_t dh, float* dst) {
    const float scale_x = (float)sw / (float)dw;
    const float scale_y = (float)sh / (float)dh;
    for (int dy = 0; dy < dh; ++dy) {
        const float y0 = (float)dy * scale_y, y1 = (float)(dy + 1) * scale_y;
        for (int dx = 0; dx < dw; ++dx) {
            const float x0 = (float)dx * scale_x, x1 = (float)(dx + 1) * scale_x;
            float sum[3] = {0.f, 0.f, 0.f};
            float total = 0.f;
            const int iy0 = (int)y0, iy1 = std::min((int)std::ceil(y1), (int)sh);
            const int ix0 = (int)x0, ix1 = std::min((int)std::ceil(x1), (int)sw);
            for (int iy = iy0; iy < iy1; ++iy) {
                const float wy = std::min((float)(iy + 1), y1) - std::max((float)iy, y0);
                for (int ix = ix0; ix < ix1; ++ix) {
                    const float wx = std::min((float)(ix + 1), x1) - std::max((float)ix, x0);
                    const float area = wx * wy;
                    const float* q = &src[((size_t)iy * sw + ix) * 3];
                    for (int c = 0; c < 3; ++c) sum[c] += q[c] * area;
                    total += area;
                }
            }
            const float inv = 1.0f / total;
            float* o = &dst[((size_t)dy * dw + dx) * 3];
            for (int c = 0; c < 3; ++c) o[c] = sum[c] * inv;
        }
    }
}

namespace {

struct Distortion { float fx, fy, cx, cy, k1, k2, p1, p2, k3; };

// distortPoint, image_io.cpp:143-153
void orc_distort_point(float x, float y, const Distortion& d, float& xd, float& yd) {
    const float r2 = x * x + y * y;
    const float r4 = r2 * r2;
    const float r6 = r4 * r2;
    const float radial = 1.0f + d.k1 * r2 + d.k2 * r4 + d.k3 * r6;
    xd = x * radial + 2.0f * d.p1 * x * y + d.p2 * (r2 + 2.0f * x * x);
    yd = y * radial + d.p1 * (r2 + 2.0f * y * y) + 2.0f * d.p2 * x * y;
}

// undistortPoint, image_io.cpp:156-171
void orc_undistort_point(float xd, float yd, const Distortion& d, float& xu, float& yu) {
    xu = xd;
    yu = yd;
    for (int i = 0; i < 20; i++) {
        const float r2 = xu * xu + yu * yu;
        const float r4 = r2 * r2;
        const float r6 = r4 * r2;
        const float radial = 1.0f + d.k1 * r2 + d.k2 * r4 + d.k3 * r6;
        const float dx = 2.0f * d.p1 * xu * yu + d.p2 * (r2 + 2.0f * xu * xu);
        const float dy = d.p1 * (r2 + 2.0f * yu * yu) + 2.0f * d.p2 * xu * yu;
        xu = (xd - dx) / radial;
        yu = (yd - dy) / radial;
    }
}

// (int)floor(v) where it is defined; beyond the int range (undefined in the
// reference) it saturates to just outside [0, n], which the clamp that
// follows treats like any other outside value.
int orc_floor_int(float v, int n) {
    const float f = std::floor(v);
    if (!(f > -1.f)) return -1;
    if (f > (float)n) return n;
    return (int)f;
}

// bilinearSample, image_io.cpp:174-201
void orc_bilinear(const float* img, int w, int h, float x, float y, float out[3]) {
    int x0 = orc_floor_int(x, w), y0 = orc_floor_int(y, h);
    int x1 = x0 + 1, y1 = y0 + 1;
    x0 = std::clamp(x0, 0, w - 1);
    x1 = std::clamp(x1, 0, w - 1);
    y0 = std::clamp(y0, 0, h - 1);
    y1 = std::clamp(y1, 0, h - 1);
    const float fx = x - std::floor(x);
    const float fy = y - std::floor(y);
    const float* p00 = &img[((size_t)y0 * w + x0) * 3];
    const float* p10 = &img[((size_t)y0 * w + x1) * 3];
    const float* p01 = &img[((size_t)y1 * w + x0) * 3];
    const float* p11 = &img[((size_t)y1 * w + x1) * 3];
    for (int c = 0; c < 3; c++) {
        const float top = p00[c] * (1.0f - fx) + p10[c] * fx;
        const float bottom = p01[c] * (1.0f - fx) + p11[c] * fx;
        out[c] = top * (1.0f - fy) + bottom * fy;
    }
}

int orc_saturating_int(float v) {
    if (!(v > -2.0e9f)) return -2000000000;
    if (v > 2.0e9f) return 2000000000;
    return (int)v;
}

Distortion orc_distortion(const float intr[4], const float dist[5]) {
    return Distortion{intr[0], intr[1], intr[2], intr[3], dist[0], dist[1], dist[2], dist[3], dist[4]};
}

}  // namespace

void orc_undistort_roi(int32_t w, int32_t h, const float intr[4], const float dist[5], int32_t roi[4]) {
    const Distortion d = orc_distortion(intr, dist);
    float top_max = -1e9f, bottom_min = 1e9f, left_max = -1e9f, right_min = 1e9f;
    const int n = 200;
    for (int i = 0; i < n; i++) {
        const float t = (float)i / (n - 1);
        float xu, yu;
        float xd = (t * w - d.cx) / d.fx, yd = (0.0f - d.cy) / d.fy;
        orc_undistort_point(xd, yd, d, xu, yu);
        top_max = std::max(top_max, yu * d.fy + d.cy);
        xd = (t * w - d.cx) / d.fx; yd = ((float)(h - 1) - d.cy) / d.fy;
        orc_undistort_point(xd, yd, d, xu, yu);
        bottom_min = std::min(bottom_min, yu * d.fy + d.cy);
        xd = (0.0f - d.cx) / d.fx; yd = (t * h - d.cy) / d.fy;
        orc_undistort_point(xd, yd, d, xu, yu);
        left_max = std::max(left_max, xu * d.fx + d.cx);
        xd = ((float)(w - 1) - d.cx) / d.fx; yd = (t * h - d.cy) / d.fy;
        orc_undistort_point(xd, yd, d, xu, yu);
        right_min = std::min(right_min, xu * d.fx + d.cx);
    }
    int rx = std::max(0, orc_saturating_int(std::ceil(left_max)));
    int ry = std::max(0, orc_saturating_int(std::ceil(top_max)));
    int rw = std::min((int)w, orc_saturating_int(std::floor(right_min))) - rx;
    int rh = std::min((int)h, orc_saturating_int(std::floor(bottom_min))) - ry;
    if (rw <= 0 || rh <= 0) { rx = 0; ry = 0; rw = w; rh = h; }
    roi[0] = rx; roi[1] = ry; roi[2] = rw; roi[3] = rh;
}

void orc_undistort(int32_t w, int32_t h, const float* src, const float intr[4], const float dist[5],
                   int32_t roi[4], float* dst) {
    const Distortion d = orc_distortion(intr, dist);
    orc_undistort_roi(w, h, intr, dist, roi);
    // the whole image remapped, then the rectangle copied out, as the reference
    std::vector<float> full((size_t)w * h * 3);
    for (int oy = 0; oy < h; oy++) {
        for (int ox = 0; ox < w; ox++) {
            const float x = ((float)ox - d.cx) / d.fx;
            const float y = ((float)oy - d.cy) / d.fy;
            float xd, yd;
            orc_distort_point(x, y, d, xd, yd);
            orc_bilinear(src, w, h, xd * d.fx + d.cx, yd * d.fy + d.cy, &full[((size_t)oy * w + ox) * 3]);
        }
    }
    for (int y = 0; y < roi[3]; y++)
        std::memcpy(&dst[(size_t)y * roi[2] * 3], &full[((size_t)(y + roi[1]) * w + roi[0]) * 3],
                    (size_t)roi[2] * 3 * sizeof(float));
}

}  // extern "C"
