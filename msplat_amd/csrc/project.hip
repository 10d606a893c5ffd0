// project.hip — projection + SH colour of every gaussian (one thread each),
// fused with the depth-key output for the binning, the intersection and
// super-tile reference totals the host reads, and the zeroing of the raster
// gradient accumulators.
//
// Follows project_and_sh_forward_kernel (.metal:1695-1787) and its helpers
// quat_to_rotmat (.metal:111-131), scale_rot_to_cov3d (.metal:175-188),
// project_cov3d_ewa (.metal:241-281), compute_cov2d_bounds (.metal:283-305),
// project_pix (.metal:308-317), get_tile_bbox (.metal:57-87) and
// sh_coeffs_to_color (.metal:587-654).  It also writes the depth sort key
// (depth bits, or 0xFFFFFFFF when culled) and value (the id) for the binning;
// the sigmoid of the opacity logit that the reference evaluates per
// intersection at pack time (.metal:2133) is evaluated once per gaussian
// here, same formula.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

struct V3 { float x, y, z; };

__device__ __forceinline__ V3 xf4x3(const float* m, V3 p) {
    return V3{m[0] * p.x + m[1] * p.y + m[2] * p.z + m[3],
              m[4] * p.x + m[5] * p.y + m[6] * p.z + m[7],
              m[8] * p.x + m[9] * p.y + m[10] * p.z + m[11]};
}

// cov3d upper triangle from exp'd scale and quaternion (w,x,y,z).
__device__ __forceinline__ void cov3d_of(const float s0, const float s1, const float s2,
                                         float glob, float4 q, float* cov) {
    const float s = 1.f / sqrtf(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z);
    const float w = q.x * s, x = q.y * s, y = q.z * s, z = q.w * s;
    // R[col][row]
    const float R00 = 1.f - 2.f * (y * y + z * z), R01 = 2.f * (x * y + w * z), R02 = 2.f * (x * z - w * y);
    const float R10 = 2.f * (x * y - w * z), R11 = 1.f - 2.f * (x * x + z * z), R12 = 2.f * (y * z + w * x);
    const float R20 = 2.f * (x * z + w * y), R21 = 2.f * (y * z - w * x), R22 = 1.f - 2.f * (x * x + y * y);
    const float g0 = glob * s0, g1 = glob * s1, g2 = glob * s2;
    const float M00 = R00 * g0, M01 = R01 * g0, M02 = R02 * g0;
    const float M10 = R10 * g1, M11 = R11 * g1, M12 = R12 * g1;
    const float M20 = R20 * g2, M21 = R21 * g2, M22 = R22 * g2;
    // tmp[j][i] = sum_k M[k][i] * M[k][j]
    cov[0] = M00 * M00 + M10 * M10 + M20 * M20;
    cov[1] = M01 * M00 + M11 * M10 + M21 * M20;
    cov[2] = M02 * M00 + M12 * M10 + M22 * M20;
    cov[3] = M01 * M01 + M11 * M11 + M21 * M21;
    cov[4] = M02 * M01 + M12 * M11 + M22 * M21;
    cov[5] = M02 * M02 + M12 * M12 + M22 * M22;
}

__device__ __forceinline__ void sh_color(int degree, V3 d, const float* dc, const float* rest,
                                         float* col) {
#pragma unroll
    for (int c = 0; c < 3; ++c) col[c] = SH_C0 * dc[c];
    if (degree < 1) return;
    const float x = d.x, y = d.y, z = d.z;
    const float xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        const float* r = rest + c;
        col[c] += SH_C1 * (-y * r[0] + z * r[3] - x * r[6]);
        if (degree < 2) continue;
        col[c] += (SH_C2_0 * xy * r[9] + SH_C2_1 * yz * r[12] + SH_C2_2 * (2.f * zz - xx - yy) * r[15] +
                   SH_C2_3 * xz * r[18] + SH_C2_4 * (xx - yy) * r[21]);
        if (degree < 3) continue;
        col[c] += (SH_C3_0 * y * (3.f * xx - yy) * r[24] + SH_C3_1 * xy * z * r[27] +
                   SH_C3_2 * y * (4.f * zz - xx - yy) * r[30] +
                   SH_C3_3 * z * (2.f * zz - 3.f * xx - 3.f * yy) * r[33] +
                   SH_C3_4 * x * (4.f * zz - xx - yy) * r[36] + SH_C3_5 * z * (xx - yy) * r[39] +
                   SH_C3_6 * x * (xx - 3.f * yy) * r[42]);
        if (degree < 4) continue;
        col[c] += (2.5033429417967046f * xy * (xx - yy) * r[45] +
                   -1.7701307697799304f * yz * (3.f * xx - yy) * r[48] +
                   0.9461746957575601f * xy * (7.f * zz - 1.f) * r[51] +
                   -0.6690465435572892f * yz * (7.f * zz - 3.f) * r[54] +
                   0.10578554691520431f * (zz * (35.f * zz - 30.f) + 3.f) * r[57] +
                   -0.6690465435572892f * xz * (7.f * zz - 3.f) * r[60] +
                   0.47308734787878004f * (xx - yy) * (7.f * zz - 1.f) * r[63] +
                   -1.7701307697799304f * xz * (xx - 3.f * yy) * r[66] +
                   0.6258357354491761f * (xx * (xx - 3.f * yy) - yy * (3.f * xx - yy)) * r[69]);
    }
}

constexpr int PROJ_T = 128;   // gaussians per workgroup

// Screen-space footprint of one visible gaussian (the part of the
// projection that does not need its SH coefficients).
struct Geo {
    int area;   // tiles hit; 0 when culled
    int nref;   // super-tiles overlapped
    float px, py, ca, cb, cc, ex, ey, z;
};

__device__ __forceinline__ Geo project_geo(const CamParams& p, int g, V3 pw, const float* sc,
                                           float4 q, GaussOut go, uint32_t* __restrict__ dkey,
                                           uint32_t* __restrict__ dval);
__device__ __forceinline__ void project_col(const CamParams& p, int g, V3 pw, const float* dc,
                                            float ol, const float* rest, const Geo& e,
                                            GaussOut go, uint32_t* __restrict__ dkey);

// PROJ_STAGE: 16-byte features_rest loads per thread, enough for PROJ_T rows
// of up to 48 floats (SH degree <= 3) or 72 floats (degree 4).
template <int PROJ_STAGE>
__global__ __launch_bounds__(PROJ_T) void k_project_fwd(
    CamParams p, const float* __restrict__ means, const float* __restrict__ scales,
    const float* __restrict__ quats, const float* __restrict__ f_dc,
    const float* __restrict__ f_rest, const float* __restrict__ opac_logits, GaussOut go,
    uint32_t* __restrict__ dkey, uint32_t* __restrict__ dval, float* __restrict__ gacc,
    unsigned long long* __restrict__ total_isect) {
    const int g0 = blockIdx.x * PROJ_T;
    const int g = g0 + threadIdx.x;
    const bool live = g < p.N;
    // Per-gaussian inputs first, so that their loads overlap the staging below.
    // The parameters (these and the features_rest rows staged below) are
    // read once per step here, and next by the Adam step after the raster
    // kernels: their loads are non-temporal, so that they do not displace the
    // records this kernel writes, which the raster kernels gather next.
    V3 pw{0.f, 0.f, 0.f};
    float sc[3] = {0.f, 0.f, 0.f}, dc[3] = {0.f, 0.f, 0.f}, ol = 0.f;
    float4 q = make_float4(1.f, 0.f, 0.f, 0.f);
    if (live) {
        pw = V3{ld_nt(means + 3 * g), ld_nt(means + 3 * g + 1), ld_nt(means + 3 * g + 2)};
#pragma unroll
        for (int k = 0; k < 3; ++k) {
            sc[k] = ld_nt(scales + 3 * (size_t)g + k);
            dc[k] = ld_nt(f_dc + 3 * (size_t)g + k);
        }
        q = ld_nt4(quats + 4 * (size_t)g);
        ol = ld_nt(opac_logits + g);
    }
    // Zero this workgroup's raster gradient accumulators (PROJ_T * 9
    // contiguous floats) with 16-byte stores; render-only calls pass none.
    if (gacc) {
        const int64_t base = (int64_t)g0 * 9;
        const int cnt = (int)min((int64_t)PROJ_T * 9, (int64_t)p.N * 9 - base);
        float4* dst4 = reinterpret_cast<float4*>(gacc + base);
        for (int i = threadIdx.x; i < cnt / 4; i += PROJ_T) dst4[i] = make_float4(0.f, 0.f, 0.f, 0.f);
        for (int i = (cnt / 4) * 4 + threadIdx.x; i < cnt; i += PROJ_T) gacc[base + i] = 0.f;
    }
    // Geometry first: which of the workgroup's gaussians are visible.
    Geo ge{};
    if (live) ge = project_geo(p, g, pw, sc, q, go, dkey, dval);
    __shared__ int s_vis[PROJ_T];
    s_vis[threadIdx.x] = ge.area > 0;
    __syncthreads();
    // Stage this workgroup's features_rest rows (PROJ_T * rest_per contiguous
    // floats, 16-byte aligned) through LDS with coalesced 16-byte loads.  All
    // of a thread's loads are issued before the first LDS store, so the
    // workgroup waits for one memory round trip, not one per load.  A vector
    // that touches only rows of culled gaussians re-reads the block's last
    // vector instead (one cached line), so culled rows cost no traffic.
    extern __shared__ float s_rest[];
    if (p.dtu > 0) {
        const int64_t base = (int64_t)g0 * p.rest_per;
        const int64_t total = (int64_t)p.N * p.rest_per;
        const int cnt = (int)min((int64_t)PROJ_T * p.rest_per, total - base);
        const int nv = cnt / 4;
        const float4* src4 = reinterpret_cast<const float4*>(f_rest + base);
        float4* dst4 = reinterpret_cast<float4*>(s_rest);
        if (nv > 0) {
            // Branch-free: indexes past the block's rows re-read its last
            // vector and store it to a spare LDS slot after the staging
            // area, so the compiler keeps all loads in flight together.
            float4 stage[PROJ_STAGE];
            // rows of the first and last float of vector i: floor((4i + 0.5) /
            // rest_per), exact in fp32 for these sizes (the quotient is never
            // within 0.5 / rest_per of an integer)
            const float inv_rest = 1.f / (float)p.rest_per;
#pragma unroll
            for (int k = 0; k < PROJ_STAGE; ++k) {
                const int i = min((int)threadIdx.x + k * PROJ_T, nv - 1);
                const int r0 = (int)(((float)(4 * i) + 0.5f) * inv_rest);
                const int r1 = min((int)(((float)(4 * i) + 3.5f) * inv_rest), PROJ_T - 1);
                const int src = (s_vis[r0] | s_vis[r1]) ? i : nv - 1;
                stage[k] = ld_nt4(reinterpret_cast<const float*>(src4 + src));
            }
#pragma unroll
            for (int k = 0; k < PROJ_STAGE; ++k) {
                const int i = threadIdx.x + k * PROJ_T;
                dst4[i < nv ? i : PROJ_T * PROJ_STAGE] = stage[k];
            }
        }
        for (int i = nv * 4 + threadIdx.x; i < cnt; i += PROJ_T) s_rest[i] = f_rest[base + i];
        __syncthreads();
    }
    const int area = ge.area;
    if (area > 0)
        project_col(p, g, pw, dc, ol, s_rest + (size_t)p.rest_per * threadIdx.x, ge, go, dkey);
    // Intersection and reference totals for the host: one atomic each per
    // workgroup, on one of ISECT_SLOTS counter pairs so that workgroups do
    // not queue on one address.
    int v = area, vr = ge.nref;
#pragma unroll
    for (int off = 32; off >= 1; off >>= 1) {
        v += __shfl_xor(v, off, 64);
        vr += __shfl_xor(vr, off, 64);
    }
    __shared__ int s_tot[2][PROJ_T / 64];
    if ((threadIdx.x & 63) == 0) {
        s_tot[0][threadIdx.x >> 6] = v;
        s_tot[1][threadIdx.x >> 6] = vr;
    }
    __syncthreads();
    if (threadIdx.x < 2) {
        long long t = 0;
#pragma unroll
        for (int k = 0; k < PROJ_T / 64; ++k) t += s_tot[threadIdx.x][k];
        if (t)
            atomicAdd(total_isect + (size_t)(blockIdx.x % ISECT_SLOTS) * ISECT_STRIDE + threadIdx.x,
                      (unsigned long long)t);
    }
}

// One gaussian's geometry: writes the culled defaults (radii, tiles hit,
// depth key / value), and radii / tiles hit when visible.
__device__ __forceinline__ Geo project_geo(const CamParams& p, int g, V3 pw, const float* sc,
                                           float4 q, GaussOut go, uint32_t* __restrict__ dkey,
                                           uint32_t* __restrict__ dval) {
    Geo r{};
    go.radii[g] = 0;
    if (go.radii_out) go.radii_out[g] = 0;
    go.tiles_hit[g] = 0;
    go.rect[g] = make_uint2(0u, 0u);
    dkey[g] = 0xFFFFFFFFu;
    dval[g] = (uint32_t)g;

    const V3 pv = xf4x3(p.vm, pw);
    if (pv.z <= p.clip) return r;

    const float s0 = exp_cw(sc[0]), s1 = exp_cw(sc[1]), s2 = exp_cw(sc[2]);
    float cov[6];
    cov3d_of(s0, s1, s2, p.glob_scale, q, cov);

    // EWA projection with the view-space clamp to 1.3 tan(fov).
    const float tan_fovx = 0.5f * (float)p.W / p.fx, tan_fovy = 0.5f * (float)p.H / p.fy;
    const float lim_x = 1.3f * tan_fovx, lim_y = 1.3f * tan_fovy;
    const float cxv = pv.z * fminf(lim_x, fmaxf(-lim_x, pv.x / pv.z));
    const float cyv = pv.z * fminf(lim_y, fmaxf(-lim_y, pv.y / pv.z));
    const float rz = 1.f / pv.z, rz2 = rz * rz;
    const float j00 = p.fx * rz, j11 = p.fy * rz;
    const float j20 = -p.fx * cxv * rz2, j21 = -p.fy * cyv * rz2;
    const float t0x = j00 * p.vm[0] + j20 * p.vm[8], t0y = j00 * p.vm[1] + j20 * p.vm[9],
                t0z = j00 * p.vm[2] + j20 * p.vm[10];
    const float t1x = j11 * p.vm[4] + j21 * p.vm[8], t1y = j11 * p.vm[5] + j21 * p.vm[9],
                t1z = j11 * p.vm[6] + j21 * p.vm[10];
    const float tv0x = t0x * cov[0] + t0y * cov[1] + t0z * cov[2];
    const float tv0y = t0x * cov[1] + t0y * cov[3] + t0z * cov[4];
    const float tv0z = t0x * cov[2] + t0y * cov[4] + t0z * cov[5];
    const float tv1x = t1x * cov[0] + t1y * cov[1] + t1z * cov[2];
    const float tv1y = t1x * cov[1] + t1y * cov[3] + t1z * cov[4];
    const float tv1z = t1x * cov[2] + t1y * cov[4] + t1z * cov[5];
    const float c2x = (tv0x * t0x + tv0y * t0y + tv0z * t0z) + 0.3f;
    const float c2y = tv0x * t1x + tv0y * t1y + tv0z * t1z;
    const float c2z = (tv1x * t1x + tv1y * t1y + tv1z * t1z) + 0.3f;

    // Conic and 3-sigma radius.
    const float det = c2x * c2z - c2y * c2y;
    if (det == 0.f) return r;
    const float inv_det = 1.f / det;
    const float ca = c2z * inv_det, cb = -c2y * inv_det, cc = c2x * inv_det;
    const float b = 0.5f * (c2x + c2z);
    const float disc = sqrtf(fmaxf(0.1f, b * b - det));
    const float radius = ceilf(3.f * sqrtf(b + disc));

    // Pixel centre.
    const float* m = p.pm;
    const float hx = m[0] * pw.x + m[1] * pw.y + m[2] * pw.z + m[3];
    const float hy = m[4] * pw.x + m[5] * pw.y + m[6] * pw.z + m[7];
    const float hw = m[12] * pw.x + m[13] * pw.y + m[14] * pw.z + m[15];
    const float rw = 1.f / (hw + 1e-6f);
    const float px = 0.5f * (float)p.W * (hx * rw) + p.cx - 0.5f;
    const float py = 0.5f * (float)p.H * (hy * rw) + p.cy - 0.5f;

    const float ex = ceilf(3.0f * sqrtf(c2x)), ey = ceilf(3.0f * sqrtf(c2z));
    int x0, y0, x1, y1;
    tile_rect(px, py, ex, ey, p.tbx, p.tby, x0, y0, x1, y1);
    const int area = (x1 - x0) * (y1 - y0);
    if (area <= 0) return r;

    go.tiles_hit[g] = area;
    go.rect[g] = make_uint2((uint32_t)x0 | (uint32_t)y0 << 16, (uint32_t)x1 | (uint32_t)y1 << 16);
    go.radii[g] = f2i(radius);
    if (go.radii_out) go.radii_out[g] = f2i(radius);
    r.area = area;
    r.nref = super_span(x0, y0, x1, y1);   // one binning reference per super-tile
    r.px = px; r.py = py; r.ca = ca; r.cb = cb; r.cc = cc; r.ex = ex; r.ey = ey; r.z = pv.z;
    return r;
}

// Colour and record of one visible gaussian: SH along normalize(p - cam_pos).
__device__ __forceinline__ void project_col(const CamParams& p, int g, V3 pw, const float* dc,
                                            float ol, const float* rest, const Geo& e,
                                            GaussOut go, uint32_t* __restrict__ dkey) {
    const float px = e.px, py = e.py, ca = e.ca, cb = e.cb, cc = e.cc, ex = e.ex, ey = e.ey;
    // SH colour along normalize(p - cam_pos).
    const float dx = pw.x - p.cam[0], dy = pw.y - p.cam[1], dz = pw.z - p.cam[2];
    const float inv = 1.f / sqrtf(dx * dx + dy * dy + dz * dz);
    const V3 dir{dx * inv, dy * inv, dz * inv};
    float col[3];
    sh_color(p.dtu, dir, dc, rest, col);
    float4* rec = go.rec + 4 * (size_t)g;
    rec[0] = make_float4(px, py, ca, cb);
    rec[1] = make_float4(cc, sigmoid(ol), col[0], col[1]);
    rec[2] = make_float4(col[2], ex, ey, e.z);
    rec[3] = make_float4(dir.x, dir.y, dir.z, 0.f);
    dkey[g] = __float_as_uint(e.z);
}

}  // namespace

void launch_project_fwd(hipStream_t s, const CamParams& p, const float* means,
                        const float* scales, const float* quats, const float* f_dc,
                        const float* f_rest, const float* opac_logits, GaussOut go,
                        uint32_t* dkey, uint32_t* dval, float* gacc,
                        unsigned long long* total_isect) {
    if (p.N <= 0) return;
    const int blocks = (p.N + PROJ_T - 1) / PROJ_T;
    // staging area of PROJ_STAGE vectors per thread plus the spare slot
    const int stage = p.rest_per <= 48 ? PROJ_T * 48 / 4 / PROJ_T : PROJ_T * 72 / 4 / PROJ_T;
    const size_t lds = p.dtu > 0 ? ((size_t)PROJ_T * stage + 1) * 16 : 0;
    if (p.rest_per <= 48)
        hipLaunchKernelGGL(k_project_fwd<PROJ_T * 48 / 4 / PROJ_T>, dim3(blocks), dim3(PROJ_T), lds,
                           s, p, means, scales, quats, f_dc, f_rest, opac_logits, go, dkey, dval,
                           gacc, total_isect);
    else
        hipLaunchKernelGGL(k_project_fwd<PROJ_T * 72 / 4 / PROJ_T>, dim3(blocks), dim3(PROJ_T), lds,
                           s, p, means, scales, quats, f_dc, f_rest, opac_logits, go, dkey, dval,
                           gacc, total_isect);
}

}  // namespace msp
