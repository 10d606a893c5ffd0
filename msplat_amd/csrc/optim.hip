// optim.hip — projection backward, SH backward and Adam, fused per gaussian.
//
// Reference: project_and_sh_backward_kernel (.metal:1813-1986) with
// project_pix_vjp (.metal:1216-1234), cov2d_to_conic_vjp (.metal:1253-1264),
// project_cov3d_ewa_vjp (.metal:1339-1407), quat_to_rotmat_vjp
// (.metal:1409-1452), scale_rot_to_cov3d_vjp (.metal:1498-1531) and
// adam_update_element (.metal:1791-1800); then fused_adam_kernel
// (.metal:1666-1689) on groups 0, 1, 2, 5 and accumulate_grad_stats
// (.metal:1643-1664).
//
// MI355X layout: the reference writes v_mean3d / v_scale / v_quat to memory
// and runs four more Adam passes over them; here one thread per gaussian
// computes the gradients in registers and applies Adam to means, scales,
// quats, opacity and f_dc directly (dense for the first four, visible-only for
// f_dc, as in the reference), plus the densify statistics.  The 45 floats of
// f_rest per gaussian are updated by a separate element-parallel kernel whose
// loads and stores are contiguous across the wave; it takes the view
// direction the projection stored with each gaussian's record.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

struct F3 { float x, y, z; };
struct M3 { float m[3][3]; };   // column-major like Metal's float3x3: m[col][row]

__device__ __forceinline__ F3 mat_vec(const M3& A, F3 v) {
    return F3{A.m[0][0] * v.x + A.m[1][0] * v.y + A.m[2][0] * v.z,
              A.m[0][1] * v.x + A.m[1][1] * v.y + A.m[2][1] * v.z,
              A.m[0][2] * v.x + A.m[1][2] * v.y + A.m[2][2] * v.z};
}
__device__ __forceinline__ M3 mat_mul(const M3& A, const M3& B) {
    M3 C;
#pragma unroll
    for (int j = 0; j < 3; ++j) {
        const F3 col = mat_vec(A, F3{B.m[j][0], B.m[j][1], B.m[j][2]});
        C.m[j][0] = col.x;
        C.m[j][1] = col.y;
        C.m[j][2] = col.z;
    }
    return C;
}
__device__ __forceinline__ M3 transpose(const M3& A) {
    M3 T;
#pragma unroll
    for (int i = 0; i < 3; ++i)
#pragma unroll
        for (int j = 0; j < 3; ++j) T.m[i][j] = A.m[j][i];
    return T;
}
__device__ __forceinline__ float dot3(F3 a, F3 b) { return a.x * b.x + a.y * b.y + a.z * b.z; }

// The backward and Adam outputs are compared with the CPU restatement to a
// relative tolerance, so their divisions and square roots use the hardware
// reciprocal and square root (v_rcp_f32 / v_sqrt_f32, about 1 ulp) rather
// than the correctly rounded multi-instruction IEEE sequences; the forward
// stages, which must match bit for bit, keep IEEE division and sqrt.
__device__ __forceinline__ float rcp_hw(float x) { return __builtin_amdgcn_rcpf(x); }
__device__ __forceinline__ float sqrt_hw(float x) { return __builtin_amdgcn_sqrtf(x); }

__device__ __forceinline__ M3 quat_to_rotmat(float4 q) {
    const float s = rcp_hw(sqrt_hw(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z));
    const float w = q.x * s, x = q.y * s, y = q.z * s, z = q.w * s;
    M3 R;
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

// adam_update_element (.metal:1791-1800); inv_bc2 = 1 / sqrt(1 - beta2^t).
__device__ __forceinline__ void adam_elem(float& p, float& m, float& v, float g, float step,
                                          float b1, float b2, float inv_bc2, float eps) {
    const float mn = fmaf(b1, m, (1.0f - b1) * g);
    const float vn = fmaf(b2, v, (1.0f - b2) * g * g);
    p -= step * mn * rcp_hw(sqrt_hw(vn) * inv_bc2 + eps);
    m = mn;
    v = vn;
}


// Element-parallel Adam on features_rest, four consecutive floats per thread
// (16-byte loads and stores).  Each 256-thread block covers 1024 consecutive
// elements; the gradient of element (gaussian g, basis b, channel c) is
// basis_b(dir_g) * v_rgb[g][c], so the block first evaluates the basis once
// per gaussian it touches (view direction from the projection record) into
// LDS.  Elements of culled gaussians and of bands above degrees_to_use keep
// their values (the reference updates visible gaussians' used bands only,
// .metal:1846-1848, 1931-1985).  Blocks take their element ranges last to
// first: the rows written last are then the first gaussians', which the next
// step's projection reads first, while they are still in the last-level
// cache.  The moments, and the record fields and accumulators read here (the
// step's last use of them), are loaded and the moments stored non-temporally,
// so that the caches keep the features_rest rows for that projection
// (non-temporal loads with ordinary stores of the same lines were slower).
constexpr int SHA_T = 256;
constexpr int SHA_E = 4 * SHA_T;
constexpr int SHA_MAXG = SHA_E / 9 + 2;   // rest_per >= 9

__device__ __forceinline__ void sh_basis15(float x, float y, float z, float* o) {
    const float xx = x * x, xy = x * y, xz = x * z, yy = y * y, yz = y * z, zz = z * z;
    o[0] = -SH_C1 * y;
    o[1] = SH_C1 * z;
    o[2] = -SH_C1 * x;
    o[3] = SH_C2_0 * xy;
    o[4] = SH_C2_1 * yz;
    o[5] = SH_C2_2 * (2.f * zz - xx - yy);
    o[6] = SH_C2_3 * xz;
    o[7] = SH_C2_4 * (xx - yy);
    o[8] = SH_C3_0 * y * (3.f * xx - yy);
    o[9] = SH_C3_1 * xy * z;
    o[10] = SH_C3_2 * y * (4.f * zz - xx - yy);
    o[11] = SH_C3_3 * z * (2.f * zz - 3.f * xx - 3.f * yy);
    o[12] = SH_C3_4 * x * (4.f * zz - xx - yy);
    o[13] = SH_C3_5 * z * (xx - yy);
    o[14] = SH_C3_6 * x * (xx - 3.f * yy);
}

// v_rgb of gaussian g from its accumulators, each channel kept only where
// the raw colour + 0.5 >= 0 (rasterize_backward_kernel masks it there,
// .metal:1083-1086; the mask is the gaussian's, so the raster backward sums
// every channel and the mask is applied here once).  NT: non-temporal loads
// (the step's last reads of the record and the accumulators).
template <bool NT>
__device__ __forceinline__ void masked_vrgb(const float* ga, const float4* rec, size_t g,
                                            float out[3]) {
    // loaded unconditionally (a conditional load would be a branch and a
    // separate memory round trip per channel)
    const float* r = reinterpret_cast<const float*>(rec + 4 * g);
    const float4 r1 = NT ? ld_nt4(r + 4) : rec[4 * g + 1];
    const float rb = NT ? ld_nt(r + 8) : r[8];
    const float v0 = NT ? ld_nt(ga + 5) : ga[5], v1 = NT ? ld_nt(ga + 6) : ga[6],
                v2 = NT ? ld_nt(ga + 7) : ga[7];
    out[0] = r1.z + 0.5f >= 0.f ? v0 : 0.f;
    out[1] = r1.w + 0.5f >= 0.f ? v1 : 0.f;
    out[2] = rb + 0.5f >= 0.f ? v2 : 0.f;
}

__global__ __launch_bounds__(SHA_T) void k_sh_rest_adam(int64_t n, int rest_per, int n_used,
                                                        const float4* __restrict__ rec,
                                                        const int* __restrict__ radii,
                                                        const float* __restrict__ gacc,
                                                        float* __restrict__ f_rest,
                                                        float* __restrict__ m,
                                                        float* __restrict__ v, AdamHP hp) {
    __shared__ float s_basis[SHA_MAXG][17];   // odd row stride: the per-gaussian writes hit distinct banks
    __shared__ float s_vrgb[SHA_MAXG][3];
    __shared__ int s_vis[SHA_MAXG];
    const int64_t eb = (int64_t)(gridDim.x - 1 - blockIdx.x) * SHA_E;
    const int gA = (int)(eb / rest_per);
    const int gB = (int)((min(eb + SHA_E, n) - 1) / rest_per);
    for (int t = threadIdx.x; t <= gB - gA; t += SHA_T) {
        const int g = gA + t;
        const bool vis = radii[g] > 0;
        s_vis[t] = vis;
        if (vis) {
            const float4 d = ld_nt4(reinterpret_cast<const float*>(rec + 4 * (size_t)g + 3));
            float bs[15];
            sh_basis15(d.x, d.y, d.z, bs);
#pragma unroll
            for (int b = 0; b < 15; ++b) s_basis[t][b] = bs[b];
            float vr[3];
            masked_vrgb<true>(gacc + (size_t)g * 9, rec, (size_t)g, vr);
#pragma unroll
            for (int c = 0; c < 3; ++c) s_vrgb[t][c] = vr[c];
        }
    }
    __syncthreads();
    const int64_t e0 = eb + 4 * threadIdx.x;
    if (e0 >= n) return;
    int g = (int)(e0 / rest_per);
    int rem = (int)(e0 - (int64_t)g * rest_per);
    const int cnt = (int)min((int64_t)4, n - e0);
    const int g_last = (int)((e0 + cnt - 1) / rest_per);
    if (!s_vis[g - gA] && !s_vis[g_last - gA]) return;
    float pv[4], mv[4], vv[4];
    const bool full = cnt == 4;
    if (full) {
        const float4 a = *reinterpret_cast<const float4*>(f_rest + e0);
        const float4 b = ld_nt4(m + e0);
        const float4 c = ld_nt4(v + e0);
        pv[0] = a.x; pv[1] = a.y; pv[2] = a.z; pv[3] = a.w;
        mv[0] = b.x; mv[1] = b.y; mv[2] = b.z; mv[3] = b.w;
        vv[0] = c.x; vv[1] = c.y; vv[2] = c.z; vv[3] = c.w;
    } else {
        for (int k = 0; k < cnt; ++k) {
            pv[k] = f_rest[e0 + k];
            mv[k] = ld_nt(m + e0 + k);
            vv[k] = ld_nt(v + e0 + k);
        }
    }
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        if (k < cnt) {
            const int li = g - gA, b = rem / 3, c = rem - 3 * (rem / 3);
            if (b < n_used && s_vis[li]) {
                const float grad = s_basis[li][b] * s_vrgb[li][c];
                adam_elem(pv[k], mv[k], vv[k], grad, hp.step[4], hp.b1, hp.b2, hp.inv_bc2[4], hp.eps);
            }
        }
        if (++rem == rest_per) { rem = 0; ++g; }
    }
    if (full) {
        *reinterpret_cast<float4*>(f_rest + e0) = make_float4(pv[0], pv[1], pv[2], pv[3]);
        st_nt4(m + e0, make_float4(mv[0], mv[1], mv[2], mv[3]));
        st_nt4(v + e0, make_float4(vv[0], vv[1], vv[2], vv[3]));
    } else {
        for (int k = 0; k < cnt; ++k) {
            f_rest[e0 + k] = pv[k];
            st_nt(m + e0 + k, mv[k]);
            st_nt(v + e0 + k, vv[k]);
        }
    }
}

struct BwdPtrs {
    float* params[6];
    float* m[6];
    float* v[6];
};

// The six arrays of three-float rows (means, log-scales and their moments)
// pass through LDS: the workgroup's 256 rows of an array are 768 contiguous
// floats, loaded and stored as 16-byte vectors (vec3: every array 16-byte
// aligned) instead of three 4-byte accesses per thread, whose non-temporal
// forms fetch the same lines once per access.
constexpr int PBA_T = 256;
constexpr int PBA_S = 6;   // staged arrays: means p, m, v, scales p, m, v

// Loads (STORE false) or stores the workgroup's nf floats of the staged
// arrays between memory and s3; the moments non-temporally.
template <bool STORE>
__device__ __forceinline__ void stage_rows3(float* const arr[PBA_S], size_t f0, int nf, bool vec3,
                                            float (*s3)[3 * PBA_T]) {
    const int t = threadIdx.x;
    const int nv = vec3 ? nf >> 2 : 0;
    for (int i = t; i < nv; i += PBA_T) {
#pragma unroll
        for (int a = 0; a < PBA_S; ++a) {
            float* m = arr[a] + f0 + 4 * (size_t)i;
            float4* s = reinterpret_cast<float4*>(&s3[a][4 * i]);
            const bool moment = a % 3 != 0;
            if (STORE) {
                if (moment) st_nt4(m, *s);
                else *reinterpret_cast<float4*>(m) = *s;
            } else {
                *s = moment ? ld_nt4(m) : *reinterpret_cast<const float4*>(m);
            }
        }
    }
    for (int i = 4 * nv + t; i < nf; i += PBA_T) {
#pragma unroll
        for (int a = 0; a < PBA_S; ++a) {
            float* m = arr[a] + f0 + i;
            const bool moment = a % 3 != 0;
            if (STORE) {
                if (moment) st_nt(m, s3[a][i]);
                else *m = s3[a][i];
            } else {
                s3[a][i] = moment ? ld_nt(m) : *m;
            }
        }
    }
}

// At least three waves per SIMD (at most 168 VGPRs): with every load of a
// thread issued in two batches (dense parameters and gradient inputs, then
// the visible-only f_dc and statistics), that keeps enough bytes in flight.
__global__ __launch_bounds__(PBA_T) __attribute__((amdgpu_waves_per_eu(3)))
void k_proj_bwd_adam(CamParams p, BwdPtrs P, AdamHP hp,
                                                       GaussOut go, const float* __restrict__ gacc,
                                                       float* __restrict__ vis,
                                                       float* __restrict__ gnorm,
                                                       float* __restrict__ max2d, float inv_max_dim,
                                                       float* __restrict__ v_mean_out,
                                                       float* __restrict__ v_scale_out,
                                                       float* __restrict__ v_quat_out, int vec3) {
    __shared__ float s3[PBA_S][3 * PBA_T];
    const int g0 = blockIdx.x * PBA_T, t = threadIdx.x;
    // threads past the last gaussian work on a copy of it and store nothing
    const bool live = g0 + t < p.N;
    const int g = live ? g0 + t : p.N - 1;
    const int nf = 3 * min(PBA_T, p.N - g0);
    float* const arr3[PBA_S] = {P.params[0], P.m[0], P.v[0], P.params[1], P.m[1], P.v[1]};
    stage_rows3<false>(arr3, 3 * (size_t)g0, nf, vec3 != 0, s3);
    // The dense parameters and moments are loaded up front, so that these
    // loads and the gradient inputs share one memory round trip.  The moments
    // are loaded and stored non-temporally (nothing else reads them in the
    // step); the parameters are not, as the next projection reads them.
    // sp / sm / sv [k]: 0-2 means, 3-5 scales, 6-9 quats, 10 opacity (the
    // visible-only f_dc update loads its own).
    float sp[11], sm[11], sv[11];
    __syncthreads();
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        sp[k] = s3[0][3 * t + k];
        sm[k] = s3[1][3 * t + k];
        sv[k] = s3[2][3 * t + k];
        sp[3 + k] = s3[3][3 * t + k];
        sm[3 + k] = s3[4][3 * t + k];
        sv[3 + k] = s3[5][3 * t + k];
    }
    {
        const float4 a = reinterpret_cast<const float4*>(P.params[2])[g];
        const float4 b = ld_nt4(P.m[2] + 4 * (size_t)g);
        const float4 c = ld_nt4(P.v[2] + 4 * (size_t)g);
        sp[6] = a.x; sp[7] = a.y; sp[8] = a.z; sp[9] = a.w;
        sm[6] = b.x; sm[7] = b.y; sm[8] = b.z; sm[9] = b.w;
        sv[6] = c.x; sv[7] = c.y; sv[8] = c.z; sv[9] = c.w;
    }
    sp[10] = P.params[5][g];
    sm[10] = ld_nt(P.m[5] + g);
    sv[10] = ld_nt(P.v[5] + g);
    const int rad = live ? go.radii[g] : 0;
    const float* ga = gacc + (size_t)g * 9;
    F3 vm{0.f, 0.f, 0.f};
    float vs[3] = {0.f, 0.f, 0.f}, vq[4] = {0.f, 0.f, 0.f, 0.f};
    const F3 pw{sp[0], sp[1], sp[2]};
    const float4 q = make_float4(sp[6], sp[7], sp[8], sp[9]);
    const float v_op = ga[8];
    if (rad > 0) {
        // Visible-only inputs (f_dc with its moments, the densify statistics)
        // are loaded before the gradient arithmetic, in one round trip.
        float dp[3], dm[3], dv[3];
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            dp[c] = P.params[3][3 * (size_t)g + c];
            dm[c] = ld_nt(P.m[3] + 3 * (size_t)g + c);
            dv[c] = ld_nt(P.v[3] + 3 * (size_t)g + c);
        }
        const float st_vis = vis[g], st_gnorm = gnorm[g], st_max2d = max2d[g];
        float vrgb[3];
        masked_vrgb<false>(ga, go.rec, (size_t)g, vrgb);
        // The raster backward sums the moments of v_sigma over the pixels
        // (m0 = sum v dx, m1 = sum v dy, m2..m4 = sum v (dx^2, dx dy, dy^2));
        // with this gaussian's conic (a, b, c) they give v_xy = (a m0 + b m1,
        // b m0 + c m1) and v_conic = (m2, m3, m4) / 2.
        const float4 r0 = go.rec[4 * (size_t)g], r1 = go.rec[4 * (size_t)g + 1];
        const float vxy0 = fmaf(r0.w, ga[1], r0.z * ga[0]);
        const float vxy1 = fmaf(r1.x, ga[1], r0.w * ga[0]);
        // project_pix_vjp: x/y rows through a fixed 1/w (the w row is dropped).
        {
            const float* m = p.pm;
            const float hw = m[12] * pw.x + m[13] * pw.y + m[14] * pw.z + m[15];
            const float rw = rcp_hw(hw + 1e-6f);
            const float vpx = 0.5f * (float)p.W * vxy0 * rw, vpy = 0.5f * (float)p.H * vxy1 * rw;
            const float vpz = 0.f;
            vm.x = m[0] * vpx + m[4] * vpy + m[8] * vpz;
            vm.y = m[1] * vpx + m[5] * vpy + m[9] * vpz;
            vm.z = m[2] * vpx + m[6] * vpy + m[10] * vpz;
            const float v_z = 0.f;   // v_depth is zero-filled and never written (.mm:1168)
            vm.x = vm.x + p.vm[8] * v_z;
            vm.y = vm.y + p.vm[9] * v_z;
            vm.z = vm.z + p.vm[10] * v_z;
        }
        // cov2d_to_conic_vjp: v_Sigma = -X G X.
        float vc2[3];
        {
            const float X[2][2] = {{r0.z, r0.w}, {r0.w, r1.x}};
            const float G[2][2] = {{0.5f * ga[2], 0.5f * ga[3]}, {0.5f * ga[3], 0.5f * ga[4]}};
            float nX[2][2], T1[2][2], S[2][2];
#pragma unroll
            for (int i = 0; i < 2; ++i)
#pragma unroll
                for (int j = 0; j < 2; ++j) nX[i][j] = -1.f * X[i][j];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i) T1[j][i] = nX[0][i] * G[j][0] + nX[1][i] * G[j][1];
#pragma unroll
            for (int j = 0; j < 2; ++j)
#pragma unroll
                for (int i = 0; i < 2; ++i) S[j][i] = T1[0][i] * X[j][0] + T1[1][i] * X[j][1];
            vc2[0] = S[0][0];
            vc2[1] = S[1][0] + S[0][1];
            vc2[2] = S[1][1];
        }
        // Recompute cov3d from scale and rotation.
        const float es[3] = {exp_cw(sp[3]), exp_cw(sp[4]), exp_cw(sp[5])};
        const M3 R = quat_to_rotmat(q);
        float cov[6];
        {
            M3 M;
#pragma unroll
            for (int j = 0; j < 3; ++j)
#pragma unroll
                for (int i = 0; i < 3; ++i) M.m[j][i] = R.m[j][i] * (p.glob_scale * es[j]);
            auto t = [&](int i, int j) {
                return M.m[0][i] * M.m[0][j] + M.m[1][i] * M.m[1][j] + M.m[2][i] * M.m[2][j];
            };
            cov[0] = t(0, 0); cov[1] = t(1, 0); cov[2] = t(2, 0);
            cov[3] = t(1, 1); cov[4] = t(2, 1); cov[5] = t(2, 2);
        }
        // project_cov3d_ewa_vjp.
        float vcov3[6];
        {
            const float* w = p.vm;
            F3 pv{w[0] * pw.x + w[1] * pw.y + w[2] * pw.z + w[3],
                  w[4] * pw.x + w[5] * pw.y + w[6] * pw.z + w[7],
                  w[8] * pw.x + w[9] * pw.y + w[10] * pw.z + w[11]};
            const float tan_fovx = 0.5f * (float)p.W / p.fx, tan_fovy = 0.5f * (float)p.H / p.fy;
            const float lim_x = 1.3f * tan_fovx, lim_y = 1.3f * tan_fovy;
            const float rz = rcp_hw(pv.z), rz2 = rz * rz;
            pv.x = pv.z * fminf(lim_x, fmaxf(-lim_x, pv.x * rz));
            pv.y = pv.z * fminf(lim_y, fmaxf(-lim_y, pv.y * rz));
            M3 Wm;
            Wm.m[0][0] = w[0]; Wm.m[0][1] = w[4]; Wm.m[0][2] = w[8];
            Wm.m[1][0] = w[1]; Wm.m[1][1] = w[5]; Wm.m[1][2] = w[9];
            Wm.m[2][0] = w[2]; Wm.m[2][1] = w[6]; Wm.m[2][2] = w[10];
            M3 J;
            J.m[0][0] = p.fx * rz; J.m[0][1] = 0.f; J.m[0][2] = 0.f;
            J.m[1][0] = 0.f; J.m[1][1] = p.fy * rz; J.m[1][2] = 0.f;
            J.m[2][0] = -p.fx * pv.x * rz2; J.m[2][1] = -p.fy * pv.y * rz2; J.m[2][2] = 0.f;
            M3 V;
            V.m[0][0] = cov[0]; V.m[0][1] = cov[1]; V.m[0][2] = cov[2];
            V.m[1][0] = cov[1]; V.m[1][1] = cov[3]; V.m[1][2] = cov[4];
            V.m[2][0] = cov[2]; V.m[2][1] = cov[4]; V.m[2][2] = cov[5];
            M3 vc;
            vc.m[0][0] = vc2[0]; vc.m[0][1] = 0.5f * vc2[1]; vc.m[0][2] = 0.f;
            vc.m[1][0] = 0.5f * vc2[1]; vc.m[1][1] = vc2[2]; vc.m[1][2] = 0.f;
            vc.m[2][0] = 0.f; vc.m[2][1] = 0.f; vc.m[2][2] = 0.f;
            const M3 T = mat_mul(J, Wm);
            const M3 vV = mat_mul(mat_mul(transpose(T), vc), T);
            const M3 A1 = mat_mul(mat_mul(vc, T), transpose(V));
            const M3 A2 = mat_mul(mat_mul(transpose(vc), T), V);
            M3 vT;
#pragma unroll
            for (int i = 0; i < 3; ++i)
#pragma unroll
                for (int j = 0; j < 3; ++j) vT.m[i][j] = A1.m[i][j] + A2.m[i][j];
            vcov3[0] = vV.m[0][0];
            vcov3[1] = vV.m[0][1] + vV.m[1][0];
            vcov3[2] = vV.m[0][2] + vV.m[2][0];
            vcov3[3] = vV.m[1][1];
            vcov3[4] = vV.m[1][2] + vV.m[2][1];
            vcov3[5] = vV.m[2][2];
            const M3 vJ = mat_mul(vT, transpose(Wm));
            const float fx_rz2 = p.fx * rz2, fy_rz2 = p.fy * rz2, rz3 = rz2 * rz;
            const F3 vt{-fx_rz2 * vJ.m[2][0], -fy_rz2 * vJ.m[2][1],
                        -fx_rz2 * vJ.m[0][0] + 2.f * p.fx * pv.x * rz3 * vJ.m[2][0] -
                            fy_rz2 * vJ.m[1][1] + 2.f * p.fy * pv.y * rz3 * vJ.m[2][1]};
            vm.x += dot3(vt, F3{Wm.m[0][0], Wm.m[0][1], Wm.m[0][2]});
            vm.y += dot3(vt, F3{Wm.m[1][0], Wm.m[1][1], Wm.m[1][2]});
            vm.z += dot3(vt, F3{Wm.m[2][0], Wm.m[2][1], Wm.m[2][2]});
        }
        // scale_rot_to_cov3d_vjp + chain rule through exp.
        {
            M3 vV;
            vV.m[0][0] = vcov3[0]; vV.m[0][1] = 0.5f * vcov3[1]; vV.m[0][2] = 0.5f * vcov3[2];
            vV.m[1][0] = 0.5f * vcov3[1]; vV.m[1][1] = vcov3[3]; vV.m[1][2] = 0.5f * vcov3[4];
            vV.m[2][0] = 0.5f * vcov3[2]; vV.m[2][1] = 0.5f * vcov3[4]; vV.m[2][2] = vcov3[5];
            M3 S{};
            S.m[0][0] = p.glob_scale * es[0];
            S.m[1][1] = p.glob_scale * es[1];
            S.m[2][2] = p.glob_scale * es[2];
            const M3 M = mat_mul(R, S);
            M3 vM = mat_mul(vV, M);
#pragma unroll
            for (int i = 0; i < 3; ++i)
#pragma unroll
                for (int j = 0; j < 3; ++j) vM.m[i][j] = 2.f * vM.m[i][j];
#pragma unroll
            for (int i = 0; i < 3; ++i)
                vs[i] = dot3(F3{R.m[i][0], R.m[i][1], R.m[i][2]},
                             F3{vM.m[i][0], vM.m[i][1], vM.m[i][2]}) * es[i];
            const M3 vR = mat_mul(vM, S);
            const float s = rcp_hw(sqrt_hw(q.w * q.w + q.x * q.x + q.y * q.y + q.z * q.z));
            const float w = q.x * s, x = q.y * s, y = q.z * s, z = q.w * s;
            const auto& Rv = vR.m;
            vq[0] = 2.f * (x * (Rv[1][2] - Rv[2][1]) + y * (Rv[2][0] - Rv[0][2]) +
                           z * (Rv[0][1] - Rv[1][0]));
            vq[1] = 2.f * (-2.f * x * (Rv[1][1] + Rv[2][2]) + y * (Rv[0][1] + Rv[1][0]) +
                           z * (Rv[0][2] + Rv[2][0]) + w * (Rv[1][2] - Rv[2][1]));
            vq[2] = 2.f * (x * (Rv[0][1] + Rv[1][0]) - 2.f * y * (Rv[0][0] + Rv[2][2]) +
                           z * (Rv[1][2] + Rv[2][1]) + w * (Rv[2][0] - Rv[0][2]));
            vq[3] = 2.f * (x * (Rv[0][2] + Rv[2][0]) + y * (Rv[1][2] + Rv[2][1]) -
                           2.f * z * (Rv[0][0] + Rv[1][1]) + w * (Rv[0][1] - Rv[1][0]));
        }
        // f_dc Adam (visible only) and densify statistics.
#pragma unroll
        for (int c = 0; c < 3; ++c)
            adam_elem(dp[c], dm[c], dv[c], SH_C0 * vrgb[c], hp.step[3], hp.b1, hp.b2, hp.inv_bc2[3],
                      hp.eps);
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            P.params[3][3 * (size_t)g + c] = dp[c];
            st_nt(P.m[3] + 3 * (size_t)g + c, dm[c]);
            st_nt(P.v[3] + 3 * (size_t)g + c, dv[c]);
        }
        vis[g] = st_vis + 1.0f;
        gnorm[g] = st_gnorm + sqrtf(vxy0 * vxy0 + vxy1 * vxy1);
        max2d[g] = fmaxf(st_max2d, (float)rad * inv_max_dim);
    }
    if (v_mean_out && live) {
        v_mean_out[3 * g] = vm.x; v_mean_out[3 * g + 1] = vm.y; v_mean_out[3 * g + 2] = vm.z;
    }
    if (v_scale_out && live) {
        v_scale_out[3 * g] = vs[0]; v_scale_out[3 * g + 1] = vs[1]; v_scale_out[3 * g + 2] = vs[2];
    }
    if (v_quat_out && live) {
        v_quat_out[4 * g] = vq[0]; v_quat_out[4 * g + 1] = vq[1];
        v_quat_out[4 * g + 2] = vq[2]; v_quat_out[4 * g + 3] = vq[3];
    }
    // Dense Adam on means, scales, quats, opacities.
    const float gr[11] = {vm.x, vm.y, vm.z, vs[0], vs[1], vs[2], vq[0], vq[1], vq[2], vq[3], v_op};
    const int grp[11] = {0, 0, 0, 1, 1, 1, 2, 2, 2, 2, 5};
#pragma unroll
    for (int k = 0; k < 11; ++k)
        adam_elem(sp[k], sm[k], sv[k], gr[k], hp.step[grp[k]], hp.b1, hp.b2, hp.inv_bc2[grp[k]], hp.eps);
#pragma unroll
    for (int k = 0; k < 3; ++k) {
        s3[0][3 * t + k] = sp[k];
        s3[1][3 * t + k] = sm[k];
        s3[2][3 * t + k] = sv[k];
        s3[3][3 * t + k] = sp[3 + k];
        s3[4][3 * t + k] = sm[3 + k];
        s3[5][3 * t + k] = sv[3 + k];
    }
    if (live) {
        reinterpret_cast<float4*>(P.params[2])[g] = make_float4(sp[6], sp[7], sp[8], sp[9]);
        st_nt4(P.m[2] + 4 * (size_t)g, make_float4(sm[6], sm[7], sm[8], sm[9]));
        st_nt4(P.v[2] + 4 * (size_t)g, make_float4(sv[6], sv[7], sv[8], sv[9]));
        P.params[5][g] = sp[10];
        st_nt(P.m[5] + g, sm[10]);
        st_nt(P.v[5] + g, sv[10]);
    }
    __syncthreads();
    stage_rows3<true>(arr3, 3 * (size_t)g0, nf, vec3 != 0, s3);
}

}  // namespace

void launch_sh_rest_adam(hipStream_t s, const CamParams& p, const float4* rec, const int* radii,
                         const float* gacc, float* f_rest, float* m, float* v, const AdamHP& hp) {
    const int dtu = p.dtu < 3 ? p.dtu : 3;
    const int n_used = dtu >= 3 ? 15 : dtu == 2 ? 8 : dtu == 1 ? 3 : 0;
    if (n_used == 0 || p.rest_per == 0 || p.N <= 0) return;
    const int64_t n = (int64_t)p.N * p.rest_per;
    const int64_t blocks = (n + SHA_E - 1) / SHA_E;
    hipLaunchKernelGGL(k_sh_rest_adam, dim3((unsigned)blocks), dim3(SHA_T), 0, s, n, p.rest_per,
                       n_used, rec, radii, gacc, f_rest, m, v, hp);
}

void launch_proj_bwd_adam(hipStream_t s, const CamParams& p, float* const params[6],
                          float* const m[6], float* const v[6], const AdamHP& hp, GaussOut go,
                          const float* gacc, float* vis, float* gnorm, float* max2d,
                          float inv_max_dim, float* v_mean_out, float* v_scale_out,
                          float* v_quat_out) {
    if (p.N <= 0) return;
    BwdPtrs P;
    for (int i = 0; i < 6; ++i) { P.params[i] = params[i]; P.m[i] = m[i]; P.v[i] = v[i]; }
    bool vec3 = true;
    for (int i = 0; i < 2; ++i)
        for (const float* q : {params[i], m[i], v[i]})
            vec3 = vec3 && reinterpret_cast<uintptr_t>(q) % 16 == 0;
    hipLaunchKernelGGL(k_proj_bwd_adam, dim3((p.N + PBA_T - 1) / PBA_T), dim3(PBA_T), 0, s, p, P,
                       hp, go, gacc, vis, gnorm, max2d, inv_max_dim, v_mean_out, v_scale_out,
                       v_quat_out, vec3 ? 1 : 0);
}


}  // namespace msp
