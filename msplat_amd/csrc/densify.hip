// densify.hip — GPU-resident densification: classify, split / duplicate
// append, cull classify and stable compaction of all 18 per-gaussian buffers.
//
// Reference: msplat_densify (msplat_metal.mm:1337-1592) with
// densify_classify_kernel (.metal:3475-3509), densify_append_split_kernel
// (.metal:3514-3600), densify_append_dup_kernel (.metal:3604-3651),
// densify_cull_classify_kernel (.metal:3656-3694), compact_scatter /
// compact_copy_back (.metal:3698-3729) and the two-level block scan
// (.metal:2368-2439).  The scans here are three-pass (block totals, scan of
// the totals, block scans with offsets) over 1024-element blocks.
//
// Compaction: the reference scatters and copies back each of the 18 buffers
// in its own pair of passes over the 3N-row worst case.  Here the host reads
// the kept count after the keep scan, then one kernel gathers every kept row
// of all 18 buffers, in order, into a packed workspace and one kernel copies
// the packed rows back (float4 stores): three launches sized by the rows that
// exist.  The order is the same stable keep-prefix order.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

__device__ __forceinline__ uint64_t splitmix64(uint64_t z) {
    z += 0x9E3779B97F4A7C15ull;
    z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
    z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
    return z ^ (z >> 31);
}

// Box–Muller from two counter-hashed uniforms per output element.
__global__ __launch_bounds__(256) void k_randn(float* __restrict__ dst, int64_t n, uint64_t seed) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    const uint64_t a = splitmix64(seed ^ (2ull * (uint64_t)i) * 0xD1B54A32D192ED03ull);
    const uint64_t b = splitmix64(a ^ 0x8BB84B93962EACC9ull);
    const float u1 = (float)((a >> 40) + 1) * (1.0f / 16777216.0f);   // (0, 1]
    const float u2 = (float)(b >> 40) * (1.0f / 16777216.0f);         // [0, 1)
    dst[i] = sqrtf(-2.0f * logf(u1)) * cosf(6.283185307179586f * u2);
}

__global__ __launch_bounds__(256) void k_classify(DensifyHP hp, const float* __restrict__ gnorm,
                                                  const float* __restrict__ vis,
                                                  const float* __restrict__ scales,
                                                  const float* __restrict__ max2d,
                                                  int* __restrict__ split, int* __restrict__ dup) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= hp.N) return;
    const float vc = vis[i];
    if (vc <= 0.0f) {
        split[i] = 0;
        dup[i] = 0;
        return;
    }
    const float avg = (gnorm[i] / vc) * hp.half_max_dim;
    const bool high = avg > hp.grad_thresh;
    const float mx = fmaxf(fmaxf(exp_cw(scales[3 * i]), exp_cw(scales[3 * i + 1])),
                           exp_cw(scales[3 * i + 2]));
    const bool large = mx > hp.size_thresh;
    bool do_split = large;
    if (hp.check_screen && max2d[i] > hp.screen_thresh) do_split = true;
    do_split = do_split && high;
    split[i] = do_split ? 1 : 0;
    dup[i] = (!large && high) ? 1 : 0;
}

struct Bufs18 {
    float* b[6];
    float* m[6];
    float* v[6];
};

__global__ __launch_bounds__(256) void k_append_split(int N, int fr, const int* __restrict__ split,
                                                      const int* __restrict__ sp,
                                                      const float* __restrict__ rnd, float lsf,
                                                      Bufs18 B) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N || split[i] == 0) return;
    const int strides[6] = {3, 3, 4, 3, fr, 1};
    const int ord = sp[i] - 1;
    const float* q = B.b[2] + 4 * (size_t)i;
    float qw = q[0], qx = q[1], qy = q[2], qz = q[3];
    const float ql = sqrtf(qw * qw + qx * qx + qy * qy + qz * qz);
    qw /= ql; qx /= ql; qy /= ql; qz /= ql;
    float* sc = B.b[1];
    float* mb = B.b[0];
    const float sx = exp_cw(sc[3 * i]), sy = exp_cw(sc[3 * i + 1]), sz = exp_cw(sc[3 * i + 2]);
    for (int k = 0; k < 2; ++k) {
        const int ch = N + 2 * ord + k, ri = ord * 2 + k;
        const float r0 = rnd[3 * ri] * sx, r1 = rnd[3 * ri + 1] * sy, r2 = rnd[3 * ri + 2] * sz;
        const float v0 = (1 - 2 * (qy * qy + qz * qz)) * r0 + 2 * (qx * qy - qw * qz) * r1 +
                         2 * (qx * qz + qw * qy) * r2;
        const float v1 = 2 * (qx * qy + qw * qz) * r0 + (1 - 2 * (qx * qx + qz * qz)) * r1 +
                         2 * (qy * qz - qw * qx) * r2;
        const float v2 = 2 * (qx * qz - qw * qy) * r0 + 2 * (qy * qz + qw * qx) * r1 +
                         (1 - 2 * (qx * qx + qy * qy)) * r2;
        mb[3 * (size_t)ch] = mb[3 * (size_t)i] + v0;
        mb[3 * (size_t)ch + 1] = mb[3 * (size_t)i + 1] + v1;
        mb[3 * (size_t)ch + 2] = mb[3 * (size_t)i + 2] + v2;
        for (int j = 0; j < 3; ++j) sc[3 * (size_t)ch + j] = sc[3 * (size_t)i + j] - lsf;
        for (int j = 0; j < 4; ++j) B.b[2][4 * (size_t)ch + j] = B.b[2][4 * (size_t)i + j];
        for (int j = 0; j < 3; ++j) B.b[3][3 * (size_t)ch + j] = B.b[3][3 * (size_t)i + j];
        for (int j = 0; j < fr; ++j) B.b[4][(size_t)fr * ch + j] = B.b[4][(size_t)fr * i + j];
        B.b[5][ch] = B.b[5][i];
        for (int gi = 0; gi < 6; ++gi)
            for (int j = 0; j < strides[gi]; ++j) {
                B.m[gi][(size_t)strides[gi] * ch + j] = 0.f;
                B.v[gi][(size_t)strides[gi] * ch + j] = 0.f;
            }
    }
    for (int j = 0; j < 3; ++j) sc[3 * (size_t)i + j] -= lsf;
}

__global__ __launch_bounds__(256) void k_append_dup(int N, int fr, const int* __restrict__ dup,
                                                    const int* __restrict__ dp,
                                                    const int* __restrict__ sp, Bufs18 B) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= N || dup[i] == 0) return;
    const int strides[6] = {3, 3, 4, 3, fr, 1};
    const int nS = sp[N - 1];
    const int dst = N + 2 * nS + dp[i] - 1;
    for (int gi = 0; gi < 6; ++gi)
        for (int j = 0; j < strides[gi]; ++j) {
            B.b[gi][(size_t)strides[gi] * dst + j] = B.b[gi][(size_t)strides[gi] * i + j];
            B.m[gi][(size_t)strides[gi] * dst + j] = 0.f;
            B.v[gi][(size_t)strides[gi] * dst + j] = 0.f;
        }
}

__global__ __launch_bounds__(256) void k_cull(DensifyHP hp, int worst, const int* __restrict__ sp,
                                              const int* __restrict__ dp,
                                              const int* __restrict__ split,
                                              const float* __restrict__ opac,
                                              const float* __restrict__ scales,
                                              const float* __restrict__ max2d,
                                              int* __restrict__ keep) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= worst) return;
    const int N = hp.N;
    const int Nn = N + 2 * sp[N - 1] + dp[N - 1];
    if (i >= Nn) {
        keep[i] = 0;
        return;
    }
    const float os = 1.0f / (1.0f + exp_cw(-opac[i]));
    bool cull = os < hp.cull_alpha;
    if (i < N && split[i] != 0) cull = true;
    if (hp.check_huge) {
        const float mx = fmaxf(fmaxf(exp_cw(scales[3 * (size_t)i]), exp_cw(scales[3 * (size_t)i + 1])),
                               exp_cw(scales[3 * (size_t)i + 2]));
        if (mx > hp.cull_scale) cull = true;
        if (hp.check_screen && i < N && max2d[i] > hp.cull_screen) cull = true;
    }
    keep[i] = cull ? 0 : 1;
}

// Appended rows end at N + 2 nSplits + nDups; count_out = {that, kept rows}.
__global__ void k_read_counts(int N, const int* sp, const int* dp, const int* kp, int64_t last,
                              int* out) {
    out[0] = N + 2 * sp[N - 1] + dp[N - 1];
    out[1] = kp[last];
}

// src_of[r] = the r-th kept row (rows i < n with keep[i], in order).
__global__ __launch_bounds__(256) void k_keep_sources(const int* __restrict__ keep,
                                                      const int* __restrict__ kp, int n,
                                                      int* __restrict__ src_of) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n && keep[i]) src_of[kp[i] - 1] = i;
}

// Workspace layout of the 18 buffers (parameters, first moments, second
// moments; six groups each): buffer k holds cnt rows of stride st[k] floats
// at float offset off[k] (a multiple of 4).
struct Packed18 {
    const float* src[18];
    float* dst[18];
    int st[18];
    int64_t off[18];
    int64_t f4_end[18];   // cumulative float4 count of the copy-back, buffers 0..k
    int vec[18];          // the buffer is 16-byte aligned (float4 stores)
};

// Gather: workgroup b takes output rows [256 b, 256 b + 256) of every buffer,
// reading each row from its source row (rows of one workgroup come mostly
// from consecutive sources, so reads coalesce like the writes).
__global__ __launch_bounds__(256) void k_gather_rows(Packed18 P, const int* __restrict__ src_of,
                                                     int cnt, float* __restrict__ ws) {
    __shared__ int s_src[256];
    const int r0 = blockIdx.x * 256, tid = threadIdx.x;
    const int nr = min(256, cnt - r0);
    if (tid < nr) s_src[tid] = src_of[r0 + tid];
    __syncthreads();
    for (int k = 0; k < 18; ++k) {
        const int st = P.st[k];
        if (st == 0) continue;
        const float* __restrict__ src = P.src[k];
        float* __restrict__ dst = ws + P.off[k] + (int64_t)r0 * st;
        // element e = lr * st + sub, advanced by 256 per step without dividing
        const int q = 256 / st, rem = 256 - q * st;
        int lr = tid / st, sub = tid - lr * st;
        for (int e = tid; e < nr * st; e += 256) {
            dst[e] = src[(int64_t)s_src[lr] * st + sub];
            lr += q;
            sub += rem;
            if (sub >= st) { sub -= st; ++lr; }
        }
    }
}

// Copy-back of the packed rows: one thread per float4 of the 18 buffers'
// kept rows; the workspace regions are 16-byte aligned, a buffer's last
// float4 may be partial, and a buffer that is not 16-byte aligned is copied
// by scalar stores.
__global__ __launch_bounds__(256) void k_copy_back_rows(Packed18 P, int cnt,
                                                        const float* __restrict__ ws) {
    const int64_t t = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= P.f4_end[17]) return;
    int k = 0;
    while (t >= P.f4_end[k]) ++k;
    const int64_t i = t - (k ? P.f4_end[k - 1] : 0);
    const int64_t nf = (int64_t)cnt * P.st[k];
    const float* s = ws + P.off[k];
    float* d = P.dst[k];
    if (4 * i + 4 <= nf && P.vec[k]) {
        reinterpret_cast<float4*>(d)[i] = reinterpret_cast<const float4*>(s)[i];
    } else {
        // this thread's own four elements only (fewer at the buffer's end)
        const int64_t e_end = 4 * i + 4 < nf ? 4 * i + 4 : nf;
        for (int64_t e = 4 * i; e < e_end; ++e) d[e] = s[e];
    }
}

// Opacity reset of afterTrain (model.cpp:280-287): logits above hi become hi.
__global__ __launch_bounds__(256) void k_clamp_max(float* __restrict__ p, int64_t n, float hi) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) p[i] = p[i] > hi ? hi : p[i];
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void launch_randn(hipStream_t s, float* dst, int64_t n, uint64_t seed) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_randn, dim3(blocks_for(n)), dim3(256), 0, s, dst, n, seed);
}

void launch_clamp_max(hipStream_t s, float* p, int64_t n, float hi) {
    if (n <= 0) return;
    hipLaunchKernelGGL(k_clamp_max, dim3(blocks_for(n)), dim3(256), 0, s, p, n, hi);
}

void launch_densify(hipStream_t s, const DensifyHP& hp, const float* gnorm, const float* vis,
                    const float* max2d, float* const bufs[6], float* const m[6],
                    float* const v[6], const float* rnd, int* split, int* dup, int* sp, int* dp,
                    int* keep, int* kp, int* tot, int* counts_out) {
    const int N = hp.N;
    const int64_t worst = 3 * (int64_t)N;
    Bufs18 B;
    for (int i = 0; i < 6; ++i) { B.b[i] = bufs[i]; B.m[i] = m[i]; B.v[i] = v[i]; }
    hipLaunchKernelGGL(k_classify, dim3(blocks_for(N)), dim3(256), 0, s, hp, gnorm, vis, bufs[1],
                       max2d, split, dup);
    launch_scan_i32(s, split, sp, N, tot);
    launch_scan_i32(s, dup, dp, N, tot);
    hipLaunchKernelGGL(k_append_split, dim3(blocks_for(N)), dim3(256), 0, s, N, hp.fr,
                       (const int*)split, (const int*)sp, rnd, logf(1.6f), B);
    hipLaunchKernelGGL(k_append_dup, dim3(blocks_for(N)), dim3(256), 0, s, N, hp.fr,
                       (const int*)dup, (const int*)dp, (const int*)sp, B);
    hipLaunchKernelGGL(k_cull, dim3(blocks_for(worst)), dim3(256), 0, s, hp, (int)worst,
                       (const int*)sp, (const int*)dp, (const int*)split, (const float*)bufs[5],
                       (const float*)bufs[1], max2d, keep);
    launch_scan_i32(s, keep, kp, worst, tot);
    hipLaunchKernelGGL(k_read_counts, dim3(1), dim3(1), 0, s, N, (const int*)sp, (const int*)dp,
                       (const int*)kp, worst - 1, counts_out);
}

int64_t densify_workspace_floats(int cnt, int fr) {
    const int64_t rows = ((int64_t)cnt + 3) & ~(int64_t)3;
    return rows * 3 * (3 + 3 + 4 + 3 + fr + 1);
}

void launch_densify_compact(hipStream_t s, int rows, int cnt, int fr, float* const bufs[6],
                            float* const m[6], float* const v[6], const int* keep,
                            const int* kp, int* src_of, float* ws) {
    if (cnt <= 0) return;
    const int strides[6] = {3, 3, 4, 3, fr, 1};
    const int64_t cap = ((int64_t)cnt + 3) & ~(int64_t)3;
    Packed18 P;
    int64_t off = 0, f4 = 0;
    for (int k = 0; k < 18; ++k) {
        const int g = k % 6, set = k / 6;
        float* b = set == 0 ? bufs[g] : set == 1 ? m[g] : v[g];
        P.src[k] = b;
        P.dst[k] = b;
        P.st[k] = strides[g];
        P.off[k] = off;
        P.vec[k] = (reinterpret_cast<uintptr_t>(b) & 15) == 0;
        off += cap * strides[g];
        f4 += ((int64_t)cnt * strides[g] + 3) / 4;
        P.f4_end[k] = f4;
    }
    hipLaunchKernelGGL(k_keep_sources, dim3(blocks_for(rows)), dim3(256), 0, s, keep, kp, rows,
                       src_of);
    hipLaunchKernelGGL(k_gather_rows, dim3(blocks_for(cnt)), dim3(256), 0, s, P,
                       (const int*)src_of, cnt, ws);
    hipLaunchKernelGGL(k_copy_back_rows, dim3(blocks_for(f4)), dim3(256), 0, s, P, cnt,
                       (const float*)ws);
}

}  // namespace msp
