// ssim.hip — separable 11-tap SSIM + L1 loss, forward and backward, on
// LDS-staged tiles with halos.
//
// Two passes with the reference's training semantics:
//   h-fwd + v-fwd + h-bwd   ssim_h_fwd_kernel (.metal:3053-3115) and
//                ssim_fused_v_fwd_h_bwd_kernel (.metal:3226-3313) in one
//                workgroup per 16x16 tile: the horizontal zero-padded sums of
//                x=gt, y=render (mu_x, mu_y, E[x^2], E[y^2], E[xy]) for the
//                tile rows +-5 and columns +-5 are computed into LDS from the
//                input (no intermediate buffer), then the vertical sums ->
//                SSIM and its derivative fields f1, f2, f3 at every centre of
//                the tile rows, including the 5-column halo outside the image
//                (whose zero statistics give f = (0, -2/C2, 2/C2)), then the
//                mirrored horizontal pass
//   v-bwd        ssim_v_bwd_kernel (.metal:3396-3464): mirrored vertical pass
//                (rows outside the image contribute nothing) and the
//                combination with the L1 sign term.
// Every sum is accumulated in the same order as the reference's separate
// kernels, so the fusion changes no bit of the result.  Each window term is
// added with one fused multiply-add (w gv gv as the product w gv, then an
// fma with gv): the reference writes a product and a sum, which its
// fast-math Metal build may contract the same way; the CPU oracle evaluates
// exactly these operations.
// The loss is reduced per workgroup into (sum SSIM, sum L1, pixel count) and
// folded by one final workgroup in a fixed order; it equals the sum over
// pixels of w*(1 - mean_c SSIM) + (1-w)*mean_c |gt - r|.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

constexpr int HALF = 5;
constexpr int WIN = 11;

// Fused forward / derivative / horizontal-backward tile: FX x FY output
// pixels per workgroup of FT threads.  The horizontal sums are needed at
// (FY + 10) x (FX + 10) positions and the derivative fields at FY x (FX + 10),
// so a wide tile spends less of its work on the halo than a 16 x 16 one;
// staging one channel at a time keeps the LDS at 48 KB for three
// workgroups (six waves per SIMD) per CU.
constexpr int FX = 32, FY = 16, FT = FX * FY;
constexpr int FHX = FX + 2 * HALF;   // 42: columns with horizontal sums / fields
constexpr int FHY = FY + 2 * HALF;   // 26: rows with horizontal sums
constexpr int FIN = FHX + 2 * HALF;  // 52: input columns
// LDS layouts, chosen so that every read of the three passes is free of bank
// conflicts (64 banks of 4 bytes; a wave's 8-byte reads are served 32 lanes
// at a time, its 16-byte reads 16 lanes at a time):
//  * input: (gt, render) of a position as one float2, rows FIN_S float2
//    apart.  The horizontal pass gives lane l the position p + l of a
//    row-major walk over FHY x FHX, so 32 lanes cover at most two row pieces,
//    [a, 42) of one row and [0, a - 10) of the next; FIN_S = 74 = 10 (mod 32)
//    puts the second piece on exactly the 8-byte bank pairs the first leaves.
//  * horizontal sums: (mu_x, mu_y, E[x^2], E[y^2]) as a float4 and E[xy] as a
//    float, row-major over FHY x FHX (the passes' lanes read consecutive
//    positions).
//  * derivative fields (f1, f2, f3) as one float4 per position: the
//    horizontal backward's 16-lane quarters read 16 consecutive positions of
//    one row.
constexpr int FIN_S = 74;

__global__ __launch_bounds__(FT) void k_ssim_fused(int W, int H, const float* __restrict__ img,
                                                   const float* __restrict__ gt,
                                                   float* __restrict__ dbuf,
                                                   float* __restrict__ loss_part) {
    __shared__ float2 s_in[FHY * FIN_S];     // (gt, render) of one channel, rows y0-5.., cols x0-10..
    __shared__ float4 s_h4[FHY * FHX];       // mu_x, mu_y, E[x^2], E[y^2]
    __shared__ float s_h1[FHY * FHX];        // E[xy]
    __shared__ float4 s_f[FY * FHX];         // f1, f2, f3, (unused)
    __shared__ float s_red[3][FT / 64];
    const int tr = threadIdx.x, lx = tr % FX, ly = tr / FX;
    const int bx = blockIdx.x * FX - HALF, by = blockIdx.y * FY - HALF;
    float ssim_sum = 0.f, l1_sum = 0.f, cnt = 0.f;
    // The three channels of this thread's input pixels (rows by .. by+25,
    // columns bx-5 .. bx+46, zero outside the image) are loaded once, into
    // registers; each channel pass copies its component into LDS.
    constexpr int NPOS = (FHY * FIN + FT - 1) / FT;
    float rg[NPOS][3], rr[NPOS][3];
#pragma unroll
    for (int k = 0; k < NPOS; ++k) {
        const int i = tr + k * FT;
        const int sy = i / FIN, sx = i - sy * FIN;
        const int gy = by + sy, gx = bx - HALF + sx;
        const bool in = i < FHY * FIN && gx >= 0 && gx < W && gy >= 0 && gy < H;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const size_t q = ((size_t)gy * W + gx) * 3 + c;
            rg[k][c] = in ? gt[q] : 0.f;
            rr[k][c] = in ? img[q] : 0.f;
        }
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        if (c > 0) __syncthreads();
#pragma unroll
        for (int k = 0; k < NPOS; ++k) {
            const int i = tr + k * FT;
            if (i < FHY * FIN) {
                const int sy = i / FIN, sx = i - sy * FIN;
                s_in[sy * FIN_S + sx] = make_float2(rg[k][c], rr[k][c]);
            }
        }
        __syncthreads();
        // horizontal zero-padded sums (ssim_h_fwd, .metal:3053-3115) at the
        // in-image positions of rows by.., columns bx..; zero elsewhere
        for (int i = tr; i < FHY * FHX; i += FT) {
            const int sy = i / FHX, sx = i - sy * FHX, gy = by + sy, gx = bx + sx;
            float mx = 0.f, my = 0.f, sxx = 0.f, syy = 0.f, cxy = 0.f;
            if (gx >= 0 && gx < W && gy >= 0 && gy < H) {
                const float2* row = s_in + sy * FIN_S + sx;
#pragma unroll
                for (int d = 0; d < WIN; ++d) {
                    const float w = GAUSS_1D[d];
                    const float2 v = row[d];
                    const float gv = v.x, rv = v.y;
                    const float wg = w * gv, wr = w * rv;
                    mx = fmaf(w, gv, mx);
                    my = fmaf(w, rv, my);
                    sxx = fmaf(wg, gv, sxx);
                    syy = fmaf(wr, rv, syy);
                    cxy = fmaf(wg, rv, cxy);
                }
            }
            s_h4[i] = make_float4(mx, my, sxx, syy);
            s_h1[i] = cxy;
        }
        __syncthreads();
        for (int i = tr; i < FY * FHX; i += FT) {
            const int dy = i / FHX, dx = i - dy * FHX;
            float mx = 0.f, my = 0.f, sx = 0.f, sy = 0.f, cxy = 0.f;
#pragma unroll
            for (int k = 0; k < WIN; ++k) {
                const float w = GAUSS_1D[k];
                const float4 h = s_h4[i + k * FHX];
                const float h4 = s_h1[i + k * FHX];
                mx = fmaf(w, h.x, mx);
                my = fmaf(w, h.y, my);
                sx = fmaf(w, h.z, sx);
                sy = fmaf(w, h.w, sy);
                cxy = fmaf(w, h4, cxy);
            }
            const float sxs = sx - mx * mx, sys = sy - my * my, sxy = cxy - mx * my;
            const float A = 2.0f * mx * my + SSIM_C1, B = 2.0f * sxy + SSIM_C2;
            const float Cd = mx * mx + my * my + SSIM_C1, D = sxs + sys + SSIM_C2;
            const float iCD = 1.0f / (Cd * D);
            const float dmu = 2.0f * B * (mx * Cd - A * my) / (Cd * Cd * D);
            const float dsyq = -A * B * iCD / D, dsxy = 2.0f * A * iCD;
            s_f[i] = make_float4(dmu - 2.0f * my * dsyq - mx * dsxy, 2.0f * dsyq, dsxy, 0.f);
            if (dx >= HALF && dx < HALF + FX) {
                const int gpx = bx + dx, gpy = by + dy + HALF;
                if (gpx >= 0 && gpx < W && gpy >= 0 && gpy < H) {
                    ssim_sum += (A * B) / (Cd * D);
                    const float2 v = s_in[(dy + HALF) * FIN_S + dx + HALF];
                    l1_sum += fabsf(v.x - v.y);
                    if (c == 0) cnt += 1.f;
                }
            }
        }
        __syncthreads();
        const int px = blockIdx.x * FX + lx, py = blockIdx.y * FY + ly;
        if (px < W && py < H) {
            float h1 = 0.f, h2 = 0.f, h3 = 0.f;
            const float4* fr = s_f + ly * FHX + lx;
#pragma unroll
            for (int d = 0; d < WIN; ++d) {
                const float w = GAUSS_1D[WIN - 1 - d];
                const float4 f = fr[d];
                h1 = fmaf(w, f.x, h1);
                h2 = fmaf(w, f.y, h2);
                h3 = fmaf(w, f.z, h3);
            }
            float* o = dbuf + ((size_t)py * W + px) * 9 + c * 3;
            o[0] = h1;
            o[1] = h2;
            o[2] = h3;
        }
    }
    // Workgroup partials of (sum SSIM, sum L1, pixels).
    const float a = wave_sum(ssim_sum), b = wave_sum(l1_sum), n = wave_sum(cnt);
    if ((tr & 63) == 0) {
        s_red[0][tr >> 6] = a;
        s_red[1][tr >> 6] = b;
        s_red[2][tr >> 6] = n;
    }
    __syncthreads();
    if (tr < 3) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < FT / 64; ++k) v += s_red[tr][k];
        loss_part[((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 3 + tr] = v;
    }
}

// Vertical backward tile: VX columns x VY rows of output pixels, 256
// threads, each thread VY / 16 rows.  The derivative fields of the tile's
// columns are read row by row as contiguous floats (VX pixels x 9 values),
// so the loads are coalesced; VY + 10 rows are read for VY outputs.  They
// are kept in LDS in the same order ([row][column][9]): the staging writes
// are consecutive, and a wave's reads of one field (4 rows x 16 columns,
// 64 consecutive positions) are 9 floats apart, an odd stride that puts the
// 64 lanes on 64 different banks.
constexpr int VX = 16, VY = 32, VR = VY + 2 * HALF;

__global__ __launch_bounds__(256) void k_ssim_v_bwd(int W, int H, const float* __restrict__ img,
                                                    const float* __restrict__ gt,
                                                    const float* __restrict__ dbuf, float w_ssim,
                                                    float inv_n, float* __restrict__ v_rendered) {
    __shared__ float s_h[VR * VX * 9];   // rows by.., columns bx.., 9 fields (channel c: 3c..3c+2)
    const int tr = threadIdx.x, lx = tr & 15, ly = tr >> 4;
    const int bx = blockIdx.x * VX, by = blockIdx.y * VY - HALF;
    const int nf = min(VX, W - bx) * 9;   // in-image floats of a row
    constexpr int ROWF = VX * 9;
    for (int i = tr; i < VR * ROWF; i += 256) {
        const int sy = i / ROWF, f = i - sy * ROWF;
        const int gy = by + sy;
        float v = 0.f;
        if (f < nf && gy >= 0 && gy < H) v = dbuf[((size_t)gy * W + bx) * 9 + f];
        s_h[i] = v;
    }
    __syncthreads();
    const int px = bx + lx;
    if (px >= W) return;
#pragma unroll
    for (int rr = 0; rr < VY / 16; ++rr) {
        const int oy = ly + 16 * rr, py = blockIdx.y * VY + oy;
        if (py >= H) break;
        for (int c = 0; c < 3; ++c) {
            const float* h1 = s_h + (oy * VX + lx) * 9 + c * 3;
            float f1 = 0.f, f2 = 0.f, f3 = 0.f;
#pragma unroll
            for (int d = 0; d < WIN; ++d) {
                const float w = GAUSS_1D[WIN - 1 - d];
                f1 = fmaf(w, h1[d * VX * 9], f1);
                f2 = fmaf(w, h1[d * VX * 9 + 1], f2);
                f3 = fmaf(w, h1[d * VX * 9 + 2], f3);
            }
            const size_t q = ((size_t)py * W + px) * 3 + c;
            const float r = img[q], g = gt[q];
            const float v_ssim = f1 + r * f2 + g * f3;
            const float v_l1 = (g > r) ? -1.0f : ((g < r) ? 1.0f : 0.0f);
            v_rendered[q] = inv_n * (-w_ssim * v_ssim + (1.0f - w_ssim) * v_l1);
        }
    }
}

// Final fold of the workgroup partials in a fixed order (float64): thread t
// adds parts t, t + 1024, ... in order, then a tree over the 1024 threads.
constexpr int LF_T = 1024;
__global__ __launch_bounds__(LF_T) void k_loss_final(int nparts, const float* __restrict__ part,
                                                     float w_ssim, float* __restrict__ out) {
    __shared__ double s[3][LF_T];
    double a = 0.0, b = 0.0, n = 0.0;
    for (int i = threadIdx.x; i < nparts; i += LF_T) {
        a += part[3 * i];
        b += part[3 * i + 1];
        n += part[3 * i + 2];
    }
    s[0][threadIdx.x] = a;
    s[1][threadIdx.x] = b;
    s[2][threadIdx.x] = n;
    __syncthreads();
    for (int off = LF_T / 2; off > 0; off >>= 1) {
        if ((int)threadIdx.x < off)
            for (int k = 0; k < 3; ++k) s[k][threadIdx.x] += s[k][threadIdx.x + off];
        __syncthreads();
    }
    if (threadIdx.x == 0) {
        const double w = w_ssim;
        // out may be coherent host memory that the host reads without a
        // stream sync: a system-scope store makes the value visible there
        __hip_atomic_store(out, (float)(w * s[2][0] - (w / 3.0) * s[0][0] + ((1.0 - w) / 3.0) * s[1][0]),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
}

}  // namespace

void launch_ssim(hipStream_t s, int H, int W, const float* img, const float* gt, float w,
                 float inv_n, float* dbuf, float* v_rendered, float* loss_part, float* loss_out) {
    const dim3 fgrid((W + FX - 1) / FX, (H + FY - 1) / FY);
    hipLaunchKernelGGL(k_ssim_fused, fgrid, dim3(FT), 0, s, W, H, img, gt, dbuf, loss_part);
    const dim3 grid((W + VX - 1) / VX, (H + VY - 1) / VY);
    hipLaunchKernelGGL(k_ssim_v_bwd, grid, dim3(256), 0, s, W, H, img, gt, dbuf, w, inv_n,
                       v_rendered);
    hipLaunchKernelGGL(k_loss_final, dim3(1), dim3(LF_T), 0, s, (int)(fgrid.x * fgrid.y),
                       loss_part, w, loss_out);
}

}  // namespace msp
