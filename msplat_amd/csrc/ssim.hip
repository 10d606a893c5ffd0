// ssim.hip — separable 11-tap SSIM + L1 loss, forward and backward, in one
// LDS-staged tile kernel.
//
// The reference's training semantics, in five separable passes per channel:
//   h-fwd        ssim_h_fwd_kernel (.metal:3053-3115): horizontal
//                zero-padded sums of x = gt, y = render (mu_x, mu_y, E[x^2],
//                E[y^2], E[xy]) at the in-image positions
//   v-fwd + h-bwd  ssim_fused_v_fwd_h_bwd_kernel (.metal:3226-3313): the
//                vertical sums -> SSIM and its derivative fields f1, f2, f3
//                at every centre of the in-image rows, including the 5-column
//                halo outside the image (whose zero statistics give
//                f = (0, -2/C2, 2/C2)), then the mirrored horizontal pass
//   v-bwd        ssim_v_bwd_kernel (.metal:3396-3464): mirrored vertical pass
//                (rows outside the image contribute nothing) and the
//                combination with the L1 sign term.
// One workgroup computes all five for a TX x TY block of output pixels,
// recomputing the halo each pass needs (rows +-10, columns +-10 of input)
// instead of passing the horizontal-backward fields through memory: the
// only HBM traffic is the two images with their halo and the gradient image.
// Every sum is accumulated in the same order as the reference's separate
// kernels, so the fusion changes no bit of the gradient image.  Each window
// term is added with one fused multiply-add (w gv gv as the product w gv,
// then an fma with gv): the reference writes a product and a sum, which its
// fast-math Metal build may contract the same way; the CPU oracle evaluates
// exactly these operations.
// The loss is reduced per workgroup into (sum SSIM, sum L1, pixel count) and
// folded in a fixed order by one workgroup of the next kernel (loss_fold in
// kernels.hpp); it equals the sum over pixels of
// w*(1 - mean_c SSIM) + (1-w)*mean_c |gt - r|.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

constexpr int HALF = 5;
constexpr int WIN = 11;

// Tile of TX x TY output pixels, NT threads, and the regions of its passes
// (rows / columns relative to the tile's first output pixel (x0, y0)):
//   input (gt, render)    rows -10 .. TY+9,  columns -10 .. TX+9   IN_H x IN_W
//   horizontal sums       rows -10 .. TY+9,  columns -5 .. TX+4    HS_H x HS_W
//   fields f1, f2, f3     rows -5 .. TY+4,   columns -5 .. TX+4    FD_H x FD_W
//   horizontal backward   rows -5 .. TY+4,   columns 0 .. TX-1     FD_H x TX
//   vertical backward     rows 0 .. TY-1,    columns 0 .. TX-1     the outputs
// For 32 x 32 outputs the horizontal sums are evaluated 2.13 times per
// output, the fields 1.72 times and the horizontal backward 1.31 times.  The
// two sum passes take two neighbouring positions per item (along the row for
// the horizontal sums, down the column for the vertical ones): the twelve
// inputs of the pair are read once instead of eleven per position, and the
// vertical pass's 21 x 42 items take one round of the 1024 threads.
constexpr int TX = 32, TY = 32, NT = 1024;
constexpr int IN_W = TX + 4 * HALF;   // 52
constexpr int IN_H = TY + 4 * HALF;   // 52
constexpr int HS_W = TX + 2 * HALF;   // 42
constexpr int HS_H = IN_H;            // 52
constexpr int FD_W = HS_W;            // 42
constexpr int FD_H = TY + 2 * HALF;   // 42
// LDS layouts, chosen so that most of the passes' accesses are free of bank
// conflicts (64 banks of 4 bytes; a wave's 8-byte reads are served 32 lanes at a time,
// its 16-byte reads 16 lanes at a time):
//  * input: (gt, render) of a position as one float2, rows IN_S float2 apart.
//    The horizontal pass gives lane l the position pair p + l of a row-major
//    walk over the HS_H x HS_W / 2 pairs and reads its inputs 16 bytes (two
//    positions) at a time, so 16 lanes cover at most two row pieces, pairs
//    [a, 21) of one row and [0, a - 5) of the next; IN_S = 74 = 10 (mod 32)
//    puts the second piece on exactly the 16-byte bank groups the first
//    leaves.
//  * horizontal sums: (mu_x, mu_y, E[x^2], E[y^2]) as a float4 and E[xy] as a
//    float, row-major over HS_H x HS_W (the vertical pass's lanes read
//    consecutive positions).  Lanes share bank groups where the vertical
//    pass's items wrap to the row pair below and in the horizontal pass's
//    two float4 stores per lane; layouts without those conflicts were
//    measured no faster.
//  * fields (f1, f2, f3) as one float4 per position, row-major over
//    FD_H x FD_W: the horizontal backward's 16-lane quarters read 16
//    consecutive positions of one row.
//  * horizontal backward (h1, h2, h3) as one float4 per position, row-major
//    over FD_H x TX: the vertical backward's lanes read consecutive columns.
// The input and the fields share one LDS area, the horizontal sums and the
// horizontal backward another (each pass reads one and writes the other):
// 74.5 KB, two workgroups per CU; 1024 threads each (at most 64 VGPRs) make
// that eight waves per SIMD, which hide the passes' LDS latency and barriers
// better than 512 threads (four waves per SIMD) did.
constexpr int IN_S = 74;
constexpr int LDS_A = IN_H * IN_S * 8;                  // input; the fields (FD_H x FD_W x 16) fit
constexpr int LDS_B = HS_H * HS_W * (16 + 4);           // horizontal sums; the backward (FD_H x TX x 16) fits
static_assert(FD_H * FD_W * 16 <= LDS_A, "fields overflow the input's area");
static_assert(FD_H * TX * 16 <= LDS_B, "horizontal backward overflows the sums' area");
static_assert(HS_W % 2 == 0 && FD_H % 2 == 0 && IN_S % 2 == 0, "two positions per item, 16-byte aligned");
constexpr int NPOS = (IN_H * IN_W + NT - 1) / NT;      // input positions per thread
constexpr int NOUT = TX * TY / NT;                      // output pixels per thread

__global__ __launch_bounds__(NT) __attribute__((amdgpu_waves_per_eu(8))) void k_ssim_tile(int W, int H, const float* __restrict__ img,
                                                  const float* __restrict__ gt, float w_ssim,
                                                  float inv_n, float* __restrict__ v_rendered,
                                                  float* __restrict__ loss_part) {
    __shared__ __align__(16) char lds_a[LDS_A];
    __shared__ __align__(16) char lds_b[LDS_B];
    __shared__ float s_red[3][NT / 64];
    float2* s_in = reinterpret_cast<float2*>(lds_a);
    float4* s_f = reinterpret_cast<float4*>(lds_a);
    float4* s_h4 = reinterpret_cast<float4*>(lds_b);
    float* s_h1 = reinterpret_cast<float*>(lds_b + HS_H * HS_W * 16);
    float4* s_hb = reinterpret_cast<float4*>(lds_b);
    const int t = threadIdx.x;
    const int x0 = blockIdx.x * TX, y0 = blockIdx.y * TY;
    float ssim_sum = 0.f, l1_sum = 0.f, cnt = 0.f;
    // The three channels of this thread's input positions (zero outside the
    // image) are loaded once, into registers; each channel pass copies its
    // component into LDS.
    float rg[NPOS][3], rr[NPOS][3];
#pragma unroll
    for (int k = 0; k < NPOS; ++k) {
        const int i = t + k * NT;
        const int iy = i / IN_W, ix = i - iy * IN_W;
        const int gy = y0 - 2 * HALF + iy, gx = x0 - 2 * HALF + ix;
        const bool in = i < IN_H * IN_W && gx >= 0 && gx < W && gy >= 0 && gy < H;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const size_t q = ((size_t)gy * W + gx) * 3 + c;
            rg[k][c] = in ? gt[q] : 0.f;
            rr[k][c] = in ? img[q] : 0.f;
        }
    }
    // this thread's output pixels: column t % TX, rows t / TX + (NT / TX) j
    const int ox = t % TX, oy0 = t / TX;
    float og[NOUT][3], orr[NOUT][3], vr[NOUT][3];
    bool oin[NOUT];
#pragma unroll
    for (int j = 0; j < NOUT; ++j) {
        const int gx = x0 + ox, gy = y0 + oy0 + (NT / TX) * j;
        oin[j] = gx < W && gy < H;
#pragma unroll
        for (int c = 0; c < 3; ++c) {
            const size_t q = ((size_t)gy * W + gx) * 3 + c;
            og[j][c] = oin[j] ? gt[q] : 0.f;
            orr[j][c] = oin[j] ? img[q] : 0.f;
            vr[j][c] = 0.f;
        }
        if (oin[j]) cnt += 1.f;
    }
#pragma unroll
    for (int c = 0; c < 3; ++c) {
        // the previous channel's vertical backward has read the horizontal
        // backward before this channel's sums overwrite it, and its fields
        // are consumed
        if (c > 0) __syncthreads();
#pragma unroll
        for (int k = 0; k < NPOS; ++k) {
            const int i = t + k * NT;
            if (i < IN_H * IN_W) {
                const int iy = i / IN_W, ix = i - iy * IN_W;
                s_in[iy * IN_S + ix] = make_float2(rg[k][c], rr[k][c]);
            }
        }
        __syncthreads();
        // horizontal zero-padded sums (ssim_h_fwd, .metal:3094-3114) at the
        // in-image positions; zero elsewhere.  An item takes two neighbouring
        // positions: their twelve inputs are six 16-byte reads (each position
        // adds its eleven terms in the reference's order).
        for (int i = t; i < HS_H * (HS_W / 2); i += NT) {
            const int hy = i / (HS_W / 2), hx = 2 * (i - hy * (HS_W / 2));
            const int gy = y0 - 2 * HALF + hy, gx = x0 - HALF + hx;
            const bool rin = gy >= 0 && gy < H;
            const bool in0 = rin && gx >= 0 && gx < W, in1 = rin && gx + 1 >= 0 && gx + 1 < W;
            // inputs hx + k, k = 0..11, read two at a time: input k is term k
            // of the first position's sums and term k - 1 of the second's
            float acc[2][5] = {};
            const float4* row = reinterpret_cast<const float4*>(s_in + hy * IN_S + hx);
#pragma unroll
            for (int q = 0; q < (WIN + 1) / 2; ++q) {
                const float4 f = row[q];
#pragma unroll
                for (int e = 0; e < 2; ++e) {
                    const int k = 2 * q + e;
                    const float gv = e ? f.z : f.x, rv = e ? f.w : f.y;
#pragma unroll
                    for (int u = 0; u < 2; ++u) {
                        const int d = k - u;
                        if (d < 0 || d >= WIN) continue;
                        const float w = GAUSS_1D[d];
                        const float wg = w * gv, wr = w * rv;
                        acc[u][0] = fmaf(w, gv, acc[u][0]);
                        acc[u][1] = fmaf(w, rv, acc[u][1]);
                        acc[u][2] = fmaf(wg, gv, acc[u][2]);
                        acc[u][3] = fmaf(wr, rv, acc[u][3]);
                        acc[u][4] = fmaf(wg, rv, acc[u][4]);
                    }
                }
            }
            float a[2][5];
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const bool in = u == 0 ? in0 : in1;
#pragma unroll
                for (int r = 0; r < 5; ++r) a[u][r] = in ? acc[u][r] : 0.f;
            }
            const int o = hy * HS_W + hx;
            s_h4[o] = make_float4(a[0][0], a[0][1], a[0][2], a[0][3]);
            s_h4[o + 1] = make_float4(a[1][0], a[1][1], a[1][2], a[1][3]);
            *reinterpret_cast<float2*>(s_h1 + o) = make_float2(a[0][4], a[1][4]);
        }
        __syncthreads();
        // vertical sums, SSIM and the derivative fields (.metal:3243-3300)
        // at the centres of the in-image rows (the fields of other rows are
        // never read: their horizontal backward is zero).  An item takes two
        // rows of one column: twelve rows of sums serve both.
        for (int i = t; i < (FD_H / 2) * FD_W; i += NT) {
            const int fy0 = 2 * (i / FD_W), fx = i - (i / FD_W) * FD_W;
            const int gx = x0 - HALF + fx;
            // rows fy0 + k, k = 0..11: row k is term k of the first row's
            // sums and term k - 1 of the second's, each added in order
            float acc[2][5] = {};
#pragma unroll
            for (int k = 0; k < WIN + 1; ++k) {
                const float4 q = s_h4[(fy0 + k) * HS_W + fx];
                const float q4 = s_h1[(fy0 + k) * HS_W + fx];
                if (k < WIN) {
                    const float w = GAUSS_1D[k];
                    acc[0][0] = fmaf(w, q.x, acc[0][0]);
                    acc[0][1] = fmaf(w, q.y, acc[0][1]);
                    acc[0][2] = fmaf(w, q.z, acc[0][2]);
                    acc[0][3] = fmaf(w, q.w, acc[0][3]);
                    acc[0][4] = fmaf(w, q4, acc[0][4]);
                }
                if (k > 0) {
                    const float w = GAUSS_1D[k - 1];
                    acc[1][0] = fmaf(w, q.x, acc[1][0]);
                    acc[1][1] = fmaf(w, q.y, acc[1][1]);
                    acc[1][2] = fmaf(w, q.z, acc[1][2]);
                    acc[1][3] = fmaf(w, q.w, acc[1][3]);
                    acc[1][4] = fmaf(w, q4, acc[1][4]);
                }
                // the sums are formed row by row (without this the compiler
                // sinks them into the per-row validity test and keeps all
                // twelve rows in registers, which spills)
                asm volatile("" : "+v"(acc[0][0]), "+v"(acc[0][1]), "+v"(acc[0][2]), "+v"(acc[0][3]),
                             "+v"(acc[0][4]), "+v"(acc[1][0]), "+v"(acc[1][1]), "+v"(acc[1][2]),
                             "+v"(acc[1][3]), "+v"(acc[1][4]));
            }
#pragma unroll
            for (int u = 0; u < 2; ++u) {
                const int fy = fy0 + u;
                const int gy = y0 - HALF + fy;
                if (gy < 0 || gy >= H) continue;
                const float mx = acc[u][0], my = acc[u][1], sx = acc[u][2], sy = acc[u][3],
                            cxy = acc[u][4];
                const float sxs = sx - mx * mx, sys = sy - my * my, sxy = cxy - mx * my;
                const float A = 2.0f * mx * my + SSIM_C1, B = 2.0f * sxy + SSIM_C2;
                const float Cd = mx * mx + my * my + SSIM_C1, D = sxs + sys + SSIM_C2;
                const float iCD = 1.0f / (Cd * D);
                const float dmu = 2.0f * B * (mx * Cd - A * my) / (Cd * Cd * D);
                const float dsyq = -A * B * iCD / D, dsxy = 2.0f * A * iCD;
                s_f[fy * FD_W + fx] = make_float4(dmu - 2.0f * my * dsyq - mx * dsxy, 2.0f * dsyq, dsxy, 0.f);
                // the tile's own in-image outputs add their SSIM to the loss
                if (fy >= HALF && fy < HALF + TY && fx >= HALF && fx < HALF + TX && gx >= 0 && gx < W)
                    ssim_sum += (A * B) / (Cd * D);
            }
        }
        __syncthreads();
        // mirrored horizontal backward at the in-image rows of the tile's
        // columns +- 5 rows (zero at rows outside the image)
        for (int i = t; i < FD_H * TX; i += NT) {
            const int by = i / TX, bx = i - by * TX;
            const int gy = y0 - HALF + by;
            float h1 = 0.f, h2 = 0.f, h3 = 0.f;
            if (gy >= 0 && gy < H) {
                const float4* fr = s_f + by * FD_W + bx;
#pragma unroll
                for (int d = 0; d < WIN; ++d) {
                    const float w = GAUSS_1D[WIN - 1 - d];
                    const float4 f = fr[d];
                    h1 = fmaf(w, f.x, h1);
                    h2 = fmaf(w, f.y, h2);
                    h3 = fmaf(w, f.z, h3);
                }
            }
            s_hb[i] = make_float4(h1, h2, h3, 0.f);
        }
        __syncthreads();
        // mirrored vertical backward (.metal:3443-3463) and the L1 term
#pragma unroll
        for (int j = 0; j < NOUT; ++j) {
            if (!oin[j]) continue;
            const int oy = oy0 + (NT / TX) * j;
            float f1 = 0.f, f2 = 0.f, f3 = 0.f;
            const float4* hr = s_hb + oy * TX + ox;
#pragma unroll
            for (int d = 0; d < WIN; ++d) {
                const float w = GAUSS_1D[WIN - 1 - d];
                const float4 h = hr[d * TX];
                f1 = fmaf(w, h.x, f1);
                f2 = fmaf(w, h.y, f2);
                f3 = fmaf(w, h.z, f3);
            }
            const float r = orr[j][c], g = og[j][c];
            const float v_ssim = f1 + r * f2 + g * f3;
            const float v_l1 = (g > r) ? -1.0f : ((g < r) ? 1.0f : 0.0f);
            vr[j][c] = inv_n * (-w_ssim * v_ssim + (1.0f - w_ssim) * v_l1);
            l1_sum += fabsf(g - r);
        }
    }
#pragma unroll
    for (int j = 0; j < NOUT; ++j) {
        if (!oin[j]) continue;
        const size_t q = ((size_t)(y0 + oy0 + (NT / TX) * j) * W + x0 + ox) * 3;
        v_rendered[q + 0] = vr[j][0];
        v_rendered[q + 1] = vr[j][1];
        v_rendered[q + 2] = vr[j][2];
    }
    // Workgroup partials of (sum SSIM, sum L1, pixels).
    const float a = wave_sum(ssim_sum), b = wave_sum(l1_sum), n = wave_sum(cnt);
    if ((t & 63) == 0) {
        s_red[0][t >> 6] = a;
        s_red[1][t >> 6] = b;
        s_red[2][t >> 6] = n;
    }
    __syncthreads();
    if (t < 3) {
        float v = 0.f;
#pragma unroll
        for (int k = 0; k < NT / 64; ++k) v += s_red[t][k];
        loss_part[((size_t)blockIdx.y * gridDim.x + blockIdx.x) * 3 + t] = v;
    }
}

}  // namespace

int launch_ssim(hipStream_t s, int H, int W, const float* img, const float* gt, float w,
                float inv_n, float* v_rendered, float* loss_part) {
    const dim3 grid((W + TX - 1) / TX, (H + TY - 1) / TY);
    hipLaunchKernelGGL(k_ssim_tile, grid, dim3(NT), 0, s, W, H, img, gt, w, inv_n, v_rendered,
                       loss_part);
    return (int)(grid.x * grid.y);
}

}  // namespace msp
