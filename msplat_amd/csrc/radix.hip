// radix.hip — device-wide scans and a stable LSD radix sort of (u32 key, u32
// value) pairs, used by the binning to order intersections without atomics.
//
// Sort: 8-bit digits, reduce-then-scan per pass over 2048-key blocks
// (256 threads x 8 keys):
//   1. per-block digit histograms in LDS -> hist[digit][block]
//   2. exclusive scan of hist in digit-major order -> scatter offsets
//   3. per-block stable ranks: each wave ranks 512 consecutive keys in eight
//      64-key rounds with an 8-ballot match of equal digits, keeping per-digit
//      running counts in LDS; wave counts are combined in wave order.
// Stability makes the result independent of how work is scheduled: equal keys
// keep their input order.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

constexpr int RT = 256;            // threads per block
constexpr int RK = 8;              // keys per thread
constexpr int RB = RT * RK;        // keys per block
constexpr int SB = 1024;           // elements per scan block

__device__ __forceinline__ int block_sum_256(int v, int* sh) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    const int t = sh[0] + sh[1] + sh[2] + sh[3];
    __syncthreads();
    return t;
}

__global__ __launch_bounds__(256) void k_block_reduce(const int* __restrict__ in, int64_t n,
                                                      int* __restrict__ tot) {
    __shared__ int sh[4];
    const int64_t base = (int64_t)blockIdx.x * SB;
    int v = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + k * 256 + threadIdx.x;
        if (i < n) v += in[i];
    }
    const int t = block_sum_256(v, sh);
    if (threadIdx.x == 0) tot[blockIdx.x] = t;
}

// Exclusive scan of nb block totals in place (one workgroup); tot[nb] = total.
__global__ __launch_bounds__(1024) void k_scan_totals(int* __restrict__ tot, int nb) {
    __shared__ int s[1024];
    const int per = (nb + 1023) / 1024;
    const int b = min((int)threadIdx.x * per, nb), e = min(b + per, nb);
    int sum = 0;
    for (int i = b; i < e; ++i) sum += tot[i];
    s[threadIdx.x] = sum;
    __syncthreads();
    for (int off = 1; off < 1024; off <<= 1) {
        const int v = threadIdx.x >= (unsigned)off ? s[threadIdx.x - off] : 0;
        __syncthreads();
        s[threadIdx.x] += v;
        __syncthreads();
    }
    int run = s[threadIdx.x] - sum;
    for (int i = b; i < e; ++i) {
        const int v = tot[i];
        tot[i] = run;
        run += v;
    }
    if (threadIdx.x == 1023) tot[nb] = s[1023];
}

// Scan of each 1024-element block plus its offset; inclusive or exclusive.
template <bool INCLUSIVE>
__global__ __launch_bounds__(256) void k_block_scan(const int* __restrict__ in,
                                                    int* __restrict__ out, int64_t n,
                                                    const int* __restrict__ tot) {
    __shared__ int ts[256];
    const int64_t base = (int64_t)blockIdx.x * SB;
    const int t = threadIdx.x;
    int v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + 4 * t + k;
        v[k] = i < n ? in[i] : 0;
    }
    const int s4 = v[0] + v[1] + v[2] + v[3];
    ts[t] = s4;
    __syncthreads();
    for (int off = 1; off < 256; off <<= 1) {
        const int x = t >= off ? ts[t - off] : 0;
        __syncthreads();
        ts[t] += x;
        __syncthreads();
    }
    int run = ts[t] - s4 + tot[blockIdx.x];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + 4 * t + k;
        if (INCLUSIVE) run += v[k];
        if (i < n) out[i] = run;
        if (!INCLUSIVE) run += v[k];
    }
}

__global__ __launch_bounds__(RT) void k_radix_hist(const uint32_t* __restrict__ keys, int64_t n,
                                                   int shift, int nblocks, int* __restrict__ hist) {
    __shared__ int h[256];
    h[threadIdx.x] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * RB;
#pragma unroll
    for (int k = 0; k < RK; ++k) {
        const int64_t i = base + k * RT + threadIdx.x;
        if (i < n) atomicAdd(&h[(keys[i] >> shift) & 0xFF], 1);
    }
    __syncthreads();
    hist[(size_t)threadIdx.x * nblocks + blockIdx.x] = h[threadIdx.x];
}

__global__ __launch_bounds__(RT) void k_radix_scatter(const uint32_t* __restrict__ kin,
                                                      const uint32_t* __restrict__ vin,
                                                      uint32_t* __restrict__ kout,
                                                      uint32_t* __restrict__ vout, int64_t n,
                                                      int shift, int nblocks,
                                                      const int* __restrict__ offs) {
    __shared__ int wcnt[4][256];
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < 4 * 256; i += RT) (&wcnt[0][0])[i] = 0;
    __syncthreads();
    const int64_t base = (int64_t)blockIdx.x * RB + (int64_t)w * (RB / 4);
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint32_t key[RK], val[RK];
    int dig[RK], rank[RK];
#pragma unroll
    for (int j = 0; j < RK; ++j) {
        const int64_t i = base + j * 64 + lane;
        const bool ok = i < n;
        key[j] = ok ? kin[i] : 0u;
        val[j] = ok ? vin[i] : 0u;
        const int d = ok ? (int)((key[j] >> shift) & 0xFF) : 256;
        dig[j] = d;
        // lanes holding the same digit in this 64-key round
        uint64_t peers = __ballot(ok);
        if (!ok) peers = ~peers;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t bb = __ballot((d >> b) & 1);
            peers &= ((d >> b) & 1) ? bb : ~bb;
        }
        const int before = __popcll(peers & lt);
        const int dd = ok ? d : 0;
        const int base_cnt = ok ? wcnt[w][dd] : 0;
        rank[j] = base_cnt + before;
        // the lowest lane of each digit group advances that digit's count
        if (ok && before == 0) wcnt[w][dd] = base_cnt + __popcll(peers);
    }
    __syncthreads();
    // digit offsets of each wave inside the block: counts of earlier waves
    {
        const int d = threadIdx.x;
        int run = 0;
#pragma unroll
        for (int ww = 0; ww < 4; ++ww) {
            const int c = wcnt[ww][d];
            wcnt[ww][d] = run;
            run += c;
        }
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < RK; ++j) {
        const int d = dig[j];
        if (d > 255) continue;
        const int64_t pos = (int64_t)offs[(size_t)d * nblocks + blockIdx.x] + wcnt[w][d] + rank[j];
        kout[pos] = key[j];
        vout[pos] = val[j];
    }
}

inline unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

int64_t scan_block_count(int64_t n) { return (n + SB - 1) / SB; }

void launch_scan_i32(hipStream_t s, const int* in, int* out, int64_t n, int* tot) {
    if (n <= 0) return;
    const int nb = (int)scan_block_count(n);
    hipLaunchKernelGGL(k_block_reduce, dim3(nb), dim3(256), 0, s, in, n, tot);
    hipLaunchKernelGGL(k_scan_totals, dim3(1), dim3(1024), 0, s, tot, nb);
    hipLaunchKernelGGL(k_block_scan<true>, dim3(nb), dim3(256), 0, s, in, out, n, (const int*)tot);
}

void launch_exclusive_scan_i32(hipStream_t s, const int* in, int* out, int64_t n, int* tot) {
    if (n <= 0) return;
    const int nb = (int)scan_block_count(n);
    hipLaunchKernelGGL(k_block_reduce, dim3(nb), dim3(256), 0, s, in, n, tot);
    hipLaunchKernelGGL(k_scan_totals, dim3(1), dim3(1024), 0, s, tot, nb);
    hipLaunchKernelGGL(k_block_scan<false>, dim3(nb), dim3(256), 0, s, in, out, n, (const int*)tot);
}

int64_t radix_temp_ints(int64_t n) {
    const int64_t nb = (n + RB - 1) / RB;
    return 256 * nb + scan_block_count(256 * nb) + 8;
}

// Sorts (k0, v0) by the bits [0, bits) of the keys; ping-pongs with (k1, v1).
// Returns true when the result ends up in (k1, v1).
bool launch_radix_sort(hipStream_t s, uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1,
                       int64_t n, int bits, int* temp) {
    if (n <= 0 || bits <= 0) return false;
    const int nb = (int)((n + RB - 1) / RB);
    int* hist = temp;
    int* tot = temp + 256 * (int64_t)nb;
    bool flip = false;
    for (int shift = 0; shift < bits; shift += 8) {
        uint32_t* ki = flip ? k1 : k0;
        uint32_t* vi = flip ? v1 : v0;
        uint32_t* ko = flip ? k0 : k1;
        uint32_t* vo = flip ? v0 : v1;
        hipLaunchKernelGGL(k_radix_hist, dim3(nb), dim3(RT), 0, s, (const uint32_t*)ki, n, shift, nb,
                           hist);
        launch_exclusive_scan_i32(s, hist, hist, 256 * (int64_t)nb, tot);
        hipLaunchKernelGGL(k_radix_scatter, dim3(nb), dim3(RT), 0, s, (const uint32_t*)ki,
                           (const uint32_t*)vi, ko, vo, n, shift, nb, (const int*)hist);
        flip = !flip;
    }
    return flip;
}

}  // namespace msp
