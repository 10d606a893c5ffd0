// radix.hip — device-wide scans and a stable LSD radix sort of (u32 key, u32
// value) pairs, used by the binning to order the gaussians by depth and
// their super-tile references by super-tile, and by the nearest-neighbour
// search to order points by cell.
//
// Sort: digits of up to 8 bits (9 for a sort of at most 9 bits, done in one
// pass), reduce-then-scan per pass over 2048-key blocks (512 threads x 4
// keys):
//   1. per-block digit histograms in LDS -> hist[digit][block], and the
//      digit totals over all blocks (one global atomic per block and digit)
//   2. one workgroup per digit scans its row of hist and adds the keys of
//      all smaller digits -> scatter offsets
//   3. per-block stable ranks: each wave ranks 256 consecutive keys in
//      four 64-key rounds with a ballot match of equal digits, keeping
//      per-digit running counts in LDS; wave counts are combined in wave
//      order; the block is reordered by digit in LDS and written out in digit
//      runs (coalesced stores).
// Stability makes the result independent of how work is scheduled: equal keys
// keep their input order.
// The depth order sorts with "cull" set: in the first pass the key
// 0xFFFFFFFF (a culled gaussian) is a digit of its own after all others, so
// the culled keys end up behind the visible ones in input order, and the
// later passes sort only the visible keys (their count, written by the first
// pass, is read on the device).  The visible keys get the order a full sort
// of all keys gives them; the culled tail is left where the first pass put
// it, and the last pass writes empty rectangles for it.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

constexpr int RT = 512;            // threads per sort block (8 waves)
constexpr int RW = RT / 64;        // waves per sort block
constexpr int RK = 4;              // keys per thread
constexpr int RB = RT * RK;        // keys per block
constexpr int WK = RK * 64;        // keys per wave (RK rounds of 64)
constexpr int SB = SCAN_BLOCK;     // elements per scan block
constexpr int MAX_PASSES = 4;      // 32-bit keys in 8-bit digits
constexpr int DMAX = 512;          // digit slots of the widest pass (9 bits, or 8 + the culled digit)
constexpr int DCOPIES = 16;        // copies of the digit totals (block b adds to copy b % 16)

// Digit of key k in a pass: bits [shift, shift + width) (mask), or mask + 1
// for the culled key 0xFFFFFFFF when cull is set.
__device__ __forceinline__ int digit_of(uint32_t k, int shift, uint32_t mask, bool cull) {
    return (cull && k == 0xFFFFFFFFu) ? (int)mask + 1 : (int)((k >> shift) & mask);
}

// Keys a pass covers: n, or the count the culling first pass wrote.
__device__ __forceinline__ int64_t pass_n(int64_t n, const int* n_dev) {
    return n_dev ? (int64_t)*n_dev : n;
}

// Sum of v over the NT threads of a block (sh: NT / 64 ints).
template <int NT>
__device__ __forceinline__ int block_sum(int v, int* sh) {
    for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int t = 0;
#pragma unroll
    for (int k = 0; k < NT / 64; ++k) t += sh[k];
    __syncthreads();
    return t;
}
__device__ __forceinline__ int block_sum_256(int v, int* sh) { return block_sum<256>(v, sh); }

// Value i of a scan's input: in[i], or in[gather[i]].
__device__ __forceinline__ int scan_in(const int* __restrict__ in,
                                       const uint32_t* __restrict__ gather, int64_t i) {
    return gather ? in[gather[i]] : in[i];
}

// Block totals of the scan input; with `gather` the input is in[gather[i]],
// which is also written to gathered[i] for the later passes.
__global__ __launch_bounds__(256) void k_block_reduce(const int* __restrict__ in, int64_t n,
                                                      int* __restrict__ tot,
                                                      const uint32_t* __restrict__ gather,
                                                      int* __restrict__ gathered) {
    __shared__ int sh[4];
    const int64_t base = (int64_t)blockIdx.x * SB;
    int v = 0;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + k * 256 + threadIdx.x;
        if (i < n) {
            const int x = scan_in(in, gather, i);
            if (gathered) gathered[i] = x;
            v += x;
        }
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
// With PREFIX the block sums the totals of the blocks before it itself (tot
// holds plain block totals); otherwise tot holds the scanned offsets.
template <bool INCLUSIVE, bool PREFIX>
__global__ __launch_bounds__(256) void k_block_scan(const int* __restrict__ in,
                                                    int* __restrict__ out, int64_t n,
                                                    const int* __restrict__ tot,
                                                    const uint32_t* __restrict__ gather) {
    __shared__ int ts[256];
    __shared__ int sh[4];
    const int64_t base = (int64_t)blockIdx.x * SB;
    const int t = threadIdx.x;
    int boff = 0;
    if (PREFIX) {
        int acc = 0;
        for (int b = t; b < (int)blockIdx.x; b += 256) acc += tot[b];
        boff = block_sum_256(acc, sh);
    } else {
        boff = tot[blockIdx.x];
    }
    int v[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + 4 * t + k;
        v[k] = i < n ? scan_in(in, gather, i) : 0;
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
    int run = ts[t] - s4 + boff;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
        const int64_t i = base + 4 * t + k;
        if (INCLUSIVE) run += v[k];
        if (i < n) out[i] = run;
        if (!INCLUSIVE) run += v[k];
    }
}

// Per-block digit counts.  D: digit slots (256, or 512 for a 9-bit or
// culling pass).  LDS atomics on one address from many lanes of a wave are
// serialised, so lanes that share a digit are counted with one atomic where
// that is common: the culled keys' digit of a culling pass, and with agg (the
// top byte of depth keys, where a wave's keys mostly share one or two
// digits) up to four groups of equal digits; the lanes left add one each.
template <int D>
__global__ __launch_bounds__(RT) void k_radix_hist(const uint32_t* __restrict__ keys, int64_t n,
                                                   const int* __restrict__ n_dev, int shift,
                                                   uint32_t mask, int cull, int agg, int nblocks,
                                                   int* __restrict__ hist, int* __restrict__ dtot,
                                                   SlotSum ss) {
    __shared__ int h[D];
    if (ss.out && blockIdx.x == 0 && threadIdx.x < 64) {
        // lane k reads slot k's pair; the wave sums them
        unsigned long long ti = 0, tr = 0;
        for (int k = threadIdx.x; k < ISECT_SLOTS; k += 64) {
            ti += __hip_atomic_load(ss.slots + (size_t)k * ISECT_STRIDE, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
            tr += __hip_atomic_load(ss.slots + (size_t)k * ISECT_STRIDE + 1, __ATOMIC_RELAXED,
                                    __HIP_MEMORY_SCOPE_AGENT);
        }
        for (int off = 32; off >= 1; off >>= 1) {
            ti += __shfl_xor(ti, off, 64);
            tr += __shfl_xor(tr, off, 64);
        }
        if (threadIdx.x == 0)
            __hip_atomic_store(ss.out, totals_word(ti, tr), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    const int64_t ne = pass_n(n, n_dev);
    const int nbe = (int)((ne + RB - 1) / RB);
    if ((int)blockIdx.x >= nbe) return;   // beyond the keys (the offsets scan only the blocks that hold some)
    // this block's key range: the ranges of one XCD's blocks are consecutive
    const int rb = xcd_order((int)blockIdx.x, nbe);
    const int64_t base = (int64_t)rb * RB;
    if (threadIdx.x < D) h[threadIdx.x] = 0;
    __syncthreads();
    const bool cl = cull != 0;
#pragma unroll
    for (int k = 0; k < RK; ++k) {
        const int64_t i = base + k * RT + threadIdx.x;
        const bool ok = i < ne;
        const int d = ok ? digit_of(keys[i], shift, mask, cl) : 0;
        bool left = ok;
        if (cl) {
            // the culled keys' digit (about a third of the keys): one atomic
            // for all of the wave's lanes that hold it
            const bool cu = ok && d == (int)mask + 1;
            const uint64_t cm = wave_ballot(cu);
            if (cm && (int)(threadIdx.x & 63) == (int)__builtin_ctzll(cm))
                atomicAdd(&h[mask + 1], __popcll(cm));
            if (cu) left = false;
        }
        if (agg) {
            for (int r = 0; r < 4; ++r) {
                const uint64_t act = wave_ballot(left);
                if (act == 0) break;
                // the lowest lane still left picks the digit of this round
                const int first = (int)__builtin_ctzll(act);
                const int dl = __builtin_amdgcn_readlane(d, first);
                const uint64_t same = wave_ballot(left && d == dl);
                if ((int)(threadIdx.x & 63) == first) atomicAdd(&h[dl], __popcll(same));
                if (left && d == dl) left = false;
            }
        }
        if (left) atomicAdd(&h[d], 1);
    }
    __syncthreads();
    const int nd = (int)mask + 1 + (cl ? 1 : 0);
    if ((int)threadIdx.x < nd) {
        const int c = h[threadIdx.x];
        hist[(size_t)threadIdx.x * nblocks + rb] = c;
        // the digit's total over all blocks, spread over DCOPIES addresses
        if (c) atomicAdd(&dtot[(blockIdx.x % DCOPIES) * D + threadIdx.x], c);
    }
}

// Exclusive scan of one value per thread over the NT threads of a block.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* sh) {
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    int x = v;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
    }
    if (lane == 63) sh[w] = x;
    __syncthreads();
    int wofs = 0;
    for (int k = 0; k < w; ++k) wofs += sh[k];
    __syncthreads();
    return wofs + x - v;
}

// Scatter offsets of one digit (one workgroup per digit d): hist[d][b]
// becomes the position of block b's first key with digit d, i.e. the keys
// of all smaller digits (sum of the dtot copies over d' < d) plus those of
// digit d in the blocks before b (exclusive scan of the row over the blocks
// that hold keys of this pass).
// With edge0 (a single-pass sort) the digit's output range [start, end)
// also goes to edge0[d], edge1[d] when the digit occurs.  With nvis the
// workgroup of digit cull_digit (the culled key's) writes its start, the
// number of visible keys, there.
template <int D>
__global__ __launch_bounds__(1024) void k_radix_offsets(int* __restrict__ hist, int nblocks,
                                                        int64_t n, const int* __restrict__ n_dev,
                                                        const int* __restrict__ dtot,
                                                        int* __restrict__ edge0,
                                                        int* __restrict__ edge1,
                                                        int* __restrict__ nvis, int cull_digit) {
    __shared__ int sh[16];
    const int d = blockIdx.x, t = threadIdx.x;
    int lower = 0;
    if (t < d) {
#pragma unroll
        for (int c = 0; c < DCOPIES; ++c) lower += dtot[c * D + t];
    }
    int carry = block_sum<1024>(lower, sh);
    const int start = carry;
    if (nvis && d == cull_digit && t == 0) *nvis = start;
    const int nbe = (int)((pass_n(n, n_dev) + RB - 1) / RB);
    int* row = hist + (size_t)d * nblocks;
    for (int c = 0; c < nbe; c += 1024) {
        const int i = c + t;
        const int v = i < nbe ? row[i] : 0;
        const int ex = block_exclusive_scan<1024>(v, sh);
        if (i < nbe) row[i] = carry + ex;
        carry += block_sum<1024>(v, sh);
    }
    if (edge0 && t == 0 && carry > start) {
        edge0[d] = start;
        edge1[d] = carry;
    }
}

// One LSD pass over the digit of each key (digit_of: dbits bits, at most D
// values).  Keys are ranked stably inside the block (each wave ranks its RB/4
// consecutive keys in 64-key rounds by ballot-matching the digit bits and
// keeps per-digit running counts), reordered by digit in LDS, and written out
// in digit runs so that neighbouring lanes store neighbouring addresses.
// With RG (the depth order's last pass) the rectangles of the values go to
// the same positions with their super-tile counts, and the positions past
// the pass's keys (the culled tail) get empty ones.
template <bool RG, int D>
__global__ __launch_bounds__(RT) void k_radix_scatter(const uint32_t* __restrict__ kin,
                                                      const uint32_t* __restrict__ vin,
                                                      uint32_t* __restrict__ kout,
                                                      uint32_t* __restrict__ vout, int64_t n,
                                                      const int* __restrict__ n_dev, int shift,
                                                      uint32_t mask, int cull, int dbits,
                                                      int nblocks, const int* __restrict__ offs,
                                                      int* __restrict__ dtot, RectGather rg) {
    // The pass's digit totals were last read by the offsets kernel: block 0
    // clears them for the next sort that uses this scratch.
    if (blockIdx.x == 0)
        for (int i = threadIdx.x; i < DCOPIES * D; i += RT) dtot[i] = 0;
    const int64_t ne = pass_n(n, n_dev);
    const int64_t bbase = (int64_t)blockIdx.x * RB;
    if (RG) {
        // output positions [ne, n) of this block's range: the culled tail
        for (int64_t p = max(bbase, ne) + threadIdx.x; p < min(bbase + RB, n); p += RT) {
            rg.rs[p] = make_uint2(0u, 0u);
            rg.cnt[p] = 0;
        }
    }
    const int nbe = (int)((ne + RB - 1) / RB);
    if ((int)blockIdx.x >= nbe) return;
    // this block's key range (as in the histogram kernel): the blocks of one
    // XCD write the neighbouring pieces of each digit's output run, which
    // then meet in that XCD's L2 instead of being written back in parts
    const int rb = xcd_order((int)blockIdx.x, nbe);
    const int64_t kbase = (int64_t)rb * RB;
    __shared__ uint32_t s_key[RB];
    __shared__ uint32_t s_val[RB];
    __shared__ int wcnt[RW][D];
    __shared__ int dstart[D];
    __shared__ int gofs[D];
    __shared__ int scan_sh[RW];
    const bool cl = cull != 0;
    const int nd = (int)mask + 1 + (cl ? 1 : 0);
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // this block's scatter offset of digit tid, loaded now so that its latency
    // overlaps the key loads and the ranking
    const int my_gofs = tid < nd ? offs[(size_t)tid * nblocks + rb] : 0;
    for (int i = tid; i < RW * D; i += RT) (&wcnt[0][0])[i] = 0;
    __syncthreads();
    const int64_t wbase = kbase + (int64_t)w * WK;
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    uint32_t key[RK], val[RK];
    int dig[RK], rank[RK];
    uint2 rc[RK];      // RG: the value's rectangle, gathered while the keys are ranked
#pragma unroll
    for (int j = 0; j < RK; ++j) {
        const int64_t i = wbase + j * 64 + lane;
        const bool ok = i < ne;
        key[j] = ok ? kin[i] : 0u;
        val[j] = ok ? vin[i] : 0u;
        if (RG) rc[j] = ok && key[j] != 0xFFFFFFFFu ? rg.rect[val[j]] : make_uint2(0u, 0u);
        const int d = ok ? digit_of(key[j], shift, mask, cl) : D;
        dig[j] = d;
        uint64_t peers = wave_ballot(ok);
        if (!ok) peers = ~peers;
        for (int b = 0; b < dbits; ++b) {
            const uint64_t bb = wave_ballot((d >> b) & 1);
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
    // per digit (threads 0..D-1): offsets of the waves in wave order, the
    // block's count and its start
    int cnt = 0;
    if (tid < D) {
        const int d = tid;
#pragma unroll
        for (int ww = 0; ww < RW; ++ww) {
            const int c = wcnt[ww][d];
            wcnt[ww][d] = cnt;
            cnt += c;
        }
        gofs[d] = my_gofs;
    }
    const int start = block_exclusive_scan<RT>(cnt, scan_sh);
    if (tid < D) dstart[tid] = start;
    __syncthreads();
    int lpos[RK];      // each key's place in the block's digit order
#pragma unroll
    for (int j = 0; j < RK; ++j) {
        const int d = dig[j];
        lpos[j] = -1;
        if (d >= D) continue;
        const int p = dstart[d] + wcnt[w][d] + rank[j];
        lpos[j] = p;
        s_key[p] = key[j];
        s_val[p] = val[j];
    }
    __syncthreads();
    const int nvalid = (int)min((int64_t)RB, ne - kbase);
    int64_t opos[RK];  // output position of block element tid + u RT
#pragma unroll
    for (int u = 0; u < RK; ++u) {
        const int p = tid + u * RT;
        opos[u] = -1;
        if (p >= nvalid) continue;
        const uint32_t k = s_key[p];
        const int d = digit_of(k, shift, mask, cl);
        const int64_t pos = (int64_t)gofs[d] + (p - dstart[d]);
        kout[pos] = k;
        vout[pos] = s_val[p];
        opos[u] = pos;
    }
    if (RG) {
        // the rectangles take the keys' LDS places and go to the same
        // output positions, with their super-tile counts
        __syncthreads();
#pragma unroll
        for (int j = 0; j < RK; ++j) {
            if (lpos[j] < 0) continue;
            s_key[lpos[j]] = rc[j].x;
            s_val[lpos[j]] = rc[j].y;
        }
        __syncthreads();
#pragma unroll
        for (int u = 0; u < RK; ++u) {
            if (opos[u] < 0) continue;
            const int p = tid + u * RT;
            const uint2 r = make_uint2(s_key[p], s_val[p]);
            rg.rs[opos[u]] = r;
            const int x0 = (int)(r.x & 0xFFFFu), y0 = (int)(r.x >> 16);
            const int x1 = (int)(r.y & 0xFFFFu), y1 = (int)(r.y >> 16);
            rg.cnt[opos[u]] = (x1 > x0 && y1 > y0) ? super_span(x0, y0, x1, y1) : 0;
        }
    }
}

inline unsigned blocks_for(int64_t n, int per) { return (unsigned)((n + per - 1) / per); }

}  // namespace

int64_t scan_block_count(int64_t n) { return (n + SB - 1) / SB; }

template <bool INCLUSIVE>
void launch_scan(hipStream_t s, const int* in, int* out, int64_t n, int* tot,
                 const uint32_t* gather, int* gathered) {
    if (n <= 0) return;
    const int nb = (int)scan_block_count(n);
    hipLaunchKernelGGL(k_block_reduce, dim3(nb), dim3(256), 0, s, in, n, tot, gather, gathered);
    if (gather) {   // the block scans read the gathered copy
        in = gathered;
        gather = nullptr;
    }
    if (nb <= SCAN_DIRECT_BLOCKS) {
        hipLaunchKernelGGL((k_block_scan<INCLUSIVE, true>), dim3(nb), dim3(256), 0, s, in, out, n,
                           (const int*)tot, gather);
    } else {
        hipLaunchKernelGGL(k_scan_totals, dim3(1), dim3(1024), 0, s, tot, nb);
        hipLaunchKernelGGL((k_block_scan<INCLUSIVE, false>), dim3(nb), dim3(256), 0, s, in, out, n,
                           (const int*)tot, gather);
    }
}

void launch_block_totals(hipStream_t s, const int* in, int64_t n, int* tot) {
    if (n <= 0) return;
    const int nb = (int)scan_block_count(n);
    hipLaunchKernelGGL(k_block_reduce, dim3(nb), dim3(256), 0, s, in, n, tot, nullptr, nullptr);
    if (nb > SCAN_DIRECT_BLOCKS) hipLaunchKernelGGL(k_scan_totals, dim3(1), dim3(1024), 0, s, tot, nb);
}

void launch_scan_i32(hipStream_t s, const int* in, int* out, int64_t n, int* tot) {
    launch_scan<true>(s, in, out, n, tot, nullptr, nullptr);
}

void launch_exclusive_scan_i32(hipStream_t s, const int* in, int* out, int64_t n, int* tot,
                               const uint32_t* gather, int* gathered) {
    launch_scan<false>(s, in, out, n, tot, gather, gathered);
}

int64_t radix_temp_ints(int64_t n) {
    const int64_t nb = (n + RB - 1) / RB;
    return DCOPIES * DMAX * MAX_PASSES + (int64_t)DMAX * nb + 16;
}

namespace {

// The three kernels of one pass with D digit slots.
template <int D>
void launch_pass(hipStream_t s, const uint32_t* ki, const uint32_t* vi, uint32_t* ko, uint32_t* vo,
                 int64_t n, const int* n_dev, int shift, uint32_t mask, bool cull, int dbits, bool agg,
                 int nb, int* hist, int* dt, const SlotSum& side, int* edge0, int* edge1, int* nvis,
                 const RectGather* rg) {
    const int nd = (int)mask + 1 + (cull ? 1 : 0);
    hipLaunchKernelGGL(k_radix_hist<D>, dim3(nb), dim3(RT), 0, s, ki, n, n_dev, shift, mask,
                       cull ? 1 : 0, agg ? 1 : 0, nb, hist, dt, side);
    hipLaunchKernelGGL(k_radix_offsets<D>, dim3(nd), dim3(1024), 0, s, hist, nb, n, n_dev,
                       (const int*)dt, edge0, edge1, cull ? nvis : nullptr, nd - 1);
    if (rg)
        hipLaunchKernelGGL((k_radix_scatter<true, D>), dim3(nb), dim3(RT), 0, s, ki, vi, ko, vo, n, n_dev,
                           shift, mask, cull ? 1 : 0, dbits, nb, (const int*)hist, dt, *rg);
    else
        hipLaunchKernelGGL((k_radix_scatter<false, D>), dim3(nb), dim3(RT), 0, s, ki, vi, ko, vo, n,
                           n_dev, shift, mask, cull ? 1 : 0, dbits, nb, (const int*)hist, dt,
                           RectGather{});
}

}  // namespace

// Sorts (k0, v0) by the bits [0, bits) of the keys; ping-pongs with (k1, v1).
// A sort of at most 9 bits takes one pass; otherwise the bits are split into
// ceil(bits / 8) passes of equal width (fewer digit values give longer runs
// per digit and block).  Returns true when the result ends up in (k1, v1).
// With rg the last pass also writes each output position's rectangle and
// super-tile count (RectGather); with ss the first kernel also does the
// SlotSum job; with edge0 / edge1 and one pass each occurring key value k
// gets its output range [edge0[k], edge1[k]) (entries of absent values are
// not written).  With cull (32-bit depth keys) the keys 0xFFFFFFFF are put
// behind the others by the first pass and the later passes sort only the
// others; positions [visible, n) of the result then hold no sorted keys,
// and rg marks them empty.
bool launch_radix_sort(hipStream_t s, uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1,
                       int64_t n, int bits, int* temp, const RectGather* rg, const SlotSum* ss,
                       int* edge0, int* edge1, bool cull) {
    if (n <= 0 || bits <= 0) return false;
    const int nb = (int)((n + RB - 1) / RB);
    const int passes = bits <= 9 ? 1 : (bits + 7) / 8;
    // Scratch layout: the digit totals first, at a fixed place whatever n is
    // (DCOPIES x DMAX per pass; each pass's scatter clears its totals for the
    // next sort on this scratch), then the per-block histograms, then the
    // visible count of a culling sort.
    int* dtot = temp;
    int* hist = temp + DCOPIES * DMAX * MAX_PASSES;
    int* nvis = hist + (size_t)DMAX * nb;
    // the digit totals arrive zeroed: fresh scratch is, and each pass's
    // scatter clears its own
    bool flip = false;
    int shift = 0;
    for (int pass = 0; pass < passes; ++pass) {
        const int width = (bits - shift + (passes - pass) - 1) / (passes - pass);
        const uint32_t mask = (1u << width) - 1u;
        const bool pcull = cull && pass == 0;
        const int nd = (int)mask + 1 + (pcull ? 1 : 0);
        int dbits = 0;
        while ((1 << dbits) < nd) ++dbits;
        uint32_t* ki = flip ? k1 : k0;
        uint32_t* vi = flip ? v1 : v0;
        uint32_t* ko = flip ? k0 : k1;
        uint32_t* vo = flip ? v0 : v1;
        int* dt = dtot + DCOPIES * DMAX * pass;
        const SlotSum side = ss && pass == 0 ? *ss : SlotSum{nullptr, nullptr};
        const int* n_dev = cull && pass > 0 ? nvis : nullptr;
        // the top byte of depth keys: a wave's keys mostly share a digit
        const bool agg = cull && shift == 24;
        const RectGather* prg = rg && pass == passes - 1 ? rg : nullptr;
        int* e0 = passes == 1 ? edge0 : nullptr;
        int* e1 = passes == 1 ? edge1 : nullptr;
        if (nd > 256)
            launch_pass<DMAX>(s, ki, vi, ko, vo, n, n_dev, shift, mask, pcull, dbits, agg, nb, hist, dt,
                              side, e0, e1, nvis, prg);
        else
            launch_pass<256>(s, ki, vi, ko, vo, n, n_dev, shift, mask, pcull, dbits, agg, nb, hist, dt,
                             side, e0, e1, nvis, prg);
        flip = !flip;
        shift += width;
    }
    return flip;
}

}  // namespace msp
