// binning.hip — tile intersection lists in depth order, without atomics.
//
// Replaces scatter_to_prealloc_bins (.metal:2025-2059) + prefix_sum
// (.metal:2312-2364) + bitonic_sort_per_tile (.metal:2064-2138) with the same
// result — per tile, the ids of the gaussians whose tile rectangle covers it,
// ascending by (depth_bits, gaussian id), and tile_bins = (start, end) of each
// tile's range in one contiguous list — built from stable radix sorts:
//   1. the projection wrote key = depth bits (0xFFFFFFFF if culled), value = id
//   2. radix sort by depth                        (order of gaussians)
//   3. tiles hit gathered in that order by the scan -> emit offsets
//   4. emit one (tile id, gaussian id) pair per intersection, depth order
//   5. stable radix sort by tile id               (depth order kept per tile)
//   6. run edges -> per-tile counts; scan -> tile_bins, chunk work items
// The rasteriser gathers each entry's projection record by id, in place of
// the reference's packed per-entry copies (.metal:2128-2137).
// Equal depths keep ascending id order because both sorts are stable and the
// first one starts from id order.  Tiles have no size limit (the reference
// drops entries beyond 2048 per tile).
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

constexpr int SCAN_T = 1024;

// Emission of the (tile id, gaussian id) pairs of 64 depth-consecutive
// gaussians by one wave, with coalesced stores.  Gaussians with fewer than
// EMIT_BIG pairs are written together: their pairs are numbered 0..S-1 in
// wave order and each lane finds the owner of its slot by a binary search
// over the lanes' running offsets.  Larger ones (close to the camera, so
// often several in one wave) are then written one at a time by the whole
// wave, 64 pairs per step.
constexpr int EMIT_BIG = 64;

__global__ __launch_bounds__(256) void k_emit(int N, int tbx, int tby, GaussOut go,
                                              const uint32_t* __restrict__ order,
                                              const int* __restrict__ eoff,
                                              const int* __restrict__ hits,
                                              uint32_t* __restrict__ tkey,
                                              uint32_t* __restrict__ tval) {
    const int lane = threadIdx.x & 63;
    const int base = blockIdx.x * blockDim.x + threadIdx.x - lane;   // wave-uniform
    if (base >= N) return;
    const int r = base + lane;
    int start = 0, h = 0, x0 = 0, y0 = 0, w = 1, g = 0;
    if (r < N) {
        h = hits[r];
        start = eoff[r];
        g = (int)order[r];
        if (h > 0) {
            const float4 r0 = go.rec[4 * (size_t)g], r2 = go.rec[4 * (size_t)g + 2];
            int x1, y1;
            tile_rect(r0.x, r0.y, r2.y, r2.z, tbx, tby, x0, y0, x1, y1);
            w = x1 - x0;
        }
    }
    // small gaussians: wave-wide numbering of their pairs
    const bool big = h >= EMIT_BIG;
    const int hs = big ? 0 : h;
    int incl = hs;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(incl, off, 64);
        if (lane >= off) incl += y;
    }
    const int sstart = incl - hs;
    const int S = __shfl(incl, 63, 64);
    for (int sb = 0; sb < S; sb += 64) {
        const int sl = sb + lane;
        // owner: the last lane whose first slot is <= sl (lanes without small
        // pairs share their first slot with the next lane and lose the tie)
        int lo = 0;
#pragma unroll
        for (int step = 32; step >= 1; step >>= 1) {
            const int cand = lo + step;
            if (__shfl(sstart, cand, 64) <= sl) lo = cand;
        }
        const int k = sl - __shfl(sstart, lo, 64);
        const int oe = __shfl(start, lo, 64);
        const int ow = __shfl(w, lo, 64);
        const int ox = __shfl(x0, lo, 64), oy = __shfl(y0, lo, 64);
        const int og = __shfl(g, lo, 64);
        if (sl < S) {
            const int q = k / ow;
            tkey[oe + k] = (uint32_t)((oy + q) * tbx + ox + (k - q * ow));
            tval[oe + k] = (uint32_t)og;
        }
    }
    // large gaussians: one at a time, the whole wave writing 64 pairs per step
    uint64_t bigm = wave_ballot(big);
    while (bigm) {
        const int L = __builtin_ctzll(bigm);
        bigm &= bigm - 1;
        const int be = __shfl(start, L, 64), bh = __shfl(h, L, 64), bw = __shfl(w, L, 64);
        const int bx = __shfl(x0, L, 64), by = __shfl(y0, L, 64), bg = __shfl(g, L, 64);
        for (int k = lane; k < bh; k += 64) {
            const int q = k / bw;
            tkey[be + k] = (uint32_t)((by + q) * tbx + bx + (k - q * bw));
            tval[be + k] = (uint32_t)bg;
        }
    }
}

__global__ __launch_bounds__(256) void k_tile_edges(int64_t I, const uint32_t* __restrict__ tkey,
                                                    int* __restrict__ tstart,
                                                    int* __restrict__ tend) {
    const int64_t p = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (p >= I) return;
    const uint32_t t = tkey[p];
    if (p == 0 || tkey[p - 1] != t) tstart[t] = (int)p;
    if (p == I - 1 || tkey[p + 1] != t) tend[t] = (int)(p + 1);
}

__global__ __launch_bounds__(SCAN_T) void k_tile_scan(int T, int* __restrict__ tstart,
                                                      int* __restrict__ tend,
                                                      unsigned long long* __restrict__ isect,
                                                      int* __restrict__ tile_bins, Items it,
                                                      TileLists tl, Meta* __restrict__ meta) {
    __shared__ long long s_c[SCAN_T];
    __shared__ int s_i[SCAN_T];
    __shared__ int s_max[SCAN_T];
    __shared__ int s_nch;
    const int tid = threadIdx.x;
    const int per = (T + SCAN_T - 1) / SCAN_T;
    const int b = min(tid * per, T), e = min(b + per, T);
    long long cs = 0;
    int is = 0, mx = 0;
    for (int t = b; t < e; ++t) {
        const int n = tend[t] - tstart[t];
        cs += n;
        is += tile_chunks(n, T);
        mx = max(mx, n);
    }
    s_c[tid] = cs;
    s_i[tid] = is;
    s_max[tid] = mx;
    if (tid == 0) s_nch = 0;
    __syncthreads();
    for (int off = 1; off < SCAN_T; off <<= 1) {
        long long c = 0;
        int i = 0;
        if (tid >= off) { c = s_c[tid - off]; i = s_i[tid - off]; }
        const int m = s_max[tid ^ off];
        __syncthreads();
        s_c[tid] += c;
        s_i[tid] += i;
        s_max[tid] = max(s_max[tid], m);
        __syncthreads();
    }
    long long off = s_c[tid] - cs;
    int ioff = s_i[tid] - is;
    for (int t = b; t < e; ++t) {
        const int n = tend[t] - tstart[t];
        // cleared for the next frame's run edges (they write present tiles only)
        tstart[t] = 0;
        tend[t] = 0;
        tile_bins[2 * t] = (int)off;
        off += n;
        tile_bins[2 * t + 1] = (int)off;
        const int K = tile_chunks(n, T);
        it.tile_K[t] = K;
        it.tile_item0[t] = ioff;
        ioff += K;
        if (K > 1) tl.chunked[atomicAdd(&s_nch, 1)] = t;
    }
    // the projection's intersection counters, copied to the host earlier
    // on the stream, cleared for the next frame
    if (tid < ISECT_SLOTS) isect[(size_t)tid * ISECT_STRIDE] = 0ull;
    __syncthreads();
    if (tid == SCAN_T - 1) {
        meta->total_isect = s_c[SCAN_T - 1];
        meta->max_count = s_max[0];
        meta->n_items = s_i[SCAN_T - 1];
        meta->n_chunked_tiles = s_nch;
        meta->n_large = 0;
        meta->n_huge = 0;
    }
}

__global__ __launch_bounds__(256) void k_build_items(int T, Items it) {
    const int t = blockIdx.x * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const int K = it.tile_K[t], i0 = it.tile_item0[t];
    for (int k = 0; k < K; ++k) {
        it.tile[i0 + k] = t;
        it.k[i0 + k] = k;
    }
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void launch_run_edges(hipStream_t s, int64_t n, const uint32_t* sorted_keys, int* start, int* end) {
    if (n > 0)
        hipLaunchKernelGGL(k_tile_edges, dim3(blocks_for(n)), dim3(256), 0, s, n, sorted_keys, start,
                           end);
}

void launch_depth_order(hipStream_t s, int N, uint32_t* dkey, uint32_t* dval, uint32_t* dkey2,
                        uint32_t* dval2, int* radix_temp, const int* tiles_hit, int* hits_sorted,
                        int* eoff, int* scan_temp, uint32_t** order_out) {
    const bool flip = launch_radix_sort(s, dkey, dval, dkey2, dval2, N, 32, radix_temp);
    uint32_t* order = flip ? dval2 : dval;
    *order_out = order;
    // emission offsets: exclusive scan of the tiles hit in depth order; the
    // scan's first kernel gathers them into hits_sorted for the emission
    if (N > 0) launch_exclusive_scan_i32(s, tiles_hit, eoff, N, scan_temp, order, hits_sorted);
}

const uint32_t* launch_tile_lists(hipStream_t s, const CamParams& p, int64_t I, GaussOut go,
                                  const uint32_t* order, const int* eoff, const int* hits,
                                  uint32_t* tkey, uint32_t* tval, uint32_t* tkey2, uint32_t* tval2,
                                  int* radix_temp, int* tstart, int* tend, int* tile_bins, Items it,
                                  TileLists tl, Meta* meta, unsigned long long* isect) {
    const int T = p.tbx * p.tby;
    const uint32_t* sorted_ids = tval;
    // tstart / tend arrive zeroed: fresh buffers are, and every tile scan
    // clears the ones it reads
    if (I > 0) {
        hipLaunchKernelGGL(k_emit, dim3(blocks_for(p.N)), dim3(256), 0, s, p.N, p.tbx, p.tby, go,
                           order, eoff, hits, tkey, tval);
        int bits = 0;
        while ((1 << bits) < T) ++bits;
        const bool flip = launch_radix_sort(s, tkey, tval, tkey2, tval2, I, bits, radix_temp);
        const uint32_t* sk = flip ? tkey2 : tkey;
        sorted_ids = flip ? tval2 : tval;
        hipLaunchKernelGGL(k_tile_edges, dim3(blocks_for(I)), dim3(256), 0, s, I, sk, tstart, tend);
    }
    hipLaunchKernelGGL(k_tile_scan, dim3(1), dim3(SCAN_T), 0, s, T, tstart, tend, isect,
                       tile_bins, it, tl, meta);
    hipLaunchKernelGGL(k_build_items, dim3(blocks_for(T)), dim3(256), 0, s, T, it);
    return sorted_ids;
}

}  // namespace msp
