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

// Run edges of the sorted tile keys: tstart[t] / tend[t] = first / one past
// the last position of key t.  Four keys per thread with one 16-byte load
// (tkey is 256-byte aligned); the neighbours across a thread's four come from
// single loads of the same or the adjacent line.
__global__ __launch_bounds__(256) void k_tile_edges(int64_t I, const uint32_t* __restrict__ tkey,
                                                    int* __restrict__ tstart,
                                                    int* __restrict__ tend) {
    const int64_t q = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    const int64_t p0 = 4 * q;
    if (p0 >= I) return;
    uint32_t k[6];      // k[1..4]: this thread's keys, k[0] / k[5]: the neighbours
    if (p0 + 4 <= I) {
        const uint4 v = reinterpret_cast<const uint4*>(tkey)[q];
        k[1] = v.x; k[2] = v.y; k[3] = v.z; k[4] = v.w;
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) k[1 + j] = p0 + j < I ? tkey[p0 + j] : 0xFFFFFFFFu;
    }
    k[0] = p0 > 0 ? tkey[p0 - 1] : 0xFFFFFFFFu;
    k[5] = p0 + 4 < I ? tkey[p0 + 4] : 0xFFFFFFFFu;
#pragma unroll
    for (int j = 1; j <= 4; ++j) {
        const int64_t p = p0 + j - 1;
        if (p >= I) break;
        const uint32_t t = k[j];
        if (p == 0 || k[j - 1] != t) tstart[t] = (int)p;
        if (p == I - 1 || k[j + 1] != t) tend[t] = (int)(p + 1);
    }
}

// Tile scan over TS_BLOCK tiles per workgroup in two kernels.  k_tile_counts:
// each block's tile count total, chunk-item total and largest count.
// k_tile_offsets: each block adds the totals of the blocks before it, scans
// its own tiles and writes tile_bins, the chunk counts and first items and
// the list of chunked tiles; the last block writes the summary.  Then
// k_build_items writes the work items (tile, chunk), one thread per item.
constexpr int TS_T = 256, TS_PER = 4, TS_BLOCK = TS_T * TS_PER;

template <bool MAX>
__device__ __forceinline__ int block_combine(int v, int* sh) {
    for (int off = 32; off >= 1; off >>= 1) {
        const int o = __shfl_xor(v, off, 64);
        v = MAX ? max(v, o) : v + o;
    }
    if ((threadIdx.x & 63) == 0) sh[threadIdx.x >> 6] = v;
    __syncthreads();
    int r = sh[0];
#pragma unroll
    for (int k = 1; k < TS_T / 64; ++k) r = MAX ? max(r, sh[k]) : r + sh[k];
    __syncthreads();
    return r;
}

__global__ __launch_bounds__(TS_T) void k_tile_counts(int T, const int* __restrict__ tstart,
                                                      const int* __restrict__ tend,
                                                      int* __restrict__ tot,
                                                      Meta* __restrict__ meta) {
    __shared__ int sh[TS_T / 64];
    const int b = blockIdx.x;
    int sn = 0, sk = 0, mx = 0;
#pragma unroll
    for (int k = 0; k < TS_PER; ++k) {
        const int t = b * TS_BLOCK + k * TS_T + (int)threadIdx.x;
        if (t < T) {
            const int n = tend[t] - tstart[t];
            sn += n;
            sk += tile_chunks(n, T);
            mx = max(mx, n);
        }
    }
    sn = block_combine<false>(sn, sh);
    sk = block_combine<false>(sk, sh);
    mx = block_combine<true>(mx, sh);
    if (threadIdx.x == 0) {
        tot[3 * b] = sn;
        tot[3 * b + 1] = sk;
        tot[3 * b + 2] = mx;
        if (b == 0) meta->n_chunked_tiles = 0;
    }
}

__global__ __launch_bounds__(TS_T) void k_tile_offsets(int T, int nb, int* __restrict__ tstart,
                                                       int* __restrict__ tend,
                                                       const int* __restrict__ tot,
                                                       unsigned long long* __restrict__ isect,
                                                       int* __restrict__ tile_bins, Items it,
                                                       TileLists tl, Meta* __restrict__ meta) {
    __shared__ int sh[TS_T / 64];
    __shared__ int s_n[TS_T], s_k[TS_T];
    const int b = blockIdx.x, tid = threadIdx.x;
    int pn = 0, pk = 0;
    for (int i = tid; i < b; i += TS_T) {
        pn += tot[3 * i];
        pk += tot[3 * i + 1];
    }
    pn = block_combine<false>(pn, sh);
    pk = block_combine<false>(pk, sh);
    // this thread's TS_PER consecutive tiles
    const int t0 = b * TS_BLOCK + TS_PER * tid;
    int n[TS_PER], K[TS_PER], sn = 0, sk = 0;
#pragma unroll
    for (int k = 0; k < TS_PER; ++k) {
        const int t = t0 + k;
        n[k] = t < T ? tend[t] - tstart[t] : 0;
        K[k] = t < T ? tile_chunks(n[k], T) : 0;
        sn += n[k];
        sk += K[k];
    }
    s_n[tid] = sn;
    s_k[tid] = sk;
    __syncthreads();
    for (int off = 1; off < TS_T; off <<= 1) {
        const int a = tid >= off ? s_n[tid - off] : 0;
        const int c = tid >= off ? s_k[tid - off] : 0;
        __syncthreads();
        s_n[tid] += a;
        s_k[tid] += c;
        __syncthreads();
    }
    int off = pn + s_n[tid] - sn, ioff = pk + s_k[tid] - sk;
#pragma unroll
    for (int k = 0; k < TS_PER; ++k) {
        const int t = t0 + k;
        if (t >= T) break;
        // cleared for the next frame's run edges (they write present tiles only)
        tstart[t] = 0;
        tend[t] = 0;
        tile_bins[2 * t] = off;
        off += n[k];
        tile_bins[2 * t + 1] = off;
        it.tile_K[t] = K[k];
        it.tile_item0[t] = ioff;
        ioff += K[k];
        if (K[k] > 1) tl.chunked[atomicAdd(&meta->n_chunked_tiles, 1)] = t;
    }
    // the projection's intersection counters, copied to the host earlier
    // on the stream, cleared for the next frame
    if (b == 0 && tid < ISECT_SLOTS) isect[(size_t)tid * ISECT_STRIDE] = 0ull;
    if (b == nb - 1 && tid == 0) {
        int mx = 0;
        for (int i = 0; i < nb; ++i) mx = max(mx, tot[3 * i + 2]);
        meta->total_isect = (int64_t)pn + s_n[TS_T - 1];
        meta->max_count = mx;
        meta->n_items = pk + s_k[TS_T - 1];
        meta->n_large = 0;
        meta->n_huge = 0;
    }
}

// Work item i: the tile t with tile_item0[t] <= i < tile_item0[t + 1] (every
// tile has at least one item, so the first items ascend), found by binary
// search, and its chunk i - tile_item0[t].
__global__ __launch_bounds__(256) void k_build_items(int T, const Meta* __restrict__ meta, Items it) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= meta->n_items) return;
    int lo = 0, hi = T - 1;
    while (lo < hi) {
        const int mid = (lo + hi + 1) >> 1;
        if (it.tile_item0[mid] <= i) lo = mid; else hi = mid - 1;
    }
    it.tile[i] = lo;
    it.k[i] = i - it.tile_item0[lo];
}

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

}  // namespace

void launch_run_edges(hipStream_t s, int64_t n, const uint32_t* sorted_keys, int* start, int* end) {
    if (n > 0)
        hipLaunchKernelGGL(k_tile_edges, dim3(blocks_for((n + 3) / 4)), dim3(256), 0, s, n,
                           sorted_keys, start, end);
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
                                  int* radix_temp, int* tstart, int* tend, int* tscan,
                                  int* tile_bins, Items it, TileLists tl, Meta* meta,
                                  unsigned long long* isect) {
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
        hipLaunchKernelGGL(k_tile_edges, dim3(blocks_for((I + 3) / 4)), dim3(256), 0, s, I, sk,
                           tstart, tend);
    }
    const int nb = (T + TS_BLOCK - 1) / TS_BLOCK;
    hipLaunchKernelGGL(k_tile_counts, dim3(nb), dim3(TS_T), 0, s, T, (const int*)tstart,
                       (const int*)tend, tscan, meta);
    hipLaunchKernelGGL(k_tile_offsets, dim3(nb), dim3(TS_T), 0, s, T, nb, tstart, tend,
                       (const int*)tscan, isect, tile_bins, it, tl, meta);
    hipLaunchKernelGGL(k_build_items, dim3(blocks_for(items_bound(T, I))), dim3(256), 0, s, T,
                       (const Meta*)meta, it);
    return sorted_ids;
}

}  // namespace msp
