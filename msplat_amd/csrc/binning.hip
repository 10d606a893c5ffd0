// binning.hip — tile offsets, key scatter and per-tile depth sort + pack.
//
// Reference pipeline: scatter_to_prealloc_bins (.metal:2025-2059) ->
// prefix_sum (.metal:2312-2364) -> bitonic_sort_per_tile (.metal:2064-2138).
// MI355X layout: the projection already counted intersections per tile, so
// the scan gives exact tile ranges and keys are scattered straight into their
// tile's range of one contiguous array (no 2048-slot bins, no per-tile cap).
// The scatter decrements the counters it claims slots with, leaving them at
// zero for the next step.  Keys are (depth_bits << 32 | gid), sorted
// ascending: by depth, ties by gaussian id, so the order does not depend on
// the order the atomics handed out slots.
//
// Sort: one 256-thread workgroup per tile, bitonic network in LDS — 16 KB for
// tiles of up to 2048 keys, 128 KB (of gfx950's 160 KB) for up to 16384, and a
// global-memory network for larger tiles.  The pack of the sorted gaussians
// (.metal:2128-2137) is fused into the same kernel.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

constexpr int SCAN_T = 1024;

__global__ __launch_bounds__(SCAN_T) void k_tile_scan(int T, const int* __restrict__ cnt,
                                                      int* __restrict__ tile_bins, Items it,
                                                      TileLists tl, Meta* __restrict__ meta) {
    __shared__ long long s_c[SCAN_T];
    __shared__ int s_i[SCAN_T];
    __shared__ int s_max[SCAN_T];
    __shared__ int s_nch, s_nl, s_nh;
    const int tid = threadIdx.x;
    const int per = (T + SCAN_T - 1) / SCAN_T;
    const int b = min(tid * per, T), e = min(b + per, T);
    long long cs = 0;
    int is = 0, mx = 0;
    for (int t = b; t < e; ++t) {
        const int n = cnt[t];
        cs += n;
        is += tile_chunks(n, T);
        mx = max(mx, n);
    }
    s_c[tid] = cs;
    s_i[tid] = is;
    s_max[tid] = mx;
    if (tid == 0) { s_nch = 0; s_nl = 0; s_nh = 0; }
    __syncthreads();
    // Hillis–Steele inclusive scans.
    for (int off = 1; off < SCAN_T; off <<= 1) {
        long long c = 0;
        int i = 0, m = 0;
        if (tid >= off) { c = s_c[tid - off]; i = s_i[tid - off]; }
        m = s_max[tid ^ off];
        __syncthreads();
        s_c[tid] += c;
        s_i[tid] += i;
        s_max[tid] = max(s_max[tid], m);
        __syncthreads();
    }
    long long off = s_c[tid] - cs;
    int ioff = s_i[tid] - is;
    for (int t = b; t < e; ++t) {
        const int n = cnt[t];
        tile_bins[2 * t] = (int)off;
        off += n;
        tile_bins[2 * t + 1] = (int)off;
        const int K = tile_chunks(n, T);
        it.tile_K[t] = K;
        it.tile_item0[t] = ioff;
        ioff += K;
        if (K > 1) tl.chunked[atomicAdd(&s_nch, 1)] = t;
        if (n > SORT_SMALL && n <= SORT_LARGE) tl.large[atomicAdd(&s_nl, 1)] = t;
        if (n > SORT_LARGE) tl.huge[atomicAdd(&s_nh, 1)] = t;
    }
    __syncthreads();
    if (tid == SCAN_T - 1) {
        meta->total_isect = s_c[SCAN_T - 1];
        meta->max_count = s_max[0];
        meta->n_items = s_i[SCAN_T - 1];
        meta->n_chunked_tiles = s_nch;
        meta->n_large = s_nl;
        meta->n_huge = s_nh;
        meta->pad = 0;
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

__global__ __launch_bounds__(256) void k_scatter(int N, int tbx, int tby, GaussOut go,
                                                 const int* __restrict__ tile_bins,
                                                 int* __restrict__ tile_cnt,
                                                 uint64_t* __restrict__ keys) {
    const int g = blockIdx.x * blockDim.x + threadIdx.x;
    if (g >= N || go.radii[g] <= 0) return;
    const float2 xy = go.xy[g], ext = go.aabb[g];
    int x0, y0, x1, y1;
    tile_rect(xy.x, xy.y, ext.x, ext.y, tbx, tby, x0, y0, x1, y1);
    const uint64_t key = ((uint64_t)__float_as_uint(go.depth[g]) << 32) | (uint64_t)(uint32_t)g;
    for (int ty = y0; ty < y1; ++ty)
        for (int tx = x0; tx < x1; ++tx) {
            const int t = ty * tbx + tx;
            const int pos = atomicSub(&tile_cnt[t], 1) - 1;
            keys[(size_t)tile_bins[2 * t] + pos] = key;
        }
}

// Pack one sorted key into the per-entry records.
__device__ __forceinline__ void pack_one(uint64_t key, int dst, const GaussOut& go, const Packed& pk) {
    const int g = (int)(uint32_t)(key & 0xFFFFFFFFull);
    const float2 xy = go.xy[g];
    const float4 c = go.conic[g];
    const float4 rgb = go.rgb[g];
    pk.ids[dst] = g;
    pk.geo[dst] = make_float4(xy.x, xy.y, c.x, c.y);
    pk.col[dst] = make_float4(c.z, c.w, rgb.x, rgb.y);
    pk.bl[dst] = rgb.z;
}

// Ascending bitonic network over data[0, npow) held in LDS.
template <typename Mem>
__device__ __forceinline__ void bitonic(Mem data, int npow) {
    for (int k = 2; k <= npow; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < (npow >> 1); i += 256) {
                const int pos = 2 * i - (i & (j - 1));
                const int partner = pos ^ j;
                const bool asc = (pos & k) == 0;
                const uint64_t a = data[pos], b = data[partner];
                if ((a > b) == asc) {
                    data[pos] = b;
                    data[partner] = a;
                }
            }
            __syncthreads();
        }
    }
}

__device__ __forceinline__ int next_pow2(int n) {
    int p = 1;
    while (p < n) p <<= 1;
    return p;
}

template <int CAP>
__device__ __forceinline__ void sort_tile_lds(int t, const int* tile_bins, const uint64_t* keys,
                                              const GaussOut& go, const Packed& pk) {
    __shared__ uint64_t data[CAP];
    const int s = tile_bins[2 * t], n = tile_bins[2 * t + 1] - s;
    const int npow = next_pow2(n);
    for (int i = threadIdx.x; i < npow; i += 256) data[i] = i < n ? keys[(size_t)s + i] : ~0ull;
    __syncthreads();
    bitonic(data, npow);
    for (int i = threadIdx.x; i < n; i += 256) pack_one(data[i], s + i, go, pk);
}

__global__ __launch_bounds__(256) void k_sort_small(const int* __restrict__ tile_bins,
                                                    const uint64_t* __restrict__ keys, GaussOut go,
                                                    Packed pk) {
    const int t = blockIdx.x;
    const int n = tile_bins[2 * t + 1] - tile_bins[2 * t];
    if (n <= 0 || n > SORT_SMALL) return;
    sort_tile_lds<SORT_SMALL>(t, tile_bins, keys, go, pk);
}

__global__ __launch_bounds__(256) void k_sort_large(const int* __restrict__ list,
                                                    const int* __restrict__ tile_bins,
                                                    const uint64_t* __restrict__ keys, GaussOut go,
                                                    Packed pk) {
    sort_tile_lds<SORT_LARGE>(list[blockIdx.x], tile_bins, keys, go, pk);
}

// Tiles beyond 16384 keys: the same network in global memory, in a private
// power-of-two region [2*start, 2*start + npow) of the scratch array.
__global__ __launch_bounds__(256) void k_sort_huge(const int* __restrict__ list,
                                                   const int* __restrict__ tile_bins,
                                                   const uint64_t* __restrict__ keys,
                                                   uint64_t* __restrict__ scratch, GaussOut go,
                                                   Packed pk) {
    const int t = list[blockIdx.x];
    const int s = tile_bins[2 * t], n = tile_bins[2 * t + 1] - s;
    const int npow = next_pow2(n);
    uint64_t* data = scratch + 2 * (size_t)s;
    for (int i = threadIdx.x; i < npow; i += 256) data[i] = i < n ? keys[(size_t)s + i] : ~0ull;
    __threadfence_block();
    __syncthreads();
    for (int k = 2; k <= npow; k <<= 1) {
        for (int j = k >> 1; j > 0; j >>= 1) {
            for (int i = threadIdx.x; i < (npow >> 1); i += 256) {
                const int pos = 2 * i - (i & (j - 1));
                const int partner = pos ^ j;
                const bool asc = (pos & k) == 0;
                const uint64_t a = data[pos], b = data[partner];
                if ((a > b) == asc) {
                    data[pos] = b;
                    data[partner] = a;
                }
            }
            __threadfence_block();
            __syncthreads();
        }
    }
    for (int i = threadIdx.x; i < n; i += 256) pack_one(data[i], s + i, go, pk);
}

}  // namespace

void launch_tile_scan(hipStream_t s, int T, const int* tile_cnt, int* tile_bins, Items it,
                      TileLists tl, Meta* meta) {
    hipLaunchKernelGGL(k_tile_scan, dim3(1), dim3(SCAN_T), 0, s, T, tile_cnt, tile_bins, it, tl,
                       meta);
}

void launch_build_items(hipStream_t s, int T, Items it) {
    hipLaunchKernelGGL(k_build_items, dim3((T + 255) / 256), dim3(256), 0, s, T, it);
}

void launch_scatter(hipStream_t s, const CamParams& p, GaussOut go, const int* tile_bins,
                    int* tile_cnt, uint64_t* keys) {
    if (p.N <= 0) return;
    hipLaunchKernelGGL(k_scatter, dim3((p.N + 255) / 256), dim3(256), 0, s, p.N, p.tbx, p.tby, go,
                       tile_bins, tile_cnt, keys);
}

void launch_sort_pack(hipStream_t s, int T, const Meta& meta, const int* tile_bins,
                      TileLists tl, uint64_t* keys, uint64_t* scratch, GaussOut go, Packed pk) {
    if (meta.total_isect <= 0) return;
    hipLaunchKernelGGL(k_sort_small, dim3(T), dim3(256), 0, s, tile_bins, keys, go, pk);
    if (meta.n_large > 0)
        hipLaunchKernelGGL(k_sort_large, dim3(meta.n_large), dim3(256), 0, s, tl.large, tile_bins,
                           keys, go, pk);
    if (meta.n_huge > 0)
        hipLaunchKernelGGL(k_sort_huge, dim3(meta.n_huge), dim3(256), 0, s, tl.huge, tile_bins,
                           keys, scratch, go, pk);
}

}  // namespace msp
