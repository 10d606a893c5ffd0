// binning.hip — tile intersection lists in depth order, without atomics on
// the lists.
//
// Replaces scatter_to_prealloc_bins (.metal:2025-2059) + prefix_sum
// (.metal:2312-2364) + bitonic_sort_per_tile (.metal:2064-2138) with the same
// result — per tile, the ids of the gaussians whose tile rectangle covers it,
// ascending by (depth_bits, gaussian id), and tile_bins = (start, end) of each
// tile's range in one contiguous list, tiles in row-major order:
//   1. the projection wrote key = depth bits (0xFFFFFFFF if culled), value =
//      id, and the number of super-tiles (SUPER x SUPER tiles) each
//      gaussian's tile rectangle overlaps
//   2. radix sort by depth                        (order of gaussians)
//   3. super-tile counts gathered in that order by the scan -> offsets
//   4. one reference (super-tile, rectangle part, gaussian id) per
//      overlapped super-tile, in depth order
//   5. stable radix sort of the references by super-tile
//   6. each super-tile's (tile, gaussian) pairs, enumerated reference by
//      reference in blocks of PAIR_BLOCK: per-block pair counts of its 256
//      tiles, their scan over the super-tile's blocks and the tile scan ->
//      tile_bins and chunk work items; then each block ranks its pairs by
//      tile (stable), reorders them in LDS and writes the gaussian ids
//      straight to their tile ranges.
// Only the references (about one per visible gaussian) go through the
// radix sort and memory; the pairs exist in LDS only, and the one write of
// each pair is its final one.
// The rasteriser gathers each entry's projection record by id, in place of
// the reference's packed per-entry copies (.metal:2128-2137).
// Equal depths keep ascending id order because both sorts and the block
// ranking are stable and the first sort starts from id order.  Tiles have no
// size limit (the reference drops entries beyond 2048 per tile).
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

inline unsigned blocks_for(int64_t n) { return (unsigned)((n + 255) / 256); }

// Reference key: bits 0-15 the super-tile (row-major over the super-tile
// grid), 16-19 / 20-23 the first tile column / row of the rectangle's part
// inside it, 24-27 / 28-31 the part's width / height minus one.  The radix
// sort orders by the super-tile bits and carries the rest.
constexpr uint32_t ST_MASK = 0xFFFFu;

__device__ __forceinline__ int ref_pairs(uint32_t k) {
    return (int)(((k >> 24) & 15u) + 1u) * (int)(((k >> 28) & 15u) + 1u);
}

// Tile rectangles gathered into depth order, and each one's super-tile
// count (0 for culled gaussians, whose rectangle is empty and whose depth
// key, 0xFFFFFFFF, sorts them last: their rectangles are not gathered).
__global__ __launch_bounds__(256) void k_depth_rects(int N, const uint32_t* __restrict__ skey,
                                                     const uint32_t* __restrict__ order,
                                                     const uint2* __restrict__ rect,
                                                     uint2* __restrict__ rs,
                                                     int* __restrict__ cnt) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= N) return;
    const uint2 rc = skey[i] != 0xFFFFFFFFu ? rect[order[i]] : make_uint2(0u, 0u);
    rs[i] = rc;
    const int x0 = (int)(rc.x & 0xFFFFu), y0 = (int)(rc.x >> 16);
    const int x1 = (int)(rc.y & 0xFFFFu), y1 = (int)(rc.y >> 16);
    cnt[i] = (x1 > x0 && y1 > y0) ? super_span(x0, y0, x1, y1) : 0;
}

// References of the gaussians in depth order: the thread of depth rank r
// writes one per super-tile its tile rectangle overlaps (row by row), from
// roff[r] on.
__global__ __launch_bounds__(256) void k_emit_refs(int N, int sbx, const uint32_t* __restrict__ order,
                                                   const int* __restrict__ roff,
                                                   const uint2* __restrict__ rs,
                                                   uint32_t* __restrict__ rkey,
                                                   uint32_t* __restrict__ rval) {
    const int r = blockIdx.x * 256 + threadIdx.x;
    if (r >= N) return;
    const uint2 rc = rs[r];
    const int x0 = (int)(rc.x & 0xFFFFu), y0 = (int)(rc.x >> 16);
    const int x1 = (int)(rc.y & 0xFFFFu), y1 = (int)(rc.y >> 16);
    if (x1 <= x0 || y1 <= y0) return;
    const uint32_t g = order[r];
    int o = roff[r];
    for (int sy = y0 / SUPER; sy * SUPER < y1; ++sy) {
        const int ly0 = max(y0 - sy * SUPER, 0), ly1 = min(y1 - sy * SUPER, SUPER);
        for (int sx = x0 / SUPER; sx * SUPER < x1; ++sx) {
            const int lx0 = max(x0 - sx * SUPER, 0), lx1 = min(x1 - sx * SUPER, SUPER);
            rkey[o] = (uint32_t)(sy * sbx + sx) | (uint32_t)lx0 << 16 | (uint32_t)ly0 << 20 |
                      (uint32_t)(lx1 - lx0 - 1) << 24 | (uint32_t)(ly1 - ly0 - 1) << 28;
            rval[o] = g;
            ++o;
        }
    }
}

// Pairs of each sorted reference, and the reference range [st_r0, st_r1)
// of each super-tile present.
__global__ __launch_bounds__(256) void k_ref_pairs(int R, const uint32_t* __restrict__ rkey,
                                                   int* __restrict__ npairs,
                                                   int* __restrict__ st_r0,
                                                   int* __restrict__ st_r1) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= R) return;
    const uint32_t k = rkey[i];
    const uint32_t st = k & ST_MASK;
    npairs[i] = ref_pairs(k);
    if (i == 0 || (rkey[i - 1] & ST_MASK) != st) st_r0[st] = i;
    if (i == R - 1 || (rkey[i + 1] & ST_MASK) != st) st_r1[st] = i + 1;
}

// Exclusive scan of one value per thread over the NT threads of a block.
template <int NT>
__device__ __forceinline__ int block_exclusive_scan(int v, int* sh, int& total) {
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
    total = 0;
#pragma unroll
    for (int k = 0; k < NT / 64; ++k) {
        if (k < w) wofs += sh[k];
        total += sh[k];
    }
    __syncthreads();
    return wofs + x - v;
}

// Pair blocks of the super-tiles (one workgroup): super-tile s holds the
// pairs [st_p0, st_p1) of the global reference-order enumeration and
// ceil((st_p1 - st_p0) / PAIR_BLOCK) blocks from bstart[s] on; bstart[S] is
// the block count.  The reference ranges are moved to st_re and cleared for
// the next call (k_ref_pairs writes those of present super-tiles only).
__global__ __launch_bounds__(1024) void k_block_table(int S, int* __restrict__ st_r0,
                                                      int* __restrict__ st_r1,
                                                      const int* __restrict__ poff,
                                                      const int* __restrict__ npairs,
                                                      int* __restrict__ st_p0,
                                                      int* __restrict__ st_p1,
                                                      int* __restrict__ st_re,
                                                      int* __restrict__ bstart) {
    __shared__ int sh[16];
    const int per = (S + 1023) / 1024;
    const int b = min((int)threadIdx.x * per, S), e = min(b + per, S);
    int sum = 0;
    for (int s = b; s < e; ++s) {
        const int r0 = st_r0[s], r1 = st_r1[s];
        int p0 = 0, p1 = 0;
        if (r1 > r0) {
            p0 = poff[r0];
            p1 = poff[r1 - 1] + npairs[r1 - 1];
        }
        st_p0[s] = p0;
        st_p1[s] = p1;
        st_re[s] = r1;
        st_r0[s] = 0;
        st_r1[s] = 0;
        sum += (p1 - p0 + PAIR_BLOCK - 1) / PAIR_BLOCK;
    }
    int total;
    int run = block_exclusive_scan<1024>(sum, sh, total);
    for (int s = b; s < e; ++s) {
        bstart[s] = run;
        run += (st_p1[s] - st_p0[s] + PAIR_BLOCK - 1) / PAIR_BLOCK;
    }
    if (threadIdx.x == 0) bstart[S] = total;
}

// Pair block records: block bb of super-tile s starts in the reference i
// whose pairs contain pair bb * PAIR_BLOCK of the super-tile (a reference
// has at most 256 pairs, so at most one block starts in it); that thread
// writes the block's (super-tile, first reference, first pair, pair count),
// the window end of the block before it (the window runs through the
// reference holding the next block's first pair) and, for the super-tile's
// last block, its window end (the super-tile's last reference).
__global__ __launch_bounds__(256) void k_block_refs(int R, const uint32_t* __restrict__ rkey,
                                                    const int* __restrict__ poff,
                                                    const int* __restrict__ npairs,
                                                    const int* __restrict__ st_p0,
                                                    const int* __restrict__ st_p1,
                                                    const int* __restrict__ st_re,
                                                    const int* __restrict__ bstart,
                                                    int4* __restrict__ blk,
                                                    int* __restrict__ blk_wend) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= R) return;
    const int s = (int)(rkey[i] & ST_MASK);
    const int a = poff[i] - st_p0[s];
    const int bb = (a + PAIR_BLOCK - 1) / PAIR_BLOCK;
    if (bb * PAIR_BLOCK < a + npairs[i]) {
        const int j = bstart[s] + bb;
        const int p0 = st_p0[s] + bb * PAIR_BLOCK;
        blk[j] = make_int4(s, i, p0, min(PAIR_BLOCK, st_p1[s] - p0));
        if (bb > 0) blk_wend[j - 1] = i + 1;
        if (j == bstart[s + 1] - 1) blk_wend[j] = st_re[s];
    }
}

// Pair block set-up shared by the count and scatter kernels.
constexpr int PT = 1024;                  // threads per pair block
constexpr int PW = PT / 64;               // waves
constexpr int PK = PAIR_BLOCK / PT;       // pairs per thread
constexpr int WP = PAIR_BLOCK / PW;       // consecutive pairs per wave
static_assert(PK == 4, "the owner scan reads one int4 per thread");

struct PairArgs {
    int S;
    const uint32_t* rkey;
    const uint32_t* rval;
    const int* poff;
    const int* bstart;
    const int4* blk;
    const int* blk_wend;
};

// LDS of a pair block: the window of references whose pairs meet the block
// (key, first pair relative to the block, gaussian id) and the owner of
// each pair (its reference's index in the window).
struct __align__(16) PairLds {
    int own[PAIR_BLOCK];
    uint32_t rk[PAIR_BLOCK];
    int ro[PAIR_BLOCK];
    uint32_t rv[PAIR_BLOCK];
    int sh[PW];
};

// Loads block j's window into LDS and finds each pair's owner.  Returns the
// block's pair count (workgroup-uniform), or -1 past the last block; s is
// the block's super-tile.  Ends with a barrier.
template <bool VAL>
__device__ __forceinline__ int pair_block_load(int j, const PairArgs& a, PairLds& L, int& s) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    // one round trip for the block count and the block's record (in bounds
    // for every block of the grid; used only below the count)
    const int nblocks = a.bstart[a.S];
    const int4 b = a.blk[j];
    const int wend = a.blk_wend[j];
    if (j >= nblocks) return -1;
    s = b.x;
    const int rf = b.y, p0 = b.z, n = b.w;
    // references rf .. wend - 1 meet the block (the last one may start
    // exactly at its end); at most PAIR_BLOCK of them start before it
    const int nwin = min(wend - rf, PAIR_BLOCK);
    reinterpret_cast<int4*>(L.own)[tid] = make_int4(0, 0, 0, 0);
    int mark[PK];
#pragma unroll
    for (int k = 0; k < PK; ++k) {
        const int i = tid + k * PT;
        mark[k] = -1;
        if (i < nwin) {
            const int r = rf + i;
            const int o = a.poff[r] - p0;
            if (o < n) {
                L.rk[i] = a.rkey[r];
                L.ro[i] = o;
                if (VAL) L.rv[i] = a.rval[r];
                if (i > 0) mark[k] = o;   // reference rf owns pair 0 (the clear value)
            }
        }
    }
    __syncthreads();
#pragma unroll
    for (int k = 0; k < PK; ++k)
        if (mark[k] >= 0) L.own[mark[k]] = tid + k * PT;
    __syncthreads();
    // owner of pair q = the last reference starting at or before q: an
    // inclusive max scan (marks ascend with q), four pairs per thread
    int4 o4 = reinterpret_cast<int4*>(L.own)[tid];
    o4.y = max(o4.y, o4.x);
    o4.z = max(o4.z, o4.y);
    o4.w = max(o4.w, o4.z);
    int x = o4.w;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x = max(x, y);
    }
    if (lane == 63) L.sh[w] = x;
    int pre = __shfl_up(x, 1, 64);
    if (lane == 0) pre = 0;
    __syncthreads();
    for (int k = 0; k < w; ++k) pre = max(pre, L.sh[k]);
    o4.x = max(o4.x, pre);
    o4.y = max(o4.y, pre);
    o4.z = max(o4.z, pre);
    o4.w = max(o4.w, pre);
    reinterpret_cast<int4*>(L.own)[tid] = o4;
    __syncthreads();
    return n;
}

// Local tile (ly * SUPER + lx) of pair q of the block and its window index.
__device__ __forceinline__ int pair_tile(const PairLds& L, int q, int& i) {
    i = L.own[q];
    const uint32_t k = L.rk[i];
    const int loc = q - L.ro[i];   // pair index within the reference, row-major
    const int w = (int)((k >> 24) & 15u) + 1;
    // loc / w for loc < 256, w <= 16: (loc + 0.5) / w stays >= 1/32 away
    // from an integer, far beyond the rounding of the float product
    const int row = (int)(((float)loc + 0.5f) * (1.f / (float)w));
    const int col = loc - row * w;
    return ((int)((k >> 20) & 15u) + row) * SUPER + (int)((k >> 16) & 15u) + col;
}

// Pairs per local tile of each block -> hist[j * 256 + local tile].
__global__ __launch_bounds__(PT) void k_pair_hist(PairArgs a, int* __restrict__ hist) {
    __shared__ PairLds L;
    __shared__ int s_h[SUPER * SUPER];
    const int j = blockIdx.x, tid = threadIdx.x;
    if (tid < SUPER * SUPER) s_h[tid] = 0;
    int s;
    const int n = pair_block_load<false>(j, a, L, s);
    if (n < 0) return;
#pragma unroll
    for (int k = 0; k < PK; ++k) {
        const int q = tid + k * PT;
        if (q < n) {
            int i;
            atomicAdd(&s_h[pair_tile(L, q, i)], 1);
        }
    }
    __syncthreads();
    if (tid < SUPER * SUPER) hist[(size_t)j * (SUPER * SUPER) + tid] = s_h[tid];
}

// Per super-tile (one workgroup; thread d + 256 g handles local tile d in
// the g-th quarter of the super-tile's blocks): each block's count of a tile
// becomes the tile's pairs in the super-tile's earlier blocks, and the tile's
// total goes to tcount (every tile of the grid lies in exactly one
// super-tile, so tcount is rewritten whole).  Two passes over the counts:
// quarter totals, then offsets.
constexpr int PO_T = 4 * SUPER * SUPER;
__global__ __launch_bounds__(PO_T) void k_pair_offsets(int tbx, int tby, int sbx,
                                                       const int* __restrict__ bstart,
                                                       int* __restrict__ hist,
                                                       int* __restrict__ tcount) {
    __shared__ int part[4][SUPER * SUPER];
    const int s = blockIdx.x, d = threadIdx.x % (SUPER * SUPER), g = threadIdx.x / (SUPER * SUPER);
    const int b0 = bstart[s], b1 = bstart[s + 1];
    const int per = (b1 - b0 + 3) / 4;
    const int q0 = min(b0 + g * per, b1), q1 = min(q0 + per, b1);
    int sum = 0;
    for (int j = q0; j < q1; j += 8) {
#pragma unroll
        for (int u = 0; u < 8; ++u)
            sum += j + u < q1 ? hist[(size_t)(j + u) * (SUPER * SUPER) + d] : 0;
    }
    part[g][d] = sum;
    __syncthreads();
    int run = 0;
    for (int k = 0; k < g; ++k) run += part[k][d];
    for (int j = q0; j < q1; j += 8) {
        int c[8];
#pragma unroll
        for (int u = 0; u < 8; ++u)
            c[u] = j + u < q1 ? hist[(size_t)(j + u) * (SUPER * SUPER) + d] : 0;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
            if (j + u < q1) hist[(size_t)(j + u) * (SUPER * SUPER) + d] = run;
            run += c[u];
        }
    }
    if (g == 0) {
        const int tx = (s % sbx) * SUPER + (d % SUPER), ty = (s / sbx) * SUPER + d / SUPER;
        if (tx < tbx && ty < tby) tcount[ty * tbx + tx] = part[0][d] + part[1][d] + part[2][d] + part[3][d];
    }
}

// Pairs of each block ranked stably by local tile (each wave ranks its WP
// consecutive pairs in 64-pair rounds by ballot-matching the tile bits,
// keeping per-tile running counts; wave counts combine in wave order),
// reordered by tile in LDS and written to their tiles' ranges: tile start
// (tile_bins) + the tile's pairs in earlier blocks (hist) + rank.
// Consecutive blocks fill neighbouring parts of the same tiles' ranges: the
// grid is a multiple of 8 and workgroup b takes block (b % 8) * (grid / 8)
// + b / 8, so that the hardware's round-robin of workgroups over the 8 XCDs
// hands each XCD a contiguous run of blocks and their partial lines meet in
// one L2.  Blocks at or past nbound do not exist.
__global__ __launch_bounds__(PT) void k_pair_scatter(PairArgs a, int nbound, int tbx, int tby,
                                                     int sbx, const int* __restrict__ hist,
                                                     const int* __restrict__ tile_bins,
                                                     uint32_t* __restrict__ ids) {
    __shared__ PairLds L;
    __shared__ uint16_t wcnt[PW][SUPER * SUPER];
    __shared__ int dstart[SUPER * SUPER];
    __shared__ int gofs[SUPER * SUPER];
    __shared__ int scan_sh[PW];
    const int j = (int)(blockIdx.x % 8) * (int)(gridDim.x / 8) + (int)(blockIdx.x / 8);
    if (j >= nbound) return;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (int i = tid; i < PW * SUPER * SUPER; i += PT) (&wcnt[0][0])[i] = 0;
    int s;
    const int n = pair_block_load<true>(j, a, L, s);
    if (n < 0) return;
    // start of each local tile's range for this block, loaded now so that
    // the loads overlap the ranking
    int my_gofs = 0;
    if (tid < SUPER * SUPER) {
        const int tx = (s % sbx) * SUPER + (tid % SUPER), ty = (s / sbx) * SUPER + tid / SUPER;
        if (tx < tbx && ty < tby)
            my_gofs = tile_bins[2 * (ty * tbx + tx)] + hist[(size_t)j * (SUPER * SUPER) + tid];
    }
    const uint64_t lt = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
    int dig[PK], rank[PK];
    uint32_t val[PK];
#pragma unroll
    for (int k = 0; k < PK; ++k) {
        const int q = w * WP + k * 64 + lane;
        const bool ok = q < n;
        int d = SUPER * SUPER, i = 0;
        if (ok) d = pair_tile(L, q, i);
        val[k] = ok ? L.rv[i] : 0u;
        dig[k] = d;
        uint64_t peers = wave_ballot(ok);
        if (!ok) peers = ~peers;
#pragma unroll
        for (int b = 0; b < 8; ++b) {
            const uint64_t bb = wave_ballot((d >> b) & 1);
            peers &= ((d >> b) & 1) ? bb : ~bb;
        }
        const int before = __popcll(peers & lt);
        const int dd = ok ? d : 0;
        const int base_cnt = ok ? (int)wcnt[w][dd] : 0;
        rank[k] = base_cnt + before;
        // the lowest lane of each tile group advances that tile's count
        if (ok && before == 0) wcnt[w][dd] = (uint16_t)(base_cnt + __popcll(peers));
    }
    __syncthreads();
    // per local tile (threads 0..255): wave offsets in wave order, the
    // block's count and its start in the reordered block
    int cnt = 0;
    if (tid < SUPER * SUPER) {
#pragma unroll
        for (int ww = 0; ww < PW; ++ww) {
            const int c = wcnt[ww][tid];
            wcnt[ww][tid] = (uint16_t)cnt;
            cnt += c;
        }
        gofs[tid] = my_gofs;
    }
    int total;
    const int start = block_exclusive_scan<PT>(cnt, scan_sh, total);
    if (tid < SUPER * SUPER) dstart[tid] = start;
    __syncthreads();
    // reorder by tile: ids into L.own, tiles into L.ro (the window is no
    // longer read)
#pragma unroll
    for (int k = 0; k < PK; ++k) {
        const int d = dig[k];
        if (d >= SUPER * SUPER) continue;
        const int p = dstart[d] + (int)wcnt[w][d] + rank[k];
        L.own[p] = (int)val[k];
        L.ro[p] = d;
    }
    __syncthreads();
    for (int p = tid; p < n; p += PT) {
        const int d = L.ro[p];
        ids[gofs[d] + (p - dstart[d])] = (uint32_t)L.own[p];
    }
}

// Run edges of sorted keys (the knn's cell ranges): tstart[k] / tend[k] =
// first / one past the last position of key k.  Four keys per thread with
// one 16-byte load (tkey is 256-byte aligned); the neighbours across a
// thread's four come from single loads of the same or the adjacent line.
__global__ __launch_bounds__(256) void k_run_edges(int64_t I, const uint32_t* __restrict__ tkey,
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

__global__ __launch_bounds__(TS_T) void k_tile_counts(int T, const int* __restrict__ tcount,
                                                      int* __restrict__ tot,
                                                      Meta* __restrict__ meta) {
    __shared__ int sh[TS_T / 64];
    const int b = blockIdx.x;
    int sn = 0, sk = 0, mx = 0;
#pragma unroll
    for (int k = 0; k < TS_PER; ++k) {
        const int t = b * TS_BLOCK + k * TS_T + (int)threadIdx.x;
        if (t < T) {
            const int n = tcount[t];
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

__global__ __launch_bounds__(TS_T) void k_tile_offsets(int T, int nb,
                                                       const int* __restrict__ tcount,
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
        n[k] = t < T ? tcount[t] : 0;
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
        tile_bins[2 * t] = off;
        off += n[k];
        tile_bins[2 * t + 1] = off;
        it.tile_K[t] = K[k];
        it.tile_item0[t] = ioff;
        ioff += K[k];
        if (K[k] > 1) tl.chunked[atomicAdd(&meta->n_chunked_tiles, 1)] = t;
    }
    // the projection's intersection and reference counters, copied to the
    // host earlier on the stream, cleared for the next frame
    if (b == 0 && tid < 2 * ISECT_SLOTS) isect[(size_t)(tid >> 1) * ISECT_STRIDE + (tid & 1)] = 0ull;
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

}  // namespace

void launch_run_edges(hipStream_t s, int64_t n, const uint32_t* sorted_keys, int* start, int* end) {
    if (n > 0)
        hipLaunchKernelGGL(k_run_edges, dim3(blocks_for((n + 3) / 4)), dim3(256), 0, s, n,
                           sorted_keys, start, end);
}

void launch_depth_order(hipStream_t s, int N, uint32_t* dkey, uint32_t* dval, uint32_t* dkey2,
                        uint32_t* dval2, int* radix_temp, const uint2* rect, uint2* rect_sorted,
                        int* rcount, int* roff, int* scan_temp, uint32_t** order_out) {
    const bool flip = launch_radix_sort(s, dkey, dval, dkey2, dval2, N, 32, radix_temp);
    uint32_t* order = flip ? dval2 : dval;
    *order_out = order;
    if (N <= 0) return;
    // reference offsets: exclusive scan of the super-tile counts in depth order
    hipLaunchKernelGGL(k_depth_rects, dim3(blocks_for(N)), dim3(256), 0, s, N,
                       (const uint32_t*)(flip ? dkey2 : dkey), (const uint32_t*)order, rect,
                       rect_sorted, rcount);
    launch_exclusive_scan_i32(s, rcount, roff, N, scan_temp);
}

void launch_tile_lists(hipStream_t s, const CamParams& p, int64_t I, int64_t R,
                       const uint32_t* order, const int* roff, const uint2* rect_sorted, RefBufs rb,
                       uint32_t* ids, int* tscan, int* tile_bins, Items it, TileLists tl,
                       Meta* meta, unsigned long long* isect) {
    const int T = p.tbx * p.tby;
    const int sbx = (p.tbx + SUPER - 1) / SUPER, S = super_tiles(p.tbx, p.tby);
    const uint32_t* rk = rb.key;
    const uint32_t* rv = rb.val;
    if (R > 0) {
        hipLaunchKernelGGL(k_emit_refs, dim3(blocks_for(p.N)), dim3(256), 0, s, p.N, sbx, order,
                           roff, rect_sorted, rb.key, rb.val);
        int bits = 0;
        while ((1 << bits) < S) ++bits;
        if (launch_radix_sort(s, rb.key, rb.val, rb.key2, rb.val2, R, bits, rb.radix_temp)) {
            rk = rb.key2;
            rv = rb.val2;
        }
        hipLaunchKernelGGL(k_ref_pairs, dim3(blocks_for(R)), dim3(256), 0, s, (int)R, rk,
                           rb.npairs, rb.st_r0, rb.st_r1);
        launch_exclusive_scan_i32(s, rb.npairs, rb.poff, R, rb.scan_temp);
    }
    // with no references every super-tile is empty: zero blocks, zero counts
    hipLaunchKernelGGL(k_block_table, dim3(1), dim3(1024), 0, s, S, rb.st_r0, rb.st_r1,
                       (const int*)rb.poff, (const int*)rb.npairs, rb.st_p0, rb.st_p1, rb.st_re,
                       rb.bstart);
    const int64_t NB = pair_blocks_bound(I, S);
    PairArgs pa{S, rk, rv, rb.poff, rb.bstart, rb.blk, rb.blk_wend};
    if (R > 0) {
        hipLaunchKernelGGL(k_block_refs, dim3(blocks_for(R)), dim3(256), 0, s, (int)R, rk,
                           (const int*)rb.poff, (const int*)rb.npairs, (const int*)rb.st_p0,
                           (const int*)rb.st_p1, (const int*)rb.st_re, (const int*)rb.bstart,
                           rb.blk, rb.blk_wend);
        hipLaunchKernelGGL(k_pair_hist, dim3((unsigned)NB), dim3(PT), 0, s, pa, rb.hist);
    }
    hipLaunchKernelGGL(k_pair_offsets, dim3(S), dim3(PO_T), 0, s, p.tbx, p.tby, sbx,
                       (const int*)rb.bstart, rb.hist, rb.tcount);
    const int nb = (T + TS_BLOCK - 1) / TS_BLOCK;
    hipLaunchKernelGGL(k_tile_counts, dim3(nb), dim3(TS_T), 0, s, T, (const int*)rb.tcount, tscan,
                       meta);
    hipLaunchKernelGGL(k_tile_offsets, dim3(nb), dim3(TS_T), 0, s, T, nb, (const int*)rb.tcount,
                       (const int*)tscan, isect, tile_bins, it, tl, meta);
    hipLaunchKernelGGL(k_build_items, dim3(blocks_for(items_bound(T, I))), dim3(256), 0, s, T,
                       (const Meta*)meta, it);
    if (R > 0)
        hipLaunchKernelGGL(k_pair_scatter, dim3((unsigned)((NB + 7) / 8 * 8)), dim3(PT), 0, s, pa,
                           (int)NB, p.tbx, p.tby, sbx, (const int*)rb.hist,
                           (const int*)tile_bins, ids);
}

}  // namespace msp
