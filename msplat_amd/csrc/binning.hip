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
//   2. radix sort by depth                        (order of gaussians);
//      its last pass also gathers each gaussian's tile rectangle into that
//      order with its super-tile count (culled gaussians, whose key
//      0xFFFFFFFF sorts them last, get an empty rectangle and 0)
//   3. exclusive scan of the counts -> reference offsets
//   4. one reference (super-tile, rectangle part, gaussian id) per
//      overlapped super-tile, in depth order
//   5. stable radix sort of the references by super-tile
//   6. each super-tile's references cut into segments of SEG_REFS: the
//      segment's pair count of each of the super-tile's 256 tiles (2-D
//      difference array of the rectangles), their scan over the super-tile's
//      segments and the tile scan -> tile_bins and chunk work items; then
//      one wave per tile row of the segment's super-tile writes the gaussian
//      ids of the references covering the row straight to their tiles'
//      ranges, ranked per tile by ballots.
// Only the references (about one per visible gaussian) go through the radix
// sort and memory; each (tile, gaussian) entry is written once, in place.
// The rasteriser gathers each entry's projection record by id, in place of
// the reference's packed per-entry copies (.metal:2128-2137).
// Equal depths keep ascending id order because both sorts and the per-tile
// ranking keep their input order and the first sort starts from id order.  Tiles have no
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

// Reference range [st_r0, st_r1) of each super-tile present.
__global__ __launch_bounds__(256) void k_ref_edges(int R, const uint32_t* __restrict__ rkey,
                                                   int* __restrict__ st_r0,
                                                   int* __restrict__ st_r1) {
    const int i = blockIdx.x * 256 + threadIdx.x;
    if (i >= R) return;
    const uint32_t st = rkey[i] & ST_MASK;
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

// References of the gaussians in depth order: the thread of depth rank r
// writes one per super-tile its tile rectangle overlaps (row by row), from
// its first reference slot on.  The slots are the exclusive scan of the
// super-tile counts, finished here: the 1024 ranks of a workgroup (one scan
// block) scan their counts in the workgroup and add the totals of the scan
// blocks before them (summed here, or already scanned when there are more
// than SCAN_DIRECT_BLOCKS of them).
constexpr int EMIT_T = SCAN_BLOCK;
__global__ __launch_bounds__(EMIT_T) void k_emit_refs(int N, int sbx, const uint32_t* __restrict__ order,
                                                      const int* __restrict__ rtot,
                                                      const uint2* __restrict__ rs,
                                                      uint32_t* __restrict__ rkey,
                                                      uint32_t* __restrict__ rval) {
    constexpr int NW = EMIT_T / 64;
    __shared__ int sh_c[NW], sh_a[NW];
    const int r = blockIdx.x * EMIT_T + threadIdx.x;
    const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
    const int nb = (N + EMIT_T - 1) / EMIT_T;
    // this thread's share of the earlier blocks' totals (none when they are
    // already scanned) and its count; one pass scans the counts and sums the
    // shares over the workgroup
    int acc = 0;
    if (nb <= SCAN_DIRECT_BLOCKS)
        for (int b = threadIdx.x; b < (int)blockIdx.x; b += EMIT_T) acc += rtot[b];
    // the rectangle and id are loaded before the scan, and the count is taken
    // from the rectangle (as rcount holds it)
    const uint2 rc = r < N ? rs[r] : make_uint2(0u, 0u);
    const uint32_t g = r < N ? order[r] : 0u;
    const int x0 = (int)(rc.x & 0xFFFFu), y0 = (int)(rc.x >> 16);
    const int x1 = (int)(rc.y & 0xFFFFu), y1 = (int)(rc.y >> 16);
    const int c = (x1 > x0 && y1 > y0) ? super_span(x0, y0, x1, y1) : 0;
    int x = c;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        const int y = __shfl_up(x, off, 64);
        if (lane >= off) x += y;
        acc += __shfl_xor(acc, off, 64);
    }
    if (lane == 63) {
        sh_c[w] = x;
        sh_a[w] = acc;
    }
    __syncthreads();
    int o = nb > SCAN_DIRECT_BLOCKS ? rtot[blockIdx.x] : 0;
#pragma unroll
    for (int k = 0; k < NW; ++k) {
        if (k < w) o += sh_c[k];
        o += sh_a[k];
    }
    o += x - c;
    if (c == 0) return;   // culled, or an empty rectangle
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

// Rectangle part of a reference key in local tile coordinates [x0, x1) x [y0, y1).
__device__ __forceinline__ void ref_rect(uint32_t k, int& x0, int& y0, int& x1, int& y1) {
    x0 = (int)((k >> 16) & 15u);
    y0 = (int)((k >> 20) & 15u);
    x1 = x0 + (int)((k >> 24) & 15u) + 1;
    y1 = y0 + (int)((k >> 28) & 15u) + 1;
}

// Tile scan blocks: TS_BLOCK tiles of the row-major tile order per
// workgroup of TS_T threads (k_tile_offsets); their sums (count, chunk
// items, largest count) are added up by k_seg_offsets.
constexpr int TS_T = 256, TS_PER = 4, TS_BLOCK = TS_T * TS_PER;

// Segments and their pair counts, one workgroup per segment (grid: the
// segments_bound of the call).  Each workgroup first works out the segment
// table itself from the super-tiles' reference ranges [st_r0, st_r1):
// super-tile s's references are cut into ceil(n / SEG_REFS) segments of
// SEG_REFS consecutive ones, numbered from sstart[s] on (sstart[S] = the
// segment count; workgroup 0 writes sstart).  That is a scan over the S
// super-tiles in every workgroup, a few values per thread at the image sizes
// this serves.  Workgroup j then records its segment (super-tile, reference
// range) in seg[j] and counts the pairs per local tile of its references ->
// hist[j * 256 + ly * 16 + lx]: the rectangles are added to a 17 x 17
// difference array (four LDS atomics each) whose 2-D prefix sums are the
// counts.
constexpr int DW = SUPER + 1;
__global__ __launch_bounds__(256) void k_seg_count(int S, const int* __restrict__ st_r0,
                                                   const int* __restrict__ st_r1,
                                                   int* __restrict__ sstart,
                                                   int4* __restrict__ seg,
                                                   const uint32_t* __restrict__ rkey,
                                                   int* __restrict__ hist, int* __restrict__ tot,
                                                   int ntb, int* __restrict__ cls,
                                                   Meta* __restrict__ meta) {
    __shared__ int diff[DW * DW];
    __shared__ int sh[4];
    __shared__ int4 s_rec;
    const int j = blockIdx.x, tid = threadIdx.x;
    if (j == 0) {
        // this frame's tile scan sums (k_seg_offsets adds to them), size-class
        // counters (k_tile_offsets adds, the item build reads) and chunked-tile
        // count start at zero; the previous frame read them before this launch
        for (int i = tid; i < 3 * ntb; i += 256) tot[i] = 0;
        if (tid < 128) cls[tid] = 0;
        if (tid == 0) meta->n_chunked_tiles = 0;
    }
    const int per = (S + 255) / 256;
    const int b = min(tid * per, S), e = min(b + per, S);
    int sum = 0;
    for (int t = b; t < e; ++t) sum += (st_r1[t] - st_r0[t] + SEG_REFS - 1) / SEG_REFS;
    if (tid == 0) s_rec = make_int4(0, 0, 0, 0);
    int nseg;
    int run = block_exclusive_scan<256>(sum, sh, nseg);
    for (int t = b; t < e; ++t) {
        const int r0 = st_r0[t], r1 = st_r1[t];
        const int n = (r1 - r0 + SEG_REFS - 1) / SEG_REFS;
        if (j == 0) sstart[t] = run;
        if (j >= run && j < run + n) {
            const int rs0 = r0 + (j - run) * SEG_REFS;
            s_rec = make_int4(t, rs0, min(rs0 + SEG_REFS, r1), 0);
        }
        run += n;
    }
    if (j == 0 && tid == 0) sstart[S] = nseg;
    __syncthreads();
    if (j >= nseg) return;
    const int4 sg = s_rec;
    if (tid == 0) seg[j] = sg;
    for (int i = tid; i < DW * DW; i += 256) diff[i] = 0;
    __syncthreads();
    for (int r = sg.y + tid; r < sg.z; r += 256) {
        int x0, y0, x1, y1;
        ref_rect(rkey[r], x0, y0, x1, y1);
        atomicAdd(&diff[y0 * DW + x0], 1);
        atomicAdd(&diff[y0 * DW + x1], -1);
        atomicAdd(&diff[y1 * DW + x0], -1);
        atomicAdd(&diff[y1 * DW + x1], 1);
    }
    __syncthreads();
    if (tid < SUPER) {   // prefix along x of row tid
        int run = 0;
        for (int x = 0; x < SUPER; ++x) {
            run += diff[tid * DW + x];
            diff[tid * DW + x] = run;
        }
    }
    __syncthreads();
    if (tid < SUPER) {   // prefix along y of column tid
        int run = 0;
        for (int y = 0; y < SUPER; ++y) {
            run += diff[y * DW + tid];
            diff[y * DW + tid] = run;
        }
    }
    __syncthreads();
    hist[(size_t)j * (SUPER * SUPER) + tid] = diff[(tid / SUPER) * DW + tid % SUPER];
}

// Per super-tile s and quarter q of its 256 tiles (workgroup (s, q); thread
// d + 64 g handles local tile 64 q + d in the g-th of 16 groups of the
// super-tile's segments): each segment's count of a tile becomes the tile's
// pairs in the super-tile's earlier segments, and the tile's total goes to
// tcount (every tile of the grid lies in exactly one super-tile, so tcount
// is rewritten whole).  Two passes over the counts: group totals, then
// offsets.  Workgroup (s, 0) also clears super-tile s's reference range for
// the next call (k_ref_edges writes those of present super-tiles only; every
// k_seg_count workgroup has read them by now).
constexpr int SO_G = 16, SO_D = 64, SO_T = SO_G * SO_D;
__global__ __launch_bounds__(SO_T) void k_seg_offsets(int tbx, int tby, int sbx,
                                                      const int* __restrict__ sstart,
                                                      int* __restrict__ hist,
                                                      int* __restrict__ tcount,
                                                      int* __restrict__ st_r0,
                                                      int* __restrict__ st_r1,
                                                      int* __restrict__ tot) {
    __shared__ int part[SO_G][SO_D];
    const int s = blockIdx.x, tile = blockIdx.y * SO_D + threadIdx.x % SO_D;
    if (blockIdx.y == 0 && threadIdx.x == 0) {
        st_r0[s] = 0;
        st_r1[s] = 0;
    }
    const int d = threadIdx.x % SO_D, g = threadIdx.x / SO_D;
    const int b0 = sstart[s], b1 = sstart[s + 1];
    const int per = (b1 - b0 + SO_G - 1) / SO_G;
    const int q0 = min(b0 + g * per, b1), q1 = min(q0 + per, b1);
    int sum = 0;
    for (int j = q0; j < q1; j += 4) {
#pragma unroll
        for (int u = 0; u < 4; ++u)
            sum += j + u < q1 ? hist[(size_t)(j + u) * (SUPER * SUPER) + tile] : 0;
    }
    part[g][d] = sum;
    __syncthreads();
    int run = 0, total = 0;
#pragma unroll
    for (int k = 0; k < SO_G; ++k) {
        if (k < g) run += part[k][d];
        total += part[k][d];
    }
    for (int j = q0; j < q1; j += 4) {
        int c[4];
#pragma unroll
        for (int u = 0; u < 4; ++u)
            c[u] = j + u < q1 ? hist[(size_t)(j + u) * (SUPER * SUPER) + tile] : 0;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
            if (j + u < q1) hist[(size_t)(j + u) * (SUPER * SUPER) + tile] = run;
            run += c[u];
        }
    }
    if (g == 0) {   // wave 0: the quarter's 64 tiles
        const int tx = (s % sbx) * SUPER + (tile % SUPER), ty = (s / sbx) * SUPER + tile / SUPER;
        const bool in = tx < tbx && ty < tby;
        const int t = ty * tbx + tx;
        if (in) tcount[t] = total;
        // The tile scan's block sums: count, chunk items and largest count of
        // each block of TS_BLOCK row-major tiles.  The quarter's 64 tiles fall
        // in a few blocks; each block's lanes add with one atomic per sum.
        const int blk = in ? t / TS_BLOCK : -1;
        const int kch = in ? tile_chunks(total, tbx * tby) : 0;
        const int lane = threadIdx.x & 63;
        uint64_t left = wave_ballot(in);
        while (left) {
            const int first = (int)__builtin_ctzll(left);
            const int bl = __builtin_amdgcn_readlane(blk, first);
            const bool mine = in && blk == bl;
            int sn = mine ? total : 0, sk = mine ? kch : 0, mx = mine ? total : 0;
            for (int off = 32; off >= 1; off >>= 1) {
                sn += __shfl_xor(sn, off, 64);
                sk += __shfl_xor(sk, off, 64);
                mx = max(mx, __shfl_xor(mx, off, 64));
            }
            if (lane == first) {
                atomicAdd(&tot[3 * bl], sn);
                atomicAdd(&tot[3 * bl + 1], sk);
                atomicMax(&tot[3 * bl + 2], mx);
            }
            left &= ~wave_ballot(mine);
        }
    }
}

// Ids of up to 64 references of one tile row (lane < cnt holds reference
// k / gaussian g), written to their tiles: for each column x of the row, the
// lanes covering tile x write to its next free slots base[x].. in lane
// order, so each store instruction writes consecutive slots of one tile.
__device__ __forceinline__ void write_row_refs(bool ok, uint32_t k, uint32_t g, int* base,
                                               uint32_t* __restrict__ ids) {
    int x0, y0, x1, y1;
    ref_rect(k, x0, y0, x1, y1);
    const uint32_t cols = ok ? ((1u << x1) - 1u) & ~((1u << x0) - 1u) : 0u;
#pragma unroll
    for (int x = 0; x < SUPER; ++x) {
        const bool on = (cols >> x) & 1u;
        const uint64_t b = wave_ballot(on);
        if (b == 0) continue;
        // covering lanes below this one
        const int below = (int)__builtin_amdgcn_mbcnt_hi(
            (uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        if (on) ids[base[x] + below] = g;
        base[x] += __popcll(b);
    }
}

// Gaussian ids of each segment written to their tiles' ranges.  The
// segment's references are staged in LDS; wave ly of the workgroup owns
// local tile row ly: it walks them in order, 64 per round, appends the ones
// whose rectangle covers its row to a ring of reference indices, and writes
// each full group of 64 (and the rest at the end) with write_row_refs.  A
// tile's next free slot starts at the tile's start + its pairs in earlier
// segments; the 16 of the row are wave-uniform (scalar registers).  Entries
// keep reference (depth) order per tile.
// Segment j's part, by a workgroup of 1024 threads (16 waves).
__device__ __forceinline__ void seg_write(int j, int S, const int* __restrict__ sstart,
                                          const int4* __restrict__ seg,
                                          const uint32_t* __restrict__ rkey,
                                          const uint32_t* __restrict__ rval,
                                          const int* __restrict__ hist,
                                          const int* __restrict__ tile_bins, int tbx, int tby,
                                          int sbx, uint32_t* __restrict__ ids) {
    __shared__ uint32_t s_k[SEG_REFS], s_g[SEG_REFS];
    // bit y: the reference covers local tile row y; zero past the segment's
    // last reference up to a multiple of 64
    __shared__ uint16_t s_m[SEG_REFS];
    __shared__ uint16_t s_q[SUPER][128];   // per row: ring of covering reference indices
    const int lane = threadIdx.x & 63, ly = threadIdx.x >> 6;
    const int nseg = sstart[S];
    const int4 sg = seg[j];
    if (j >= nseg) return;
    const int s = sg.x;
    const int n = sg.z - sg.y;
    const int n64 = (n + 63) & ~63;
    for (int i = threadIdx.x; i < n64; i += 1024) {
        uint32_t k = 0u, m = 0u;
        if (i < n) {
            k = rkey[sg.y + i];
            s_k[i] = k;
            s_g[i] = rval[sg.y + i];
            const uint32_t y0 = (k >> 20) & 15u, y1 = y0 + ((k >> 28) & 15u) + 1u;
            m = ((1u << y1) - 1u) & ~((1u << y0) - 1u);
        }
        s_m[i] = (uint16_t)m;
    }
    const int ty = (s / sbx) * SUPER + ly;
    int myb = 0;
    if (lane < SUPER) {
        const int tx = (s % sbx) * SUPER + lane;
        if (tx < tbx && ty < tby)
            myb = tile_bins[2 * (ty * tbx + tx)] + hist[(size_t)j * (SUPER * SUPER) + ly * SUPER + lane];
    }
    int base[SUPER];
#pragma unroll
    for (int x = 0; x < SUPER; ++x) base[x] = __builtin_amdgcn_readlane(myb, x);
    __syncthreads();
    int head = 0, tail = 0;   // wave-uniform ring positions (tail - head <= 127)
    for (int r0 = 0; r0 < n; r0 += 64) {
        const int r = r0 + lane;
        const bool cov = (s_m[r] >> ly) & 1u;
        const uint64_t b = wave_ballot(cov);
        const int below = (int)__builtin_amdgcn_mbcnt_hi(
            (uint32_t)(b >> 32), __builtin_amdgcn_mbcnt_lo((uint32_t)b, 0u));
        if (cov) s_q[ly][(tail + below) & 127] = (uint16_t)r;
        tail += __popcll(b);
        if (tail - head >= 64) {
            __builtin_amdgcn_wave_barrier();
            const int i = s_q[ly][(head + lane) & 127];
            write_row_refs(true, s_k[i], s_g[i], base, ids);
            head += 64;
            __builtin_amdgcn_wave_barrier();
        }
    }
    if (tail > head) {
        __builtin_amdgcn_wave_barrier();
        const bool ok = head + lane < tail;
        const int i = ok ? s_q[ly][(head + lane) & 127] : 0;
        write_row_refs(ok, s_k[i], s_g[i], base, ids);
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

// Tile scan over TS_BLOCK tiles per workgroup: k_seg_offsets has added up
// each block's tile count total, chunk-item total and largest count.
// k_tile_offsets: each block adds the totals of the blocks before it, scans
// its own tiles and writes tile_bins, the chunk counts and first items and
// the list of chunked tiles; the last block writes the summary.  Then
// build_items (in k_lists_and_items) writes the work items (tile, chunk), one
// thread per item.

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

// Size class of a tile of n entries in K work items: floor(log2) of the
// entries of one item (0 for an empty tile).  The raster kernels take items
// and tiles in descending class, so the longest ones start first.
__device__ __forceinline__ int size_class(int n, int K) {
    const int w = K == 1 ? n : min(n, CHUNK);
    return w > 0 ? 31 - __clz(w) : 0;
}

__global__ __launch_bounds__(TS_T) void k_tile_offsets(int T, int nb,
                                                       const int* __restrict__ tcount,
                                                       const int* __restrict__ tot,
                                                       unsigned long long* __restrict__ isect,
                                                       int* __restrict__ tile_bins, Items it,
                                                       TileLists tl, Meta* __restrict__ meta) {
    __shared__ int sh[TS_T / 64];
    __shared__ int s_n[TS_T], s_k[TS_T];
    __shared__ int s_cls[64];       // this block's items / tiles per size class
    const int b = blockIdx.x, tid = threadIdx.x;
    if (tid < 64) s_cls[tid] = 0;
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
        const int c = size_class(n[k], K[k]);
        atomicAdd(&s_cls[c], K[k]);
        atomicAdd(&s_cls[32 + c], 1);
    }
    __syncthreads();
    if (tid < 32) {
        if (s_cls[tid]) atomicAdd(&it.cls[tid], s_cls[tid]);
        if (s_cls[32 + tid]) atomicAdd(&it.cls[64 + tid], s_cls[32 + tid]);
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

// Slot of this lane's element in descending size-class order: base[c] is
// the first slot of class c (the elements of higher classes before it) and
// fill[c] the class's running fill; the lanes of a wave with the same class
// take consecutive slots with one atomic.
__device__ __forceinline__ int class_slot(bool ok, int c, const int* base, int* fill) {
    const int lane = threadIdx.x & 63;
    uint64_t peers = wave_ballot(ok);
#pragma unroll
    for (int bit = 0; bit < 5; ++bit) {
        const uint64_t bb = wave_ballot((c >> bit) & 1);
        peers &= ((c >> bit) & 1) ? bb : ~bb;
    }
    const uint64_t lt = lane == 0 ? 0ull : (~0ull >> (64 - lane));
    const int before = __popcll(peers & lt);
    int first = 0;
    if (ok && before == 0) first = atomicAdd(&fill[c], __popcll(peers));
    // the group's first slot from its lowest lane
    first = __shfl(first, __builtin_ctzll(peers | (1ull << 63)), 64);
    return base[c] + first + before;
}

// Work item i: the tile t with tile_item0[t] <= i < tile_item0[t + 1] (every
// tile has at least one item, so the first items ascend), found by binary
// search, and its chunk i - tile_item0[t].  Each item, and each tile (thread
// i < T), also takes its slot in the launch orders, heaviest class first.
// Items vb * blockDim.x .. of the workgroup's share (any block size).
__device__ __forceinline__ void build_items(int vb, int T, const Meta* __restrict__ meta,
                                            const int* __restrict__ tile_bins, Items it) {
    __shared__ int s_base[2][32];
    const int i = vb * (int)blockDim.x + (int)threadIdx.x;
    if (threadIdx.x < 64) {
        // first slot of each class: the elements of all higher classes
        const int k = threadIdx.x >> 5, c = threadIdx.x & 31;
        int sum = 0;
        for (int d = 31; d > c; --d) sum += it.cls[64 * k + d];
        s_base[k][c] = sum;
    }
    __syncthreads();
    const int n_items = meta->n_items;
    const bool item_ok = i < n_items;
    int c = 0;
    if (item_ok) {
        int lo = 0, hi = T - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (it.tile_item0[mid] <= i) lo = mid; else hi = mid - 1;
        }
        it.tile[i] = lo;
        it.k[i] = i - it.tile_item0[lo];
        c = size_class(tile_bins[2 * lo + 1] - tile_bins[2 * lo], it.tile_K[lo]);
    }
    if (__syncthreads_or(item_ok)) {
        const int slot = class_slot(item_ok, c, s_base[0], it.cls + 32);
        if (item_ok) it.order[slot] = i;
    }
    const bool tile_ok = i < T;
    int ct = 0;
    if (tile_ok) ct = size_class(tile_bins[2 * i + 1] - tile_bins[2 * i], it.tile_K[i]);
    if (__syncthreads_or(tile_ok)) {
        const int slot = class_slot(tile_ok, ct, s_base[1], it.cls + 96);
        if (tile_ok) it.tile_order[slot] = i;
    }
}

// The tile lists' last two jobs in one launch, both reading the tile
// ranges of the tile scan and nothing of each other: workgroups 0 .. nsb - 1
// write segment j's ids (seg_write), the rest build the work items and the
// launch orders (build_items), so the item build runs beside the id writes
// instead of after a launch of its own.
__global__ __launch_bounds__(1024) void k_lists_and_items(int nsb, int S, const int* __restrict__ sstart,
                                                          const int4* __restrict__ seg,
                                                          const uint32_t* __restrict__ rkey,
                                                          const uint32_t* __restrict__ rval,
                                                          const int* __restrict__ hist,
                                                          const int* __restrict__ tile_bins, int tbx,
                                                          int tby, int sbx, uint32_t* __restrict__ ids,
                                                          int T, const Meta* __restrict__ meta,
                                                          Items it) {
    if ((int)blockIdx.x >= nsb) {
        build_items((int)blockIdx.x - nsb, T, meta, tile_bins, it);
        return;
    }
    seg_write((int)blockIdx.x, S, sstart, seg, rkey, rval, hist, tile_bins, tbx, tby, sbx, ids);
}

}  // namespace

void launch_run_edges(hipStream_t s, int64_t n, const uint32_t* sorted_keys, int* start, int* end) {
    if (n > 0)
        hipLaunchKernelGGL(k_run_edges, dim3(blocks_for((n + 3) / 4)), dim3(256), 0, s, n,
                           sorted_keys, start, end);
}

void launch_depth_order(hipStream_t s, int N, uint32_t* dkey, uint32_t* dval, uint32_t* dkey2,
                        uint32_t* dval2, int* radix_temp, const uint2* rect, uint2* rect_sorted,
                        int* rcount, int* rtot, const SlotSum* ss, uint32_t** order_out) {
    // the sort's last pass gathers the rectangles into depth order and
    // counts their super-tiles
    const RectGather rg{rect, rect_sorted, rcount};
    // culled gaussians (key 0xFFFFFFFF) go behind the visible ones in the
    // first pass and the later passes sort only the visible ones
    const bool flip = launch_radix_sort(s, dkey, dval, dkey2, dval2, N, 32, radix_temp, &rg, ss,
                                        nullptr, nullptr, true);
    uint32_t* order = flip ? dval2 : dval;
    *order_out = order;
    if (N <= 0) return;
    // the block totals of the super-tile counts in depth order (the reference
    // emission finishes their scan)
    launch_block_totals(s, rcount, N, rtot);
}

void launch_tile_lists(hipStream_t s, const CamParams& p, int64_t I, int64_t R,
                       const uint32_t* order, const int* rtot,
                       const uint2* rect_sorted, RefBufs rb,
                       uint32_t* ids, int* tscan, int* tile_bins, Items it, TileLists tl,
                       Meta* meta, unsigned long long* isect) {
    const int T = p.tbx * p.tby;
    const int sbx = (p.tbx + SUPER - 1) / SUPER, S = super_tiles(p.tbx, p.tby);
    const uint32_t* rk = rb.key;
    const uint32_t* rv = rb.val;
    if (R > 0) {
        hipLaunchKernelGGL(k_emit_refs, dim3((unsigned)((p.N + EMIT_T - 1) / EMIT_T)), dim3(EMIT_T), 0, s,
                           p.N, sbx, order, rtot, rect_sorted, rb.key, rb.val);
        int bits = 0;
        while ((1 << bits) < S) ++bits;
        // a single-pass sort (at most 512 super-tiles, 9 bits) writes the
        // super-tiles' reference ranges itself; otherwise they are found in
        // the sorted keys
        if (launch_radix_sort(s, rb.key, rb.val, rb.key2, rb.val2, R, bits, rb.radix_temp, nullptr,
                              nullptr, rb.st_r0, rb.st_r1)) {
            rk = rb.key2;
            rv = rb.val2;
        }
        if (bits == 0 || bits > 9)   // one super-tile (no sort), or a two-pass sort
            hipLaunchKernelGGL(k_ref_edges, dim3(blocks_for(R)), dim3(256), 0, s, (int)R, rk,
                               rb.st_r0, rb.st_r1);
    }
    // with no references every super-tile is empty: no segments (workgroup 0
    // still writes the segment table), zero counts
    const int64_t NS = segments_bound(R, S);
    const int nb = (T + TS_BLOCK - 1) / TS_BLOCK;
    hipLaunchKernelGGL(k_seg_count, dim3((unsigned)NS), dim3(256), 0, s, S,
                       (const int*)rb.st_r0, (const int*)rb.st_r1, rb.sstart, rb.seg, rk, rb.hist,
                       tscan, nb, it.cls, meta);
    hipLaunchKernelGGL(k_seg_offsets, dim3(S, SUPER * SUPER / SO_D), dim3(SO_T), 0, s, p.tbx,
                       p.tby, sbx,
                       (const int*)rb.sstart, rb.hist, rb.tcount, rb.st_r0, rb.st_r1, tscan);
    hipLaunchKernelGGL(k_tile_offsets, dim3(nb), dim3(TS_T), 0, s, T, nb, (const int*)rb.tcount,
                       (const int*)tscan, isect, tile_bins, it, tl, meta);
    // segment ids (with any references) and work items in one launch
    const int nsb = R > 0 ? (int)NS : 0;
    const int nib = (int)((std::max<int64_t>(items_bound(T, I), T) + 1023) / 1024);
    hipLaunchKernelGGL(k_lists_and_items, dim3((unsigned)(nsb + nib)), dim3(1024), 0, s, nsb, S,
                       (const int*)rb.sstart, (const int4*)rb.seg, rk, rv, (const int*)rb.hist,
                       (const int*)tile_bins, p.tbx, p.tby, sbx, ids, T, (const Meta*)meta, it);
}

}  // namespace msp
