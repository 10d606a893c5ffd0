// raster.hip — alpha compositing forward, chunk merge and backward.
//
// Work decomposition: one 256-thread workgroup (four wave64) per (tile,
// chunk) item; each wave owns one 8x8 quadrant of the 16x16 tile, one lane per
// pixel.  Sorted entries (gaussian ids; each entry's projection record is
// gathered by id) are staged through LDS 256 at a time and read by all lanes
// as broadcasts.  A tile that is rasterised in one piece writes the
// final image directly; a chunked tile writes per-pixel chunk state that the
// merge kernel folds front to back.
//
// Semantics follow the reference exactly:
//   forward      nd_rasterize_forward_kernel (.metal:472-585)
//   chunked fwd  rasterize_forward_chunked_kernel (.metal:2633-2741)
//   merge        rasterize_forward_merge_kernel (.metal:2746-2799)
//   prefix/sfx   compute_chunk_prefix_suffix_kernel (.metal:2804-2840)
//   backward     rasterize_backward_kernel (.metal:898-1099) and
//                rasterize_backward_chunked_kernel (.metal:2844-3031)
// with these MI355X differences: each loaded entry carries a conservative
// mask of the 8x8 wave quadrants it can reach and a wave walks only the
// entries of its own quadrant; a workgroup-wide vote stops the forward once
// every pixel of the item has terminated; the backward reduces each
// gaussian's per-pixel terms across the 64 lanes of a wave (eight of them
// transposed through LDS, the ninth by DPP) and nine lanes issue one float
// atomic each.
#include "common.hpp"
#include "kernels.hpp"

namespace msp {

namespace {

struct Px {
    int i, j;      // pixel row / column
    int lp;        // local pixel index within the tile (ly * 16 + lx)
    bool inside;
};

__device__ __forceinline__ Px pixel_of(int t, int tbx, int W, int H) {
    const int tid = threadIdx.x, w = tid >> 6, l = tid & 63;
    const int lx = (w & 1) * 8 + (l & 7), ly = (w >> 1) * 8 + (l >> 3);
    Px p;
    p.j = (t % tbx) * BLOCK + lx;
    p.i = (t / tbx) * BLOCK + ly;
    p.lp = ly * BLOCK + lx;
    p.inside = p.i < H && p.j < W;
    return p;
}

// Pair counters: WORK_SLOTS copies of the counter set, one 128-byte line
// each, picked by block id, so that the atomics of concurrent workgroups do
// not serialise on one address; the host sums the slots.
__device__ __forceinline__ unsigned long long* work_slot(unsigned long long* work) {
    return work + (size_t)(blockIdx.x % WORK_SLOTS) * WORK_SLOT_U64;
}

__device__ __forceinline__ void item_range(const Items& it, const int* tile_bins, int item,
                                           int& t, int& K, int& cs, int& ce) {
    t = it.tile[item];
    const int k = it.k[item];
    K = it.tile_K[t];
    const int s = tile_bins[2 * t], e = tile_bins[2 * t + 1];
    if (K == 1) {
        cs = s;
        ce = e;
    } else {
        cs = s + k * CHUNK;
        ce = min(cs + CHUNK, e);
    }
}

// Minimum over the segment X = const, Y in [y0, y1] of
// q(X, Y) = 0.5 (a X^2 + c Y^2) + b X Y  (c > 0, ic = 1 / c).
__device__ __forceinline__ float qmin_edge(float a, float b, float c, float ic, float X, float y0,
                                           float y1) {
    const float Y = fminf(fmaxf(-b * X * ic, y0), y1);
    return 0.5f * (a * X * X + c * Y * Y) + b * X * Y;
}

// Conservative quadrant mask of one entry: bit w is set when the entry can
// reach alpha >= 1/255 at a pixel of wave w's 8x8 quadrant of the tile at
// (tx0, ty0).  The reach is sigma < min(5.55, ln(255 o)); the test takes the
// exact minimum of the convex quadratic sigma over the quadrant's pixel
// rectangle (zero when the centre lies inside, else the least of the four
// edge minima) and compares it with the threshold plus a margin far above
// fp32 rounding.  Entries outside a quadrant are exactly the ones the
// per-pixel tests would skip there, so culling them changes no result.
__device__ __forceinline__ int quad_mask(float x, float y, float a, float b, float c, float o,
                                         int tx0, int ty0) {
    if (!(o >= 0.0039f)) return o == o ? 0 : 0xF;      // alpha <= o < 1/255 everywhere
    const float det = a * c - b * b;
    if (!(det > 0.f) || !(a > 0.f) || !(c > 0.f) || !(a < 1e30f) || !(c < 1e30f) ||
        !(fabsf(b) < 1e30f) || !(fabsf(x) < 1e30f) || !(fabsf(y) < 1e30f))
        return 0xF;
    const float thr = fminf(5.55f, __logf(255.f * o) + 0.05f) * 1.002f + 1e-3f;
    const float ia = 1.f / a, ic = 1.f / c;
    int m = 0;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const float qx0 = (float)(tx0 + (q & 1) * 8), qy0 = (float)(ty0 + (q >> 1) * 8);
        // offsets d = centre - pixel over the quadrant's pixels
        const float dx0 = x - (qx0 + 7.f), dx1 = x - qx0;
        const float dy0 = y - (qy0 + 7.f), dy1 = y - qy0;
        const bool inside = dx0 <= 0.f && dx1 >= 0.f && dy0 <= 0.f && dy1 >= 0.f;
        const float e = fminf(fminf(qmin_edge(a, b, c, ic, dx0, dy0, dy1),
                                    qmin_edge(a, b, c, ic, dx1, dy0, dy1)),
                              fminf(qmin_edge(c, b, a, ia, dy0, dx0, dx1),
                                    qmin_edge(c, b, a, ia, dy1, dx0, dx1)));
        if (inside || e < thr) m |= 1 << q;
    }
    return m;
}

// The reference's range early-out, skip when sigma < 0 || sigma >= 5.55
// (.metal:551, 1029, 2718, 2976), folded into the alpha test: sigma's bits
// are clamped with one unsigned min to those of 5.55f (0x40B1999A), so sigma
// in [+0, 5.55) keeps its value and everything else (negative, -0, >= 5.55,
// +inf, NaN) becomes 5.55, where alpha = min(0.999, o exp(-5.55)) <=
// 0.0038875 < 1/255 for every opacity in [0, 1] and the alpha test rejects
// the pair.  One vector min replaces two compares and two scalar ands per
// entry step; the decision differs from the reference's only for sigma = -0
// or NaN (a degenerate conic), which are rejected here, and for a NaN
// opacity (alpha 0.999 wherever the entry is walked).
__device__ __forceinline__ float sigma_clamp(float s) {
    return __uint_as_float(min(__float_as_uint(s), 0x40B1999Au));
}

// Entry record at byte offset qb of an LDS array of float4.
__device__ __forceinline__ float4 lds_f4(const float4* base, int qb) {
    return *static_cast<const float4*>(
        __builtin_assume_aligned(reinterpret_cast<const char*>(base) + qb, 16));
}

// LDS row of one reduced value: the 64 lane partials.  The 8-lane groups of
// odd rows read their two 16-byte halves in the opposite order, so that the
// two groups served in the same LDS cycle (rows 2p and 2p + 1) read
// disjoint banks.
constexpr int RED_ROW = 64;

// Sum over the 64 lanes of a wave of eight values per lane, through the
// wave's own LDS area red[8][RED_ROW], in three parts: red8_write puts each
// lane's eight values in rows 0..7; red8_issue loads, for lane l, the eight
// partials 8 (l & 7) .. 8 (l & 7) + 7 of row l >> 3; red8_finish adds them
// and combines the eight lanes of each group by DPP (xor 1, xor 2, mirror
// within 8), so that lane 8k ends with the total of value k.  The raster
// backward reads a step's partials back one evaluated step after it wrote
// them, so that the LDS round trip overlaps that step's arithmetic.  Only
// this wave touches red, and a wave's LDS accesses are performed in order:
// a read issued before the next write sees the earlier partials, with no
// barrier; wave barriers keep the compiler from moving the accesses across
// each other.  All lanes must be active.
__device__ __forceinline__ void red8_write(const float* v, int lane, float* red) {
#pragma unroll
    for (int k = 0; k < 8; ++k) red[k * RED_ROW + lane] = v[k];
}
__device__ __forceinline__ void red8_issue(int lane, const float* red, float4& a, float4& b) {
    const int g = lane >> 3, h = (g & 1) << 2;
    const float* rb = red + g * RED_ROW + (lane & 7) * 8;
    a = *reinterpret_cast<const float4*>(rb + h);
    b = *reinterpret_cast<const float4*>(rb + (h ^ 4));
}
__device__ __forceinline__ float red8_finish(float4 a, float4 b) {
    float u = ((a.x + a.y) + (a.z + a.w)) + ((b.x + b.y) + (b.z + b.w));
    u += dpp<0xB1>(u);     // quad_perm [1,0,3,2]
    u += dpp<0x4E>(u);     // quad_perm [2,3,0,1]
    u += dpp<0x141>(u);    // row_half_mirror: lane ^ 7 within each 8 lanes
    // completed here, with every lane active, so that the move and the add
    // stay one DPP add (sunk into a caller's lane-masked block they are two)
    asm volatile("" : "+v"(u));
    return u;
}

// Forward of the entries [cs, ce) at this lane's pixel, from the state
// (T, C, last) passed in: entries are staged 256 at a time through LDS and
// each wave walks the entries of its quadrant in order.  live: the lanes
// whose pixel still composites (wave-uniform mask).  Every thread of the
// workgroup calls this with the same range (it holds workgroup barriers).
// MASKS (the training forward): each staged entry's quadrant mask is also
// stored for the backward.
template <bool COUNT, bool MASKS = false>
__device__ __forceinline__ void fwd_range(int cs, int ce, uint64_t live, float fx, float fy,
                                          int tx0, int ty0, const Entries& pk, float4* s_geo,
                                          float4* s_col, float4* s_aux, float& T, float& C0,
                                          float& C1, float& C2, int& last, unsigned& ncl,
                                          unsigned& nwit) {
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;
    for (int b = cs; b < ce; b += 256) {
        if (__syncthreads_and(live == 0)) break;
        const int idx = b + tid;
        int mask = 0;
        float bl_raw = 0.f;
        if (idx < ce) {
            const float4* r = pk.rec + 4 * (size_t)pk.ids[idx];
            const float4 g = r[0];
            const float4 c = r[1];
            bl_raw = r[2].x;
            mask = quad_mask(g.x, g.y, g.z, g.w, c.x, c.y, tx0, ty0);
            if (MASKS) pk.qmask[idx] = (uint8_t)mask;
            s_geo[tid] = g;
            s_col[tid] = make_float4(c.x, c.y, fmaxf(c.z + 0.5f, 0.f), fmaxf(c.w + 0.5f, 0.f));
        }
        s_aux[tid] = make_float4(fmaxf(bl_raw + 0.5f, 0.f), __int_as_float(mask), 0.f, 0.f);
        __syncthreads();
        const int nb = min(256, ce - b);
        // this batch's last contributor as the entry's LDS byte offset (a
        // vector register copy per step), turned into the index at the end
        int lqb = INT_MIN;
        for (int ch = 0; ch < nb; ch += 64) {
            const int q = ch + lane;
            uint64_t m = wave_ballot(q < nb && ((__float_as_int(s_aux[q].y) >> w) & 1));
            if (COUNT) nwit += __popcll(m);
            // the chunk's byte offset in a VGPR: each entry's offset is then
            // one vector shift-add from the bit index, shared by its LDS reads
            int chb = ch * (int)sizeof(float4);
            asm volatile("" : "+v"(chb));
            while (m) {
                const int qb = chb + pop_low_bit(m) * (int)sizeof(float4);
                const float4 g = lds_f4(s_geo, qb);
                const float4 c = lds_f4(s_col, qb);
                const float cb = lds_f4(s_aux, qb).x;
                const float dx = g.x - fx, dy = g.y - fy;
                const float sigma = fmaf(0.5f, fmaf(g.z, dx * dx, c.x * dy * dy), g.w * dx * dy);
                const float alpha = fminf(0.999f, c.y * exp_neg_raster(sigma_clamp(sigma)));
                // hit: live && !(alpha < 1/255) (sigma out of range: alpha < 1/255)
                const uint64_t hm = live & mask_uge(alpha, 1.f / 255.f);
                const float nT = T * (1.f - alpha);
                const uint64_t sm = hm & mask_le(nT, 1e-4f);     // stops here
                const uint64_t cm = hm & ~sm;                    // composites
                // the colour reads complete behind the exp above, not inside
                // the update block
                asm volatile("" ::"v"(c.z), "v"(c.w), "v"(cb));
                // only the compositing lanes execute the update (an exec-masked
                // block: no per-lane selects)
                if (lane_of(cm)) {
                    const float vis = alpha * T;
                    C0 = fmaf(c.z, vis, C0);
                    C1 = fmaf(c.w, vis, C1);
                    C2 = fmaf(cb, vis, C2);
                    T = nT;
                    lqb = qb;
                    if (COUNT) ++ncl;
                }
                if (sm) {      // at most once per pixel: the entry before this one
                    if (lane_of(sm)) lqb = qb - (int)sizeof(float4);
                    live &= ~sm;
                }
            }
            if (live == 0) break;
        }
        if (lqb != INT_MIN) last = b + (lqb >> 4);   // sizeof(float4) = 16; -16 gives b - 1
    }
}

template <bool COUNT>
__device__ __forceinline__ void add_work(unsigned long long* work, unsigned ncl, unsigned nwit) {
    if (!COUNT || !work) return;
    unsigned long long* ws = work_slot(work);
    unsigned ncomp = ncl;
    for (int off = 32; off >= 1; off >>= 1) ncomp += __shfl_xor(ncomp, off, 64);
    const int lane = threadIdx.x & 63;
    if (lane == 0 && ncomp) atomicAdd(ws, (unsigned long long)ncomp);
    if (lane == 0 && nwit) atomicAdd(ws + 2, (unsigned long long)nwit);
}

// One work item of the training forward: its chunk's state (chunked tile)
// or the tile's final pixels (tile in one piece).
template <bool COUNT>
__device__ __forceinline__ void fwd_item(int item, int W, int H, int tbx, float bg0, float bg1,
                                         float bg2, const Items& it, const int* tile_bins,
                                         const Entries& pk, float* final_T, int* final_idx,
                                         float* out_img, const ChunkBufs& cb,
                                         unsigned long long* work, float4* s_geo, float4* s_col,
                                         float4* s_aux) {
    int t, K, cs, ce;
    item_range(it, tile_bins, item, t, K, cs, ce);
    const Px px = pixel_of(t, tbx, W, H);
    float fx = (float)px.j, fy = (float)px.i;
    // opaque to the compiler, so that the loop keeps the converted
    // coordinates instead of converting the integers again every step
    asm volatile("" : "+v"(fx), "+v"(fy));
    const int tx0 = (t % tbx) * BLOCK, ty0 = (t / tbx) * BLOCK;

    float T = 1.f, C0 = 0.f, C1 = 0.f, C2 = 0.f;
    int last = cs - 1;
    unsigned ncl = 0;       // pairs composited by this lane
    unsigned nwit = 0;      // entries this wave evaluated (wave-uniform)
    fwd_range<COUNT, true>(cs, ce, wave_ballot(px.inside), fx, fy, tx0, ty0, pk, s_geo, s_col, s_aux, T,
                           C0, C1, C2, last, ncl, nwit);
    add_work<COUNT>(work, ncl, nwit);
    if (!px.inside) return;
    if (K == 1) {
        const size_t pix = (size_t)px.i * W + px.j;
        final_T[pix] = T;
        final_idx[pix] = last;
        out_img[3 * pix + 0] = clamp01(fmaf(bg0, T, C0));
        out_img[3 * pix + 1] = clamp01(fmaf(bg1, T, C1));
        out_img[3 * pix + 2] = clamp01(fmaf(bg2, T, C2));
    } else {
        const size_t o = (size_t)item * TILE_PIX + px.lp;
        cb.cT[o] = T;
        cb.cC[3 * o + 0] = C0;
        cb.cC[3 * o + 1] = C1;
        cb.cC[3 * o + 2] = C2;
        cb.cidx[o] = last;
    }
}

// Chunks 0 .. kmax - 1 of every tile, one item per workgroup.
template <bool COUNT>
__global__ __launch_bounds__(256) void k_raster_fwd(int W, int H, int tbx, float bg0, float bg1,
                                                    float bg2, const Meta* __restrict__ meta,
                                                    Items it,
                                                    const int* __restrict__ tile_bins, Entries pk,
                                                    float* __restrict__ final_T,
                                                    int* __restrict__ final_idx,
                                                    float* __restrict__ out_img, ChunkBufs cb,
                                                    unsigned long long* __restrict__ work,
                                                    int kmax) {
    __shared__ float4 s_geo[256];    // x, y, conic a, b
    __shared__ float4 s_col[256];    // conic c, opacity, clamped r, g
    __shared__ float4 s_aux[256];    // clamped b, mask (bits); 16-byte stride shares the address
    // items in launch order (heaviest size class first)
    if ((int)blockIdx.x >= meta->n_items) return;
    const int item = it.order[blockIdx.x];
    if (it.k[item] >= kmax) return;
    fwd_item<COUNT>(item, W, H, tbx, bg0, bg1, bg2, it, tile_bins, pk, final_T, final_idx, out_img, cb,
             work, s_geo, s_col, s_aux);
}

// Chunks kmin and later of the tiles not marked done, the workgroups striding
// over the items (few items qualify, so a small grid visits them all).
template <bool COUNT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k_raster_fwd_tail(int W, int H, int tbx,
                                                         const Meta* __restrict__ meta, Items it,
                                                         const int* __restrict__ tile_bins,
                                                         Entries pk, ChunkBufs cb,
                                                         unsigned long long* __restrict__ work,
                                                         int kmin, const int* __restrict__ done) {
    __shared__ float4 s_geo[256];
    __shared__ float4 s_col[256];
    __shared__ float4 s_aux[256];
    const int n = meta->n_items;
    for (int item = blockIdx.x; item < n; item += gridDim.x) {
        if (it.k[item] < kmin || done[it.tile[item]]) continue;
        // chunked tiles only (k >= kmin > 0): no final pixels are written
        fwd_item<COUNT>(item, W, H, tbx, 0.f, 0.f, 0.f, it, tile_bins, pk, nullptr, nullptr, nullptr, cb,
                 work, s_geo, s_col, s_aux);
    }
}

// Render-only forward, one workgroup per tile.  A tile rasterised in one
// piece is the forward above.  A chunked tile's chunks are rasterised in
// order, each from T = 1 as rasterize_forward_chunked_kernel does
// (.metal:2633-2741), and folded into the pixel's running state as the merge
// does (.metal:2746-2799): colour += chunk colour * T_running, T_running *=
// chunk T, final index = the chunk's last contributor, until T_running <=
// 1e-4.  A pixel past that cutoff takes no part in later chunks, and the
// workgroup stops once every pixel is past it: the chunks behind the cutoff,
// which only the backward's suffix sums read, are not rasterised.  The
// results are those of the chunk items plus the merge, bit for bit.
// At most 64 VGPRs (8 waves per SIMD; 71 unbounded, 7 waves): 1.5% more
// render FPS at config 3.
template <bool COUNT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k_render_tiles(int W, int H, int tbx, float bg0,
                                                      float bg1, float bg2, Items it,
                                                      const int* __restrict__ tile_bins,
                                                      Entries pk, float* __restrict__ final_T,
                                                      int* __restrict__ final_idx,
                                                      float* __restrict__ out_img,
                                                      unsigned long long* __restrict__ work) {
    __shared__ float4 s_geo[256];
    __shared__ float4 s_col[256];
    __shared__ float4 s_aux[256];
    const int t = it.tile_order[blockIdx.x];   // heaviest size class first
    const int K = it.tile_K[t];
    const int s = tile_bins[2 * t], e = tile_bins[2 * t + 1];
    const Px px = pixel_of(t, tbx, W, H);
    float fx = (float)px.j, fy = (float)px.i;
    asm volatile("" : "+v"(fx), "+v"(fy));
    const int tx0 = (t % tbx) * BLOCK, ty0 = (t / tbx) * BLOCK;
    unsigned ncl = 0, nwit = 0;
    float Tr = 1.f, R0 = 0.f, R1 = 0.f, R2 = 0.f;
    int li;
    if (K == 1) {
        li = s - 1;
        fwd_range<COUNT>(s, e, wave_ballot(px.inside), fx, fy, tx0, ty0, pk, s_geo, s_col, s_aux, Tr, R0,
                  R1, R2, li, ncl, nwit);
    } else {
        li = -1;
        bool done = !px.inside;
        for (int k = 0; k < K; ++k) {
            if (__syncthreads_and(done)) break;
            const int cs = s + k * CHUNK, ce = min(cs + CHUNK, e);
            float T = 1.f, C0 = 0.f, C1 = 0.f, C2 = 0.f;
            int last = cs - 1;
            fwd_range<COUNT>(cs, ce, wave_ballot(!done), fx, fy, tx0, ty0, pk, s_geo, s_col, s_aux, T,
                      C0, C1, C2, last, ncl, nwit);
            if (!done) {
                R0 = fmaf(C0, Tr, R0);
                R1 = fmaf(C1, Tr, R1);
                R2 = fmaf(C2, Tr, R2);
                Tr *= T;
                if (last >= 0) li = last;
                if (Tr <= 1e-4f) done = true;
            }
        }
    }
    add_work<COUNT>(work, ncl, nwit);
    if (!px.inside) return;
    const size_t pix = (size_t)px.i * W + px.j;
    final_T[pix] = Tr;
    final_idx[pix] = li;
    out_img[3 * pix + 0] = clamp01(fmaf(bg0, Tr, R0));
    out_img[3 * pix + 1] = clamp01(fmaf(bg1, Tr, R1));
    out_img[3 * pix + 2] = clamp01(fmaf(bg2, Tr, R2));
}

// Training forward of the chunked tiles in two launches: chunks k < P first;
// then, for a tile with more than P chunks, chunk k >= P only if some pixel
// of the tile still has a nonzero running transmittance after the first P
// (pT_P = T_0 T_1 ... T_{P-1}, multiplied in chunk order as the merge does).
// Where every pixel's pT_P is exactly 0, every later chunk j has pT_j = 0:
// its colour enters the suffix sums as pT_j * C_j = 0, it lies past every
// pixel's merge cutoff (T_running = pT <= 1e-4 before it), so the merge
// gives it index -1 and the backward skips it.  Its state would change no
// output bit, so it is not computed; the merge reads only the first P chunks
// of such a tile.  k_chunk_done marks those tiles.
__global__ __launch_bounds__(256) void k_chunk_done(int W, int H, int tbx,
                                                    const Meta* __restrict__ meta,
                                                    const int* __restrict__ chunked, Items it,
                                                    ChunkBufs cb, int* __restrict__ done) {
    constexpr int P = FWD_P;
    __shared__ int s_any;
    const int nch = meta->n_chunked_tiles;
    for (int b = blockIdx.x; b < nch; b += gridDim.x) {
        const int t = chunked[b];
        const int K = it.tile_K[t], i0 = it.tile_item0[t];
        if (K <= P) {
            if (threadIdx.x == 0) done[t] = 0;
            continue;
        }
        __syncthreads();     // the previous tile's s_any has been read
        if (threadIdx.x == 0) s_any = 0;
        __syncthreads();
        const int lp = threadIdx.x, lx = lp & 15, ly = lp >> 4;
        const int j = (t % tbx) * BLOCK + lx, i = (t / tbx) * BLOCK + ly;
        if (i < H && j < W) {
            // all P loads in flight, then the product in chunk order
            float c[P];
#pragma unroll
            for (int k = 0; k < P; ++k) c[k] = cb.cT[(size_t)(i0 + k) * TILE_PIX + lp];
            float pT = 1.f;
#pragma unroll
            for (int k = 0; k < P; ++k) pT *= c[k];
            if (pT != 0.f) s_any = 1;
        }
        __syncthreads();
        if (threadIdx.x == 0) done[t] = s_any ? 0 : 1;
    }
}

__global__ __launch_bounds__(256) void k_raster_merge(int W, int H, int tbx, float bg0,
                                                      float bg1, float bg2,
                                                      const Meta* __restrict__ meta,
                                                      const int* __restrict__ chunked, Items it,
                                                      float* __restrict__ final_T,
                                                      int* __restrict__ final_idx,
                                                      float* __restrict__ out_img, ChunkBufs cb,
                                                      int with_suffix, const int* __restrict__ done,
                                                      int P) {
    if ((int)blockIdx.x >= meta->n_chunked_tiles) return;
    const int t = chunked[blockIdx.x];
    const int K = it.tile_K[t], i0 = it.tile_item0[t];
    // chunks with state: all K, or the first P of a tile whose later chunks
    // were not computed (they carry pT = 0 and change no output)
    const int Kc = (done && done[t]) ? min(K, P) : K;
    const int lp = threadIdx.x, lx = lp & 15, ly = lp >> 4;
    const int j = (t % tbx) * BLOCK + lx, i = (t / tbx) * BLOCK + ly;
    if (i >= H || j >= W) return;
    float Tr = 1.f, R0 = 0.f, R1 = 0.f, R2 = 0.f;
    int li = -1, cutoff = K;
    // Chunks are folded front to back, stopping at an empty chunk or once
    // T <= 1e-4.  The state of MG chunks is loaded ahead of folding them
    // (every k < K is a valid chunk), so a tile with hundreds of chunks
    // costs one memory round trip per MG chunks instead of two per chunk.
    constexpr int MG = 8;
    bool stop = false;
    for (int k0 = 0; k0 < Kc && !stop; k0 += MG) {
        int cf[MG];
        float cT[MG], c0[MG], c1[MG], c2[MG];
#pragma unroll
        for (int u = 0; u < MG; ++u) {
            const int k = min(k0 + u, Kc - 1);
            const size_t o = (size_t)(i0 + k) * TILE_PIX + lp;
            cf[u] = cb.cidx[o];
            cT[u] = cb.cT[o];
            c0[u] = cb.cC[3 * o + 0];
            c1[u] = cb.cC[3 * o + 1];
            c2[u] = cb.cC[3 * o + 2];
        }
#pragma unroll
        for (int u = 0; u < MG; ++u) {
            const int k = k0 + u;
            if (k >= Kc || (cf[u] < 0 && k > 0)) {
                stop = true;
                break;
            }
            R0 = fmaf(c0[u], Tr, R0);
            R1 = fmaf(c1[u], Tr, R1);
            R2 = fmaf(c2[u], Tr, R2);
            Tr *= cT[u];
            if (cf[u] >= 0) li = cf[u];
            if (Tr <= 1e-4f) {
                cutoff = k + 1;
                stop = true;
                break;
            }
        }
    }
    for (int k = cutoff; k < K; ++k) cb.cidx[(size_t)(i0 + k) * TILE_PIX + lp] = -1;
    const size_t pix = (size_t)i * W + j;
    final_T[pix] = Tr;
    final_idx[pix] = li;
    out_img[3 * pix + 0] = clamp01(fmaf(bg0, Tr, R0));
    out_img[3 * pix + 1] = clamp01(fmaf(bg1, Tr, R1));
    out_img[3 * pix + 2] = clamp01(fmaf(bg2, Tr, R2));
    if (!with_suffix) return;
    // prefix products of T and suffix sums of the chunk colours, each over
    // all chunks with state (the rest add pT * C = 0), with the loads of MG
    // chunks issued ahead of their stores
    float pT = 1.f;
    for (int k0 = 0; k0 < Kc; k0 += MG) {
        float t[MG];
#pragma unroll
        for (int u = 0; u < MG; ++u)
            t[u] = cb.cT[(size_t)(i0 + min(k0 + u, Kc - 1)) * TILE_PIX + lp];
#pragma unroll
        for (int u = 0; u < MG; ++u) {
            if (k0 + u >= Kc) break;
            cb.pT[(size_t)(i0 + k0 + u) * TILE_PIX + lp] = pT;
            pT *= t[u];
        }
    }
    float a0 = 0.f, a1 = 0.f, a2 = 0.f;
    for (int k1 = Kc - 1; k1 >= 0; k1 -= MG) {
        float pp[MG], q0[MG], q1[MG], q2[MG];
#pragma unroll
        for (int u = 0; u < MG; ++u) {
            const size_t o = (size_t)(i0 + max(k1 - u, 0)) * TILE_PIX + lp;
            pp[u] = cb.pT[o];
            q0[u] = cb.cC[3 * o + 0];
            q1[u] = cb.cC[3 * o + 1];
            q2[u] = cb.cC[3 * o + 2];
        }
#pragma unroll
        for (int u = 0; u < MG; ++u) {
            if (k1 - u < 0) break;
            const size_t o = (size_t)(i0 + k1 - u) * TILE_PIX + lp;
            cb.aC[3 * o + 0] = a0;
            cb.aC[3 * o + 1] = a1;
            cb.aC[3 * o + 2] = a2;
            a0 += pp[u] * q0[u];
            a1 += pp[u] * q1[u];
            a2 += pp[u] * q2[u];
        }
    }
}

// COUNT: count the wave's evaluated entries and gradient pairs into work
// (a launch without counters runs the variant that does not count).
template <bool COUNT>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(8))) void k_raster_bwd(int W, int H, int tbx, float bg0, float bg1,
                                                    float bg2, const Meta* __restrict__ meta,
                                                    Items it,
                                                    const int* __restrict__ tile_bins, Entries pk,
                                                    const float* __restrict__ final_T,
                                                    const int* __restrict__ final_idx,
                                                    ChunkBufs cb, const float* __restrict__ v_out,
                                                    float* __restrict__ gacc,
                                                    unsigned long long* __restrict__ work,
                                                    LossFold lf) {
    __shared__ float4 s_geo[256];    // x, y, conic a, b
    __shared__ float4 s_col[256];    // conic c, opacity, clamped r, g
    __shared__ float4 s_aux[256];    // clamped b, opacity - 1, accumulator byte offset, mask
    // per-wave gradient reductions; its first word holds the workgroup's
    // largest final index before the entry loop uses the area
    __shared__ float4 s_red4[4 * 8 * RED_ROW / 4];
    int& s_max = *reinterpret_cast<int*>(s_red4);
    // Workgroup 0 folds the loss partials of the SSIM tiles (in the reduction
    // area) and takes no item: dispatched first, it runs beside the heaviest
    // items instead of at the end of the launch.
    static_assert(sizeof(s_red4) >= 3 * 256 * sizeof(double), "loss fold area");
    if (blockIdx.x == 0) {
        if (lf.part) loss_fold(lf, reinterpret_cast<double*>(s_red4));
        return;
    }
    // items in launch order (heaviest size class first)
    const int bi = (int)blockIdx.x - 1;
    if (bi >= meta->n_items) return;
    const int item = it.order[bi];
    int t, K, cs, ce;
    item_range(it, tile_bins, item, t, K, cs, ce);
    const Px px = pixel_of(t, tbx, W, H);
    const float fx = (float)px.j, fy = (float)px.i;
    const int tid = threadIdx.x, lane = tid & 63, w = tid >> 6;

    float T = 1.f, Tfin = 1.f, B0 = 0.f, B1 = 0.f, B2 = 0.f, vo0 = 0.f, vo1 = 0.f, vo2 = 0.f;
    // bf = cs - 1 for pixels outside the image: no entry passes e_idx <= bf
    int bf = cs - 1;
    unsigned ngrad = 0;     // pairs of this wave that carry a gradient (wave-uniform)
    // After the reductions lane 8k holds the k-th of the eight LDS sums and
    // lane 63 the ninth; each adds it at byte kofs of the gaussian's nine
    // accumulators, all nine in one atomic instruction.
    const bool own = (lane & 7) == 0 || lane == 63;
    const uint32_t kofs = lane == 63 ? 32u : (uint32_t)(lane >> 3) * 4u;
    float* red = reinterpret_cast<float*>(s_red4) + w * 8 * RED_ROW;
    // The gradient sums of an evaluated step are completed during the next
    // one: pend says a step's eight partials are in red, pofs is that
    // gaussian's accumulator byte offset and puo its per-lane opacity term.
    bool pend = false;
    uint32_t pofs = 0u;
    float puo = 0.f;
    unsigned nwit = 0;      // entries this wave evaluated (wave-uniform)
    if (px.inside) {
        const size_t pix = (size_t)px.i * W + px.j;
        Tfin = final_T[pix];
        vo0 = v_out[3 * pix + 0];
        vo1 = v_out[3 * pix + 1];
        vo2 = v_out[3 * pix + 2];
        if (K == 1) {
            T = Tfin;
            bf = final_idx[pix];
        } else {
            const size_t o = (size_t)item * TILE_PIX + px.lp;
            T = cb.pT[o] * cb.cT[o];
            B0 = cb.aC[3 * o + 0];
            B1 = cb.aC[3 * o + 1];
            B2 = cb.aC[3 * o + 2];
            bf = cb.cidx[o];
        }
    }
    // The colour terms of v_alpha enter only as sum_k v_out_k (...)_k:
    // D = sum_k v_out_k B_k (accumulated colour behind) and TB = sum_k
    // v_out_k T_final bg_k are carried instead of the three channels.
    // E = D + TB, the two carried together: D changes, TB does not
    const float TB = fmaf(Tfin * bg2, vo2, fmaf(Tfin * bg1, vo1, (Tfin * bg0) * vo0));
    float E = fmaf(B2, vo2, fmaf(B1, vo1, B0 * vo0)) + TB;
    // wave-uniform (readfirstlane): the entry loop indexes then live in scalar registers
    const int wave_bf = __builtin_amdgcn_readfirstlane(wave_max_i(bf));
    if (tid == 0) s_max = cs - 1;
    __syncthreads();
    if (lane == 0) atomicMax(&s_max, wave_bf);
    __syncthreads();
    const int hi = min(ce - 1, s_max);

    for (int top = hi; top >= cs; top -= 256) {
        __syncthreads();
        const int idx = top - tid;
        // the entry's quadrant mask from the forward; an entry that reaches
        // no quadrant is not gathered
        const int mask = idx >= cs ? (int)pk.qmask[idx] : 0;
        if (mask) {
            const int gid = (int)pk.ids[idx];
            const float4* r = pk.rec + 4 * (size_t)gid;
            const float4 g = r[0];
            float4 c = r[1];
            const float braw = r[2].x;
            s_geo[tid] = g;
            s_col[tid] = make_float4(c.x, c.y, fmaxf(c.z + 0.5f, 0.f), fmaxf(c.w + 0.5f, 0.f));
            // z: byte offset of the gaussian's accumulators (N * 36 < 2^31)
            s_aux[tid] = make_float4(fmaxf(braw + 0.5f, 0.f), c.y - 1.f, __int_as_float(gid * 36),
                                     __int_as_float(mask));
        } else {
            s_aux[tid].w = __int_as_float(0);
        }
        __syncthreads();
        const int nb = min(256, top - cs + 1);
        const int q0 = max(0, top - wave_bf);
        const int qlo = top - bf;      // this pixel takes entries qq >= qlo (e_idx <= bf)
        // in bytes of the LDS arrays, so that the step's index test compares
        // two VGPRs; clamped to [0, 256] first, which keeps the test's outcome
        // for every qq in [0, 256) (bf = -1 of a cut-off chunk makes qlo a
        // global entry index, too large to scale)
        const int qlob = min(max(qlo, 0), 256) * (int)sizeof(float4);
        for (int ch = (q0 / 64) * 64; ch < nb; ch += 64) {
            const int q = ch + lane;
            uint64_t m = wave_ballot(q >= q0 && q < nb &&
                                     ((__float_as_int(s_aux[q].w) >> w) & 1));
            if (COUNT) nwit += __popcll(m);
            // the chunk's byte offset in a VGPR: each entry's offset is then
            // one vector shift-add from the bit index, shared by its LDS reads
            int chb = ch * (int)sizeof(float4);
            asm volatile("" : "+v"(chb));
            while (m) {
                const int qb = chb + pop_low_bit(m) * (int)sizeof(float4);
                const float4 g = lds_f4(s_geo, qb);
                const float4 c = lds_f4(s_col, qb);
                const float4 x = lds_f4(s_aux, qb);
                const float dx = g.x - fx, dy = g.y - fy;
                const float sigma = fmaf(0.5f, fmaf(g.z, dx * dx, c.x * dy * dy), g.w * dx * dy);
                const float alpha = fminf(0.999f, c.y * exp_neg_raster(sigma_clamp(sigma)));
                // valid: qq >= qlo && !(alpha < 1/255) (sigma out of range: alpha < 1/255)
                const uint64_t vmask = mask_ge_i(qb, qlob) & mask_uge(alpha, 1.f / 255.f);
                if (vmask == 0) continue;
                // the previous evaluated step's partials (written a step ago):
                // read now (unused when there is none), summed below, after
                // this step's arithmetic
                float4 pa, pb;
                __builtin_amdgcn_wave_barrier();
                red8_issue(lane, red, pa, pb);
                // Branch-free per lane: lanes without a gradient run the same
                // steps with alpha = 0, which leaves their state as it is
                // (1 / (1 - 0) = 1 exactly, so Tn = T; fac = 0, so E is
                // unchanged) and makes every term they contribute zero.
                const uint64_t gmask = vmask & mask_lt(alpha, 0.999f);
                const float ag = lane_of(gmask) ? alpha : 0.f;
                if (COUNT) ngrad += (unsigned)__popcll(gmask);
                const float r0 = c.z, r1 = c.w, r2 = x.x;   // max(raw + 0.5, 0)
                // hardware reciprocal (1 ulp, exact at 1): the backward is
                // compared with a tolerance
                const float ra = __builtin_amdgcn_rcpf(1.f - ag);
                const float Tn = T * ra;
                const float fac = ag * Tn;
                // v_alpha = sum_k (r_k Tn - (B_k + T_final bg_k) ra) v_out_k
                const float RV = fmaf(r2, vo2, fmaf(r1, vo1, r0 * vo0));
                const float v_alpha = fmaf(Tn, RV, -ra * E);
                E = fmaf(fac, RV, E);
                T = Tn;
                // v_sigma: zero (signed) on the lanes without a gradient
                const float vsg = -ag * v_alpha;
                // v_xy = v_sigma (a dx + b dy, b dx + c dy) and v_conic =
                // v_sigma / 2 (dx^2, dx dy, dy^2) are linear in the moments
                // below with the gaussian's own conic, the same in every
                // tile: the moments are summed, the projection backward
                // applies the conic once per gaussian.
                const float w0 = vsg * dx, w1 = vsg * dy;
                float v[8];
                v[0] = w0;
                v[1] = w1;
                v[2] = w0 * dx;
                v[3] = w0 * dy;
                v[4] = w1 * dy;
                v[5] = fac * vo0;
                v[6] = fac * vo1;
                v[7] = fac * vo2;
                // The previous step's sums follow this step's arithmetic
                // (the empty asm keeps them there, so that the loads' latency
                // is spent on it); the opacity (logit) term -v_sigma (1 - o)
                // goes to lane 63 of them (lanes 60..62 are no owners).  v_rgb
                // of a channel whose raw colour + 0.5 < 0 is dropped by its
                // consumers (the mask is per gaussian, not per pixel).
                asm volatile("" : "+v"(pa.x), "+v"(pa.y), "+v"(pa.z), "+v"(pa.w), "+v"(pb.x),
                             "+v"(pb.y), "+v"(pb.z), "+v"(pb.w) : "v"(v[7]), "v"(v[4]));
                if (pend) {
                    const float s = wave_sum_into_lane63(puo, red8_finish(pa, pb));
                    float* ap = reinterpret_cast<float*>(reinterpret_cast<char*>(gacc) + (pofs + kofs));
                    if (own) atomicAdd(ap, s);
                }
                __builtin_amdgcn_wave_barrier();
                red8_write(v, lane, red);
                __builtin_amdgcn_wave_barrier();
                pend = true;
                pofs = (uint32_t)__builtin_amdgcn_readfirstlane(__float_as_int(x.z));
                puo = vsg * x.y;
            }
        }
    }
    if (pend) {   // the last evaluated step's sums
        __builtin_amdgcn_wave_barrier();
        float4 pa, pb;
        red8_issue(lane, red, pa, pb);
        const float s = wave_sum_into_lane63(puo, red8_finish(pa, pb));
        float* ap = reinterpret_cast<float*>(reinterpret_cast<char*>(gacc) + (pofs + kofs));
        if (own) atomicAdd(ap, s);
    }
    if (COUNT && work) {
        unsigned long long* ws = work_slot(work);
        if (lane == 0 && ngrad) atomicAdd(ws + 1, (unsigned long long)ngrad);
        if (lane == 0 && nwit) atomicAdd(ws + 3, (unsigned long long)nwit);
    }
}

// Algorithmic work of the most recent forward (+ backward): one thread per
// pixel walks its item's entries in the order of the per-pixel loops of the
// reference kernels, without quadrant culling or lockstep, and counts
// (pixel, entry) pairs: forward tested / sigma in range / composited,
// backward tested / sigma in range / carrying a gradient.  The counts
// define the algorithmic flops of the roofline; they change no state.
__global__ __launch_bounds__(256) void k_raster_work(int W, int H, int tbx,
                                                     const Meta* __restrict__ meta, Items it,
                                                     const int* __restrict__ tile_bins, Entries pk,
                                                     const int* __restrict__ final_idx,
                                                     ChunkBufs cb,
                                                     unsigned long long* __restrict__ out) {
    const int item = blockIdx.x;
    if (item >= meta->n_items) return;
    int t, K, cs, ce;
    item_range(it, tile_bins, item, t, K, cs, ce);
    const Px px = pixel_of(t, tbx, W, H);
    unsigned n[6] = {0u, 0u, 0u, 0u, 0u, 0u};
    if (px.inside) {
        const float fx = (float)px.j, fy = (float)px.i;
        float T = 1.f;
        for (int i = cs; i < ce; ++i) {
            ++n[0];
            const float4* r = pk.rec + 4 * (size_t)pk.ids[i];
            const float4 g = r[0];
            const float4 c = r[1];
            const float dx = g.x - fx, dy = g.y - fy;
            const float sigma = fmaf(0.5f, fmaf(g.z, dx * dx, c.x * dy * dy), g.w * dx * dy);
            if (!(sigma < 0.f || sigma >= 5.55f)) ++n[1];
            const float alpha = fminf(0.999f, c.y * exp_neg_raster(sigma_clamp(sigma)));
            if (alpha < 1.f / 255.f) continue;
            const float nT = T * (1.f - alpha);
            if (nT <= 1e-4f) break;
            ++n[2];
            T = nT;
        }
        const int bf = K == 1 ? final_idx[(size_t)px.i * W + px.j]
                              : cb.cidx[(size_t)item * TILE_PIX + px.lp];
        for (int i = min(bf, ce - 1); i >= cs; --i) {
            ++n[3];
            const float4* r = pk.rec + 4 * (size_t)pk.ids[i];
            const float4 g = r[0];
            const float4 c = r[1];
            const float dx = g.x - fx, dy = g.y - fy;
            const float sigma = fmaf(0.5f, fmaf(g.z, dx * dx, c.x * dy * dy), g.w * dx * dy);
            if (!(sigma < 0.f || sigma >= 5.55f)) ++n[4];
            const float alpha = fminf(0.999f, c.y * exp_neg_raster(sigma_clamp(sigma)));
            if (alpha < 1.f / 255.f || !(alpha < 0.999f)) continue;
            ++n[5];
        }
    }
#pragma unroll
    for (int k = 0; k < 6; ++k) {
        unsigned long long v = n[k];
        for (int off = 32; off >= 1; off >>= 1) v += __shfl_xor(v, off, 64);
        if ((threadIdx.x & 63) == 0) atomicAdd(&out[k], v);
    }
}

}  // namespace

void launch_raster_work(hipStream_t s, const CamParams& p, int64_t max_items, const Meta* meta,
                        Items it, const int* tile_bins, Entries pk, const int* final_idx,
                        ChunkBufs cb, unsigned long long* out) {
    if (max_items <= 0) return;
    hipLaunchKernelGGL(k_raster_work, dim3((unsigned)max_items), dim3(256), 0, s, p.W, p.H, p.tbx,
                       meta, it, tile_bins, pk, final_idx, cb, out);
}

void launch_raster_fwd(hipStream_t s, const CamParams& p, int64_t max_items, const Meta* meta,
                       Items it, const int* tile_bins, Entries pk, float* final_T, int* final_idx,
                       float* out_img, ChunkBufs cb, unsigned long long* work, const int* chunked,
                       int* done) {
    if (max_items <= 0) return;
    // chunks 0 .. FWD_P - 1 of every tile, then the tiles' later chunks that
    // k_chunk_done does not mark as past an all-zero running transmittance
    // the counting variants only when pair counters are asked for
    if (work)
        hipLaunchKernelGGL(k_raster_fwd<true>, dim3((unsigned)max_items), dim3(256), 0, s, p.W, p.H,
                           p.tbx, p.bg[0], p.bg[1], p.bg[2], meta, it, tile_bins, pk, final_T,
                           final_idx, out_img, cb, work, FWD_P);
    else
        hipLaunchKernelGGL(k_raster_fwd<false>, dim3((unsigned)max_items), dim3(256), 0, s, p.W, p.H,
                           p.tbx, p.bg[0], p.bg[1], p.bg[2], meta, it, tile_bins, pk, final_T,
                           final_idx, out_img, cb, work, FWD_P);
    const int T = p.tbx * p.tby;
    hipLaunchKernelGGL(k_chunk_done, dim3((unsigned)std::min(T, 256)), dim3(256), 0, s, p.W, p.H,
                       p.tbx, meta, chunked, it, cb, done);
    const dim3 tg((unsigned)std::min<int64_t>(max_items, 1024));
    if (work)
        hipLaunchKernelGGL(k_raster_fwd_tail<true>, tg, dim3(256), 0, s, p.W, p.H, p.tbx, meta, it,
                           tile_bins, pk, cb, work, FWD_P, (const int*)done);
    else
        hipLaunchKernelGGL(k_raster_fwd_tail<false>, tg, dim3(256), 0, s, p.W, p.H, p.tbx, meta, it,
                           tile_bins, pk, cb, work, FWD_P, (const int*)done);
}

void launch_render_tiles(hipStream_t s, const CamParams& p, Items it, const int* tile_bins,
                         Entries pk, float* final_T, int* final_idx, float* out_img,
                         unsigned long long* work) {
    const int T = p.tbx * p.tby;
    if (T <= 0) return;
    if (work)
        hipLaunchKernelGGL(k_render_tiles<true>, dim3((unsigned)T), dim3(256), 0, s, p.W, p.H, p.tbx,
                           p.bg[0], p.bg[1], p.bg[2], it, tile_bins, pk, final_T, final_idx, out_img,
                           work);
    else
        hipLaunchKernelGGL(k_render_tiles<false>, dim3((unsigned)T), dim3(256), 0, s, p.W, p.H, p.tbx,
                           p.bg[0], p.bg[1], p.bg[2], it, tile_bins, pk, final_T, final_idx, out_img,
                           work);
}

void launch_raster_merge(hipStream_t s, const CamParams& p, const Meta* meta, const int* chunked,
                         Items it, float* final_T, int* final_idx, float* out_img, ChunkBufs cb,
                         bool with_suffix, const int* done) {
    const int T = p.tbx * p.tby;
    hipLaunchKernelGGL(k_raster_merge, dim3(T), dim3(256), 0, s, p.W, p.H, p.tbx, p.bg[0], p.bg[1],
                       p.bg[2], meta, chunked, it, final_T, final_idx, out_img, cb,
                       with_suffix ? 1 : 0, done, FWD_P);
}

void launch_raster_bwd(hipStream_t s, const CamParams& p, int64_t max_items, const Meta* meta,
                       Items it, const int* tile_bins, Entries pk, const float* final_T,
                       const int* final_idx, ChunkBufs cb, const float* v_out, float* gacc,
                       unsigned long long* work, const LossFold& lf) {
    // workgroup 0 folds the loss, the others take the items
    const int64_t g = std::max<int64_t>(max_items, 0) + 1;
    if (work)
        hipLaunchKernelGGL(k_raster_bwd<true>, dim3((unsigned)g), dim3(256), 0, s, p.W, p.H,
                           p.tbx, p.bg[0], p.bg[1], p.bg[2], meta, it, tile_bins, pk, final_T,
                           final_idx, cb, v_out, gacc, work, lf);
    else
        hipLaunchKernelGGL(k_raster_bwd<false>, dim3((unsigned)g), dim3(256), 0, s, p.W, p.H,
                           p.tbx, p.bg[0], p.bg[1], p.bg[2], meta, it, tile_bins, pk, final_T,
                           final_idx, cb, v_out, gacc, work, lf);
}

}  // namespace msp
