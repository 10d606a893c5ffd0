// kernels.hpp — launch interface between the C-ABI orchestration (context.hip)
// and the kernel translation units.  Host-callable launchers only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msp {

// Camera / render constants shared by projection, binning and raster.
struct CamParams {
    int N;
    float glob_scale;
    float vm[16];
    float pm[16];
    float fx, fy, cx, cy;
    int W, H;
    int tbx, tby;
    float clip;
    int degree;          // SH degree of the stored coefficients
    int dtu;             // degrees_to_use (clamped to degree)
    int rest_per;        // floats per gaussian in features_rest
    float cam[3];
    float bg[3];
};

// Per-gaussian outputs of the projection (internal layout).  One 64-byte
// record per gaussian so that the per-intersection gathers touch one cache
// line:  rec[4g+0] = (x, y, conic_a, conic_b)
//        rec[4g+1] = (conic_c, sigmoid(opacity), r, g)   raw SH colour
//        rec[4g+2] = (b, extent_x, extent_y, depth)
//        rec[4g+3] = (view direction normalize(p - cam), 0)
struct GaussOut {
    float4* rec;
    int* radii;
    int* radii_out;      // optional second copy of the radii (the caller's), or null
    int* tiles_hit;
    uint2* rect;         // tile rectangle: (x0 | y0 << 16, x1 | y1 << 16), 0 when culled
};

// Tile-sorted entries: ids[i] is the gaussian of entry i; the rasteriser
// gathers its projection record rec[4 id .. 4 id + 2] (one 64-byte line).
struct Entries {
    const uint32_t* ids;
    const float4* rec;
    // One byte per entry: the 4-bit quadrant mask that the training
    // forward computes for every entry it stages, read back by the backward
    // (which walks only entries up to the last contributor, all of them
    // staged by the forward) instead of computing it again.
    uint8_t* qmask;
};

// Work items of the rasteriser: item i covers chunk item_k[i] of tile item_tile[i].
struct Items {
    int* tile;
    int* k;
    int* tile_K;         // chunks per tile
    int* tile_item0;     // first item of each tile
    int* order;          // items, heaviest size class first (the raster launch order)
    int* tile_order;     // tiles, heaviest size class first (the render launch order)
    int* cls;            // 4 x 32 counters of the size classes (items, tiles; counts, fills)
};

// Host-visible summary written by the tile scan.
struct Meta {
    int64_t total_isect;
    int32_t max_count;
    int32_t n_items;
    int32_t n_chunked_tiles;   // tiles with more than one chunk
    int32_t n_large;           // unused (0)
    int32_t n_huge;            // unused (0)
    int32_t pad;
};

// Tile lists written by the tile scan (order within a list is arbitrary).
struct TileLists {
    int* chunked;
    int* large;
    int* huge;
};


// Per-pixel chunk state, indexed by item * 256 + local pixel.
struct ChunkBufs {
    float* cT;
    float* cC;           // x3
    int* cidx;
    float* pT;
    float* aC;           // x3
};

// Intersection-total counters of the projection: ISECT_SLOTS u64 counter
// pairs ISECT_STRIDE u64 apart (one 128-byte line each); the first of a pair
// counts (gaussian, tile) pairs, the second (gaussian, super-tile)
// references; the totals are the sums over the slots, formed by the first
// kernel of the depth sort (SlotSum) for the host.
constexpr int ISECT_SLOTS = 64;
constexpr int ISECT_STRIDE = 16;
constexpr size_t ISECT_BYTES = (size_t)ISECT_SLOTS * ISECT_STRIDE * 8;
void launch_project_fwd(hipStream_t s, const CamParams& p, const float* means,
                        const float* scales, const float* quats, const float* f_dc,
                        const float* f_rest, const float* opac_logits, GaussOut go,
                        uint32_t* dkey, uint32_t* dval, float* gacc,
                        unsigned long long* total_isect);

// Scans and radix sort (radix.hip).  With `gather` the scanned values are
// in[gather[i]], also stored to gathered[i] (n ints).
constexpr int SCAN_BLOCK = 1024;   // elements per scan block
int64_t scan_block_count(int64_t n);
// Above this many 1024-element blocks a scan runs its block totals through a
// one-workgroup scan; up to it, each block adds up the totals before it.
constexpr int SCAN_DIRECT_BLOCKS = 2048;
// The first half of a scan: the totals of the 1024-element blocks of in,
// turned into exclusive block offsets when there are more than
// SCAN_DIRECT_BLOCKS blocks (the consumer then reads tot[b] directly).
void launch_block_totals(hipStream_t s, const int* in, int64_t n, int* tot);
void launch_scan_i32(hipStream_t s, const int* in, int* out, int64_t n, int* block_tot);
void launch_exclusive_scan_i32(hipStream_t s, const int* in, int* out, int64_t n, int* block_tot,
                               const uint32_t* gather = nullptr, int* gathered = nullptr);
int64_t radix_temp_ints(int64_t n);
// Optional side job of a sort's first kernel, for the depth order: its
// workgroup 0 sums the projection's ISECT_SLOTS counter pairs and writes the
// two totals to *out (coherent host memory) as one 64-bit word,
// totals_word(I, R), which the host polls.
struct SlotSum {
    const unsigned long long* slots;
    unsigned long long* out;
};
// Bit 63 set (so that a zeroed word means "not yet"), the intersection total
// in bits 31..61 and the reference total in bits 0..30, each saturated at
// 2^31 - 1.
__host__ __device__ inline unsigned long long totals_word(unsigned long long i, unsigned long long r) {
    const unsigned long long cap = 0x7FFFFFFFull;
    return (1ull << 63) | ((i < cap ? i : cap) << 31) | (r < cap ? r : cap);
}
// Optional epilogue of a sort's last pass, for the depth order: output
// position i also gets rs[i] = rect[value] and cnt[i] = the super-tile count
// of that rectangle (both zero for the culled key 0xFFFFFFFF, and at the
// positions of a culling sort's culled tail).
struct RectGather {
    const uint2* rect;
    uint2* rs;
    int* cnt;
};
bool launch_radix_sort(hipStream_t s, uint32_t* k0, uint32_t* v0, uint32_t* k1, uint32_t* v1,
                       int64_t n, int bits, int* temp, const RectGather* rg = nullptr,
                       const SlotSum* ss = nullptr, int* edge0 = nullptr, int* edge1 = nullptr,
                       bool cull = false);

// Super-tiles: SUPER x SUPER tiles of the tile grid.  A gaussian's tile
// rectangle is cut into one reference per super-tile it overlaps; the
// references are sorted by super-tile and each super-tile's references are
// processed in segments of SEG_REFS.
constexpr int SUPER = 16;
constexpr int SEG_REFS = 1024;
inline int super_tiles(int tbx, int tby) {
    return ((tbx + SUPER - 1) / SUPER) * ((tby + SUPER - 1) / SUPER);
}
// Upper bound of the segments of R references over S super-tiles.
inline int64_t segments_bound(int64_t R, int64_t S) { return R / SEG_REFS + S + 1; }
// Super-tiles overlapped by the non-empty tile rectangle [x0, x1) x [y0, y1).
__host__ __device__ inline int super_span(int x0, int y0, int x1, int y1) {
    return ((x1 - 1) / SUPER - x0 / SUPER + 1) * ((y1 - 1) / SUPER - y0 / SUPER + 1);
}

// Binning (binning.hip).  The projection adds the intersection and
// reference totals to the counters above (needed on the host before
// launch_tile_lists); launch_depth_order orders the gaussians by depth,
// gathers their tile rectangles in that order (rect_sorted), with their
// super-tile counts (rcount) and the counts' 1024-block totals (rtot, as
// launch_block_totals leaves them), from which launch_tile_lists' reference
// emission takes each gaussian's first reference slot.
void launch_depth_order(hipStream_t s, int N, uint32_t* dkey, uint32_t* dval, uint32_t* dkey2,
                        uint32_t* dval2, int* radix_temp, const uint2* rect, uint2* rect_sorted,
                        int* rcount, int* rtot, const SlotSum* ss, uint32_t** order_out);

// Scratch of launch_tile_lists for R references, S super-tiles, NS =
// segments_bound(R, S) segments and T tiles.
struct RefBufs {
    uint32_t *key, *val, *key2, *val2;   // R each: references, ping-pong
    int* radix_temp;                     // radix_temp_ints(R)
    int* st_r0;                          // S: reference range of each super-tile;
    int* st_r1;                          //    S; both zero between calls
    int* sstart;                         // S + 1: first segment of each super-tile
    int4* seg;                           // NS: (super-tile, first reference, end reference)
    int* hist;                           // NS * 256: pairs per local tile and segment
    int* tcount;                         // T: pairs per tile
};
// Writes the tile-sorted gaussian ids (I of them) to ids, tile_bins, the
// work items and the summary in meta.
void launch_tile_lists(hipStream_t s, const CamParams& p, int64_t I, int64_t R,
                       const uint32_t* order, const int* rtot,
                       const uint2* rect_sorted, RefBufs rb,
                       uint32_t* ids, int* tscan, int* tile_bins, Items it, TileLists tl,
                       Meta* meta, unsigned long long* isect);
// Ints of the tile scan's scratch (tscan) for T tiles.
inline int64_t tile_scan_ints(int64_t T) { return 3 * ((T + 1023) / 1024) + 8; }

// Raster pair counters: WORK_SLOTS sets of four u64 counters, each set in
// its own 128-byte line (WORK_SLOT_U64 apart); totals are the sums over sets.
constexpr int WORK_SLOTS = 64;
constexpr int WORK_SLOT_U64 = 16;

// Upper bound of the number of (tile, chunk) work items for I intersections.
inline int64_t items_bound(int64_t T, int64_t I) { return T + I / 512 + I / 2048 + 1; }

// Rasterisation (raster.hip); grids are sized by items_bound / T and the
// kernels read the exact counts from meta.  A non-null `work` (the counter
// sets above) makes the forward add its composited (pixel, entry) pairs to
// counter 0 and its wave-wide entry steps to counter 2, the backward its
// pairs that carry a gradient to counter 1 and its wave-wide entry steps to
// counter 3.
// Training forward: every work item's chunk state (chunked tiles) or final
// pixels (tiles in one piece).  A chunked tile with more than FWD_P chunks
// whose running transmittance is exactly 0 at every pixel after its first
// FWD_P chunks is marked in done[tile] (T ints) and its later chunks, which
// change no output, are not computed; chunked is the tile scan's list.
constexpr int FWD_P = 16;
void launch_raster_fwd(hipStream_t s, const CamParams& p, int64_t max_items, const Meta* meta,
                       Items it, const int* tile_bins, Entries pk, float* final_T, int* final_idx,
                       float* out_img, ChunkBufs cb, unsigned long long* work, const int* chunked,
                       int* done);
// Render-only forward, one workgroup per tile (chunked tiles rasterised chunk
// by chunk up to the merge cutoff); writes the final image, T and index.
void launch_render_tiles(hipStream_t s, const CamParams& p, Items it, const int* tile_bins,
                         Entries pk, float* final_T, int* final_idx, float* out_img,
                         unsigned long long* work);
void launch_raster_merge(hipStream_t s, const CamParams& p, const Meta* meta, const int* chunked,
                         Items it, float* final_T, int* final_idx, float* out_img, ChunkBufs cb,
                         bool with_suffix, const int* done);
// Fold of the SSIM tiles' loss partials into the loss sum, done by one
// workgroup of a later kernel (the raster backward's first): in float64, in a
// fixed order (thread t adds parts t, t + blockDim.x, ... in order, then a
// tree over the threads), stored to out (which may be coherent host memory
// that the host reads without a stream sync: a system-scope store makes the
// value visible there).  s: 3 x blockDim.x doubles of LDS; blockDim.x a power
// of two.  Every thread of the workgroup calls it.
struct LossFold {
    const float* part;
    int nparts;
    float w;
    float* out;
};
__device__ inline void loss_fold(const LossFold& lf, double* s) {
    const int t = threadIdx.x, nt = blockDim.x;
    double a = 0.0, b = 0.0, n = 0.0;
    for (int i = t; i < lf.nparts; i += nt) {
        a += lf.part[3 * i];
        b += lf.part[3 * i + 1];
        n += lf.part[3 * i + 2];
    }
    s[t] = a;
    s[nt + t] = b;
    s[2 * nt + t] = n;
    __syncthreads();
    for (int off = nt / 2; off > 0; off >>= 1) {
        if (t < off)
            for (int k = 0; k < 3; ++k) s[k * nt + t] += s[k * nt + t + off];
        __syncthreads();
    }
    if (t == 0) {
        const double w = lf.w;
        __hip_atomic_store(lf.out, (float)(w * s[2 * nt] - (w / 3.0) * s[0] + ((1.0 - w) / 3.0) * s[nt]),
                           __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
    }
    __syncthreads();
}
// Workgroup 0 of the launch folds the loss when lf.part is set (loss_fold);
// the items take workgroups 1 ...
void launch_raster_bwd(hipStream_t s, const CamParams& p, int64_t max_items, const Meta* meta,
                       Items it, const int* tile_bins, Entries pk, const float* final_T,
                       const int* final_idx, ChunkBufs cb, const float* v_out, float* gacc,
                       unsigned long long* work, const LossFold& lf);
// Adds the six pair counts of the most recent forward/backward into out[6].
void launch_raster_work(hipStream_t s, const CamParams& p, int64_t max_items, const Meta* meta,
                        Items it, const int* tile_bins, Entries pk, const int* final_idx,
                        ChunkBufs cb, unsigned long long* out);

// The loss: SSIM + L1 forward and backward per 32x32 tile; writes the loss
// gradient image and one partial (sum SSIM, sum L1, pixels) per tile, and
// returns the number of partials.
int launch_ssim(hipStream_t s, int H, int W, const float* img, const float* gt, float w,
                float inv_n, float* v_rendered, float* loss_part);



struct AdamHP {
    float step[6];
    float inv_bc2[6];   // 1 / sqrt(1 - beta2^t) per parameter group
    float b1, b2, eps;
};

void launch_sh_rest_adam(hipStream_t s, const CamParams& p, const float4* rec, const int* radii,
                         const float* gacc, float* f_rest, float* m, float* v, const AdamHP& hp);
void launch_proj_bwd_adam(hipStream_t s, const CamParams& p, float* const params[6],
                          float* const m[6], float* const v[6], const AdamHP& hp,
                          GaussOut go, const float* gacc, float* vis, float* gnorm,
                          float* max2d, float inv_max_dim, float* v_mean_out,
                          float* v_scale_out, float* v_quat_out);

// Densification.
struct DensifyHP {
    int N;
    float grad_thresh, size_thresh, screen_thresh;
    int check_screen;
    float cull_alpha, cull_scale, cull_screen;
    int check_huge;
    float half_max_dim;
    int fr;
};
void launch_randn(hipStream_t s, float* dst, int64_t n, uint64_t seed);
void launch_clamp_max(hipStream_t s, float* p, int64_t n, float hi);
// Classify, split / duplicate append, cull flags and keep scan; writes
// counts_out[0] = rows after appending, counts_out[1] = rows kept.
void launch_densify(hipStream_t s, const DensifyHP& hp, const float* gnorm, const float* vis,
                    const float* max2d, float* const bufs[6], float* const m[6],
                    float* const v[6], const float* rnd, int* split, int* dup, int* sp,
                    int* dp, int* keep, int* kp, int* block_tot, int* counts_out);
// Stable compaction of the cnt kept rows (of `rows` rows) of all 18 buffers
// through a workspace of densify_workspace_floats(cnt, fr) floats.
int64_t densify_workspace_floats(int cnt, int fr);
void launch_densify_compact(hipStream_t s, int rows, int cnt, int fr, float* const bufs[6],
                            float* const m[6], float* const v[6], const int* keep,
                            const int* kp, int* src_of, float* ws);

// Evaluation images: RGBA8 display conversion and PSNR / L1 / SSIM.
struct EvalWindow {
    int ws, pad;      // taps (odd, <= 11) and ws / 2
    float w[11];      // normalised Gaussian taps, computed on the host in fp32
};
int64_t eval_partial_count(int H, int W);
void launch_to_rgba8(hipStream_t s, const float* img, int64_t n, uint32_t* rgba);
void launch_image_metrics(hipStream_t s, const float* img, const float* gt, int H, int W,
                          const EvalWindow& win, double* part, double* out3);

// Nearest-neighbour scales of a point cloud (uniform grid).
struct KnnGrid {
    float lo[3];
    float h, inv_h;     // cell edge and its reciprocal
    float margin;       // bound on the cell-assignment rounding, in distance
    int dim[3];
};
void launch_knn_cells(hipStream_t s, int64_t n, const float* xyz, const KnnGrid& g,
                      uint32_t* key, uint32_t* val);
void launch_knn_search(hipStream_t s, int64_t n, const float* xyz, const KnnGrid& g,
                       const uint32_t* order, const int* cstart, const int* cend,
                       float* mean_dist);
// Run edges of sorted keys (sorted_keys 16-byte aligned): start[k] / end[k] =
// first / one past the last position of key k; keys absent keep their value.
void launch_run_edges(hipStream_t s, int64_t n, const uint32_t* sorted_keys, int* start, int* end);

// Target images: area resize and Brown-Conrady undistortion (image.hip).
struct UndistortParams {
    float fx, fy, cx, cy;
    float k1, k2, p1, p2, k3;
    int roi_x, roi_y, roi_w, roi_h;   // crop rectangle of the undistorted image
};
void undistort_roi(int w, int h, UndistortParams& u);   // host: fills roi_*
void launch_resize_area(hipStream_t s, const float* src, int sw, int sh, float* dst, int dw,
                        int dh);
void launch_undistort(hipStream_t s, const float* src, int w, int h, const UndistortParams& u,
                      float* dst);

}  // namespace msp
