// context.hip — the C ABI (include/msplat_hip.h): context, buffer cache and
// the stage order of one render / train step on a single HIP stream.
//
// Replaces MetalContext + FusedTensorCache + forward_pipeline /
// msplat_render / msplat_train_step / msplat_densify
// (msplat_metal.mm:173-288, 348-454, 462-769, 771-1330, 1337-1592).
// Stage order (.mm:1295-1326): zero -> project -> scan/scatter/sort ->
// raster forward (+merge) -> SSIM fwd/bwd -> raster backward ->
// projection backward + Adam + grad stats.  Intermediate buffers live in a
// grow-only cache owned by the context.  One host synchronisation per step:
// after the depth sort the host reads the intersection total (8 bytes) to size
// the intersection buffers exactly, instead of the reference's fixed 16N
// capacity and 2048-per-tile bins; every later grid is an upper bound whose
// surplus workgroups exit on the exact counts the GPU wrote.
#include "../../include/msplat_hip.h"
#include "common.hpp"
#include "kernels.hpp"

#include <algorithm>
#include <chrono>
#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <string>
#include <vector>

// Workspace of msplat_hip_image_metrics_noalloc: the per-workgroup fp64
// partials of the metric kernels (three per 64x16 output tile, at most
// kNoallocEvalParts tiles) followed by the three folded sums.  One copy per
// GPU for the life of the process (1.5 MiB).  Host code uses the address that
// hipGetSymbolAddress returns for the current device, never the array's name.
constexpr int kNoallocEvalParts = 65536;
constexpr int kNoallocScratchDoubles = 3 * kNoallocEvalParts + 4;
static __device__ __align__(256) double scratch[kNoallocScratchDoubles];

namespace {

using namespace msp;

// Device address of `scratch` per device ordinal, resolved once per device by
// msplat_hip_init with that device current.
constexpr int kMaxDevices = 64;
double* g_scratch_dev[kMaxDevices] = {};

// Stage names: the reference profiler's train stages (msplat_metal.mm:30-34),
// "stage.part" where this build runs a stage as two kernels.  The
// reference's blit_zero (zeroing the gradient buffers) is fused into
// proj_sh_fwd (the projection zeroes each gaussian's accumulators) and its
// grad_stats into proj_sh_bwd_adam.dense.  densify brackets a densification
// call (msplat_densify, which the reference does not profile).
constexpr int kNumStages = 9;
constexpr int kMaxMarks = 12;
const char* kStageNames[kNumStages] = {"proj_sh_fwd",
                                       "prefix_sort_pack.depth_sort",
                                       "prefix_sort_pack.tile_lists",
                                       "rast_fwd",
                                       "loss_fwd_bwd",
                                       "rast_bwd",
                                       "proj_sh_bwd_adam.sh_rest",
                                       "proj_sh_bwd_adam.dense",
                                       "densify"};
enum Stage { S_PROJ, S_DEPTH, S_TILES, S_RFWD, S_LOSS, S_RBWD, S_SHADAM, S_PBWD, S_DENSIFY, S_END };

struct Buf {
    void* p = nullptr;
    size_t bytes = 0;
};

struct Ctx {
    int device = -1;
    hipStream_t own = nullptr;
    hipStream_t stream = nullptr;
    // Stage timing: one event per stage boundary of the current call; the
    // previous call's intervals are folded into the running sums at the next
    // call's host synchronisation point, so timing adds no synchronisation.
    // Each event costs the GPU a few microseconds of idle time between the
    // kernels it sits between, so a caller may bracket only some stages.
    bool timing = false;
    uint32_t stage_mask = ~0u;
    bool stage_open = false;   // the latest event opened a bracketed stage
    hipEvent_t ev[2][kMaxMarks] = {};
    int mark_stage[2][kMaxMarks] = {};
    int n_marks[2] = {0, 0};
    int cur = 0;
    double stage_sum[kNumStages] = {};
    int64_t stage_cnt[kNumStages] = {};
    int64_t calls = 0;
    std::vector<double> call_ms;   // bracketed milliseconds of each timed call since the last drain

    // per gaussian
    Buf rec, radii, tiles_hit, rect, gacc;
    Buf dkey, dval, dkey2, dval2, rect_sorted, hits, dtemp, stemp;
    // per tile
    Buf tcount, tscan, tile_bins, tile_K, tile_item0, l_chunked, tile_done;
    // per super-tile, per super-tile reference, per pair block
    Buf st_r0, st_r1, sstart;
    Buf rkey, rval, rkey2, rval2, rtemp;
    Buf seg, phist;
    // per intersection: the tile-sorted gaussian ids
    Buf tval, qmask;
    // per item
    Buf it_tile, it_k, it_order, tile_order, it_cls, c_T, c_C, c_idx, c_pT, c_aC;
    // per pixel
    Buf final_T, final_idx, out_img, v_rendered, loss_part;
    // scalars
    Buf meta_d, loss_d, count_d, work_d;
    // intersection and reference totals of the projection: ISECT_SLOTS
    // counter pairs, one per 128-byte line (workgroup b adds to slot b %
    // ISECT_SLOTS), summed by the depth sort's first kernel
    Buf isect_d;
    uint64_t* isect_h = nullptr;     // totals_word(I, R), written by the depth sort's first kernel
    unsigned long long* isect_hd = nullptr;   // isect_h as a device pointer
    bool isect_dirty = false;   // counters written and not yet cleared by a tile scan
    // evaluation: per-workgroup fp64 partials and the three sums
    Buf eval_part, eval_out;
    // nearest-neighbour scales: cell keys / point ids (ping-pong), sort
    // scratch, cell ranges
    Buf knn_k, knn_v, knn_k2, knn_v2, knn_tmp, knn_s, knn_e;
    Meta* meta_h = nullptr;
    float* loss_h = nullptr;
    float* loss_hd = nullptr;   // loss_h as a device pointer: the loss kernel writes loss_h[1]
    int* radii_dst = nullptr;   // the caller's radii_out of the current train step, or null
    int* count_h = nullptr;
    // densify scratch
    Buf d_split, d_dup, d_sp, d_dp, d_keep, d_kp, d_tot, d_scratch, d_rnd, d_src;

    const uint32_t* sorted_ids = nullptr;   // tile-sorted gaussian ids (tval)
    Meta meta{};
    bool meta_valid = false;
    // Loss of the most recent train step known to have completed (NaN before
    // any); each step copies its loss to loss_h[1] asynchronously.
    float last_loss = __builtin_nanf("");
    float loss_scale = 1.f;
    bool loss_pending = false;
    int64_t max_items = 0;
    int last_N = 0, last_T = 0, last_W = 0, last_H = 0;
    bool have_bwd = false;
};

Ctx* g_ctx = nullptr;
std::string g_err;

int fail(int code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof(buf), fmt, ap);
    va_end(ap);
    g_err = buf;
    return code;
}

#define HIP_TRY(expr)                                                                        \
    do {                                                                                     \
        hipError_t e_ = (expr);                                                              \
        if (e_ != hipSuccess)                                                                \
            return fail(MSPLAT_ERR_HIP, "%s failed: %s (%s:%d)", #expr, hipGetErrorString(e_), \
                        __FILE__, __LINE__);                                                 \
    } while (0)

// Grow-only device buffer; new memory is zero-filled.
int ensure(Buf& b, size_t bytes) {
    if (bytes == 0) bytes = 16;
    if (bytes <= b.bytes) return MSPLAT_OK;
    size_t want = std::max(bytes, b.bytes + b.bytes / 4);
    want = (want + 255) & ~(size_t)255;
    if (b.p) {
        HIP_TRY(hipStreamSynchronize(g_ctx->stream));
        HIP_TRY(hipFree(b.p));
        b.p = nullptr;
        b.bytes = 0;
    }
    if (hipMalloc(&b.p, want) != hipSuccess) {
        b.p = nullptr;
        return fail(MSPLAT_ERR_NOMEM, "hipMalloc of %zu bytes failed", want);
    }
    b.bytes = want;
    HIP_TRY(hipMemsetAsync(b.p, 0, want, g_ctx->stream));
    return MSPLAT_OK;
}

#define ENSURE(b, n)                      \
    do {                                  \
        int r_ = ensure((b), (n));        \
        if (r_ != MSPLAT_OK) return r_;   \
    } while (0)

template <typename T>
T* P(Buf& b) { return reinterpret_cast<T*>(b.p); }

void free_all(Ctx* c) {
    Buf* bufs[] = {&c->rec, &c->radii, &c->tiles_hit, &c->rect, &c->rect_sorted,
                   &c->gacc, &c->dkey, &c->dval, &c->dkey2, &c->dval2, &c->hits,
                   &c->dtemp, &c->stemp, &c->tcount, &c->tscan, &c->tile_done, &c->tile_bins, &c->tile_K,
                   &c->tile_item0, &c->l_chunked, &c->st_r0, &c->st_r1, &c->sstart,
                   &c->rkey, &c->rval, &c->rkey2, &c->rval2, &c->rtemp, &c->seg, &c->phist,
                   &c->tval, &c->qmask,
                   &c->it_tile, &c->it_k, &c->it_order, &c->tile_order, &c->it_cls, &c->c_T, &c->c_C,
                   &c->c_idx, &c->c_pT, &c->c_aC, &c->final_T, &c->final_idx, &c->out_img,
                   &c->v_rendered, &c->loss_part, &c->meta_d, &c->loss_d,
                   &c->count_d, &c->work_d, &c->isect_d, &c->eval_part, &c->eval_out, &c->knn_k, &c->knn_v, &c->knn_k2, &c->knn_v2,
                   &c->knn_tmp, &c->knn_s, &c->knn_e, &c->d_split, &c->d_dup, &c->d_sp, &c->d_dp, &c->d_keep, &c->d_kp,
                   &c->d_tot, &c->d_scratch, &c->d_rnd, &c->d_src};
    for (Buf* b : bufs)
        if (b->p) { (void)hipFree(b->p); b->p = nullptr; b->bytes = 0; }
    if (c->meta_h) (void)hipHostFree(c->meta_h);
    if (c->loss_h) (void)hipHostFree(c->loss_h);
    if (c->count_h) (void)hipHostFree(c->count_h);
    if (c->isect_h) (void)hipHostFree(c->isect_h);
    for (auto& row : c->ev)
        for (auto& e : row)
            if (e) (void)hipEventDestroy(e);
    if (c->own) (void)hipStreamDestroy(c->own);
}

GaussOut gauss_out(Ctx* c) {
    GaussOut go;
    go.rec = P<float4>(c->rec);
    go.radii = P<int>(c->radii);
    go.radii_out = c->radii_dst;
    go.tiles_hit = P<int>(c->tiles_hit);
    go.rect = P<uint2>(c->rect);
    return go;
}

Items items(Ctx* c) {
    Items it;
    it.tile = P<int>(c->it_tile);
    it.k = P<int>(c->it_k);
    it.tile_K = P<int>(c->tile_K);
    it.tile_item0 = P<int>(c->tile_item0);
    it.order = P<int>(c->it_order);
    it.tile_order = P<int>(c->tile_order);
    it.cls = P<int>(c->it_cls);
    return it;
}

Entries packed(Ctx* c) {
    Entries pk;
    pk.ids = c->sorted_ids;
    pk.rec = P<float4>(c->rec);
    pk.qmask = P<uint8_t>(c->qmask);
    return pk;
}

ChunkBufs chunks(Ctx* c) {
    ChunkBufs cb;
    cb.cT = P<float>(c->c_T);
    cb.cC = P<float>(c->c_C);
    cb.cidx = P<int>(c->c_idx);
    cb.pT = P<float>(c->c_pT);
    cb.aC = P<float>(c->c_aC);
    return cb;
}

int sh_bases(int degree) { return degree == 0 ? 1 : degree == 1 ? 4 : degree == 2 ? 9 : degree == 3 ? 16 : 25; }

// Raster pair counters (composited forward, gradient-carrying backward),
// accumulated while stage timing is enabled for the rasteriser's stage st;
// otherwise null, and the kernels then run without counting.
unsigned long long* work_counters(Ctx* c, int st) {
    return c->timing && ((c->stage_mask >> st) & 1u) ? P<unsigned long long>(c->work_d) : nullptr;
}

// Record the start of stage `st` (S_END closes the call).  Only stages in
// the mask get an event, plus the one that closes a bracketed stage.
void stage_mark(Ctx* c, int st) {
    if (!c->timing) return;
    const bool want = st < kNumStages && ((c->stage_mask >> st) & 1u);
    if (!want && !c->stage_open) return;
    int& n = c->n_marks[c->cur];
    if (n >= kMaxMarks) return;
    (void)hipEventRecord(c->ev[c->cur][n], c->stream);
    c->mark_stage[c->cur][n] = want ? st : -1;
    c->stage_open = want;
    ++n;
}

// Fold the finished intervals of the other event set into the sums.
void stage_fold(Ctx* c, int set) {
    const int n = c->n_marks[set];
    double call = 0.0;
    for (int i = 0; i + 1 < n; ++i) {
        float t = 0.f;
        if (hipEventElapsedTime(&t, c->ev[set][i], c->ev[set][i + 1]) == hipSuccess) {
            const int st = c->mark_stage[set][i];
            if (st >= 0 && st < kNumStages) {
                c->stage_sum[st] += t;
                c->stage_cnt[st] += 1;
                call += t;
            }
        }
    }
    if (n > 1) {
        c->calls += 1;
        if (c->call_ms.size() < (1u << 16)) c->call_ms.push_back(call);
    }
    c->n_marks[set] = 0;
}

// Start a new call: its marks go to the other event set.
void stage_begin(Ctx* c) {
    if (!c->timing) return;
    c->cur ^= 1;
    c->n_marks[c->cur] = 0;
    c->stage_open = false;
}

constexpr int kMaxPoints = 0x7FFFFFFF / 36;

int check_render_args(const MsplatRenderArgs* a) {
    if (!a) return fail(MSPLAT_ERR_ARG, "null args");
    if (a->num_points < 0) return fail(MSPLAT_ERR_ARG, "num_points < 0");
    // the raster backward addresses a gaussian's nine accumulators at byte
    // offset 36 * id in 32 bits
    if (a->num_points > kMaxPoints)
        return fail(MSPLAT_ERR_ARG, "num_points %d exceeds the limit of %d gaussians",
                    a->num_points, kMaxPoints);
    if (a->img_width == 0 || a->img_height == 0) return fail(MSPLAT_ERR_ARG, "empty image");
    if ((uint64_t)a->img_width * a->img_height > (1ull << 31) / 16)
        return fail(MSPLAT_ERR_ARG, "image too large");
    if (a->degree > 4) return fail(MSPLAT_ERR_ARG, "SH degree %u > 4", a->degree);
    const int tbx = (int)((a->img_width + BLOCK - 1) / BLOCK);
    const int tby = (int)((a->img_height + BLOCK - 1) / BLOCK);
    if (a->tile_bounds[0] != tbx || a->tile_bounds[1] != tby)
        return fail(MSPLAT_ERR_ARG, "tile_bounds (%d,%d) != (%d,%d) for a %ux%u image",
                    a->tile_bounds[0], a->tile_bounds[1], tbx, tby, a->img_width, a->img_height);
    if (a->num_points > 0 && (!a->means3d || !a->scales || !a->quats || !a->features_dc ||
                              !a->opacities || (a->degree > 0 && !a->features_rest)))
        return fail(MSPLAT_ERR_ARG, "null gaussian array");
    if (reinterpret_cast<uintptr_t>(a->quats) % 16 != 0)
        return fail(MSPLAT_ERR_ARG, "quats must be 16-byte aligned");
    return MSPLAT_OK;
}

CamParams cam_params(const MsplatRenderArgs* a) {
    CamParams p;
    p.N = a->num_points;
    p.glob_scale = a->glob_scale;
    std::memcpy(p.vm, a->viewmat, sizeof(p.vm));
    std::memcpy(p.pm, a->projmat, sizeof(p.pm));
    p.fx = a->fx; p.fy = a->fy; p.cx = a->cx; p.cy = a->cy;
    p.W = (int)a->img_width;
    p.H = (int)a->img_height;
    p.tbx = a->tile_bounds[0];
    p.tby = a->tile_bounds[1];
    p.clip = a->clip_thresh;
    p.degree = (int)a->degree;
    p.dtu = (int)std::min(a->degrees_to_use, a->degree);
    p.rest_per = (sh_bases(p.degree) - 1) * 3;
    for (int i = 0; i < 3; ++i) { p.cam[i] = a->cam_pos[i]; p.bg[i] = a->background[i]; }
    return p;
}

// forward_pipeline (.mm:462-750): project -> depth order -> tile lists -> raster (+merge).
// The image goes to dst_img, or to the context's own buffer when NULL.
// Waits for the totals word of the current frame (bit 63 set) in coherent
// host memory.  With no gaussians nothing writes it: the stream is drained
// instead, so that the caller may rely on the earlier work having completed
// either way.  A failed or stopped stream ends the wait with its error: the
// stream is queried once the wait has lasted 20 ms, then every 20 ms (a
// stream query queues a packet that holds the GPU for about 5 us between
// two kernels, so a frame's ordinary wait of a millisecond or two makes none).
hipError_t wait_totals(Ctx* c, int N, uint64_t* word) {
    if (N <= 0) {
        *word = 0;
        return hipStreamSynchronize(c->stream);
    }
    using clock = std::chrono::steady_clock;
    auto next_query = clock::now() + std::chrono::milliseconds(20);
    for (unsigned k = 1;; ++k) {
        const uint64_t w = __atomic_load_n(&c->isect_h[0], __ATOMIC_ACQUIRE);
        if (w >> 63) {
            *word = w;
            return hipSuccess;
        }
        if ((k & 255) == 0 && clock::now() >= next_query) {
            next_query = clock::now() + std::chrono::milliseconds(20);
            const hipError_t e = hipStreamQuery(c->stream);
            if (e == hipSuccess) {   // drained: the word must be there now
                const uint64_t v = __atomic_load_n(&c->isect_h[0], __ATOMIC_ACQUIRE);
                if (v >> 63) {
                    *word = v;
                    return hipSuccess;
                }
                return hipErrorUnknown;
            }
            if (e != hipErrorNotReady) return e;
        }
        __builtin_ia32_pause();
    }
}

int forward(Ctx* c, const MsplatRenderArgs* a, bool training, float* dst_img = nullptr,
            int32_t* radii_dst = nullptr) {
    const CamParams p = cam_params(a);
    const int N = p.N, T = p.tbx * p.tby;
    const size_t Px = (size_t)p.W * p.H;
    const size_t Nn = (size_t)std::max(N, 1);
    ENSURE(c->rec, Nn * 64);
    ENSURE(c->radii, Nn * 4);
    // the projection also writes the radii into the caller's buffer when it
    // gives one (no copy after the step)
    c->radii_dst = radii_dst;
    ENSURE(c->tiles_hit, Nn * 4);
    ENSURE(c->rect, Nn * 8);
    ENSURE(c->rect_sorted, Nn * 8);
    ENSURE(c->gacc, Nn * 36);
    ENSURE(c->dkey, Nn * 4);
    ENSURE(c->dval, Nn * 4);
    ENSURE(c->dkey2, Nn * 4);
    ENSURE(c->dval2, Nn * 4);
    ENSURE(c->hits, Nn * 4);
    ENSURE(c->dtemp, (size_t)radix_temp_ints(N) * 4);
    ENSURE(c->stemp, ((size_t)scan_block_count(N) + 8) * 4);
    ENSURE(c->tcount, (size_t)T * 4);
    ENSURE(c->tscan, (size_t)tile_scan_ints(T) * 4);
    const int nst = super_tiles(p.tbx, p.tby);
    if (nst > 65536 || p.tbx > 65535 || p.tby > 65535)
        return fail(MSPLAT_ERR_ARG, "%dx%d tiles exceed the binning's limits (65535 per side, "
                    "65536 super-tiles of %dx%d)", p.tbx, p.tby, SUPER, SUPER);
    ENSURE(c->st_r0, (size_t)nst * 4);
    ENSURE(c->st_r1, (size_t)nst * 4);
    ENSURE(c->sstart, ((size_t)nst + 1) * 4);
    ENSURE(c->tile_bins, (size_t)T * 8);
    ENSURE(c->tile_K, (size_t)T * 4);
    ENSURE(c->tile_item0, (size_t)T * 4);
    ENSURE(c->l_chunked, (size_t)T * 4);
    ENSURE(c->tile_done, (size_t)T * 4);
    ENSURE(c->final_T, Px * 4);
    ENSURE(c->final_idx, Px * 4);
    ENSURE(c->out_img, Px * 12);
    ENSURE(c->meta_d, sizeof(Meta));
    c->last_N = N; c->last_T = T; c->last_W = p.W; c->last_H = p.H;
    c->have_bwd = false;

    // The projection adds up the intersection and reference totals, which
    // the depth sort's first kernel writes to coherent host memory (isect_h,
    // one word with a ready bit) while the GPU goes on sorting: the host
    // polls that word, without an event on the stream.  (isect_h is zeroed
    // first.  The device counters arrive zeroed: fresh buffers are, and the
    // tile scan of the previous frame cleared them, unless that frame
    // stopped before it.)
    ENSURE(c->isect_d, ISECT_BYTES);
    if (c->isect_dirty) HIP_TRY(hipMemsetAsync(c->isect_d.p, 0, ISECT_BYTES, c->stream));
    c->isect_dirty = true;
    __atomic_store_n(&c->isect_h[0], (uint64_t)0, __ATOMIC_RELEASE);
    stage_mark(c, S_PROJ);
    GaussOut go = gauss_out(c);
    launch_project_fwd(c->stream, p, a->means3d, a->scales, a->quats, a->features_dc,
                       a->features_rest, a->opacities, go, P<uint32_t>(c->dkey),
                       P<uint32_t>(c->dval), training ? P<float>(c->gacc) : nullptr,
                       P<unsigned long long>(c->isect_d));
    stage_mark(c, S_DEPTH);
    uint32_t* order = nullptr;
    const SlotSum totals{P<unsigned long long>(c->isect_d), c->isect_hd};
    launch_depth_order(c->stream, N, P<uint32_t>(c->dkey), P<uint32_t>(c->dval),
                       P<uint32_t>(c->dkey2), P<uint32_t>(c->dval2), P<int>(c->dtemp),
                       P<uint2>(c->rect), P<uint2>(c->rect_sorted), P<int>(c->hits),
                       P<int>(c->stemp), &totals, &order);
    uint64_t word = 0;
    HIP_TRY(wait_totals(c, N, &word));
    // everything queued before the sort's first kernel has completed now,
    // the previous call's loss kernel included
    if (c->loss_pending) {
        c->last_loss = c->loss_h[1] * c->loss_scale;
        c->loss_pending = false;
    }
    const int64_t I64 = (int64_t)((word >> 31) & 0x7FFFFFFFull);
    const int64_t R64 = (int64_t)(word & 0x7FFFFFFFull);
    if (I64 > (int64_t)0x7FFFFFFF - 4096)
        return fail(MSPLAT_ERR_ARG, "%lld tile intersections exceed the 32-bit index range",
                    (long long)I64);
    const size_t I = (size_t)std::max<int64_t>(I64, 1);
    const size_t R = (size_t)std::max<int64_t>(R64, 1);
    const size_t NS = (size_t)segments_bound(R64, nst);
    ENSURE(c->tval, I * 4);
    ENSURE(c->qmask, I);
    ENSURE(c->rkey, R * 4);
    ENSURE(c->rval, R * 4);
    ENSURE(c->rkey2, R * 4);
    ENSURE(c->rval2, R * 4);
    ENSURE(c->rtemp, (size_t)radix_temp_ints((int64_t)R) * 4);
    ENSURE(c->seg, NS * 16);
    ENSURE(c->phist, NS * SUPER * SUPER * 4);
    const int64_t max_items = items_bound(T, I64);
    ENSURE(c->it_tile, (size_t)max_items * 4);
    ENSURE(c->it_k, (size_t)max_items * 4);
    ENSURE(c->it_order, (size_t)max_items * 4);
    ENSURE(c->tile_order, (size_t)T * 4);
    ENSURE(c->it_cls, 4 * 32 * 4);
    const size_t S = (size_t)max_items * TILE_PIX;
    ENSURE(c->c_T, S * 4);
    ENSURE(c->c_C, S * 12);
    ENSURE(c->c_idx, S * 4);
    if (training) {
        ENSURE(c->c_pT, S * 4);
        ENSURE(c->c_aC, S * 12);
    }
    c->max_items = max_items;
    stage_mark(c, S_TILES);
    TileLists tl{P<int>(c->l_chunked), nullptr, nullptr};
    Items it = items(c);
    RefBufs rb;
    rb.key = P<uint32_t>(c->rkey);
    rb.val = P<uint32_t>(c->rval);
    rb.key2 = P<uint32_t>(c->rkey2);
    rb.val2 = P<uint32_t>(c->rval2);
    rb.radix_temp = P<int>(c->rtemp);
    rb.st_r0 = P<int>(c->st_r0);
    rb.st_r1 = P<int>(c->st_r1);
    rb.sstart = P<int>(c->sstart);
    rb.seg = P<int4>(c->seg);
    rb.hist = P<int>(c->phist);
    rb.tcount = P<int>(c->tcount);
    launch_tile_lists(c->stream, p, I64, R64, order, P<int>(c->stemp),
                      P<uint2>(c->rect_sorted), rb,
                      P<uint32_t>(c->tval), P<int>(c->tscan), P<int>(c->tile_bins), it, tl,
                      P<Meta>(c->meta_d), P<unsigned long long>(c->isect_d));
    c->sorted_ids = P<uint32_t>(c->tval);
    c->isect_dirty = false;   // the tile scan clears the counters
    Entries pk = packed(c);
    float* img = dst_img ? dst_img : P<float>(c->out_img);
    stage_mark(c, S_RFWD);
    ChunkBufs cb = chunks(c);
    if (training) {
        // every chunk's state is kept: the backward's suffix sums run over
        // all chunks of a tile
        launch_raster_fwd(c->stream, p, max_items, P<Meta>(c->meta_d), it, P<int>(c->tile_bins),
                          pk, P<float>(c->final_T), P<int>(c->final_idx), img, cb,
                          work_counters(c, S_RFWD), P<int>(c->l_chunked), P<int>(c->tile_done));
        launch_raster_merge(c->stream, p, P<Meta>(c->meta_d), P<int>(c->l_chunked), it,
                            P<float>(c->final_T), P<int>(c->final_idx), img, cb, true,
                            P<int>(c->tile_done));
    } else {
        launch_render_tiles(c->stream, p, it, P<int>(c->tile_bins), pk, P<float>(c->final_T),
                            P<int>(c->final_idx), img, work_counters(c, S_RFWD));
    }
    // the previous call's stage times (it has completed: the event above
    // follows it), read once this call's kernels are queued
    if (c->timing) stage_fold(c, c->cur ^ 1);
    HIP_TRY(hipGetLastError());
    c->meta_valid = false;
    return MSPLAT_OK;
}

}  // namespace

extern "C" {

int msplat_hip_init(int device) {
    if (g_ctx) {
        if (g_ctx->device == device) return MSPLAT_OK;
        return fail(MSPLAT_ERR_ARG, "already initialised on device %d", g_ctx->device);
    }
    int n = 0;
    HIP_TRY(hipGetDeviceCount(&n));
    if (device < 0 || device >= n) return fail(MSPLAT_ERR_ARG, "device %d of %d", device, n);
    if (device >= kMaxDevices) return fail(MSPLAT_ERR_ARG, "device %d beyond %d", device, kMaxDevices);
    HIP_TRY(hipSetDevice(device));
    if (!g_scratch_dev[device]) {
        void* sp = nullptr;
        HIP_TRY(hipGetSymbolAddress(&sp, HIP_SYMBOL(scratch)));
        if (!sp) return fail(MSPLAT_ERR_HIP, "hipGetSymbolAddress(scratch) returned null");
        g_scratch_dev[device] = static_cast<double*>(sp);
    }
    Ctx* c = new Ctx();
    c->device = device;
    g_ctx = c;
    if (hipStreamCreate(&c->own) != hipSuccess) {   // blocking stream, default priority
        g_ctx = nullptr;
        delete c;
        return fail(MSPLAT_ERR_HIP, "hipStreamCreate failed");
    }
    c->stream = c->own;
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->meta_h), sizeof(Meta)));
    // coherent: the host reads the previous step's loss without a stream
    // sync once a later kernel has published the totals word (isect_h)
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->loss_h), 16,
                          hipHostMallocMapped | hipHostMallocCoherent));
    HIP_TRY(hipHostGetDevicePointer(reinterpret_cast<void**>(&c->loss_hd), c->loss_h, 0));
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->count_h), 16));
    HIP_TRY(hipHostMalloc(reinterpret_cast<void**>(&c->isect_h), 16,
                          hipHostMallocMapped | hipHostMallocCoherent));
    HIP_TRY(hipHostGetDevicePointer(reinterpret_cast<void**>(&c->isect_hd), c->isect_h, 0));
    for (auto& row : c->ev)
        // timing only (their times are read once later work shows they have
        // completed): no system-scope fence, which costs the GPU about 1 us
        // more per event
        for (auto& e : row) HIP_TRY(hipEventCreateWithFlags(&e, hipEventDisableSystemFence));
    return MSPLAT_OK;
}

int msplat_hip_shutdown(void) {
    if (!g_ctx) return MSPLAT_OK;
    (void)hipStreamSynchronize(g_ctx->stream);
    free_all(g_ctx);
    delete g_ctx;
    g_ctx = nullptr;
    return MSPLAT_OK;
}

const char* msplat_hip_last_error(void) { return g_err.c_str(); }

int msplat_hip_set_stream(void* s) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    g_ctx->stream = s ? reinterpret_cast<hipStream_t>(s) : g_ctx->own;
    return MSPLAT_OK;
}

void* msplat_hip_get_stream(void) { return g_ctx ? (void*)g_ctx->stream : nullptr; }

int msplat_hip_alloc(void** ptr, size_t bytes) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!ptr) return fail(MSPLAT_ERR_ARG, "null ptr");
    if (hipMalloc(ptr, bytes ? bytes : 4) != hipSuccess) return fail(MSPLAT_ERR_NOMEM, "hipMalloc(%zu)", bytes);
    return MSPLAT_OK;
}

int msplat_hip_alloc_mapped(void** ptr, size_t bytes) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!ptr) return fail(MSPLAT_ERR_ARG, "null ptr");
    void* h = nullptr;
    if (hipHostMalloc(&h, bytes ? bytes : 4, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
        return fail(MSPLAT_ERR_NOMEM, "hipHostMalloc(%zu)", bytes);
    void* d = nullptr;
    if (hipHostGetDevicePointer(&d, h, 0) != hipSuccess || d != h) {
        (void)hipHostFree(h);
        return fail(MSPLAT_ERR_HIP, "mapped host memory is not at the same device address");
    }
    *ptr = h;
    return MSPLAT_OK;
}

int msplat_hip_free_mapped(void* ptr) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (ptr) {
        HIP_TRY(hipStreamSynchronize(g_ctx->stream));
        HIP_TRY(hipHostFree(ptr));
    }
    return MSPLAT_OK;
}

int msplat_hip_free(void* ptr) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (ptr) {
        HIP_TRY(hipStreamSynchronize(g_ctx->stream));
        HIP_TRY(hipFree(ptr));
    }
    return MSPLAT_OK;
}

int msplat_hip_memset(void* ptr, int value, size_t bytes) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    HIP_TRY(hipMemsetAsync(ptr, value, bytes, g_ctx->stream));
    return MSPLAT_OK;
}

int msplat_hip_memcpy_h2d(void* dst, const void* src, size_t bytes) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyHostToDevice, g_ctx->stream));
    HIP_TRY(hipStreamSynchronize(g_ctx->stream));
    return MSPLAT_OK;
}

int msplat_hip_memcpy_d2h(void* dst, const void* src, size_t bytes) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDeviceToHost, g_ctx->stream));
    HIP_TRY(hipStreamSynchronize(g_ctx->stream));
    return MSPLAT_OK;
}

int msplat_hip_memcpy_d2d(void* dst, const void* src, size_t bytes) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    HIP_TRY(hipMemcpyAsync(dst, src, bytes, hipMemcpyDefault, g_ctx->stream));
    return MSPLAT_OK;
}

int msplat_hip_commit(void) { return g_ctx ? MSPLAT_OK : fail(MSPLAT_ERR_NOINIT, "not initialised"); }

int msplat_hip_sync(void) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->loss_pending) {
        c->last_loss = c->loss_h[1] * c->loss_scale;
        c->loss_pending = false;
    }
    return MSPLAT_OK;
}

int msplat_hip_render(const MsplatRenderArgs* a, float* out_img) {
    // argument errors are reported whether or not a context exists
    int r = check_render_args(a);
    if (r != MSPLAT_OK) return r;
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    stage_begin(c);
    r = forward(c, a, false, out_img);
    if (r != MSPLAT_OK) return r;
    stage_mark(c, S_END);
    return MSPLAT_OK;
}

int msplat_hip_train_step(const MsplatTrainArgs* a, int32_t* radii_out, float* loss_out) {
    if (!a) return fail(MSPLAT_ERR_ARG, "null args");
    int r = check_render_args(&a->r);
    if (r != MSPLAT_OK) return r;
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (a->num_adam_groups != 6) return fail(MSPLAT_ERR_ARG, "num_adam_groups must be 6");
    if (!a->gt) return fail(MSPLAT_ERR_ARG, "null gt");
    const float* rp[6] = {a->r.means3d, a->r.scales, a->r.quats, a->r.features_dc,
                          a->r.features_rest, a->r.opacities};
    for (int g = 0; g < 6; ++g) {
        if (g == 4 && a->r.degree == 0) continue;
        if (a->adam_params[g] != rp[g])
            return fail(MSPLAT_ERR_ARG, "adam_params[%d] must alias the render array", g);
        if (!a->adam_exp_avg[g] || !a->adam_exp_avg_sq[g])
            return fail(MSPLAT_ERR_ARG, "null Adam state for group %d", g);
    }
    if (!a->vis_counts || !a->xys_grad_norm || !a->max_2d_size)
        return fail(MSPLAT_ERR_ARG, "null grad-stat array");
    stage_begin(c);
    r = forward(c, &a->r, true, nullptr, radii_out);
    if (r != MSPLAT_OK) return r;
    const CamParams p = cam_params(&a->r);
    const size_t Px = (size_t)p.W * p.H;
    const dim3 sgrid((p.W + 15) / 16, (p.H + 15) / 16);
    ENSURE(c->v_rendered, Px * 12);
    ENSURE(c->loss_part, (size_t)sgrid.x * sgrid.y * 12);
    ENSURE(c->loss_d, 16);
    stage_mark(c, S_LOSS);
    // the loss sum goes straight to pinned host memory (loss_h[1])
    const int nparts = launch_ssim(c->stream, p.H, p.W, P<float>(c->out_img), a->gt, a->ssim_weight,
                                   a->loss_inv_n, P<float>(c->v_rendered), P<float>(c->loss_part));
    // the raster backward's workgroup 0 folds the partials into loss_h[1]
    const LossFold lf{P<float>(c->loss_part), nparts, a->ssim_weight, c->loss_hd + 1};
    stage_mark(c, S_RBWD);
    launch_raster_bwd(c->stream, p, c->max_items, P<Meta>(c->meta_d), items(c),
                      P<int>(c->tile_bins), packed(c),
                      P<float>(c->final_T), P<int>(c->final_idx), chunks(c),
                      P<float>(c->v_rendered), P<float>(c->gacc), work_counters(c, S_RBWD), lf);
    AdamHP hp;
    for (int g = 0; g < 6; ++g) { hp.step[g] = a->adam_step_sizes[g]; hp.inv_bc2[g] = 1.0f / a->adam_bc2_sqrts[g]; }
    hp.b1 = a->adam_beta1;
    hp.b2 = a->adam_beta2;
    hp.eps = a->adam_eps;
    GaussOut go = gauss_out(c);
    // The two Adam kernels are independent (same inputs, disjoint outputs).
    // The projection backward runs first, right after the raster backward,
    // while the records and accumulators it gathers are still in cache; the
    // streaming f_rest Adam loses less by going second.
    stage_mark(c, S_PBWD);
    launch_proj_bwd_adam(c->stream, p, a->adam_params, a->adam_exp_avg, a->adam_exp_avg_sq, hp, go,
                         P<float>(c->gacc), a->vis_counts, a->xys_grad_norm, a->max_2d_size,
                         a->inv_max_dim, a->v_mean3d_out, a->v_scale_out, a->v_quat_out);
    stage_mark(c, S_SHADAM);
    launch_sh_rest_adam(c->stream, p, go.rec, go.radii, P<float>(c->gacc), a->adam_params[4],
                        a->adam_exp_avg[4], a->adam_exp_avg_sq[4], hp);
    stage_mark(c, S_END);
    c->have_bwd = true;
    HIP_TRY(hipGetLastError());
    if (loss_out) {
        HIP_TRY(hipStreamSynchronize(c->stream));
        *loss_out = c->loss_h[1] / (float)(p.H * p.W);
        c->last_loss = *loss_out;
        c->loss_pending = false;
    } else {
        // read once a later wait on the stream has passed this step
        c->loss_scale = 1.f / (float)(p.H * p.W);
        c->loss_pending = true;
    }
    return MSPLAT_OK;
}

int msplat_hip_last_loss(float* loss, int wait) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!loss) return fail(MSPLAT_ERR_ARG, "null loss");
    if (c->loss_pending && wait) {
        HIP_TRY(hipStreamSynchronize(c->stream));
        c->last_loss = c->loss_h[1] * c->loss_scale;
        c->loss_pending = false;
    }
    *loss = c->last_loss;
    return MSPLAT_OK;
}

int msplat_hip_clamp_max(float* p, int64_t n, float hi) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (n < 0 || (n > 0 && !p)) return fail(MSPLAT_ERR_ARG, "bad clamp arguments");
    launch_clamp_max(g_ctx->stream, p, n, hi);
    HIP_TRY(hipGetLastError());
    return MSPLAT_OK;
}

int msplat_hip_image_to_rgba8(const float* img, int64_t n_pixels, uint8_t* rgba) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (n_pixels < 0 || (n_pixels > 0 && (!img || !rgba)))
        return fail(MSPLAT_ERR_ARG, "bad rgba8 arguments");
    if (reinterpret_cast<uintptr_t>(rgba) % 4 != 0)
        return fail(MSPLAT_ERR_ARG, "rgba must be 4-byte aligned");
    launch_to_rgba8(g_ctx->stream, img, n_pixels, reinterpret_cast<uint32_t*>(rgba));
    HIP_TRY(hipGetLastError());
    return MSPLAT_OK;
}

namespace {
// Arguments and window of the image metrics, exactly as ssim_eval builds the
// window (ssim.cpp:68-75), in fp32.
int metrics_setup(const float* img, const float* gt, int32_t height, int32_t width,
                  int32_t window_size, float sigma, const MsplatImageMetrics* out, EvalWindow& win) {
    if (!img || !gt || !out) return fail(MSPLAT_ERR_ARG, "null metrics argument");
    if (height <= 0 || width <= 0 || (int64_t)height * width > (int64_t)1 << 30)
        return fail(MSPLAT_ERR_ARG, "bad image size %dx%d", width, height);
    if (window_size < 1 || window_size > 11 || window_size % 2 == 0)
        return fail(MSPLAT_ERR_ARG, "window size %d: odd and at most 11", window_size);
    if (!(sigma > 0.f)) return fail(MSPLAT_ERR_ARG, "sigma must be positive");
    win.ws = window_size;
    win.pad = window_size / 2;
    float ksum = 0.f;
    for (int i = 0; i < window_size; ++i) {
        const float x = (float)(i - window_size / 2);
        win.w[i] = std::exp(-(x * x) / (2.0f * sigma * sigma));
        ksum += win.w[i];
    }
    for (int i = 0; i < window_size; ++i) win.w[i] /= ksum;
    for (int i = window_size; i < 11; ++i) win.w[i] = 0.f;
    return MSPLAT_OK;
}

// Run the metric kernels with the given partials / sums buffers and read the
// three sums back (into a stack array: no allocation).
int metrics_run(Ctx* c, const float* img, const float* gt, int32_t height, int32_t width,
                const EvalWindow& win, double* part, double* out3, MsplatImageMetrics* out) {
    launch_image_metrics(c->stream, img, gt, height, width, win, part, out3);
    HIP_TRY(hipGetLastError());
    double sums[3];
    HIP_TRY(hipMemcpyAsync(sums, out3, sizeof(sums), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    const double n = (double)height * (double)width * 3.0;
    const double mse = sums[1] / n;
    out->psnr = (float)(10.0f * std::log10(1.0 / mse));
    out->ssim = (float)(sums[0] / (double)((int64_t)height * width * 3));
    out->l1 = (float)(sums[2] / n);
    return MSPLAT_OK;
}
}  // namespace

int msplat_hip_image_metrics(const float* img, const float* gt, int32_t height, int32_t width,
                             int32_t window_size, float sigma, MsplatImageMetrics* out) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    EvalWindow win;
    int r = metrics_setup(img, gt, height, width, window_size, sigma, out, win);
    if (r != MSPLAT_OK) return r;
    ENSURE(c->eval_part, (size_t)eval_partial_count(height, width) * 3 * sizeof(double));
    ENSURE(c->eval_out, 3 * sizeof(double));
    return metrics_run(c, img, gt, height, width, win, P<double>(c->eval_part),
                       P<double>(c->eval_out), out);
}

int msplat_hip_image_metrics_noalloc(const float* img, const float* gt, int32_t height,
                                     int32_t width, int32_t window_size, float sigma,
                                     MsplatImageMetrics* out) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    EvalWindow win;
    int r = metrics_setup(img, gt, height, width, window_size, sigma, out, win);
    if (r != MSPLAT_OK) return r;
    const int64_t parts = eval_partial_count(height, width);
    if (parts > kNoallocEvalParts)
        return fail(MSPLAT_ERR_ARG,
                    "%dx%d image needs %lld metric tiles; the allocation-free workspace holds %d "
                    "(64x16 pixels each)",
                    width, height, (long long)parts, kNoallocEvalParts);
    double* ws = g_scratch_dev[c->device];
    if (!ws) return fail(MSPLAT_ERR_NOINIT, "workspace address of device %d not resolved", c->device);
    // every partial and the three sums are written before they are read: the
    // previous call's contents need no clearing
    return metrics_run(c, img, gt, height, width, win, ws, ws + 3 * (size_t)kNoallocEvalParts, out);
}

int msplat_hip_resize_area(const float* src, int32_t src_w, int32_t src_h, float* dst,
                           int32_t dst_w, int32_t dst_h) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!src || !dst) return fail(MSPLAT_ERR_ARG, "null resize argument");
    if (src_w <= 0 || src_h <= 0 || (int64_t)src_w * src_h > (int64_t)1 << 30)
        return fail(MSPLAT_ERR_ARG, "bad source size %dx%d", src_w, src_h);
    if (dst_w <= 0 || dst_h <= 0 || (int64_t)dst_w * dst_h > (int64_t)1 << 30)
        return fail(MSPLAT_ERR_ARG, "bad destination size %dx%d", dst_w, dst_h);
    launch_resize_area(g_ctx->stream, src, src_w, src_h, dst, dst_w, dst_h);
    HIP_TRY(hipGetLastError());
    return MSPLAT_OK;
}

namespace {
int undistort_params(int32_t width, int32_t height, const float intr[4], const float dist[5],
                     UndistortParams& u) {
    if (!intr || !dist) return fail(MSPLAT_ERR_ARG, "null undistortion argument");
    if (width <= 0 || height <= 0 || (int64_t)width * height > (int64_t)1 << 30)
        return fail(MSPLAT_ERR_ARG, "bad image size %dx%d", width, height);
    for (int i = 0; i < 4; ++i)
        if (!std::isfinite(intr[i])) return fail(MSPLAT_ERR_ARG, "intrinsics must be finite");
    for (int i = 0; i < 5; ++i)
        if (!std::isfinite(dist[i])) return fail(MSPLAT_ERR_ARG, "distortion must be finite");
    if (intr[0] == 0.f || intr[1] == 0.f) return fail(MSPLAT_ERR_ARG, "fx, fy must be nonzero");
    u = UndistortParams{intr[0], intr[1], intr[2], intr[3], dist[0], dist[1], dist[2], dist[3],
                        dist[4], 0, 0, 0, 0};
    return MSPLAT_OK;
}
}  // namespace

int msplat_undistort_roi(int32_t width, int32_t height, const float intrinsics[4],
                         const float distortion[5], int32_t roi[4]) {
    UndistortParams u;
    const int r = undistort_params(width, height, intrinsics, distortion, u);
    if (r != MSPLAT_OK) return r;
    if (!roi) return fail(MSPLAT_ERR_ARG, "null roi");
    undistort_roi(width, height, u);
    roi[0] = u.roi_x; roi[1] = u.roi_y; roi[2] = u.roi_w; roi[3] = u.roi_h;
    return MSPLAT_OK;
}

int msplat_hip_undistort(const float* src, int32_t width, int32_t height, const float intrinsics[4],
                         const float distortion[5], const int32_t roi[4], float* dst) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!src || !dst || !roi) return fail(MSPLAT_ERR_ARG, "null undistortion argument");
    UndistortParams u;
    const int r = undistort_params(width, height, intrinsics, distortion, u);
    if (r != MSPLAT_OK) return r;
    if (roi[0] < 0 || roi[1] < 0 || roi[2] <= 0 || roi[3] <= 0 || roi[2] > width - roi[0] ||
        roi[3] > height - roi[1])
        return fail(MSPLAT_ERR_ARG, "roi (%d,%d %dx%d) outside the %dx%d image", roi[0], roi[1],
                    roi[2], roi[3], width, height);
    u.roi_x = roi[0]; u.roi_y = roi[1]; u.roi_w = roi[2]; u.roi_h = roi[3];
    launch_undistort(g_ctx->stream, src, width, height, u, dst);
    HIP_TRY(hipGetLastError());
    return MSPLAT_OK;
}

int msplat_hip_knn_mean_dist(const float* xyz, int64_t n, float* mean_dist) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!xyz || !mean_dist) return fail(MSPLAT_ERR_ARG, "null knn argument");
    if (n < 4) return fail(MSPLAT_ERR_ARG, "%lld points: at least 4 are needed", (long long)n);
    if (n > 0x7FFFFFFF) return fail(MSPLAT_ERR_ARG, "too many points");
    // bounding box on the host (an initialisation-time call)
    std::vector<float> host((size_t)n * 3);
    HIP_TRY(hipMemcpyAsync(host.data(), xyz, host.size() * 4, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    float lo[3], hi[3];
    for (int k = 0; k < 3; ++k) { lo[k] = INFINITY; hi[k] = -INFINITY; }
    for (int64_t i = 0; i < n; ++i)
        for (int k = 0; k < 3; ++k) {
            const float v = host[3 * i + k];
            if (!std::isfinite(v)) return fail(MSPLAT_ERR_ARG, "point %lld is not finite", (long long)i);
            lo[k] = std::min(lo[k], v);
            hi[k] = std::max(hi[k], v);
        }
    // cell edge: about one point per cell, at most 4 n cells and 1024 per axis
    double ext[3], emax = 0.0, amax = 0.0;
    for (int k = 0; k < 3; ++k) {
        ext[k] = (double)hi[k] - (double)lo[k];
        emax = std::max(emax, ext[k]);
        amax = std::max(amax, std::max(std::fabs((double)lo[k]), std::fabs((double)hi[k])));
    }
    KnnGrid g;
    double h = emax > 0.0 ? emax / std::cbrt((double)n) : 1.0;
    auto dims_for = [&](double hh, int* d) {
        double cells = 1.0;
        for (int k = 0; k < 3; ++k) {
            d[k] = (int)std::min(1024.0, std::max(1.0, std::ceil(ext[k] / hh)));
            cells *= d[k];
        }
        return cells;
    };
    for (int it = 0; it < 40 && dims_for(h, g.dim) < 0.5 * (double)n; ++it) {
        if (std::max(g.dim[0], std::max(g.dim[1], g.dim[2])) >= 1024) break;
        h *= 0.8;
    }
    while (dims_for(h, g.dim) > 4.0 * (double)n) h *= 1.25;
    if (emax > 0.0) h = std::max(h, emax / 1024.0);
    dims_for(h, g.dim);
    for (int k = 0; k < 3; ++k) g.lo[k] = lo[k];
    g.h = (float)h;
    g.inv_h = (float)(1.0 / h);
    g.margin = (float)(1e-3 * h + 1e-6 * amax);
    const int64_t cells = (int64_t)g.dim[0] * g.dim[1] * g.dim[2];
    int bits = 1;
    while (((int64_t)1 << bits) < cells) ++bits;
    const size_t N = (size_t)n;
    ENSURE(c->knn_k, N * 4);
    ENSURE(c->knn_v, N * 4);
    ENSURE(c->knn_k2, N * 4);
    ENSURE(c->knn_v2, N * 4);
    ENSURE(c->knn_tmp, (size_t)radix_temp_ints(n) * 4);
    ENSURE(c->knn_s, (size_t)cells * 4);
    ENSURE(c->knn_e, (size_t)cells * 4);
    HIP_TRY(hipMemsetAsync(c->knn_s.p, 0, (size_t)cells * 4, c->stream));
    HIP_TRY(hipMemsetAsync(c->knn_e.p, 0, (size_t)cells * 4, c->stream));
    launch_knn_cells(c->stream, n, xyz, g, P<uint32_t>(c->knn_k), P<uint32_t>(c->knn_v));
    const bool flip = launch_radix_sort(c->stream, P<uint32_t>(c->knn_k), P<uint32_t>(c->knn_v),
                                        P<uint32_t>(c->knn_k2), P<uint32_t>(c->knn_v2), n, bits,
                                        P<int>(c->knn_tmp));
    const uint32_t* sk = flip ? P<uint32_t>(c->knn_k2) : P<uint32_t>(c->knn_k);
    const uint32_t* order = flip ? P<uint32_t>(c->knn_v2) : P<uint32_t>(c->knn_v);
    launch_run_edges(c->stream, n, sk, P<int>(c->knn_s), P<int>(c->knn_e));
    launch_knn_search(c->stream, n, xyz, g, order, P<int>(c->knn_s), P<int>(c->knn_e), mean_dist);
    HIP_TRY(hipGetLastError());
    return MSPLAT_OK;
}

int msplat_hip_randn(float* dst, int64_t n, uint64_t seed) {
    if (!g_ctx) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    launch_randn(g_ctx->stream, dst, n, seed);
    HIP_TRY(hipGetLastError());
    return MSPLAT_OK;
}

int msplat_hip_densify(const MsplatDensifyArgs* a, int32_t* new_count) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!a || !new_count) return fail(MSPLAT_ERR_ARG, "null args");
    const int N = a->N;
    if (N <= 0) { *new_count = N; return MSPLAT_OK; }
    const int64_t worst = 3 * (int64_t)N;
    if (worst > a->buf_capacity)
        return fail(MSPLAT_ERR_ARG, "3*N = %lld exceeds buf_capacity %d", (long long)worst,
                    a->buf_capacity);
    for (int g = 0; g < 6; ++g)
        if (!a->bufs[g] || !a->adam_exp_avg_buf[g] || !a->adam_exp_avg_sq_buf[g])
            if (!(g == 4 && a->fr_stride == 0)) return fail(MSPLAT_ERR_ARG, "null buffer %d", g);
    ENSURE(c->d_split, (size_t)N * 4);
    ENSURE(c->d_dup, (size_t)N * 4);
    ENSURE(c->d_sp, (size_t)N * 4);
    ENSURE(c->d_dp, (size_t)N * 4);
    ENSURE(c->d_keep, (size_t)worst * 4);
    ENSURE(c->d_kp, (size_t)worst * 4);
    ENSURE(c->d_tot, (size_t)scan_block_count(worst) * 4 + 64);
    ENSURE(c->count_d, 16);
    stage_begin(c);
    stage_mark(c, S_DENSIFY);
    const float* rnd = a->random_samples;
    if (!rnd) {
        ENSURE(c->d_rnd, (size_t)2 * N * 3 * 4);
        launch_randn(c->stream, P<float>(c->d_rnd), (int64_t)2 * N * 3, a->seed);
        rnd = P<float>(c->d_rnd);
    }
    DensifyHP hp;
    hp.N = N;
    hp.grad_thresh = a->grad_thresh;
    hp.size_thresh = a->size_thresh;
    hp.screen_thresh = a->screen_thresh;
    hp.check_screen = a->check_screen;
    hp.cull_alpha = a->cull_alpha_thresh;
    hp.cull_scale = a->cull_scale_thresh;
    hp.cull_screen = a->cull_screen_size;
    hp.check_huge = a->check_huge;
    hp.half_max_dim = a->half_max_dim;
    hp.fr = a->fr_stride;
    launch_densify(c->stream, hp, a->xys_grad_norm, a->vis_counts, a->max_2d_size, a->bufs,
                   a->adam_exp_avg_buf, a->adam_exp_avg_sq_buf, rnd, P<int>(c->d_split),
                   P<int>(c->d_dup), P<int>(c->d_sp), P<int>(c->d_dp), P<int>(c->d_keep),
                   P<int>(c->d_kp), P<int>(c->d_tot), P<int>(c->count_d));
    HIP_TRY(hipGetLastError());
    // rows after appending and rows kept size the compaction exactly
    HIP_TRY(hipMemcpyAsync(c->count_h, c->count_d.p, 8, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    const int rows = c->count_h[0], kept = c->count_h[1];
    if (rows < 0 || rows > worst || kept < 0 || kept > rows)
        return fail(MSPLAT_ERR_HIP, "densify counts out of range: %d rows, %d kept (N = %d)", rows,
                    kept, N);
    ENSURE(c->d_src, (size_t)std::max(kept, 1) * 4);
    ENSURE(c->d_scratch, (size_t)densify_workspace_floats(kept, a->fr_stride) * 4);
    launch_densify_compact(c->stream, rows, kept, a->fr_stride, a->bufs, a->adam_exp_avg_buf,
                           a->adam_exp_avg_sq_buf, P<int>(c->d_keep), P<int>(c->d_kp),
                           P<int>(c->d_src), P<float>(c->d_scratch));
    HIP_TRY(hipGetLastError());
    stage_mark(c, S_END);
    HIP_TRY(hipStreamSynchronize(c->stream));
    if (c->timing) {   // the previous call and this one have completed
        stage_fold(c, c->cur ^ 1);
        stage_fold(c, c->cur);
    }
    *new_count = kept;
    return MSPLAT_OK;
}

int msplat_hip_enable_stage_timing(int enable) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    c->timing = enable != 0;
    if (c->timing) {
        const size_t wb = (size_t)WORK_SLOTS * WORK_SLOT_U64 * sizeof(unsigned long long);
        ENSURE(c->work_d, wb);
        HIP_TRY(hipMemsetAsync(c->work_d.p, 0, wb, c->stream));
    }
    c->n_marks[0] = c->n_marks[1] = 0;
    for (int i = 0; i < kNumStages; ++i) { c->stage_sum[i] = 0.0; c->stage_cnt[i] = 0; }
    c->calls = 0;
    c->call_ms.clear();
    return MSPLAT_OK;
}

int msplat_hip_set_stage_timing_mask(uint32_t mask) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    c->stage_mask = mask;
    return MSPLAT_OK;
}

int msplat_hip_drain_stage_times(double* ms, int64_t* counts, const char** names, int max_stages,
                                 int* n_stages, int64_t* n_calls) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    HIP_TRY(hipStreamSynchronize(c->stream));
    stage_fold(c, c->cur);
    stage_fold(c, c->cur ^ 1);
    const int n = std::min(max_stages, kNumStages);
    for (int i = 0; i < n; ++i) {
        if (ms) ms[i] = c->stage_sum[i];
        if (counts) counts[i] = c->stage_cnt[i];
        if (names) names[i] = kStageNames[i];
        c->stage_sum[i] = 0.0;
        c->stage_cnt[i] = 0;
    }
    if (n_stages) *n_stages = n;
    if (n_calls) *n_calls = c->calls;
    c->calls = 0;
    return MSPLAT_OK;
}

int msplat_hip_drain_call_times(double* ms, int max_calls, int* n_calls) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!n_calls || (max_calls > 0 && !ms)) return fail(MSPLAT_ERR_ARG, "null argument");
    HIP_TRY(hipStreamSynchronize(c->stream));
    stage_fold(c, c->cur);
    stage_fold(c, c->cur ^ 1);
    const int n = (int)std::min<size_t>((size_t)std::max(max_calls, 0), c->call_ms.size());
    for (int i = 0; i < n; ++i) ms[i] = c->call_ms[i];
    *n_calls = n;
    c->call_ms.clear();
    return MSPLAT_OK;
}

int msplat_hip_drain_raster_counters(int64_t counts[4]) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!counts) return fail(MSPLAT_ERR_ARG, "null counts");
    for (int k = 0; k < 4; ++k) counts[k] = 0;
    if (!c->timing) return MSPLAT_OK;
    std::vector<unsigned long long> h((size_t)WORK_SLOTS * WORK_SLOT_U64);
    const size_t bytes = h.size() * sizeof(unsigned long long);
    HIP_TRY(hipMemcpyAsync(h.data(), c->work_d.p, bytes, hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    HIP_TRY(hipMemsetAsync(c->work_d.p, 0, bytes, c->stream));
    for (int sl = 0; sl < WORK_SLOTS; ++sl)
        for (int k = 0; k < 4; ++k) counts[k] += (int64_t)h[(size_t)sl * WORK_SLOT_U64 + k];
    return MSPLAT_OK;
}

int msplat_hip_raster_work(int64_t counts[6]) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!counts) return fail(MSPLAT_ERR_ARG, "null counts");
    ENSURE(c->count_d, 64);
    HIP_TRY(hipMemsetAsync(c->count_d.p, 0, 48, c->stream));
    CamParams p{};
    p.W = c->last_W;
    p.H = c->last_H;
    p.tbx = (p.W + BLOCK - 1) / BLOCK;
    p.tby = (p.H + BLOCK - 1) / BLOCK;
    unsigned long long* d = P<unsigned long long>(c->count_d);
    if (c->last_N > 0 && c->meta_d.p)
        launch_raster_work(c->stream, p, c->max_items, P<Meta>(c->meta_d), items(c),
                           P<int>(c->tile_bins), packed(c), P<int>(c->final_idx), chunks(c), d);
    unsigned long long h[6];
    HIP_TRY(hipMemcpyAsync(h, d, sizeof(h), hipMemcpyDeviceToHost, c->stream));
    HIP_TRY(hipStreamSynchronize(c->stream));
    for (int k = 0; k < 6; ++k) counts[k] = (int64_t)h[k];
    return MSPLAT_OK;
}

int msplat_hip_copy_intermediate(const char* name, void* dst, size_t* nbytes) {
    Ctx* c = g_ctx;
    if (!c) return fail(MSPLAT_ERR_NOINIT, "not initialised");
    if (!name || !nbytes) return fail(MSPLAT_ERR_ARG, "null args");
    if (!c->meta_valid) {
        HIP_TRY(hipMemcpyAsync(c->meta_h, c->meta_d.p, sizeof(Meta), hipMemcpyDeviceToHost, c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));
        c->meta = *c->meta_h;
        c->meta_valid = true;
    }
    const size_t N = (size_t)c->last_N, T = (size_t)c->last_T, Px = (size_t)c->last_W * c->last_H;
    const size_t I = (size_t)std::max<int64_t>(c->meta.total_isect, 0);
    const std::string n(name);
    // Direct copies.
    struct D { const char* name; Buf* b; size_t bytes; };
    const D direct[] = {
        {"radii", &c->radii, N * 4},
        {"num_tiles_hit", &c->tiles_hit, N * 4}, {"tile_bins", &c->tile_bins, T * 8},
        {"final_Ts", &c->final_T, Px * 4},
        {"final_index", &c->final_idx, Px * 4}, {"out_img", &c->out_img, Px * 12},
        {"v_rendered", &c->v_rendered, Px * 12}, {"gacc", &c->gacc, N * 36},
        {"tile_done", &c->tile_done, T * 4},
    };
    for (const D& d : direct) {
        if (n != d.name) continue;
        *nbytes = d.bytes;
        if (!dst || d.bytes == 0) return MSPLAT_OK;
        HIP_TRY(hipMemcpyAsync(dst, d.b->p, d.bytes, hipMemcpyDeviceToHost, c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));
        return MSPLAT_OK;
    }
    if (n == "gaussian_ids") {
        *nbytes = I * 4;
        if (!dst || I == 0) return MSPLAT_OK;
        HIP_TRY(hipMemcpyAsync(dst, c->sorted_ids, I * 4, hipMemcpyDeviceToHost, c->stream));
        HIP_TRY(hipStreamSynchronize(c->stream));
        return MSPLAT_OK;
    }
    if (n == "meta") {
        *nbytes = sizeof(Meta);
        if (dst) std::memcpy(dst, &c->meta, sizeof(Meta));
        return MSPLAT_OK;
    }
    // Repacked views of the internal layouts.
    std::vector<float> h;
    // Fields of the 64-byte projection records: (name, floats, record offsets).
    struct F { const char* name; int per; int off[3]; };
    const F fields[] = {{"xys", 2, {0, 1, 0}},       {"conics", 3, {2, 3, 4}},
                        {"opacity_sigmoid", 1, {5, 0, 0}}, {"colors", 3, {6, 7, 8}},
                        {"aabb", 2, {9, 10, 0}},    {"depths", 1, {11, 0, 0}}};
    for (const F& f : fields) {
        if (n != f.name) continue;
        *nbytes = N * f.per * 4;
        if (!dst) return MSPLAT_OK;
        h.resize(N * 16);
        if (N) {
            HIP_TRY(hipMemcpyAsync(h.data(), c->rec.p, N * 64, hipMemcpyDeviceToHost, c->stream));
            HIP_TRY(hipStreamSynchronize(c->stream));
        }
        float* o = static_cast<float*>(dst);
        for (size_t g = 0; g < N; ++g)
            for (int k = 0; k < f.per; ++k) o[g * f.per + k] = h[16 * g + f.off[k]];
        return MSPLAT_OK;
    }
    const int q0 = n == "v_xy" ? 0 : n == "v_conic" ? 2 : n == "v_rgb" ? 5 : n == "v_opacity" ? 8 : -1;
    if (q0 >= 0) {
        const int per = n == "v_xy" ? 2 : n == "v_opacity" ? 1 : 3;
        *nbytes = N * per * 4;
        if (!dst) return MSPLAT_OK;
        h.resize(N * 9);
        const bool need_rec = q0 == 0 || q0 == 5;
        std::vector<float> r(need_rec ? N * 16 : 0);
        if (N) {
            HIP_TRY(hipMemcpyAsync(h.data(), c->gacc.p, N * 36, hipMemcpyDeviceToHost, c->stream));
            if (need_rec)
                HIP_TRY(hipMemcpyAsync(r.data(), c->rec.p, N * 64, hipMemcpyDeviceToHost, c->stream));
            HIP_TRY(hipStreamSynchronize(c->stream));
        }
        float* o = static_cast<float*>(dst);
        for (size_t g = 0; g < N; ++g) {
            const float* a = &h[g * 9];
            if (q0 == 0) {
                // v_xy from the v_sigma moments and the conic (a, b, c) of
                // the record, as the projection backward forms it; gaussians
                // without raster gradient (culled: stale record) give 0
                const float* q = &r[g * 16];
                const bool any = a[0] != 0.f || a[1] != 0.f;
                o[2 * g] = any ? std::fma(q[3], a[1], q[2] * a[0]) : 0.f;
                o[2 * g + 1] = any ? std::fma(q[4], a[1], q[3] * a[0]) : 0.f;
            } else if (q0 == 2) {
                for (int k = 0; k < 3; ++k) o[3 * g + k] = 0.5f * a[2 + k];
            } else if (q0 == 5) {
                // channels whose raw colour + 0.5 < 0 carry no gradient
                const float raw[3] = {r[g * 16 + 6], r[g * 16 + 7], r[g * 16 + 8]};
                for (int k = 0; k < 3; ++k) o[3 * g + k] = raw[k] + 0.5f >= 0.f ? a[5 + k] : 0.f;
            } else {
                for (int k = 0; k < per; ++k) o[g * per + k] = a[q0 + k];
            }
        }
        return MSPLAT_OK;
    }
    return fail(MSPLAT_ERR_ARG, "unknown intermediate '%s'", name);
}

}  // extern "C"
