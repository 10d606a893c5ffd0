// common.hpp — device-side math shared by the gfx950 kernels.
//
// Numerics: every kernel is compiled with -ffp-contract=off and correctly
// rounded fp32 division / sqrt, so a*b+c rounds twice unless written as
// fmaf(), which is used exactly where msplat_metal.metal writes fma().
// exp() is the Cody–Waite / Taylor exp below, built only from +, *, fma and
// integer ops so that it gives the same bits on every IEEE target.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace msp {

constexpr int BLOCK = 16;              // tile edge (msplat.hpp:4-5)
constexpr int TILE_PIX = BLOCK * BLOCK;
constexpr int CHUNK = 512;             // depth chunk (.metal:2616)
// Largest tile rasterised in one piece outside chunk mode: the reference's
// monolithic kernel keeps at most 2048 entries per tile (.metal:2021) and
// drops the rest; tiles of up to 8192 are rasterised in one piece here,
// uncapped, and larger ones in 512-entry chunks.
constexpr int MONO_MAX = 8192;
constexpr int CHUNK_MODE_TILES = 400;  // below this many tiles every tile is chunked (.mm:876)

// SH constants (.metal:14-39).
constexpr float SH_C0 = 0.28209479177387814f;
constexpr float SH_C1 = 0.4886025119029199f;
constexpr float SH_C2_0 = 1.0925484305920792f, SH_C2_1 = -1.0925484305920792f,
                SH_C2_2 = 0.31539156525252005f, SH_C2_3 = -1.0925484305920792f,
                SH_C2_4 = 0.5462742152960396f;
constexpr float SH_C3_0 = -0.5900435899266435f, SH_C3_1 = 2.890611442640554f,
                SH_C3_2 = -0.4570457994644658f, SH_C3_3 = 0.3731763325901154f,
                SH_C3_4 = -0.4570457994644658f, SH_C3_5 = 1.445305721320277f,
                SH_C3_6 = -0.5900435899266435f;

// 11-tap Gaussian (sigma 1.5) of the separable SSIM (.metal:3041-3045).
static constexpr float GAUSS_1D[11] = {
    0.0010283801f, 0.0075987581f, 0.0360007721f, 0.1093606895f, 0.2130055377f, 0.2660117249f,
    0.2130055377f, 0.1093606895f, 0.0360007721f, 0.0075987581f, 0.0010283801f};
constexpr float SSIM_C1 = 0.0001f;
constexpr float SSIM_C2 = 0.0009f;

// exp(x): Cody–Waite reduction x = k ln2 + r with ln2 split into a 16-bit head
// and a tail, degree-7 Taylor polynomial in Horner form, scaling by 2^k via the
// exponent field.  x < -87 -> 0 (no subnormal results), x > 88 -> +inf.
__device__ __forceinline__ float exp_cw(float x) {
    if (x != x) return x;
    if (x < -87.0f) return 0.0f;
    if (x > 88.0f) return __int_as_float(0x7f800000);
    const float k = rintf(x * 1.44269504f);
    float r = fmaf(k, -0.693145751953125f, x);
    r = fmaf(k, -1.42860682e-6f, r);
    float p = 1.98412698e-4f;
    p = fmaf(p, r, 1.38888889e-3f);
    p = fmaf(p, r, 8.33333333e-3f);
    p = fmaf(p, r, 4.16666667e-2f);
    p = fmaf(p, r, 1.66666667e-1f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    const int ki = (int)k;
    return p * __int_as_float((ki + 127) << 23);
}

// exp(x) of the rasteriser's -sigma (x in (-5.55, 0], or NaN): k = rint(x
// log2 e), r = x - k ln2 with one fma (|r| <= ln2/2 up to rounding), a
// degree-6 polynomial whose coefficients come from a Remez exchange for
// least relative error of e^r on [-ln2/2, ln2/2] (rounded to float), and
// p * 2^k by ldexp.  Within 1.02 ulp of exp over [-5.6, 0]; 11 vector
// operations.  NaN propagates; for |x| > 87 the result is unspecified (the
// rasteriser never uses it there).
__device__ __forceinline__ float exp_raster(float x) {
    const float k = rintf(x * 0x1.715476p+0f);
    const float r = fmaf(k, -0x1.62e430p-1f, x);
    float p = 0x1.6ab980p-10f;
    p = fmaf(p, r, 0x1.126d0cp-7f);
    p = fmaf(p, r, 0x1.55589ap-5f);
    p = fmaf(p, r, 0x1.55540ap-3f);
    p = fmaf(p, r, 0x1.fffffap-2f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return ldexpf(p, (int)k);
}

// exp_raster(-s), bit for bit, in a form without a negated operand: with
// r' = -r = fma(k, ln2, s) the Horner steps run on u_j = (-1)^j p_j, since
// fma(u_{j+1}, r', (-1)^j c_j) = (-1)^j fma(p_{j+1}, r, c_j) (round to
// nearest is odd-symmetric; the p_j of |r| <= ln2/2 are far from 0, so no
// signed zero arises).  Every step is then a two-VGPR multiply-add with a
// literal (v_fmamk / v_fmaak), where the negated form needs a three-operand
// fma with the constant in a scalar register.
__device__ __forceinline__ float exp_neg_raster(float s) {
    const float k = rintf(s * -0x1.715476p+0f);
    const float r = fmaf(k, 0x1.62e430p-1f, s);
    float u = 0x1.6ab980p-10f;
    u = fmaf(u, r, -0x1.126d0cp-7f);
    u = fmaf(u, r, 0x1.55589ap-5f);
    u = fmaf(u, r, -0x1.55540ap-3f);
    u = fmaf(u, r, 0x1.fffffap-2f);
    u = fmaf(u, r, -1.0f);
    u = fmaf(u, r, 1.0f);
    return ldexpf(u, (int)k);
}

__device__ __forceinline__ float sigmoid(float o) { return 1.f / (1.f + exp_cw(-o)); }

// float -> int with the operand clamped to [-2^30, 2^30] first: one defined
// result for every input (the plain conversion is undefined out of range).
__device__ __forceinline__ int f2i(float v) {
    return (int)fminf(fmaxf(v, -1073741824.f), 1073741824.f);
}

__device__ __forceinline__ float clamp01(float v) { return fminf(fmaxf(v, 0.f), 1.f); }

// Tile rectangle of a gaussian: get_tile_bbox (.metal:57-87).
__device__ __forceinline__ void tile_rect(float x, float y, float ex, float ey, int tbx, int tby,
                                          int& x0, int& y0, int& x1, int& y1) {
    const float tcx = x / (float)BLOCK, tcy = y / (float)BLOCK;
    const float trx = ex / (float)BLOCK, try_ = ey / (float)BLOCK;
    x0 = min(max(0, f2i(tcx - trx)), tbx);
    x1 = min(max(0, f2i(tcx + trx + 1)), tbx);
    y0 = min(max(0, f2i(tcy - try_)), tby);
    y1 = min(max(0, f2i(tcy + try_ + 1)), tby);
}

// Number of depth chunks a tile with n entries is rasterised in.
__device__ __host__ __forceinline__ int tile_chunks(int n, int num_tiles) {
    if (n <= 0) return 1;
    if (num_tiles < CHUNK_MODE_TILES || n > MONO_MAX) return (n + CHUNK - 1) / CHUNK;
    return 1;
}

// ---------------------------------------------------------------- wave64 ops
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), CTRL, 0xF, 0xF, true));
}

// Lane mask of a predicate over the active lanes.  Takes the condition as a
// bool so that the compare result is used directly (HIP's __ballot takes an
// int and first turns the condition into a 0/1 value).
__device__ __forceinline__ uint64_t wave_ballot(bool p) { return __builtin_amdgcn_ballot_w64(p); }

// Lane masks of single compares (one v_cmp writing an SGPR pair), to be
// combined with scalar ands; lane_of(mask) turns a mask back into the
// per-lane condition without a vector instruction.  Predicates: "u"
// versions are true for NaN operands, as !(a < b) is.
__device__ __forceinline__ uint64_t mask_lt(float a, float b) { return __builtin_amdgcn_fcmpf(a, b, 4); }
__device__ __forceinline__ uint64_t mask_le(float a, float b) { return __builtin_amdgcn_fcmpf(a, b, 5); }
__device__ __forceinline__ uint64_t mask_uge(float a, float b) { return __builtin_amdgcn_fcmpf(a, b, 11); }
__device__ __forceinline__ uint64_t mask_ult(float a, float b) { return __builtin_amdgcn_fcmpf(a, b, 12); }
__device__ __forceinline__ uint64_t mask_ge_i(int a, int b) { return __builtin_amdgcn_sicmp(a, b, 39); }
__device__ __forceinline__ bool lane_of(uint64_t m) { return __builtin_amdgcn_inverse_ballot_w64(m); }

// Index of the lowest set bit of a nonzero wave-uniform mask, cleared from the
// mask: s_ff1 then s_bitset0, two scalar ALU instructions where m &= m - 1
// takes a 64-bit decrement and an and.
__device__ __forceinline__ int pop_low_bit(uint64_t& m) {
    int bit;
    asm volatile("s_ff1_i32_b64 %0, %1\n\ts_bitset0_b64 %1, %0" : "=&s"(bit), "+s"(m));
    return bit;
}

// Sum over the 64 lanes; every lane gets the total.  All lanes must be active.
__device__ __forceinline__ float wave_sum(float v) {
    v += dpp<0xB1>(v);    // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);    // quad_perm [2,3,0,1]
    v += dpp<0x124>(v);   // row_ror:4
    v += dpp<0x128>(v);   // row_ror:8   -> every lane holds its 16-lane row sum
    const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
    const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
    const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
    const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
    return (r0 + r1) + (r2 + r3);
}

// Sum over the 64 lanes, total in lane 63: row sums by row DPP, then the
// gfx9 row_bcast:15 / row_bcast:31 adds carry rows 0..2 into row 3 (rows
// outside the row mask keep their value).  The two masked adds are written
// as assembly because the compiler does not fold a row-masked DPP move into
// the add; the s_nop 1 before each covers the VALU-write -> DPP-read hazard
// (two wait states) and the one after covers a DPP reader that may follow.
// All lanes must be active.
__device__ __forceinline__ float wave_sum_to_last(float v) {
    v += dpp<0xB1>(v);                 // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);                 // quad_perm [2,3,0,1]
    v += dpp<0x124>(v);                // row_ror:4
    v += dpp<0x128>(v);                // row_ror:8  -> row sums
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %0, %0 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %0, %0 row_bcast:31 row_mask:0xc bank_mask:0xf\n\t"
        "s_nop 1"
        : "+v"(v));
    return v;
}

// The same sum with its total written into lane 63 of dst: the last masked
// add goes to dst in row 3, bank 3 only (lanes 60..63: row_mask selects the
// 16-lane row, bank_mask the group of four lanes within it), so lanes 60..62
// of dst receive partial sums and every other lane keeps its dst value.
// All lanes must be active.
__device__ __forceinline__ float wave_sum_into_lane63(float v, float dst) {
    v += dpp<0xB1>(v);                 // quad_perm [1,0,3,2]
    v += dpp<0x4E>(v);                 // quad_perm [2,3,0,1]
    v += dpp<0x124>(v);                // row_ror:4
    v += dpp<0x128>(v);                // row_ror:8  -> row sums
    asm volatile(
        "s_nop 1\n\t"
        "v_add_f32_dpp %1, %1, %1 row_bcast:15 row_mask:0xa bank_mask:0xf\n\t"
        "s_nop 1\n\t"
        "v_add_f32_dpp %0, %1, %1 row_bcast:31 row_mask:0x8 bank_mask:0x8\n\t"
        "s_nop 1"
        : "+v"(dst), "+v"(v));
    return dst;
}

__device__ __forceinline__ int wave_max_i(int v) {
    for (int off = 32; off >= 1; off >>= 1) v = max(v, __shfl_xor(v, off, 64));
    return v;
}

// Loads and stores marked non-temporal (nt): for data touched once here and
// not again before the next step, so that it does not take the place of
// lines that a later kernel reads.
typedef float ntf4 __attribute__((ext_vector_type(4)));
__device__ __forceinline__ float ld_nt(const float* p) { return __builtin_nontemporal_load(p); }
__device__ __forceinline__ float4 ld_nt4(const float* p) {
    const ntf4 v = __builtin_nontemporal_load(reinterpret_cast<const ntf4*>(p));
    return make_float4(v.x, v.y, v.z, v.w);
}
__device__ __forceinline__ void st_nt(float* p, float v) { __builtin_nontemporal_store(v, p); }
__device__ __forceinline__ void st_nt4(float* p, float4 v) {
    __builtin_nontemporal_store(ntf4{v.x, v.y, v.z, v.w}, reinterpret_cast<ntf4*>(p));
}

// Work index of workgroup b < n such that the workgroups of one XCD take
// consecutive indices: the hardware places workgroups on its 8 XCDs round
// robin (XCD b % 8), so XCD x's workgroups x, x + 8, ... get a contiguous
// run of indices.  A bijection of [0, n).
__device__ __forceinline__ int xcd_order(int b, int n) {
    const int x = b & 7, q = n >> 3, rem = n & 7;
    return x * q + min(x, rem) + (b >> 3);
}

__device__ __forceinline__ unsigned lane_id() { return __lane_id(); }

}  // namespace msp
