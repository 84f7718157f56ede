// Shared device helpers for the gfx950 W8A8 kernels.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/fni8amd.h"

typedef int32_t i32x4 __attribute__((ext_vector_type(4)));

// Every float operation below rounds once: no contraction into FMA (the
// library is also built with -ffp-contract=off and correctly rounded fp32 division).
#pragma clang fp contract(off)

#define FNI8_QUANT_EPS 1e-6f
#define FNI8_QMAX 127.0f

namespace fni8 {

// 16x16x64 int8 MFMA (CDNA4).  srcA lane l carries 16 int8 of row (l % 16),
// srcB lane l carries 16 int8 of column (l % 16); both use the same k subset,
// chosen by (l / 16).  Result lane l, register r holds D[4*(l/16) + r][l % 16].
__device__ __forceinline__ i32x4 mfma_i8(i32x4 a, i32x4 b, i32x4 c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ float h2f(uint16_t h) {
    return (float)__builtin_bit_cast(_Float16, h);
}

// fp32 -> fp16, round to nearest even.  Emitted as its own v_cvt_f16_f32 so the
// compiler cannot fold a preceding multiply into a mixed-precision FMA (whose
// +0 addend would turn a -0 product into +0).
__device__ __forceinline__ uint16_t f2h(float f) {
    uint32_t r;
    asm("v_cvt_f16_f32 %0, %1" : "=v"(r) : "v"(f));
    return (uint16_t)(r & 0xffffu);
}

// Row scale from the max fp16 magnitude bits of the row.  Integer max over
// (bits & 0x7fff) orders every finite value, inf and NaN correctly, so a NaN
// anywhere in the row propagates into the scale (torch.amax semantics).
__device__ __forceinline__ float row_scale_from_bits(uint32_t amax_bits) {
    float amax = h2f((uint16_t)amax_bits);
    if (amax != amax) return amax;
    return (amax > FNI8_QUANT_EPS ? amax : FNI8_QUANT_EPS) / FNI8_QMAX;
}

// q = clamp(rint(x / s), -127, 127); a NaN quotient quantizes to 0.
__device__ __forceinline__ int32_t quant_one(float x, float s) {
    float v = x / s;
    if (v != v) return 0;
    v = __builtin_rintf(v);
    v = v > FNI8_QMAX ? FNI8_QMAX : v;
    v = v < -FNI8_QMAX ? -FNI8_QMAX : v;
    return (int32_t)v;
}

// y = fp16(((float)acc * as) * ws (+ bias)), one rounding per operation.
__device__ __forceinline__ uint16_t dequant_one(int32_t acc, float as, float ws,
                                                const uint16_t* bias, int n) {
    float v = (float)acc * as;
    v = v * ws;
    if (bias) v = v + h2f(bias[n]);
    return f2h(v);
}

// exp(x) for x in [-86, 88].  Cody-Waite reduction x = k ln2 + r, |r| <= ln2/2,
// with ln2 split into a 15-bit head (k * head is exact for |k| <= 127) and a
// tail; exp(r) by its degree-7 Taylor polynomial in Horner form (truncation
// below 0.14 ulp on the interval); 2^k applied through the exponent field
// (k + 127 stays in [3, 254], so the result is a normal number).
__device__ __forceinline__ float exp_cw(float x) {
    const float k = __builtin_rintf(x * 0x1.715476p+0f);
    float r = __builtin_fmaf(-k, 0x1.62e4p-1f, x);
    r = __builtin_fmaf(-k, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;              // 1/7!
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);  // 1/6!
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);   // 1/5!
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);   // 1/4!
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);   // 1/3!
    p = __builtin_fmaf(p, r, 0.5f);
    p = __builtin_fmaf(p, r, 1.0f);
    p = __builtin_fmaf(p, r, 1.0f);
    const float two_k = __builtin_bit_cast(float, (uint32_t)((int)k + 127) << 23);
    return p * two_k;
}

// ---- wave reductions and the division-free quantization --------------------
// DPP lane permutations (gfx9 encodings).
constexpr int kDppXor1 = 0xB1;         // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;         // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141;  // lane i <-> 7-i within 8
constexpr int kDppMirror = 0x140;      // lane i <-> 15-i within 16

template <int CTRL>
__device__ __forceinline__ int dpp(int v) {
    return __builtin_amdgcn_update_dpp(v, v, CTRL, 0xf, 0xf, false);
}

// Sum over each group of 8 consecutive lanes; every lane of the group gets it.
__device__ __forceinline__ int sum8(int v) {
    v += dpp<kDppXor1>(v);
    v += dpp<kDppXor2>(v);
    v += dpp<kDppHalfMirror>(v);
    return v;
}

// Max over the wave of non-negative values, returned as a wave-uniform value.
__device__ __forceinline__ uint32_t wave_max_uniform(uint32_t v) {
    int t = (int)v;
    int o;
    o = dpp<kDppXor1>(t); t = o > t ? o : t;
    o = dpp<kDppXor2>(t); t = o > t ? o : t;
    o = dpp<kDppHalfMirror>(t); t = o > t ? o : t;
    o = dpp<kDppMirror>(t); t = o > t ? o : t;
    int a = __builtin_amdgcn_readlane(t, 0), b = __builtin_amdgcn_readlane(t, 16);
    int c = __builtin_amdgcn_readlane(t, 32), d = __builtin_amdgcn_readlane(t, 48);
    a = a > b ? a : b;
    c = c > d ? c : d;
    return (uint32_t)(a > c ? a : c);
}

// q for one fp16 value given the row's finite scale s and yr = fl(1/s)
// (correctly rounded): t = fl(x*yr), r = fma(-t, s, x) is exact, and
// fma(r, yr, t) == fl(x/s) for every non-zero fp16 |x| <= amax (Markstein's
// correction; checked exhaustively over all fp16 (x, amax) pairs by the CPU
// test suite), so rint of it equals quant_one's rint(x / s).
//
// The rounding to an integer is one addition: for |v| < 2^22, adding
// 1.5 * 2^23 rounds v to the nearest integer, ties to even (the default
// rounding mode), and leaves it in the low bits of the sum as a two's
// complement value.  No clamp is needed: |x| <= amax and s = fl(amax / 127)
// (or eps / 127 > amax / 127) keep |v| <= 127 * (1 + 2^-23) < 127.5.
__device__ __forceinline__ uint32_t quant_fast(float x, float s, float yr) {
    const float t = x * yr;
    const float r = __builtin_fmaf(-t, s, x);
    const float v = __builtin_fmaf(r, yr, t);
    return __builtin_bit_cast(uint32_t, v + 12582912.0f) & 0xffu;
}

// t = fl(h * yr) for the fp16 value in half HI of `packed`, as one v_fma_mix_f32
// with a -0 addend: fma(h, yr, -0) rounds h * yr once and keeps the sign of a
// zero product, so it is bitwise the product, without a separate f16 -> f32
// conversion.
template <int HI>
__device__ __forceinline__ float mul_half(uint32_t packed, float yr) {
    float t;
    if constexpr (HI)
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[1,0,0] op_sel_hi:[1,0,0]"
            : "=v"(t) : "v"(packed), "v"(yr), "v"(-0.0f));
    else
        asm("v_fma_mix_f32 %0, %1, %2, %3 op_sel:[0,0,0] op_sel_hi:[1,0,0]"
            : "=v"(t) : "v"(packed), "v"(yr), "v"(-0.0f));
    return t;
}

// quant_fast for half HI of `packed`; the low byte of the result is q (the
// upper bytes hold the rounding constant and are discarded by the packing).
template <int HI>
__device__ __forceinline__ uint32_t quant_half(uint32_t packed, float s, float yr) {
    const float x = h2f((uint16_t)(HI ? packed >> 16 : packed & 0xffffu));
    const float t = mul_half<HI>(packed, yr);
    const float r = __builtin_fmaf(-t, s, x);  // emitted as v_fma_mix_f32 on the fp16 x
    const float v = __builtin_fmaf(r, yr, t);
    return __builtin_bit_cast(uint32_t, v + 12582912.0f);
}

// Low bytes of four words -> one word (b0 | b1 << 8 | b2 << 16 | b3 << 24),
// three byte permutes.
__device__ __forceinline__ uint32_t pack_low_bytes(uint32_t b0, uint32_t b1, uint32_t b2,
                                                   uint32_t b3) {
    const uint32_t p01 = __builtin_amdgcn_perm(b1, b0, 0x0c0c0400u);
    const uint32_t p23 = __builtin_amdgcn_perm(b3, b2, 0x0c0c0400u);
    return __builtin_amdgcn_perm(p23, p01, 0x05040100u);
}

// 8 fp16 (one 16-byte chunk) -> 8 int8; zeros unless `live` (finite scale, real row).
// About 4.75 VALU operations per element: two mixed-precision FMAs, one FMA,
// one addition, and 3/4 of a byte permute.
__device__ __forceinline__ uint2 quant_chunk(uint4 v, float s, float yr, bool live) {
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
    uint32_t out[2];
#pragma unroll
    for (int i = 0; i < 2; i++) {
        const uint32_t a = w4[2 * i], b = w4[2 * i + 1];
        const uint32_t q = pack_low_bytes(quant_half<0>(a, s, yr), quant_half<1>(a, s, yr),
                                          quant_half<0>(b, s, yr), quant_half<1>(b, s, yr));
        out[i] = live ? q : 0u;
    }
    return make_uint2(out[0], out[1]);
}

// Running max of fp16 magnitude bits, two halves at a time: m holds two
// 16-bit maxima (v_pk_max_u16 over (w & 0x7fff7fff)); amax_fold gives the row's.
typedef unsigned short u16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t amax_step(uint32_t m, uint32_t w) {
    const u16x2 a = __builtin_bit_cast(u16x2, m);
    const u16x2 b = __builtin_bit_cast(u16x2, w & 0x7fff7fffu);
    return __builtin_bit_cast(uint32_t, __builtin_elementwise_max(a, b));
}
__device__ __forceinline__ uint32_t amax_chunk(uint32_t m, uint4 v) {
    return amax_step(amax_step(amax_step(amax_step(m, v.x), v.y), v.z), v.w);
}
__device__ __forceinline__ uint32_t amax_fold(uint32_t m) {
    const uint32_t lo = m & 0xffffu, hi = m >> 16;
    return lo > hi ? lo : hi;
}

__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
        uint32_t o = (uint32_t)__shfl_xor((int)v, off, 64);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ int wave_sum_i32(int v) {
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) v += __shfl_xor(v, off, 64);
    return v;
}

__device__ __forceinline__ int wave_incl_scan_i32(int v, int lane) {
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
        int o = __shfl_up(v, off, 64);
        if (lane >= off) v += o;
    }
    return v;
}

// Grouped GEMM tile lookup: expert segments seg_off[E+1] are cut into tiles of
// `bm` rows; tile `slot` (counted over all experts in order) is located by one
// wave with a running prefix over chunks of 64 experts.  Returns false when
// `slot` is past the last tile.  Every lane of the wave gets the same answer.
// Rows are bounded by `rows` (the caller's allocation): a tile starting at or
// beyond it is dropped and r1 is clamped to it, so a seg_off whose last entry
// exceeds the buffers loses rows instead of reading or writing past them.
__device__ __forceinline__ bool find_group_tile(const int32_t* __restrict__ seg_off, int E,
                                                int bm, int slot, int rows, int& e_out,
                                                int& r0, int& r1) {
    const int lane = threadIdx.x & 63;
    int base = 0;
    for (int c = 0; c < E; c += 64) {
        int e = c + lane;
        int lo = 0, hi = 0;
        if (e < E) {
            lo = seg_off[e];
            hi = seg_off[e + 1];
        }
        int tiles = (hi - lo + bm - 1) / bm;
        int incl = wave_incl_scan_i32(tiles, lane);
        int excl = incl - tiles;
        bool mine = (e < E) && (slot >= base + excl) && (slot < base + incl);
        unsigned long long bal = __ballot(mine);
        if (bal) {
            int src = __builtin_ctzll(bal);
            int eo = __shfl(e, src, 64);
            int lo_s = __shfl(lo, src, 64);
            int hi_s = __shfl(hi, src, 64);
            int ex_s = __shfl(excl, src, 64);
            e_out = eo;
            r0 = lo_s + (slot - base - ex_s) * bm;
            r1 = r0 + bm < hi_s ? r0 + bm : hi_s;
            r1 = r1 < rows ? r1 : rows;
            return r0 >= 0 && r0 < r1;
        }
        base += __shfl(incl, 63, 64);
    }
    return false;
}

// Grouped GEMM work lookup in XCD order.  The work is every (expert e, n-tile
// j, row tile r of e's segment), listed expert by expert, n-tile by n-tile,
// row tile fastest: the row tiles that share one expert's weight tile are
// neighbours, and one expert's n-tiles share its activation rows.  Workgroup i
// of a 1-D grid runs on XCD i % 8 (the round-robin dispatch over the eight
// XCDs), so item = remap(i) gives XCD x the contiguous run of items
// [x*q + min(x, rem), ...) (q = W / 8, rem = W % 8 for W items): an expert's
// weight and activation tiles are fetched into that XCD's L2 once and reused
// there, instead of by up to eight L2s.  The remap is a bijection on [0, W),
// so the result does not depend on the dispatch.  W is bounded by the grid (a
// seg_off beyond the launch's bound loses its last items) and rows as in
// find_group_tile.  Every lane of the wave gets the same answer; false past
// the last item.
__device__ __forceinline__ bool find_group_item(const int32_t* __restrict__ seg_off, int E,
                                                int bm, int ntn, int rows, int& e_out,
                                                int& r0, int& r1, int& j_out) {
    const int lane = threadIdx.x & 63;
    // One pass of loads: up to 4 chunks of 64 experts (E <= 256) stay in
    // registers for the search, so the search needs no second round trip.
    constexpr int CH = 4;
    int lo[CH], hi[CH], items[CH], incl[CH], cbase[CH];
    int W = 0;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int e = c * 64 + lane;
        lo[c] = 0;
        hi[c] = 0;
        if (e < E) {
            lo[c] = seg_off[e];
            hi[c] = seg_off[e + 1];
        }
        const int tiles = hi[c] > lo[c] ? (hi[c] - lo[c] + bm - 1) / bm : 0;
        items[c] = tiles * ntn;
        incl[c] = wave_incl_scan_i32(items[c], lane);
        cbase[c] = W;
        W += __shfl(incl[c], 63, 64);
    }
    for (int c = CH * 64; c < E; c += 64) {  // E > 256: the rest, counted only
        const int e = c + lane;
        int t = 0;
        if (e < E) {
            const int l = seg_off[e], h = seg_off[e + 1];
            t = h > l ? (h - l + bm - 1) / bm : 0;
        }
        W += wave_sum_i32(t) * ntn;
    }
    W = W < (int)gridDim.x ? W : (int)gridDim.x;
    const int i = blockIdx.x;
    if (i >= W) return false;
    const int q = W >> 3, rem = W & 7, x = i & 7;
    const int item = x * q + (x < rem ? x : rem) + (i >> 3);
    auto take = [&](int e, int l, int h, int its, int ex, int base) {
        const int tiles = its / ntn;
        const int local = item - base - ex;
        e_out = e;
        j_out = local / tiles;
        r0 = l + (local % tiles) * bm;
        r1 = r0 + bm < h ? r0 + bm : h;
        r1 = r1 < rows ? r1 : rows;
        return r0 >= 0 && r0 < r1;
    };
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int excl = incl[c] - items[c];
        const bool mine = (c * 64 + lane < E) && (item >= cbase[c] + excl) &&
                          (item < cbase[c] + incl[c]);
        const unsigned long long bal = __ballot(mine);
        if (bal) {
            const int src = __builtin_ctzll(bal);
            return take(c * 64 + src, __shfl(lo[c], src, 64), __shfl(hi[c], src, 64),
                        __shfl(items[c], src, 64), __shfl(excl, src, 64), cbase[c]);
        }
    }
    int base = cbase[CH - 1] + __shfl(incl[CH - 1], 63, 64);
    for (int c = CH * 64; c < E; c += 64) {
        const int e = c + lane;
        int l = 0, h = 0;
        if (e < E) {
            l = seg_off[e];
            h = seg_off[e + 1];
        }
        const int its = (h > l ? (h - l + bm - 1) / bm : 0) * ntn;
        const int inc = wave_incl_scan_i32(its, lane);
        const int excl = inc - its;
        const bool mine = (e < E) && (item >= base + excl) && (item < base + inc);
        const unsigned long long bal = __ballot(mine);
        if (bal) {
            const int src = __builtin_ctzll(bal);
            return take(c + src, __shfl(l, src, 64), __shfl(h, src, 64), __shfl(its, src, 64),
                        __shfl(excl, src, 64), base);
        }
        base += __shfl(inc, 63, 64);
    }
    return false;
}

}  // namespace fni8

// Host-side launch helpers shared by the translation units.
namespace fni8h {
int launch_quant_rowwise(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                         int64_t ldq, float* s, hipStream_t st);
// `work` (work_bytes, 256-byte aligned; may be NULL) lets a dense prefill GEMM
// split K across workgroups.
int launch_gemm(const int8_t* aq, int64_t lda, const float* as, const int32_t* row_index,
                int64_t M, int64_t K, const int8_t* w, const float* ws, int64_t N,
                int64_t E, const int32_t* seg_off, const uint16_t* bias, uint16_t* y,
                int64_t ldy, int32_t* acc_out, hipStream_t st, int8_t* work = nullptr,
                int64_t work_bytes = 0);
// Decode (M <= 4) GEMV with the quantization fused in; returns 1 when the
// shape is not taken (the caller then quantizes and runs launch_gemm).
int launch_decode_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                        const float* ws, int64_t N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                        int8_t* xq_out, float* xs_out, int32_t* acc_out, hipStream_t st);
// The same GEMV on pre-quantized activations; returns 1 when not taken.
int launch_decode_q(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                    const int8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                    int64_t ldy, int32_t* acc_out, hipStream_t st);
// Decode GEMM on MFMA, fp16 activations quantized in the kernel (M <= 4, one
// launch); xq_out (row stride K) and xs_out receive the quantized activations.
// Returns 1 when not taken.
int launch_decode_mfma_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                             const int8_t* w, const float* ws, int64_t N, const uint16_t* bias,
                             uint16_t* y, int64_t ldy, int8_t* xq_out, float* xs_out,
                             int32_t* acc_out, hipStream_t st);
// Grouped expert GEMM on MFMA for small segments (<= 48 rows per expert on
// average); returns 1 when not taken.
int launch_decode_mfma_grouped(const int8_t* aq, int64_t lda, const float* as,
                               const int32_t* row_index, int64_t R_max, int64_t K,
                               const int8_t* w, const float* ws, int64_t E, int64_t N,
                               const int32_t* seg_off, const uint16_t* bias, uint16_t* y,
                               int64_t ldy, int32_t* acc_out, hipStream_t st);
// Decode linear for 5 <= M <= 16 in one launch, the quantization shared per XCD
// through `work`; returns 1 when not taken (the caller then uses two launches).
int64_t coop_workspace_bytes(int64_t M, int64_t N, int64_t K);
void set_coop_wait_ticks(int64_t ticks);
// The bound (100 MHz real-time ticks) on a GEMM workgroup's wait for the rows
// its XCD's producers publish.
uint64_t xcd_wait_ticks();
int launch_decode_coop(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                       const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                       int64_t ldy, int8_t* xq_out, float* xs_out, int32_t* acc_out,
                       int8_t* work, int64_t work_bytes, hipStream_t st);
// Decode GEMM (M <= 64, pre-quantized activations) on MFMA; returns 1 when not taken.
int launch_decode_mfma(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                       const int8_t* w, const float* ws, int64_t N, const uint16_t* bias,
                       uint16_t* y, int64_t ldy, int32_t* acc_out, hipStream_t st);
int launch_tile32(const int8_t* aq, int64_t lda, const float* as, const int32_t* row_index,
                  int64_t M, int64_t K, const int8_t* w, const float* ws, int64_t N, int64_t E,
                  const int32_t* seg_off, const uint16_t* bias, uint16_t* y, int64_t ldy,
                  int32_t* acc_out, hipStream_t st);
// Dense prefill GEMM, two wave groups taking turns at MFMA and memory work
// (K % 128 == 0); returns 1 when not taken.  With a workspace of at least
// pp_workspace_bytes(M, N, K) bytes it may split K over workgroups.
int launch_pp(const int8_t* aq, int64_t lda, const float* as, int64_t M, int64_t K,
              const int8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
              int64_t ldy, int32_t* acc_out, int8_t* work, int64_t work_bytes, hipStream_t st);
int64_t pp_workspace_bytes(int64_t M, int64_t N, int64_t K);
// Forces the prefill GEMM's tile (bm x bn) and split-K factor where the shape
// allows it; bm = 0 restores the automatic choice.
void set_gemm_plan(int64_t bm, int64_t bn, int64_t split);
int launch_moe_sort(const int32_t* topi, int64_t T, int64_t k, int64_t E, int32_t* seg_off,
                    int32_t* row_token, int32_t* pos, hipStream_t st);
int launch_moe_combine(const uint16_t* yr, int64_t H, const int32_t* topi,
                       const uint16_t* topw, const int32_t* pos, int64_t T, int64_t k,
                       uint16_t* out, hipStream_t st);
int launch_act_and_mul(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, int act,
                       uint16_t* out, int64_t ldo, hipStream_t st);
// With a workspace of act_quant_workspace_bytes(M, I) bytes (256-byte aligned),
// few rows are split over several workgroups each; NULL = one workgroup a row.
int launch_act_and_mul_quant(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, int act,
                             int8_t* q, int64_t ldq, float* s, int8_t* work, int64_t work_bytes,
                             hipStream_t st);
int64_t act_quant_workspace_bytes(int64_t M, int64_t I);
// RMSNorm; with q non-NULL the normed row is quantized into q/s instead of
// being written to out.  res_out receives x + res (only with res).
int launch_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* res, int64_t ldr,
                   const uint16_t* w, float eps, int unit, int64_t M, int64_t K, uint16_t* out,
                   int64_t ldo, uint16_t* res_out, int64_t ldro, int8_t* q, int64_t ldq,
                   float* s, hipStream_t st);
int launch_gemm_w4a8(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                     const uint8_t* w, const float* ws, int64_t N, int64_t G,
                     const uint16_t* bias, uint16_t* y, int64_t ldy, hipStream_t st);
// W4A8 decode (M <= 4) with the quantization fused in; 1 when not taken.
int launch_linear_w4a8_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                             const uint8_t* w, const float* ws, int64_t N, int64_t G,
                             const uint16_t* bias, uint16_t* y, int64_t ldy, int8_t* xq_out,
                             float* xs_out, hipStream_t st);
// W4A8 decode on MFMA (2 <= M <= 4) with the quantization fused in; xq_out
// (row stride K) and xs_out receive the quantized activations.  1 when not taken.
int launch_linear_w4a8_mfma_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                                  const uint8_t* w, const float* ws, int64_t N, int64_t G,
                                  const uint16_t* bias, uint16_t* y, int64_t ldy,
                                  int8_t* xq_out, float* xs_out, hipStream_t st);
// W4A8 decode GEMM (9 <= M <= 64, wide N) with the weight rows split over the
// waves and one shared activation tile; 1 when not taken.
int launch_w4a8_rowblock(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                         const uint8_t* w, const float* ws, int64_t N, int64_t G,
                         const uint16_t* bias, uint16_t* y, int64_t ldy, hipStream_t st);
// Grouped W4A8 GEMM over expert segments (K % 256 == 0, G in {64, 128, 256}).
int launch_gemm_w4a8_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                             int64_t R_max, int64_t K, const uint8_t* w, const float* ws,
                             int64_t E, int64_t N, int64_t G, const int32_t* seg_off,
                             const uint16_t* bias, uint16_t* y, hipStream_t st);
// The W4A8 tile kernel in its expert-segment form (128-row segment tiles).
int launch_w4a8_tile_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                             int64_t R_max, int64_t K, const uint8_t* w, const float* ws,
                             int64_t E, int64_t N, int64_t G, const int32_t* seg_off,
                             const uint16_t* bias, uint16_t* y, hipStream_t st);
int launch_moe_route(const float* logits, int64_t ldl, int64_t T, int64_t E, int scoring,
                     const float* bias, int64_t groups, int64_t topk_group, int64_t k, int renorm,
                     float scale, uint16_t* topw, int32_t* topi, hipStream_t st);
void set_error_detail(const char* fmt, ...);
}  // namespace fni8h
