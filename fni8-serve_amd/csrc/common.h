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

__device__ __forceinline__ uint16_t f2h(float f) {
    return __builtin_bit_cast(uint16_t, (_Float16)f);  // v_cvt_f16_f32, round to nearest even
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
__device__ __forceinline__ bool find_group_tile(const int32_t* __restrict__ seg_off, int E,
                                                int bm, int slot, int& e_out, int& r0,
                                                int& r1) {
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
            return true;
        }
        base += __shfl(incl, 63, 64);
    }
    return false;
}

}  // namespace fni8

// Host-side launch helpers shared by the translation units.
namespace fni8h {
int launch_quant_rowwise(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                         int64_t ldq, float* s, hipStream_t st);
int launch_gemm(const int8_t* aq, int64_t lda, const float* as, const int32_t* row_index,
                int64_t M, int64_t K, const int8_t* w, const float* ws, int64_t N,
                int64_t E, const int32_t* seg_off, const uint16_t* bias, uint16_t* y,
                int64_t ldy, int32_t* acc_out, hipStream_t st);
// Decode (M <= 4) GEMV with the quantization fused in; returns 1 when the
// shape is not taken (the caller then quantizes and runs launch_gemm).
int launch_decode_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                        const float* ws, int64_t N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                        int8_t* xq_out, float* xs_out, int32_t* acc_out, hipStream_t st);
// The same GEMV on pre-quantized activations; returns 1 when not taken.
int launch_decode_q(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                    const int8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                    int64_t ldy, int32_t* acc_out, hipStream_t st);
int launch_tile32(const int8_t* aq, int64_t lda, const float* as, const int32_t* row_index,
                  int64_t M, int64_t K, const int8_t* w, const float* ws, int64_t N, int64_t E,
                  const int32_t* seg_off, const uint16_t* bias, uint16_t* y, int64_t ldy,
                  int32_t* acc_out, hipStream_t st);
int launch_moe_sort(const int32_t* topi, int64_t T, int64_t k, int64_t E, int32_t* seg_off,
                    int32_t* row_token, int32_t* pos, hipStream_t st);
int launch_moe_combine(const uint16_t* yr, int64_t H, const int32_t* topi,
                       const uint16_t* topw, const int32_t* pos, int64_t T, int64_t k,
                       uint16_t* out, hipStream_t st);
void set_error_detail(const char* fmt, ...);
}  // namespace fni8h
