// Tile helpers shared by the 8-wave MFMA GEMM kernels (gemm_tile32.hip,
// gemm_pp.hip): the XCD-aware order of dense tiles and the LDS-staged fp16
// epilogue of 32x32 accumulator blocks.
#pragma once

#include <type_traits>

#include "common.h"

namespace fni8t {

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// XCD-aware order of the dense tiles: consecutive workgroup ids land on
// different XCDs, so each XCD gets a contiguous band of tiles, walked 8
// m-tiles at a time.
// `bid` is the tile's number in launch order (the workgroup id when every
// workgroup owns one tile).
template <int BM, int BN>
__device__ __forceinline__ void dense_tile_at(int bid, int M, int N, int& m0, int& m1, int& n0) {
    const int ntiles_n = (N + BN - 1) / BN;
    const int ntiles_m = (M + BM - 1) / BM;
    const int total = ntiles_m * ntiles_n;
    if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
    constexpr int GM = 8;
    const int group = bid / (GM * ntiles_n);
    const int first_m = group * GM;
    const int gsize = min(ntiles_m - first_m, GM);
    const int in_group = bid - group * GM * ntiles_n;
    m0 = (first_m + in_group % gsize) * BM;
    m1 = min(M, m0 + BM);
    n0 = (in_group / gsize) * BN;
}
template <int BM, int BN>
__device__ __forceinline__ void dense_tile(int M, int N, int& m0, int& m1, int& n0) {
    dense_tile_at<BM, BN>(blockIdx.x, M, N, m0, m1, n0);
}

// ---- epilogue ---------------------------------------------------------------
// The kernels issue their MFMAs as D = W * X^T (weight fragment as the A
// operand), so a 32x32 accumulator block of lane l holds token row l % 32 and,
// in registers 4q..4q+3, the four consecutive output columns
// 8q + 4*(l/32) + 0..3.  The epilogue dequantizes in registers,
// fp16(((float)acc * as[m]) * ws[n] (+ bias[n])) with a per-lane row scale,
// stages the fp16 tile in LDS once (8-byte writes), and streams it back as
// 16-byte row chunks.
//
// LDS: the fp16 tile at offset 0 (it overlaps the main loop's stages, which
// are dead by then), and the scales (row scales, column scales, bias as fp32)
// in a region of their own at tile_scale_offset, written before the last
// barrier of the main loop.
template <int BM, int BN>
constexpr size_t tile_stage_lds() {
    return (size_t)BM * BN * 2;
}
template <int BM, int BN>
constexpr size_t tile_scale_lds() {
    return (size_t)(BM + 2 * BN) * 4;
}
// Offset of the scale region given the main loop's LDS bytes; the kernel's LDS
// is tile_scale_offset + tile_scale_lds.
template <int BM, int BN>
constexpr size_t tile_scale_offset(size_t main_lds) {
    return main_lds > tile_stage_lds<BM, BN>() ? main_lds : tile_stage_lds<BM, BN>();
}

// Thread t's share of the scales (row scale of tile row t for t < BM, column
// scale and bias of tile column t for t < BN; 0 past the tile's edge), loaded
// at kernel start so that their latency hides behind the main loop.  Nothing
// uses them before store_tile_scales (the bias stays raw fp16 bits until then,
// and its conversion to fp32 is exact), so no wait is placed on them early.
struct TileScales {
    float a, w;
    uint32_t b;
};
template <int BM, int BN, bool GROUPED>
__device__ __forceinline__ TileScales load_tile_scales(int tid, int m0, int m1, int n0, int N,
                                                       const int32_t* __restrict__ row_index,
                                                       const float* __restrict__ as,
                                                       const float* __restrict__ wsexp,
                                                       const uint16_t* __restrict__ bexp) {
    TileScales v{0.f, 0.f, 0u};
    if (tid < BM && m0 + tid < m1) {
        const int mr = m0 + tid;
        v.a = as[(GROUPED && row_index != nullptr) ? row_index[mr] : mr];
    }
    if (tid < BN && n0 + tid < N) {
        v.w = wsexp[n0 + tid];
        if (bexp != nullptr) v.b = bexp[n0 + tid];
    }
    return v;
}
template <int BM, int BN>
__device__ __forceinline__ void store_tile_scales(const TileScales& v, float* sl, int tid) {
    if (tid < BM) sl[tid] = v.a;
    if (tid < BN) {
        sl[BM + tid] = v.w;
        // converted here, in an instruction the compiler cannot hoist next to
        // the load (which would put a wait for it in front of the main loop)
        float bf;
        asm volatile("v_cvt_f32_f16 %0, %1" : "=v"(bf) : "v"(v.b));
        sl[BM + BN + tid] = bf;
    }
}

// two fp32 -> packed fp16, round to nearest even (the rounding of v_cvt_f16_f32)
__device__ __forceinline__ uint32_t cvt_pk_f16(float lo, float hi) {
    uint32_t r;
    asm("v_cvt_pk_f16_f32 %0, %1, %2" : "=v"(r) : "v"(lo), "v"(hi));
    return r;
}

// 8-byte unit u of staged row r sits at unit u ^ (r & 15): the 16 rows of one
// write pass (lanes 16k..16k+15) land in 16 distinct units of 128 bytes.
// Needs BN % 64 == 0 (whole 16-unit groups per row).
//
// Preconditions: the caller's accumulators are complete, store_tile_scales has
// run, and a workgroup barrier followed both (the main loop's LDS is dead).
// roff, coff: tile-local row and column of the wave's first 32x32 block.
template <int BM, int BN, bool WRITE_ACC, int FM, int FN>
__device__ __forceinline__ void tile_epilogue(const i32x16 (&acc)[FM][FN], int8_t* smem,
                                              const float* sl, int tid, int lane, int roff,
                                              int coff, int m0, int m1, int n0, int N,
                                              bool has_bias, uint16_t* __restrict__ y,
                                              int64_t ldy, int32_t* __restrict__ acc_out) {
    static_assert(BN % 64 == 0, "staging swizzle works on 128-byte groups");
    constexpr int NT = 512;
    constexpr int RS = BN * 2;  // bytes per staged row
    const float* as_l = sl;
    const float* ws_l = sl + BM;
    const float* b_l = sl + BM + BN;
    uint8_t* st = reinterpret_cast<uint8_t*>(smem);
    const int lr = lane & 31, lh = lane >> 5;
    // roff is a multiple of 32, so the lane's staged rows all share the swizzle
    // lr & 15, and its write offsets depend on (j, q) only
    const int sw = lr & 15;
    uint8_t* wbase = st + (roff + lr) * RS;
    int woff[FN][4];
#pragma unroll
    for (int j = 0; j < FN; j++)
#pragma unroll
        for (int q = 0; q < 4; q++)
            woff[j][q] = ((((coff + j * 32 + 8 * q + 4 * lh) >> 2) ^ sw) << 3);
    auto convert = [&](auto bias_c) {
        constexpr bool BIAS = decltype(bias_c)::value;
        // column scales (and bias) of the lane's 4*FN*4 columns, read once
        float4 w4[FN][4], b4[FN][4];
#pragma unroll
        for (int j = 0; j < FN; j++)
#pragma unroll
            for (int q = 0; q < 4; q++) {
                const int col = coff + j * 32 + 8 * q + 4 * lh;
                w4[j][q] = *reinterpret_cast<const float4*>(ws_l + col);
                if constexpr (BIAS) b4[j][q] = *reinterpret_cast<const float4*>(b_l + col);
            }
#pragma unroll
        for (int i = 0; i < FM; i++) {
            const int row = roff + i * 32 + lr;
            const float asc = as_l[row];
#pragma unroll
            for (int j = 0; j < FN; j++)
#pragma unroll
                for (int q = 0; q < 4; q++) {
                    float v0 = (float)acc[i][j][4 * q + 0] * asc;
                    float v1 = (float)acc[i][j][4 * q + 1] * asc;
                    float v2 = (float)acc[i][j][4 * q + 2] * asc;
                    float v3 = (float)acc[i][j][4 * q + 3] * asc;
                    v0 = v0 * w4[j][q].x;
                    v1 = v1 * w4[j][q].y;
                    v2 = v2 * w4[j][q].z;
                    v3 = v3 * w4[j][q].w;
                    if constexpr (BIAS) {
                        v0 = v0 + b4[j][q].x;
                        v1 = v1 + b4[j][q].y;
                        v2 = v2 + b4[j][q].z;
                        v3 = v3 + b4[j][q].w;
                    }
                    uint2 pk;
                    pk.x = cvt_pk_f16(v0, v1);
                    pk.y = cvt_pk_f16(v2, v3);
                    *reinterpret_cast<uint2*>(wbase + i * 32 * RS + woff[j][q]) = pk;
                    if constexpr (WRITE_ACC) {
                        const int mr = m0 + row, n = n0 + coff + j * 32 + 8 * q + 4 * lh;
                        if (mr < m1) {
                            int32_t* ap = acc_out + (int64_t)mr * N + n;
#pragma unroll
                            for (int t = 0; t < 4; t++)
                                if (n + t < N) ap[t] = acc[i][j][4 * q + t];
                        }
                    }
                }
        }
    };
    if (has_bias)
        convert(std::true_type{});
    else
        convert(std::false_type{});
    __syncthreads();

    constexpr int CPR = BN / 8;  // 16-byte chunks per row
    // one 16-byte chunk back from LDS in logical order (the two 8-byte units of
    // an odd-swizzled row come back swapped)
    auto fetch = [&](int row, int k) {
        const int rsw = row & 15;
        uint4 v = *reinterpret_cast<const uint4*>(st + row * RS + (((2 * k) ^ (rsw & 14)) << 3));
        if (rsw & 1) {
            const uint32_t x0 = v.x, x1 = v.y;
            v.x = v.z;
            v.y = v.w;
            v.z = x0;
            v.w = x1;
        }
        return v;
    };
    auto put = [&](uint16_t* yp, int col, uint4 v) {
        if (col + 7 < N && ((uintptr_t)yp & 15) == 0) {
            *reinterpret_cast<uint4*>(yp) = v;
        } else {
            const uint32_t w32[4] = {v.x, v.y, v.z, v.w};
            for (int t = 0; t < 8 && col + t < N; t++)
                yp[t] = (uint16_t)(w32[t >> 1] >> (16 * (t & 1)));
        }
    };
    if constexpr (NT % CPR == 0 && (NT / CPR) % 16 == 0) {
        // each thread keeps one column chunk and steps by NT/CPR rows (a
        // multiple of 16, so its swizzle is fixed)
        constexpr int RSTEP = NT / CPR;
        const int k = tid % CPR, r0 = tid / CPR;
        const int col = n0 + k * 8;
        if (col < N) {
            uint16_t* yp = y + (int64_t)(m0 + r0) * ldy + col;
#pragma unroll
            for (int it = 0; it < BM / RSTEP; it++) {
                const int row = r0 + it * RSTEP;
                if (m0 + row < m1) put(yp, col, fetch(row, k));
                yp += (int64_t)RSTEP * ldy;
            }
        }
    } else {
        for (int c = tid; c < BM * CPR; c += NT) {
            const int row = c / CPR, k = c % CPR;
            const int mr = m0 + row, col = n0 + k * 8;
            if (mr >= m1 || col >= N) continue;
            put(y + (int64_t)mr * ldy + col, col, fetch(row, k));
        }
    }
}

}  // namespace fni8t
