// Tile helpers shared by the 8-wave MFMA GEMM kernels (gemm_tile32.hip,
// gemm_pp.hip): the XCD-aware order of dense tiles and the LDS-staged fp16
// epilogue of a 2 x 4 wave layout of 32x32 accumulator blocks.
#pragma once

#include "common.h"

namespace fni8t {

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// XCD-aware order of the dense tiles: consecutive workgroup ids land on
// different XCDs, so each XCD gets a contiguous band of tiles, walked 8
// m-tiles at a time.
template <int BM, int BN>
__device__ __forceinline__ void dense_tile(int M, int N, int& m0, int& m1, int& n0) {
    const int ntiles_n = (N + BN - 1) / BN;
    const int ntiles_m = (M + BM - 1) / BM;
    const int total = ntiles_m * ntiles_n;
    int bid = blockIdx.x;
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

// LDS bytes the epilogue needs: row scales, column scales, bias as fp32, and
// half the tile as int32 (rows padded by 8 columns).
template <int BM, int BN>
constexpr size_t tile_epilogue_lds() {
    return (size_t)(BM + 2 * BN) * 4 + (size_t)(BM / 2) * (BN + 8) * 4;
}

// Epilogue of the tile kernels (8 waves, 2 x 4): the accumulators go to LDS as
// int32 (half the tile at a time), then every thread streams 16-byte rows back,
// applies fp16(((float)acc * as[m]) * ws[n] (+ bias[n])) with a wave-uniform row
// scale and writes 8 contiguous bytes per lane.  Column scales and the bias
// (converted to fp32 once, which is exact) are staged in LDS and read four at a
// time.  The caller has finished with its LDS stages (a barrier before the call).
// wm: the wave's half of the tile (rows wm*BM/2..); roff, coff: the row (inside
// that half) and column of the wave's first 32x32 block.
template <int BM, int BN, bool GROUPED, bool WRITE_ACC, int FM = BM / 64, int FN = BN / 128>
__device__ __forceinline__ void tile_epilogue(const i32x16 (&acc)[FM][FN], int8_t* smem, int tid,
                                              int lane, int wm, int roff, int coff, int m0, int m1, int n0,
                                              int N, const int32_t* __restrict__ row_index,
                                              const float* __restrict__ as,
                                              const float* __restrict__ wsexp,
                                              const uint16_t* __restrict__ bexp,
                                              uint16_t* __restrict__ y, int64_t ldy,
                                              int32_t* __restrict__ acc_out) {
    constexpr int NT = 512;
    constexpr int HALF = BM / 2;          // rows staged per pass (one wave-row)
    constexpr int OTS = BN + 8;           // int32 row stride of the staging tile
    float* as_l = reinterpret_cast<float*>(smem);
    float* ws_l = as_l + BM;
    float* b_l = ws_l + BN;
    int32_t* ot = reinterpret_cast<int32_t*>(b_l + BN);
    const bool has_bias = bexp != nullptr;
    for (int t = tid; t < BM; t += NT) {
        const int mr = m0 + t;
        float v = 0.f;
        if (mr < m1) v = as[(GROUPED && row_index != nullptr) ? row_index[mr] : mr];
        as_l[t] = v;
    }
    for (int t = tid; t < BN; t += NT) {
        const bool in = n0 + t < N;
        ws_l[t] = in ? wsexp[n0 + t] : 0.f;
        b_l[t] = (in && has_bias) ? fni8::h2f(bexp[n0 + t]) : 0.f;
    }

#pragma unroll
    for (int pass = 0; pass < 2; pass++) {
        if (wm == pass) {
            // lane l, register r of block (i, j): row 8*(r/4) + 4*(l/32) + r%4, col l%32
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 16; r++) {
                        const int row = roff + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
                        const int col = coff + j * 32 + (lane & 31);
                        ot[row * OTS + col] = acc[i][j][r];
                    }
        }
        __syncthreads();
        // stream the staged half: BN/4 chunks of 4 columns per row; a wave covers
        // whole rows, so the row scale is uniform across the wave
        constexpr int CHR = BN / 4;
        for (int c = tid; c < HALF * CHR; c += NT) {
            const int rl = c / CHR, cl = (c % CHR) * 4;
            const int row_t = pass * HALF + rl;
            const int mr = m0 + row_t;
            const int col = n0 + cl;
            if (mr >= m1 || col >= N) continue;
            const i32x4 a4 = *reinterpret_cast<const i32x4*>(ot + rl * OTS + cl);
            const float4 w4 = *reinterpret_cast<const float4*>(ws_l + cl);
            const float asc = as_l[row_t];
            float v[4] = {(float)a4[0] * asc, (float)a4[1] * asc, (float)a4[2] * asc,
                          (float)a4[3] * asc};
            v[0] = v[0] * w4.x;
            v[1] = v[1] * w4.y;
            v[2] = v[2] * w4.z;
            v[3] = v[3] * w4.w;
            if (has_bias) {
                const float4 b4 = *reinterpret_cast<const float4*>(b_l + cl);
                v[0] = v[0] + b4.x;
                v[1] = v[1] + b4.y;
                v[2] = v[2] + b4.z;
                v[3] = v[3] + b4.w;
            }
            uint16_t h[4];
#pragma unroll
            for (int q = 0; q < 4; q++) h[q] = fni8::f2h(v[q]);
            uint16_t* yp = y + (int64_t)mr * ldy + col;
            if (col + 3 < N && ((uintptr_t)yp & 7) == 0) {
                uint2 pk;
                pk.x = h[0] | ((uint32_t)h[1] << 16);
                pk.y = h[2] | ((uint32_t)h[3] << 16);
                *reinterpret_cast<uint2*>(yp) = pk;
            } else {
                for (int q = 0; q < 4 && col + q < N; q++) yp[q] = h[q];
            }
            if constexpr (WRITE_ACC) {
                for (int q = 0; q < 4 && col + q < N; q++) acc_out[(int64_t)mr * N + col + q] = a4[q];
            }
        }
        __syncthreads();
    }
}

}  // namespace fni8t
