// Decode GEMM for 4 < M <= 64 tokens on pre-quantized int8 activations (gfx950).
//
//   y[m, n] = fp16(((float)sum_k xq[m, k] * w[n, k]) * xs[m] * ws[n] (+ bias[n]))
//
// Still HBM-bound (the weight stream is N*K bytes against M*K of activations),
// but with M up to 64 the products belong on MFMA.  Layout of the work:
//   * A workgroup owns 16*NB weight rows; its WAVES waves split K into equal
//     shares of 128-byte slabs.
//   * Weights stream with the coalesced pattern of the decode GEMV: each wave
//     load instruction covers 8 rows x 128 contiguous bytes (lane l: row l/8,
//     bytes 16*(l%8) of the slab), non-temporal, register double-buffered one
//     batch of SB slabs ahead.  That lane layout is not the MFMA operand
//     layout, so every slab goes through a wave-private LDS tile (16-byte
//     chunks XOR-swizzled by row, conflict-free both ways) and comes back as
//     the B fragments of v_mfma_i32_16x16x64_i8 (lane l: row l%16, bytes
//     16*(l/16) of a 64-byte half-slab).
//   * The activation fragments (A operand, lane l: token l%16 of an MT tile,
//     same bytes) are read from L2 and prefetched with the weights.
//   * Two accumulator sets (one per half-slab) break the MFMA dependency
//     chain; waves meet once at the end in an LDS reduction, then the fp16
//     epilogue.
// Integer accumulation is exact, so the result does not depend on the K split.
#include "common.h"

namespace {

__device__ __forceinline__ i32x4 ld16(const int8_t* p) {
    return *reinterpret_cast<const i32x4*>(p);
}
__device__ __forceinline__ i32x4 ld16_nt(const int8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
}

// 16-byte chunk position of (row, chunk) inside a 128-byte row of an LDS tile.
__device__ __forceinline__ int swz(int row, int chunk) {
    return ((chunk ^ (row & 7) ^ ((row >> 3) & 7)) & 7) * 16;
}

template <int MT, int NB, int WAVES, int SB>
__global__ __launch_bounds__(WAVES * 64) void decode_mfma_kernel(
    const int8_t* __restrict__ xq, int64_t ldx, const float* __restrict__ xs, int M, int K,
    const int8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out) {
    constexpr int ROWS = 16 * NB;
    constexpr int TILE = ROWS * 128;  // one slab of the wave's rows
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    i32x4* red = reinterpret_cast<i32x4*>(smem);  // after the main loop: [WAVES][MT*NB][64]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * ROWS;
    const int per = (K >> 7) / WAVES;  // slabs per wave (exact: the launcher checks)
    const int s0 = wave * per, nb = per / SB;

    // load side: lane -> (row rq + 8h, chunk c)
    const int rq = lane >> 3, c = lane & 7;
    const int8_t* wsrc[2 * NB];
    int woff[2 * NB];
#pragma unroll
    for (int h = 0; h < 2 * NB; h++) {
        const int row = h * 8 + rq;
        int n = n0 + row;
        n = n < N ? n : N - 1;  // rows past N load real memory, never stored
        wsrc[h] = w + (int64_t)n * K + (int64_t)s0 * 128 + c * 16;
        woff[h] = row * 128 + swz(row, c);
    }
    // MFMA side: lane -> (row r, chunk 4q + g)
    const int r = lane & 15, g = lane >> 4;
    int roff[NB][2];
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
        for (int q = 0; q < 2; q++) roff[b][q] = (b * 16 + r) * 128 + swz(b * 16 + r, 4 * q + g);
    const int8_t* xrow[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        int m = mt * 16 + r;
        m = m < M ? m : M - 1;  // tokens past M compute into rows never stored
        xrow[mt] = xq + (int64_t)m * ldx + (int64_t)s0 * 128 + g * 16;
    }

    i32x4 wa[SB][2 * NB], wb[SB][2 * NB];
    i32x4 xa[SB][2][MT], xb[SB][2][MT];
    auto load = [&](i32x4 (&dw)[SB][2 * NB], i32x4 (&dx)[SB][2][MT], int bt) {
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < 2 * NB; h++) dw[j][h] = ld16_nt(wsrc[h] + (int64_t)(bt * SB + j) * 128);
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
                    dx[j][q][mt] = ld16(xrow[mt] + (int64_t)(bt * SB + j) * 128 + q * 64);
    };
    i32x4 acc[2][MT][NB];
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[q][mt][b] = i32x4{0, 0, 0, 0};

    int8_t* st = smem + wave * (SB * TILE);
    auto compute = [&](const i32x4 (&wv)[SB][2 * NB], const i32x4 (&ax)[SB][2][MT]) {
        // The tile is private to the wave and LDS executes a wave's accesses in
        // order; the barriers only keep the compiler from reordering across them.
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < 2 * NB; h++) *reinterpret_cast<i32x4*>(st + j * TILE + woff[h]) = wv[j][h];
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
            i32x4 bf[NB][2];
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int q = 0; q < 2; q++) bf[b][q] = *reinterpret_cast<const i32x4*>(st + j * TILE + roff[b][q]);
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int b = 0; b < NB; b++)
                        acc[q][mt][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(ax[j][q][mt], bf[b][q],
                                                                             acc[q][mt][b], 0, 0, 0);
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };
    load(wa, xa, 0);
    for (int bt = 0; bt < nb - 1; bt++) {
        load(wb, xb, bt + 1);
        compute(wa, xa);
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int h = 0; h < 2 * NB; h++) wa[j][h] = wb[j][h];
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) xa[j][q][mt] = xb[j][q][mt];
        }
    }
    compute(wa, xa);

    __syncthreads();  // the reduction area overlaps the tiles
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int b = 0; b < NB; b++)
            red[(wave * MT * NB + mt * NB + b) * 64 + lane] = acc[0][mt][b] + acc[1][mt][b];
    __syncthreads();
    // result lane l, register i of block (mt, b): token mt*16 + 4*(l/16) + i, row b*16 + l%16
    for (int idx = tid; idx < MT * NB * 64; idx += WAVES * 64) {
        const int mb = idx >> 6, ln = idx & 63, mt = mb / NB, b = mb % NB;
        i32x4 s = red[mb * 64 + ln];
#pragma unroll
        for (int wv = 1; wv < WAVES; wv++) s += red[(wv * MT * NB + mb) * 64 + ln];
        const int col = n0 + b * 16 + (ln & 15);
        if (col >= N) continue;
        const float wsc = ws[col];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = mt * 16 + (ln >> 4) * 4 + i;
            if (m >= M) continue;
            y[(int64_t)m * ldy + col] = fni8::dequant_one(s[i], xs[m], wsc, bias, col);
            if (acc_out != nullptr) acc_out[(int64_t)m * N + col] = s[i];
        }
    }
}

template <int MT, int NB, int WAVES, int SB>
int launch(const int8_t* xq, int64_t ldx, const float* xs, int M, int K, const int8_t* w,
           const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
           int32_t* acc_out, hipStream_t st) {
    const int slabs = K >> 7;
    if (slabs % WAVES != 0 || (slabs / WAVES) % SB != 0) return 1;
    constexpr size_t tiles = (size_t)WAVES * SB * 16 * NB * 128;
    constexpr size_t red = (size_t)WAVES * MT * NB * 64 * 16;
    constexpr size_t lds = tiles > red ? tiles : red;
    static_assert(lds <= 64 * 1024, "decode GEMM LDS budget");
    hipLaunchKernelGGL((decode_mfma_kernel<MT, NB, WAVES, SB>),
                       dim3((unsigned)((N + 16 * NB - 1) / (16 * NB))), dim3(WAVES * 64), lds, st,
                       xq, ldx, xs, M, K, w, ws, N, bias, y, ldy, acc_out);
    return FNI8_OK;
}

// Launch shapes by M tile and weight shape, measured on MI355X over the
// Qwen3-8B decode linears (36 distinct weight copies, weights from HBM):
// wide N takes 32/64-row workgroups (activation fragments reused across row
// blocks), long K and narrow N 8 waves over 16 rows.  Other shapes take the
// first generic entry whose wave split divides K.
template <int MT>
int launch_mt(const int8_t* xq, int64_t ldx, const float* xs, int M, int K, const int8_t* w,
              const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
              int32_t* acc_out, hipStream_t st) {
#define FNI8_DM(NB, WV, SB)                                                                    \
    do {                                                                                       \
        const int rc = launch<MT, NB, WV, SB>(xq, ldx, xs, M, K, w, ws, N, bias, y, ldy,       \
                                              acc_out, st);                                    \
        if (rc != 1) return rc;                                                                \
    } while (0)
    const bool wide = N >= 16384, longk = K >= 8192, narrow = N <= 4096;
    if constexpr (MT == 1) {
        if (wide) FNI8_DM(2, 4, 1);
        else if (longk || narrow) FNI8_DM(1, 8, 1);
        else FNI8_DM(2, 4, 2);
    } else if constexpr (MT == 2) {
        if (wide) FNI8_DM(2, 4, 1);
        else if (longk || narrow) FNI8_DM(1, 4, 2);
        else FNI8_DM(2, 8, 1);
    } else {
        if (wide) FNI8_DM(4, 4, 1);
        else if (longk) FNI8_DM(1, 4, 1);
        else if (narrow) FNI8_DM(1, 8, 1);
        else FNI8_DM(2, 4, 1);
    }
    FNI8_DM(1, 4, 1);
    FNI8_DM(1, 2, 1);
    FNI8_DM(1, 1, 1);
#undef FNI8_DM
    return 1;
}

}  // namespace

namespace fni8h {

// Returns 1 when the shape is not taken (M outside 1..64, K % 128 != 0,
// misaligned operands), else an FNI8 code.
int launch_decode_mfma(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                       const int8_t* w, const float* ws, int64_t N, const uint16_t* bias,
                       uint16_t* y, int64_t ldy, int32_t* acc_out, hipStream_t st) {
    if (M < 1 || M > 64 || K % 128 != 0 || ldq % 16 != 0 || (uintptr_t)xq % 16 != 0 ||
        (uintptr_t)w % 16 != 0)
        return 1;
    const int m = (int)M, k = (int)K, n = (int)N;
    if (M <= 16) return launch_mt<1>(xq, ldq, xs, m, k, w, ws, n, bias, y, ldy, acc_out, st);
    if (M <= 32) return launch_mt<2>(xq, ldq, xs, m, k, w, ws, n, bias, y, ldy, acc_out, st);
    return launch_mt<4>(xq, ldq, xs, m, k, w, ws, n, bias, y, ldy, acc_out, st);
}

}  // namespace fni8h
