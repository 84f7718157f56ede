// Decode GEMMs on MFMA (gfx950): int8 activations for 4 < M <= 64 tokens, and
// fp16 activations quantized inside the kernel for M <= 4 (one launch per linear).
//
//   y[m, n] = fp16(((float)sum_k q[m, k] * w[n, k]) * s[m] * ws[n] (+ bias[n]))
//
// HBM-bound: the weight stream is N*K bytes against M*K of activations.  What
// limits these kernels on MI355X is the per-CU vector memory path (address
// unit and L1), which spends a cycle per cache line touched: so every global
// load instruction is laid out to cover whole 128-byte lines.  Layout:
//   * A workgroup owns 16*NB weight rows; its WAVES waves split K into equal
//     shares of 128-byte slabs.
//   * Weights: each wave load instruction covers 8 rows x 128 contiguous bytes
//     (lane l: row l/8, bytes 16*(l%8) of the slab), non-temporal, register
//     double-buffered one batch of SB slabs ahead.
//   * int8 activations (decode_mfma_kernel) stream the same way: 8 tokens x
//     128 bytes per instruction, prefetched with the weights.  Reading them in
//     the MFMA operand layout instead (16 tokens x 64 bytes per instruction)
//     touches twice the lines and measured 10-20% slower at M = 16..64.
//   * Neither lane layout is the MFMA operand layout, so each slab goes through
//     a wave-private LDS tile (16-byte chunks XOR-swizzled by row, conflict-free
//     both ways) and comes back as the operands of v_mfma_i32_16x16x64_i8
//     (lane l: row l%16, bytes 16*(l/16) of a 64-byte half-slab).
//   * Two accumulator sets (one per half-slab) break the MFMA dependency chain;
//     waves meet once at the end in an LDS reduction, then the fp16 epilogue.
// Integer accumulation is exact, so the result does not depend on the K split.
//
// Fused quantization (decode_mfma_fused_kernel, M <= 4): every workgroup reads
// the M fp16 rows of x (each wave its own K share, 1 KB per load instruction),
// reduces each row's max magnitude (DPP, then one barrier across the waves),
// then, slab by slab inside the weight stream, quantizes its share into a
// wave-private int8 area of LDS that feeds the A operand of that slab's MFMAs.
// The loads of the first weight batch are issued before the maxima, so the
// prologue runs while they are in flight, and the quantization's VALU work
// overlaps the later batches.  Each workgroup quantizes the rows for itself (no
// workgroup waits for another); on MFMA the dot products cost no VALU time,
// which is what made the dot4 GEMV slow at M = 4.
#include "decode_tile.h"

namespace {

using fni8dec::ld16;
using fni8dec::ld16_nt;
using fni8dec::lds_barrier;
using fni8dec::reduce_store;
using fni8dec::swz;
using fni8dec::WeightLanes;

// ---- int8 activations, M <= 16*MT ------------------------------------------
// GROUPED: the expert-segment form of the MoE layer (segments seg_off[E+1] of
// sorted rows; tile slot blockIdx.x is one 16*MT-row piece of one expert's
// segment, blockIdx.y the weight-row block; sorted row r reads activation row
// rmap[r]; weights, scales and bias are stacked per expert).
template <int MT, int NB, int WAVES, int SB, bool GROUPED, int RB = 2 * NB>
__global__ __launch_bounds__(WAVES * 64) void decode_mfma_kernel(
    const int8_t* __restrict__ xq, int64_t ldx, const float* __restrict__ xs,
    const int32_t* __restrict__ rmap, int M, int K, const int8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int E, const int32_t* __restrict__ seg_off,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out) {
    constexpr int ROWS = 16 * NB;
    constexpr int TROWS = ROWS + 16 * MT;  // weight rows, then token rows
    constexpr int TILE = TROWS * 128;      // one slab of the wave's rows
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    i32x4* red = reinterpret_cast<i32x4*>(smem);  // after the main loop: [WAVES][MT*NB][64]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int n0, r0 = 0;
    if constexpr (GROUPED) {
        // every wave finds the same tile; past the last tile the whole
        // workgroup leaves before any barrier
        int e, r1;
        if (!fni8::find_group_tile(seg_off, E, 16 * MT, blockIdx.x, M, e, r0, r1)) return;
        M = r1 - r0;
        n0 = blockIdx.y * (8 * RB);
        w += (int64_t)e * N * K;
        ws += (int64_t)e * N;
        if (bias != nullptr) bias += (int64_t)e * N;
    } else {
        n0 = blockIdx.x * (8 * RB);
    }
    const int per = (K >> 7) / WAVES;  // slabs per wave (exact: the launcher checks)
    const int s0 = wave * per, nb = per / SB;
    const int rq = lane >> 3, c = lane & 7, r = lane & 15, g = lane >> 4;

    WeightLanes<NB, RB> wl;
    wl.init(w, n0, N, K, s0, lane);
    // activation rows: load lane -> (token h*8 + rq, chunk c); tokens past M
    // repeat token M-1 (computed, never stored)
    const int8_t* xsrc[2 * MT];
    int xwoff[2 * MT];
#pragma unroll
    for (int h = 0; h < 2 * MT; h++) {
        const int tok = h * 8 + rq;
        const int row = r0 + (tok < M ? tok : M - 1);
        const int src = (GROUPED && rmap != nullptr) ? rmap[row] : row;
        xsrc[h] = xq + (int64_t)src * ldx + (int64_t)s0 * 128 + c * 16;
        xwoff[h] = (ROWS + tok) * 128 + swz(tok, c);
    }
    int aoff[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int q = 0; q < 2; q++) aoff[mt][q] = (ROWS + mt * 16 + r) * 128 + swz(mt * 16 + r, 4 * q + g);

    i32x4 wa[SB][RB], wb[SB][RB];
    i32x4 xa[SB][2 * MT], xb[SB][2 * MT];
    auto load = [&](i32x4 (&dw)[SB][RB], i32x4 (&dx)[SB][2 * MT], int bt) {
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < RB; h++) dw[j][h] = ld16_nt(wl.src[h] + (int64_t)(bt * SB + j) * 128);
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < 2 * MT; h++) dx[j][h] = ld16(xsrc[h] + (int64_t)(bt * SB + j) * 128);
    };
    i32x4 acc[2][MT][NB];
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int b = 0; b < NB; b++) acc[q][mt][b] = i32x4{0, 0, 0, 0};

    int8_t* st = smem + wave * (SB * TILE);
    auto compute = [&](const i32x4 (&wv)[SB][RB], const i32x4 (&xv)[SB][2 * MT]) {
        // The tile is private to the wave and LDS executes a wave's accesses in
        // order; the barriers only keep the compiler from reordering across them.
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int h = 0; h < RB; h++) *reinterpret_cast<i32x4*>(st + j * TILE + wl.woff[h]) = wv[j][h];
#pragma unroll
            for (int h = 0; h < 2 * MT; h++) *reinterpret_cast<i32x4*>(st + j * TILE + xwoff[h]) = xv[j][h];
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
            i32x4 bf[NB][2], af[MT][2];
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int q = 0; q < 2; q++) bf[b][q] = *reinterpret_cast<const i32x4*>(st + j * TILE + wl.roff[b][q]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int q = 0; q < 2; q++) af[mt][q] = *reinterpret_cast<const i32x4*>(st + j * TILE + aoff[mt][q]);
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int b = 0; b < NB; b++) acc[q][mt][b] = fni8::mfma_i8(af[mt][q], bf[b][q], acc[q][mt][b]);
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
            for (int h = 0; h < RB; h++) wa[j][h] = wb[j][h];
#pragma unroll
            for (int h = 0; h < 2 * MT; h++) xa[j][h] = xb[j][h];
        }
    }
    compute(wa, xa);

    __syncthreads();  // the reduction area overlaps the tiles
    reduce_store<MT, NB, WAVES, 8 * RB>(acc, red, wave, lane, tid, n0, r0, M, N, xs,
                                GROUPED ? rmap : nullptr, ws, bias, y, ldy, acc_out);
}

// ---- fp16 activations, M <= 4, quantized in the kernel, slab by slab ---------
// The prologue keeps only the row maxima: slab t of the wave's share is held as
// one 16-byte chunk per lane (lane l: token l/16, elements (l%16)*8 .. +8 of
// the slab), and it is quantized into the A-operand area just before the MFMAs
// that read it, so the quantization's VALU work runs while later weight batches
// are in flight.  (Quantizing the whole share in the prologue instead, before
// the weight stream could be consumed, measured 2-11% slower: M = 4, QKV 7.99
// against 7.11 us, down 12.21 against 11.29.)  PER = 4*PQ slabs per wave
// (K = 512 * WAVES * PQ).  EB: the second weight batch is issued right after
// the row-max barrier.
template <int NB, int WAVES, int SB, int PQ, int RB = 2 * NB, bool EB = false>
__global__ __launch_bounds__(WAVES * 64) void decode_mfma_fused_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int M, int K, const int8_t* __restrict__ w,
    const float* __restrict__ ws, int N, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, int64_t ldy, int8_t* __restrict__ xq_out,
    float* __restrict__ xs_out, int32_t* __restrict__ acc_out) {
    constexpr int MM = 4;                  // token rows: 64 lanes = 4 rows x 16 chunks of a slab
    constexpr int ROWS = 16 * NB;
    constexpr int TILE = ROWS * 128;
    constexpr int PER = 4 * PQ;            // slabs per wave
    constexpr int NBT = PER / SB;          // batches per wave
    constexpr int XAREA = PER * MM * 128;  // the wave's int8 activations: [PER][MM tokens][128]
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t* tiles = smem;                                     // [WAVES][SB][TILE]
    int8_t* xarea = smem + WAVES * SB * TILE;                 // [WAVES][XAREA]
    uint32_t* amx = reinterpret_cast<uint32_t*>(xarea + WAVES * XAREA);  // [WAVES][MM]
    float* scl = reinterpret_cast<float*>(amx + WAVES * MM);  // [MM]
    i32x4* red = reinterpret_cast<i32x4*>(smem);              // after the main loop

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * (8 * RB);
    const int s0 = wave * PER;
    const int r = lane & 15, g = lane >> 4;
    const int xm = lane >> 4, xc = lane & 15;  // this lane's token and 8-element chunk of a slab
    const bool xlive = xm < M;

    // 1. this lane's chunk of every slab of the share (activation loads first)
    uint4 xv[PER];
    const uint16_t* xrow = x + (int64_t)(xlive ? xm : 0) * ldx + (int64_t)s0 * 128 + xc * 8;
#pragma unroll
    for (int t = 0; t < PER; t++)
        xv[t] = xlive ? *reinterpret_cast<const uint4*>(xrow + t * 128) : make_uint4(0, 0, 0, 0);
    // 2. first weight batch
    WeightLanes<NB, RB> wl;
    wl.init(w, n0, N, K, s0, lane);
    i32x4 wa[SB][RB], wb[SB][RB];
#pragma unroll
    for (int j = 0; j < SB; j++)
#pragma unroll
        for (int h = 0; h < RB; h++) wa[j][h] = ld16_nt(wl.src[h] + (int64_t)j * 128);

    // 3. row maxima: over the lane's chunks, then its 16-lane group (one token),
    //    then across the waves
    uint32_t mx = 0;
#pragma unroll
    for (int t = 0; t < PER; t++) mx = fni8::amax_chunk(mx, xv[t]);
    {
        int v = (int)fni8::amax_fold(mx), o;
        o = fni8::dpp<fni8::kDppXor1>(v); v = o > v ? o : v;
        o = fni8::dpp<fni8::kDppXor2>(v); v = o > v ? o : v;
        o = fni8::dpp<fni8::kDppHalfMirror>(v); v = o > v ? o : v;
        o = fni8::dpp<fni8::kDppMirror>(v); v = o > v ? o : v;
        if (xc == 0) amx[wave * MM + xm] = (uint32_t)v;
    }
    lds_barrier();
    if constexpr (EB && NBT > 1) {
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < RB; h++) wb[j][h] = ld16_nt(wl.src[h] + (int64_t)(SB + j) * 128);
    }
    uint32_t a = amx[xm];
#pragma unroll
    for (int wv = 1; wv < WAVES; wv++) a = amx[wv * MM + xm] > a ? amx[wv * MM + xm] : a;
    const float sc = fni8::row_scale_from_bits(a);
    const bool live = xlive && __builtin_isfinite(sc);  // NaN/inf scale: every q is 0
    const float yr = 1.0f / sc;                          // correctly rounded (build flag)
    if (wave == 0 && xc == 0) {
        scl[xm] = sc;
        if (blockIdx.x == 0 && xlive) xs_out[xm] = sc;
    }
    int8_t* xw = xarea + wave * XAREA;
    const int xoff = xm * 128 + swz(xm, xc >> 1) + (xc & 1) * 8;  // in a slab's [MM][128]
    const int tok = r < M ? r : M - 1;  // tokens past M repeat M-1 (never stored)
    int aoff[2];
#pragma unroll
    for (int q = 0; q < 2; q++) aoff[q] = tok * 128 + swz(tok, 4 * q + g);

    // 4. the weight stream, each slab's activations quantized just before use
    i32x4 acc[2][1][NB];
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[q][0][b] = i32x4{0, 0, 0, 0};
    int8_t* st = tiles + wave * (SB * TILE);
    auto compute = [&](const i32x4 (&wv)[SB][RB], int bt) {
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const int t = bt * SB + j;
            const uint2 q = fni8::quant_chunk(xv[t], sc, yr, live);
            *reinterpret_cast<uint2*>(xw + t * (MM * 128) + xoff) = q;
            if (blockIdx.x == 0 && xlive)
                *reinterpret_cast<uint2*>(xq_out + (int64_t)xm * K + (int64_t)(s0 + t) * 128 + xc * 8) = q;
#pragma unroll
            for (int h = 0; h < RB; h++) *reinterpret_cast<i32x4*>(st + j * TILE + wl.woff[h]) = wv[j][h];
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const int8_t* xs_ = xw + (bt * SB + j) * (MM * 128);
            const i32x4 a0 = ld16(xs_ + aoff[0]), a1 = ld16(xs_ + aoff[1]);
            i32x4 bf[NB][2];
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int q = 0; q < 2; q++) bf[b][q] = *reinterpret_cast<const i32x4*>(st + j * TILE + wl.roff[b][q]);
#pragma unroll
            for (int b = 0; b < NB; b++) {
                acc[0][0][b] = fni8::mfma_i8(a0, bf[b][0], acc[0][0][b]);
                acc[1][0][b] = fni8::mfma_i8(a1, bf[b][1], acc[1][0][b]);
            }
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };
#pragma unroll
    for (int bt = 0; bt < NBT - 1; bt++) {
        if (!EB || bt > 0) {
#pragma unroll
            for (int j = 0; j < SB; j++)
#pragma unroll
                for (int h = 0; h < RB; h++) wb[j][h] = ld16_nt(wl.src[h] + (int64_t)((bt + 1) * SB + j) * 128);
        }
        compute(wa, bt);
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < RB; h++) wa[j][h] = wb[j][h];
    }
    compute(wa, NBT - 1);

    __syncthreads();  // the reduction area overlaps the tiles
    reduce_store<1, NB, WAVES, 8 * RB>(acc, red, wave, lane, tid, n0, 0, M, N, scl, nullptr, ws,
                                       bias, y, ldy, acc_out);
}

template <int MT, int NB, int WAVES, int SB, bool GROUPED = false, int RB = 2 * NB>
int launch(const int8_t* xq, int64_t ldx, const float* xs, int M, int K, const int8_t* w,
           const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
           int32_t* acc_out, hipStream_t st, const int32_t* rmap = nullptr, int E = 0,
           const int32_t* seg_off = nullptr) {
    const int slabs = K >> 7;
    if (slabs % WAVES != 0 || (slabs / WAVES) % SB != 0) return 1;
    constexpr size_t tiles = (size_t)WAVES * SB * (16 * NB + 16 * MT) * 128;
    constexpr size_t red = (size_t)WAVES * MT * NB * 64 * 16;
    constexpr size_t lds = tiles > red ? tiles : red;
    static_assert(lds <= 160 * 1024, "decode GEMM LDS budget");
    auto kern = decode_mfma_kernel<MT, NB, WAVES, SB, GROUPED, RB>;
    if constexpr (lds > 64 * 1024) {
        static const bool ok = hipFuncSetAttribute((const void*)kern,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)lds) == hipSuccess;
        if (!ok) return 1;
    }
    const unsigned nblk = (unsigned)((N + 8 * RB - 1) / (8 * RB));
    // grouped: one slot per 16*MT-row piece of a segment; at most
    // ceil(M / (16*MT)) + E of them are non-empty
    const dim3 grid = GROUPED ? dim3((unsigned)((M + 16 * MT - 1) / (16 * MT) + E), nblk) : dim3(nblk);
    hipLaunchKernelGGL(kern, grid, dim3(WAVES * 64), lds, st, xq, ldx, xs, rmap, M, K, w, ws, N, E,
                       seg_off, bias, y, ldy, acc_out);
    return FNI8_OK;
}

template <int NB, int WAVES, int SB, int PQ, int RB = 2 * NB, bool EB = false>
int launch_fused(const uint16_t* x, int64_t ldx, int M, int K, const int8_t* w, const float* ws,
               int N, const uint16_t* bias, uint16_t* y, int64_t ldy, int8_t* xq_out,
               float* xs_out, int32_t* acc_out, hipStream_t st) {
    static_assert((4 * PQ) % SB == 0, "batches must divide the share");
    if (K != 512 * WAVES * PQ || M > 4) return 1;
    constexpr size_t tiles = (size_t)WAVES * SB * 16 * NB * 128;
    constexpr size_t lds_main = tiles + (size_t)WAVES * 4 * PQ * 512 + WAVES * 16 + 16;
    constexpr size_t red = (size_t)WAVES * NB * 64 * 16;
    constexpr size_t lds = lds_main > red ? lds_main : red;
    if constexpr (lds > 160 * 1024) {
        return 1;
    } else {
        auto kern = decode_mfma_fused_kernel<NB, WAVES, SB, PQ, RB, EB>;
        static const bool ok = hipFuncSetAttribute((const void*)kern,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   160 * 1024) == hipSuccess;
        if (!ok) return 1;
        hipLaunchKernelGGL(kern, dim3((unsigned)((N + 8 * RB - 1) / (8 * RB))), dim3(WAVES * 64),
                           lds, st, x, ldx, M, K, w, ws, N, bias, y, ldy, xq_out, xs_out, acc_out);
        return FNI8_OK;
    }
}

// True when 24-row workgroups fill the CUs better than 32-row ones in whole
// rounds (N = 6144: 256 workgroups against 192 on 256 CUs).
bool prefer_24_rows(int N) {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        return n;
    }();
    auto fill = [](int wgs) { return (double)wgs / (double)(((wgs + cus - 1) / cus) * cus); };
    return fill((N + 23) / 24) > fill((N + 31) / 32) + 1e-9;
}

// Launch shapes by M tile and weight shape, measured on MI355X over the
// Qwen3-8B decode linears (a sweep of every shape within the LDS budget, 24
// distinct weight copies, weights from HBM).
// Other shapes take the first generic entry whose wave split divides K.
template <int MT>
int launch_mt(const int8_t* xq, int64_t ldx, const float* xs, int M, int K, const int8_t* w,
              const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
              int32_t* acc_out, hipStream_t st) {
#define FNI8_DM_RB(NB, WV, SB, RB)                                                             \
    do {                                                                                       \
        const int rc = launch<MT, NB, WV, SB, false, RB>(xq, ldx, xs, M, K, w, ws, N, bias, y, \
                                                         ldy, acc_out, st);                    \
        if (rc != 1) return rc;                                                                \
    } while (0)
#define FNI8_DM(NB, WV, SB) FNI8_DM_RB(NB, WV, SB, 2 * NB)
    const bool wide = N >= 16384, longk = K >= 8192, narrow = N <= 4096;
    const bool rows24 = !wide && !narrow && prefer_24_rows(N);  // QKV: 24-row workgroups
    if constexpr (MT == 1) {
        if (wide) FNI8_DM(2, 2, 1);
        else if (longk) FNI8_DM(1, 8, 2);
        else if (narrow) FNI8_DM(1, 4, 2);
        else if (rows24) FNI8_DM_RB(2, 8, 1, 3);
        else FNI8_DM(2, 8, 1);
    } else if constexpr (MT == 2) {
        if (wide) FNI8_DM(2, 2, 1);
        else if (longk || narrow) FNI8_DM(1, 4, 2);
        else if (rows24) FNI8_DM_RB(2, 4, 2, 3);
        else FNI8_DM(2, 4, 2);
    } else {
        // wide at 33..64 tokens: 48-row workgroups (three MFMA blocks) read the
        // activation tile once per 48 weight rows instead of 32 (gate_up at 64
        // tokens: 27.3 -> 26.0 us; even at 48 tokens, slower below)
        if (wide) FNI8_DM_RB(3, 2, 1, 6);
        else if (longk) FNI8_DM(1, 4, 2);
        else if (narrow) FNI8_DM(1, 8, 1);
        else if (rows24) FNI8_DM_RB(2, 8, 1, 3);
        else FNI8_DM(2, 8, 1);
    }
    FNI8_DM(1, 4, 1);
    FNI8_DM(1, 2, 1);
    FNI8_DM(1, 1, 1);
#undef FNI8_DM
#undef FNI8_DM_RB
    return 1;
}

// Grouped (MoE) shapes, from a sweep over the 128-expert top-8 routing
// (gate_up 1536x2048, down 2048x768) at T = 16, 64 and 256: a short K (down's 6
// slabs) takes one wave over 32 weight rows; otherwise 2-wave workgroups.
template <int MT>
int launch_grouped_mt(const int8_t* xq, int64_t ldx, const float* xs, const int32_t* rmap, int R,
                      int K, const int8_t* w, const float* ws, int E, int N,
                      const int32_t* seg_off, const uint16_t* bias, uint16_t* y, int64_t ldy,
                      int32_t* acc_out, hipStream_t st) {
#define FNI8_DG(NB, WV, SB)                                                                     \
    do {                                                                                        \
        const int rc = launch<MT, NB, WV, SB, true>(xq, ldx, xs, R, K, w, ws, N, bias, y, ldy,  \
                                                    acc_out, st, rmap, E, seg_off);             \
        if (rc != 1) return rc;                                                                 \
    } while (0)
    if (K <= 1024) FNI8_DG(2, 1, 1);
    FNI8_DG(2, 2, 1);
    FNI8_DG(1, 2, 1);
    FNI8_DG(2, 1, 1);
    FNI8_DG(1, 1, 1);
#undef FNI8_DG
    return 1;
}

int launch_fused_table(const uint16_t* x, int64_t ldx, int M, int K, const int8_t* w,
                       const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                       int8_t* xq_out, float* xs_out, int32_t* acc_out, hipStream_t st) {
#define FNI8_DF_RBE(NB, WV, SB, PQ, RB, EB)                                                  \
    do {                                                                                     \
        const int rc = launch_fused<NB, WV, SB, PQ, RB, EB>(x, ldx, M, K, w, ws, N, bias, y, \
                                                            ldy, xq_out, xs_out, acc_out, st); \
        if (rc != 1) return rc;                                                              \
    } while (0)
#define FNI8_DF_RB(NB, WV, SB, PQ, RB) FNI8_DF_RBE(NB, WV, SB, PQ, RB, false)
#define FNI8_DF(NB, WV, SB, PQ) FNI8_DF_RB(NB, WV, SB, PQ, 2 * NB)
    // Measured at 3 and 4 tokens over the Qwen3-8B linears (36 layers of
    // distinct weights; six launch tables, every variant bit-identical).
    const bool wide = N >= 16384, narrow = N <= 4096;
    if (wide) {
        FNI8_DF(2, 4, 2, 2);
        FNI8_DF(2, 8, 1, 3);
    } else if (narrow) {
        // second weight batch issued right after the row maxima (O and down)
        FNI8_DF_RBE(1, 4, 2, 2, 2, true);
        FNI8_DF_RBE(1, 8, 2, 3, 2, true);
    } else {
        if (prefer_24_rows(N)) FNI8_DF_RB(2, 4, 2, 2, 3);  // QKV: 24-row workgroups
        FNI8_DF(2, 8, 1, 1);
        FNI8_DF(2, 8, 1, 3);
    }
    // generic entries: K = 1024, 2048, 3072, 4096, 5120, 6144, 8192, 12288
    FNI8_DF(1, 2, 2, 1);
    FNI8_DF(1, 4, 2, 1);
    FNI8_DF(1, 2, 2, 3);
    FNI8_DF(1, 8, 2, 1);
    FNI8_DF(1, 2, 2, 5);
    FNI8_DF(1, 4, 2, 3);
    FNI8_DF(1, 8, 2, 2);
    FNI8_DF(1, 8, 1, 3);
#undef FNI8_DF
#undef FNI8_DF_RB
#undef FNI8_DF_RBE
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

// Grouped expert GEMM (MoE) on MFMA for small segments: returns 1 when not
// taken (more than 48 rows per expert on average, K % 128 != 0, misaligned
// operands), so the caller uses the tile kernel.  The tile height follows the
// average segment: 16 rows up to 8 rows per expert, else 32 (64-row tiles
// measured 1.5-2x slower on skewed routings: most segments are small).
int launch_decode_mfma_grouped(const int8_t* aq, int64_t lda, const float* as,
                               const int32_t* row_index, int64_t R_max, int64_t K,
                               const int8_t* w, const float* ws, int64_t E, int64_t N,
                               const int32_t* seg_off, const uint16_t* bias, uint16_t* y,
                               int64_t ldy, int32_t* acc_out, hipStream_t st) {
    if (R_max < 1 || E < 1 || K % 128 != 0 || lda % 16 != 0 || (uintptr_t)aq % 16 != 0 ||
        (uintptr_t)w % 16 != 0)
        return 1;
    // Above 4 rows per expert on average the tile kernel takes the segments:
    // on the 128-expert top-8 projections it is 17-30% faster for skewed
    // routing from 4 rows up, and from 16 rows up for uniform routing too
    // (at 4-8 uniform rows this kernel is ~10% faster).
    if ((double)R_max / (double)E > 4.0) return 1;
    return launch_grouped_mt<1>(aq, lda, as, row_index, (int)R_max, (int)K, w, ws, (int)E, (int)N,
                                seg_off, bias, y, ldy, acc_out, st);
}

// fp16 activations, M <= 4, quantization fused: returns 1 when the shape is
// not taken (K not 512 * waves * PQ for a table entry, misaligned operands).
// xq_out (row stride K) and xs_out receive the quantized activations.
int launch_decode_mfma_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                             const int8_t* w, const float* ws, int64_t N, const uint16_t* bias,
                             uint16_t* y, int64_t ldy, int8_t* xq_out, float* xs_out,
                             int32_t* acc_out, hipStream_t st) {
    if (M < 1 || M > 4 || K % 512 != 0 || ldx % 8 != 0 || (uintptr_t)x % 16 != 0 ||
        (uintptr_t)w % 16 != 0 || xq_out == nullptr || xs_out == nullptr ||
        (uintptr_t)xq_out % 8 != 0)
        return 1;
    const int rc = launch_fused_table(x, ldx, (int)M, (int)K, w, ws, (int)N, bias, y, ldy, xq_out,
                                      xs_out, acc_out, st);
    if (rc != FNI8_OK) return rc;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("decode launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

}  // namespace fni8h
