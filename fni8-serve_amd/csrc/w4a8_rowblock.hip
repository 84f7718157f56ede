// W4A8 decode GEMM on MFMA with the weight rows split over the waves (gemm_w4a8
// of `fni8.linear` for int4 QTensors, fni8serve/layers/linear.py:9, :63-65),
// for 9 to 64 tokens of int8 activations on wide weights (N >= 16384).
//
// w4a8_mfma_kernel (w4a8.hip) splits K over the waves of a 16-row workgroup and
// moves every group's int32 sums through LDS to fold them in order; each
// workgroup then reads all M*K activation bytes for 16*K/2 weight bytes, which
// at 64 tokens is eight times the weight stream (from L2).  Here a workgroup
// owns 16*WAVES weight rows instead, one 16-row block per wave:
//   * Every wave walks the whole K in slabs of 256 codes.  The slab's
//     activations (16*MT tokens x 256 bytes) are loaded once per workgroup,
//     spread over all its lanes (16 lanes per 256-byte token row, whole cache
//     lines), and staged in an LDS tile that all waves read; two tiles
//     alternate, so one barrier per batch of SB slabs orders the writes.
//   * Each wave streams its own 16 rows (8 rows x 128 packed bytes per load
//     instruction, non-temporal) through a wave-private LDS tile into the B
//     operand of v_mfma_i32_16x16x64_i8, unpacked to 16 * code (w4a8_common.h).
//   * Lane l holds weight row l % 16 and tokens 16*mt + 4*(l/16) + i of the
//     MFMA results, so it folds its own group sums in registers:
//     accf = fma((float)(16*acc_g >> 4), ws[n, g], accf) in ascending g from
//     +0, then y = fp16(accf * xs[m] (+ bias[n])) -- the arithmetic of every
//     W4A8 kernel here, so the bits are the same.
// Activation loads for tokens past M are skipped: those tile rows hold stale
// values whose products land in outputs that are never stored.  Weight rows
// past N repeat row N-1 (computed, never stored).
//
// GROUPED: the expert-segment form of the MoE layer's projections (one launch
// for all experts).  Segments seg_off[E+1] of sorted rows; blockIdx.x is one
// 16*MT-row piece of one expert's segment, blockIdx.y the weight-row block;
// sorted row r reads activation row rmap[r] (row r without a map) and its scale;
// weights, scales and bias are stacked per expert; y is in sorted-row order.
#include "w4a8_common.h"

namespace {

template <int MT, int WAVES, int SB, int G, bool GROUPED = false>
__global__ __launch_bounds__(WAVES * 64) void w4a8_rowblock_kernel(
    const int8_t* __restrict__ xq, int64_t ldx, const float* __restrict__ xs,
    const int32_t* __restrict__ rmap, int M, int K, const uint8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int E, const int32_t* __restrict__ seg_off,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy) {
    constexpr int NT = WAVES * 64;
    constexpr int TOK = 16 * MT;
    constexpr int XT = 2 * TOK * 128;          // a slab's activations: [half][TOK][128 bytes]
    constexpr int WT = 16 * 128;               // a wave's 16 weight rows of one slab
    constexpr int XCH = 16 * TOK;              // 16-byte activation chunks per slab
    constexpr int XL = (XCH + NT - 1) / NT;    // per lane
    constexpr int KBG = G / 64;                // MFMA k-blocks per group
    constexpr int GPS = 256 / G;               // groups per slab
    constexpr int GPB = SB * GPS;              // groups per batch
    static_assert(G >= 64 && G <= 256 && MT >= 1 && MT <= 4, "w4a8 row-block shape");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    int8_t* xt = smem;                                     // [2][SB][XT]
    int8_t* wt = smem + 2 * SB * XT + wave * (SB * WT);    // this wave's [SB][WT]
    const int nb = (K >> 8) / SB;                          // batches (the launcher makes it exact)
    const int ng = K / G;
    int r0 = 0, rblk = blockIdx.x;
    if constexpr (GROUPED) {
        // every wave finds the same tile; past the last tile the whole
        // workgroup leaves before any barrier
        int e, r1;
        if (!fni8::find_group_tile(seg_off, E, TOK, blockIdx.x, M, e, r0, r1)) return;
        M = r1 - r0;
        rblk = blockIdx.y;
        w += (int64_t)e * N * (K >> 1);
        ws += (int64_t)e * N * ng;
        if (bias != nullptr) bias += (int64_t)e * N;
    }
    // activation row of the tile's token t (t < M)
    auto src_row = [&](int t) -> int {
        if constexpr (GROUPED) return rmap != nullptr ? rmap[r0 + t] : r0 + t;
        return t;
    };
    const int n0 = rblk * (16 * WAVES) + 16 * wave;  // the wave's first weight row
    const int rq = lane >> 3, c = lane & 7, r = lane & 15, g = lane >> 4;

    // weight load lanes: row h*8 + rq of the wave's block, 16-byte chunk c
    const uint8_t* wsrc[2];
    int woff[2];
#pragma unroll
    for (int h = 0; h < 2; h++) {
        const int row = h * 8 + rq;
        const int n = n0 + row < N ? n0 + row : N - 1;
        wsrc[h] = w + (int64_t)n * (K >> 1) + c * 16;
        woff[h] = row * 128 + swz(row, c);
    }
    // activation load lanes: chunk q = i*NT + tid is token q/16, half (q/8)%2,
    // chunk q%8 of the slab
    const int8_t* xsrc[XL];
    int xoff[XL];
    bool xlive[XL];
#pragma unroll
    for (int i = 0; i < XL; i++) {
        const int q = i * NT + tid;
        const int tok = q >> 4, hf = (q >> 3) & 1, cc = q & 7;
        xlive[i] = q < XCH && tok < M;
        xsrc[i] = xq + (int64_t)src_row(tok < M ? tok : 0) * ldx + hf * 128 + cc * 16;
        const int row = hf * TOK + (tok < TOK ? tok : 0);
        xoff[i] = row * 128 + swz(row, cc);
    }
    // operand lanes: k-block j of the slab is codes 64j..64j+63; lane (r, g)
    // holds codes 64j + 16g .. +15 of weight row / token r
    int boff[4], aoff[MT][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
        boff[j] = r * 128 + swz(r, 2 * j + (g >> 1)) + 8 * (g & 1);
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int row = (j >> 1) * TOK + mt * 16 + r;
            aoff[mt][j] = row * 128 + swz(row, 4 * (j & 1) + g);
        }
    }
    const float* wsrow = ws + (int64_t)(n0 + r < N ? n0 + r : N - 1) * ng;

    i32x4 xa[SB][XL], xb[SB][XL], wa[SB][2], wb[SB][2];
    float sa[GPB], sb[GPB];
    auto load = [&](i32x4 (&xr)[SB][XL], i32x4 (&wr)[SB][2], float (&sr)[GPB], int bt) {
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const int64_t s = (int64_t)bt * SB + j;
#pragma unroll
            for (int h = 0; h < 2; h++)
                wr[j][h] = __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(wsrc[h] + s * 128));
#pragma unroll
            for (int i = 0; i < XL; i++)
                if (xlive[i]) xr[j][i] = *reinterpret_cast<const i32x4*>(xsrc[i] + s * 256);
        }
#pragma unroll
        for (int q = 0; q < GPB; q++) sr[q] = wsrow[bt * GPB + q];
    };

    float accf[MT][4];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int i = 0; i < 4; i++) accf[mt][i] = 0.0f;

    load(xa, wa, sa, 0);
    for (int bt = 0; bt < nb; bt++) {
        int8_t* xtb = xt + (bt & 1) * (SB * XT);
        // Stage batch bt.  The activation tile it overwrites was last read in
        // batch bt-2, before every wave passed the barrier of batch bt-1; the
        // weight tile is private to the wave, and LDS executes a wave's
        // accesses in order.
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int i = 0; i < XL; i++)
                if (xlive[i]) *reinterpret_cast<i32x4*>(xtb + j * XT + xoff[i]) = xa[j][i];
#pragma unroll
            for (int h = 0; h < 2; h++) *reinterpret_cast<i32x4*>(wt + j * WT + woff[h]) = wa[j][h];
        }
        lds_barrier();
        if (bt + 1 < nb) load(xb, wb, sb, bt + 1);
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int gj = 0; gj < GPS; gj++) {
                i32x4 acc[MT];
#pragma unroll
                for (int mt = 0; mt < MT; mt++) acc[mt] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int kb = 0; kb < KBG; kb++) {
                    const int jb = gj * KBG + kb;
                    const uint2 pk = *reinterpret_cast<const uint2*>(wt + j * WT + boff[jb]);
                    const i32x4 bf = unpack16x16(pk.x, pk.y);
#pragma unroll
                    for (int mt = 0; mt < MT; mt++) {
                        const i32x4 af = *reinterpret_cast<const i32x4*>(xtb + j * XT + aoff[mt][jb]);
                        acc[mt] = fni8::mfma_i8(af, bf, acc[mt]);
                    }
                }
                const float sc = sa[j * GPS + gj];
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int i = 0; i < 4; i++)
                        accf[mt][i] = __builtin_fmaf((float)(acc[mt][i] >> 4), sc, accf[mt][i]);
            }
        }
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int i = 0; i < XL; i++) xa[j][i] = xb[j][i];
#pragma unroll
            for (int h = 0; h < 2; h++) wa[j][h] = wb[j][h];
        }
#pragma unroll
        for (int q = 0; q < GPB; q++) sa[q] = sb[q];
    }

    const int n = n0 + r;
    if (n < N) {
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int i = 0; i < 4; i++) {
                const int m = mt * 16 + 4 * g + i;
                if (m < M) {
                    float v = accf[mt][i] * xs[src_row(m)];
                    if (bias) v = v + fni8::h2f(bias[n]);
                    y[(int64_t)(r0 + m) * ldy + n] = fni8::f2h(v);
                }
            }
    }
}

constexpr size_t kLdsLimit = 160 * 1024;

template <int MT, int WAVES, int SB>
constexpr size_t kRowblockLds = (size_t)SB * (2 * 2 * 16 * MT * 128 + WAVES * 16 * 128);

template <int MT, int WAVES, int SB, int G>
int rowblock_launch(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                    const uint8_t* w, const float* ws, int64_t N, const uint16_t* bias,
                    uint16_t* y, int64_t ldy, hipStream_t st) {
    constexpr size_t lds = kRowblockLds<MT, WAVES, SB>;
    if constexpr (lds > kLdsLimit) {
        return 1;
    } else {
        if ((K >> 8) % SB != 0) return 1;
        auto kern = &w4a8_rowblock_kernel<MT, WAVES, SB, G>;
        if constexpr (lds > 64 * 1024) {
            static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)lds) == hipSuccess;
            if (!ok) {
                fni8h::set_error_detail("w4a8 row-block: cannot raise the LDS limit to %zu bytes",
                                        lds);
                return FNI8_ERR_LAUNCH;
            }
        }
        const dim3 grid((unsigned)((N + 16 * WAVES - 1) / (16 * WAVES)));
        hipLaunchKernelGGL(kern, grid, dim3(WAVES * 64), lds, st, xq, ldq, xs, nullptr, (int)M,
                           (int)K, w, ws, (int)N, 0, nullptr, bias, y, ldy);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            fni8h::set_error_detail("w4a8 row-block launch: %s", hipGetErrorString(e));
            return FNI8_ERR_LAUNCH;
        }
        return FNI8_OK;
    }
}

// Grouped form: activation rows of stride K, y of stride N; the grid's x
// dimension bounds the segment tiles (sum over experts of ceil(len / (16*MT))
// <= R_max / (16*MT) + E), its y dimension the weight-row blocks.
template <int MT, int WAVES, int SB, int G>
int rowblock_grouped_launch(const int8_t* aq, const float* as, const int32_t* rmap,
                            int64_t R_max, int64_t K, const uint8_t* w, const float* ws,
                            int64_t E, int64_t N, const int32_t* seg_off, const uint16_t* bias,
                            uint16_t* y, hipStream_t st) {
    constexpr size_t lds = kRowblockLds<MT, WAVES, SB>;
    static_assert(lds <= kLdsLimit, "LDS budget");
    auto kern = &w4a8_rowblock_kernel<MT, WAVES, SB, G, true>;
    if constexpr (lds > 64 * 1024) {
        static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)lds) == hipSuccess;
        if (!ok) {
            fni8h::set_error_detail("w4a8 grouped: cannot raise the LDS limit to %zu bytes", lds);
            return FNI8_ERR_LAUNCH;
        }
    }
    const dim3 grid((unsigned)((R_max + 16 * MT - 1) / (16 * MT) + E),
                    (unsigned)((N + 16 * WAVES - 1) / (16 * WAVES)));
    hipLaunchKernelGGL(kern, grid, dim3(WAVES * 64), lds, st, aq, K, as, rmap, (int)R_max,
                       (int)K, w, ws, (int)N, (int)E, seg_off, bias, y, N);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fni8h::set_error_detail("w4a8 grouped launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

template <int G>
int grouped_by_tile(const int8_t* aq, const float* as, const int32_t* rmap, int64_t R_max,
                    int64_t K, const uint8_t* w, const float* ws, int64_t E, int64_t N,
                    const int32_t* seg_off, const uint16_t* bias, uint16_t* y, hipStream_t st) {
    // Segment tiles of 16, 32 or 64 rows by the mean rows per expert, four
    // waves.  Measured on the Qwen3-30B-A3B projections (128 experts, top-8,
    // uniform routing; gate_up [1536, 2048], down [2048, 768]), µs against the
    // earlier 16-row, two-wave, two-slab shape: T = 16 gate_up 30.44 / 32.69,
    // down 18.87 / 21.97 (16-row tiles); T = 256 gate_up 62.61 / 81.28, down
    // 40.41 / 49.11 (32-row tiles).  One slab per batch was faster than two at
    // every small-segment point; 64-row tiles keep two where K allows.
    // With few rows (T = 1: 8 of 128 experts) four-wave workgroups would leave
    // the grid under two per CU; the two-wave shape stays there.
    const double avg = (double)R_max / (double)E;
    const bool sb2 = (K >> 8) % 2 == 0;
    const int64_t active = R_max < E ? R_max : E;  // segments that can be non-empty
    if (avg <= 8.0 && active * ((N + 63) / 64) < 512)
        return sb2 ? rowblock_grouped_launch<1, 2, 2, G>(aq, as, rmap, R_max, K, w, ws, E, N,
                                                         seg_off, bias, y, st)
                   : rowblock_grouped_launch<1, 2, 1, G>(aq, as, rmap, R_max, K, w, ws, E, N,
                                                         seg_off, bias, y, st);
    if (avg <= 8.0)
        return rowblock_grouped_launch<1, 4, 1, G>(aq, as, rmap, R_max, K, w, ws, E, N, seg_off,
                                                   bias, y, st);
    if (avg <= 32.0)
        return rowblock_grouped_launch<2, 4, 1, G>(aq, as, rmap, R_max, K, w, ws, E, N, seg_off,
                                                   bias, y, st);
    return sb2 ? rowblock_grouped_launch<4, 4, 2, G>(aq, as, rmap, R_max, K, w, ws, E, N,
                                                     seg_off, bias, y, st)
               : rowblock_grouped_launch<4, 4, 1, G>(aq, as, rmap, R_max, K, w, ws, E, N,
                                                     seg_off, bias, y, st);
}

}  // namespace

namespace fni8h {

// Launch shapes measured on MI355X over the Qwen3-8B linears at G = 128 (36
// weight copies, weights from HBM), against w4a8_mfma_kernel, µs:
//   gate_up 24576 x 4096 at 16 / 24 / 32 / 48 / 64 tokens: 14.90 (two waves) /
//     18.42 / 19.16 / 23.33 / 27.69 (four waves) against 16.03 / 26.77 / 29.43 /
//     41.23 / 60.49
//   at 5 and 8 tokens 14.6 / 14.5 against 13.7 / 13.8 (the K-split kernel loads
//     one 8-token group there, two from 9 tokens on)
// Two slabs per batch were faster than one on every shape.  Narrow N (QKV, O
// and down, N <= 6144) stays on the K-split kernel: with 16 weight rows per
// wave and a whole-K walk, 64-192 workgroups cannot stream the weights as fast
// (1.04-2.3x its time from 5 to 64 tokens).
int launch_w4a8_rowblock(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                         const uint8_t* w, const float* ws, int64_t N, int64_t G,
                         const uint16_t* bias, uint16_t* y, int64_t ldy, hipStream_t st) {
    if (M <= 8 || M > 64 || N < 16384 || N > INT32_MAX || K % 512 != 0 || K > 65536) return 1;
    if (ldq % 16 != 0 || ((uintptr_t)xq % 16) != 0 || ((uintptr_t)w % 16) != 0) return 1;
    const int mt = (int)((M + 15) / 16);
#define FNI8_W4RB(MTV, WV, GV) \
    return rowblock_launch<MTV, WV, 2, GV>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st)
#define FNI8_W4RB_MT(GV)                    \
    switch (mt) {                           \
        case 1: FNI8_W4RB(1, 2, GV);        \
        case 2: FNI8_W4RB(2, 4, GV);        \
        case 3: FNI8_W4RB(3, 4, GV);        \
        default: FNI8_W4RB(4, 4, GV);       \
    }
    switch (G) {
        case 64: FNI8_W4RB_MT(64)
        case 128: FNI8_W4RB_MT(128)
        case 256: FNI8_W4RB_MT(256)
        default: return 1;
    }
#undef FNI8_W4RB_MT
#undef FNI8_W4RB
}

// Grouped W4A8 over expert segments (K a multiple of 256, G in {64, 128, 256}:
// the caller checks).
int launch_gemm_w4a8_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                             int64_t R_max, int64_t K, const uint8_t* w, const float* ws,
                             int64_t E, int64_t N, int64_t G, const int32_t* seg_off,
                             const uint16_t* bias, uint16_t* y, hipStream_t st) {
    if (R_max == 0) return FNI8_OK;
    // 64 or more rows per expert on average: 128x128 segment tiles of the
    // prefill tile kernel (w4a8.hip)
    if (R_max >= 64 * E)
        return launch_w4a8_tile_grouped(aq, as, row_index, R_max, K, w, ws, E, N, G, seg_off,
                                        bias, y, st);
    switch (G) {
        case 64: return grouped_by_tile<64>(aq, as, row_index, R_max, K, w, ws, E, N, seg_off, bias, y, st);
        case 128: return grouped_by_tile<128>(aq, as, row_index, R_max, K, w, ws, E, N, seg_off, bias, y, st);
        default: return grouped_by_tile<256>(aq, as, row_index, R_max, K, w, ws, E, N, seg_off, bias, y, st);
    }
}

}  // namespace fni8h
