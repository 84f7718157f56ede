// W4A8 decode linear on MFMA with the per-token quantization fused in: 2 to 4
// tokens of fp16 activations against per_group_i4 weights in one launch
// (`fni8.linear` for int4 QTensors, fni8serve/layers/linear.py:8-10, :63-65).
//
// The kernel is w4a8_mfma_kernel (w4a8.hip) with a quantization prologue in
// place of the int8 activation stream:
//   * K is consumed in rounds of WAVES*SB slabs of 256 codes; wave w owns the
//     SB slabs from (r*WAVES + w)*SB of round r, so over the whole K each wave
//     owns PER = 2*PC slabs.  It reads the fp16 activations of exactly those
//     slabs (half a wave per slab, 8 elements per lane, whole 128-byte lines).
//   * Each token's max magnitude: integer max over the fp16 bits per lane, DPP
//     across the wave, one LDS barrier across the waves.
//   * Each wave quantizes its slabs into a private int8 area of LDS laid out
//     as the A operand of v_mfma_i32_16x16x64_i8: [slab][128-code half][MM
//     tokens][128 bytes], 16-byte chunks swizzled by token.  The quantization
//     is that of fni8_quantize_rowwise_f16 (division-free, the same bits);
//     workgroup 0 also writes xq and xs for the caller.
//   * The first weight round is issued before the row maxima and the second
//     right after their barrier, so both stream while the quantization runs.
//   * Products, group sums and the fold are w4a8_mfma_kernel's: exact int32
//     group sums, folded as fma((float)acc_g, ws[n, g], accf) in ascending g,
//     then y = fp16(accf * xs[m] (+ bias[n])).  The output bits therefore equal
//     a quantize launch followed by w4a8_mfma_kernel.
// Every workgroup quantizes all M rows for itself (M*K elements, a few hundred
// VALU cycles per wave); no workgroup waits for another.
#include <type_traits>

#include "w4a8_common.h"

namespace {

// PC: fp16 chunks per token per lane (half the wave's slabs, K = 512*WAVES*PC).
// MM: token rows of the int8 activation area; the MFMA A operand has 16 rows,
// tokens past M repeat token M-1 (computed, never stored).
template <int NB, int WAVES, int SB, int G, int PC, int MM = 4>
__global__ __launch_bounds__(WAVES * 64) void w4a8_mfma_fused_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int M, int K, const uint8_t* __restrict__ w,
    const float* __restrict__ ws, int N, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, int64_t ldy, int8_t* __restrict__ xq_out,
    float* __restrict__ xs_out) {
    constexpr int ROWS = 16 * NB;
    constexpr int TILE = ROWS * 128;          // the weight rows of one slab
    constexpr int KBG = G / 64;               // MFMA k-blocks per group
    constexpr int GPS = 256 / G;              // groups per slab
    constexpr int GPR = WAVES * SB * GPS;     // groups per round
    constexpr int EL = NB * 256;              // output elements of the workgroup (16 token rows)
    constexpr int EPT = EL / (WAVES * 64);    // folded by each thread
    constexpr int PER = 2 * PC;               // slabs per wave
    constexpr int NR = PER / SB;              // rounds
    constexpr int XAREA = PER * 2 * MM * 128;  // the wave's int8 activations
    constexpr bool KEEP = MM * PC <= 16;      // fp16 chunks kept in registers between passes
    static_assert(G >= 64 && G <= 256 && (WAVES == 1 || WAVES == 2 || WAVES == 4) &&
                      PER % SB == 0 && EL % (WAVES * 64) == 0 && MM <= 16,
                  "w4a8 fused mfma shape");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int32_t* gs = reinterpret_cast<int32_t*>(smem + WAVES * SB * TILE);  // [2][GPR][EL]
    int8_t* xarea = reinterpret_cast<int8_t*>(gs + 2 * GPR * EL);         // [WAVES][XAREA]
    uint32_t* amx = reinterpret_cast<uint32_t*>(xarea + WAVES * XAREA);  // [WAVES][MM]
    float* scl = reinterpret_cast<float*>(amx + WAVES * MM);             // [MM]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * ROWS;
    const int ng = K / G;
    const int rq = lane >> 3, c = lane & 7, r = lane & 15, g = lane >> 4;
    const int64_t kh = K >> 1;

    // first code of the wave's slab p
    auto kofs = [&](int p) -> int { return (((p / SB) * WAVES + wave) * SB + p % SB) * 256; };
    // chunk j of this lane: token j / PC, slab 2 * (j % PC) + (lane >> 5) of the
    // wave, elements (lane & 31) * 8 .. + 8 of that slab
    const int hs = lane >> 5, e8 = (lane & 31) * 8;
    auto xchunk = [&](int j) -> uint4 {
        const int m = j / PC;
        if (m < M)
            return *reinterpret_cast<const uint4*>(x + (int64_t)m * ldx + kofs(2 * (j % PC) + hs) +
                                                   e8);
        return make_uint4(0, 0, 0, 0);
    };

    // 1. activation loads first (the compiler then waits for them without
    //    waiting for the weight loads issued after)
    uint4 xv[KEEP ? MM * PC : 1];
    if constexpr (KEEP) {
#pragma unroll
        for (int j = 0; j < MM * PC; j++) xv[j] = xchunk(j);
    }

    // 2. first weight round.  Load lanes: weight row h*8 + rq (rows past N
    //    repeat row N-1, never stored), 16-byte chunk c of the slab.
    const uint8_t* wsrc[2 * NB];
    int woff[2 * NB];
#pragma unroll
    for (int h = 0; h < 2 * NB; h++) {
        const int row = h * 8 + rq;
        const int n = n0 + row < N ? n0 + row : N - 1;
        wsrc[h] = w + (int64_t)n * kh + (int64_t)wave * SB * 128 + c * 16;
        woff[h] = row * 128 + swz(row, c);
    }
    i32x4 wa[SB][2 * NB], wb[SB][2 * NB];
    auto load = [&](i32x4 (&dw)[SB][2 * NB], int rd) {
        const int64_t s = (int64_t)rd * WAVES * SB;
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < 2 * NB; h++)
                dw[j][h] = __builtin_nontemporal_load(
                    reinterpret_cast<const i32x4*>(wsrc[h] + (s + j) * 128));
    };
    load(wa, 0);

    // 3. row max magnitudes: one wave-uniform value per token, then across the waves
#pragma unroll
    for (int m = 0; m < MM; m++) {
        uint32_t mx = 0;
#pragma unroll
        for (int jj = 0; jj < PC; jj++)
            mx = fni8::amax_chunk(mx, KEEP ? xv[m * PC + jj] : xchunk(m * PC + jj));
        mx = fni8::wave_max_uniform(fni8::amax_fold(mx));
        if (lane == 0) amx[wave * MM + m] = mx;
    }
    lds_barrier();
    if constexpr (NR > 1) load(wb, 1);

    // 4. quantize this wave's slabs into its LDS area
    int8_t* xw = xarea + wave * XAREA;
#pragma unroll
    for (int m = 0; m < MM; m++) {
        uint32_t a = amx[m];
#pragma unroll
        for (int wv = 1; wv < WAVES; wv++) a = amx[wv * MM + m] > a ? amx[wv * MM + m] : a;
        const float sc = fni8::row_scale_from_bits(a);
        const bool live = m < M && __builtin_isfinite(sc);  // NaN/inf scale: every q is 0
        const float yr = 1.0f / sc;                          // correctly rounded (build flag)
        if (wave == 0 && lane == 0) {
            scl[m] = sc;
            if (blockIdx.x == 0 && m < M) xs_out[m] = sc;
        }
        if (m >= M) continue;
#pragma unroll
        for (int jj = 0; jj < PC; jj++) {
            const uint2 q = fni8::quant_chunk(KEEP ? xv[m * PC + jj] : xchunk(m * PC + jj), sc, yr, live);
            const int p = 2 * jj + hs, hf = e8 >> 7, b = e8 & 127;
            *reinterpret_cast<uint2*>(xw + ((p * 2 + hf) * MM + m) * 128 + swz(m, b >> 4) + (b & 15)) = q;
            if (blockIdx.x == 0)
                *reinterpret_cast<uint2*>(xq_out + (int64_t)m * K + kofs(p) + e8) = q;
        }
    }

    // operand lanes: k-block j of a slab is codes 64j..64j+63; lane (r, g)
    // holds codes 64j + 16g .. +15 of weight row / token r
    const int tok = r < M ? r : M - 1;
    int boff[NB][4], aoff[2];
#pragma unroll
    for (int j = 0; j < 4; j++)
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int row = b * 16 + r;
            boff[b][j] = row * 128 + swz(row, 2 * j + (g >> 1)) + 8 * (g & 1);
        }
#pragma unroll
    for (int q = 0; q < 2; q++) aoff[q] = tok * 128 + swz(tok, 4 * q + g);

    // 5. the weight stream, group sums and fold of w4a8_mfma_kernel
    int8_t* st = smem + wave * (SB * TILE);
    auto compute = [&](const i32x4 (&wv)[SB][2 * NB], int rd, int32_t* gsb) {
        // The tile and the activation area are private to the wave and LDS
        // executes a wave's accesses in order; the barriers only keep the
        // compiler from reordering across them.
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
            const int8_t* xa = xw + (rd * SB + j) * (2 * MM * 128);
#pragma unroll
            for (int gj = 0; gj < GPS; gj++) {
                i32x4 acc[NB];
#pragma unroll
                for (int b = 0; b < NB; b++) acc[b] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int kb = 0; kb < KBG; kb++) {
                    const int jb = gj * KBG + kb;
                    i32x4 bf[NB];
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const uint2 pk = *reinterpret_cast<const uint2*>(st + j * TILE + boff[b][jb]);
                        bf[b] = unpack16x16(pk.x, pk.y);
                    }
                    const i32x4 af =
                        *reinterpret_cast<const i32x4*>(xa + (jb >> 1) * (MM * 128) + aoff[jb & 1]);
#pragma unroll
                    for (int b = 0; b < NB; b++) acc[b] = fni8::mfma_i8(af, bf[b], acc[b]);
                }
                const int gl = (wave * SB + j) * GPS + gj;
#pragma unroll
                for (int b = 0; b < NB; b++)
                    *reinterpret_cast<i32x4*>(gsb + gl * EL + (b * 64 + lane) * 4) = acc[b];
            }
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };

    // fold ownership: element e = (k*WAVES + wave)*64 + lane of the MFMA
    // result layout [NB][64 lanes][4]: block (k*WAVES + wave) / 4, weight row
    // lane / 4 of it, token 4 * ((k*WAVES + wave) % 4) + lane % 4
    const float* wrow[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int n = n0 + b * 16 + (lane >> 2);
        wrow[b] = ws + (int64_t)(n < N ? n : N - 1) * ng;
    }
    float accf[EPT];
#pragma unroll
    for (int k = 0; k < EPT; k++) accf[k] = 0.0f;
    float wsv[NB][GPR];
    auto fold = [&](const int32_t* gsb) {
#pragma unroll
        for (int gl = 0; gl < GPR; gl++)
#pragma unroll
            for (int k = 0; k < EPT; k++) {
                const int b = ((k * WAVES) >> 2) % NB;  // (k*WAVES + wave) / 4: no carry
                const int32_t v = gsb[gl * EL + (k * WAVES + wave) * 64 + lane];
                accf[k] = __builtin_fmaf((float)(v >> 4), wsv[b][gl], accf[k]);
            }
    };

#pragma unroll 1
    for (int rd = 0; rd < NR; rd++) {
        if (rd > 0 && rd + 1 < NR) load(wb, rd + 1);  // rd = 1 is already in flight
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int gl = 0; gl < GPR; gl++) wsv[b][gl] = wrow[b][rd * GPR + gl];
        int32_t* gsb = gs + (rd & 1) * GPR * EL;
        compute(wa, rd, gsb);
        lds_barrier();
        fold(gsb);
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < 2 * NB; h++) wa[j][h] = wb[j][h];
    }

#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int mb = (k * WAVES) >> 2;
        const int n = n0 + (mb % NB) * 16 + (lane >> 2);
        const int m = 4 * (((k * WAVES) & 3) + wave) + (lane & 3);
        if (m < M && n < N) {
            float v = accf[k] * scl[m];
            if (bias) v = v + fni8::h2f(bias[n]);
            y[(int64_t)m * ldy + n] = fni8::f2h(v);
        }
    }
}

constexpr size_t kLdsLimit = 160 * 1024;

template <int NB, int WAVES, int SB, int G, int PC, int MM = 4>
constexpr size_t kFusedLds = (size_t)WAVES * SB * 16 * NB * 128 +               // weight tiles
                             (size_t)2 * WAVES * SB * (256 / G) * NB * 256 * 4 +  // group sums
                             (size_t)WAVES * 2 * PC * 2 * MM * 128 +             // activations
                             (size_t)WAVES * MM * 4 + MM * 4;                    // maxima, scales

template <int NB, int WAVES, int SB, int G, int PC>
int fused_launch(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const uint8_t* w,
                 const float* ws, int64_t N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                 int8_t* xq_out, float* xs_out, hipStream_t st) {
    constexpr size_t lds = kFusedLds<NB, WAVES, SB, G, PC>;
    if constexpr (lds > kLdsLimit) {
        return 1;
    } else {
        auto kern = &w4a8_mfma_fused_kernel<NB, WAVES, SB, G, PC>;
        if constexpr (lds > 64 * 1024) {
            static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                       hipFuncAttributeMaxDynamicSharedMemorySize,
                                                       (int)lds) == hipSuccess;
            if (!ok) {
                fni8h::set_error_detail("w4a8 fused mfma: cannot raise the LDS limit to %zu bytes",
                                        lds);
                return FNI8_ERR_LAUNCH;
            }
        }
        const dim3 grid((unsigned)((N + 16 * NB - 1) / (16 * NB)));
        hipLaunchKernelGGL(kern, grid, dim3(WAVES * 64), lds, st, x, ldx, (int)M, (int)K, w, ws,
                           (int)N, bias, y, ldy, xq_out, xs_out);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) {
            fni8h::set_error_detail("w4a8 fused mfma launch: %s", hipGetErrorString(e));
            return FNI8_ERR_LAUNCH;
        }
        return FNI8_OK;
    }
}

// One launch shape (16*NB weight rows, waves, slabs per round) for group size
// G: 1 when K does not split into whole rounds of it with an instantiated chunk
// count (1, 2, 3, 4, 6 or 8, at most PCMAX).
template <int NB, int WAVES, int SB, int G, int PCMAX>
int fused_shape(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const uint8_t* w,
                const float* ws, int64_t N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                int8_t* xq_out, float* xs_out, hipStream_t st) {
    if (K % (512 * WAVES) != 0) return 1;
    const int64_t pc = K / (512 * WAVES);
    if (pc > PCMAX || (2 * pc) % SB != 0) return 1;
#define FNI8_W4F(PCV)                                                                          \
    if constexpr (PCV <= PCMAX)                                                                \
        return fused_launch<NB, WAVES, SB, G, PCV>(x, ldx, M, K, w, ws, N, bias, y, ldy,       \
                                                   xq_out, xs_out, st);                        \
    return 1
    switch (pc) {
        case 1: FNI8_W4F(1);
        case 2: FNI8_W4F(2);
        case 3: FNI8_W4F(3);
        case 4: FNI8_W4F(4);
        case 6: FNI8_W4F(6);
        case 8: FNI8_W4F(8);
        default: return 1;
    }
#undef FNI8_W4F
}

// Launch shapes measured on MI355X over the Qwen3-8B linears at G = 128 (36
// weight copies, weights from HBM), against a quantize launch plus
// w4a8_mfma_kernel, µs at 2 / 3 / 4 tokens:
//   QKV  6144 x 4096: 6.93 / 7.32 / 7.63 (32 rows) against 8.86 / 8.89 / 8.95
//   O    4096 x 4096: 5.97 / 6.25 / 6.50 against 7.67 / 7.68 / 7.69
//   gate_up 24576 x 4096 (32 rows, two waves): 13.98 / 14.65 against 15.83 / 15.87;
//     16.29 against 15.86 at 4 tokens
//   down 4096 x 12288: 14.29 against 15.54 at 2 tokens; 16.52 / 18.61 against
//     15.58 / 15.62 at 3 / 4
// Every workgroup quantizes all M rows of K, so the fused form loses where that
// redundant work outgrows the launch it saves: long K from 3 tokens, wide N at
// 4.  Those shapes return 1 (quantize launch, then the MFMA kernel).
template <int G>
int fused_table(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const uint8_t* w,
                const float* ws, int64_t N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                int8_t* xq_out, float* xs_out, hipStream_t st) {
#define FNI8_W4FS(NBV, WV, SBV, PCM)                                                            \
    do {                                                                                        \
        const int rc = fused_shape<NBV, WV, SBV, G, PCM>(x, ldx, M, K, w, ws, N, bias, y, ldy,  \
                                                         xq_out, xs_out, st);                   \
        if (rc != 1) return rc;                                                                 \
    } while (0)
    if (K > 4096) {
        if (M == 2) FNI8_W4FS(1, 4, 2, 8);
        return 1;
    }
    if (N >= 16384) {
        if (M <= 3) FNI8_W4FS(2, 2, 1, 4);
        return 1;
    }
    if (M == 4 && N > 4096) FNI8_W4FS(2, 4, 2, 2);
    FNI8_W4FS(1, 4, 2, 2);
    FNI8_W4FS(1, 2, 1, 4);
#undef FNI8_W4FS
    return 1;
}

}  // namespace

namespace fni8h {

int launch_linear_w4a8_mfma_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                                  const uint8_t* w, const float* ws, int64_t N, int64_t G,
                                  const uint16_t* bias, uint16_t* y, int64_t ldy,
                                  int8_t* xq_out, float* xs_out, hipStream_t st) {
    if (M < 2 || M > 4 || K > 65536 || N > INT32_MAX) return 1;
    if (ldx % 8 != 0 || ((uintptr_t)x % 16) != 0 || ((uintptr_t)w % 16) != 0 ||
        ((uintptr_t)xq_out % 8) != 0)
        return 1;
    switch (G) {
        case 64: return fused_table<64>(x, ldx, M, K, w, ws, N, bias, y, ldy, xq_out, xs_out, st);
        case 128: return fused_table<128>(x, ldx, M, K, w, ws, N, bias, y, ldy, xq_out, xs_out, st);
        case 256: return fused_table<256>(x, ldx, M, K, w, ws, N, bias, y, ldy, xq_out, xs_out, st);
        default: return 1;
    }
}

}  // namespace fni8h
