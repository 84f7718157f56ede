// W4A8 linear (gfx950): int8 per-token activations against per_group_i4 weights,
// `gemm_w4a8` of `fni8.linear` for int4 QTensors (fni8serve/layers/linear.py:9,
// :63-65; weight format fni8serve/convert.py:69-79).
//
// Weights: packed uint8 [N, K/2], code k of row n in byte k/2 of the row, low
// nibble for even k, high nibble for odd k, each a 4-bit two's complement
// value in [-8, 7]; fp32 scales [N, K/G], one per group of G consecutive k.
//
// Arithmetic: acc_g = sum over the group of xq[m, k] * code[n, k] (exact
// int32); accf = fma((float)acc_g, ws[n, g], accf) over g = 0, 1, ... from
// accf = +0 (one rounding per group, ascending g); y = fp16(accf * xs[m]
// (+ bias[n])), one rounding per operation.
//
// Unpacking never reorders the codes: the low nibbles of a packed dword are
// the codes of k = 0, 2, 4, 6 of its 8-code block, the high nibbles those of
// k = 1, 3, 5, 7; the activations are split the same way (v_perm), and a dot
// product does not care in which order its terms come.  Sign extension of a
// nibble u in each byte is ((u ^ 8) + 0x78) ^ 0x80: the sum stays below 0x88,
// so no carry crosses a byte.
#include "w4a8_common.h"

namespace {

typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ uint32_t sext4(uint32_t u) {
    return ((u ^ 0x08080808u) + 0x78787878u) ^ 0x80808080u;
}

// One packed dword (8 codes) -> the codes of even k and of odd k, int8 x 4 each.
__device__ __forceinline__ void unpack8(uint32_t w, uint32_t& ev, uint32_t& od) {
    ev = sext4(w & 0x0f0f0f0fu);
    od = sext4((w >> 4) & 0x0f0f0f0fu);
}

// Activation bytes x0..x7 (lo = x0..x3, hi = x4..x7) -> (x0 x2 x4 x6), (x1 x3 x5 x7).
__device__ __forceinline__ void split8(uint32_t lo, uint32_t hi, uint32_t& ev, uint32_t& od) {
    ev = __builtin_amdgcn_perm(hi, lo, 0x06040200u);
    od = __builtin_amdgcn_perm(hi, lo, 0x07050301u);
}

__device__ __forceinline__ int dot4(uint32_t a, uint32_t b, int c) {
    return __builtin_amdgcn_sdot4((int)a, (int)b, c, false);
}

// ---- decode: dot4 GEMV, MT tokens ------------------------------------------
//
// The workgroup stages the MT activation rows in LDS, already split into even
// and odd k.  Each wave owns kRows weight rows; per iteration lane l streams
// 16 bytes (32 codes) of each row, chunk 64 * it + l, so a wave reads 1 KB of
// contiguous row per row and instruction.  A group is CPG = G / 32 adjacent
// lanes: their int32 sums are added exactly, written to LDS, and lane
// r * MT + m folds the iteration's groups of row r, token m into its fp32
// accumulator in ascending g.
constexpr int kGemvThreads = 256;
constexpr int kRows = 4;

// Orders a wave's LDS writes before its own lanes' later reads (DS operations
// of one wave complete in issue order); no other wave takes part.
__device__ __forceinline__ void wave_lds_sync() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0)
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

template <int MT, int CPG>
__global__ __launch_bounds__(kGemvThreads) void w4a8_gemv_kernel(
    const int8_t* __restrict__ xq, int64_t ldq, const float* __restrict__ xs, int K,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy) {
    extern __shared__ uint32_t xlds[];  // [MT][K / 8][2]: even, odd dwords
    constexpr int GPI = 64 / CPG;       // groups per iteration
    __shared__ int32_t gacc[kGemvThreads / 64][kRows * MT][GPI];
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int KB = K / 8;  // 8-code blocks per row

    for (int i = tid; i < MT * KB; i += kGemvThreads) {
        const int m = i / KB, b = i - m * KB;
        const uint2 v = *reinterpret_cast<const uint2*>(xq + (int64_t)m * ldq + 8 * b);
        uint32_t ev, od;
        split8(v.x, v.y, ev, od);
        xlds[2 * i] = ev;
        xlds[2 * i + 1] = od;
    }
    __syncthreads();

    const int n_base = (blockIdx.x * (kGemvThreads / 64) + wave) * kRows;
    const int KC = K / 32;  // 16-byte chunks per packed row
    const int ng = K / (32 * CPG);
    const int64_t row_bytes = K / 2;
    const uint8_t* wr[kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++) {
        const int n = n_base + r < N ? n_base + r : N - 1;
        wr[r] = w + (int64_t)n * row_bytes;
    }
    const int fr = lane / MT, fm = lane - fr * MT;  // the (row, token) this lane folds
    const int fn = n_base + fr;
    float accf = 0.0f;

    const int iters = (KC + 63) / 64;
    uint4 cur[kRows];
#pragma unroll
    for (int r = 0; r < kRows; r++)
        cur[r] = lane < KC ? *reinterpret_cast<const uint4*>(wr[r] + 16 * lane)
                           : make_uint4(0, 0, 0, 0);
    for (int it = 0; it < iters; it++) {
        const int c = it * 64 + lane;
        uint4 nxt[kRows];
        const int cn = c + 64;
#pragma unroll
        for (int r = 0; r < kRows; r++)
            nxt[r] = cn < KC ? *reinterpret_cast<const uint4*>(wr[r] + 16 * (int64_t)cn)
                             : make_uint4(0, 0, 0, 0);
        int acc[kRows][MT];
#pragma unroll
        for (int r = 0; r < kRows; r++)
#pragma unroll
            for (int m = 0; m < MT; m++) acc[r][m] = 0;
        if (c < KC) {
#pragma unroll
            for (int d = 0; d < 4; d++) {
                uint32_t xe[MT], xo[MT];
#pragma unroll
                for (int m = 0; m < MT; m++) {
                    const uint2 xv = *reinterpret_cast<const uint2*>(xlds + 2 * (m * KB + 4 * c + d));
                    xe[m] = xv.x;
                    xo[m] = xv.y;
                }
#pragma unroll
                for (int r = 0; r < kRows; r++) {
                    const uint32_t wd = d == 0 ? cur[r].x : d == 1 ? cur[r].y : d == 2 ? cur[r].z : cur[r].w;
                    uint32_t ev, od;
                    unpack8(wd, ev, od);
#pragma unroll
                    for (int m = 0; m < MT; m++) acc[r][m] = dot4(od, xo[m], dot4(ev, xe[m], acc[r][m]));
                }
            }
        }
#pragma unroll
        for (int d = 1; d < CPG; d <<= 1)
#pragma unroll
            for (int r = 0; r < kRows; r++)
#pragma unroll
                for (int m = 0; m < MT; m++) acc[r][m] += __shfl_xor(acc[r][m], d, 64);
        if ((lane % CPG) == 0 && c < KC) {
#pragma unroll
            for (int r = 0; r < kRows; r++)
#pragma unroll
                for (int m = 0; m < MT; m++) gacc[wave][r * MT + m][lane / CPG] = acc[r][m];
        }
        wave_lds_sync();  // the group sums live in this wave's rows of gacc only
        if (lane < kRows * MT && fn < N) {
            const int g0 = it * GPI;
            const int cnt = ng - g0 < GPI ? ng - g0 : GPI;
            const float* wsr = ws + (int64_t)fn * ng + g0;
            for (int q = 0; q < cnt; q++)
                accf = __builtin_fmaf((float)gacc[wave][lane][q], wsr[q], accf);
        }
        wave_lds_sync();  // the folds have read gacc before the next iteration writes it
#pragma unroll
        for (int r = 0; r < kRows; r++) cur[r] = nxt[r];
    }
    if (lane < kRows * MT && fn < N) {
        float v = accf * xs[fm];
        if (bias) v = v + fni8::h2f(bias[fn]);
        y[(int64_t)fm * ldy + fn] = fni8::f2h(v);
    }
}

// ---- decode: streaming GEMV with full-line loads -----------------------------
//
// The layout of the W8A8 decode GEMV: a workgroup owns 8 * RH weight rows and
// its WAVES waves split K into equal shares of 128-byte packed slabs (256
// codes).  Every wave load instruction covers 8 rows x 128 contiguous bytes
// (lane l: row l / 8, bytes 16 (l % 8) .. + 16 of a slab), non-temporal and
// double-buffered SB slabs ahead.  Lane l dots its 32 codes with the
// activations (LDS, split into even / odd k); the CPG lanes of a group add
// their sums exactly (DPP), and the group's leader stores it in LDS.  After
// the stream, thread j * M + m folds row j, token m in ascending group order.
// FUSED: x arrives as fp16 and is quantized here (the per-token quantization
// of fni8_quantize_rowwise_f16, division-free, same bits); workgroup 0 also
// writes xq and xs for the caller.
// EB: the prologue's barriers wait for LDS traffic only, and the second weight
// batch is issued before the quantization, so its latency overlaps that VALU work.
template <int MM, int RH, int WAVES, int SB, int KCH, int CPG, bool FUSED, bool EB = false>
__global__ __launch_bounds__(WAVES * 64) void w4a8_stream_kernel(
    const void* __restrict__ xin, int64_t ldx, const float* __restrict__ xs_in, int M, int K,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int8_t* __restrict__ xq_out, float* __restrict__ xs_out) {
    constexpr int NT = WAVES * 64;
    constexpr int ROWS = RH * 8;
    constexpr int GPS = 8 / CPG;  // groups per slab
    extern __shared__ __attribute__((aligned(16))) uint32_t lds[];
    const int KB = K >> 3;        // 8-code blocks per row
    const int ng = K / (32 * CPG);
    uint32_t* xl = lds;                                           // [MM][KB][2]
    int32_t* gsum = reinterpret_cast<int32_t*>(lds + 2 * MM * KB);  // [ROWS][MM][ng]
    float* scl = reinterpret_cast<float*>(gsum + ROWS * MM * ng);   // [MM]
    uint32_t* amx = reinterpret_cast<uint32_t*>(scl + MM);          // [WAVES][MM]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * ROWS;
    const int rq = lane >> 3, c = lane & 7;
    const int per = (K >> 8) / WAVES;  // slabs per wave (the launcher makes it exact)
    const int s0 = wave * per;
    const int nb = per / SB;
    const uint8_t* wsrc[RH];
#pragma unroll
    for (int h = 0; h < RH; h++) {
        int n = n0 + h * 8 + rq;
        n = n < N ? n : N - 1;
        wsrc[h] = w + (int64_t)n * (K >> 1) + (int64_t)s0 * 128 + c * 16;
    }
    i32x4 wa[SB][RH], wb[SB][RH];
    auto load = [&](i32x4 (&dst)[SB][RH], int b) {
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < RH; h++)
                dst[j][h] = __builtin_nontemporal_load(
                    reinterpret_cast<const i32x4*>(wsrc[h] + (int64_t)(b * SB + j) * 128));
    };

    // ---- activations into LDS: int8, split into even / odd k ----------------
    if constexpr (FUSED) {
        const uint16_t* x = reinterpret_cast<const uint16_t*>(xin);
        uint4 xr[MM][KCH];
#pragma unroll
        for (int m = 0; m < MM; m++)
#pragma unroll
            for (int i = 0; i < KCH; i++) {
                const int ch = tid + i * NT;
                const int mr = m < M ? m : 0, cc = ch < KB ? ch : KB - 1;
                const uint4 v = *reinterpret_cast<const uint4*>(x + (int64_t)mr * ldx + cc * 8);
                xr[m][i] = (m < M && ch < KB) ? v : make_uint4(0, 0, 0, 0);
            }
        load(wa, 0);
#pragma unroll
        for (int m = 0; m < MM; m++) {
            uint32_t am = 0;
#pragma unroll
            for (int i = 0; i < KCH; i++) am = fni8::amax_chunk(am, xr[m][i]);
            am = fni8::wave_max_uniform(fni8::amax_fold(am));
            if (lane == 0) amx[wave * MM + m] = am;
        }
        if constexpr (EB) {
            lds_barrier();
            if (nb > 1) load(wb, 1);
        } else {
            __syncthreads();
        }
#pragma unroll
        for (int m = 0; m < MM; m++) {
            uint32_t a = amx[m];
#pragma unroll
            for (int wv = 1; wv < WAVES; wv++) a = amx[wv * MM + m] > a ? amx[wv * MM + m] : a;
            const float sc = fni8::row_scale_from_bits(a);
            const bool live = m < M && __builtin_isfinite(sc);
            const float yr = 1.0f / sc;
            if (tid == 0) {
                scl[m] = sc;
                if (xs_out != nullptr && blockIdx.x == 0 && m < M) xs_out[m] = sc;
            }
#pragma unroll
            for (int i = 0; i < KCH; i++) {
                const int ch = tid + i * NT;
                if (ch < KB) {
                    const uint2 q = fni8::quant_chunk(xr[m][i], sc, yr, live);
                    uint2 eo;
                    split8(q.x, q.y, eo.x, eo.y);
                    *reinterpret_cast<uint2*>(xl + 2 * (m * KB + ch)) = eo;
                    if (xq_out != nullptr && blockIdx.x == 0 && m < M)
                        *reinterpret_cast<uint2*>(xq_out + (int64_t)m * K + ch * 8) = q;
                }
            }
        }
    } else {
        const int8_t* xq = reinterpret_cast<const int8_t*>(xin);
        load(wa, 0);
        for (int i = tid; i < MM * KB; i += NT) {
            const int m = i / KB, b = i - m * KB;
            uint2 eo = make_uint2(0, 0);
            if (m < M) {
                const uint2 v = *reinterpret_cast<const uint2*>(xq + (int64_t)m * ldx + 8 * b);
                split8(v.x, v.y, eo.x, eo.y);
            }
            *reinterpret_cast<uint2*>(xl + 2 * i) = eo;
        }
        if (tid < MM) scl[tid] = tid < M ? xs_in[tid] : 0.f;
        if (EB && nb > 1) load(wb, 1);
    }
    if constexpr (EB)
        lds_barrier();
    else
        __syncthreads();

    // ---- weight stream: per-slab group sums into LDS -------------------------
    auto compute = [&](const i32x4 (&wv)[SB][RH], int b) {
#pragma unroll
        for (int j = 0; j < SB; j++) {
            const int slab = s0 + b * SB + j;
            uint4 xv[MM][2];
#pragma unroll
            for (int m = 0; m < MM; m++) {
                const uint32_t* src = xl + 2 * (m * KB + slab * 32 + c * 4);
                xv[m][0] = *reinterpret_cast<const uint4*>(src);
                xv[m][1] = *reinterpret_cast<const uint4*>(src + 4);
            }
#pragma unroll
            for (int h = 0; h < RH; h++) {
                const uint32_t w4[4] = {(uint32_t)wv[j][h][0], (uint32_t)wv[j][h][1],
                                        (uint32_t)wv[j][h][2], (uint32_t)wv[j][h][3]};
                uint32_t ev[4], od[4];
#pragma unroll
                for (int d = 0; d < 4; d++) unpack8(w4[d], ev[d], od[d]);
#pragma unroll
                for (int m = 0; m < MM; m++) {
                    int a = 0;
                    a = dot4(ev[0], xv[m][0].x, a);
                    a = dot4(od[0], xv[m][0].y, a);
                    a = dot4(ev[1], xv[m][0].z, a);
                    a = dot4(od[1], xv[m][0].w, a);
                    a = dot4(ev[2], xv[m][1].x, a);
                    a = dot4(od[2], xv[m][1].y, a);
                    a = dot4(ev[3], xv[m][1].z, a);
                    a = dot4(od[3], xv[m][1].w, a);
                    if (CPG >= 2) a += fni8::dpp<fni8::kDppXor1>(a);
                    if (CPG >= 4) a += fni8::dpp<fni8::kDppXor2>(a);
                    if (CPG >= 8) a += fni8::dpp<fni8::kDppHalfMirror>(a);
                    if ((c % CPG) == 0)
                        gsum[((h * 8 + rq) * MM + m) * ng + slab * GPS + c / CPG] = a;
                }
            }
        }
    };
    for (int b = 0; b < nb - 1; b++) {
        if (!EB || b > 0) load(wb, b + 1);  // with EB, batch 1 went out in the prologue
        compute(wa, b);
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < RH; h++) wa[j][h] = wb[j][h];
    }
    compute(wa, nb - 1);
    __syncthreads();

    // ---- fold: one thread per (row, token), groups in ascending order --------
    if (tid < ROWS * M) {
        const int ej = tid % ROWS, em = tid / ROWS;
        const int n = n0 + ej;
        if (n < N) {
            const int32_t* gs = gsum + (ej * MM + em) * ng;
            const float* wr = ws + (int64_t)n * ng;
            float accf = 0.0f;
            for (int g = 0; g < ng; g++) accf = __builtin_fmaf((float)gs[g], wr[g], accf);
            float v = accf * scl[em];
            if (bias) v = v + fni8::h2f(bias[n]);
            y[(int64_t)em * ldy + n] = fni8::f2h(v);
        }
    }
}

// ---- decode on MFMA: int8 activations, up to 64 tokens -----------------------
//
// The W8A8 decode layout with packed weights.  A workgroup owns 16*NB weight
// rows.  One load instruction covers 8 rows x 128 packed bytes (a "slab" of
// 256 codes per row), or 8 tokens x 128 activation bytes, so every load
// touches whole cache lines.  Both go through a wave-private LDS tile
// (16-byte chunks XOR-swizzled by row, conflict-free both ways) and come back
// in the operand layout of v_mfma_i32_16x16x64_i8.
//
// Unpacking: a lane's B operand for one 64-code k-block is 16 codes of one
// row in natural k order, 8 packed bytes.  Each nibble is moved to the high
// half of its byte, where the byte reads as int8 16 * code exactly (the nibble
// is two's complement).  The MFMA then sums 16 * acc_g, and an arithmetic
// shift by 4 recovers acc_g exactly (|acc_g| <= 127 * 8 * 256).  Per packed
// dword that is one shift, two v_perm and two masks, with no sign-extension.
//
// The fold needs each group's exact sum in ascending g, while the waves of a
// workgroup split K.  They do so in rounds: round r covers WAVES*SB slabs and
// wave w the SB slabs from (r*WAVES + w)*SB.  Each wave writes its groups'
// int32 sums to LDS.  After one barrier, every thread folds its own output
// elements through the round's groups in order.  The group-sum area is double
// buffered, so one barrier per round suffices: a wave writes round r+2's sums
// only after the barrier of round r+1, and every thread reaches that barrier
// after folding round r.  (swz, unpack16x16: w4a8_common.h.)

template <int MT, int NB, int WAVES, int SB, int G>
__global__ __launch_bounds__(WAVES * 64) void w4a8_mfma_kernel(
    const int8_t* __restrict__ xq, int64_t ldx, const float* __restrict__ xs, int M, int K,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy) {
    constexpr int ROWS = 16 * NB, TOK = 16 * MT;
    constexpr int TILE = (ROWS + 2 * TOK) * 128;  // weight rows, then 2 activation halves per token
    constexpr int KBG = G / 64;                    // MFMA k-blocks per group
    constexpr int GPS = 256 / G;                   // groups per slab
    constexpr int GPR = WAVES * SB * GPS;          // groups per round
    constexpr int EL = MT * NB * 256;              // output elements of the workgroup
    constexpr int EPT = EL / (WAVES * 64);         // folded by each thread
    // WAVES in {1, 2, 4}: then (k*WAVES + wave) / 4 == (k*WAVES) / 4 for every
    // wave, which keeps each thread's weight-row block a compile-time constant
    static_assert(G >= 64 && G <= 256 && (WAVES == 1 || WAVES == 2 || WAVES == 4) &&
                      EL % (WAVES * 64) == 0, "w4a8 mfma shape");
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int32_t* gs = reinterpret_cast<int32_t*>(smem + WAVES * SB * TILE);  // [2][GPR][EL]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * ROWS;
    const int ng = K / G;
    const int rounds = (K >> 8) / (WAVES * SB);
    const int rq = lane >> 3, c = lane & 7, r = lane & 15, g = lane >> 4;
    const int64_t kh = K >> 1;

    // load lanes: weight row h*8 + rq (rows past N repeat row N-1, never
    // stored), activation token h*8 + rq (past M repeats M-1), chunk c
    const uint8_t* wsrc[2 * NB];
    int woff[2 * NB];
#pragma unroll
    for (int h = 0; h < 2 * NB; h++) {
        const int row = h * 8 + rq;
        const int n = n0 + row < N ? n0 + row : N - 1;
        wsrc[h] = w + (int64_t)n * kh + (int64_t)wave * SB * 128 + c * 16;
        woff[h] = row * 128 + swz(row, c);
    }
    const int8_t* xsrc[2 * MT];
    int xoff[2 * MT][2];
#pragma unroll
    for (int h = 0; h < 2 * MT; h++) {
        const int tok = h * 8 + rq;
        xsrc[h] = xq + (int64_t)(tok < M ? tok : M - 1) * ldx + (int64_t)wave * SB * 256 + c * 16;
#pragma unroll
        for (int p = 0; p < 2; p++) {
            const int row = ROWS + p * TOK + tok;
            xoff[h][p] = row * 128 + swz(row, c);
        }
    }
    // operand lanes: k-block j of the slab is codes 64j..64j+63; lane (r, g)
    // holds codes 64j + 16g .. +15 of weight row / token r
    int boff[NB][4], aoff[MT][4];
#pragma unroll
    for (int j = 0; j < 4; j++) {
#pragma unroll
        for (int b = 0; b < NB; b++) {
            const int row = b * 16 + r;
            boff[b][j] = row * 128 + swz(row, 2 * j + (g >> 1)) + 8 * (g & 1);
        }
#pragma unroll
        for (int mt = 0; mt < MT; mt++) {
            const int row = ROWS + (j >> 1) * TOK + mt * 16 + r;
            aoff[mt][j] = row * 128 + swz(row, 4 * (j & 1) + g);
        }
    }

    i32x4 wa[SB][2 * NB], wb[SB][2 * NB];
    i32x4 xa[SB][4 * MT], xb[SB][4 * MT];
    auto load = [&](i32x4 (&dw)[SB][2 * NB], i32x4 (&dx)[SB][4 * MT], int rd) {
        const int64_t s = (int64_t)rd * WAVES * SB;
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < 2 * NB; h++)
                dw[j][h] = __builtin_nontemporal_load(
                    reinterpret_cast<const i32x4*>(wsrc[h] + (s + j) * 128));
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < 2 * MT; h++)
                if (h * 8 < M)  // load groups wholly past the last token are skipped
#pragma unroll
                    for (int p = 0; p < 2; p++)
                        dx[j][2 * h + p] =
                            *reinterpret_cast<const i32x4*>(xsrc[h] + (s + j) * 256 + p * 128);
    };

    int8_t* st = smem + wave * (SB * TILE);
    auto compute = [&](const i32x4 (&wv)[SB][2 * NB], const i32x4 (&xv)[SB][4 * MT], int32_t* gsb) {
        // The tile is private to the wave and LDS executes a wave's accesses in
        // order; the barriers only keep the compiler from reordering across them.
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int h = 0; h < 2 * NB; h++) *reinterpret_cast<i32x4*>(st + j * TILE + woff[h]) = wv[j][h];
#pragma unroll
            for (int h = 0; h < 2 * MT; h++)
                if (h * 8 < M)  // rows past the last token keep stale values (never stored)
#pragma unroll
                    for (int p = 0; p < 2; p++)
                        *reinterpret_cast<i32x4*>(st + j * TILE + xoff[h][p]) = xv[j][2 * h + p];
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int gj = 0; gj < GPS; gj++) {
                i32x4 acc[MT][NB];
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int b = 0; b < NB; b++) acc[mt][b] = i32x4{0, 0, 0, 0};
#pragma unroll
                for (int kb = 0; kb < KBG; kb++) {
                    const int jb = gj * KBG + kb;
                    i32x4 bf[NB], af[MT];
#pragma unroll
                    for (int b = 0; b < NB; b++) {
                        const uint2 pk = *reinterpret_cast<const uint2*>(st + j * TILE + boff[b][jb]);
                        bf[b] = unpack16x16(pk.x, pk.y);
                    }
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
                        af[mt] = *reinterpret_cast<const i32x4*>(st + j * TILE + aoff[mt][jb]);
#pragma unroll
                    for (int mt = 0; mt < MT; mt++)
#pragma unroll
                        for (int b = 0; b < NB; b++) acc[mt][b] = fni8::mfma_i8(af[mt], bf[b], acc[mt][b]);
                }
                const int gl = (wave * SB + j) * GPS + gj;
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int b = 0; b < NB; b++)
                        *reinterpret_cast<i32x4*>(gsb + gl * EL + ((mt * NB + b) * 64 + lane) * 4) =
                            acc[mt][b];
            }
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };

    // fold ownership: element e = (k*WAVES + wave)*64 + lane of the MFMA
    // result layout [MT*NB][64 lanes][4]: block (k*WAVES + wave) / 4, weight
    // row lane / 4 of it, token 4 * ((k*WAVES + wave) % 4) + lane % 4
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

    load(wa, xa, 0);
    for (int rd = 0; rd < rounds; rd++) {
        if (rd + 1 < rounds) load(wb, xb, rd + 1);
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int gl = 0; gl < GPR; gl++) wsv[b][gl] = wrow[b][rd * GPR + gl];
        int32_t* gsb = gs + (rd & 1) * GPR * EL;
        compute(wa, xa, gsb);
        lds_barrier();
        fold(gsb);
#pragma unroll
        for (int j = 0; j < SB; j++) {
#pragma unroll
            for (int h = 0; h < 2 * NB; h++) wa[j][h] = wb[j][h];
#pragma unroll
            for (int h = 0; h < 4 * MT; h++) xa[j][h] = xb[j][h];
        }
    }

#pragma unroll
    for (int k = 0; k < EPT; k++) {
        const int mb = (k * WAVES) >> 2;
        const int n = n0 + (mb % NB) * 16 + (lane >> 2);
        const int m = (mb / NB) * 16 + 4 * (((k * WAVES) & 3) + wave) + (lane & 3);
        if (m < M && n < N) {
            float v = accf[k] * xs[m];
            if (bias) v = v + fni8::h2f(bias[n]);
            y[(int64_t)m * ldy + n] = fni8::f2h(v);
        }
    }
}

// ---- prefill: MFMA tile, group-wise fp32 fold --------------------------------
//
// Workgroup of 4 waves (2 x 2) over a BM x BN tile; each wave a (BM/2) x (BN/2)
// block of 32x32 accumulators.  K is consumed in steps of KS = min(G, 128)
// codes: the activation step (split into even / odd k) and the unpacked weight
// step go to LDS and the 32x32x32 int8 MFMAs add them into int32
// accumulators; after the last step of a group every accumulator is folded
// into its fp32 sum with the group scale of its column and reset.  The next
// step's global loads are in flight during the current step's MFMAs.
// GROUPED: the expert-segment form (the MoE layer's projections, one launch):
// blockIdx.x is one BM-row tile of one expert's sorted segment, blockIdx.y the
// column tile; sorted row r reads activation row rmap[r] (row r without a map)
// and its scale; weights, scales and bias are stacked per expert.
template <int BM, int BN, int G, bool GROUPED = false>
__global__ __launch_bounds__(256) void w4a8_tile_kernel(
    const int8_t* __restrict__ xq, int64_t ldq, const float* __restrict__ xs,
    const int32_t* __restrict__ rmap, int M, int K, const uint8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int E, const int32_t* __restrict__ seg_off,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy) {
    constexpr int NT = 256;
    constexpr int KS = G < 128 ? G : 128;   // codes per K-step
    constexpr int SPG = G / KS;             // steps per group
    constexpr int LDSR = KS + 16;           // padded LDS row (bytes)
    constexpr int WTM = BM / 2, WTN = BN / 2;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int A_TOT = BM * (KS / 16), B_TOT = BN * (KS / 32);  // 16-byte chunks per step
    constexpr int A_CH = (A_TOT + NT - 1) / NT, B_CH = (B_TOT + NT - 1) / NT;
    __shared__ __attribute__((aligned(16))) int8_t smem[(BM + BN) * LDSR];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 1, wn = wave & 1;
    const int ng = K / G;
    const int nsteps = K / KS;
    // output rows [m0, mend)
    int m0 = blockIdx.y * BM, mend = M, n0 = blockIdx.x * BN;
    if constexpr (GROUPED) {
        // every wave finds the same tile; past the last tile the whole
        // workgroup leaves before any barrier
        int e, r0, r1;
        if (!fni8::find_group_tile(seg_off, E, BM, blockIdx.x, M, e, r0, r1)) return;
        m0 = r0;
        mend = r1;
        n0 = blockIdx.y * BN;
        w += (int64_t)e * N * (K / 2);
        ws += (int64_t)e * N * ng;
        if (bias != nullptr) bias += (int64_t)e * N;
    }
    // activation row of output row r
    auto src_row = [&](int r) -> int {
        if constexpr (GROUPED) return rmap != nullptr ? rmap[r] : r;
        return r;
    };

    const int8_t* asrc[A_CH];
    const uint8_t* bsrc[B_CH];
#pragma unroll
    for (int i = 0; i < A_CH; i++) {
        const int c = (tid + i * NT) % A_TOT;  // threads past the step's chunks repeat one
        int mr = m0 + c / (KS / 16);
        mr = mr < mend ? mr : mend - 1;
        asrc[i] = xq + (int64_t)src_row(mr) * ldq + (c % (KS / 16)) * 16;
    }
#pragma unroll
    for (int i = 0; i < B_CH; i++) {
        const int c = (tid + i * NT) % B_TOT;
        int nr = n0 + c / (KS / 32);
        nr = nr < N ? nr : N - 1;
        bsrc[i] = w + (int64_t)nr * (K / 2) + (c % (KS / 32)) * 16;
    }
    uint4 ra[A_CH], rb[B_CH];
    auto gload = [&](int s) {
#pragma unroll
        for (int i = 0; i < A_CH; i++) ra[i] = *reinterpret_cast<const uint4*>(asrc[i] + (int64_t)s * KS);
#pragma unroll
        for (int i = 0; i < B_CH; i++)
            rb[i] = *reinterpret_cast<const uint4*>(bsrc[i] + (int64_t)s * (KS / 2));
    };
    auto sstore = [&]() {
#pragma unroll
        for (int i = 0; i < A_CH; i++) {
            const int c = tid + i * NT;
            if (A_TOT % NT != 0 && c >= A_TOT) continue;
            uint4 o;
            split8(ra[i].x, ra[i].y, o.x, o.y);
            split8(ra[i].z, ra[i].w, o.z, o.w);
            *reinterpret_cast<uint4*>(smem + (c / (KS / 16)) * LDSR + (c % (KS / 16)) * 16) = o;
        }
#pragma unroll
        for (int i = 0; i < B_CH; i++) {
            const int c = tid + i * NT;
            if (B_TOT % NT != 0 && c >= B_TOT) continue;
            uint4 o0, o1;
            unpack8(rb[i].x, o0.x, o0.y);
            unpack8(rb[i].y, o0.z, o0.w);
            unpack8(rb[i].z, o1.x, o1.y);
            unpack8(rb[i].w, o1.z, o1.w);
            int8_t* dst = smem + (BM + c / (KS / 32)) * LDSR + (c % (KS / 32)) * 32;
            *reinterpret_cast<uint4*>(dst) = o0;
            *reinterpret_cast<uint4*>(dst + 16) = o1;
        }
    };

    i32x16 acc[FM][FN];
    float accf[FM][FN][16];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            acc[i][j] = i32x16{};
#pragma unroll
            for (int r = 0; r < 16; r++) accf[i][j][r] = 0.0f;
        }

    // the group scales of this lane's accumulator columns
    const float* wsc[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        int n = n0 + wn * WTN + j * 32 + (lane & 31);
        n = n < N ? n : N - 1;
        wsc[j] = ws + (int64_t)n * ng;
    }

    const int fo = (lane & 31) * LDSR + (lane >> 5) * 16;
    gload(0);
    for (int s = 0; s < nsteps; s++) {
        sstore();
        __syncthreads();
        if (s + 1 < nsteps) gload(s + 1);
        const int8_t* ab = smem + (wm * WTM) * LDSR + fo;
        const int8_t* bb = smem + (BM + wn * WTN) * LDSR + fo;
#pragma unroll
        for (int ks = 0; ks < KS / 32; ks++) {
            i32x4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; i++)
                af[i] = *reinterpret_cast<const i32x4*>(ab + i * 32 * LDSR + ks * 32);
#pragma unroll
            for (int j = 0; j < FN; j++)
                bf[j] = *reinterpret_cast<const i32x4*>(bb + j * 32 * LDSR + ks * 32);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
        if ((s + 1) % SPG == 0) {
            const int g = s / SPG;
            float wsv[FN];
#pragma unroll
            for (int j = 0; j < FN; j++) wsv[j] = wsc[j][g];
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) {
#pragma unroll
                    for (int r = 0; r < 16; r++)
                        accf[i][j][r] = __builtin_fmaf((float)acc[i][j][r], wsv[j], accf[i][j][r]);
                    acc[i][j] = i32x16{};
                }
        }
        __syncthreads();
    }

    // lane l, register r of block (i, j): row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int mr = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (mr >= mend) continue;
            const float asc = xs[src_row(mr)];
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int n = n0 + wn * WTN + j * 32 + (lane & 31);
                if (n >= N) continue;
                float v = accf[i][j][r] * asc;
                if (bias) v = v + fni8::h2f(bias[n]);
                y[(int64_t)mr * ldy + n] = fni8::f2h(v);
            }
        }
}

// ---- prefill: 8-wave MFMA tile, two LDS stages -------------------------------
//
// The W8A8 prefill pipeline (8 waves as 2 x 4, two LDS stages, global loads
// staged in registers, LDS-only barriers) with the group-wise fold.  A BM x BN
// = 128 x 256 tile gives each wave a 64 x 64 block: int32 accumulators for the
// current group plus fp32 running sums, 128 registers.  A K-step is KS =
// min(G, 128) codes.  The packed weight step is unpacked as it goes to LDS,
// each nibble into the high half of its byte (16 * code, natural k order), so
// the activations go to LDS unchanged; the sums come out 16x and an
// arithmetic shift restores them exactly before the fold.  With two waves per
// SIMD, one wave's fold overlaps the other's MFMAs.
template <int BM, int BN, int G>
__global__ __launch_bounds__(512) void w4a8_tile8_kernel(
    const int8_t* __restrict__ xq, int64_t ldq, const float* __restrict__ xs, int M, int K,
    const uint8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy) {
    constexpr int NT = 512;
    constexpr int KS = G < 128 ? G : 128;  // codes per K-step
    constexpr int SPG = G / KS;            // steps per group
    constexpr int LDSR = KS + 16;          // padded LDS row (bytes)
    constexpr int WTM = BM / 2, WTN = BN / 4;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int A_TOT = BM * (KS / 16), B_TOT = BN * (KS / 32);  // 16-byte chunks per step
    constexpr int A_CH = (A_TOT + NT - 1) / NT, B_CH = (B_TOT + NT - 1) / NT;
    constexpr int STAGE = (BM + BN) * LDSR;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];

    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
    const int wm = wave >> 2, wn = wave & 3;
    const int m0 = blockIdx.y * BM, n0 = blockIdx.x * BN;
    const int ng = K / G, nsteps = K / KS;

    // rows past the end repeat the last valid row (their results are never
    // stored); threads past a step's chunk count repeat a chunk and skip the store
    const int8_t* asrc[A_CH];
    const uint8_t* bsrc[B_CH];
#pragma unroll
    for (int i = 0; i < A_CH; i++) {
        const int c = (tid + i * NT) % A_TOT;
        int mr = m0 + c / (KS / 16);
        mr = mr < M ? mr : M - 1;
        asrc[i] = xq + (int64_t)mr * ldq + (c % (KS / 16)) * 16;
    }
#pragma unroll
    for (int i = 0; i < B_CH; i++) {
        const int c = (tid + i * NT) % B_TOT;
        int nr = n0 + c / (KS / 32);
        nr = nr < N ? nr : N - 1;
        bsrc[i] = w + (int64_t)nr * (K / 2) + (c % (KS / 32)) * 16;
    }
    uint4 ra[A_CH], rb[B_CH];
    auto gload = [&](int s) {
#pragma unroll
        for (int i = 0; i < A_CH; i++) ra[i] = *reinterpret_cast<const uint4*>(asrc[i] + (int64_t)s * KS);
#pragma unroll
        for (int i = 0; i < B_CH; i++)
            rb[i] = *reinterpret_cast<const uint4*>(bsrc[i] + (int64_t)s * (KS / 2));
    };
    auto sstore = [&](int buf) {
        int8_t* st = smem + buf * STAGE;
#pragma unroll
        for (int i = 0; i < A_CH; i++) {
            const int c = tid + i * NT;
            if (A_TOT % NT != 0 && c >= A_TOT) continue;
            *reinterpret_cast<uint4*>(st + (c / (KS / 16)) * LDSR + (c % (KS / 16)) * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; i++) {
            const int c = tid + i * NT;
            if (B_TOT % NT != 0 && c >= B_TOT) continue;
            int8_t* dst = st + (BM + c / (KS / 32)) * LDSR + (c % (KS / 32)) * 32;
            *reinterpret_cast<i32x4*>(dst) = unpack16x16(rb[i].x, rb[i].y);
            *reinterpret_cast<i32x4*>(dst + 16) = unpack16x16(rb[i].z, rb[i].w);
        }
    };

    i32x16 acc[FM][FN];
    float accf[FM][FN][16];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) {
            acc[i][j] = i32x16{};
#pragma unroll
            for (int r = 0; r < 16; r++) accf[i][j][r] = 0.0f;
        }
    const float* wsc[FN];
#pragma unroll
    for (int j = 0; j < FN; j++) {
        int n = n0 + wn * WTN + j * 32 + (lane & 31);
        n = n < N ? n : N - 1;
        wsc[j] = ws + (int64_t)n * ng;
    }

    // fragment read: lane l takes row l % 32 of a 32-row block and bytes
    // 16 * (l / 32) of each 32-byte sub-step (the 32x32x32 operand layout)
    const int fo = (lane & 31) * LDSR + (lane >> 5) * 16;
    auto compute = [&](int buf) {
        const int8_t* ab = smem + buf * STAGE + (wm * WTM) * LDSR + fo;
        const int8_t* bb = smem + buf * STAGE + (BM + wn * WTN) * LDSR + fo;
#pragma unroll
        for (int ks = 0; ks < KS / 32; ks++) {
            i32x4 af[FM], bf[FN];
#pragma unroll
            for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const i32x4*>(ab + i * 32 * LDSR + ks * 32);
#pragma unroll
            for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const i32x4*>(bb + j * 32 * LDSR + ks * 32);
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
                    acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(af[i], bf[j], acc[i][j], 0, 0, 0);
        }
    };
    auto fold = [&](int g) {
        float wsv[FN];
#pragma unroll
        for (int j = 0; j < FN; j++) wsv[j] = wsc[j][g];
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) {
#pragma unroll
                for (int r = 0; r < 16; r++)
                    accf[i][j][r] = __builtin_fmaf((float)(acc[i][j][r] >> 4), wsv[j], accf[i][j][r]);
                acc[i][j] = i32x16{};
            }
    };

    gload(0);
    sstore(0);
    if (nsteps > 1) gload(1);
    lds_barrier();
    for (int s = 0; s < nsteps; s++) {
        compute(s & 1);
        if ((s + 1) % SPG == 0) fold(s / SPG);
        if (s + 1 < nsteps) {
            sstore((s + 1) & 1);  // that stage was read by step s - 1, before the last barrier
            if (s + 2 < nsteps) gload(s + 2);
        }
        lds_barrier();
    }

    // lane l, register r of block (i, j): row 8*(r/4) + 4*(l/32) + r%4, column l%32
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int r = 0; r < 16; r++) {
            const int mr = m0 + wm * WTM + i * 32 + 8 * (r >> 2) + 4 * (lane >> 5) + (r & 3);
            if (mr >= M) continue;
            const float asc = xs[mr];
#pragma unroll
            for (int j = 0; j < FN; j++) {
                const int n = n0 + wn * WTN + j * 32 + (lane & 31);
                if (n >= N) continue;
                float v = accf[i][j][r] * asc;
                if (bias) v = v + fni8::h2f(bias[n]);
                y[(int64_t)mr * ldy + n] = fni8::f2h(v);
            }
        }
}

int launch_error(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fni8h::set_error_detail("%s launch: %s", what, hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

constexpr size_t kLdsBytes = 160 * 1024;
constexpr int64_t kSliceMaxM = 16;  // rows up to which the sliced GEMV beats the tile grid
constexpr int64_t kMfmaMinM = 1;    // above this many rows the MFMA decode kernel runs first

// Static LDS of w4a8_gemv_kernel<MT, CPG>: the per-wave group sums.
template <int MT, int CPG>
constexpr size_t kGemvStatic = (size_t)(kGemvThreads / 64) * kRows * MT * (64 / CPG) * 4;

template <int MT, int CPG>
int gemv_launch(const int8_t* xq, int64_t ldq, const float* xs, int64_t K, const uint8_t* w,
                const float* ws, int64_t N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                hipStream_t st) {
    const size_t lds = (size_t)MT * K;  // bytes: even + odd dwords of every 8-code block
    if (lds > 64 * 1024 - kGemvStatic<MT, CPG>) {
        static const bool ok =
            hipFuncSetAttribute(reinterpret_cast<const void*>(&w4a8_gemv_kernel<MT, CPG>),
                                hipFuncAttributeMaxDynamicSharedMemorySize,
                                (int)(kLdsBytes - kGemvStatic<MT, CPG>)) == hipSuccess;
        if (!ok) {
            fni8h::set_error_detail("w4a8 gemv: cannot raise the LDS limit to %zu bytes", lds);
            return FNI8_ERR_LAUNCH;
        }
    }
    const int rows_per_wg = (kGemvThreads / 64) * kRows;
    const dim3 grid((unsigned)((N + rows_per_wg - 1) / rows_per_wg));
    hipLaunchKernelGGL((w4a8_gemv_kernel<MT, CPG>), grid, dim3(kGemvThreads), lds, st, xq, ldq,
                       xs, (int)K, w, ws, (int)N, bias, y, ldy);
    return launch_error("w4a8 gemv");
}

template <int MT>
int gemv_by_group(int64_t G, const int8_t* xq, int64_t ldq, const float* xs, int64_t K,
                  const uint8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                  int64_t ldy, hipStream_t st) {
    switch (G) {
        case 32: return gemv_launch<MT, 1>(xq, ldq, xs, K, w, ws, N, bias, y, ldy, st);
        case 64: return gemv_launch<MT, 2>(xq, ldq, xs, K, w, ws, N, bias, y, ldy, st);
        case 128: return gemv_launch<MT, 4>(xq, ldq, xs, K, w, ws, N, bias, y, ldy, st);
        default: return gemv_launch<MT, 8>(xq, ldq, xs, K, w, ws, N, bias, y, ldy, st);
    }
}

template <int G>
int tile_launch(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                const uint8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                int64_t ldy, hipStream_t st) {
    constexpr int BM = 128, BN = 128;
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    hipLaunchKernelGGL((w4a8_tile_kernel<BM, BN, G>), grid, dim3(256), 0, st, xq, ldq, xs, nullptr,
                       (int)M, (int)K, w, ws, (int)N, 0, nullptr, bias, y, ldy);
    return launch_error("w4a8 tile");
}

// Grouped form: activation rows of stride K, y of stride N; the grid's x
// dimension bounds the segment tiles (sum over experts of ceil(len / 128) <=
// R_max / 128 + E), its y dimension the column tiles.
template <int G>
int tile_grouped_launch(const int8_t* aq, const float* as, const int32_t* rmap, int64_t R_max,
                        int64_t K, const uint8_t* w, const float* ws, int64_t E, int64_t N,
                        const int32_t* seg_off, const uint16_t* bias, uint16_t* y,
                        hipStream_t st) {
    constexpr int BM = 128, BN = 128;
    const dim3 grid((unsigned)((R_max + BM - 1) / BM + E), (unsigned)((N + BN - 1) / BN));
    hipLaunchKernelGGL((w4a8_tile_kernel<BM, BN, G, true>), grid, dim3(256), 0, st, aq, K, as,
                       rmap, (int)R_max, (int)K, w, ws, (int)N, (int)E, seg_off, bias, y, N);
    return launch_error("w4a8 grouped tile");
}

template <int G>
int tile8_launch(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                 const uint8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                 int64_t ldy, hipStream_t st) {
    constexpr int BM = 128, BN = 256, KS = G < 128 ? G : 128;
    constexpr size_t lds = (size_t)2 * (BM + BN) * (KS + 16);
    auto kern = &w4a8_tile8_kernel<BM, BN, G>;
    static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                               hipFuncAttributeMaxDynamicSharedMemorySize,
                                               (int)lds) == hipSuccess;
    if (!ok) {
        fni8h::set_error_detail("w4a8 tile: cannot raise the LDS limit to %zu bytes", lds);
        return FNI8_ERR_LAUNCH;
    }
    const dim3 grid((unsigned)((N + BN - 1) / BN), (unsigned)((M + BM - 1) / BM));
    hipLaunchKernelGGL(kern, grid, dim3(512), lds, st, xq, ldq, xs, (int)M, (int)K, w, ws, (int)N,
                       bias, y, ldy);
    return launch_error("w4a8 tile");
}

// LDS bytes of w4a8_stream_kernel: activations, group sums, scales.
size_t stream_lds(int MM, int RH, int WAVES, int64_t K, int CPG) {
    const int64_t ng = K / (32 * CPG);
    return (size_t)MM * K + (size_t)RH * 8 * MM * ng * 4 + MM * 4 + WAVES * MM * 4;
}

// The early second batch (EB) measured even or faster on every Qwen3-8B shape at
// one token (gate_up 11.54 -> 11.23 us), so every launch takes it.
template <int MM, int RH, int WAVES, int SB, int KCH, int CPG, bool FUSED, bool EB = true>
int stream_launch(const void* x, int64_t ldx, const float* xs_in, int64_t M, int64_t K,
                  const uint8_t* w, const float* ws, int64_t N, const uint16_t* bias,
                  uint16_t* y, int64_t ldy, int8_t* xq_out, float* xs_out, hipStream_t st) {
    auto kern = &w4a8_stream_kernel<MM, RH, WAVES, SB, KCH, CPG, FUSED, EB>;
    const size_t lds = stream_lds(MM, RH, WAVES, K, CPG);
    if (lds > 64 * 1024) {
        static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)kLdsBytes) == hipSuccess;
        if (!ok) {
            fni8h::set_error_detail("w4a8 stream: cannot raise the LDS limit to %zu bytes", lds);
            return FNI8_ERR_LAUNCH;
        }
    }
    const dim3 grid((unsigned)((N + RH * 8 - 1) / (RH * 8)));
    hipLaunchKernelGGL(kern, grid, dim3(WAVES * 64), lds, st, x, ldx, xs_in, (int)M, (int)K, w,
                       ws, (int)N, bias, y, ldy, xq_out, xs_out);
    return launch_error("w4a8 stream");
}

// LDS bytes of w4a8_mfma_kernel: the wave tiles, then the two group-sum areas.
template <int MT, int NB, int WAVES, int SB, int G>
constexpr size_t kMfmaLds = (size_t)WAVES * SB * (16 * NB + 32 * MT) * 128 +
                            (size_t)2 * WAVES * SB * (256 / G) * MT * NB * 256 * 4;

template <int MT, int NB, int WAVES, int SB, int G>
int mfma_launch(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                const uint8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                int64_t ldy, hipStream_t st) {
    constexpr size_t lds = kMfmaLds<MT, NB, WAVES, SB, G>;
    if constexpr (lds > kLdsBytes) return 1;
    if ((K >> 8) % (WAVES * SB) != 0) return 1;
    auto kern = &w4a8_mfma_kernel<MT, NB, WAVES, SB, G>;
    if constexpr (lds > 64 * 1024) {
        static const bool ok = hipFuncSetAttribute(reinterpret_cast<const void*>(kern),
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)lds) == hipSuccess;
        if (!ok) {
            fni8h::set_error_detail("w4a8 mfma: cannot raise the LDS limit to %zu bytes", lds);
            return FNI8_ERR_LAUNCH;
        }
    }
    const dim3 grid((unsigned)((N + 16 * NB - 1) / (16 * NB)));
    hipLaunchKernelGGL(kern, grid, dim3(WAVES * 64), lds, st, xq, ldq, xs, (int)M, (int)K, w, ws,
                       (int)N, bias, y, ldy);
    return launch_error("w4a8 mfma");
}

// Launch shape by token tiles and weight shape, measured on MI355X over the
// Qwen3-8B linears at G = 128 (24 distinct weight copies per shape, weights
// from HBM); other shapes take the first entry whose round divides K's slabs.
template <int MT, int G>
int mfma_table(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
               const uint8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
               int64_t ldy, hipStream_t st) {
#define FNI8_W4M(NB, WV, SB)                                                                 \
    do {                                                                                     \
        const int rc = mfma_launch<MT, NB, WV, SB, G>(xq, ldq, xs, M, K, w, ws, N, bias, y,  \
                                                      ldy, st);                              \
        if (rc != 1) return rc;                                                              \
    } while (0)
    const bool wide = N >= 16384, narrow = N <= 4096;
    if constexpr (MT == 1) {
        if (wide) FNI8_W4M(1, 2, 1);
        FNI8_W4M(1, 4, 2);
    } else if constexpr (MT == 2) {
        if (narrow) FNI8_W4M(1, 4, 2);
    } else {
        if (!narrow) FNI8_W4M(1, 2, 1);
    }
    FNI8_W4M(1, 4, 1);
    FNI8_W4M(1, 2, 1);
    FNI8_W4M(1, 1, 1);
#undef FNI8_W4M
    return 1;
}

// 1 when the shape is not taken: group size 64..256, K a multiple of 256, at
// most 64 tokens, 16-byte aligned activation rows.
int mfma_dispatch(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                  const uint8_t* w, const float* ws, int64_t N, int64_t G, const uint16_t* bias,
                  uint16_t* y, int64_t ldy, hipStream_t st) {
    if (M < 1 || M > 64 || G < 64 || K % 256 != 0 || K > 65536) return 1;
    if (ldq % 16 != 0 || ((uintptr_t)xq % 16) != 0 || ((uintptr_t)w % 16) != 0) return 1;
    const int mt = (int)((M + 15) / 16);
#define FNI8_W4M_G(MTV)                                                                         \
    switch (G) {                                                                                \
        case 64: return mfma_table<MTV, 64>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st);     \
        case 128: return mfma_table<MTV, 128>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st);   \
        default: return mfma_table<MTV, 256>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st);    \
    }
    switch (mt) {
        case 1: FNI8_W4M_G(1)
        case 2: FNI8_W4M_G(2)
        case 3: FNI8_W4M_G(3)
        default: FNI8_W4M_G(4)
    }
#undef FNI8_W4M_G
}

// 1 when the shape is not taken: K a multiple of 1024 (four waves of whole
// 256-code slabs), at most 4 tokens, LDS within the limit.
// One stream launch shape for MM token rows, or 1 when the shape does not fit
// it (slab split, activation chunks per thread, LDS).
template <int MM, int RH, int WAVES, int SB, bool FUSED>
int stream_try(const void* x, int64_t ldx, const float* xs_in, int64_t M, int64_t K,
               const uint8_t* w, const float* ws, int64_t N, int64_t G, const uint16_t* bias,
               uint16_t* y, int64_t ldy, int8_t* xq_out, float* xs_out, hipStream_t st) {
    if ((K / 256) % (WAVES * SB) != 0 || stream_lds(MM, RH, WAVES, K, (int)(G / 32)) > kLdsBytes)
        return 1;
    const int64_t kch = (K / 8 + WAVES * 64 - 1) / (WAVES * 64);
    if (kch > 8) return 1;
#define FNI8_W4T(KCHV, CPGV)                                                               \
    return stream_launch<MM, RH, WAVES, SB, KCHV, CPGV, FUSED>(x, ldx, xs_in, M, K, w, ws, N, \
                                                               bias, y, ldy, xq_out, xs_out, st)
#define FNI8_W4T_CPG(KCHV)                  \
    switch (G) {                            \
        case 32: FNI8_W4T(KCHV, 1);         \
        case 64: FNI8_W4T(KCHV, 2);         \
        case 128: FNI8_W4T(KCHV, 4);        \
        default: FNI8_W4T(KCHV, 8);         \
    }
    if (kch <= 2) { FNI8_W4T_CPG(2) }
    else if (kch <= 4) { FNI8_W4T_CPG(4) }
    else { FNI8_W4T_CPG(8) }
#undef FNI8_W4T_CPG
#undef FNI8_W4T
}

template <bool FUSED>
int stream_dispatch(const void* x, int64_t ldx, const float* xs_in, int64_t M, int64_t K,
                    const uint8_t* w, const float* ws, int64_t N, int64_t G,
                    const uint16_t* bias, uint16_t* y, int64_t ldy, int8_t* xq_out,
                    float* xs_out, hipStream_t st) {
    constexpr int WAVES = 4, RH = 2;
    if (M > 4 || K % (256 * WAVES) != 0 || K > 32768) return 1;
    if (M == 1) {
        // One token: launch shapes from a sweep over the Qwen3-8B linears at G = 128
        // (36 weight copies, bit-exact against the generic shape), confirmed in an
        // in-process A/B: QKV 5.88 -> 5.27 us, O 4.72 -> 4.51, down 9.43 -> 8.77.
        // gate_up (N >= 16384) keeps the generic shape (even or slower otherwise).
#define FNI8_W4ONE(RHV, WV, SBV)                                                             \
        do {                                                                                 \
            const int rc = stream_try<1, RHV, WV, SBV, FUSED>(x, ldx, xs_in, M, K, w, ws, N, \
                                                              G, bias, y, ldy, xq_out,       \
                                                              xs_out, st);                   \
            if (rc != 1) return rc;                                                          \
        } while (0)
        if (K <= 4096) {
            if (N <= 4096) FNI8_W4ONE(2, 8, 1);
            else if (N < 16384) FNI8_W4ONE(1, 8, 1);
        } else {
            FNI8_W4ONE(1, 4, 3);
        }
#undef FNI8_W4ONE
    }
    const int per = (int)(K / 256 / WAVES);
    const int CPG = (int)(G / 32);
    const int MM = M == 1 ? 1 : (M == 2 ? 2 : 4);
    if (stream_lds(MM, RH, WAVES, K, CPG) > kLdsBytes) return 1;
    if (FUSED && (ldx % 8 != 0 || ((uintptr_t)x % 16) != 0)) return 1;
    if (!FUSED && (ldx % 8 != 0 || ((uintptr_t)x % 8) != 0)) return 1;
    const int kch = (int)((K / 8 + WAVES * 64 - 1) / (WAVES * 64));
#define FNI8_W4S(MMV, SBV, KCHV, CPGV) \
    return stream_launch<MMV, RH, WAVES, SBV, KCHV, CPGV, FUSED>(x, ldx, xs_in, M, K, w, ws, N, \
                                                                 bias, y, ldy, xq_out, xs_out, st)
#define FNI8_W4S_CPG(MMV, SBV, KCHV)                       \
    switch (CPG) {                                         \
        case 1: FNI8_W4S(MMV, SBV, KCHV, 1);               \
        case 2: FNI8_W4S(MMV, SBV, KCHV, 2);               \
        case 4: FNI8_W4S(MMV, SBV, KCHV, 4);               \
        default: FNI8_W4S(MMV, SBV, KCHV, 8);              \
    }
#define FNI8_W4S_KCH(MMV, SBV)                                                       \
    if (kch <= 2) { FNI8_W4S_CPG(MMV, SBV, 2) }                                      \
    else if (kch <= 4) { FNI8_W4S_CPG(MMV, SBV, 4) }                                 \
    else if (kch <= 8) { FNI8_W4S_CPG(MMV, SBV, 8) }                                 \
    else { FNI8_W4S_CPG(MMV, SBV, 16) }
#define FNI8_W4S_SB(MMV)                                          \
    if (per % 4 == 0) { FNI8_W4S_KCH(MMV, 4) }                     \
    else if (per % 3 == 0) { FNI8_W4S_KCH(MMV, 3) }                \
    else if (per % 2 == 0) { FNI8_W4S_KCH(MMV, 2) }                \
    else { FNI8_W4S_KCH(MMV, 1) }
    if (MM == 1) { FNI8_W4S_SB(1) }
    else if (MM == 2) { FNI8_W4S_SB(2) }
    else { FNI8_W4S_SB(4) }
#undef FNI8_W4S_SB
#undef FNI8_W4S_KCH
#undef FNI8_W4S_CPG
#undef FNI8_W4S
}

}  // namespace

namespace fni8h {

int launch_gemm_w4a8(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                     const uint8_t* w, const float* ws, int64_t N, int64_t G,
                     const uint16_t* bias, uint16_t* y, int64_t ldy, hipStream_t st) {
    if (M == 0) return FNI8_OK;
    if (M > 8) {  // wide N: the row-block kernel (w4a8_rowblock.hip)
        const int rc = launch_w4a8_rowblock(xq, ldq, xs, M, K, w, ws, N, G, bias, y, ldy, st);
        if (rc != 1) return rc;
    }
    if (M > kMfmaMinM) {
        const int rc = mfma_dispatch(xq, ldq, xs, M, K, w, ws, N, G, bias, y, ldy, st);
        if (rc != 1) return rc;
    }
    // Up to kSliceMaxM rows: the streaming GEMV on slices of at most 4 rows (each
    // slice streams the weights again, still cheaper at these sizes than a tile
    // grid of N / 128 workgroups, too few to fill the chip).  The full-line
    // kernel takes K a multiple of 1024; the smaller GEMV covers the rest.
    if (M <= kSliceMaxM && ldq % 8 == 0 && ((uintptr_t)xq % 8) == 0) {
        for (int64_t m0 = 0; m0 < M; m0 += 4) {
            const int64_t mt = M - m0 < 4 ? M - m0 : 4;
            const int8_t* xq0 = xq + m0 * ldq;
            const float* xs0 = xs + m0;
            uint16_t* y0 = y + m0 * ldy;
            int rc = stream_dispatch<false>(xq0, ldq, xs0, mt, K, w, ws, N, G, bias, y0, ldy,
                                            nullptr, nullptr, st);
            if (rc == 1 && (size_t)4 * K <= kLdsBytes - 32 * 1024) {
                switch (mt) {
                    case 1: rc = gemv_by_group<1>(G, xq0, ldq, xs0, K, w, ws, N, bias, y0, ldy, st); break;
                    case 2: rc = gemv_by_group<2>(G, xq0, ldq, xs0, K, w, ws, N, bias, y0, ldy, st); break;
                    case 3: rc = gemv_by_group<3>(G, xq0, ldq, xs0, K, w, ws, N, bias, y0, ldy, st); break;
                    default: rc = gemv_by_group<4>(G, xq0, ldq, xs0, K, w, ws, N, bias, y0, ldy, st);
                }
            }
            if (rc == 1) break;  // neither GEMV takes the shape: the tile kernel does
            if (rc) return rc;
            if (m0 + 4 >= M) return FNI8_OK;
        }
    }
    switch (G) {
        case 32: return tile_launch<32>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st);
        case 64: return tile_launch<64>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st);
        case 128: return tile_launch<128>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st);
        // G = 256 folds every other step: the 8-wave two-stage kernel is 6-35%
        // faster there (Qwen3-8B shapes at 2048 tokens).  At G <= 128 it folds
        // every step with all eight waves in lockstep, one workgroup per CU, and
        // is 30-45% slower than the 4-wave kernel, which fits two workgroups.
        default: return tile8_launch<256>(xq, ldq, xs, M, K, w, ws, N, bias, y, ldy, st);
    }
}

int launch_w4a8_tile_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                             int64_t R_max, int64_t K, const uint8_t* w, const float* ws,
                             int64_t E, int64_t N, int64_t G, const int32_t* seg_off,
                             const uint16_t* bias, uint16_t* y, hipStream_t st) {
    switch (G) {
        case 64: return tile_grouped_launch<64>(aq, as, row_index, R_max, K, w, ws, E, N, seg_off, bias, y, st);
        case 128: return tile_grouped_launch<128>(aq, as, row_index, R_max, K, w, ws, E, N, seg_off, bias, y, st);
        default: return tile_grouped_launch<256>(aq, as, row_index, R_max, K, w, ws, E, N, seg_off, bias, y, st);
    }
}

int launch_linear_w4a8_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                             const uint8_t* w, const float* ws, int64_t N, int64_t G,
                             const uint16_t* bias, uint16_t* y, int64_t ldy, int8_t* xq_out,
                             float* xs_out, hipStream_t st) {
    if (M == 0) return FNI8_OK;
    // One token: the streaming kernel with the quantization fused.  From two
    // tokens on, the MFMA decode kernel beats the VALU-bound stream kernel
    // (Qwen3-8B shapes at 4 tokens, with a quantize launch in front: 9.7 / 8.0
    // / 17.7 / 16.0 us against 12.0 / 9.2 / 26.9 / 20.9 us); up to 4 tokens it
    // runs with the quantization fused (w4a8_fused.hip), else after a quantize
    // launch (the caller's, on a 1).
    if (M > 1 && G >= 64 && K % 256 == 0)
        return M <= 4 ? launch_linear_w4a8_mfma_fused(x, ldx, M, K, w, ws, N, G, bias, y, ldy,
                                                      xq_out, xs_out, st)
                      : 1;
    return stream_dispatch<true>(x, ldx, nullptr, M, K, w, ws, N, G, bias, y, ldy, xq_out,
                                 xs_out, st);
}

}  // namespace fni8h
