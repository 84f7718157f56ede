// Decode W8A8 linear for M <= 4 tokens (gfx950): one launch per linear, with
// the per-token quantization fused into the GEMV.
//
//   y[m, n] = fp16(((float)sum_k q[m, k] * w[n, k]) * s[m] * ws[n] (+ bias[n]))
//   s[m]    = max(amax_k |x[m, k]|, eps) / 127,  q = clamp(rint(x / s), -127, 127)
//
// The weight stream is the whole cost (HBM-bound: N*K bytes against 2MK + 2MN
// of activations and outputs), so the kernel is laid out around it:
//   * A workgroup owns 8*RH weight rows; its WAVES waves split K into equal
//     shares of 128-byte slabs.  Every wave load instruction covers 8 rows x
//     128 contiguous bytes (lane l: row l/8, bytes 16*(l%8)..+16 of a slab), so
//     each row contributes a full 128-byte line per instruction.  Loads are
//     non-temporal (each weight byte is read once) and register double-buffered:
//     the next SB slabs are in flight while the current ones are consumed.
//   * The int8 dot products run on v_dot4_i32_i8: lane l accumulates its
//     16-byte column slice of every slab in private int32 sums (one per row and
//     token), so the only cross-lane work is one 8-lane DPP reduction and one
//     cross-wave LDS reduction at the end.
//   * Quantization (FUSED): the workgroup issues the loads of the M fp16 rows
//     of x and then its first weight batch, reduces each row's max magnitude
//     (DPP + LDS) while the weights are in flight, and quantizes the rows into
//     LDS as int8.  Every workgroup does this for itself -- M*K elements, small
//     next to the 8*RH*K weight bytes it streams -- so no workgroup waits for
//     another.  Workgroup 0 also writes xq/xs for the caller.
//
// Exact quantization without a division per element: with y = fl(1/s)
// (correctly rounded, once per row), t = fl(x*y) and r = fma(-t, s, x) (exact),
// fl(x/s) == fma(r, y, t) for every non-zero fp16 x with |x| <= amax (Markstein's
// correction theorem; also checked exhaustively over all fp16 (x, amax) pairs by
// the CPU test suite).  For x = 0 the two differ at most in the sign of zero,
// which rint maps to the same integer 0.
#include "common.h"

namespace {

// Barrier that waits for LDS traffic only (the compiler's __syncthreads also
// drains the weight loads in flight).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

__device__ __forceinline__ i32x4 ld16_nt(const int8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
}

// MM: token rows handled (M <= MM); RH: 8-row groups per workgroup; WAVES: K
// split; SB: 128-byte slabs per load batch (must divide each wave's share);
// KCH: 16-byte chunks of each activation row per thread (K <= 16 * KCH * 64 *
// WAVES / (FUSED ? 2 : 1)); FUSED: x is fp16 (quantized here), else x is int8
// with scales xs_in.
// EB: the prologue's barriers wait for LDS traffic only, and the second weight
// batch is issued before the quantization (its latency then overlaps the
// quantization's VALU work).
template <int MM, int RH, int WAVES, int SB, int KCH, bool FUSED, bool EB = false>
__global__ __launch_bounds__(WAVES * 64) void decode_gemv_kernel(
    const void* __restrict__ xin, int64_t ldx, const float* __restrict__ xs_in, int M, int K,
    const int8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int8_t* __restrict__ xq_out, float* __restrict__ xs_out, int32_t* __restrict__ acc_out) {
    constexpr int NT = WAVES * 64;
    constexpr int ROWS = RH * 8;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    int8_t* xq_l = smem;                                               // [MM][K] int8
    int32_t* red = reinterpret_cast<int32_t*>(smem + (size_t)MM * K);  // [WAVES][MM][ROWS]
    float* scl = reinterpret_cast<float*>(red + WAVES * MM * ROWS);    // [MM] row scales
    uint32_t* amx = reinterpret_cast<uint32_t*>(scl + MM);             // [WAVES][MM]

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int n0 = blockIdx.x * ROWS;
    const int rq = lane >> 3, c = lane & 7;

    // weight sources: rows n0 + h*8 + rq (clamped), column slice c of each slab
    const int per = (K >> 7) / WAVES;  // slabs per wave (the launcher makes it exact)
    const int s0 = wave * per;
    const int nb = per / SB;           // load batches per wave
    const int8_t* wsrc[RH];
#pragma unroll
    for (int h = 0; h < RH; h++) {
        int n = n0 + h * 8 + rq;
        n = n < N ? n : N - 1;
        wsrc[h] = w + (int64_t)n * K + (int64_t)s0 * 128 + c * 16;
    }
    i32x4 wa[SB][RH], wb[SB][RH];
    auto load = [&](i32x4 (&dst)[SB][RH], int b) {
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < RH; h++)
                dst[j][h] = ld16_nt(wsrc[h] + (int64_t)(b * SB + j) * 128);
    };

    // epilogue thread: output row j of the tile, token m; its weight scale early
    const int ej = tid % ROWS, em = tid / ROWS;
    const bool eact = tid < ROWS * M && n0 + ej < N;
    const float wscale = eact ? ws[n0 + ej] : 0.f;

    // ---- activations into LDS as int8 --------------------------------------
    // The activation loads are issued first and the first weight batch right
    // after them, so the weights stay in flight while the rows are reduced and
    // quantized (loads complete in issue order).
    if constexpr (FUSED) {
        const uint16_t* x = reinterpret_cast<const uint16_t*>(xin);
        const int chunks = K >> 3;  // 16-byte chunks (8 fp16) per row
        uint4 xr[MM][KCH];
#pragma unroll
        for (int m = 0; m < MM; m++)
#pragma unroll
            for (int i = 0; i < KCH; i++) {
                const int ch = tid + i * NT;
                const int mr = m < M ? m : 0, cc = ch < chunks ? ch : chunks - 1;
                const uint4 v = *reinterpret_cast<const uint4*>(x + (int64_t)mr * ldx + cc * 8);
                const bool ok = m < M && ch < chunks;
                xr[m][i] = ok ? v : make_uint4(0, 0, 0, 0);
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
            const float s = fni8::row_scale_from_bits(a);
            const bool live = m < M && __builtin_isfinite(s);  // rows past M quantize to 0
            const float yr = 1.0f / s;  // correctly rounded (build flag)
            if (tid == 0) {
                scl[m] = s;
                if (xs_out != nullptr && blockIdx.x == 0 && m < M) xs_out[m] = s;
            }
#pragma unroll
            for (int i = 0; i < KCH; i++) {
                const int ch = tid + i * NT;
                if (ch < chunks) {
                    const uint2 q = fni8::quant_chunk(xr[m][i], s, yr, live);
                    *reinterpret_cast<uint2*>(xq_l + (size_t)m * K + ch * 8) = q;
                    if (xq_out != nullptr && blockIdx.x == 0 && m < M)
                        *reinterpret_cast<uint2*>(xq_out + (int64_t)m * K + ch * 8) = q;
                }
            }
        }
    } else {
        const int8_t* xq = reinterpret_cast<const int8_t*>(xin);
        const int chunks = K >> 4;  // 16 int8 per chunk
        i32x4 xr[MM][KCH];
#pragma unroll
        for (int m = 0; m < MM; m++)
#pragma unroll
            for (int i = 0; i < KCH; i++) {
                const int ch = tid + i * NT;
                const int mr = m < M ? m : 0, cc = ch < chunks ? ch : chunks - 1;
                const i32x4 v = *reinterpret_cast<const i32x4*>(xq + (int64_t)mr * ldx + cc * 16);
                xr[m][i] = (m < M && ch < chunks) ? v : i32x4{0, 0, 0, 0};
            }
        load(wa, 0);
#pragma unroll
        for (int m = 0; m < MM; m++) {
#pragma unroll
            for (int i = 0; i < KCH; i++) {
                const int ch = tid + i * NT;
                if (ch < chunks) *reinterpret_cast<i32x4*>(xq_l + (size_t)m * K + ch * 16) = xr[m][i];
            }
            if (tid == 0) scl[m] = m < M ? xs_in[m] : 0.f;
        }
        if (EB && nb > 1) load(wb, 1);
    }
    if constexpr (EB)
        lds_barrier();
    else
        __syncthreads();

    // ---- weight stream ------------------------------------------------------
    int32_t acc[RH][MM];
#pragma unroll
    for (int h = 0; h < RH; h++)
#pragma unroll
        for (int m = 0; m < MM; m++) acc[h][m] = 0;

    const int8_t* xl = xq_l + (size_t)s0 * 128 + c * 16;
    auto compute = [&](const i32x4 (&wv)[SB][RH], int b) {
        i32x4 xv[SB][MM];
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int m = 0; m < MM; m++)
                xv[j][m] = *reinterpret_cast<const i32x4*>(xl + (size_t)m * K + (b * SB + j) * 128);
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int m = 0; m < MM; m++)
#pragma unroll
                for (int h = 0; h < RH; h++) {
                    int a = acc[h][m];
                    a = __builtin_amdgcn_sdot4(wv[j][h][0], xv[j][m][0], a, false);
                    a = __builtin_amdgcn_sdot4(wv[j][h][1], xv[j][m][1], a, false);
                    a = __builtin_amdgcn_sdot4(wv[j][h][2], xv[j][m][2], a, false);
                    a = __builtin_amdgcn_sdot4(wv[j][h][3], xv[j][m][3], a, false);
                    acc[h][m] = a;
                }
    };
    // steady state: prefetch batch b+1, consume batch b; the last batch is peeled
    for (int b = 0; b < nb - 1; b++) {
        if (!EB || b > 0) load(wb, b + 1);  // with EB, batch 1 went out in the prologue
        compute(wa, b);
#pragma unroll
        for (int j = 0; j < SB; j++)
#pragma unroll
            for (int h = 0; h < RH; h++) wa[j][h] = wb[j][h];
    }
    compute(wa, nb - 1);

    // ---- reductions: 8 lanes of a row (DPP), then the waves (LDS) -----------
#pragma unroll
    for (int h = 0; h < RH; h++)
#pragma unroll
        for (int m = 0; m < MM; m++) {
            const int a = fni8::sum8(acc[h][m]);
            if (c == 0) red[(wave * MM + m) * ROWS + h * 8 + rq] = a;
        }
    __syncthreads();
    if (eact) {
        int32_t sum = 0;
#pragma unroll
        for (int wv = 0; wv < WAVES; wv++) sum += red[(wv * MM + em) * ROWS + ej];
        const int n = n0 + ej;
        y[(int64_t)em * ldy + n] = fni8::dequant_one(sum, scl[em], wscale, bias, n);
        if (acc_out != nullptr) acc_out[(int64_t)em * N + n] = sum;
    }
}

template <int MM, int RH, int WAVES, int SB, int KCH, bool FUSED, bool EB = false>
int launch_gemv(const void* x, int64_t ldx, const float* xs_in, int M, int K, const int8_t* w,
                const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                int8_t* xq_out, float* xs_out, int32_t* acc_out, hipStream_t st) {
    constexpr int ROWS = RH * 8;
    const int slabs = K >> 7;
    if (K % 128 != 0 || slabs % WAVES != 0 || (slabs / WAVES) % SB != 0) return 1;
    const int64_t per_thread = FUSED ? (int64_t)8 * KCH * 64 * WAVES : (int64_t)16 * KCH * 64 * WAVES;
    if ((int64_t)K > per_thread) return 1;
    const size_t lds = (size_t)MM * K + (size_t)WAVES * MM * ROWS * 4 + MM * 4 + WAVES * MM * 4;
    if (lds > 160 * 1024) return 1;
    auto kern = decode_gemv_kernel<MM, RH, WAVES, SB, KCH, FUSED, EB>;
    if (lds > 64 * 1024) {
        // The dynamic LDS limit is a per-function attribute; setting it again
        // with the same value is idempotent, so a race between threads is harmless.
        static bool attr_set = false;
        if (!attr_set) {
            hipError_t e = hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, 160 * 1024);
            if (e != hipSuccess) {
                fni8h::set_error_detail("LDS attribute: %s", hipGetErrorString(e));
                return FNI8_ERR_LAUNCH;
            }
            attr_set = true;
        }
    }
    const unsigned grid = (unsigned)((N + ROWS - 1) / ROWS);
    hipLaunchKernelGGL(kern, dim3(grid), dim3(WAVES * 64), lds, st, x, ldx, xs_in, M, K, w, ws,
                       N, bias, y, ldy, xq_out, xs_out, acc_out);
    return FNI8_OK;
}

// Launch shapes, measured on MI355X over the Qwen3-8B decode shapes (24-36
// distinct weight copies, so every byte streams from HBM; the one-token entries
// from a sweep of rows x waves x batch): the waves split K; 8-row workgroups
// take every shape but the narrow N = 4096, K = 4096 one (16-row).  Shapes the tuned
// entries do not divide take the first generic entry whose batch size divides
// the per-wave share of K.
template <bool FUSED>
int launch_decode_gemv(const void* x, int64_t ldx, const float* xs_in, int M, int K,
                       const int8_t* w, const float* ws, int N, const uint16_t* bias, uint16_t* y,
                       int64_t ldy, int8_t* xq_out, float* xs_out, int32_t* acc_out,
                       hipStream_t st) {
#define FNI8_GEMV_E(MM, RH, WV, SB, KCH, EB)                                                   \
    do {                                                                                       \
        const int rc = launch_gemv<MM, RH, WV, SB, KCH, FUSED, EB>(                            \
            x, ldx, xs_in, M, K, w, ws, N, bias, y, ldy, xq_out, xs_out, acc_out, st);         \
        if (rc != 1) return rc;                                                                \
    } while (0)
#define FNI8_GEMV(MM, RH, WV, SB, KCH) FNI8_GEMV_E(MM, RH, WV, SB, KCH, false)
#define FNI8_GEMV_GENERIC(MM)                \
    do {                                     \
        if (K <= 4096) {                     \
            FNI8_GEMV(MM, 2, 4, 4, 2);       \
            FNI8_GEMV(MM, 2, 4, 2, 2);       \
            FNI8_GEMV(MM, 2, 4, 1, 2);       \
        }                                    \
        if (K <= 12288) {                    \
            FNI8_GEMV(MM, 2, 8, 4, 3);       \
            FNI8_GEMV(MM, 2, 8, 2, 3);       \
            FNI8_GEMV(MM, 2, 8, 1, 3);       \
        }                                    \
        FNI8_GEMV(MM, 2, 8, 4, 6);           \
        FNI8_GEMV(MM, 2, 8, 2, 6);           \
        FNI8_GEMV(MM, 2, 8, 1, 6);           \
        return 1;                            \
    } while (0)
    if (M <= 1) {
        if (K <= 4096) {
            if (N <= 4096) FNI8_GEMV(1, 2, 4, 8, 2);
            else if (N <= 8192) FNI8_GEMV(1, 1, 4, 4, 2);
            else FNI8_GEMV(1, 1, 4, 2, 2);
        } else {
            FNI8_GEMV(1, 1, 8, 4, 3);
        }
        FNI8_GEMV_GENERIC(1);
    }
    if (M <= 2) {
        if (K <= 4096) {
            if (N <= 4096) FNI8_GEMV(2, 2, 4, 8, 2);
            else if (N <= 8192) FNI8_GEMV(2, 2, 4, 4, 2);
            else FNI8_GEMV(2, 4, 4, 4, 2);
        } else {
            // early second batch: down at 2 tokens 11.61 -> 10.73 us (QKV and
            // gate_up lose 3-6% with it; O has a single batch per wave)
            FNI8_GEMV_E(2, 2, 4, 4, 6, true);
        }
        FNI8_GEMV_GENERIC(2);
    }
    if (K <= 4096) {
        if (N <= 4096) FNI8_GEMV(4, 2, 4, 4, 2);
        else FNI8_GEMV(4, 4, 4, 4, 2);
    } else {
        FNI8_GEMV(4, 2, 8, 4, 3);
    }
    FNI8_GEMV_GENERIC(4);
#undef FNI8_GEMV_GENERIC
#undef FNI8_GEMV
#undef FNI8_GEMV_E
}

}  // namespace

namespace fni8h {

// Returns 1 when the shape is not taken (M > 4, K not a whole number of
// per-wave slab batches, K too long, misaligned rows), so the caller uses the
// two-launch path; otherwise an FNI8 code.
int launch_decode_fused(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                        const float* ws, int64_t N, const uint16_t* bias, uint16_t* y, int64_t ldy,
                        int8_t* xq_out, float* xs_out, int32_t* acc_out, hipStream_t st) {
    if (M < 1 || M > 4 || K % 128 != 0 || ldx % 8 != 0 || (uintptr_t)x % 16 != 0 ||
        (uintptr_t)w % 16 != 0 || (xq_out != nullptr && (uintptr_t)xq_out % 8 != 0))
        return 1;
    int rc = launch_decode_gemv<true>(x, ldx, nullptr, (int)M, (int)K, w, ws, (int)N, bias, y, ldy,
                                      xq_out, xs_out, acc_out, st);
    if (rc) return rc;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("decode launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

// Pre-quantized int8 activations (M <= 4): the same kernel without the
// quantize phase.  Returns 1 when the shape is not taken.
int launch_decode_q(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                    const int8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                    int64_t ldy, int32_t* acc_out, hipStream_t st) {
    if (M < 1 || M > 4 || K % 128 != 0 || ldq % 16 != 0 || (uintptr_t)xq % 16 != 0 ||
        (uintptr_t)w % 16 != 0)
        return 1;
    return launch_decode_gemv<false>(xq, ldq, xs, (int)M, (int)K, w, ws, (int)N, bias, y, ldy,
                                     nullptr, nullptr, acc_out, st);
}

}  // namespace fni8h
