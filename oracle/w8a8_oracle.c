/*
 * CPU oracle for the W8A8 linear path.  TEST INFRASTRUCTURE ONLY: it is the
 * checker the HIP kernels are compared against, never the thing that runs in
 * the product path.  Only tests, the smoke check and the CPU-baseline leg of
 * the benchmark load it.
 *
 * What it restates (reference = Josephur/fni8-serve):
 *   - per-token symmetric activation quantization, the step `fni8.linear`
 *     performs before its int8 GEMM (fni8serve/layers/linear.py:5-10, call at
 *     :69).  `fni8` is a closed wheel that is absent here, so the exact
 *     convention is the reference's own Python quant idiom, evaluated in fp32:
 *         s = amax(|row|).clamp_min(eps) / 127 ;  q = round(x / s).clamp(-127, 127)
 *     (tests/test_smoke.py:16-17, tests/test_layers.py:31-32,
 *      tests/test_linear_attn.py:169-170, tests/test_mla.py:60-62,
 *      tests/test_qwen3_5.py:458-459; eps = 1e-6 as in test_layers.py:31).
 *     torch.round is round-half-to-even; so is rintf here.
 *   - the int8 x int8 -> int32 GEMM `gemm_w8a8` (linear.py:9): y = xq . W^T with
 *     W int8 [N, K] row-major (the per_row_i8 QTensor layout,
 *     fni8serve/models/weights.py:18-25).  Exact integer dot products.
 *   - the dequant epilogue: y = fp16(((float)acc * a_s[m]) * w_s[n] (+ bias[n]))
 *     in fp32, one rounding per operation, no fused multiply-add.
 *   - the MoE expert loop (fni8serve/models/moe.py:97-105): rows routed to an
 *     expert are gathered in (token, slot) order, run through the expert, and
 *     combined with `index_add_` in ascending expert order in fp16.
 *
 * Non-finite inputs: amax is taken on the fp16 magnitude bits, so a NaN in a
 * row makes that row's scale NaN and an inf makes it inf; any x/s that is NaN
 * quantizes to 0.  Such rows dequantize to NaN.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

#define FNI8_QUANT_EPS 1e-6f
#define FNI8_QMAX 127.0f

/* ---- fp16 <-> fp32 (IEEE binary16, round to nearest even) ---------------- */

float oracle_f16_to_f32(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    uint32_t exp = (h >> 10) & 0x1fu;
    uint32_t mant = h & 0x3ffu;
    uint32_t bits;
    if (exp == 0) {
        if (mant == 0) {
            bits = sign;
        } else { /* subnormal: normalise */
            int e = -1;
            do { mant <<= 1; e++; } while ((mant & 0x400u) == 0);
            mant &= 0x3ffu;
            bits = sign | ((uint32_t)(127 - 15 - e) << 23) | (mant << 13);
        }
    } else if (exp == 31) {
        bits = sign | 0x7f800000u | (mant << 13);
    } else {
        bits = sign | ((exp + 127 - 15) << 23) | (mant << 13);
    }
    float f;
    memcpy(&f, &bits, 4);
    return f;
}

uint16_t oracle_f32_to_f16(float f) {
    uint32_t x;
    memcpy(&x, &f, 4);
    uint16_t sign = (uint16_t)((x >> 16) & 0x8000u);
    uint32_t ax = x & 0x7fffffffu;
    if (ax > 0x7f800000u) /* NaN -> quiet NaN */
        return (uint16_t)(sign | 0x7e00u | ((ax >> 13) & 0x3ffu));
    if (ax >= 0x477ff000u) /* >= 65520 rounds to inf */
        return (uint16_t)(sign | 0x7c00u);
    if (ax >= 0x38800000u) { /* normal binary16 range, >= 2^-14 */
        uint32_t mant = ax & 0x7fffffu;
        uint32_t exp = (ax >> 23) - 127 + 15;
        uint32_t h = (exp << 10) | (mant >> 13);
        uint32_t rem = mant & 0x1fffu;
        if (rem > 0x1000u || (rem == 0x1000u && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
    if (ax <= 0x33000000u) /* <= 2^-25 rounds (ties even) to zero */
        return sign;
    { /* subnormal binary16: count units of 2^-24 */
        uint32_t e = ax >> 23;
        uint32_t m = (ax & 0x7fffffu) | 0x800000u;
        uint32_t shift = 126 - e;
        uint32_t h = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t half = 1u << (shift - 1);
        if (rem > half || (rem == half && (h & 1u))) h++;
        return (uint16_t)(sign | h);
    }
}

void oracle_f16_to_f32_n(const uint16_t* h, float* f, int64_t n) {
    for (int64_t i = 0; i < n; i++) f[i] = oracle_f16_to_f32(h[i]);
}

void oracle_f32_to_f16_n(const float* f, uint16_t* h, int64_t n) {
    for (int64_t i = 0; i < n; i++) h[i] = oracle_f32_to_f16(f[i]);
}

/* ---- per-token activation quantization ----------------------------------- */

static float row_scale(uint16_t amax_bits) {
    float amax = oracle_f16_to_f32(amax_bits);
    if (amax != amax) return amax; /* NaN propagates, as torch.amax does */
    return (amax > FNI8_QUANT_EPS ? amax : FNI8_QUANT_EPS) / FNI8_QMAX;
}

static int8_t quant_one(float x, float s) {
    float v = x / s;
    if (v != v) return 0;
    v = rintf(v);
    if (v > FNI8_QMAX) v = FNI8_QMAX;
    if (v < -FNI8_QMAX) v = -FNI8_QMAX;
    return (int8_t)v;
}

/* x fp16 [M, K] with row stride ldx -> q int8 [M, K] (row stride ldq), s fp32 [M] */
void oracle_quant_rowwise_f16(const uint16_t* x, int64_t M, int64_t K, int64_t ldx,
                              int8_t* q, int64_t ldq, float* s) {
    for (int64_t m = 0; m < M; m++) {
        const uint16_t* xr = x + m * ldx;
        uint16_t amax_bits = 0;
        for (int64_t k = 0; k < K; k++) {
            uint16_t b = (uint16_t)(xr[k] & 0x7fffu);
            if (b > amax_bits) amax_bits = b;
        }
        float sc = row_scale(amax_bits);
        s[m] = sc;
        for (int64_t k = 0; k < K; k++) q[m * ldq + k] = quant_one(oracle_f16_to_f32(xr[k]), sc);
    }
}

/* ---- int8 GEMM: acc[m, n] = sum_k a[m, k] * w[n, k] (exact int32) ---------- */

void oracle_gemm_i8(const int8_t* a, int64_t lda, int64_t M, int64_t K,
                    const int8_t* w, int64_t ldw, int64_t N,
                    int32_t* acc, int64_t ldacc) {
#pragma omp parallel for schedule(static)
    for (int64_t n = 0; n < N; n++) {
        const int8_t* wr = w + n * ldw;
        for (int64_t m = 0; m < M; m++) {
            const int8_t* ar = a + m * lda;
            int32_t sum = 0;
            for (int64_t k = 0; k < K; k++) sum += (int32_t)ar[k] * (int32_t)wr[k];
            acc[m * ldacc + n] = sum;
        }
    }
}

/* ---- dequant epilogue ------------------------------------------------------ */

static uint16_t dequant_one(int32_t acc, float as, float ws, const uint16_t* bias, int64_t n) {
    float v = (float)acc;
    v = v * as;
    v = v * ws;
    if (bias) v = v + oracle_f16_to_f32(bias[n]);
    return oracle_f32_to_f16(v);
}

void oracle_dequant_f16(const int32_t* acc, int64_t ldacc, int64_t M, int64_t N,
                        const float* as, const float* ws, const uint16_t* bias,
                        uint16_t* y, int64_t ldy) {
    for (int64_t m = 0; m < M; m++)
        for (int64_t n = 0; n < N; n++)
            y[m * ldy + n] = dequant_one(acc[m * ldacc + n], as[m], ws[n], bias, n);
}

/* The whole W8A8 linear: quant -> GEMM -> epilogue.  xq/xs/acc receive the
 * intermediates (caller-owned, row strides K, K and N). */
void oracle_linear_w8a8_f16(const uint16_t* x, int64_t ldx, int64_t M, int64_t K,
                            const int8_t* w, const float* ws, int64_t N,
                            const uint16_t* bias, uint16_t* y, int64_t ldy,
                            int8_t* xq, float* xs, int32_t* acc) {
    oracle_quant_rowwise_f16(x, M, K, ldx, xq, K, xs);
    oracle_gemm_i8(xq, K, M, K, w, K, N, acc, N);
    oracle_dequant_f16(acc, N, M, N, xs, ws, bias, y, ldy);
}

/* ---- MoE: routing sort, grouped GEMM, combine ------------------------------ */

/* Stable counting sort of the T*k (token, slot) pairs by expert id.  The order
 * inside an expert's segment is ascending token then slot: the order
 * `(topi == e).nonzero()` yields at moe.py:100-103.
 * seg_off [E+1]; row_token/row_slot [T*k]; pos [T*k] maps (t, j) -> sorted row. */
int oracle_moe_sort(const int32_t* topi, int64_t T, int64_t k, int64_t E,
                    int32_t* seg_off, int32_t* row_token, int32_t* row_slot, int32_t* pos) {
    for (int64_t e = 0; e <= E; e++) seg_off[e] = 0;
    for (int64_t i = 0; i < T * k; i++) {
        int32_t e = topi[i];
        if (e < 0 || e >= E) return -1;
        seg_off[e + 1]++;
    }
    for (int64_t e = 0; e < E; e++) seg_off[e + 1] += seg_off[e];
    for (int64_t e = 0; e < E; e++) {
        int32_t cur = seg_off[e];
        for (int64_t i = 0; i < T * k; i++) {
            if (topi[i] != e) continue;
            row_token[cur] = (int32_t)(i / k);
            row_slot[cur] = (int32_t)(i % k);
            pos[i] = cur;
            cur++;
        }
    }
    return 0;
}

/* Grouped W8A8 GEMM over expert segments.  Sorted row r of expert e reads
 * activation row a_row = (row_index ? row_index[r] : r) of aq/as, and the
 * expert's weight w[e] int8 [N, K] with scales ws[e] fp32 [N].  This is the
 * per-expert loop of moe.py:99-104 with the per-token quantization hoisted
 * (quantization is row-local, so gathering before or after quantizing gives
 * identical int8 rows). */
void oracle_grouped_w8a8_f16(const int8_t* aq, const float* as, int64_t K,
                             const int32_t* row_index,
                             const int8_t* w, const float* ws, int64_t E, int64_t N,
                             const int32_t* seg_off, const uint16_t* bias /* [E, N] or NULL */,
                             uint16_t* y /* [R, N] */, int32_t* acc /* [R, N] or NULL */) {
    for (int64_t e = 0; e < E; e++) {
        const int8_t* we = w + e * N * K;
        const float* wse = ws + e * N;
        const uint16_t* be = bias ? bias + e * N : 0;
#pragma omp parallel for schedule(static)
        for (int64_t r = seg_off[e]; r < seg_off[e + 1]; r++) {
            int64_t ar = row_index ? row_index[r] : r;
            const int8_t* a = aq + ar * K;
            for (int64_t n = 0; n < N; n++) {
                const int8_t* wr = we + n * K;
                int32_t sum = 0;
                for (int64_t kk = 0; kk < K; kk++) sum += (int32_t)a[kk] * (int32_t)wr[kk];
                if (acc) acc[r * N + n] = sum;
                y[r * N + n] = dequant_one(sum, as[ar], wse[n], be, n);
            }
        }
    }
}

/* Weighted combine (moe.py:97-105): out[t] starts at +0 (zeros_like), then for
 * the token's experts in ascending expert id, out[t] += fp16(contrib * w) with
 * fp16 rounding after the product and after the add. */
void oracle_moe_combine_f16(const uint16_t* yr /* [R, H] sorted rows */, int64_t H,
                            const int32_t* topi, const uint16_t* topw, const int32_t* pos,
                            int64_t T, int64_t k, uint16_t* out /* [T, H] */) {
    for (int64_t t = 0; t < T; t++) {
        int32_t order[64];
        int64_t kk = k < 64 ? k : 64;
        for (int64_t j = 0; j < kk; j++) order[j] = (int32_t)j;
        for (int64_t a = 1; a < kk; a++) { /* insertion sort by expert id */
            int32_t v = order[a];
            int64_t b = a - 1;
            while (b >= 0 && topi[t * k + order[b]] > topi[t * k + v]) { order[b + 1] = order[b]; b--; }
            order[b + 1] = v;
        }
        for (int64_t h = 0; h < H; h++) {
            uint16_t o = 0;
            for (int64_t j = 0; j < kk; j++) {
                int64_t slot = order[j];
                float c = oracle_f16_to_f32(yr[(int64_t)pos[t * k + slot] * H + h]);
                float wgt = oracle_f16_to_f32(topw[t * k + slot]);
                uint16_t p = oracle_f32_to_f16(c * wgt);
                o = oracle_f32_to_f16(oracle_f16_to_f32(o) + oracle_f16_to_f32(p));
            }
            out[t * H + h] = o;
        }
    }
}
