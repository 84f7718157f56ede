/*
 * CPU oracle for the W4A8 linear (per_group_i4 int4 weights).  TEST
 * INFRASTRUCTURE ONLY: the CPU restatement the HIP kernels are compared against.
 *
 * What it restates (reference = Josephur/fni8-serve):
 *   - the weight format of per_group_i4 (fni8serve/convert.py:69-79, unpacked
 *     at fni8serve/layers/linear.py:32-45): packed uint8 [N, K/2], code k in
 *     byte k/2, low nibble for even k and high nibble for odd k, a nibble u
 *     meaning u - 16 when u >= 8; fp32 scale [N, K/G] per group of G codes;
 *   - `gemm_w4a8`, the int4 GEMM of `fni8.linear` (linear.py:9), whose closed
 *     arithmetic is replaced by this library's convention: per group the exact
 *     int32 sum acc_g = sum of xq[m, k] * code[n, k]; accf = fmaf(acc_g,
 *     ws[n, g], accf) over g = 0, 1, ... from +0; y = fp16(accf * xs[m]
 *     (+ bias[n])), one rounding per operation;
 *   - the activation quantization is the W8A8 one (oracle_quant_rowwise_f16).
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>

uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);
void oracle_quant_rowwise_f16(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                              int64_t ldq, float* s);

static int code_at(const uint8_t* row, int64_t k) {
    const uint8_t b = row[k / 2];
    const int u = (k & 1) ? (b >> 4) : (b & 0xf);
    return u >= 8 ? u - 16 : u;
}

/* gacc: [M, N, K/G] int32 group sums, or NULL. */
void oracle_gemm_w4a8(const int8_t* xq, const float* xs, int64_t M, int64_t K,
                      const uint8_t* w, const float* ws, int64_t N, int64_t G,
                      const uint16_t* bias, uint16_t* y, int32_t* gacc) {
    const int64_t ng = K / G;
    for (int64_t m = 0; m < M; m++) {
        const int8_t* xr = xq + m * K;
        for (int64_t n = 0; n < N; n++) {
            const uint8_t* wr = w + n * (K / 2);
            float accf = 0.0f;
            for (int64_t g = 0; g < ng; g++) {
                int32_t acc = 0;
                for (int64_t k = g * G; k < (g + 1) * G; k++) acc += (int32_t)xr[k] * code_at(wr, k);
                if (gacc) gacc[(m * N + n) * ng + g] = acc;
                accf = fmaf((float)acc, ws[n * ng + g], accf);
            }
            float v = accf * xs[m];
            if (bias) v = v + oracle_f16_to_f32(bias[n]);
            y[m * N + n] = oracle_f32_to_f16(v);
        }
    }
}

void oracle_linear_w4a8_f16(const uint16_t* x, int64_t M, int64_t K, const uint8_t* w,
                            const float* ws, int64_t N, int64_t G, const uint16_t* bias,
                            uint16_t* y, int8_t* xq, float* xs) {
    oracle_quant_rowwise_f16(x, M, K, K, xq, K, xs);
    oracle_gemm_w4a8(xq, xs, M, K, w, ws, N, G, bias, y, NULL);
}
