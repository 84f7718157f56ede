/*
 * CPU oracle for the producers of the linears' fp16 inputs: act_and_mul and
 * RMSNorm, alone and followed by the per-token quantization.  TEST
 * INFRASTRUCTURE ONLY: the CPU restatement the HIP kernels are compared against.
 *
 * What it restates (reference = Josephur/fni8-serve):
 *   - act_and_mul: out = act(gate) * up over a merged [.., 2I] row, first half
 *     gate (fni8serve/layers/activation.py:20-42: SiluAndMul, GeluAndMul with
 *     approximate="tanh").  The fused `fni8.act_and_mul` is closed; its eager
 *     fallback is `F.silu(gate) * up` / `F.gelu(gate, approximate="tanh") * up`.
 *     The build's convention, evaluated in fp32 with one rounding per
 *     operation and a single rounding to fp16 at the end:
 *         gate(g) = g / (1 + exp(t)),  t = -g (silu)
 *                   or t = -(2 sqrt(2/pi)) * (g + 0.044715 * g^3)   (gelu_tanh:
 *                   0.5 g (1 + tanh y) == g * sigmoid(2y))
 *         t clamped to [-86, 88] (NaN -> -86), out = fp16(gate(g) * up)
 *     with exp by Cody-Waite reduction and a degree-7 Taylor polynomial
 *     (exp_cw below).
 *   - RMSNorm (fni8serve/layers/norm.py:37-58):
 *         h = residual ? fp16(x + residual) : x          (norm.py:56-58)
 *         out = fp16((h * r) * w), r = 1 / sqrt(ss / K + eps),
 *         w = weight, or 1 + weight with unit_offset (Gemma, norm.py:42)
 *     in fp32 (norm.py:38-43 computes in fp32 and casts back).  ss, the sum
 *     of squares, is taken in the fixed order of sumsq_fixed below.
 *   - the quantized forms: oracle_quant_rowwise_f16 applied to those fp16 rows.
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

uint16_t oracle_f32_to_f16(float f);
float oracle_f16_to_f32(uint16_t h);
void oracle_quant_rowwise_f16(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                              int64_t ldq, float* s);

#define ACT_SILU 0
#define ACT_GELU_TANH 1

static float bits_f(uint32_t b) {
    float f;
    memcpy(&f, &b, 4);
    return f;
}

/* exp(x) for x in [-86, 88].  x = k ln2 + r with k = rint(x * log2(e)); ln2
 * is split into a head with 15 significant bits (k * head exact for
 * |k| <= 127) and the fp32 tail of ln2 - head; exp(r), |r| <= ln2 / 2, by the
 * Taylor polynomial of degree 7 in Horner form; times 2^k built in the
 * exponent field. */
float oracle_exp_cw(float x) {
    const float k = rintf(x * 0x1.715476p+0f);
    float r = fmaf(-k, 0x1.62e4p-1f, x);
    r = fmaf(-k, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = fmaf(p, r, 0x1.6c16c2p-10f);
    p = fmaf(p, r, 0x1.111112p-7f);
    p = fmaf(p, r, 0x1.555556p-5f);
    p = fmaf(p, r, 0x1.555556p-3f);
    p = fmaf(p, r, 0.5f);
    p = fmaf(p, r, 1.0f);
    p = fmaf(p, r, 1.0f);
    return p * bits_f((uint32_t)((int)k + 127) << 23);
}

static float gated(float g, float t) {
    t = t >= -86.0f ? t : -86.0f;
    t = t <= 88.0f ? t : 88.0f;
    return g / (1.0f + oracle_exp_cw(t));
}

float oracle_act_f32(float g, int act) {
    if (act == ACT_SILU) return gated(g, -g);
    const float g3 = (g * g) * g;
    const float inner = g + 0x1.6e4e26p-5f * g3;
    return gated(g, -(0x1.988454p+0f * inner));
}

void oracle_act_and_mul_f16(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, int act,
                            uint16_t* out, int64_t ldo) {
    for (int64_t m = 0; m < M; m++) {
        const uint16_t* xr = x + m * ldx;
        for (int64_t i = 0; i < I; i++) {
            const float a = oracle_act_f32(oracle_f16_to_f32(xr[i]), act);
            out[m * ldo + i] = oracle_f32_to_f16(a * oracle_f16_to_f32(xr[I + i]));
        }
    }
}

void oracle_act_and_mul_quant_f16(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, int act,
                                  uint16_t* tmp, int8_t* q, int64_t ldq, float* s) {
    oracle_act_and_mul_f16(x, ldx, M, I, act, tmp, I);
    oracle_quant_rowwise_f16(tmp, M, I, I, q, ldq, s);
}

/* Sum of squares in the fixed order: the row is cut into 8-element chunks;
 * accumulator L (of 256) adds, from +0, chunks L, L + 256, ... in turn, each
 * chunk's elements in order; within each group of 64 accumulators,
 * p[l] = p[l] + p[l ^ d] for d = 32, 16, 8, 4, 2, 1; then
 * (w0 + w1) + (w2 + w3) over the four groups. */
float oracle_sumsq_fixed(const uint16_t* h, int64_t K) {
    float lane[256];
    for (int l = 0; l < 256; l++) lane[l] = 0.0f;
    for (int64_t c = 0; 8 * c < K; c++) {
        const int l = (int)(c % 256);
        const int64_t end = 8 * c + 8 < K ? 8 * c + 8 : K;
        for (int64_t k = 8 * c; k < end; k++) {
            const float f = oracle_f16_to_f32(h[k]);
            lane[l] = lane[l] + f * f;
        }
    }
    float wsum[4];
    for (int w = 0; w < 4; w++) {
        float p[64], n[64];
        for (int l = 0; l < 64; l++) p[l] = lane[64 * w + l];
        for (int d = 32; d > 0; d >>= 1) {
            for (int l = 0; l < 64; l++) n[l] = p[l] + p[l ^ d];
            memcpy(p, n, sizeof p);
        }
        wsum[w] = p[0];
    }
    return (wsum[0] + wsum[1]) + (wsum[2] + wsum[3]);
}

/* res (or NULL), res_out (or NULL, written only with res), tmp: K fp16 of
 * scratch for h. */
void oracle_rmsnorm_f16(const uint16_t* x, int64_t ldx, const uint16_t* res, int64_t ldr,
                        const uint16_t* w, float eps, int unit, int64_t M, int64_t K,
                        uint16_t* out, int64_t ldo, uint16_t* res_out, int64_t ldro,
                        uint16_t* tmp) {
    for (int64_t m = 0; m < M; m++) {
        const uint16_t* xr = x + m * ldx;
        for (int64_t k = 0; k < K; k++) {
            tmp[k] = res ? oracle_f32_to_f16(oracle_f16_to_f32(xr[k]) +
                                             oracle_f16_to_f32(res[m * ldr + k]))
                         : xr[k];
            if (res && res_out) res_out[m * ldro + k] = tmp[k];
        }
        const float ss = oracle_sumsq_fixed(tmp, K);
        const float r = 1.0f / sqrtf(ss / (float)K + eps);
        for (int64_t k = 0; k < K; k++) {
            const float wf = unit ? 1.0f + oracle_f16_to_f32(w[k]) : oracle_f16_to_f32(w[k]);
            out[m * ldo + k] = oracle_f32_to_f16((oracle_f16_to_f32(tmp[k]) * r) * wf);
        }
    }
}

void oracle_rmsnorm_quant_f16(const uint16_t* x, int64_t ldx, const uint16_t* res, int64_t ldr,
                              const uint16_t* w, float eps, int unit, int64_t M, int64_t K,
                              uint16_t* normed, int8_t* q, int64_t ldq, float* s,
                              uint16_t* res_out, int64_t ldro, uint16_t* tmp) {
    oracle_rmsnorm_f16(x, ldx, res, ldr, w, eps, unit, M, K, normed, K, res_out, ldro, tmp);
    oracle_quant_rowwise_f16(normed, M, K, K, q, ldq, s);
}

void oracle_exp_cw_n(const float* x, float* y, int64_t n) {
    for (int64_t i = 0; i < n; i++) y[i] = oracle_exp_cw(x[i]);
}

void oracle_act_f32_n(const float* g, float* y, int64_t n, int act) {
    for (int64_t i = 0; i < n; i++) y[i] = oracle_act_f32(g[i], act);
}
