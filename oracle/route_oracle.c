/*
 * CPU oracle for the MoE router.  TEST INFRASTRUCTURE ONLY: the CPU
 * restatement the HIP routing kernel is compared against.
 *
 * Restates the routing of SparseMoE.forward (reference
 * fni8serve/models/moe.py:62-97), evaluated in fp32 with one rounding per
 * operation:
 *   scores   softmax over all experts (moe.py:68-70) -- m = max logit,
 *            e_i = exp(max(l_i - m, -86)), s = sum of e_i in the fixed order
 *            below, p_i = e_i / s, a NaN logit making the row NaN -- or
 *            sigmoid (moe.py:65-67): p_i = 1 / (1 + exp(clamp(-l_i, -86, 88)))
 *   sel      p + bias (moe.py:67, selection only)
 *   groups   (moe.py:72-82) group score = max of sel over each group of E/G
 *            consecutive experts (NaN wins); the topk_group best groups stay,
 *            the other experts' sel becomes -inf
 *   top-k    (moe.py:84-88) largest sel first, NaN above +inf, ties to the
 *            lower index, -0 ranked as +0
 *   weights  softmax: the selected sel; sigmoid: the selected p (moe.py:86);
 *            renormalised by max(sum in slot order, 1e-9) (moe.py:89-90),
 *            times the scaling factor, rounded to fp16 (moe.py:91)
 * Sum order of the softmax denominator: experts are dealt to 64 accumulators
 * (expert e to accumulator e % 64, each summing its experts in increasing e
 * from +0), then p[l] = p[l] + p[l ^ d] for d = 32, 16, 8, 4, 2, 1.
 * exp is oracle_exp_cw (act_norm_oracle.c).
 *
 * Build: oracle/Makefile (gcc -O3 -ffp-contract=off, no fast-math).
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

float oracle_exp_cw(float x);
uint16_t oracle_f32_to_f16(float f);

static float nan_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    return a > b ? a : b;
}

static uint32_t rank_key(float v) {
    if (v != v) return 0xffffffffu;
    if (v == 0.0f) v = 0.0f;
    uint32_t u;
    memcpy(&u, &v, 4);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

/* index of the best untaken entry: larger key, then smaller index */
static int best_of(const uint32_t* key, const uint8_t* taken, int n) {
    int best = -1;
    for (int i = 0; i < n; i++) {
        if (taken[i]) continue;
        if (best < 0 || key[i] > key[best]) best = i;
    }
    return best;
}

void oracle_moe_route(const float* logits, int64_t T, int64_t E, int64_t ldl, int scoring,
                      const float* bias, int64_t groups, int64_t topk_group, int64_t k,
                      int renorm, float scale, uint16_t* topw, int32_t* topi) {
    float p[1024], sel[1024], acc[64];
    uint32_t key[1024];
    uint8_t taken[1024];
    for (int64_t t = 0; t < T; t++) {
        const float* l = logits + t * ldl;
        if (scoring == 0) {
            float m = -INFINITY;
            for (int64_t e = 0; e < E; e++) m = nan_max(m, l[e]);
            for (int a = 0; a < 64; a++) acc[a] = 0.0f;
            for (int64_t e = 0; e < E; e++) {
                float d = l[e] - m;
                d = d >= -86.0f ? d : -86.0f;
                p[e] = oracle_exp_cw(d);
                acc[e % 64] = acc[e % 64] + p[e];
            }
            for (int d = 32; d > 0; d >>= 1) {
                float n[64];
                for (int a = 0; a < 64; a++) n[a] = acc[a] + acc[a ^ d];
                memcpy(acc, n, sizeof acc);
            }
            const float s = acc[0];
            for (int64_t e = 0; e < E; e++) p[e] = (m != m) ? NAN : p[e] / s;
        } else {
            for (int64_t e = 0; e < E; e++) {
                float x = -l[e];
                x = x >= -86.0f ? x : -86.0f;
                x = x <= 88.0f ? x : 88.0f;
                p[e] = l[e] != l[e] ? l[e] : 1.0f / (1.0f + oracle_exp_cw(x));
            }
        }
        for (int64_t e = 0; e < E; e++) sel[e] = bias ? p[e] + bias[e] : p[e];
        if (groups > 0) {
            const int64_t per = E / groups;
            uint32_t gkey[64];
            uint8_t gtaken[64], kept[64];
            for (int64_t g = 0; g < groups; g++) {
                float gm = -INFINITY;
                for (int64_t e = g * per; e < (g + 1) * per; e++) gm = nan_max(gm, sel[e]);
                gkey[g] = rank_key(gm);
                gtaken[g] = 0;
                kept[g] = 0;
            }
            for (int64_t r = 0; r < topk_group; r++) {
                const int g = best_of(gkey, gtaken, (int)groups);
                gtaken[g] = 1;
                kept[g] = 1;
            }
            for (int64_t e = 0; e < E; e++)
                if (!kept[e / per]) sel[e] = -INFINITY;
        }
        for (int64_t e = 0; e < E; e++) {
            key[e] = rank_key(sel[e]);
            taken[e] = 0;
        }
        float w[32];
        float sum = 0.0f;
        for (int64_t r = 0; r < k; r++) {
            const int e = best_of(key, taken, (int)E);
            taken[e] = 1;
            w[r] = scoring == 0 ? sel[e] : p[e];
            topi[t * k + r] = e;
            sum = sum + w[r];
        }
        float denom = sum >= 1e-9f ? sum : 1e-9f;
        if (sum != sum) denom = sum;
        for (int64_t r = 0; r < k; r++) {
            float v = renorm ? w[r] / denom : w[r];
            v = v * scale;
            topw[t * k + r] = oracle_f32_to_f16(v);
        }
    }
}
