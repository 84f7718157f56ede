/*
 * Exhaustive check of the division-free quantization used by the GPU decode
 * kernels.  TEST INFRASTRUCTURE ONLY (loaded by tests/test_oracle.py).
 *
 * The oracle quantizes with a correctly rounded division, q = rint(fl(x / s)),
 * s = fl(max(amax, eps) / 127) (w8a8_oracle.c, after the reference's quant
 * idiom, fni8serve tests/test_smoke.py:16-17).  The fused decode kernel instead
 * computes, once per row, y = fl(1 / s), and per element
 *     t = fl(x * y);  r = fma(-t, s, x);  v = fma(r, y, t);  q = rint(v)
 * (Markstein's correction: r is exact, and v is the correctly rounded quotient
 * when y is the correctly rounded reciprocal).  Both x and amax are fp16, so the
 * claim can be checked on every input: for each finite fp16 amax >= 0 and every
 * fp16 x with |x| <= amax, compare v with fl(x / s) bit for bit (x != 0; for
 * x = +-0 the two may differ only in the sign of zero) and rint(v) with
 * rint(fl(x / s)).
 *
 * The kernels then round without rint, clamp or a float-to-int conversion:
 * the int8 is the low byte of the bits of v + 1.5 * 2^23 (for |v| < 2^22 the
 * addition rounds v to an integer, ties to even, and leaves it in the low bits
 * in two's complement).  out[3] counts pairs where that byte differs from the
 * oracle's int8, clamp(rint(fl(x / s)), -127, 127).
 *
 * mode 0 checks those formulas; mode 1 drops the correction (v = t), the
 * plausible shortcut; mode 2 adds 2^23 instead of 1.5 * 2^23 (a plausible slip
 * that breaks negative values) -- so that tests can show the check detects both.
 * out[0] = pairs checked, out[1] = quotient mismatches with x != 0,
 * out[2] = rounded-integer mismatches (any x), out[3] = int8 byte mismatches.
 */
#include <math.h>
#include <stdint.h>
#include <string.h>

static float h2f_bits(uint16_t h) {
    const uint32_t sign = (h >> 15) & 1u, e = (h >> 10) & 31u, m = h & 1023u;
    float v;
    if (e == 0) v = ldexpf((float)m, -24);
    else v = ldexpf((float)(m | 1024u), (int)e - 25);
    return sign ? -v : v;
}

void oracle_quant_identity_check(int mode, int64_t* out) {
    int64_t pairs = 0, bad_quot = 0, bad_int = 0, bad_byte = 0;
    const float magic = mode == 2 ? 8388608.0f : 12582912.0f;
#pragma omp parallel for schedule(dynamic, 64) reduction(+ : pairs, bad_quot, bad_int, bad_byte)
    for (int a = 0; a < 0x7c00; a++) {
        const float amax = h2f_bits((uint16_t)a);
        const float num = amax > 1e-6f ? amax : 1e-6f;
        const float s = num / 127.0f;
        const float y = 1.0f / s;
        for (int xb = 0; xb <= a; xb++) {
            for (int sg = 0; sg < 2; sg++) {
                const float x = h2f_bits((uint16_t)(xb | (sg << 15)));
                const float v = x / s;
                const float t = x * y;
                const float r = fmaf(-t, s, x);
                const float v2 = mode == 1 ? t : fmaf(r, y, t);
                pairs++;
                if (x != 0.0f && memcmp(&v, &v2, sizeof v) != 0) bad_quot++;
                if (rintf(v) != rintf(v2)) bad_int++;
                float qf = rintf(v);
                qf = qf > 127.0f ? 127.0f : (qf < -127.0f ? -127.0f : qf);
                const int8_t q_ref = (int8_t)qf;
                const float sum = v2 + magic;
                uint32_t bits;
                memcpy(&bits, &sum, sizeof bits);
                if ((int8_t)(uint8_t)(bits & 0xffu) != q_ref) bad_byte++;
            }
        }
    }
    out[0] = pairs;
    out[1] = bad_quot;
    out[2] = bad_int;
    out[3] = bad_byte;
}
