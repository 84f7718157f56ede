// MoE router: scores -> (group-limited) top-k -> weights, one wave per token
// (gfx950).  Replaces the chain of small launches of SparseMoE's routing
// (fni8serve/models/moe.py:62-97: softmax or sigmoid, the selection bias,
// the group mask, torch.topk, gather, renormalisation, scaling, cast) with
// one launch and no host synchronisation, so an MoE layer can be captured in a
// HIP graph.
//
// Lane l of the wave holds experts l, l + 64, ... (E / 64 of them, E <= 1024).
// Arithmetic, all fp32, one rounding per operation:
//   softmax   m = max(l); e_i = exp(max(l_i - m, -86)); s = sum of e_i (lane
//             sums in expert order, then p[l] += p[l ^ d], d = 32..1);
//             p_i = e_i / s.  A NaN logit makes the whole row NaN.
//   sigmoid   p_i = 1 / (1 + exp(clamp(-l_i, -86, 88))); NaN stays NaN.
//   sel_i     p_i (+ bias_i)
//   groups    group score = max of sel over the group (NaN wins); the
//             topk_group best groups are kept (same order as top-k), the
//             others' sel set to -inf (groups <= 64)
//   top-k     k times: the largest sel, NaN above +inf, ties to the lower
//             index (torch.topk's order); -0 ranks as +0
//   weights   softmax: the selected sel; sigmoid: the selected p (unbiased);
//             renorm: w_j / max(w_0 + ... + w_{k-1}, 1e-9) (slot order);
//             then w_j * scale, rounded to fp16.
// exp is fni8::exp_cw (Cody-Waite reduction + degree-7 Taylor polynomial).
#include "common.h"

namespace {

constexpr int kRouteThreads = 256;  // four tokens per workgroup

__device__ __forceinline__ float nan_max(float a, float b) {
    if (a != a) return a;
    if (b != b) return b;
    return a > b ? a : b;
}

__device__ __forceinline__ float wave_nan_max(float v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) v = nan_max(v, __shfl_xor(v, d, 64));
    return v;
}

// Order key of a selection score: NaN above everything, -0 as +0, then the
// usual float order (sign-magnitude mapped onto unsigned order).
__device__ __forceinline__ uint32_t rank_key(float v) {
    if (v != v) return 0xffffffffu;
    if (v == 0.0f) v = 0.0f;
    const uint32_t u = __builtin_bit_cast(uint32_t, v);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Argmax over the wave of (key, index): larger key, then smaller index.
// Key 0 marks taken or absent entries: every real score ranks above it
// (-inf maps to 0x007fffff).
__device__ __forceinline__ uint64_t wave_best(uint64_t v) {
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) {
        const uint64_t o = __shfl_xor(v, d, 64);
        v = o > v ? o : v;
    }
    return v;
}

__device__ __forceinline__ uint64_t pack(uint32_t key, int idx) {
    return ((uint64_t)key << 32) | (uint32_t)(0xffffffffu - (uint32_t)idx);
}

__device__ __forceinline__ int unpack_index(uint64_t v) {
    return (int)(0xffffffffu - (uint32_t)(v & 0xffffffffu));
}

template <int PL>
__global__ __launch_bounds__(kRouteThreads) void moe_route_kernel(
    const float* __restrict__ logits, int64_t ldl, int T, int E, int scoring,
    const float* __restrict__ bias, int groups, int topk_group, int k, int renorm, float scale,
    uint16_t* __restrict__ topw, int32_t* __restrict__ topi) {
    const int lane = threadIdx.x & 63;
    const int t = blockIdx.x * (kRouteThreads / 64) + (threadIdx.x >> 6);
    if (t >= T) return;  // whole waves exit together
    const float* lr = logits + (int64_t)t * ldl;

    float p[PL], sel[PL];
    uint32_t key[PL];
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int e = lane + 64 * j;
        p[j] = e < E ? lr[e] : -__builtin_inff();
    }
    if (scoring == FNI8_SCORE_SOFTMAX) {
        float m = -__builtin_inff();
#pragma unroll
        for (int j = 0; j < PL; j++)
            if (lane + 64 * j < E) m = nan_max(m, p[j]);
        m = wave_nan_max(m);
        float s = 0.0f;
#pragma unroll
        for (int j = 0; j < PL; j++) {
            if (lane + 64 * j < E) {
                float d = p[j] - m;
                d = d >= -86.0f ? d : -86.0f;  // d <= 0 (a NaN row is handled below)
                p[j] = fni8::exp_cw(d);
                s = s + p[j];
            }
        }
#pragma unroll
        for (int d = 32; d > 0; d >>= 1) s = s + __shfl_xor(s, d, 64);
        const bool nan_row = m != m;
#pragma unroll
        for (int j = 0; j < PL; j++)
            p[j] = nan_row ? __builtin_nanf("") : p[j] / s;
    } else {
#pragma unroll
        for (int j = 0; j < PL; j++) {
            const float l = p[j];
            float x = -l;
            x = x >= -86.0f ? x : -86.0f;
            x = x <= 88.0f ? x : 88.0f;
            p[j] = l != l ? l : 1.0f / (1.0f + fni8::exp_cw(x));
        }
    }
#pragma unroll
    for (int j = 0; j < PL; j++) {
        const int e = lane + 64 * j;
        sel[j] = (bias && e < E) ? p[j] + bias[e] : p[j];
    }

    if (groups > 0) {
        // Group scores, lane g holding group g's (groups <= 64); then
        // topk_group rounds of the best remaining group.
        const int per = E / groups;
        float gs = -__builtin_inff();
        for (int g = 0; g < groups; g++) {
            float gm = -__builtin_inff();
#pragma unroll
            for (int j = 0; j < PL; j++) {
                const int e = lane + 64 * j;
                if (e < E && e / per == g) gm = nan_max(gm, sel[j]);
            }
            gm = wave_nan_max(gm);
            if (lane == g) gs = gm;
        }
        uint32_t gkey = lane < groups ? rank_key(gs) : 0u;
        uint64_t kept = 0;
        for (int r = 0; r < topk_group; r++) {
            const uint64_t best = wave_best(gkey ? pack(gkey, lane) : 0ull);
            const int g = unpack_index(best);
            kept |= 1ull << g;
            if (lane == g) gkey = 0u;
        }
#pragma unroll
        for (int j = 0; j < PL; j++) {
            const int e = lane + 64 * j;
            if (e < E && !((kept >> (e / per)) & 1)) sel[j] = -__builtin_inff();
        }
    }

#pragma unroll
    for (int j = 0; j < PL; j++) key[j] = (lane + 64 * j < E) ? rank_key(sel[j]) : 0u;

    // k rounds of the wave argmax; the owner lane marks its entry taken, lane r
    // keeps slot r, and the weights are summed in slot order as they come.
    float my_w = 0.0f, sum = 0.0f;
    int my_idx = 0;
    for (int r = 0; r < k; r++) {
        uint64_t mine = 0;
        float mine_w = 0.0f;
#pragma unroll
        for (int j = 0; j < PL; j++) {
            const uint64_t c = key[j] ? pack(key[j], lane + 64 * j) : 0ull;
            if (c > mine) {
                mine = c;
                mine_w = scoring == FNI8_SCORE_SOFTMAX ? sel[j] : p[j];
            }
        }
        const uint64_t best = wave_best(mine);
        const int e = unpack_index(best);
        const float wr = __shfl(mine_w, e & 63, 64);
        sum = sum + wr;
        if (lane == r) {
            my_w = wr;
            my_idx = e;
        }
        if (lane == (e & 63)) {
#pragma unroll
            for (int j = 0; j < PL; j++)
                if (lane + 64 * j == e) key[j] = 0u;
        }
    }
    if (lane < k) {
        float v = my_w;
        if (renorm) {
            float denom = sum >= 1e-9f ? sum : 1e-9f;
            if (sum != sum) denom = sum;
            v = v / denom;
        }
        v = v * scale;
        topw[(int64_t)t * k + lane] = fni8::f2h(v);
        topi[(int64_t)t * k + lane] = my_idx;
    }
}

}  // namespace

namespace fni8h {

int launch_moe_route(const float* logits, int64_t ldl, int64_t T, int64_t E, int scoring,
                     const float* bias, int64_t groups, int64_t topk_group, int64_t k, int renorm,
                     float scale, uint16_t* topw, int32_t* topi, hipStream_t st) {
    if (T == 0) return FNI8_OK;
    const int pl = (int)((E + 63) / 64);
    const dim3 grid((unsigned)((T + 3) / 4)), block(kRouteThreads);
#define FNI8_ROUTE(PL)                                                                        \
    hipLaunchKernelGGL(moe_route_kernel<PL>, grid, block, 0, st, logits, ldl, (int)T, (int)E, \
                       scoring, bias, (int)groups, (int)topk_group, (int)k, renorm, scale,     \
                       topw, topi)
    if (pl <= 1) FNI8_ROUTE(1);
    else if (pl <= 2) FNI8_ROUTE(2);
    else if (pl <= 4) FNI8_ROUTE(4);
    else if (pl <= 8) FNI8_ROUTE(8);
    else FNI8_ROUTE(16);
#undef FNI8_ROUTE
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("moe_route launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

}  // namespace fni8h
