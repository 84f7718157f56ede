// The producers of the linears' fp16 inputs, each alone or with the per-token
// int8 quantization of its output fused in (gfx950):
//
//   act_and_mul   out = fp16(act(gate) * up) over a merged [.., 2I] row, first
//                 half gate, second half up (fni8serve/layers/activation.py:20-42);
//                 act = silu or the tanh form of gelu.
//   rmsnorm       h = x (+ residual, rounded to fp16);
//                 out = fp16((h * 1/sqrt(mean(h^2) + eps)) * w), w = weight or
//                 1 + weight (fni8serve/layers/norm.py:37-58).
//
// The fused forms write int8 + one fp32 scale per row instead of the fp16 row,
// bit-identical to quantizing the unfused output, so the down projection (after
// act_and_mul) and QKV / gate_up (after rmsnorm) skip an fp16 round trip through
// HBM and a launch.  All four are HBM-bound streaming kernels: one workgroup per
// row for the row-wise ones, the row held in registers between its reduction
// and its output.
//
// Every float operation is one IEEE fp32 rounding (the library is built with
// -ffp-contract=off and correctly rounded division and square root), and the
// sum of squares has a fixed order (below), so a CPU restatement of the same
// operations reproduces every output bit.
#include "decode_tile.h"

namespace {

constexpr int kThreads = 256;

// ---- activations ------------------------------------------------------------

// g / (1 + exp(t)), t clamped to [-86, 88] (a NaN t is taken as -86; a NaN g
// still gives NaN).
__device__ __forceinline__ float gated(float g, float t) {
    t = t >= -86.0f ? t : -86.0f;
    t = t <= 88.0f ? t : 88.0f;
    return g / (1.0f + fni8::exp_cw(t));
}

// silu(g) = g * sigmoid(g).  gelu, tanh form: 0.5 g (1 + tanh(y)) with
// y = sqrt(2/pi) (g + 0.044715 g^3), which is g * sigmoid(2y) -- the same
// division, with no cancellation near tanh = -1.
template <int ACT>
__device__ __forceinline__ float act_fn(float g) {
    if (ACT == FNI8_ACT_SILU) return gated(g, -g);
    const float g3 = (g * g) * g;
    const float inner = g + 0x1.6e4e26p-5f * g3;  // 0.044715
    return gated(g, -(0x1.988454p+0f * inner));   // 2 sqrt(2/pi)
}

template <int ACT>
__device__ __forceinline__ uint16_t act_mul(uint16_t g, uint16_t u) {
    return fni8::f2h(act_fn<ACT>(fni8::h2f(g)) * fni8::h2f(u));
}

// 8 gates and the 8 matching ups (16-byte chunks) -> 8 fp16 outputs.
template <int ACT>
__device__ __forceinline__ uint4 act_chunk(uint4 g, uint4 u) {
    const uint32_t gw[4] = {g.x, g.y, g.z, g.w}, uw[4] = {u.x, u.y, u.z, u.w};
    uint32_t o[4];
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const uint32_t lo = act_mul<ACT>((uint16_t)(gw[i] & 0xffffu), (uint16_t)(uw[i] & 0xffffu));
        const uint32_t hi = act_mul<ACT>((uint16_t)(gw[i] >> 16), (uint16_t)(uw[i] >> 16));
        o[i] = lo | (hi << 16);
    }
    return make_uint4(o[0], o[1], o[2], o[3]);
}

// the running max of magnitude bits, as one 16-bit maximum
__device__ __forceinline__ uint32_t chunk_amax(uint4 v, uint32_t amax) {
    const uint32_t m = fni8::amax_fold(fni8::amax_chunk(0u, v));
    return m > amax ? m : amax;
}

// Row max over a workgroup of TPB threads (every thread gets it).
template <int TPB = kThreads>
__device__ __forceinline__ uint32_t block_amax(uint32_t amax, uint32_t* red) {
    const int tid = threadIdx.x;
    amax = fni8::wave_max_uniform(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < TPB / 64; i++) amax = red[i] > amax ? red[i] : amax;
    return amax;
}

// Elementwise act_and_mul, 16-byte chunks (I % 8 == 0, aligned rows).
template <int ACT>
__global__ __launch_bounds__(kThreads) void act_mul_vec_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t I,
    uint16_t* __restrict__ out, int64_t ldo) {
    const int64_t cpr = I / 8;
    const int64_t total = M * cpr;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t m = idx / cpr, c = idx - m * cpr;
        const uint16_t* xr = x + m * ldx + 8 * c;
        const uint4 g = *reinterpret_cast<const uint4*>(xr);
        const uint4 u = *reinterpret_cast<const uint4*>(xr + I);
        *reinterpret_cast<uint4*>(out + m * ldo + 8 * c) = act_chunk<ACT>(g, u);
    }
}

// Elementwise act_and_mul, any I and alignment.
template <int ACT>
__global__ __launch_bounds__(kThreads) void act_mul_any_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t M, int64_t I,
    uint16_t* __restrict__ out, int64_t ldo) {
    const int64_t total = M * I;
    for (int64_t idx = (int64_t)blockIdx.x * kThreads + threadIdx.x; idx < total;
         idx += (int64_t)gridDim.x * kThreads) {
        const int64_t m = idx / I, i = idx - m * I;
        const uint16_t* xr = x + m * ldx;
        out[m * ldo + i] = act_mul<ACT>(xr[i], xr[I + i]);
    }
}

// act_and_mul + per-token quantization, one workgroup of TPB threads per row:
// lane `tid` holds chunks tid, tid + TPB, ... (CH of them) of the activated
// row in registers through the row max, then quantizes them.  Few rows take
// TPB = 1024, so that each SIMD has four waves to hide the exp / division
// dependency chains; many rows take 256.
template <int ACT, int CH, int TPB>
__global__ __launch_bounds__(TPB) void act_quant_vec_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int I, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ s) {
    __shared__ uint32_t red[TPB / 64];
    const int m = blockIdx.x, tid = threadIdx.x;
    const uint16_t* xr = x + (int64_t)m * ldx;
    uint4 a[CH];
    uint32_t amax = 0;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int k = (c * TPB + tid) * 8;
        if (k < I) {
            const uint4 g = *reinterpret_cast<const uint4*>(xr + k);
            const uint4 u = *reinterpret_cast<const uint4*>(xr + I + k);
            a[c] = act_chunk<ACT>(g, u);
            amax = chunk_amax(a[c], amax);
        }
    }
    amax = block_amax<TPB>(amax, red);
    const float sc = fni8::row_scale_from_bits(amax);
    const bool live = __builtin_isfinite(sc);
    const float yr = 1.0f / sc;
    if (tid == 0) s[m] = sc;
    int8_t* qr = q + (int64_t)m * ldq;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int k = (c * TPB + tid) * 8;
        if (k < I) *reinterpret_cast<uint2*>(qr + k) = fni8::quant_chunk(a[c], sc, yr, live);
    }
}

// act_and_mul + quantization for few rows (16-byte chunks): a row's
// activations are VALU work (an exp and a division per element), too much for
// the one workgroup per row above when there are fewer rows than CUs.  So G
// workgroups share a row, each activating 1/G of its chunks in registers, and
// the row maximum is assembled from their partial maxima, exchanged through the
// L2 of the XCD they run on (the exchange rules of decode_tile.h): workgroup b
// takes part (b/8) % G of row (b/8/G)*8 + b%8, so the G parts of a row have
// ids equal mod 8 and share an XCD under the round-robin dispatch.  Each part
// stores its maximum and then a flag holding the dispatch tag into its XCD's
// region of the workspace, and polls the other parts' flags there (bounded);
// a part whose flag does not arrive in time is recomputed (its maximum only),
// so the result is the same bits whatever the placement.
// Workspace: [8 XCDs][rows rounded up to 8][G] 128-byte lines (flag, maximum).
constexpr int kSplitLine = 16;  // u64 words per line

template <int ACT, int CH>
__global__ __launch_bounds__(kThreads) void act_quant_split_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int M, int I, int G, int8_t* __restrict__ q,
    int64_t ldq, float* __restrict__ s, uint64_t* __restrict__ work, uint64_t wait_ticks) {
    __shared__ uint32_t red[kThreads / 64];
    __shared__ uint32_t found[2];  // [0] max over the parts received, [1] bit mask of missing parts
    const int b = blockIdx.x, tid = threadIdx.x, lane = tid & 63;
    const int wave = tid >> 6;
    const int qd = b >> 3, part = qd % G, row = (qd / G) * 8 + (b & 7);
    if (row >= M) return;
    const int cpr = I / 8;                 // 16-byte chunks of the row
    const int per = (cpr + G - 1) / G;     // chunks of a part (<= CH * kThreads)
    const uint16_t* xr = x + (int64_t)row * ldx;
    auto part_chunks = [&](int p, uint4 (&a)[CH], bool keep) -> uint32_t {
        const int c0 = p * per, c1 = min(cpr, c0 + per);
        uint32_t m = 0;
#pragma unroll
        for (int j = 0; j < CH; j++) {
            const int c = c0 + j * kThreads + tid;
            if (c < c1) {
                const uint4 g = *reinterpret_cast<const uint4*>(xr + 8 * c);
                const uint4 u = *reinterpret_cast<const uint4*>(xr + I + 8 * c);
                const uint4 v = act_chunk<ACT>(g, u);
                m = chunk_amax(v, m);
                if (keep) a[j] = v;
            }
        }
        return m;
    };
    uint4 a[CH];
    uint32_t amax = block_amax(part_chunks(part, a, true), red);

    const int mpad = (M + 7) & ~7;
    uint64_t* lines = work + ((int64_t)fni8dec::xcc_id() * mpad + row) * G * kSplitLine;
    const uint64_t tag = fni8dec::dispatch_tag();
    if (tid == 0) {
        lines[part * kSplitLine + 1] = amax;
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
        fni8dec::publish_flag(lines + part * kSplitLine, tag);
    }
    // wave 0: lane p waits for part p's flag, then reads its maximum
    if (wave == 0) {
        const bool mine = lane < G && lane != part;
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        bool seen = !mine;
        for (;;) {
            if (!seen) seen = fni8dec::poll_flag(lines + lane * kSplitLine) == tag;
            if (__ballot(!seen) == 0 || __builtin_amdgcn_s_memrealtime() - t0 >= wait_ticks) break;
            __builtin_amdgcn_s_sleep(2);
        }
        uint32_t m = 0;
        if (mine && seen) m = (uint32_t)fni8dec::poll_flag(lines + lane * kSplitLine + 1);
        m = fni8::wave_max_uniform(m);
        const uint64_t miss = __ballot(mine && !seen);
        if (lane == 0) {
            found[0] = m;
            found[1] = (uint32_t)miss;
        }
    }
    __syncthreads();
    amax = found[0] > amax ? found[0] : amax;
    const uint32_t miss = __builtin_amdgcn_readfirstlane(found[1]);
    for (int p = 0; p < G; p++) {
        if (!((miss >> p) & 1u)) continue;
        __syncthreads();  // red is reused
        uint4 tmp[CH];
        const uint32_t mp = block_amax(part_chunks(p, tmp, false), red);
        amax = mp > amax ? mp : amax;
    }
    const float sc = fni8::row_scale_from_bits(amax);
    const bool live = __builtin_isfinite(sc);
    const float yr = 1.0f / sc;
    if (part == 0 && tid == 0) s[row] = sc;
    int8_t* qr = q + (int64_t)row * ldq;
    const int c0 = part * per, c1 = min(cpr, c0 + per);
#pragma unroll
    for (int j = 0; j < CH; j++) {
        const int c = c0 + j * kThreads + tid;
        if (c < c1) *reinterpret_cast<uint2*>(qr + 8 * c) = fni8::quant_chunk(a[j], sc, yr, live);
    }
}

// act_and_mul + quantization, any I and alignment: the activation is computed
// twice (max pass, quantize pass); both give the same bits.
template <int ACT>
__global__ __launch_bounds__(kThreads) void act_quant_any_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int64_t I, int8_t* __restrict__ q,
    int64_t ldq, float* __restrict__ s) {
    __shared__ uint32_t red[kThreads / 64];
    const int64_t m = blockIdx.x;
    const uint16_t* xr = x + m * ldx;
    uint32_t amax = 0;
    for (int64_t i = threadIdx.x; i < I; i += kThreads) {
        const uint32_t b = act_mul<ACT>(xr[i], xr[I + i]) & 0x7fffu;
        amax = b > amax ? b : amax;
    }
    amax = block_amax(amax, red);
    const float sc = fni8::row_scale_from_bits(amax);
    if (threadIdx.x == 0) s[m] = sc;
    int8_t* qr = q + m * ldq;
    for (int64_t i = threadIdx.x; i < I; i += kThreads)
        qr[i] = (int8_t)fni8::quant_one(fni8::h2f(act_mul<ACT>(xr[i], xr[I + i])), sc);
}

// ---- RMSNorm ----------------------------------------------------------------
//
// Order of the sum of squares (each square of an fp16 value is exact in fp32):
// the row is cut into 8-element chunks; lane L of the 256 accumulates, from
// +0, the chunks L, L + 256, L + 512, ... in turn, each chunk's elements in
// order; then, within each wave of 64 lanes, p[l] += p[l ^ d] for
// d = 32, 16, 8, 4, 2, 1 (every lane ends with the same value); then
// (w0 + w1) + (w2 + w3) over the four waves.

__device__ __forceinline__ uint32_t add_pair(uint32_t a, uint32_t b) {
    const uint32_t lo = fni8::f2h(fni8::h2f((uint16_t)(a & 0xffffu)) + fni8::h2f((uint16_t)(b & 0xffffu)));
    const uint32_t hi = fni8::f2h(fni8::h2f((uint16_t)(a >> 16)) + fni8::h2f((uint16_t)(b >> 16)));
    return lo | (hi << 16);
}

__device__ __forceinline__ uint4 add_chunk(uint4 a, uint4 b) {
    return make_uint4(add_pair(a.x, b.x), add_pair(a.y, b.y), add_pair(a.z, b.z),
                      add_pair(a.w, b.w));
}

__device__ __forceinline__ float chunk_sumsq(uint4 v, float p) {
    const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
    for (int i = 0; i < 4; i++) {
        const float lo = fni8::h2f((uint16_t)(w4[i] & 0xffffu));
        const float hi = fni8::h2f((uint16_t)(w4[i] >> 16));
        p = p + lo * lo;
        p = p + hi * hi;
    }
    return p;
}

// The fixed cross-lane order above; returns 1 / sqrt(sum / K + eps).
__device__ __forceinline__ float block_inv_rms(float p, int K, float eps, float* red) {
    const int tid = threadIdx.x;
#pragma unroll
    for (int d = 32; d > 0; d >>= 1) p = p + __shfl_xor(p, d, 64);
    if ((tid & 63) == 0) red[tid >> 6] = p;
    __syncthreads();
    const float ss = (red[0] + red[1]) + (red[2] + red[3]);
    const float mean = ss / (float)K;
    return 1.0f / __builtin_sqrtf(mean + eps);
}

__device__ __forceinline__ uint16_t norm_one(uint16_t h, float r, uint16_t w, bool unit) {
    const float wf = unit ? 1.0f + fni8::h2f(w) : fni8::h2f(w);
    return fni8::f2h((fni8::h2f(h) * r) * wf);
}

__device__ __forceinline__ uint32_t norm_pair(uint32_t h, float r, uint32_t w, bool unit) {
    return (uint32_t)norm_one((uint16_t)(h & 0xffffu), r, (uint16_t)(w & 0xffffu), unit) |
           ((uint32_t)norm_one((uint16_t)(h >> 16), r, (uint16_t)(w >> 16), unit) << 16);
}

__device__ __forceinline__ uint4 norm_chunk(uint4 h, float r, uint4 w, bool unit) {
    return make_uint4(norm_pair(h.x, r, w.x, unit), norm_pair(h.y, r, w.y, unit),
                      norm_pair(h.z, r, w.z, unit), norm_pair(h.w, r, w.w, unit));
}

// One workgroup per row, 16-byte chunks (K % 8 == 0, aligned rows); lane tid
// holds chunks tid, tid + 256, ... of h in registers.  QUANT: write int8 + scale
// instead of the fp16 row.
template <int CH, bool RES, bool QUANT>
__global__ __launch_bounds__(kThreads) void rmsnorm_vec_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ res, int64_t ldr,
    const uint16_t* __restrict__ w, float eps, int unit, int K, uint16_t* __restrict__ out,
    int64_t ldo, uint16_t* __restrict__ res_out, int64_t ldro, int8_t* __restrict__ q,
    int64_t ldq, float* __restrict__ s) {
    __shared__ float redf[kThreads / 64];
    __shared__ uint32_t redu[kThreads / 64];
    const int m = blockIdx.x, tid = threadIdx.x;
    const uint16_t* xr = x + (int64_t)m * ldx;
    uint4 h[CH];
    float p = 0.0f;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int k = (c * kThreads + tid) * 8;
        if (k < K) {
            h[c] = *reinterpret_cast<const uint4*>(xr + k);
            if (RES) {
                h[c] = add_chunk(h[c], *reinterpret_cast<const uint4*>(res + (int64_t)m * ldr + k));
                if (res_out) *reinterpret_cast<uint4*>(res_out + (int64_t)m * ldro + k) = h[c];
            }
            p = chunk_sumsq(h[c], p);
        }
    }
    const float r = block_inv_rms(p, K, eps, redf);
    uint32_t amax = 0;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int k = (c * kThreads + tid) * 8;
        if (k < K) {
            h[c] = norm_chunk(h[c], r, *reinterpret_cast<const uint4*>(w + k), unit != 0);
            if (QUANT)
                amax = chunk_amax(h[c], amax);
            else
                *reinterpret_cast<uint4*>(out + (int64_t)m * ldo + k) = h[c];
        }
    }
    if (!QUANT) return;
    amax = block_amax(amax, redu);
    const float sc = fni8::row_scale_from_bits(amax);
    const bool live = __builtin_isfinite(sc);
    const float yr = 1.0f / sc;
    if (tid == 0) s[m] = sc;
    int8_t* qr = q + (int64_t)m * ldq;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int k = (c * kThreads + tid) * 8;
        if (k < K) *reinterpret_cast<uint2*>(qr + k) = fni8::quant_chunk(h[c], sc, yr, live);
    }
}

// Any K and alignment: the same chunk-to-lane order with scalar loads; h and
// the normed values are recomputed from the inputs in each pass (same bits).
template <bool QUANT>
__global__ __launch_bounds__(kThreads) void rmsnorm_any_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, const uint16_t* __restrict__ res, int64_t ldr,
    const uint16_t* __restrict__ w, float eps, int unit, int64_t K, uint16_t* __restrict__ out,
    int64_t ldo, uint16_t* __restrict__ res_out, int64_t ldro, int8_t* __restrict__ q,
    int64_t ldq, float* __restrict__ s) {
    __shared__ float redf[kThreads / 64];
    __shared__ uint32_t redu[kThreads / 64];
    const int64_t m = blockIdx.x;
    const uint16_t* xr = x + m * ldx;
    const uint16_t* rr = res ? res + m * ldr : nullptr;
    auto hval = [&](int64_t k) -> uint16_t {
        return rr ? fni8::f2h(fni8::h2f(xr[k]) + fni8::h2f(rr[k])) : xr[k];
    };
    float p = 0.0f;
    for (int64_t c = threadIdx.x; 8 * c < K; c += kThreads) {
        const int64_t end = 8 * c + 8 < K ? 8 * c + 8 : K;
        for (int64_t k = 8 * c; k < end; k++) {
            const uint16_t hv = hval(k);
            if (res_out) res_out[m * ldro + k] = hv;
            const float f = fni8::h2f(hv);
            p = p + f * f;
        }
    }
    const float r = block_inv_rms(p, (int)K, eps, redf);
    if (!QUANT) {
        for (int64_t k = threadIdx.x; k < K; k += kThreads)
            out[m * ldo + k] = norm_one(hval(k), r, w[k], unit != 0);
        return;
    }
    uint32_t amax = 0;
    for (int64_t k = threadIdx.x; k < K; k += kThreads) {
        const uint32_t b = norm_one(hval(k), r, w[k], unit != 0) & 0x7fffu;
        amax = b > amax ? b : amax;
    }
    amax = block_amax(amax, redu);
    const float sc = fni8::row_scale_from_bits(amax);
    if (threadIdx.x == 0) s[m] = sc;
    for (int64_t k = threadIdx.x; k < K; k += kThreads)
        q[m * ldq + k] = (int8_t)fni8::quant_one(fni8::h2f(norm_one(hval(k), r, w[k], unit != 0)), sc);
}

int launch_error(const char* what) {
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        fni8h::set_error_detail("%s launch: %s", what, hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

bool al16(const void* p) { return ((uintptr_t)p % 16) == 0; }

// Chunks per lane rounded up to the register-resident variants, 0 if too long.
int chunks_per_lane(int64_t K, int tpb = kThreads) {
    const int64_t c = (K / 8 + tpb - 1) / tpb;
    if (c <= 1) return 1;
    if (c <= 2) return 2;
    if (c <= 4) return 4;
    if (c <= 8) return 8;
    if (c <= 16) return 16;
    return 0;
}

unsigned stream_grid(int64_t work) {
    const int64_t b = (work + kThreads - 1) / kThreads;
    return (unsigned)(b < 8192 ? (b > 0 ? b : 1) : 8192);
}

template <int ACT>
int act_mul_launch(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, uint16_t* out,
                   int64_t ldo, hipStream_t st) {
    const bool vec = I % 8 == 0 && ldx % 8 == 0 && ldo % 8 == 0 && al16(x) && al16(out);
    if (vec)
        hipLaunchKernelGGL(act_mul_vec_kernel<ACT>, dim3(stream_grid(M * (I / 8))), dim3(kThreads),
                           0, st, x, ldx, M, I, out, ldo);
    else
        hipLaunchKernelGGL(act_mul_any_kernel<ACT>, dim3(stream_grid(M * I)), dim3(kThreads), 0,
                           st, x, ldx, M, I, out, ldo);
    return launch_error("act_and_mul");
}

template <int ACT, int TPB>
bool act_quant_vec_launch(int ch, const uint16_t* x, int64_t ldx, int64_t M, int64_t I,
                          int8_t* q, int64_t ldq, float* s, hipStream_t st) {
    const dim3 grid((unsigned)M), block(TPB);
#define FNI8_ACTQ(CH)                                                                  \
    hipLaunchKernelGGL((act_quant_vec_kernel<ACT, CH, TPB>), grid, block, 0, st, x, ldx, \
                       (int)I, q, ldq, s)
    switch (ch) {
        case 1: FNI8_ACTQ(1); return true;
        case 2: FNI8_ACTQ(2); return true;
        case 4: FNI8_ACTQ(4); return true;
        case 8: FNI8_ACTQ(8); return true;
        case 16: FNI8_ACTQ(16); return true;
        default: return false;
    }
#undef FNI8_ACTQ
}

// Rows per launch below which a row gets a 1024-thread workgroup.
constexpr int64_t kFewRows = 256;
// Rows per launch up to which, given a workspace, G workgroups share a row
// (G = the row's 16-byte chunks over 256 threads x kSplitChunks, 2..8).
constexpr int64_t kSplitRows = 128;
constexpr int kSplitChunks = 1;
constexpr int kSplitMaxParts = 8;

int act_quant_parts(int64_t M, int64_t I) {
    if (M < 1 || M > kSplitRows || I % 8 != 0) return 0;
    const int64_t per_wg = (int64_t)kThreads * kSplitChunks;
    const int64_t g = (I / 8 + per_wg - 1) / per_wg;
    return g >= 2 && g <= kSplitMaxParts ? (int)g : 0;
}

template <int ACT>
int act_quant_launch(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, int8_t* q,
                     int64_t ldq, float* s, uint64_t* work, int64_t work_bytes,
                     hipStream_t st) {
    const bool vec = I % 8 == 0 && ldx % 8 == 0 && ldq % 8 == 0 && al16(x) &&
                     ((uintptr_t)q % 8) == 0;
    bool done = false;
    const int G = act_quant_parts(M, I);
    if (vec && G > 0 && work != nullptr &&
        work_bytes >= fni8h::act_quant_workspace_bytes(M, I) && ((uintptr_t)work % 256) == 0) {
        const unsigned grid = (unsigned)(((M + 7) / 8) * 8 * G);
        hipLaunchKernelGGL((act_quant_split_kernel<ACT, kSplitChunks>), dim3(grid),
                           dim3(kThreads), 0, st, x, ldx, (int)M, (int)I, G, q, ldq, s, work,
                           fni8h::xcd_wait_ticks());
        done = true;
    } else if (vec && M < kFewRows)
        done = act_quant_vec_launch<ACT, 1024>(chunks_per_lane(I, 1024), x, ldx, M, I, q, ldq,
                                               s, st);
    else if (vec)
        done = act_quant_vec_launch<ACT, kThreads>(chunks_per_lane(I), x, ldx, M, I, q, ldq, s,
                                                   st);
    if (!done)
        hipLaunchKernelGGL(act_quant_any_kernel<ACT>, dim3((unsigned)M), dim3(kThreads), 0, st,
                           x, ldx, I, q, ldq, s);
    return launch_error("act_and_mul_quant");
}

template <bool QUANT>
int rmsnorm_launch(const uint16_t* x, int64_t ldx, const uint16_t* res, int64_t ldr,
                   const uint16_t* w, float eps, int unit, int64_t M, int64_t K, uint16_t* out,
                   int64_t ldo, uint16_t* res_out, int64_t ldro, int8_t* q, int64_t ldq,
                   float* s, hipStream_t st) {
    bool vec = K % 8 == 0 && ldx % 8 == 0 && al16(x) && al16(w);
    if (res) vec = vec && ldr % 8 == 0 && al16(res);
    if (res_out) vec = vec && ldro % 8 == 0 && al16(res_out);
    if (QUANT) vec = vec && ldq % 8 == 0 && ((uintptr_t)q % 8) == 0;
    else vec = vec && ldo % 8 == 0 && al16(out);
    const int ch = vec ? chunks_per_lane(K) : 0;
    const dim3 grid((unsigned)M), block(kThreads);
#define FNI8_NORM(CH, RES)                                                                     \
    hipLaunchKernelGGL((rmsnorm_vec_kernel<CH, RES, QUANT>), grid, block, 0, st, x, ldx, res, \
                       ldr, w, eps, unit, (int)K, out, ldo, res_out, ldro, q, ldq, s)
#define FNI8_NORM2(CH) \
    if (res) FNI8_NORM(CH, true); else FNI8_NORM(CH, false); break
    switch (ch) {
        case 1: FNI8_NORM2(1);
        case 2: FNI8_NORM2(2);
        case 4: FNI8_NORM2(4);
        case 8: FNI8_NORM2(8);
        case 16: FNI8_NORM2(16);
        default:
            hipLaunchKernelGGL(rmsnorm_any_kernel<QUANT>, grid, block, 0, st, x, ldx, res, ldr, w,
                               eps, unit, K, out, ldo, res_out, ldro, q, ldq, s);
    }
#undef FNI8_NORM2
#undef FNI8_NORM
    return launch_error(QUANT ? "rmsnorm_quant" : "rmsnorm");
}

}  // namespace

namespace fni8h {

int launch_act_and_mul(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, int act,
                       uint16_t* out, int64_t ldo, hipStream_t st) {
    if (M == 0) return FNI8_OK;
    return act == FNI8_ACT_SILU ? act_mul_launch<FNI8_ACT_SILU>(x, ldx, M, I, out, ldo, st)
                                : act_mul_launch<FNI8_ACT_GELU_TANH>(x, ldx, M, I, out, ldo, st);
}

int64_t act_quant_workspace_bytes(int64_t M, int64_t I) {
    const int G = act_quant_parts(M, I);
    if (G == 0) return 0;
    return (int64_t)8 * ((M + 7) / 8 * 8) * G * kSplitLine * 8;
}

int launch_act_and_mul_quant(const uint16_t* x, int64_t ldx, int64_t M, int64_t I, int act,
                             int8_t* q, int64_t ldq, float* s, int8_t* work, int64_t work_bytes,
                             hipStream_t st) {
    if (M == 0) return FNI8_OK;
    uint64_t* w = reinterpret_cast<uint64_t*>(work);
    return act == FNI8_ACT_SILU
               ? act_quant_launch<FNI8_ACT_SILU>(x, ldx, M, I, q, ldq, s, w, work_bytes, st)
               : act_quant_launch<FNI8_ACT_GELU_TANH>(x, ldx, M, I, q, ldq, s, w, work_bytes, st);
}

int launch_rmsnorm(const uint16_t* x, int64_t ldx, const uint16_t* res, int64_t ldr,
                   const uint16_t* w, float eps, int unit, int64_t M, int64_t K, uint16_t* out,
                   int64_t ldo, uint16_t* res_out, int64_t ldro, int8_t* q, int64_t ldq,
                   float* s, hipStream_t st) {
    if (M == 0) return FNI8_OK;
    if (q)
        return rmsnorm_launch<true>(x, ldx, res, ldr, w, eps, unit, M, K, nullptr, 0, res_out,
                                    ldro, q, ldq, s, st);
    return rmsnorm_launch<false>(x, ldx, res, ldr, w, eps, unit, M, K, out, ldo, res_out, ldro,
                                 nullptr, 0, nullptr, st);
}

}  // namespace fni8h
