// Per-token symmetric int8 quantization of fp16 activations (gfx950).
//
// One workgroup per row.  The row's max magnitude is an integer max over the
// fp16 magnitude bits (DPP reduction within the wave, then one LDS step across
// waves); then q = clamp(rint(x / s), -127, 127) from the same registers,
// computed without a per-element division (fni8::quant_chunk: one correctly
// rounded reciprocal per row and an exact FMA correction).
// HBM-bound: 2K bytes read + K + 4 written per row.
#include "common.h"

namespace {

constexpr int kQuantThreads = 256;

// Fast path: rows 16-byte aligned and K % 8 == 0.  Each lane loads up to CH
// 16-byte chunks (8 fp16 each) once, keeps them in registers for both the max
// and the quantize pass, and stores 8 int8 per chunk.
template <int CH>
__global__ __launch_bounds__(kQuantThreads) void quant_rowwise_regs_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int K, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ s) {
    __shared__ uint32_t red[kQuantThreads / 64];
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    const uint16_t* xr = x + (int64_t)m * ldx;
    int8_t* qr = q + (int64_t)m * ldq;

    uint4 v[CH];
    uint32_t amax = 0;
#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int k = (c * kQuantThreads + tid) * 8;
        v[c] = k < K ? *reinterpret_cast<const uint4*>(xr + k) : make_uint4(0, 0, 0, 0);
        amax = fni8::amax_chunk(amax, v[c]);
    }
    amax = fni8::wave_max_uniform(fni8::amax_fold(amax));
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < kQuantThreads / 64; i++) amax = red[i] > amax ? red[i] : amax;
    const float sc = fni8::row_scale_from_bits(amax);
    const bool live = __builtin_isfinite(sc);  // NaN/inf scale: every q is 0
    const float yr = 1.0f / sc;                // correctly rounded (build flag)
    if (tid == 0) s[m] = sc;

#pragma unroll
    for (int c = 0; c < CH; c++) {
        const int k = (c * kQuantThreads + tid) * 8;
        if (k >= K) continue;
        *reinterpret_cast<uint2*>(qr + k) = fni8::quant_chunk(v[c], sc, yr, live);
    }
}

// General path (any K % 4 == 0, any alignment): two passes, scalar elements.
__global__ __launch_bounds__(kQuantThreads) void quant_rowwise_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int K, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ s) {
    __shared__ uint32_t red[kQuantThreads / 64];
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    const uint16_t* xr = x + (int64_t)m * ldx;
    int8_t* qr = q + (int64_t)m * ldq;
    uint32_t amax = 0;
    for (int k = tid; k < K; k += kQuantThreads) {
        const uint32_t b = xr[k] & 0x7fffu;
        amax = b > amax ? b : amax;
    }
    amax = fni8::wave_max_u32(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < kQuantThreads / 64; i++) amax = red[i] > amax ? red[i] : amax;
    const float sc = fni8::row_scale_from_bits(amax);
    if (tid == 0) s[m] = sc;
    for (int k = tid; k < K; k += kQuantThreads)
        qr[k] = (int8_t)fni8::quant_one(fni8::h2f(xr[k]), sc);
}

}  // namespace

namespace fni8h {

int launch_quant_rowwise(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                         int64_t ldq, float* s, hipStream_t st) {
    if (M == 0) return FNI8_OK;
    const bool vec = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) &&
                     ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
    const int64_t chunks = (K / 8 + kQuantThreads - 1) / kQuantThreads;  // per lane
    dim3 grid((unsigned)M), block(kQuantThreads);
    if (vec && chunks <= 1)
        hipLaunchKernelGGL(quant_rowwise_regs_kernel<1>, grid, block, 0, st, x, ldx, (int)K, q, ldq, s);
    else if (vec && chunks <= 2)
        hipLaunchKernelGGL(quant_rowwise_regs_kernel<2>, grid, block, 0, st, x, ldx, (int)K, q, ldq, s);
    else if (vec && chunks <= 4)
        hipLaunchKernelGGL(quant_rowwise_regs_kernel<4>, grid, block, 0, st, x, ldx, (int)K, q, ldq, s);
    else if (vec && chunks <= 8)
        hipLaunchKernelGGL(quant_rowwise_regs_kernel<8>, grid, block, 0, st, x, ldx, (int)K, q, ldq, s);
    else
        hipLaunchKernelGGL(quant_rowwise_kernel, grid, block, 0, st, x, ldx, (int)K, q, ldq, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("quantize launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

}  // namespace fni8h
