// Per-token symmetric int8 quantization of fp16 activations (gfx950).
//
// One workgroup per row.  Pass 1 takes the row's max magnitude as an integer
// max over the fp16 magnitude bits (wave64 xor-shuffle reduction, then one LDS
// step across waves); pass 2 re-reads the row (an L2 hit) and writes
// q = clamp(rint(x / s), -127, 127).  HBM-bound: 2K bytes read + K + 4 written
// per row.
#include "common.h"

namespace {

constexpr int kQuantThreads = 256;

// VEC: rows are 16-byte aligned and K % 8 == 0, so each lane moves 8 fp16
// (one 16-byte load) and stores 8 int8 (one 8-byte store).
template <bool VEC>
__global__ __launch_bounds__(kQuantThreads) void quant_rowwise_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int K, int8_t* __restrict__ q, int64_t ldq,
    float* __restrict__ s) {
    __shared__ uint32_t red[kQuantThreads / 64];
    const int m = blockIdx.x;
    const int tid = threadIdx.x;
    const uint16_t* xr = x + (int64_t)m * ldx;
    int8_t* qr = q + (int64_t)m * ldq;

    uint32_t amax = 0;
    if constexpr (VEC) {
        for (int k = tid * 8; k < K; k += kQuantThreads * 8) {
            uint4 v = *reinterpret_cast<const uint4*>(xr + k);
            uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                uint32_t lo = w4[i] & 0x7fffu, hi = (w4[i] >> 16) & 0x7fffu;
                amax = lo > amax ? lo : amax;
                amax = hi > amax ? hi : amax;
            }
        }
    } else {
        for (int k = tid; k < K; k += kQuantThreads) {
            uint32_t b = xr[k] & 0x7fffu;
            amax = b > amax ? b : amax;
        }
    }
    amax = fni8::wave_max_u32(amax);
    if ((tid & 63) == 0) red[tid >> 6] = amax;
    __syncthreads();
    amax = red[0];
#pragma unroll
    for (int i = 1; i < kQuantThreads / 64; i++) amax = red[i] > amax ? red[i] : amax;
    const float sc = fni8::row_scale_from_bits(amax);
    if (tid == 0) s[m] = sc;

    if constexpr (VEC) {
        for (int k = tid * 8; k < K; k += kQuantThreads * 8) {
            uint4 v = *reinterpret_cast<const uint4*>(xr + k);
            uint32_t w4[4] = {v.x, v.y, v.z, v.w};
            uint32_t packed[2] = {0, 0};
#pragma unroll
            for (int i = 0; i < 4; i++) {
                int32_t q0 = fni8::quant_one(fni8::h2f((uint16_t)(w4[i] & 0xffffu)), sc);
                int32_t q1 = fni8::quant_one(fni8::h2f((uint16_t)(w4[i] >> 16)), sc);
                uint32_t pair = ((uint32_t)q0 & 0xffu) | (((uint32_t)q1 & 0xffu) << 8);
                packed[i >> 1] |= pair << ((i & 1) * 16);
            }
            *reinterpret_cast<uint2*>(qr + k) = make_uint2(packed[0], packed[1]);
        }
    } else {
        for (int k = tid; k < K; k += kQuantThreads)
            qr[k] = (int8_t)fni8::quant_one(fni8::h2f(xr[k]), sc);
    }
}

}  // namespace

namespace fni8h {

int launch_quant_rowwise(const uint16_t* x, int64_t M, int64_t K, int64_t ldx, int8_t* q,
                         int64_t ldq, float* s, hipStream_t st) {
    if (M == 0) return FNI8_OK;
    const bool vec = (K % 8 == 0) && (ldx % 8 == 0) && (ldq % 8 == 0) &&
                     ((uintptr_t)x % 16 == 0) && ((uintptr_t)q % 8 == 0);
    dim3 grid((unsigned)M), block(kQuantThreads);
    if (vec)
        hipLaunchKernelGGL(quant_rowwise_kernel<true>, grid, block, 0, st, x, ldx, (int)K, q, ldq, s);
    else
        hipLaunchKernelGGL(quant_rowwise_kernel<false>, grid, block, 0, st, x, ldx, (int)K, q, ldq, s);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("quantize launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

}  // namespace fni8h
