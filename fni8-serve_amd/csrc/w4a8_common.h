// Device helpers shared by the W4A8 kernels (w4a8.hip, w4a8_fused.hip).
#pragma once

#include "common.h"

namespace {

// Waits for this wave's LDS traffic, then meets the other waves.  Unlike
// __syncthreads it leaves the outstanding global loads (the next round's
// weights) in flight.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// 16-byte chunk position of (row, chunk) inside a 128-byte row of a wave's
// LDS tile: eight consecutive rows, and rows eight apart, land on distinct
// positions, so full-line stores and operand reads are both conflict-free.
__device__ __forceinline__ int swz(int row, int chunk) {
    return ((chunk ^ (row & 7) ^ ((row >> 3) & 7)) & 7) * 16;
}

// 8 packed bytes (16 codes) -> 16 int8 in natural k order, each 16 * code.
// Each nibble moves to the high half of its byte, where the byte reads as
// int8 16 * code exactly (the nibble is two's complement): one shift, two
// v_perm and two masks per packed dword, no sign extension.
__device__ __forceinline__ i32x4 unpack16x16(uint32_t lo, uint32_t hi) {
    const uint32_t sl = lo << 4, sh = hi << 4;
    i32x4 r;
    r[0] = (int)(__builtin_amdgcn_perm(lo, sl, 0x05010400u) & 0xf0f0f0f0u);
    r[1] = (int)(__builtin_amdgcn_perm(lo, sl, 0x07030602u) & 0xf0f0f0f0u);
    r[2] = (int)(__builtin_amdgcn_perm(hi, sh, 0x05010400u) & 0xf0f0f0f0u);
    r[3] = (int)(__builtin_amdgcn_perm(hi, sh, 0x07030602u) & 0xf0f0f0f0u);
    return r;
}

}  // namespace
