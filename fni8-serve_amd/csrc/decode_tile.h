// Pieces shared by the MFMA decode kernels (gfx950): the coalesced weight-lane
// layout, the wave-private LDS tile swizzle, and the cross-wave reduction with
// the fp16 epilogue.
//
// Weights stream 8 rows x 128 contiguous bytes per wave load instruction (lane
// l: row l/8, bytes 16*(l%8) of a 128-byte slab), so every row contributes a
// full cache line per instruction.  That is not the operand layout of
// v_mfma_i32_16x16x64_i8 (lane l: row l%16, bytes 16*(l/16) of a 64-byte
// half-slab), so each slab passes through a wave-private LDS tile whose
// 16-byte chunks are XOR-swizzled by row: conflict-free on the way in and out.
#pragma once

#include "common.h"

extern "C" __device__ uint64_t fni8_llvm_dispatch_id() __asm("llvm.amdgcn.dispatch.id");

namespace fni8dec {

// ---- exchange between the workgroups of one XCD -------------------------------
// The 8 XCDs of MI355X each have their own L2, shared by that XCD's CUs, and
// not kept coherent with the other XCDs' L2s inside a kernel.  Workgroups of
// one XCD can therefore hand data to each other through their L2: the writer
// stores the data, waits until every store is acknowledged by the L2, then
// stores a flag; the reader polls the flag with an atomic (atomics execute in
// the L2; a plain load, even after a workgroup-scope L1 invalidate, kept
// returning a stale flag from the reader's L1) and then loads the data, which
// no workgroup of the kernel read before the flag was set, so no L1 holds a
// stale copy (the L1 is invalidated at every kernel start).  Both sides check
// the XCD they run on with xcc_id(); a flag holds dispatch_tag(), so a flag left
// by an earlier launch never matches and the memory needs no reset.

// Index (0..7) of the XCD this wave runs on.
__device__ __forceinline__ uint32_t xcc_id() {
    uint32_t v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    return v & 7u;
}

// A value no earlier dispatch produced: the dispatch id (the AQL packet index,
// strictly increasing per queue and new on every graph replay) mixed with the
// queue's address.
__device__ __forceinline__ uint64_t dispatch_tag() {
    const uint64_t q = (uint64_t)__builtin_amdgcn_queue_ptr();
    return fni8_llvm_dispatch_id() ^ (q * 0x9E3779B97F4A7C15ull);
}

// Atomic read of a flag word, executed in the L2 of this XCD.  Waits for every
// vector memory operation of the wave.
__device__ __forceinline__ uint64_t poll_flag(const uint64_t* p) {
    uint64_t v;
    const uint64_t zero = 0;
    asm volatile("global_atomic_or_x2 %0, %1, %2, off sc0\n\ts_waitcnt vmcnt(0)"
                 : "=v"(v) : "v"(p), "v"(zero) : "memory");
    return v;
}

// Store a flag once this wave's earlier global stores are acknowledged by the
// L2 (the caller makes the other waves' stores complete first, e.g. with
// s_waitcnt vmcnt(0) in every wave and a barrier).
__device__ __forceinline__ void publish_flag(uint64_t* p, uint64_t tag) {
    __hip_atomic_store(p, tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}

__device__ __forceinline__ i32x4 ld16(const void* p) {
    return *reinterpret_cast<const i32x4*>(p);
}
__device__ __forceinline__ i32x4 ld16_nt(const int8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
}

// 16-byte chunk position of (row, chunk) inside a 128-byte row of an LDS tile:
// rows r and r' with r = r' mod 4 get different chunk positions, so the 16
// lanes of one ds_read_b128 pass (16 rows, one chunk) hit 16 distinct slots.
__device__ __forceinline__ int swz(int row, int chunk) {
    return ((chunk ^ (row & 7) ^ ((row >> 3) & 7)) & 7) * 16;
}

// Barrier that waits for LDS traffic only: the compiler's __syncthreads also
// waits for every outstanding global load, which would drain the weight
// prefetch.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Weight side of one wave: pointers and LDS offsets for the RB load
// instructions of a slab, and the B-fragment offsets for the MFMA.
// RB = 8-row load groups of the workgroup (at most 2 * NB): a workgroup may own
// fewer rows than its NB MFMA blocks span, so that the workgroup count fits the
// CUs (6144 rows in 24-row workgroups are 256 of them); the MFMA reads the
// unloaded rows of the tile as whatever they hold, and those columns are never
// stored.
template <int NB, int RB = 2 * NB>
struct WeightLanes {
    static_assert(RB >= 1 && RB <= 2 * NB, "load groups within the MFMA blocks");
    const int8_t* src[RB];
    int woff[RB];
    int roff[NB][2];
    __device__ __forceinline__ void init(const int8_t* w, int n0, int N, int64_t K, int s0,
                                         int lane) {
        const int rq = lane >> 3, c = lane & 7, r = lane & 15, g = lane >> 4;
#pragma unroll
        for (int h = 0; h < RB; h++) {
            const int row = h * 8 + rq;
            int n = n0 + row;
            n = n < N ? n : N - 1;  // rows past N load real memory, never stored
            src[h] = w + (int64_t)n * K + (int64_t)s0 * 128 + c * 16;
            woff[h] = row * 128 + swz(row, c);
        }
#pragma unroll
        for (int b = 0; b < NB; b++)
#pragma unroll
            for (int q = 0; q < 2; q++) roff[b][q] = (b * 16 + r) * 128 + swz(b * 16 + r, 4 * q + g);
    }
};

// Cross-wave reduction and epilogue.  acc[q][mt][b]: lane l, register i holds
// token mt*16 + 4*(l/16) + i, row b*16 + l%16.  Token m of the tile is output
// row r0 + m; its activation scale is xs[rmap[r0 + m]] (xs[r0 + m] without a
// row map).  `red` needs WAVES * MT * NB * 1 KB of LDS.
template <int MT, int NB, int WAVES, int WROWS = 16 * NB>
__device__ __forceinline__ void reduce_store(i32x4 (&acc)[2][MT][NB], i32x4* red, int wave,
                                             int lane, int tid, int n0, int r0, int M, int N,
                                             const float* xs, const int32_t* __restrict__ rmap,
                                             const float* __restrict__ ws,
                                             const uint16_t* __restrict__ bias,
                                             uint16_t* __restrict__ y, int64_t ldy,
                                             int32_t* __restrict__ acc_out) {
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int b = 0; b < NB; b++)
            red[(wave * MT * NB + mt * NB + b) * 64 + lane] = acc[0][mt][b] + acc[1][mt][b];
    __syncthreads();
    for (int idx = tid; idx < MT * NB * 64; idx += WAVES * 64) {
        const int mb = idx >> 6, ln = idx & 63, mt = mb / NB, b = mb % NB;
        i32x4 s = red[mb * 64 + ln];
#pragma unroll
        for (int wv = 1; wv < WAVES; wv++) s += red[(wv * MT * NB + mb) * 64 + ln];
        const int col = n0 + b * 16 + (ln & 15);
        if (b * 16 + (ln & 15) >= WROWS || col >= N) continue;
        const float wsc = ws[col];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int m = mt * 16 + (ln >> 4) * 4 + i;
            if (m >= M) continue;
            const int row = r0 + m;
            const float xsc = xs[rmap != nullptr ? rmap[row] : row];
            y[(int64_t)row * ldy + col] = fni8::dequant_one(s[i], xsc, wsc, bias, col);
            if (acc_out != nullptr) acc_out[(int64_t)row * N + col] = s[i];
        }
    }
}

}  // namespace fni8dec
