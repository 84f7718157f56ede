// Decode W8A8 linear for 5..16 tokens in one launch (gfx950): the per-token
// quantization runs once per XCD and reaches the GEMM workgroups of that XCD
// through its L2, instead of a separate quantize launch.
//
//   y[m, n] = fp16(((float)sum_k q[m, k] * w[n, k]) * s[m] * ws[n] (+ bias[n]))
//
// Why: from 5 tokens the linear was a quantize launch plus a GEMM launch, each
// paying the launch floor and a load/store round trip.  Quantizing inside
// every GEMM workgroup instead (as the 1..4-token kernels do) repeats M*K
// elements of VALU work per workgroup, which at 16 tokens costs more than the
// launch it saves.  MI355X has 8 XCDs, each with its own L2 shared by its 32
// CUs, so the rows only need quantizing once per XCD.
//
// Grid: 8*M producer workgroups, then one GEMM workgroup per 8*RB weight rows.
// Workgroup i runs on XCD i % 8 (round-robin dispatch; the kernel reads the
// real XCD from the HW_REG_XCC_ID register, so it never relies on the order),
// so producers 8r .. 8r+7 quantize token row r once on each XCD.
//   * Producer: loads its fp16 row, reduces the max magnitude (DPP + one LDS
//     step), quantizes it (division-free, exact: fni8::quant_chunk), and stores
//     the int8 row and its scale into its XCD's region of the workspace; then,
//     once every store is acknowledged by the L2, a flag word holding a tag
//     unique to this dispatch.  Producers with i % 8 == 0 also write the
//     caller's xq / xs.
//   * GEMM workgroup: issues its first weight batch, then one wave polls its
//     XCD's flags with atomics, which execute in that L2 and so see the
//     producers' stores (plain loads, even after a workgroup-scope L1
//     invalidate, kept returning a stale flag from this CU's L1 on MI355X).
//     Once every row carries this dispatch's tag it streams the int8 rows from
//     the L2 next to the weights, on MFMA (v_mfma_i32_16x16x64_i8), as
//     decode_mfma_kernel does.  No L1 line of the region can be stale: the L1
//     is invalidated at every kernel start, and in this kernel no workgroup
//     reads a region line before its flag carries this dispatch's tag.
//   * The tag is the dispatch id (the AQL packet index: strictly increasing per
//     queue, and new on every graph replay) mixed with the queue address, so a
//     flag left by an earlier call never matches: the workspace needs no
//     clearing and no reset.
//   * Every wait is bounded (s_memrealtime): a GEMM workgroup that does not see
//     its rows within the bound quantizes them itself, into the same region
//     (the bytes are identical whoever writes them), and goes on.  So the
//     kernel terminates and returns the same bits whatever the dispatch order
//     or residency; only the time changes.
// Integer accumulation is exact and the quantization deterministic, so the
// result equals the two-launch path bit for bit.
//
// Measured on MI355X (per call, 36 layers of distinct weights, against two
// launches): QKV 8.83 -> 8.08 us at 5 tokens and 9.28 -> 8.73 at 16, down
// 13.53 -> 11.97 and 14.56 -> 13.46, O 8.36 -> 7.72 at 5 tokens and even at 16.
// The producers publish 1.4-2.4 us after the first workgroup starts and the
// GEMM workgroups see it 0.5-1 us later, about what the kernel boundary cost.
// On gate_up (768 GEMM workgroups polling) and above 16 tokens it was slower,
// so the launch table takes QKV and down up to 16 tokens and O up to 8.
#include "decode_tile.h"

namespace {

using fni8dec::dispatch_tag;
using fni8dec::ld16;
using fni8dec::ld16_nt;
using fni8dec::lds_barrier;
using fni8dec::poll_flag;
using fni8dec::publish_flag;
using fni8dec::reduce_store;
using fni8dec::swz;
using fni8dec::WeightLanes;
using fni8dec::xcc_id;

// Workspace: one region per XCD -- flags [16] u64, one per 128-byte line (the
// polls of one XCD's workgroups then spread over the L2 channels instead of
// queueing on one line), scales [16] f32, then the int8 rows [M][K].
constexpr int kMaxRows = 16;
constexpr int kFlagStride = 16;  // u64 words: one flag per 128-byte line
constexpr int kFlagBytes = kMaxRows * kFlagStride * 8;  // 2048
constexpr int kHeadBytes = kFlagBytes + 256;            // flags, then 16 scales
constexpr int kXcds = 8;
constexpr int kFallbackRows = 4;  // rows a GEMM workgroup quantizes per pass on the fallback
// Bound on a GEMM workgroup's wait for the producers: 100 us of the 100 MHz
// real-time counter (producers normally publish within a few us).  A test
// hook (fni8_debug_coop_wait_ticks) can lower it to force the fallback.
constexpr int64_t kWaitTicks = 10000;
int64_t g_wait_ticks = kWaitTicks;

// Load the fp16 chunks of token rows r0 .. r0+nr-1 (thread tid: chunk tid + i*NT).
template <int WAVES, int XCH, int NR>
__device__ __forceinline__ void load_rows(uint4 (&xv)[NR][XCH], const uint16_t* __restrict__ x,
                                          int64_t ldx, int r0, int nr) {
    constexpr int NT = WAVES * 64;
#pragma unroll
    for (int j = 0; j < NR; j++) {
        if (j >= nr) break;
#pragma unroll
        for (int i = 0; i < XCH; i++)
            xv[j][i] = *reinterpret_cast<const uint4*>(x + (int64_t)(r0 + j) * ldx +
                                                       (int64_t)(threadIdx.x + i * NT) * 8);
    }
}

// Quantize token rows r0 .. r0+nr-1 (K = XCH * 8 * NT) into the region (rxq,
// rxs), and into the caller's xq / xs when `out` is set; then publish their
// flags.  Every thread of the workgroup calls it; amx is WAVES words of LDS.
template <int WAVES, int XCH, int NR>
__device__ __forceinline__ void produce_rows(const uint4 (&xv)[NR][XCH], int r0, int nr, int K,
                                             int8_t* rxq, float* rxs, uint64_t* flags, bool out,
                                             int8_t* __restrict__ xq_out,
                                             float* __restrict__ xs_out, uint64_t tag,
                                             uint32_t* amx) {
    constexpr int NT = WAVES * 64;
    const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
#pragma unroll
    for (int j = 0; j < NR; j++) {
        if (j >= nr) break;
        const int r = r0 + j;
        uint32_t m = 0;
#pragma unroll
        for (int i = 0; i < XCH; i++) m = fni8::amax_chunk(m, xv[j][i]);
        m = fni8::wave_max_uniform(fni8::amax_fold(m));
        if (lane == 0) amx[wave] = m;
        lds_barrier();
        uint32_t a = amx[0];
#pragma unroll
        for (int wv = 1; wv < WAVES; wv++) a = amx[wv] > a ? amx[wv] : a;
        lds_barrier();  // amx is reused by the next row
        const float sc = fni8::row_scale_from_bits(a);
        const bool live = __builtin_isfinite(sc);  // NaN/inf scale: every q is 0
        const float yr = 1.0f / sc;                // correctly rounded (build flag)
        if (tid == 0) {
            rxs[r] = sc;
            if (out) xs_out[r] = sc;
        }
#pragma unroll
        for (int i = 0; i < XCH; i++) {
            const int64_t k = (int64_t)(tid + i * NT) * 8;
            const uint2 q = fni8::quant_chunk(xv[j][i], sc, yr, live);
            *reinterpret_cast<uint2*>(rxq + (int64_t)r * K + k) = q;
            if (out) *reinterpret_cast<uint2*>(xq_out + (int64_t)r * K + k) = q;
        }
    }
    // every wave's stores acknowledged by the L2, then the flags.  The wait is
    // explicit: in CU mode the compiler's workgroup barrier does not wait for
    // global stores.
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    __syncthreads();
    if (tid < nr) publish_flag(flags + (r0 + tid) * kFlagStride, tag);
}

// NB: 16-row MFMA blocks; RB: 8-row load groups (the workgroup's weight rows
// are 8*RB); WAVES: K split; PER: 128-byte slabs per wave (K = 128 * PER *
// WAVES exactly); WB: slabs per batch, two batches in flight.  Only the first
// batch is issued before the wait: every weight load issued before it delays
// the producers' loads of x, which queue behind it in the memory system.
template <int NB, int RB, int WAVES, int PER, int WB>
__global__ __launch_bounds__(WAVES * 64) void decode_coop_kernel(
    const uint16_t* __restrict__ x, int64_t ldx, int M, int K, const int8_t* __restrict__ w,
    const float* __restrict__ ws, int N, const uint16_t* __restrict__ bias,
    uint16_t* __restrict__ y, int64_t ldy, int8_t* __restrict__ xq_out,
    float* __restrict__ xs_out, int32_t* __restrict__ acc_out, int8_t* __restrict__ work,
    int64_t region_bytes, uint64_t wait_ticks) {
    static_assert(PER % WB == 0 && PER % 4 == 0, "batches divide the share; whole fp16 chunks");
    constexpr int MT = 1;                  // one 16-token MFMA tile
    constexpr int XCH = PER / 4;           // 16-byte fp16 chunks of one row per thread
    constexpr int ROWS = 16 * NB;
    constexpr int TROWS = ROWS + 16 * MT;  // weight rows, then token rows
    constexpr int TILE = TROWS * 128;      // one slab of the wave's rows
    constexpr int NBT = PER / WB;          // weight batches per wave
    constexpr size_t kTiles = (size_t)WAVES * WB * TILE;
    constexpr size_t kRed = (size_t)WAVES * MT * NB * 64 * 16;
    constexpr size_t kMain = kTiles > kRed ? kTiles : kRed;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];
    uint32_t* amx = reinterpret_cast<uint32_t*>(smem + kMain);  // [WAVES]
    uint32_t* ready = amx + WAVES;                              // [1]
    i32x4* red = reinterpret_cast<i32x4*>(smem);                // after the main loop

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const uint32_t xcc = xcc_id();
    const uint64_t tag = dispatch_tag();
    int8_t* region = work + (int64_t)xcc * region_bytes;
    uint64_t* flags = reinterpret_cast<uint64_t*>(region);
    float* rxs = reinterpret_cast<float*>(region + kFlagBytes);
    int8_t* rxq = region + kHeadBytes;
    const int b = blockIdx.x;

    // ---- producers: workgroup b quantizes token row b / 8 ------------------
    if (b < kXcds * M) {
        uint4 xp[1][XCH];
        load_rows<WAVES, XCH, 1>(xp, x, ldx, b >> 3, 1);
        produce_rows<WAVES, XCH, 1>(xp, b >> 3, 1, K, rxq, rxs, flags, (b & 7) == 0, xq_out,
                                    xs_out, tag, amx);
        return;
    }

    // ---- GEMM workgroup -----------------------------------------------------
    const int n0 = (b - kXcds * M) * (8 * RB);
    const int s0 = wave * PER;
    const int rq = lane >> 3, c = lane & 7, r = lane & 15, g = lane >> 4;
    WeightLanes<NB, RB> wl;
    wl.init(w, n0, N, K, s0, lane);

    i32x4 wv[2][WB][RB];
    auto load_w = [&](i32x4 (&dw)[WB][RB], int bt) {
#pragma unroll
        for (int j = 0; j < WB; j++)
#pragma unroll
            for (int h = 0; h < RB; h++) dw[j][h] = ld16_nt(wl.src[h] + (int64_t)(bt * WB + j) * 128);
    };
    load_w(wv[0], 0);

    // wait for this XCD's rows: wave 0 polls, the other waves hold at the barrier
    if (wave == 0) {
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        bool ok = false;
        for (;;) {
            uint64_t f = tag;
            if (lane < M) f = poll_flag(flags + lane * kFlagStride);
            ok = __ballot(f != tag) == 0;
            if (ok || __builtin_amdgcn_s_memrealtime() - t0 >= wait_ticks) break;
            __builtin_amdgcn_s_sleep(4);
        }
        if (lane == 0) ready[0] = ok ? 1u : 0u;
    }
    lds_barrier();
    if (ready[0] == 0) {
        // no producer published in time: quantize every row here (same bytes)
        for (int r0 = 0; r0 < M; r0 += kFallbackRows) {
            const int nr = M - r0 < kFallbackRows ? M - r0 : kFallbackRows;
            uint4 xf[kFallbackRows][XCH];
            load_rows<WAVES, XCH, kFallbackRows>(xf, x, ldx, r0, nr);
            produce_rows<WAVES, XCH, kFallbackRows>(xf, r0, nr, K, rxq, rxs, flags, false, xq_out,
                                                    xs_out, tag, amx);
        }
    }

    // activation rows of the region: load lane -> (token h*8 + rq, chunk c);
    // tokens past M repeat token M-1 (computed, never stored)
    const int8_t* xsrc[2 * MT];
    int xwoff[2 * MT];
#pragma unroll
    for (int h = 0; h < 2 * MT; h++) {
        const int tok = h * 8 + rq;
        xsrc[h] = rxq + (int64_t)(tok < M ? tok : M - 1) * K + (int64_t)s0 * 128 + c * 16;
        xwoff[h] = (ROWS + tok) * 128 + swz(tok, c);
    }
    int aoff[MT][2];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int q = 0; q < 2; q++) aoff[mt][q] = (ROWS + mt * 16 + r) * 128 + swz(mt * 16 + r, 4 * q + g);

    i32x4 xv[2][WB][2 * MT];
    auto load_x = [&](i32x4 (&dx)[WB][2 * MT], int bt) {
#pragma unroll
        for (int j = 0; j < WB; j++)
#pragma unroll
            for (int h = 0; h < 2 * MT; h++) dx[j][h] = ld16(xsrc[h] + (int64_t)(bt * WB + j) * 128);
    };
    load_x(xv[0], 0);
    if constexpr (NBT > 1) {
        load_w(wv[1], 1);
        load_x(xv[1], 1);
    }

    i32x4 acc[2][MT][NB];
#pragma unroll
    for (int q = 0; q < 2; q++)
#pragma unroll
        for (int mt = 0; mt < MT; mt++)
#pragma unroll
            for (int nb = 0; nb < NB; nb++) acc[q][mt][nb] = i32x4{0, 0, 0, 0};

    int8_t* st = smem + wave * (WB * TILE);
    auto compute = [&](const i32x4 (&wt)[WB][RB], const i32x4 (&xt)[WB][2 * MT]) {
        // The tile is private to the wave and LDS executes a wave's accesses in
        // order; the barriers only keep the compiler from reordering across them.
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < WB; j++) {
#pragma unroll
            for (int h = 0; h < RB; h++) *reinterpret_cast<i32x4*>(st + j * TILE + wl.woff[h]) = wt[j][h];
#pragma unroll
            for (int h = 0; h < 2 * MT; h++) *reinterpret_cast<i32x4*>(st + j * TILE + xwoff[h]) = xt[j][h];
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
#pragma unroll
        for (int j = 0; j < WB; j++) {
            i32x4 bf[NB][2], af[MT][2];
#pragma unroll
            for (int nb = 0; nb < NB; nb++)
#pragma unroll
                for (int q = 0; q < 2; q++) bf[nb][q] = *reinterpret_cast<const i32x4*>(st + j * TILE + wl.roff[nb][q]);
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
#pragma unroll
                for (int q = 0; q < 2; q++) af[mt][q] = *reinterpret_cast<const i32x4*>(st + j * TILE + aoff[mt][q]);
#pragma unroll
            for (int q = 0; q < 2; q++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++)
#pragma unroll
                    for (int nb = 0; nb < NB; nb++) acc[q][mt][nb] = fni8::mfma_i8(af[mt][q], bf[nb][q], acc[q][mt][nb]);
        }
        __builtin_amdgcn_wave_barrier();
        asm volatile("" ::: "memory");
    };
#pragma unroll
    for (int bt = 0; bt < NBT; bt++) {
        compute(wv[bt & 1], xv[bt & 1]);
        if (bt + 2 < NBT) {
            load_w(wv[bt & 1], bt + 2);
            load_x(xv[bt & 1], bt + 2);
        }
    }

    __syncthreads();  // the reduction area overlaps the tiles
    reduce_store<MT, NB, WAVES, 8 * RB>(acc, red, wave, lane, tid, n0, 0, M, N, rxs, nullptr, ws,
                                        bias, y, ldy, acc_out);
}

// One launch shape per weight shape, each the fastest measured for its
// Qwen3-8B linear at 5..16 tokens (36 layers of distinct weights).
struct CoopShape {
    int nb, rb, waves, per, wb;
};

bool coop_shape(int64_t M, int64_t N, int64_t K, CoopShape* s) {
    if (M < 5 || M > kMaxRows || N >= 16384) return false;    // gate_up: two launches are faster
    if (N <= 4096 && K == 4096) {                             // O: even with two launches above 8
        if (M > 8) return false;
        *s = {1, 2, 4, 8, 2};
    }
    else if (N <= 4096 && K == 12288) *s = {1, 2, 8, 12, 4};  // down
    else if (K == 4096) *s = {2, 3, 8, 4, 2};                 // QKV: 24-row workgroups
    else return false;
    return true;
}

template <int NB, int RB, int WAVES, int PER, int WB>
int launch_coop(const uint16_t* x, int64_t ldx, int M, int K, const int8_t* w, const float* ws,
                int N, const uint16_t* bias, uint16_t* y, int64_t ldy, int8_t* xq_out,
                float* xs_out, int32_t* acc_out, int8_t* work, int64_t region_bytes,
                hipStream_t st) {
    constexpr int TILE = (16 * NB + 16) * 128;
    constexpr size_t tiles = (size_t)WAVES * WB * TILE;
    constexpr size_t red = (size_t)WAVES * NB * 64 * 16;
    constexpr size_t lds = (tiles > red ? tiles : red) + (WAVES + 1) * 4;
    static_assert(lds <= 160 * 1024, "decode LDS budget");
    auto kern = decode_coop_kernel<NB, RB, WAVES, PER, WB>;
    if constexpr (lds > 64 * 1024) {
        static const bool ok = hipFuncSetAttribute((const void*)kern,
                                                   hipFuncAttributeMaxDynamicSharedMemorySize,
                                                   (int)lds) == hipSuccess;
        if (!ok) return 1;
    }
    const unsigned nblk = (unsigned)((N + 8 * RB - 1) / (8 * RB));
    hipLaunchKernelGGL(kern, dim3(kXcds * M + nblk), dim3(WAVES * 64), lds, st, x, ldx, M, K, w,
                       ws, N, bias, y, ldy, xq_out, xs_out, acc_out, work, region_bytes,
                       fni8h::xcd_wait_ticks());
    return FNI8_OK;
}

}  // namespace

namespace fni8h {

void set_coop_wait_ticks(int64_t ticks) {
    __atomic_store_n(&g_wait_ticks, ticks < 0 ? kWaitTicks : ticks, __ATOMIC_RELAXED);
}

uint64_t xcd_wait_ticks() { return (uint64_t)__atomic_load_n(&g_wait_ticks, __ATOMIC_RELAXED); }

// Zero for shapes the one-launch path does not take, so callers allocate
// nothing for them.
int64_t coop_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    CoopShape s;
    if (!coop_shape(M, N, K, &s)) return 0;
    return (int64_t)kXcds * (kHeadBytes + ((M * K + 255) & ~(int64_t)255));
}

// fp16 activations, 5 <= M <= 16: one launch with the quantization shared per
// XCD through `work` (at least coop_workspace_bytes(M, N, K), 256-byte
// aligned, any contents).  Returns 1 when the shape is not taken.
int launch_decode_coop(const uint16_t* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                       const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
                       int64_t ldy, int8_t* xq_out, float* xs_out, int32_t* acc_out,
                       int8_t* work, int64_t work_bytes, hipStream_t st) {
    const int64_t need = coop_workspace_bytes(M, N, K);
    CoopShape s;
    if (need == 0 || !coop_shape(M, N, K, &s) || work == nullptr || work_bytes < need ||
        (uintptr_t)work % 256 != 0 || ldx % 8 != 0 || (uintptr_t)x % 16 != 0 ||
        (uintptr_t)w % 16 != 0 || xq_out == nullptr || xs_out == nullptr ||
        (uintptr_t)xq_out % 8 != 0)
        return 1;
    const int64_t region = need / kXcds;
    const int m = (int)M, k = (int)K, n = (int)N;
    int rc = 1;
    if (s.waves == 4)
        rc = launch_coop<1, 2, 4, 8, 2>(x, ldx, m, k, w, ws, n, bias, y, ldy, xq_out, xs_out,
                                        acc_out, work, region, st);
    else if (s.per == 12)
        rc = launch_coop<1, 2, 8, 12, 4>(x, ldx, m, k, w, ws, n, bias, y, ldy, xq_out, xs_out,
                                         acc_out, work, region, st);
    else
        rc = launch_coop<2, 3, 8, 4, 2>(x, ldx, m, k, w, ws, n, bias, y, ldy, xq_out, xs_out,
                                        acc_out, work, region, st);
    if (rc != FNI8_OK) return rc;
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("decode launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

}  // namespace fni8h
