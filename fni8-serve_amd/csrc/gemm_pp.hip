// Prefill GEMM, "ping-pong" form (gfx950, v_mfma_i32_32x32x32_i8).
//
// Workgroup: 8 waves in two groups of four (one wave of each group per SIMD).
// Group g owns rows g*BM/2.. of the BM x BN macro tile; inside it wave s owns
// BM/2 rows x BN/4 columns (tiles 256x256, 128x256, 256x128), or BM/4 x BN/2 for
// the 256x192 tile, as 32x32 blocks of int32 accumulators.  The groups take
// turns: while one group issues its MFMAs for a 64-byte K unit, the other reads
// its operand fragments for the same unit from LDS and issues the global->LDS
// copies, then they swap at a workgroup barrier.  Each SIMD thus always has one
// wave feeding the MFMA pipe and one wave doing memory work; the barriers keep
// the two groups exactly one slot apart.  (Counters on MI355X: the barriers
// themselves cost nothing measurable -- removing them from a compute-only copy
// of the loop did not change its time.)
//
// Operands reach LDS by direct global->LDS copies (global_load_lds_dwordx4: 64
// lanes x 16 bytes into 1 KB of contiguous LDS per instruction), so staging
// costs no VGPRs and no LDS write instructions.  K is consumed in 128-byte
// k-tiles through two LDS stages; the copy of k-tile t+2 is issued as soon as
// every wave has finished reading k-tile t.  The copies are not visible to the
// compiler (inline assembly), so their completion is tracked by explicit
// `s_waitcnt vmcnt` at fixed points of the schedule, followed by a barrier.
//
// LDS layout of a stage: rows of 128 bytes (A rows, then B rows), the eight
// 16-byte chunks of row r stored at chunk index c ^ ((r >> 1) & 7).  A fragment
// read (lane l: row l%32, one 16-byte chunk) then hits 16 distinct 16-byte
// slots in every group of 16 lanes (no bank conflicts), while each copy
// instruction still fetches whole 128-byte row segments from memory.  Only the
// k-order inside a k-tile changes, identically for A and B, which leaves every
// int32 dot product unchanged.
//
// The MFMAs compute D = W * X^T (weight fragment first), so each lane ends with
// four consecutive output columns per register group; the epilogue
// (tile_common.h) dequantizes in registers, stages the fp16 tile once in LDS and
// writes coalesced 16-byte row chunks.
#include <type_traits>

#include "tile_common.h"

namespace {

using fni8t::i32x16;

// one 16-byte chunk per lane, global -> LDS at M0 + lane * 16; `base` is a
// wave-uniform address, `voff` a per-lane byte offset below 2^32
__device__ __forceinline__ void copy16_s(uint32_t lds, const int8_t* base, uint32_t voff) {
    asm volatile("s_mov_b32 m0, %0\n\ts_nop 0\n\tglobal_load_lds_dwordx4 %1, %2"
                 :: "s"(lds), "v"(voff), "s"(base) : "memory", "m0");
}

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" :: "n"(N) : "memory");
}

// workgroup barrier that nothing is scheduled across
__device__ __forceinline__ void slot_barrier() {
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_barrier" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
}

// WC: waves of a group along N (4: a wave owns BM/2 rows x BN/4 columns; 2: a
// wave owns BM/4 x BN/2, for BN = 192 where BN/4 is not a multiple of 32).
template <int BM, int BN, bool WRITE_ACC, int WC = 4>
__global__ __launch_bounds__(512) void gemm_pp_kernel(
    const int8_t* __restrict__ aq, int64_t lda, const float* __restrict__ as, int M, int K,
    const int8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out) {
    constexpr int BK = 128, CPR = BK / 16;   // bytes and 16-byte chunks per row per k-tile
    constexpr int STAGE = (BM + BN) * BK;    // bytes per LDS stage (two stages)
    constexpr int D = STAGE / 8192;          // copy instructions per wave per k-tile
    constexpr int AINS = BM * CPR / 64;      // the first AINS instructions of a stage cover A
    constexpr int WR = 4 / WC;                           // waves of a group along M
    constexpr int FM = BM / (64 * WR), FN = BN / (32 * WC);
    static_assert(WC == 4 || WC == 2, "wave arrangement inside a group");
    static_assert(FM * 64 * WR == BM && FN * 32 * WC == BN, "whole 32x32 blocks per wave");
    static_assert(D * 8192 == STAGE, "a stage must split evenly over the 8 waves");
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = wave >> 2, s = wave & 3;
    const int wrow = g * (BM / 2) + (s / WC) * (FM * 32);  // first row of the wave's blocks
    const int wcol = (s % WC) * (FN * 32);                 // first column

    int m0, m1, n0;
    fni8t::dense_tile<BM, BN>(M, N, m0, m1, n0);
    const int KT = K / BK;
    // the epilogue's scales, issued before every copy: the waits for the first
    // k-tile cover them
    const fni8t::TileScales tsc =
        fni8t::load_tile_scales<BM, BN, false>(tid, m0, m1, n0, N, nullptr, as, ws, bias);

    // Copy sources.  Instruction i of wave w fills stage slots [(w*D+i)*64, +64)
    // (16-byte slots; row = slot / 8); rows past the tile's end repeat its last
    // row (their products land in rows that are never stored).
    uint32_t voff[D];
#pragma unroll
    for (int i = 0; i < D; i++) {
        const int slot = (wave * D + i) * 64 + lane;
        const int row = slot / CPR, p = slot % CPR;
        if (wave * D + i < AINS) {
            const int c = p ^ ((row >> 1) & 7);
            int mr = m0 + row;
            mr = mr < m1 ? mr : m1 - 1;
            voff[i] = (uint32_t)((int64_t)(mr - m0) * lda + c * 16);
        } else {
            const int rb = row - BM;
            const int c = p ^ ((rb >> 1) & 7);
            int nr = n0 + rb;
            nr = nr < N ? nr : N - 1;
            voff[i] = (uint32_t)((int64_t)(nr - n0) * K + c * 16);
        }
    }
    const int8_t* abase = aq + (int64_t)m0 * lda;
    const int8_t* bbase = w + (int64_t)n0 * K;
    const uint32_t lds0 = (uint32_t)(uintptr_t)smem;
    auto issue = [&](int t, int stage) {
#pragma unroll
        for (int i = 0; i < D; i++) {
            const uint32_t l = lds0 + stage * STAGE + (wave * D + i) * 1024;
            // one instruction, its base chosen by a scalar select (wave-uniform)
            const bool a_ins = wave * D + i < AINS;
            copy16_s(l, (a_ins ? abase : bbase) + t * BK, voff[i]);
        }
    };

    // fragment offsets: lane reads row (lane & 31) of a 32-row block, logical
    // chunk 2q + (lane >> 5) for the 32-byte k step q of the k-tile
    const int fr = lane & 31, fh = lane >> 5;
    const int fsw = (fr >> 1) & 7;
    int loff[4];
#pragma unroll
    for (int q = 0; q < 4; q++) loff[q] = fr * BK + (((2 * q + fh) ^ fsw) * 16);

    i32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = i32x16{};

    // prologue: k-tiles 0 and 1 in flight, wait for k-tile 0; group 1 then runs
    // one slot behind group 0
    issue(0, 0);
    if (KT > 1) {
        issue(1, 1);
        wait_vmcnt<D>();
    } else {
        wait_vmcnt<0>();
    }
    slot_barrier();
    if (g == 1) slot_barrier();

    // Slots: group 0 reads unit u while group 1 computes unit u-1, then group 0
    // computes unit u while group 1 reads it.  Two 64-byte units per k-tile.
    // Copy of k-tile t+1 is issued in the first read slot of k-tile t (its stage
    // last held k-tile t-1, read completely by then); each wave waits for its own
    // copies of k-tile t+1 before the barrier that precedes group 0's first read
    // of it (group 1 at the end of its read slot, group 0 after its MFMAs).
    for (int t0 = 0; t0 < KT; t0 += 2) {
#pragma unroll
        for (int uu = 0; uu < 4; uu++) {
            const int t = t0 + (uu >> 1);
            const int h = uu & 1;
            const int stage = uu >> 1;
            const bool live = t < KT;
            i32x4 af[2][FM], bf[2][FN];
            if (live) {
                if (h == 0 && t >= 1 && t + 1 < KT) issue(t + 1, stage ^ 1);
                const int8_t* sb = smem + stage * STAGE;
#pragma unroll
                for (int ks = 0; ks < 2; ks++) {
#pragma unroll
                    for (int i = 0; i < FM; i++)
                        af[ks][i] = *reinterpret_cast<const i32x4*>(
                            sb + (wrow + i * 32) * BK + loff[h * 2 + ks]);
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        bf[ks][j] = *reinterpret_cast<const i32x4*>(
                            sb + BM * BK + (wcol + j * 32) * BK + loff[h * 2 + ks]);
                }
                // fragments in registers before the slot ends: once every wave
                // has passed the barrier the stage may be refilled
                asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                if (g == 1 && h == 1 && t + 1 < KT) wait_vmcnt<0>();
            }
            slot_barrier();
            if (live) {
                // the MFMA wave of each SIMD issues ahead of the memory wave
                __builtin_amdgcn_s_setprio(1);
#pragma unroll
                for (int ks = 0; ks < 2; ks++)
#pragma unroll
                    for (int i = 0; i < FM; i++)
#pragma unroll
                        for (int j = 0; j < FN; j++)
                            acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[ks][j], af[ks][i],
                                                                              acc[i][j], 0, 0, 0);
                __builtin_amdgcn_s_setprio(0);
                if (g == 0 && h == 1 && t + 1 < KT) wait_vmcnt<0>();
            }
            slot_barrier();
        }
    }
    if (g == 0) slot_barrier();
    float* sl = reinterpret_cast<float*>(smem + fni8t::tile_scale_offset<BM, BN>(2 * STAGE));
    fni8t::store_tile_scales<BM, BN>(tsc, sl, tid);
    __syncthreads();  // every copy has landed and every wave is done with the stages

    fni8t::tile_epilogue<BM, BN, WRITE_ACC, FM, FN>(acc, smem, sl, tid, lane, wrow, wcol, m0, m1,
                                                    n0, N, bias != nullptr, y, ldy, acc_out);
}

template <int BM, int BN, int WC = 4>
int launch(const int8_t* aq, int64_t lda, const float* as, int M, int K, const int8_t* w,
           const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
           int32_t* acc_out, hipStream_t st) {
    constexpr size_t main_lds = (size_t)2 * (BM + BN) * 128;
    constexpr size_t lds =
        fni8t::tile_scale_offset<BM, BN>(main_lds) + fni8t::tile_scale_lds<BM, BN>();
    static_assert(lds <= 160 * 1024, "LDS budget");
    const dim3 grid(((N + BN - 1) / BN) * (unsigned)((M + BM - 1) / BM));
    // The LDS limit is a per-function attribute: each instantiation sets it once
    // (a repeated set with the same value is harmless).
    auto run = [&](auto acc_c) -> int {
        constexpr bool ACC = decltype(acc_c)::value;
        const auto kern = gemm_pp_kernel<BM, BN, ACC, WC>;
        static bool attr_set = false;
        if (!attr_set) {
            hipError_t e = hipFuncSetAttribute((const void*)kern,
                                               hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
            if (e != hipSuccess) {
                fni8h::set_error_detail("LDS attribute (%zu bytes): %s", lds, hipGetErrorString(e));
                return FNI8_ERR_LAUNCH;
            }
            attr_set = true;
        }
        hipLaunchKernelGGL(kern, grid, dim3(512), lds, st, aq, lda, as, M, K, w, ws, N, bias, y,
                           ldy, acc_out);
        return FNI8_OK;
    };
    if (acc_out) return run(std::true_type{});
    return run(std::false_type{});
}

int cu_count() {
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        return n;
    }();
    return cus;
}

}  // namespace

namespace fni8h {

// Returns 1 when the shape is not taken (the caller falls back), else an FNI8 code.
// Dense only; needs K % 128 == 0 and 16-byte aligned operand rows.  Tiles: the
// shape from {256x256, 256x192, 128x256, 256x128} with the least estimated
// time, counting whole rounds of one workgroup per CU and each tile's time
// relative to 256x256, measured on MI355X over the Qwen3-8B prefill GEMMs:
// 256x192 takes 0.79 of it for 0.75 of the products (the 2x2 wave arrangement
// reads 5 fragments per 6 MFMAs instead of 6 per 8), the half-size tiles about
// 2/3 (each of their k-tiles moves 3/4 of the bytes for 1/2 of the products).
// QKV (N = 6144) at M = 4096 is the case 256x192 exists for: 512 tiles make two
// full rounds on 256 CUs where 256x256 leaves the second round half empty
// (117 -> 103 us).  Between the two half-size tiles, long K (down, K = 12288)
// runs 256x128 4% faster and short K 128x256 3% faster.
// Expert segments stay on the 32x32x32 tile kernel: the MoE projections have
// short K (768 and 2048 bytes, 6 and 16 k-tiles), where a grouped form of this
// kernel (128x256 segment tiles) measured 18% slower at T = 4096 (473 against
// 399 us for gate_up + down) -- its pipeline and epilogue are not amortised.
int launch_pp(const int8_t* aq, int64_t lda, const float* as, int64_t M, int64_t K,
              const int8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
              int64_t ldy, int32_t* acc_out, hipStream_t st) {
    if (K % 128 != 0 || lda % 16 != 0 || ((uintptr_t)aq & 15) || ((uintptr_t)w & 15)) return 1;
    // per-lane copy offsets are 32-bit: a tile's rows span at most 256 rows
    if (256 * K >= ((int64_t)1 << 32) || 256 * lda >= ((int64_t)1 << 32)) return 1;
    const int m = (int)M, k = (int)K, n = (int)N;
    const int cus = cu_count();
    const bool longk = K >= 8192;
    // candidates in order of preference on equal estimates
    const int kTiles[4][2] = {{256, 256}, {256, 192}, {longk ? 256 : 128, longk ? 128 : 256},
                              {longk ? 128 : 256, longk ? 256 : 128}};
    constexpr double kCost[4] = {1.0, 0.79, 0.5 / 0.75, 0.5 / 0.75};  // time of one tile
    int best = 0;
    double best_t = 1e30;
    int64_t best_wgs = 0;
    for (int i = 0; i < 4; i++) {
        const int64_t wgs = ((M + kTiles[i][0] - 1) / kTiles[i][0]) * ((N + kTiles[i][1] - 1) / kTiles[i][1]);
        const double tm = (double)((wgs + cus - 1) / cus) * kCost[i];
        if (tm < best_t - 1e-9) {
            best_t = tm;
            best = i;
            best_wgs = wgs;
        }
    }
    // Too few workgroups for these tiles (prefill M = 512 except gate_up): the
    // caller's smaller-tile kernel fills the CUs better.
    if (4 * best_wgs < 3 * (int64_t)cus) return 1;
    const int bm = kTiles[best][0], bn = kTiles[best][1];
    if (bn == 192) return launch<256, 192, 2>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, st);
    if (bm == 256 && bn == 256) return launch<256, 256>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, st);
    if (bm == 128) return launch<128, 256>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, st);
    return launch<256, 128>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, st);
}

}  // namespace fni8h
