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

#include "decode_tile.h"
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

// Split-K (SPLIT > 1): the SPLIT workgroups of one output tile each take a
// contiguous 1/SPLIT of the k-tiles.  Their ids are equal mod 8, so with the
// round-robin dispatch over the 8 XCDs they run on one XCD and hand over
// through its L2 (the exchange rules of decode_tile.h).  The workgroup of the
// last split (the highest id of the tile, dispatched last) owns the tile:
//   * every other split stores its raw int32 accumulators as a partial tile,
//     waits until the stores are acknowledged by the L2, and publishes a flag
//     holding the dispatch's tag in the flag region of the XCD it runs on;
//   * the owner polls its own XCD's flags (L2 atomics, a bounded wait), adds
//     each partial tile whose flag it sees to its accumulators, recomputes any
//     other split's k-tiles itself, and runs the epilogue.
// A flag is only seen by a workgroup on the XCD that wrote it, so a partial
// tile is only read from the L2 that holds it; where the placement differs
// from the round-robin one, or a partner runs late, the owner recomputes.  The
// output is therefore the same bits whatever the placement, and bit-identical
// to SPLIT = 1 (int32 addition is exact).  A flag left by an earlier launch
// holds another tag, so the workspace needs no clearing.
constexpr int kFlagWords = 16;  // u64 words: one flag per 128-byte line
constexpr int kXcds = 8;

// Workspace of a split plan: the flags (8 XCD regions of tiles * SPLIT lines,
// rounded up to 256 bytes), then SPLIT - 1 partial tiles of BM * BN int32 per
// tile.
__host__ __device__ inline int64_t split_flag_bytes(int64_t tiles, int split) {
    return (kXcds * tiles * split * kFlagWords * 8 + 255) & ~(int64_t)255;
}
int64_t split_work_bytes(int64_t tiles, int bm, int bn, int split) {
    if (split <= 1) return 0;
    return split_flag_bytes(tiles, split) + tiles * (split - 1) * (int64_t)bm * bn * 4;
}

// WC: waves of a group along N (4: a wave owns BM/2 rows x BN/4 columns; 2: a
// wave owns BM/4 x BN/2, for BN = 192 where BN/4 is not a multiple of 32).
template <int BM, int BN, bool WRITE_ACC, int WC = 4, int SPLIT = 1>
__global__ __launch_bounds__(512) void gemm_pp_kernel(
    const int8_t* __restrict__ aq, int64_t lda, const float* __restrict__ as, int M, int K,
    const int8_t* __restrict__ w, const float* __restrict__ ws, int N,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out, int8_t* __restrict__ work, uint64_t wait_ticks) {
    constexpr int BK = 128, CPR = BK / 16;   // bytes and 16-byte chunks per row per k-tile
    constexpr int STAGE = (BM + BN) * BK;    // bytes per LDS stage (two stages)
    constexpr int D = STAGE / 8192;          // copy instructions per wave per k-tile
    constexpr int AINS = BM * CPR / 64;      // the first AINS instructions of a stage cover A
    constexpr int WR = 4 / WC;                           // waves of a group along M
    constexpr int FM = BM / (64 * WR), FN = BN / (32 * WC);
    static_assert(WC == 4 || WC == 2, "wave arrangement inside a group");
    static_assert(FM * 64 * WR == BM && FN * 32 * WC == BN, "whole 32x32 blocks per wave");
    static_assert(D * 8192 == STAGE, "a stage must split evenly over the 8 waves");
    static_assert(SPLIT == 1 || SPLIT == 2 || SPLIT == 4, "split-K factor");
    extern __shared__ __attribute__((aligned(1024))) int8_t smem[];

    const int tid = threadIdx.x, lane = tid & 63;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int g = wave >> 2, s = wave & 3;
    const int wrow = g * (BM / 2) + (s / WC) * (FM * 32);  // first row of the wave's blocks
    const int wcol = (s % WC) * (FN * 32);                 // first column

    // workgroup b: split (b / 8) % SPLIT of tile (b / 8 / SPLIT) * 8 + b % 8
    int tile = blockIdx.x, split = 0;
    if constexpr (SPLIT > 1) {
        const int q = tile >> 3;
        split = q % SPLIT;
        tile = (q / SPLIT) * 8 + (tile & 7);
    }
    int m0, m1, n0;
    fni8t::dense_tile_at<BM, BN>(tile, M, N, m0, m1, n0);
    const int KTS = K / BK / SPLIT;  // k-tiles of one split
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

    // Accumulates k-tiles [tb, tb + nt) into acc.  Starts and ends with every
    // copy landed and every wave past its last LDS read, so it can run again.
    auto kloop = [&](int tb, int nt) {
        const int8_t* ab = abase + (int64_t)tb * BK;
        const int8_t* bb = bbase + (int64_t)tb * BK;
        auto issue = [&](int t, int stage) {
#pragma unroll
            for (int i = 0; i < D; i++) {
                const uint32_t l = lds0 + stage * STAGE + (wave * D + i) * 1024;
                // one instruction, its base chosen by a scalar select (wave-uniform)
                const bool a_ins = wave * D + i < AINS;
                copy16_s(l, (a_ins ? ab : bb) + (int64_t)t * BK, voff[i]);
            }
        };
        // prologue: k-tiles 0 and 1 in flight, wait for k-tile 0; group 1 then
        // runs one slot behind group 0
        issue(0, 0);
        if (nt > 1) {
            issue(1, 1);
            wait_vmcnt<D>();
        } else {
            wait_vmcnt<0>();
        }
        slot_barrier();
        if (g == 1) slot_barrier();

        // Slots: group 0 reads unit u while group 1 computes unit u-1, then group
        // 0 computes unit u while group 1 reads it.  Two 64-byte units per
        // k-tile.  Copy of k-tile t+1 is issued in the first read slot of k-tile
        // t (its stage last held k-tile t-1, read completely by then); each wave
        // waits for its own copies of k-tile t+1 before the barrier that precedes
        // group 0's first read of it (group 1 at the end of its read slot, group
        // 0 after its MFMAs).
        for (int t0 = 0; t0 < nt; t0 += 2) {
#pragma unroll
            for (int uu = 0; uu < 4; uu++) {
                const int t = t0 + (uu >> 1);
                const int h = uu & 1;
                const int stage = uu >> 1;
                const bool live = t < nt;
                i32x4 af[2][FM], bf[2][FN];
                if (live) {
                    if (h == 0 && t >= 1 && t + 1 < nt) issue(t + 1, stage ^ 1);
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
                    // fragments in registers before the slot ends: once every
                    // wave has passed the barrier the stage may be refilled
                    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
                    if (g == 1 && h == 1 && t + 1 < nt) wait_vmcnt<0>();
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
                                acc[i][j] = __builtin_amdgcn_mfma_i32_32x32x32_i8(
                                    bf[ks][j], af[ks][i], acc[i][j], 0, 0, 0);
                    __builtin_amdgcn_s_setprio(0);
                    if (g == 0 && h == 1 && t + 1 < nt) wait_vmcnt<0>();
                }
                slot_barrier();
            }
        }
        if (g == 0) slot_barrier();
    };

    if constexpr (SPLIT == 1) {
        kloop(0, KTS);
    } else {
        constexpr int64_t PART = (int64_t)BM * BN * 4;  // bytes of one partial tile
        static_assert(FM * FN * 4 * 512 * 16 == PART, "16 bytes per thread per register group");
        const int tiles = ((M + BM - 1) / BM) * ((N + BN - 1) / BN);
        const uint32_t xcc = fni8dec::xcc_id();
        // this XCD's flags of the tile: [SPLIT] lines
        uint64_t* flags = reinterpret_cast<uint64_t*>(work) +
                          (((int64_t)xcc * tiles + tile) * SPLIT) * kFlagWords;
        int8_t* parts = work + split_flag_bytes(tiles, SPLIT) + (int64_t)tile * (SPLIT - 1) * PART;
        const uint64_t tag = fni8dec::dispatch_tag();
        constexpr size_t main_lds = (size_t)2 * (BM + BN) * 128;
        constexpr size_t word_off =
            fni8t::tile_scale_offset<BM, BN>(main_lds) + fni8t::tile_scale_lds<BM, BN>();
        uint32_t* ready = reinterpret_cast<uint32_t*>(smem + word_off);
        // One call site of the main loop: its own split's k-tiles, and for the
        // owner, if some partner's tile does not arrive within the wait bound,
        // the whole K range once more from zero.
        int tb = split * KTS, nt = KTS;
        bool merge = false;
        for (int pass = 0;; pass++) {
            kloop(tb, nt);
            if (split != SPLIT - 1 || pass > 0) break;
            if (wave == 0) {
                bool ok = true;
                for (int sp = 0; sp < SPLIT - 1 && ok; sp++) {
                    const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
                    for (;;) {
                        uint64_t f = tag;
                        if (lane == 0) f = fni8dec::poll_flag(flags + sp * kFlagWords);
                        ok = __ballot(f != tag) == 0;
                        if (ok || __builtin_amdgcn_s_memrealtime() - t0 >= wait_ticks) break;
                        __builtin_amdgcn_s_sleep(2);
                    }
                }
                if (lane == 0) ready[0] = ok ? 1u : 0u;
            }
            __syncthreads();
            if (__builtin_amdgcn_readfirstlane(ready[0]) != 0) {
                merge = true;
                break;
            }
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++) acc[i][j] = i32x16{};
            tb = 0;
            nt = KTS * SPLIT;
        }
        if (split != SPLIT - 1) {
            // chunk c = (i*FN + j)*4 + r of every thread: 8 KB contiguous per c
            uint4* dst = reinterpret_cast<uint4*>(parts + split * PART) + tid;
#pragma unroll
            for (int i = 0; i < FM; i++)
#pragma unroll
                for (int j = 0; j < FN; j++)
#pragma unroll
                    for (int r = 0; r < 4; r++)
                        dst[((i * FN + j) * 4 + r) * 512] =
                            make_uint4((uint32_t)acc[i][j][4 * r], (uint32_t)acc[i][j][4 * r + 1],
                                       (uint32_t)acc[i][j][4 * r + 2], (uint32_t)acc[i][j][4 * r + 3]);
            asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            __syncthreads();
            if (tid == 0) fni8dec::publish_flag(flags + split * kFlagWords, tag);
            return;
        }
        if (merge) {
#pragma unroll 1
            for (int sp = 0; sp < SPLIT - 1; sp++) {
                const uint4* src = reinterpret_cast<const uint4*>(parts + sp * PART) + tid;
#pragma unroll
                for (int i = 0; i < FM; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++) {
                        uint4 v[4];
#pragma unroll
                        for (int r = 0; r < 4; r++) v[r] = src[((i * FN + j) * 4 + r) * 512];
#pragma unroll
                        for (int r = 0; r < 4; r++) {
                            acc[i][j][4 * r] = (int32_t)((uint32_t)acc[i][j][4 * r] + v[r].x);
                            acc[i][j][4 * r + 1] = (int32_t)((uint32_t)acc[i][j][4 * r + 1] + v[r].y);
                            acc[i][j][4 * r + 2] = (int32_t)((uint32_t)acc[i][j][4 * r + 2] + v[r].z);
                            acc[i][j][4 * r + 3] = (int32_t)((uint32_t)acc[i][j][4 * r + 3] + v[r].w);
                        }
                    }
            }
        }
        // test visibility: the owner's own flag line in this XCD's region records
        // whether it merged its partners' tiles (1) or recomputed the tile (0)
        if (tid == 0) flags[(SPLIT - 1) * kFlagWords] = merge ? 1ull : 0ull;
    }

    float* sl = reinterpret_cast<float*>(smem + fni8t::tile_scale_offset<BM, BN>(2 * STAGE));
    fni8t::store_tile_scales<BM, BN>(tsc, sl, tid);
    __syncthreads();  // every copy has landed and every wave is done with the stages

    fni8t::tile_epilogue<BM, BN, WRITE_ACC, FM, FN>(acc, smem, sl, tid, lane, wrow, wcol, m0, m1,
                                                    n0, N, bias != nullptr, y, ldy, acc_out);
}

template <int BM, int BN, int WC = 4, int SPLIT = 1>
int launch(const int8_t* aq, int64_t lda, const float* as, int M, int K, const int8_t* w,
           const float* ws, int N, const uint16_t* bias, uint16_t* y, int64_t ldy,
           int32_t* acc_out, int8_t* work, hipStream_t st) {
    constexpr size_t main_lds = (size_t)2 * (BM + BN) * 128;
    constexpr size_t lds = fni8t::tile_scale_offset<BM, BN>(main_lds) +
                           fni8t::tile_scale_lds<BM, BN>() + (SPLIT > 1 ? 16 : 0);
    static_assert(lds <= 160 * 1024, "LDS budget");
    const dim3 grid(((N + BN - 1) / BN) * (unsigned)((M + BM - 1) / BM) * SPLIT);
    const uint64_t wait_ticks = SPLIT > 1 ? fni8h::xcd_wait_ticks() : 0;
    // The LDS limit is a per-function attribute: each instantiation sets it once
    // (a repeated set with the same value is harmless).
    auto run = [&](auto acc_c) -> int {
        constexpr bool ACC = decltype(acc_c)::value;
        const auto kern = gemm_pp_kernel<BM, BN, ACC, WC, SPLIT>;
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
                           ldy, acc_out, work, wait_ticks);
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

// ---- tile and split-K choice ---------------------------------------------------
// Tiles: {256x256, 256x192, 128x256, 256x128}, and 64x128 for long K at
// M <= 256 (below); each tile's time per k-tile
// relative to 256x256, measured on MI355X over the Qwen3-8B prefill GEMMs:
// 256x192 takes 0.79 of it for 0.75 of the products (the 2x2 wave arrangement
// reads 5 fragments per 6 MFMAs instead of 6 per 8), the half-size tiles about
// 2/3 (each of their k-tiles moves 3/4 of the bytes for 1/2 of the products).
// QKV (N = 6144) at M = 4096 is the case 256x192 exists for: 512 tiles make two
// full rounds on 256 CUs where 256x256 leaves the second round half empty
// (117 -> 103 us).  Between the two half-size tiles, long K (down, K = 12288)
// runs 256x128 4% faster and short K 128x256 3% faster.
//
// Split-K (2 or 4) is considered when a workspace is given and the tiles fill
// less than one round of the CUs: it multiplies the workgroups and divides the
// k-tiles per workgroup; the hand-over of each partial tile is charged by its
// size.  Expert segments stay on the 32x32x32 tile kernel: the MoE projections
// have short K (768 and 2048 bytes, 6 and 16 k-tiles), where a grouped form of
// this kernel (128x256 segment tiles) measured 18% slower at T = 4096 (473
// against 399 us for gate_up + down) -- its pipeline and epilogue are not
// amortised.
struct PpPlan {
    int bm, bn, split;
    int64_t work;  // workspace bytes
};

constexpr double kPartCost = 1.0;     // per 256x256 partial tile merged, in 256x256 k-tiles
constexpr double kHandoffCost = 1.0;  // counter and last store latency, same unit
// k-tiles per split at least: with 16 (K = 4096 split in 2) every split plan
// measured slower than the best unsplit one on Qwen3-8B's shapes at M = 256..2048
constexpr int kMinSplitKt = 24;

int g_force_bm = 0, g_force_bn = 0, g_force_split = 0;

bool plan_valid(int64_t M, int64_t N, int64_t K, int bm, int bn, int split, int64_t work_bytes,
                int64_t& need) {
    const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
    const int64_t kt = K / 128;
    need = split_work_bytes(tiles, bm, bn, split);
    if (split == 1) return true;
    return kt % split == 0 && tiles % 8 == 0 && need <= work_bytes;
}

// False when the shape is not taken by this kernel.
bool pp_plan(int64_t M, int64_t N, int64_t K, int64_t work_bytes, PpPlan& out) {
    const int cus = cu_count();
    const int fbm = __atomic_load_n(&g_force_bm, __ATOMIC_RELAXED);
    const int fbn = __atomic_load_n(&g_force_bn, __ATOMIC_RELAXED);
    const int fsp = __atomic_load_n(&g_force_split, __ATOMIC_RELAXED);
    int64_t need = 0;
    if (fbm > 0 && plan_valid(M, N, K, fbm, fbn, fsp, work_bytes, need)) {
        out = PpPlan{fbm, fbn, fsp, need};
        return true;
    }
    // Long K on a single row of 256-row tiles (down at M <= 256): 64x128 tiles
    // split 4, three workgroups per CU (LDS 50 KB each).  Measured at M = 256:
    // 32.7 us against 41.3 for 256x128 split 4 and 55 on the tile kernel.
    if (K >= 8192 && M <= 256 && plan_valid(M, N, K, 64, 128, 4, work_bytes, need) &&
        (K / 128) / 4 >= kMinSplitKt) {
        out = PpPlan{64, 128, 4, need};
        return true;
    }
    // candidates in order of preference on equal estimates; of the half-size
    // tiles 256x128 first for long K and for a single row of tiles (M <= 256,
    // where it reads each weight row once: gate_up at M = 256 45 against 50 us)
    const bool wide_first = K >= 8192 || M <= 256;
    const int kTiles[4][2] = {{256, 256}, {256, 192}, {wide_first ? 256 : 128, wide_first ? 128 : 256},
                              {wide_first ? 128 : 256, wide_first ? 256 : 128}};
    constexpr double kCost[4] = {1.0, 0.79, 0.5 / 0.75, 0.5 / 0.75};  // per k-tile
    constexpr int kSplits[3] = {1, 2, 4};
    const int64_t kt = K / 128;
    double best_t = 1e30;
    int64_t best_wgs = 0;
    int best_split = 1;
    for (int sidx = 0; sidx < 3; sidx++) {
        const int split = kSplits[sidx];
        for (int i = 0; i < 4; i++) {
            const int bm = kTiles[i][0], bn = kTiles[i][1];
            if (split > 1 && bn == 192) continue;
            if (!plan_valid(M, N, K, bm, bn, split, work_bytes, need)) continue;
            const int64_t tiles = ((M + bm - 1) / bm) * ((N + bn - 1) / bn);
            const int64_t wgs = tiles * split;
            if (split > 1 && (wgs > cus || kt / split < kMinSplitKt)) continue;
            double tm = (double)((wgs + cus - 1) / cus) * kCost[i] * (double)(kt / split);
            if (split > 1)
                tm += (split - 1) * kPartCost * (double)(bm * bn) / 65536.0 + kHandoffCost;
            if (tm < best_t - 1e-9) {
                best_t = tm;
                best_wgs = wgs;
                best_split = split;
                out = PpPlan{bm, bn, split, need};
            }
        }
    }
    // Too few workgroups for unsplit tiles (prefill M = 512 except gate_up):
    // the caller's smaller-tile kernel fills the CUs better.  Split plans exist
    // for exactly those shapes and measured faster than it (down at M = 256:
    // 41 us on 128 workgroups of 256x128 split 4, against 55).
    return best_split > 1 || 4 * best_wgs >= 3 * (int64_t)cus;
}

}  // namespace

namespace fni8h {

void set_gemm_plan(int64_t bm, int64_t bn, int64_t split) {
    const bool ok = (bm == 256 && (bn == 256 || bn == 192 || bn == 128)) ||
                    (bm == 128 && bn == 256) || (bm == 64 && bn == 128);
    const bool sp = split == 1 || ((split == 2 || split == 4) && bn != 192);
    const bool on = ok && sp;
    __atomic_store_n(&g_force_split, on ? (int)split : 0, __ATOMIC_RELAXED);
    __atomic_store_n(&g_force_bn, on ? (int)bn : 0, __ATOMIC_RELAXED);
    __atomic_store_n(&g_force_bm, on ? (int)bm : 0, __ATOMIC_RELAXED);
}

bool pp_shape_ok(const int8_t* aq, int64_t lda, int64_t K, const int8_t* w) {
    if (K % 128 != 0 || lda % 16 != 0 || ((uintptr_t)aq & 15) || ((uintptr_t)w & 15)) return false;
    // per-lane copy offsets are 32-bit: a tile's rows span at most 256 rows
    return 256 * K < ((int64_t)1 << 32) && 256 * lda < ((int64_t)1 << 32);
}

int64_t pp_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M <= 64 || K % 128 != 0 || 256 * K >= ((int64_t)1 << 32)) return 0;
    PpPlan p;
    if (!pp_plan(M, N, K, INT64_MAX, p)) return 0;
    return p.work;
}

// Returns 1 when the shape is not taken (the caller falls back), else an FNI8 code.
// Dense only; needs K % 128 == 0 and 16-byte aligned operand rows.
int launch_pp(const int8_t* aq, int64_t lda, const float* as, int64_t M, int64_t K,
              const int8_t* w, const float* ws, int64_t N, const uint16_t* bias, uint16_t* y,
              int64_t ldy, int32_t* acc_out, int8_t* work, int64_t work_bytes, hipStream_t st) {
    if (!pp_shape_ok(aq, lda, K, w)) return 1;
    PpPlan p;
    if (!pp_plan(M, N, K, work != nullptr ? work_bytes : 0, p)) return 1;
    const int m = (int)M, k = (int)K, n = (int)N;
    const int bm = p.bm, bn = p.bn;
    if (bm == 64) {  // three workgroups per CU
        if (p.split == 4) return launch<64, 128, 4, 4>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
        if (p.split == 2) return launch<64, 128, 4, 2>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
        return launch<64, 128>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, nullptr, st);
    }
    if (p.split == 4) {
        if (bm == 256 && bn == 256) return launch<256, 256, 4, 4>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
        if (bm == 128) return launch<128, 256, 4, 4>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
        return launch<256, 128, 4, 4>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
    }
    if (p.split == 2) {
        if (bm == 256 && bn == 256) return launch<256, 256, 4, 2>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
        if (bm == 128) return launch<128, 256, 4, 2>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
        return launch<256, 128, 4, 2>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, work, st);
    }
    if (bn == 192) return launch<256, 192, 2>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, nullptr, st);
    if (bm == 256 && bn == 256) return launch<256, 256>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, nullptr, st);
    if (bm == 128) return launch<128, 256>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, nullptr, st);
    return launch<256, 128>(aq, lda, as, m, k, w, ws, n, bias, y, ldy, acc_out, nullptr, st);
}

}  // namespace fni8h
