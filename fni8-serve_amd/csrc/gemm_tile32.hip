// Prefill GEMM on v_mfma_i32_32x32x32_i8 (gfx950).
//
// On gfx950 the 32x32x32 int8 MFMA retires twice the int8 work per cycle of
// the 16x16x64 form (measured on MI355X: 4.76 vs 2.64 POPS of pure MFMA), so
// the compute-bound path uses it exclusively.
//
// Workgroup: 8 waves (2 x 4), macro tile BM x BN, each wave a (BM/2) x (BN/4)
// block of 32x32 accumulators (16 int32 per lane each).  K is consumed in BK-byte
// steps through two LDS stages (rows padded by 16 bytes: conflict-free 16-byte
// reads for the 32-row MFMA fragment pattern), with global loads staged in
// registers two steps ahead: step k+2 is fetched while step k computes.  The
// steady-state loop is branch-free (two steps per trip, tail peeled), which
// keeps every register-array index static.
//
// The MFMAs compute D = W * X^T (weight fragment first); the epilogue
// (tile_common.h) dequantizes fp16(((float)acc * as[m]) * ws[n] (+ bias[n])) in
// registers, stages the fp16 tile once in LDS and writes coalesced 16-byte row
// chunks.
#include <type_traits>

#include "tile_common.h"

namespace {

using fni8t::i32x16;
using fni8t::dense_tile;
using fni8t::tile_epilogue;

__device__ __forceinline__ i32x4 ld16(const int8_t* p) {
    return *reinterpret_cast<const i32x4*>(p);
}

// Barrier for the LDS stages: waits for this wave's LDS traffic only.  The
// compiler's __syncthreads also waits for every outstanding global load, which
// would drain the loads issued two steps ahead at every step.
__device__ __forceinline__ void lds_barrier() {
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <int BM, int BN, int BK, bool GROUPED, bool WRITE_ACC>
__global__ __launch_bounds__(512) void gemm_tile32_kernel(
    const int8_t* __restrict__ aq, int64_t lda, const float* __restrict__ as,
    const int32_t* __restrict__ row_index, int M, int K, const int8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int E, const int32_t* __restrict__ seg_off,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out) {
    constexpr int WAVES_M = 2, WAVES_N = 4, NT = 512;
    constexpr int LDSR = BK + 16;   // padded LDS row (bytes)
    constexpr int CPR = BK / 16;    // 16-byte chunks per row per step
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int FM = WTM / 32, FN = WTN / 32;
    constexpr int A_CH = BM * CPR / NT, B_CH = BN * CPR / NT;
    static_assert(A_CH * NT == BM * CPR && B_CH * NT == BN * CPR, "tile/threads mismatch");
    constexpr int BUF = (BM + BN) * LDSR;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;

    int m0, m1, n0;
    const int8_t* wexp = w;
    const float* wsexp = ws;
    const uint16_t* bexp = bias;
    if constexpr (GROUPED) {  // one work item (expert, n-tile, row tile) per workgroup
        int e, j;
        if (!fni8::find_group_item(seg_off, E, BM, (N + BN - 1) / BN, M, e, m0, m1, j)) return;
        n0 = j * BN;
        wexp += (int64_t)e * N * K;
        wsexp += (int64_t)e * N;
        if (bias) bexp += (int64_t)e * N;
    } else {
        dense_tile<BM, BN>(M, N, m0, m1, n0);
    }
    // the epilogue's scales, issued before the operand loads (the main loop's
    // waits cover them)
    const fni8t::TileScales tsc = fni8t::load_tile_scales<BM, BN, GROUPED>(
        tid, m0, m1, n0, N, row_index, as, wsexp, bexp);

    // Global sources of this thread's chunks; rows past the end are clamped to
    // the last valid row (their products land in rows that are never written).
    const int8_t* asrc[A_CH];
    const int8_t* bsrc[B_CH];
#pragma unroll
    for (int i = 0; i < A_CH; i++) {
        const int c = tid + i * NT;
        int mr = m0 + c / CPR;
        mr = mr < m1 ? mr : m1 - 1;
        int src = mr;
        if (GROUPED && row_index != nullptr) src = row_index[mr];
        asrc[i] = aq + (int64_t)src * lda + (c % CPR) * 16;
    }
#pragma unroll
    for (int i = 0; i < B_CH; i++) {
        const int c = tid + i * NT;
        int nr = n0 + c / CPR;
        nr = nr < N ? nr : N - 1;
        bsrc[i] = wexp + (int64_t)nr * K + (c % CPR) * 16;
    }

    i32x4 ra[2][A_CH], rb[2][B_CH];
    auto gload = [&](int kt, auto slot_c) {
        constexpr int slot = decltype(slot_c)::value;
        const int64_t ko = (int64_t)kt * BK;
#pragma unroll
        for (int i = 0; i < A_CH; i++) ra[slot][i] = ld16(asrc[i] + ko);
#pragma unroll
        for (int i = 0; i < B_CH; i++) rb[slot][i] = ld16(bsrc[i] + ko);
    };
    auto sstore = [&](auto buf_c, auto slot_c) {
        constexpr int buf = decltype(buf_c)::value, slot = decltype(slot_c)::value;
        int8_t* base = smem + buf * BUF;
#pragma unroll
        for (int i = 0; i < A_CH; i++) {
            const int c = tid + i * NT;
            *reinterpret_cast<i32x4*>(base + (c / CPR) * LDSR + (c % CPR) * 16) = ra[slot][i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; i++) {
            const int c = tid + i * NT;
            *reinterpret_cast<i32x4*>(base + (BM + c / CPR) * LDSR + (c % CPR) * 16) = rb[slot][i];
        }
    };

    i32x16 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = i32x16{};

    // Fragment read: lane l takes row l%32 of a 32-row block and the k-half
    // (l/32)*16 of each 32-byte k sub-step -- the 32x32x32 operand layout.
    // Only the wave's first LIVE 32-row blocks are computed: in a segment's last
    // row tile the blocks wholly past its end are skipped (their accumulators stay
    // zero and their rows are never written).
    const int fo = (lane & 31) * LDSR + (lane >> 5) * 16;
    auto compute = [&](auto buf_c, auto live_c) {
        constexpr int buf = decltype(buf_c)::value;
        constexpr int LIVE = decltype(live_c)::value;
        if constexpr (LIVE > 0) {
            const int8_t* ab = smem + buf * BUF + (wm * WTM) * LDSR + fo;
            const int8_t* bb = smem + buf * BUF + (BM + wn * WTN) * LDSR + fo;
#pragma unroll
            for (int ks = 0; ks < BK / 32; ks++) {
                i32x4 af[LIVE], bf[FN];
#pragma unroll
                for (int i = 0; i < LIVE; i++)
                    af[i] = *reinterpret_cast<const i32x4*>(ab + i * 32 * LDSR + ks * 32);
#pragma unroll
                for (int j = 0; j < FN; j++)
                    bf[j] = *reinterpret_cast<const i32x4*>(bb + j * 32 * LDSR + ks * 32);
#pragma unroll
                for (int i = 0; i < LIVE; i++)
#pragma unroll
                    for (int j = 0; j < FN; j++)
                        acc[i][j] =
                            __builtin_amdgcn_mfma_i32_32x32x32_i8(bf[j], af[i], acc[i][j], 0, 0, 0);
            }
        }
    };

    using C0 = std::integral_constant<int, 0>;
    using C1 = std::integral_constant<int, 1>;
    const int KT = K / BK;  // even and >= 2 (checked by the launcher)
    // Every variant runs the same loads, LDS stores and barriers; only the
    // MFMA work differs.
    auto mainloop = [&](auto live_c) {
        gload(0, C0{});
        gload(1, C1{});
        sstore(C0{}, C0{});
        lds_barrier();
        for (int kt = 0; kt < KT - 2; kt += 2) {
            gload(kt + 2, C0{});
            compute(C0{}, live_c);
            sstore(C1{}, C1{});
            lds_barrier();
            gload(kt + 3, C1{});
            compute(C1{}, live_c);
            sstore(C0{}, C0{});
            lds_barrier();
        }
        compute(C0{}, live_c);
        sstore(C1{}, C1{});
        lds_barrier();
        compute(C1{}, live_c);
    };
    if constexpr (GROUPED && FM <= 2) {
        // live 32-row blocks of this wave, made wave-uniform (scalar branch)
        const int left = m1 - m0 - wm * WTM;
        const int live = __builtin_amdgcn_readfirstlane(left <= 0 ? 0 : (left + 31) >> 5);
        if (live >= FM)
            mainloop(std::integral_constant<int, FM>{});
        else if (live == 1)
            mainloop(C1{});
        else
            mainloop(C0{});
    } else {
        mainloop(std::integral_constant<int, FM>{});
    }
    float* sl = reinterpret_cast<float*>(smem + fni8t::tile_scale_offset<BM, BN>(2 * BUF));
    fni8t::store_tile_scales<BM, BN>(tsc, sl, tid);
    __syncthreads();  // every wave is done with the LDS stages

    tile_epilogue<BM, BN, WRITE_ACC, FM, FN>(acc, smem, sl, tid, lane, wm * WTM, wn * WTN, m0, m1,
                                             n0, N, bexp != nullptr, y, ldy, acc_out);
}

template <int BM, int BN, int BK, bool GROUPED>
int launch(const int8_t* aq, int64_t lda, const float* as, const int32_t* row_index, int M,
           int K, const int8_t* w, const float* ws, int N, int E, const int32_t* seg_off,
           const uint16_t* bias, uint16_t* y, int64_t ldy, int32_t* acc_out, unsigned slots,
           hipStream_t st) {
    constexpr size_t main_lds = 2 * (BM + BN) * (BK + 16);
    constexpr size_t lds =
        fni8t::tile_scale_offset<BM, BN>(main_lds) + fni8t::tile_scale_lds<BM, BN>();
    static_assert(lds <= 160 * 1024, "LDS budget");
    const unsigned ntn = (unsigned)((N + BN - 1) / BN);
    // grouped: an upper bound of the work items (slots row tiles per n-tile)
    dim3 grid = GROUPED ? dim3(slots * ntn) : dim3(ntn * (unsigned)((M + BM - 1) / BM));
    // The LDS limit is a per-function attribute, so each instantiation (with and
    // without the accumulator output) is set once, by its own flag; setting it
    // again with the same value is idempotent, so a race between threads is harmless.
    auto run = [&](auto acc_c) -> int {
        constexpr bool ACC = decltype(acc_c)::value;
        const auto kern = gemm_tile32_kernel<BM, BN, BK, GROUPED, ACC>;
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
        hipLaunchKernelGGL(kern, grid, dim3(512), lds, st, aq, lda, as, row_index, M, K, w, ws, N,
                           E, seg_off, bias, y, ldy, acc_out);
        return FNI8_OK;
    };
    if (acc_out) return run(std::true_type{});
    return run(std::false_type{});
}

}  // namespace

namespace fni8h {

// Returns 1 if the shape was not taken (the caller falls back), else an FNI8 code.
int launch_tile32(const int8_t* aq, int64_t lda, const float* as, const int32_t* row_index,
                  int64_t M, int64_t K, const int8_t* w, const float* ws, int64_t N, int64_t E,
                  const int32_t* seg_off, const uint16_t* bias, uint16_t* y, int64_t ldy,
                  int32_t* acc_out, hipStream_t st) {
    // K steps of 128 (or 64) bytes, an even number of them
    const bool k128 = K % 256 == 0, k64 = !k128 && K % 128 == 0;
    if (!(k128 || k64)) return 1;
    const int m = (int)M, k = (int)K, n = (int)N, e = (int)E;
    if (E > 0) {
        // Segment tiles by average rows per expert, measured on the 128-expert
        // top-8 MoE projections at T = 32..4096: 64x128 up to 40 rows (less
        // padding in each expert's last tile), 128x128 above (6-14% faster than
        // 128x256 at T = 1024..4096: twice the n-tiles fill the CUs better).
        if (k128 && (double)M / (double)E <= 40.0)
            return launch<64, 128, 128, true>(aq, lda, as, row_index, m, k, w, ws, n, e, seg_off,
                                              bias, y, ldy, acc_out,
                                              (unsigned)((M + 63) / 64 + E), st);
        const unsigned slots = (unsigned)((M + 127) / 128 + E);
        if (k128)
            return launch<128, 128, 128, true>(aq, lda, as, row_index, m, k, w, ws, n, e, seg_off,
                                               bias, y, ldy, acc_out, slots, st);
        return launch<128, 128, 64, true>(aq, lda, as, row_index, m, k, w, ws, n, e, seg_off, bias,
                                          y, ldy, acc_out, slots, st);
    }
    // Dense: the tile whose workgroups fill the CUs best in whole rounds (one
    // workgroup per CU at a time: the LDS stages take most of the 160 KB);
    // ties go to the bigger tile, which reads fewer bytes per MFMA op.  On the
    // Qwen3-8B shapes at M = 512..4096 this picks the fastest of the six
    // measured tiles in every case.
    static const int cus = [] {
        int dev = 0, n = 0;
        if (hipGetDevice(&dev) != hipSuccess ||
            hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
            n <= 0)
            n = 256;
        return n;
    }();
    constexpr int kTiles[6][2] = {{256, 256}, {128, 256}, {256, 128}, {128, 128}, {64, 256}, {64, 128}};
    int best = 0;
    double best_fill = -1.0;
    for (int i = 0; i < 6; i++) {
        const int64_t wgs = ((M + kTiles[i][0] - 1) / kTiles[i][0]) * ((N + kTiles[i][1] - 1) / kTiles[i][1]);
        const double fill = (double)wgs / (double)(((wgs + cus - 1) / cus) * cus);
        if (fill > best_fill + 1e-9) {
            best_fill = fill;
            best = i;
        }
    }
#define FNI8_T32(BM, BN)                                                                          \
    return k128 ? launch<BM, BN, 128, false>(aq, lda, as, row_index, m, k, w, ws, n, e, seg_off,  \
                                             bias, y, ldy, acc_out, 0, st)                        \
                : launch<BM, BN, 64, false>(aq, lda, as, row_index, m, k, w, ws, n, e, seg_off,   \
                                            bias, y, ldy, acc_out, 0, st)
#define FNI8_T32_K128(BM, BN)                                                                     \
    return launch<BM, BN, 128, false>(aq, lda, as, row_index, m, k, w, ws, n, e, seg_off, bias, y,  \
                                      ldy, acc_out, 0, st)
    // 64-row tiles need 128-byte K steps (one 16-byte chunk per thread and operand)
    if (!k128 && best >= 4) best = 3;
    switch (best) {
        case 0: FNI8_T32(256, 256);
        case 1: FNI8_T32(128, 256);
        case 2: FNI8_T32(256, 128);
        case 3: FNI8_T32(128, 128);
        case 4: FNI8_T32_K128(64, 256);
        default: FNI8_T32_K128(64, 128);
    }
#undef FNI8_T32_K128
#undef FNI8_T32
}

}  // namespace fni8h
