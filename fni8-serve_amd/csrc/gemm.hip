// int8 x int8 -> int32 GEMM with the fused dequant epilogue (gfx950).
//
//   y[m, n] = fp16(((float)sum_k a[m, k] * w[n, k]) * as[m] * ws[n] (+ bias[n]))
//
// Both operands are K-contiguous (the per_row_i8 weight is [N, K] row-major),
// which is exactly the per-lane layout of v_mfma_i32_16x16x64_i8: every lane
// feeds 16 consecutive int8 of one row of A and of one row of B, so neither
// operand needs a transpose anywhere.
//
// Three kernels, each with a dense and a grouped (expert segment) form:
//   skinny  M <= 64 (decode) and small expert segments.  HBM-bound weight
//           streaming: a workgroup owns 16 weight rows, its waves split K,
//           every lane streams 16-byte loads of W straight into MFMA operands
//           (no LDS staging: each weight byte is used once), partial sums are
//           reduced across waves through LDS, then the epilogue.
//   tile    M > 64 (prefill) and large expert segments.  MFMA-bound: a
//           BM x BN macro tile per workgroup, A/B K-slices of 64 bytes staged
//           through double-buffered LDS (80-byte padded rows: conflict-free
//           16-byte reads), one barrier per K step, global loads of step k+1
//           in flight during the MFMAs of step k.  Workgroup ids are remapped
//           so each XCD (own L2) walks a contiguous band of tiles.
//   generic any K % 4 == 0 or unaligned operands: one output per lane with
//           v_dot4_i32_i8.  Correct, not fast.
// Integer accumulation is exact, so every kernel (and any split of K) gives
// bit-identical accumulators.
#include "common.h"

namespace {

using fni8::mfma_i8;

__device__ __forceinline__ i32x4 ld16(const int8_t* p) {
    return *reinterpret_cast<const i32x4*>(p);
}

// Streaming load: non-temporal hint, for data read exactly once.
__device__ __forceinline__ i32x4 ld16_stream(const int8_t* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const i32x4*>(p));
}

// ---------------------------------------------------------------------------
// skinny kernel
// ---------------------------------------------------------------------------
// MT: 16-row blocks of activations (M <= 16 * MT); NB: 16-row blocks of weight
// rows per workgroup (every wave streams all NB blocks over its K share, so
// each activation fragment feeds NB MFMAs); WAVES: waves splitting K;
// U: 64-byte K units per loop trip (U * NB 16-byte weight loads in flight per
// lane).  Weight loads are non-temporal: each byte is used once, so they are
// kept from displacing the activations in L2.
template <int MT, int NB, int WAVES, int U, bool GROUPED>
__global__ __launch_bounds__(WAVES * 64) void gemm_skinny_kernel(
    const int8_t* __restrict__ aq, int64_t lda, const float* __restrict__ as,
    const int32_t* __restrict__ row_index, int M, int K, const int8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int E, const int32_t* __restrict__ seg_off,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out) {
    constexpr int BM = 16 * MT;
    constexpr int BN = 16 * NB;
    __shared__ i32x4 red[WAVES][MT * NB][64];

    const int lane = threadIdx.x & 63;
    const int wave = threadIdx.x >> 6;
    // dense: x = n-tile, y = m-tile; grouped: x = segment tile slot, y = n-tile
    const int nt = GROUPED ? blockIdx.y : blockIdx.x;

    int m0, m1;
    const int8_t* wexp = w;
    const float* wsexp = ws;
    const uint16_t* bexp = bias;
    if constexpr (GROUPED) {
        int e;
        if (!fni8::find_group_tile(seg_off, E, BM, blockIdx.x, M, e, m0, m1)) return;
        wexp += (int64_t)e * N * K;
        wsexp += (int64_t)e * N;
        if (bias) bexp += (int64_t)e * N;
    } else {
        m0 = blockIdx.y * BM;
        m1 = min(M, m0 + BM);
    }

    const int r = lane & 15, g = lane >> 4;
    const int8_t* wrow[NB];
    bool nvalid[NB];
    float wsc[NB];
#pragma unroll
    for (int b = 0; b < NB; b++) {
        const int n = nt * BN + b * 16 + r;
        nvalid[b] = n < N;
        wrow[b] = wexp + (int64_t)(nvalid[b] ? n : 0) * K + g * 16;
        wsc[b] = nvalid[b] ? wsexp[n] : 0.f;  // epilogue scale, fetched early
    }
    const int8_t* arow[MT];
    bool avalid[MT];
#pragma unroll
    for (int mt = 0; mt < MT; mt++) {
        const int mr = m0 + mt * 16 + r;
        avalid[mt] = mr < m1;
        int src = mr;
        if (GROUPED && row_index != nullptr && avalid[mt]) src = row_index[mr];
        arow[mt] = aq + (int64_t)(avalid[mt] ? src : 0) * lda + g * 16;
    }

    const int units = K >> 6;
    const int per = (units + WAVES - 1) / WAVES;
    const int u0 = wave * per;
    const int u1 = min(units, u0 + per);

    i32x4 acc[MT][NB];
#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int b = 0; b < NB; b++) acc[mt][b] = i32x4{0, 0, 0, 0};

    for (int u = u0; u < u1; u += U) {
        i32x4 bw[NB][U];
        i32x4 ax[MT][U];
#pragma unroll
        for (int j = 0; j < U; j++) {
            const bool ok = (u + j) < u1;
#pragma unroll
            for (int b = 0; b < NB; b++)
                bw[b][j] = (ok && nvalid[b]) ? ld16_stream(wrow[b] + (int64_t)(u + j) * 64)
                                             : i32x4{0, 0, 0, 0};
#pragma unroll
            for (int mt = 0; mt < MT; mt++)
                ax[mt][j] = (ok && avalid[mt]) ? ld16(arow[mt] + (int64_t)(u + j) * 64)
                                               : i32x4{0, 0, 0, 0};
        }
#pragma unroll
        for (int j = 0; j < U; j++)
#pragma unroll
            for (int b = 0; b < NB; b++)
#pragma unroll
                for (int mt = 0; mt < MT; mt++) acc[mt][b] = mfma_i8(ax[mt][j], bw[b][j], acc[mt][b]);
    }

#pragma unroll
    for (int mt = 0; mt < MT; mt++)
#pragma unroll
        for (int b = 0; b < NB; b++) red[wave][mt * NB + b][lane] = acc[mt][b];
    __syncthreads();

    // Each (m-block, n-block) result is summed over the waves by one wave-sized
    // group of threads; a thread keeps the lane layout of the MFMA result.
    for (int idx = threadIdx.x; idx < MT * NB * 64; idx += WAVES * 64) {
        const int mb = idx >> 6, ln = idx & 63;
        const int mt = mb / NB, b = mb % NB;
        i32x4 s = red[0][mb][ln];
#pragma unroll
        for (int wv = 1; wv < WAVES; wv++) s += red[wv][mb][ln];
        const int col = nt * BN + b * 16 + (ln & 15);
        if (col >= N) continue;
        // ln == lane (the stride is a whole number of waves), so wsc[b] is this
        // column's scale.
        const float wscale = wsc[b];
#pragma unroll
        for (int i = 0; i < 4; i++) {
            const int mr = m0 + mt * 16 + (ln >> 4) * 4 + i;
            if (mr >= m1) continue;
            int src = mr;
            if (GROUPED && row_index != nullptr) src = row_index[mr];
            y[(int64_t)mr * ldy + col] = fni8::dequant_one(s[i], as[src], wscale, bexp, col);
            if (acc_out) acc_out[(int64_t)mr * N + col] = s[i];
        }
    }
}

// ---------------------------------------------------------------------------
// tiled kernel
// ---------------------------------------------------------------------------
constexpr int kBK = 64;
constexpr int kLdsRow = 80;  // 64 data bytes + 16 pad

template <int BM, int BN, int WAVES_M, int WAVES_N, bool GROUPED>
__global__ __launch_bounds__(WAVES_M * WAVES_N * 64) void gemm_tile_kernel(
    const int8_t* __restrict__ aq, int64_t lda, const float* __restrict__ as,
    const int32_t* __restrict__ row_index, int M, int K, const int8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int E, const int32_t* __restrict__ seg_off,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out) {
    constexpr int NT = WAVES_M * WAVES_N * 64;
    constexpr int WTM = BM / WAVES_M, WTN = BN / WAVES_N;
    constexpr int FM = WTM / 16, FN = WTN / 16;
    constexpr int A_CH = BM * 4 / NT, B_CH = BN * 4 / NT;  // 16-byte chunks per thread
    static_assert(A_CH * NT == BM * 4 && B_CH * NT == BN * 4, "tile/threads mismatch");
    constexpr int BUF = (BM + BN) * kLdsRow;
    extern __shared__ __attribute__((aligned(16))) int8_t smem[];

    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wm = wave / WAVES_N, wn = wave % WAVES_N;
    const int ntiles_n = (N + BN - 1) / BN;

    int m0, m1, n0;
    const int8_t* wexp = w;
    const float* wsexp = ws;
    const uint16_t* bexp = bias;
    if constexpr (GROUPED) {  // x = segment tile slot, y = n-tile
        n0 = blockIdx.y * BN;
        int e;
        if (!fni8::find_group_tile(seg_off, E, BM, blockIdx.x, M, e, m0, m1)) return;
        wexp += (int64_t)e * N * K;
        wsexp += (int64_t)e * N;
        if (bias) bexp += (int64_t)e * N;
    } else {
        // XCD-aware order: consecutive ids land on different XCDs, so give each
        // XCD a contiguous band of the tile space, then walk it in groups of
        // 8 m-tiles for L2 reuse of both operands.
        const int ntiles_m = (M + BM - 1) / BM;
        const int total = ntiles_m * ntiles_n;
        int bid = blockIdx.x;
        if ((total & 7) == 0) bid = (bid & 7) * (total >> 3) + (bid >> 3);
        constexpr int GM = 8;
        const int group = bid / (GM * ntiles_n);
        const int first_m = group * GM;
        const int gsize = min(ntiles_m - first_m, GM);
        const int in_group = bid - group * GM * ntiles_n;
        const int pm = first_m + in_group % gsize;
        const int pn = in_group / gsize;
        m0 = pm * BM;
        m1 = min(M, m0 + BM);
        n0 = pn * BN;
    }

    // Global source pointers for this thread's chunks.  Rows past the end are
    // clamped to the last valid row: they load real memory whose products
    // land only in output rows that are never written.
    const int8_t* asrc[A_CH];
    const int8_t* bsrc[B_CH];
#pragma unroll
    for (int i = 0; i < A_CH; i++) {
        const int c = tid + i * NT;
        int mr = m0 + (c >> 2);
        mr = mr < m1 ? mr : m1 - 1;
        int src = mr;
        if (GROUPED && row_index != nullptr) src = row_index[mr];
        asrc[i] = aq + (int64_t)src * lda + (c & 3) * 16;
    }
#pragma unroll
    for (int i = 0; i < B_CH; i++) {
        const int c = tid + i * NT;
        int nr = n0 + (c >> 2);
        nr = nr < N ? nr : N - 1;
        bsrc[i] = wexp + (int64_t)nr * K + (c & 3) * 16;
    }

    i32x4 ra[A_CH], rb[B_CH];
    auto gload = [&](int kt) {
        const int64_t ko = (int64_t)kt * kBK;
#pragma unroll
        for (int i = 0; i < A_CH; i++) ra[i] = ld16(asrc[i] + ko);
#pragma unroll
        for (int i = 0; i < B_CH; i++) rb[i] = ld16(bsrc[i] + ko);
    };
    auto sstore = [&](int buf) {
        int8_t* base = smem + buf * BUF;
#pragma unroll
        for (int i = 0; i < A_CH; i++) {
            const int c = tid + i * NT;
            *reinterpret_cast<i32x4*>(base + (c >> 2) * kLdsRow + (c & 3) * 16) = ra[i];
        }
#pragma unroll
        for (int i = 0; i < B_CH; i++) {
            const int c = tid + i * NT;
            *reinterpret_cast<i32x4*>(base + (BM + (c >> 2)) * kLdsRow + (c & 3) * 16) = rb[i];
        }
    };

    i32x4 acc[FM][FN];
#pragma unroll
    for (int i = 0; i < FM; i++)
#pragma unroll
        for (int j = 0; j < FN; j++) acc[i][j] = i32x4{0, 0, 0, 0};

    const int KT = K / kBK;
    gload(0);
    sstore(0);
    __syncthreads();

    const int frag_off = (lane & 15) * kLdsRow + (lane >> 4) * 16;
    for (int kt = 0; kt < KT; kt++) {
        const int cur = kt & 1;
        if (kt + 1 < KT) gload(kt + 1);
        const int8_t* abase = smem + cur * BUF + (wm * WTM) * kLdsRow + frag_off;
        const int8_t* bbase = smem + cur * BUF + (BM + wn * WTN) * kLdsRow + frag_off;
        i32x4 af[FM], bf[FN];
#pragma unroll
        for (int i = 0; i < FM; i++) af[i] = *reinterpret_cast<const i32x4*>(abase + i * 16 * kLdsRow);
#pragma unroll
        for (int j = 0; j < FN; j++) bf[j] = *reinterpret_cast<const i32x4*>(bbase + j * 16 * kLdsRow);
#pragma unroll
        for (int i = 0; i < FM; i++)
#pragma unroll
            for (int j = 0; j < FN; j++) acc[i][j] = mfma_i8(af[i], bf[j], acc[i][j]);
        if (kt + 1 < KT) sstore(cur ^ 1);
        __syncthreads();
    }

    // Epilogue straight from the accumulators: lane holds D[4*(lane/16)+r][lane%16].
#pragma unroll
    for (int j = 0; j < FN; j++) {
        const int col = n0 + wn * WTN + j * 16 + (lane & 15);
        if (col >= N) continue;
        const float wsc = wsexp[col];
#pragma unroll
        for (int i = 0; i < FM; i++) {
#pragma unroll
            for (int r = 0; r < 4; r++) {
                const int mr = m0 + wm * WTM + i * 16 + (lane >> 4) * 4 + r;
                if (mr >= m1) continue;
                int src = mr;
                if (GROUPED && row_index != nullptr) src = row_index[mr];
                y[(int64_t)mr * ldy + col] = fni8::dequant_one(acc[i][j][r], as[src], wsc, bexp, col);
                if (acc_out) acc_out[(int64_t)mr * N + col] = acc[i][j][r];
            }
        }
    }
}

// ---------------------------------------------------------------------------
// generic kernel: one output per lane, v_dot4_i32_i8 over 4-byte words
// ---------------------------------------------------------------------------
template <bool GROUPED>
__global__ __launch_bounds__(256) void gemm_generic_kernel(
    const int8_t* __restrict__ aq, int64_t lda, const float* __restrict__ as,
    const int32_t* __restrict__ row_index, int M, int K, const int8_t* __restrict__ w,
    const float* __restrict__ ws, int N, int E, const int32_t* __restrict__ seg_off,
    const uint16_t* __restrict__ bias, uint16_t* __restrict__ y, int64_t ldy,
    int32_t* __restrict__ acc_out) {
    const int n = blockIdx.x * 256 + threadIdx.x;
    const int mr = blockIdx.y;
    if (n >= N || mr >= M) return;
    const int8_t* wexp = w;
    const float* wsexp = ws;
    const uint16_t* bexp = bias;
    int src = mr;
    if constexpr (GROUPED) {
        if (mr >= seg_off[E]) return;
        int lo = 0, hi = E;  // expert e with seg_off[e] <= mr < seg_off[e+1]
        while (hi - lo > 1) {
            int mid = (lo + hi) >> 1;
            if (seg_off[mid] <= mr) lo = mid; else hi = mid;
        }
        wexp += (int64_t)lo * N * K;
        wsexp += (int64_t)lo * N;
        if (bias) bexp += (int64_t)lo * N;
        if (row_index != nullptr) src = row_index[mr];
    }
    const int32_t* a4 = reinterpret_cast<const int32_t*>(aq + (int64_t)src * lda);
    const int32_t* w4 = reinterpret_cast<const int32_t*>(wexp + (int64_t)n * K);
    int32_t sum = 0;
    for (int k = 0; k < (K >> 2); k++) sum = __builtin_amdgcn_sdot4(a4[k], w4[k], sum, false);
    y[(int64_t)mr * ldy + n] = fni8::dequant_one(sum, as[src], wsexp[n], bexp, n);
    if (acc_out) acc_out[(int64_t)mr * N + n] = sum;
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
struct Args {
    const int8_t* aq;
    int64_t lda;
    const float* as;
    const int32_t* row_index;
    int M, K;
    const int8_t* w;
    const float* ws;
    int N, E;
    const int32_t* seg_off;
    const uint16_t* bias;
    uint16_t* y;
    int64_t ldy;
    int32_t* acc_out;
};

template <int MT, int NB, int WAVES, int U, bool GROUPED>
void launch_skinny(const Args& a, unsigned mslots, hipStream_t st) {
    const unsigned ntn = (unsigned)((a.N + 16 * NB - 1) / (16 * NB));
    dim3 grid = GROUPED ? dim3(mslots, ntn) : dim3(ntn, mslots), block(WAVES * 64);
    hipLaunchKernelGGL((gemm_skinny_kernel<MT, NB, WAVES, U, GROUPED>), grid, block, 0, st,
                       a.aq, a.lda, a.as, a.row_index, a.M, a.K, a.w, a.ws, a.N, a.E,
                       a.seg_off, a.bias, a.y, a.ldy, a.acc_out);
}

template <int BM, int BN, int WM, int WN, bool GROUPED>
int launch_tile(const Args& a, unsigned ytiles, hipStream_t st) {
    constexpr size_t lds = 2 * (BM + BN) * kLdsRow;
    auto kern = gemm_tile_kernel<BM, BN, WM, WN, GROUPED>;
    // The dynamic LDS limit is a per-function attribute; setting it again with
    // the same value is idempotent, so a race between threads is harmless.
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
    const unsigned ntn = (unsigned)((a.N + BN - 1) / BN);
    dim3 grid, block(WM * WN * 64);
    if constexpr (GROUPED)
        grid = dim3(ytiles, ntn);
    else
        grid = dim3(ntn * (unsigned)((a.M + BM - 1) / BM));
    hipLaunchKernelGGL(kern, grid, block, lds, st, a.aq, a.lda, a.as, a.row_index, a.M, a.K,
                       a.w, a.ws, a.N, a.E, a.seg_off, a.bias, a.y, a.ldy, a.acc_out);
    return FNI8_OK;
}

template <bool GROUPED>
void launch_generic(const Args& a, hipStream_t st) {
    dim3 grid((unsigned)((a.N + 255) / 256), (unsigned)a.M), block(256);
    hipLaunchKernelGGL(gemm_generic_kernel<GROUPED>, grid, block, 0, st, a.aq, a.lda, a.as,
                       a.row_index, a.M, a.K, a.w, a.ws, a.N, a.E, a.seg_off, a.bias, a.y,
                       a.ldy, a.acc_out);
}

// Decode launch shapes, chosen by measurement on MI355X (weights streamed from
// HBM): 4-wave groups with 16 loads in flight per lane for K = 4096, 8 waves x 4
// loads for long K; two weight blocks per wave once M >= 16 on wide N so each
// activation fragment is reused.
void launch_decode(const Args& a, hipStream_t st) {
    const int M = a.M, N = a.N, K = a.K;
    const bool wide = N >= 16384, longk = K >= 8192, mid = N >= 6144;
    if (M <= 4) {
        if (longk) launch_skinny<1, 1, 8, 4, false>(a, 1, st);
        else launch_skinny<1, 1, 4, 16, false>(a, 1, st);
    } else if (M <= 16) {
        if (wide) launch_skinny<1, 2, 2, 16, false>(a, 1, st);
        else if (longk) launch_skinny<1, 1, 16, 4, false>(a, 1, st);
        else if (mid) launch_skinny<1, 2, 2, 16, false>(a, 1, st);
        else launch_skinny<1, 1, 4, 16, false>(a, 1, st);
    } else if (M <= 32) {
        if (wide || (mid && !longk)) launch_skinny<2, 2, 4, 8, false>(a, 1, st);
        else if (longk) launch_skinny<2, 1, 16, 4, false>(a, 1, st);
        else launch_skinny<2, 1, 4, 16, false>(a, 1, st);
    } else {
        if (wide) launch_skinny<4, 2, 4, 4, false>(a, 1, st);
        else if (longk) launch_skinny<4, 1, 8, 4, false>(a, 1, st);
        else if (mid) launch_skinny<4, 2, 8, 2, false>(a, 1, st);
        else launch_skinny<4, 1, 4, 8, false>(a, 1, st);
    }
}

}  // namespace

namespace fni8h {

int launch_gemm(const int8_t* aq, int64_t lda, const float* as, const int32_t* row_index,
                int64_t M, int64_t K, const int8_t* w, const float* ws, int64_t N,
                int64_t E, const int32_t* seg_off, const uint16_t* bias, uint16_t* y,
                int64_t ldy, int32_t* acc_out, hipStream_t st, int8_t* work,
                int64_t work_bytes) {
    if (M == 0) return FNI8_OK;
    Args a{aq, lda, as, row_index, (int)M, (int)K, w, ws, (int)N, (int)E, seg_off, bias, y,
           ldy, acc_out};
    const bool grouped = E > 0;
    const bool fast = (K % 64 == 0) && (lda % 16 == 0) && ((uintptr_t)aq % 16 == 0) &&
                      ((uintptr_t)w % 16 == 0);
    int rc = FNI8_OK;
    if (!fast) {
        if (grouped) launch_generic<true>(a, st); else launch_generic<false>(a, st);
    } else if (grouped) {
        // Expert segments: average rows per expert picks the kernel -- the MFMA
        // decode kernel in grouped form up to 4 rows per expert (the skinny
        // kernel where it does not take the shape), the tile kernel above.
        const double avg = (double)M / (double)E;
        if (avg <= 4.0) {
            rc = launch_decode_mfma_grouped(aq, lda, as, row_index, M, K, w, ws, E, N, seg_off,
                                            bias, y, ldy, acc_out, st);
            if (rc == 1) {
                rc = FNI8_OK;
                const unsigned slots = (unsigned)((M + 15) / 16 + E);
                if (K >= 1024) launch_skinny<1, 1, 4, 8, true>(a, slots, st);
                else launch_skinny<1, 1, 2, 8, true>(a, slots, st);
            }
        } else {
            rc = launch_tile32(aq, lda, as, row_index, M, K, w, ws, N, E, seg_off, bias, y, ldy,
                               acc_out, st);
            if (rc == 1) {
                const unsigned slots = (unsigned)((M + 127) / 128 + E);
                rc = launch_tile<128, 128, 2, 2, true>(a, slots, st);
            }
        }
    } else if (M <= 64) {
        rc = launch_decode_q(aq, lda, as, M, K, w, ws, N, bias, y, ldy, acc_out, st);
        if (rc == 1) rc = launch_decode_mfma(aq, lda, as, M, K, w, ws, N, bias, y, ldy, acc_out, st);
        if (rc == 1) {
            rc = FNI8_OK;
            launch_decode(a, st);
        }
    } else {
        rc = launch_pp(aq, lda, as, M, K, w, ws, N, bias, y, ldy, acc_out, work, work_bytes, st);
        if (rc == 1)
            rc = launch_tile32(aq, lda, as, row_index, M, K, w, ws, N, 0, seg_off, bias, y, ldy,
                               acc_out, st);
        if (rc == 1) {  // K not a multiple of 128: the 16x16x64 tile kernel
            const int64_t t256 = ((M + 255) / 256) * ((N + 255) / 256);
            if (t256 >= 256)
                rc = launch_tile<256, 256, 2, 4, false>(a, 0, st);
            else
                rc = launch_tile<128, 128, 2, 2, false>(a, 0, st);
        }
    }
    if (rc) return rc;
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("gemm launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

}  // namespace fni8h
