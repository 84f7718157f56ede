// MoE routing sort and weighted combine (gfx950).
//
// sort:    one workgroup per expert.  Pass 1 counts ids below and equal to the
//          expert (block reduction) -> the segment start, with no global
//          atomics.  Pass 2 walks the T*k ids in order and places the expert's
//          entries with a block-wide exclusive scan, so the segment keeps the
//          (token, slot) order of `(topi == e).nonzero()` -- a deterministic,
//          stable counting sort.  The ids are read twice per workgroup from L2.
// combine: one workgroup per token; each lane owns 8 consecutive hidden
//          elements and sums the token's expert rows in ascending expert id
//          with fp16 rounding after every product and add, matching the
//          sequential index_add_ of the per-expert loop.
#include "common.h"

namespace {

constexpr int kSortThreads = 256;
constexpr int kSortPer = 4;  // ids per thread per chunk
constexpr int kMaxTopK = 32;

__device__ __forceinline__ int block_excl_scan(int v, int* lds, int& total) {
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int incl = fni8::wave_incl_scan_i32(v, lane);
    if (lane == 63) lds[wave] = incl;
    __syncthreads();
    int before = 0;
    total = 0;
#pragma unroll
    for (int i = 0; i < kSortThreads / 64; i++) {
        const int t = lds[i];
        before += i < wave ? t : 0;
        total += t;
    }
    __syncthreads();
    return before + incl - v;
}

__global__ __launch_bounds__(kSortThreads) void moe_sort_kernel(
    const int32_t* __restrict__ topi, int Tk, int k, int E, int32_t* __restrict__ seg_off,
    int32_t* __restrict__ row_token, int32_t* __restrict__ pos) {
    __shared__ int lds[kSortThreads / 64];
    const int e = blockIdx.x;
    const int tid = threadIdx.x;

    int lt = 0, eq = 0;
    for (int i = tid; i < Tk; i += kSortThreads) {
        const int id = topi[i];
        lt += (id >= 0 && id < e) ? 1 : 0;
        eq += id == e ? 1 : 0;
    }
    int tot_lt, tot_eq;
    block_excl_scan(lt, lds, tot_lt);
    block_excl_scan(eq, lds, tot_eq);
    if (tid == 0) {
        seg_off[e] = tot_lt;
        if (e == E - 1) seg_off[E] = tot_lt + tot_eq;
    }

    int base = tot_lt;
    for (int c0 = 0; c0 < Tk; c0 += kSortThreads * kSortPer) {
        const int i0 = c0 + tid * kSortPer;
        bool hit[kSortPer];
        int cnt = 0;
#pragma unroll
        for (int j = 0; j < kSortPer; j++) {
            hit[j] = (i0 + j < Tk) && topi[i0 + j] == e;
            cnt += hit[j] ? 1 : 0;
        }
        int chunk_total;
        int p = base + block_excl_scan(cnt, lds, chunk_total);
#pragma unroll
        for (int j = 0; j < kSortPer; j++) {
            if (hit[j]) {
                row_token[p] = (i0 + j) / k;
                pos[i0 + j] = p;
                p++;
            } else if (e == 0 && i0 + j < Tk) {
                const int id = topi[i0 + j];
                if (id < 0 || id >= E) pos[i0 + j] = -1;  // out-of-range id: no row
            }
        }
        base += chunk_total;
    }
}

// Combine for k <= KM (the common top-8): the slots are sorted by expert id
// with an odd-even transposition network (static register indices, stable, so
// the order is that of the insertion sort below), all k rows of the token are
// loaded up front, then summed in that order with the same fp16 roundings.
template <int KM>
__global__ __launch_bounds__(256) void moe_combine_small_kernel(
    const uint16_t* __restrict__ yr, int H, const int32_t* __restrict__ topi,
    const uint16_t* __restrict__ topw, const int32_t* __restrict__ pos, int k,
    int Tk, uint16_t* __restrict__ out) {
    const int t = blockIdx.x;
    int eid[KM], ord[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) {
        eid[j] = j < k ? topi[(int64_t)t * k + j] : 0x7fffffff;
        ord[j] = j;
    }
#pragma unroll
    for (int r = 0; r < KM; r++)
#pragma unroll
        for (int a = r & 1; a + 1 < KM; a += 2)
            if (eid[a] > eid[a + 1]) {
                const int e0 = eid[a], o0 = ord[a];
                eid[a] = eid[a + 1];
                ord[a] = ord[a + 1];
                eid[a + 1] = e0;
                ord[a + 1] = o0;
            }
    int64_t row[KM];
    float wgt[KM];
    bool ok[KM];
#pragma unroll
    for (int j = 0; j < KM; j++) {
        ok[j] = false;
        row[j] = 0;
        wgt[j] = 0.f;
        if (j < k) {
            const int slot = ord[j];
            row[j] = pos[(int64_t)t * k + slot];
            wgt[j] = fni8::h2f(topw[(int64_t)t * k + slot]);
            ok[j] = row[j] >= 0 && row[j] < Tk;
        }
    }
    for (int h0 = threadIdx.x * 8; h0 < H; h0 += 256 * 8) {
        uint4 v[KM];
#pragma unroll
        for (int j = 0; j < KM; j++)
            v[j] = ok[j] ? *reinterpret_cast<const uint4*>(yr + row[j] * H + h0) : make_uint4(0, 0, 0, 0);
        uint16_t ob[8];
#pragma unroll
        for (int i = 0; i < 8; i++) ob[i] = 0;
#pragma unroll
        for (int j = 0; j < KM; j++) {
            if (!ok[j]) continue;
            const uint32_t w4[4] = {v[j].x, v[j].y, v[j].z, v[j].w};
#pragma unroll
            for (int i = 0; i < 8; i++) {
                const uint16_t c = (uint16_t)(w4[i >> 1] >> ((i & 1) * 16));
                const uint16_t pr = fni8::f2h(fni8::h2f(c) * wgt[j]);
                ob[i] = fni8::f2h(fni8::h2f(ob[i]) + fni8::h2f(pr));
            }
        }
        uint4 st;
        st.x = ob[0] | ((uint32_t)ob[1] << 16);
        st.y = ob[2] | ((uint32_t)ob[3] << 16);
        st.z = ob[4] | ((uint32_t)ob[5] << 16);
        st.w = ob[6] | ((uint32_t)ob[7] << 16);
        *reinterpret_cast<uint4*>(out + (int64_t)t * H + h0) = st;
    }
}

template <bool VEC>
__global__ __launch_bounds__(256) void moe_combine_kernel(
    const uint16_t* __restrict__ yr, int H, const int32_t* __restrict__ topi,
    const uint16_t* __restrict__ topw, const int32_t* __restrict__ pos, int k,
    int Tk, uint16_t* __restrict__ out) {
    const int t = blockIdx.x;
    int order[kMaxTopK];
    int eid[kMaxTopK];
    for (int j = 0; j < k; j++) {
        eid[j] = topi[(int64_t)t * k + j];
        order[j] = j;
    }
    for (int a = 1; a < k; a++) {  // insertion sort of the slots by expert id
        const int v = order[a];
        int b = a - 1;
        while (b >= 0 && eid[order[b]] > eid[v]) {
            order[b + 1] = order[b];
            b--;
        }
        order[b + 1] = v;
    }
    if constexpr (VEC) {
        for (int h0 = threadIdx.x * 8; h0 < H; h0 += 256 * 8) {
            float o[8];
            uint16_t ob[8];
#pragma unroll
            for (int i = 0; i < 8; i++) ob[i] = 0;
            for (int j = 0; j < k; j++) {
                const int slot = order[j];
                const float wgt = fni8::h2f(topw[(int64_t)t * k + slot]);
                const int64_t row = pos[(int64_t)t * k + slot];
                if (row < 0 || row >= Tk) continue;
                const uint4 v = *reinterpret_cast<const uint4*>(yr + row * H + h0);
                const uint32_t w4[4] = {v.x, v.y, v.z, v.w};
#pragma unroll
                for (int i = 0; i < 8; i++) {
                    const uint16_t c = (uint16_t)(w4[i >> 1] >> ((i & 1) * 16));
                    const uint16_t pr = fni8::f2h(fni8::h2f(c) * wgt);
                    o[i] = fni8::h2f(ob[i]) + fni8::h2f(pr);
                    ob[i] = fni8::f2h(o[i]);
                }
            }
            uint4 st;
            st.x = ob[0] | ((uint32_t)ob[1] << 16);
            st.y = ob[2] | ((uint32_t)ob[3] << 16);
            st.z = ob[4] | ((uint32_t)ob[5] << 16);
            st.w = ob[6] | ((uint32_t)ob[7] << 16);
            *reinterpret_cast<uint4*>(out + (int64_t)t * H + h0) = st;
        }
    } else {
        for (int h = threadIdx.x; h < H; h += 256) {
            uint16_t ob = 0;
            for (int j = 0; j < k; j++) {
                const int slot = order[j];
                const float wgt = fni8::h2f(topw[(int64_t)t * k + slot]);
                const int64_t row = pos[(int64_t)t * k + slot];
                if (row < 0 || row >= Tk) continue;
                const uint16_t pr = fni8::f2h(fni8::h2f(yr[row * H + h]) * wgt);
                ob = fni8::f2h(fni8::h2f(ob) + fni8::h2f(pr));
            }
            out[(int64_t)t * H + h] = ob;
        }
    }
}

}  // namespace

namespace fni8h {

int launch_moe_sort(const int32_t* topi, int64_t T, int64_t k, int64_t E, int32_t* seg_off,
                    int32_t* row_token, int32_t* pos, hipStream_t st) {
    hipLaunchKernelGGL(moe_sort_kernel, dim3((unsigned)E), dim3(kSortThreads), 0, st, topi,
                       (int)(T * k), (int)k, (int)E, seg_off, row_token, pos);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("moe_sort launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

int launch_moe_combine(const uint16_t* yr, int64_t H, const int32_t* topi,
                       const uint16_t* topw, const int32_t* pos, int64_t T, int64_t k,
                       uint16_t* out, hipStream_t st) {
    if (T == 0) return FNI8_OK;
    const bool vec = (H % 8 == 0) && ((uintptr_t)yr % 16 == 0) && ((uintptr_t)out % 16 == 0);
    if (vec && k <= 8)
        hipLaunchKernelGGL(moe_combine_small_kernel<8>, dim3((unsigned)T), dim3(256), 0, st, yr,
                           (int)H, topi, topw, pos, (int)k, (int)(T * k), out);
    else if (vec)
        hipLaunchKernelGGL(moe_combine_kernel<true>, dim3((unsigned)T), dim3(256), 0, st, yr,
                           (int)H, topi, topw, pos, (int)k, (int)(T * k), out);
    else
        hipLaunchKernelGGL(moe_combine_kernel<false>, dim3((unsigned)T), dim3(256), 0, st, yr,
                           (int)H, topi, topw, pos, (int)k, (int)(T * k), out);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) {
        set_error_detail("moe_combine launch: %s", hipGetErrorString(e));
        return FNI8_ERR_LAUNCH;
    }
    return FNI8_OK;
}

}  // namespace fni8h
