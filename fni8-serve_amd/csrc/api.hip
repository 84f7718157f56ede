// extern "C" entry points: argument checks, then the launches on the caller's
// stream.  Nothing here allocates device memory or synchronises.
#include <stdarg.h>
#include <stdio.h>
#include <string.h>

#include <mutex>

#include "common.h"

namespace fni8h {

static thread_local char g_detail[512];

void set_error_detail(const char* fmt, ...) {
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(g_detail, sizeof g_detail, fmt, ap);
    va_end(ap);
}

}  // namespace fni8h

namespace {

using fni8h::set_error_detail;

constexpr int64_t kMaxDim = (int64_t)1 << 31;
constexpr int kMaxDevices = 64;
// 0 = unknown, 1 = gfx950, -1 = other.  Written once per device; a repeated
// write of the same value from two threads is harmless.
int g_device_ok[kMaxDevices];

int scratch_address(int8_t** out);

int check_device() {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0) {
        set_error_detail("no current HIP device");
        return FNI8_ERR_DEVICE;
    }
    if (dev < kMaxDevices && g_device_ok[dev] == 1) return FNI8_OK;
    hipDeviceProp_t prop;
    if (hipGetDeviceProperties(&prop, dev) != hipSuccess) {
        set_error_detail("hipGetDeviceProperties failed on device %d", dev);
        return FNI8_ERR_DEVICE;
    }
    const bool ok = strncmp(prop.gcnArchName, "gfx950", 6) == 0;
    if (!ok) {
        if (dev < kMaxDevices) g_device_ok[dev] = -1;
        set_error_detail("device %d is %s; these kernels are built for gfx950", dev,
                         prop.gcnArchName);
        return FNI8_ERR_DEVICE;
    }
    // The first call on a device also looks up the no-allocation entry point's
    // scratch address, so that a later call of that entry point under graph
    // capture makes no runtime query.
    int8_t* sp = nullptr;
    const int rc = scratch_address(&sp);
    if (rc) return rc;
    if (dev < kMaxDevices) g_device_ok[dev] = 1;
    return FNI8_OK;
}

// ---- scratch of fni8_linear_w8a8_f16_noalloc ---------------------------------
// The quantized activations (int8 [M, K], row stride K) and their scales
// (fp32 [M]) of the entry point that allocates nothing live in this array: one
// copy per GPU, resident from the library's load on that GPU until the process
// ends.  Every call on a GPU shares its copy (overlapping calls race).
constexpr int64_t kNoAllocQBytes = (int64_t)48 << 20;  // M * K (every Qwen3-8B linear to M = 4096)
constexpr int64_t kNoAllocRows = 65536;                // M
static __device__ __align__(256) int8_t scratch[kNoAllocQBytes + kNoAllocRows * 4];

// Device address of `scratch` on the current device, looked up once per device
// with that device current (in host code `scratch` names a host-side stand-in,
// not device memory).
void* g_scratch_dev[kMaxDevices];
std::mutex g_scratch_mu;

int scratch_address(int8_t** out) {
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        set_error_detail("no usable current device for the scratch lookup");
        return FNI8_ERR_DEVICE;
    }
    void* p = __atomic_load_n(&g_scratch_dev[dev], __ATOMIC_ACQUIRE);
    if (p == nullptr) {
        std::lock_guard<std::mutex> lock(g_scratch_mu);
        p = g_scratch_dev[dev];
        if (p == nullptr) {
            const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
            if (e != hipSuccess || p == nullptr) {
                set_error_detail("scratch lookup on device %d: %s", dev, hipGetErrorString(e));
                return FNI8_ERR_LAUNCH;
            }
            __atomic_store_n(&g_scratch_dev[dev], p, __ATOMIC_RELEASE);
        }
    }
    *out = static_cast<int8_t*>(p);
    return FNI8_OK;
}

bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }

#define REQUIRE(cond, code, ...)          \
    do {                                  \
        if (!(cond)) {                    \
            set_error_detail(__VA_ARGS__); \
            return (code);                \
        }                                 \
    } while (0)

int check_gemm_shape(int64_t M, int64_t K, int64_t N) {
    REQUIRE(M >= 0 && M < kMaxDim, FNI8_ERR_SHAPE, "M=%lld out of range", (long long)M);
    REQUIRE(N > 0 && N < kMaxDim, FNI8_ERR_SHAPE, "N=%lld out of range", (long long)N);
    REQUIRE(K > 0 && K < kMaxDim, FNI8_ERR_SHAPE, "K=%lld out of range", (long long)K);
    REQUIRE(K % 4 == 0, FNI8_ERR_SHAPE, "K=%lld is not a multiple of 4", (long long)K);
    return FNI8_OK;
}

int check_w4a8(int64_t M, int64_t K, int64_t N, int64_t G, const uint8_t* w, const float* ws,
               const void* bias, const void* y, int64_t ldy) {
    REQUIRE(w && ws && y, FNI8_ERR_NULL, "w, ws and y are required");
    REQUIRE(M >= 0 && M < kMaxDim && N > 0 && N < kMaxDim && K > 0 && K < kMaxDim,
            FNI8_ERR_SHAPE, "M=%lld N=%lld K=%lld out of range", (long long)M, (long long)N,
            (long long)K);
    REQUIRE(G == 32 || G == 64 || G == 128 || G == 256, FNI8_ERR_SHAPE,
            "group size %lld not supported (32, 64, 128, 256)", (long long)G);
    REQUIRE(K % 32 == 0 && K % G == 0, FNI8_ERR_SHAPE,
            "K=%lld must be a multiple of 32 and of the group size %lld", (long long)K,
            (long long)G);
    REQUIRE(ldy >= N, FNI8_ERR_STRIDE, "ldy=%lld < N=%lld", (long long)ldy, (long long)N);
    REQUIRE(aligned(w, 16) && aligned(ws, 4) && aligned(bias, 2) && aligned(y, 2),
            FNI8_ERR_ALIGN, "w must be 16-byte aligned; ws, bias, y element-aligned");
    return FNI8_OK;
}

int check_rmsnorm(const void* x, int64_t ldx, const void* residual, int64_t ldr,
                  const void* weight, float eps, int64_t M, int64_t K, int64_t ldo,
                  const void* residual_out, int64_t ldro) {
    REQUIRE(x && weight, FNI8_ERR_NULL, "x and weight are required");
    REQUIRE(M >= 0 && M < kMaxDim && K > 0 && K < kMaxDim, FNI8_ERR_SHAPE,
            "M=%lld K=%lld out of range", (long long)M, (long long)K);
    REQUIRE(eps >= 0.0f && eps < __builtin_inff(), FNI8_ERR_SHAPE, "eps must be finite and >= 0");
    REQUIRE(ldx >= K && ldo >= K, FNI8_ERR_STRIDE, "ldx=%lld or output stride %lld < K=%lld",
            (long long)ldx, (long long)ldo, (long long)K);
    REQUIRE(!residual || ldr >= K, FNI8_ERR_STRIDE, "ldr=%lld < K", (long long)ldr);
    REQUIRE(!residual || !residual_out || ldro >= K, FNI8_ERR_STRIDE, "ldro=%lld < K",
            (long long)ldro);
    REQUIRE(aligned(x, 2) && aligned(residual, 2) && aligned(weight, 2) &&
                aligned(residual_out, 2),
            FNI8_ERR_ALIGN, "fp16 operands misaligned");
    return FNI8_OK;
}

int linear_launch(const void* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                  const float* ws, int64_t N, const void* bias, void* y, int64_t ldy, int8_t* xq,
                  float* xs, int32_t* acc_out, int8_t* work, int64_t work_bytes, hipStream_t st);

int check_linear(const void* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                 const float* ws, int64_t N, const void* bias, const void* y, int64_t ldy,
                 const int8_t* xq, const float* xs, const int32_t* acc_out) {
    REQUIRE(x && w && ws && y && xq && xs, FNI8_ERR_NULL,
            "x, w, ws, y, xq and xs are required");
    int rc = check_gemm_shape(M, K, N);
    if (rc) return rc;
    REQUIRE(ldx >= K && ldy >= N, FNI8_ERR_STRIDE, "ldx=%lld < K or ldy=%lld < N",
            (long long)ldx, (long long)ldy);
    REQUIRE(aligned(x, 2) && aligned(xq, 4) && aligned(w, 4), FNI8_ERR_ALIGN,
            "x, xq or w misaligned");
    REQUIRE(aligned(xs, 4) && aligned(ws, 4) && aligned(y, 2) && aligned(bias, 2) &&
                aligned(acc_out, 4),
            FNI8_ERR_ALIGN, "scale/output pointers misaligned");
    return FNI8_OK;
}

}  // namespace

extern "C" {

const char* fni8_strerror(int code) {
    switch (code) {
        case FNI8_OK: return "ok";
        case FNI8_ERR_NULL: return "required pointer is NULL";
        case FNI8_ERR_SHAPE: return "shape out of range";
        case FNI8_ERR_ALIGN: return "pointer or stride misaligned";
        case FNI8_ERR_STRIDE: return "leading dimension smaller than the row";
        case FNI8_ERR_LAUNCH: return "HIP launch error";
        case FNI8_ERR_DEVICE: return "unsupported or missing device";
        default: return "unknown error";
    }
}

const char* fni8_last_error(void) { return fni8h::g_detail; }

const char* fni8_version(void) { return "fni8amd 0.1.0 gfx950"; }

int fni8_init(void) {
    fni8h::g_detail[0] = 0;
    int count = 0, cur = 0;
    if (hipGetDeviceCount(&count) != hipSuccess || count <= 0) {
        set_error_detail("no HIP device");
        return FNI8_ERR_DEVICE;
    }
    if (hipGetDevice(&cur) != hipSuccess) cur = 0;
    int rc = FNI8_OK;
    for (int d = 0; d < count && d < kMaxDevices; d++) {
        hipDeviceProp_t prop;
        if (hipGetDeviceProperties(&prop, d) != hipSuccess ||
            strncmp(prop.gcnArchName, "gfx950", 6) != 0)
            continue;  // other devices are left alone
        if (hipSetDevice(d) != hipSuccess) {
            set_error_detail("hipSetDevice(%d) failed", d);
            rc = FNI8_ERR_DEVICE;
            break;
        }
        rc = check_device();
        if (rc) break;
    }
    (void)hipSetDevice(cur);
    return rc;
}

int fni8_quantize_rowwise_f16(const void* x, int64_t M, int64_t K, int64_t ldx, int8_t* xq,
                              int64_t ldq, float* xs, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(x && xq && xs, FNI8_ERR_NULL, "x, xq and xs are required");
    REQUIRE(M >= 0 && M < kMaxDim, FNI8_ERR_SHAPE, "M=%lld out of range", (long long)M);
    REQUIRE(K > 0 && K < kMaxDim && K % 4 == 0, FNI8_ERR_SHAPE,
            "K=%lld must be positive and a multiple of 4", (long long)K);
    REQUIRE(ldx >= K && ldq >= K, FNI8_ERR_STRIDE, "ldx=%lld ldq=%lld < K=%lld",
            (long long)ldx, (long long)ldq, (long long)K);
    REQUIRE(aligned(x, 2) && aligned(xs, 4), FNI8_ERR_ALIGN, "x or xs misaligned");
    int rc = check_device();
    if (rc) return rc;
    return fni8h::launch_quant_rowwise((const uint16_t*)x, M, K, ldx, xq, ldq, xs,
                                       (hipStream_t)stream);
}

int fni8_gemm_w8a8(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                   const int8_t* w, const float* ws, int64_t N, const void* bias, void* y,
                   int64_t ldy, int32_t* acc_out, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(xq && xs && w && ws && y, FNI8_ERR_NULL, "xq, xs, w, ws and y are required");
    int rc = check_gemm_shape(M, K, N);
    if (rc) return rc;
    REQUIRE(ldq >= K && ldy >= N, FNI8_ERR_STRIDE, "ldq=%lld < K or ldy=%lld < N",
            (long long)ldq, (long long)ldy);
    REQUIRE(ldq % 4 == 0 && aligned(xq, 4) && aligned(w, 4), FNI8_ERR_ALIGN,
            "int8 operands need 4-byte aligned rows");
    REQUIRE(aligned(xs, 4) && aligned(ws, 4) && aligned(y, 2) && aligned(bias, 2) &&
                aligned(acc_out, 4),
            FNI8_ERR_ALIGN, "scale/output pointers misaligned");
    rc = check_device();
    if (rc) return rc;
    return fni8h::launch_gemm(xq, ldq, xs, nullptr, M, K, w, ws, N, 0, nullptr,
                              (const uint16_t*)bias, (uint16_t*)y, ldy, acc_out,
                              (hipStream_t)stream);
}

int fni8_linear_w8a8_f16(const void* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                         const float* ws, int64_t N, const void* bias, void* y, int64_t ldy,
                         int8_t* xq, float* xs, int32_t* acc_out, void* stream) {
    fni8h::g_detail[0] = 0;
    int rc = check_linear(x, ldx, M, K, w, ws, N, bias, y, ldy, xq, xs, acc_out);
    if (rc) return rc;
    rc = check_device();
    if (rc) return rc;
    return linear_launch(x, ldx, M, K, w, ws, N, bias, y, ldy, xq, xs, acc_out, nullptr, 0,
                         (hipStream_t)stream);
}

int fni8_linear_w8a8_f16_ws(const void* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                            const float* ws, int64_t N, const void* bias, void* y, int64_t ldy,
                            int8_t* xq, float* xs, int32_t* acc_out, void* workspace,
                            int64_t workspace_bytes, void* stream) {
    fni8h::g_detail[0] = 0;
    int rc = check_linear(x, ldx, M, K, w, ws, N, bias, y, ldy, xq, xs, acc_out);
    if (rc) return rc;
    REQUIRE(workspace_bytes >= 0 && (!workspace || aligned(workspace, 256)), FNI8_ERR_ALIGN,
            "workspace must be 256-byte aligned with a size >= 0");
    rc = check_device();
    if (rc) return rc;
    return linear_launch(x, ldx, M, K, w, ws, N, bias, y, ldy, xq, xs, acc_out,
                         static_cast<int8_t*>(workspace), workspace ? workspace_bytes : 0,
                         (hipStream_t)stream);
}

int64_t fni8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K) {
    if (M < 0 || N <= 0 || K <= 0 || M >= kMaxDim || N >= kMaxDim || K >= kMaxDim) return 0;
    if (M <= 16) return fni8h::coop_workspace_bytes(M, N, K);
    return fni8h::pp_workspace_bytes(M, N, K);
}

int fni8_gemm_w8a8_ws(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                      const int8_t* w, const float* ws, int64_t N, const void* bias, void* y,
                      int64_t ldy, int32_t* acc_out, void* workspace, int64_t workspace_bytes,
                      void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(xq && xs && w && ws && y, FNI8_ERR_NULL, "xq, xs, w, ws and y are required");
    int rc = check_gemm_shape(M, K, N);
    if (rc) return rc;
    REQUIRE(ldq >= K && ldy >= N, FNI8_ERR_STRIDE, "ldq=%lld < K or ldy=%lld < N",
            (long long)ldq, (long long)ldy);
    REQUIRE(ldq % 4 == 0 && aligned(xq, 4) && aligned(w, 4), FNI8_ERR_ALIGN,
            "int8 operands need 4-byte aligned rows");
    REQUIRE(aligned(xs, 4) && aligned(ws, 4) && aligned(y, 2) && aligned(bias, 2) &&
                aligned(acc_out, 4),
            FNI8_ERR_ALIGN, "scale/output pointers misaligned");
    REQUIRE(workspace_bytes >= 0 && (!workspace || aligned(workspace, 256)), FNI8_ERR_ALIGN,
            "workspace must be 256-byte aligned with a size >= 0");
    rc = check_device();
    if (rc) return rc;
    return fni8h::launch_gemm(xq, ldq, xs, nullptr, M, K, w, ws, N, 0, nullptr,
                              (const uint16_t*)bias, (uint16_t*)y, ldy, acc_out,
                              (hipStream_t)stream, static_cast<int8_t*>(workspace),
                              workspace ? workspace_bytes : 0);
}

void fni8_debug_coop_wait_ticks(int64_t ticks) { fni8h::set_coop_wait_ticks(ticks); }

void fni8_debug_gemm_plan(int64_t bm, int64_t bn, int64_t split) {
    fni8h::set_gemm_plan(bm, bn, split);
}

int fni8_linear_w8a8_f16_noalloc(const void* x, int64_t ldx, int64_t M, int64_t K,
                                 const int8_t* w, const float* ws, int64_t N, const void* bias,
                                 void* y, int64_t ldy, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(x && w && ws && y, FNI8_ERR_NULL, "x, w, ws and y are required");
    int rc = check_gemm_shape(M, K, N);
    if (rc) return rc;
    REQUIRE(M <= kNoAllocRows && M * K <= kNoAllocQBytes, FNI8_ERR_SHAPE,
            "M=%lld K=%lld exceeds the no-allocation scratch (M <= %lld and M*K <= %lld bytes)",
            (long long)M, (long long)K, (long long)kNoAllocRows, (long long)kNoAllocQBytes);
    REQUIRE(ldx >= K && ldy >= N, FNI8_ERR_STRIDE, "ldx=%lld < K or ldy=%lld < N",
            (long long)ldx, (long long)ldy);
    REQUIRE(aligned(x, 2) && aligned(w, 4) && aligned(ws, 4) && aligned(y, 2) && aligned(bias, 2),
            FNI8_ERR_ALIGN, "x, w, ws, y or bias misaligned");
    rc = check_device();
    if (rc) return rc;
    int8_t* sp = nullptr;
    rc = scratch_address(&sp);
    if (rc) return rc;
    // xq: M rows of K bytes at the start; xs: M floats after the xq area; the
    // rest of the xq area (past M * K, 256-aligned) is the workspace of the
    // one-launch decode path and of the split-K prefill GEMM (where its plan
    // fits).  Every byte the GEMM reads is written by this call's quantization
    // first, and the workspace needs no clearing, so nothing is cleared between
    // calls.
    const int64_t work_off = (M * K + 255) & ~(int64_t)255;
    return linear_launch(x, ldx, M, K, w, ws, N, bias, y, ldy, sp,
                         reinterpret_cast<float*>(sp + kNoAllocQBytes), nullptr, sp + work_off,
                         kNoAllocQBytes - work_off, (hipStream_t)stream);
}

}  // extern "C"

namespace {

// The launches of the whole W8A8 linear on caller-checked arguments.
int linear_launch(const void* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                  const float* ws, int64_t N, const void* bias, void* y, int64_t ldy, int8_t* xq,
                  float* xs, int32_t* acc_out, int8_t* work, int64_t work_bytes, hipStream_t st) {
    int rc;
    // 5..16 tokens with a workspace: one launch, the quantization shared per XCD
    if (M >= 5 && work != nullptr) {
        rc = fni8h::launch_decode_coop((const uint16_t*)x, ldx, M, K, w, ws, N,
                                       (const uint16_t*)bias, (uint16_t*)y, ldy, xq, xs, acc_out,
                                       work, work_bytes, st);
        if (rc != 1) return rc;
    }
    // Decode sizes: one launch, the quantization fused into the GEMM -- on MFMA
    // for 3..4 tokens, as a dot4 GEMV for 1..2 (and shapes the MFMA kernel does
    // not take), where the streaming loop without an LDS pass is faster.
    if (M >= 3) {
        rc = fni8h::launch_decode_mfma_fused((const uint16_t*)x, ldx, M, K, w, ws, N,
                                             (const uint16_t*)bias, (uint16_t*)y, ldy, xq, xs,
                                             acc_out, st);
        if (rc != 1) return rc;
    }
    rc = fni8h::launch_decode_fused((const uint16_t*)x, ldx, M, K, w, ws, N, (const uint16_t*)bias,
                                    (uint16_t*)y, ldy, xq, xs, acc_out, st);
    if (rc != 1) return rc;
    rc = fni8h::launch_quant_rowwise((const uint16_t*)x, M, K, ldx, xq, K, xs, st);
    if (rc) return rc;
    return fni8h::launch_gemm(xq, K, xs, nullptr, M, K, w, ws, N, 0, nullptr,
                              (const uint16_t*)bias, (uint16_t*)y, ldy, acc_out, st, work,
                              work_bytes);
}

}  // namespace

extern "C" {

int fni8_moe_sort(const int32_t* topi, int64_t T, int64_t k, int64_t E, int32_t* seg_off,
                  int32_t* row_token, int32_t* pos, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(topi && seg_off && row_token && pos, FNI8_ERR_NULL,
            "topi, seg_off, row_token and pos are required");
    REQUIRE(T >= 0 && k > 0 && k <= 32 && E > 0 && E < 65536 && T * k < kMaxDim,
            FNI8_ERR_SHAPE, "T=%lld k=%lld E=%lld out of range (k <= 32)", (long long)T,
            (long long)k, (long long)E);
    REQUIRE(aligned(topi, 4) && aligned(seg_off, 4) && aligned(row_token, 4) && aligned(pos, 4),
            FNI8_ERR_ALIGN, "int32 arrays misaligned");
    int rc = check_device();
    if (rc) return rc;
    return fni8h::launch_moe_sort(topi, T, k, E, seg_off, row_token, pos, (hipStream_t)stream);
}

int fni8_gemm_w8a8_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                           int64_t R_max, int64_t K, const int8_t* w, const float* ws,
                           int64_t E, int64_t N, const int32_t* seg_off, const void* bias,
                           void* y, int32_t* acc_out, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(aq && as && w && ws && seg_off && y, FNI8_ERR_NULL,
            "aq, as, w, ws, seg_off and y are required");
    int rc = check_gemm_shape(R_max, K, N);
    if (rc) return rc;
    REQUIRE(E > 0 && E < 65536, FNI8_ERR_SHAPE, "E=%lld out of range", (long long)E);
    REQUIRE(aligned(aq, 4) && aligned(w, 4) && aligned(as, 4) && aligned(ws, 4) &&
                aligned(row_index, 4) && aligned(seg_off, 4) && aligned(y, 2) &&
                aligned(bias, 2) && aligned(acc_out, 4),
            FNI8_ERR_ALIGN, "grouped operands misaligned");
    rc = check_device();
    if (rc) return rc;
    return fni8h::launch_gemm(aq, K, as, row_index, R_max, K, w, ws, N, E, seg_off,
                              (const uint16_t*)bias, (uint16_t*)y, N, acc_out,
                              (hipStream_t)stream);
}

int fni8_gemm_w4a8_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                           int64_t R_max, int64_t K, const uint8_t* w, const float* ws,
                           int64_t E, int64_t N, int64_t G, const int32_t* seg_off,
                           const void* bias, void* y, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(aq && as && w && ws && seg_off && y, FNI8_ERR_NULL,
            "aq, as, w, ws, seg_off and y are required");
    int rc = check_w4a8(R_max, K, N, G, w, ws, bias, y, N);
    if (rc) return rc;
    REQUIRE(E > 0 && E < 65536, FNI8_ERR_SHAPE, "E=%lld out of range", (long long)E);
    REQUIRE(G >= 64 && K % 256 == 0 && N < (1 << 21), FNI8_ERR_SHAPE,
            "grouped W4A8 needs G in {64, 128, 256}, K a multiple of 256 and N < 2^21 "
            "(G=%lld K=%lld N=%lld)", (long long)G, (long long)K, (long long)N);
    REQUIRE(aligned(aq, 16) && aligned(as, 4) && aligned(row_index, 4) && aligned(seg_off, 4),
            FNI8_ERR_ALIGN, "aq must be 16-byte aligned; as, row_index, seg_off 4-byte aligned");
    rc = check_device();
    if (rc) return rc;
    return fni8h::launch_gemm_w4a8_grouped(aq, as, row_index, R_max, K, w, ws, E, N, G, seg_off,
                                           (const uint16_t*)bias, (uint16_t*)y,
                                           (hipStream_t)stream);
}

int fni8_moe_combine_f16(const void* y_sorted, int64_t H, const int32_t* topi,
                         const void* topw, const int32_t* pos, int64_t T, int64_t k,
                         void* out, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(y_sorted && topi && topw && pos && out, FNI8_ERR_NULL,
            "y_sorted, topi, topw, pos and out are required");
    REQUIRE(H > 0 && H < kMaxDim && T >= 0 && T < kMaxDim && k > 0 && k <= 32 &&
                T * k < kMaxDim,
            FNI8_ERR_SHAPE, "H=%lld T=%lld k=%lld out of range (k <= 32)", (long long)H,
            (long long)T, (long long)k);
    REQUIRE(aligned(y_sorted, 2) && aligned(topw, 2) && aligned(out, 2) && aligned(topi, 4) &&
                aligned(pos, 4),
            FNI8_ERR_ALIGN, "combine operands misaligned");
    int rc = check_device();
    if (rc) return rc;
    return fni8h::launch_moe_combine((const uint16_t*)y_sorted, H, topi, (const uint16_t*)topw,
                                     pos, T, k, (uint16_t*)out, (hipStream_t)stream);
}

int fni8_gemm_w4a8(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                   const uint8_t* w, const float* ws, int64_t N, int64_t G, const void* bias,
                   void* y, int64_t ldy, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(xq && xs, FNI8_ERR_NULL, "xq and xs are required");
    int rc = check_w4a8(M, K, N, G, w, ws, bias, y, ldy);
    if (rc) return rc;
    REQUIRE(ldq >= K, FNI8_ERR_STRIDE, "ldq=%lld < K=%lld", (long long)ldq, (long long)K);
    REQUIRE(ldq % 16 == 0 && aligned(xq, 16) && aligned(xs, 4), FNI8_ERR_ALIGN,
            "xq rows must be 16-byte aligned");
    rc = check_device();
    if (rc) return rc;
    return fni8h::launch_gemm_w4a8(xq, ldq, xs, M, K, w, ws, N, G, (const uint16_t*)bias,
                                   (uint16_t*)y, ldy, (hipStream_t)stream);
}

int fni8_linear_w4a8_f16(const void* x, int64_t ldx, int64_t M, int64_t K, const uint8_t* w,
                         const float* ws, int64_t N, int64_t G, const void* bias, void* y,
                         int64_t ldy, int8_t* xq, float* xs, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(x && xq && xs, FNI8_ERR_NULL, "x, xq and xs are required");
    int rc = check_w4a8(M, K, N, G, w, ws, bias, y, ldy);
    if (rc) return rc;
    REQUIRE(ldx >= K, FNI8_ERR_STRIDE, "ldx=%lld < K=%lld", (long long)ldx, (long long)K);
    REQUIRE(aligned(x, 2) && aligned(xq, 16) && aligned(xs, 4), FNI8_ERR_ALIGN,
            "x, xq or xs misaligned");
    rc = check_device();
    if (rc) return rc;
    hipStream_t st = (hipStream_t)stream;
    // decode sizes: one launch, the quantization fused into the stream kernel
    rc = fni8h::launch_linear_w4a8_fused((const uint16_t*)x, ldx, M, K, w, ws, N, G,
                                         (const uint16_t*)bias, (uint16_t*)y, ldy, xq, xs, st);
    if (rc != 1) return rc;
    rc = fni8h::launch_quant_rowwise((const uint16_t*)x, M, K, ldx, xq, K, xs, st);
    if (rc) return rc;
    return fni8h::launch_gemm_w4a8(xq, K, xs, M, K, w, ws, N, G, (const uint16_t*)bias,
                                   (uint16_t*)y, ldy, st);
}

int fni8_moe_route(const float* logits, int64_t T, int64_t E, int64_t ldl, int scoring,
                   const float* bias, int64_t groups, int64_t topk_group, int64_t k, int renorm,
                   float scale, void* topw, int32_t* topi, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(logits && topw && topi, FNI8_ERR_NULL, "logits, topw and topi are required");
    REQUIRE(T >= 0 && T < kMaxDim && E >= 1 && E <= 1024, FNI8_ERR_SHAPE,
            "T=%lld E=%lld out of range (E <= 1024)", (long long)T, (long long)E);
    REQUIRE(k >= 1 && k <= 32 && k <= E, FNI8_ERR_SHAPE, "k=%lld out of range (1..min(32, E))",
            (long long)k);
    REQUIRE(scoring == FNI8_SCORE_SOFTMAX || scoring == FNI8_SCORE_SIGMOID, FNI8_ERR_SHAPE,
            "unknown scoring function %d", scoring);
    REQUIRE(groups == 0 || (groups >= 1 && groups <= 64 && E % groups == 0 && topk_group >= 1 &&
                            topk_group <= groups),
            FNI8_ERR_SHAPE, "groups=%lld topk_group=%lld invalid for E=%lld", (long long)groups,
            (long long)topk_group, (long long)E);
    REQUIRE(scale == scale && scale > -__builtin_inff() && scale < __builtin_inff(),
            FNI8_ERR_SHAPE, "scale must be finite");
    REQUIRE(ldl >= E, FNI8_ERR_STRIDE, "ldl=%lld < E=%lld", (long long)ldl, (long long)E);
    REQUIRE(aligned(logits, 4) && aligned(bias, 4) && aligned(topw, 2) && aligned(topi, 4),
            FNI8_ERR_ALIGN, "router operands misaligned");
    int rc = check_device();
    if (rc) return rc;
    return fni8h::launch_moe_route(logits, ldl, T, E, scoring, bias, groups, topk_group, k,
                                   renorm ? 1 : 0, scale, (uint16_t*)topw, topi,
                                   (hipStream_t)stream);
}

int fni8_act_and_mul_f16(const void* x, int64_t ldx, int64_t M, int64_t I, int act, void* out,
                         int64_t ldo, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(x && out, FNI8_ERR_NULL, "x and out are required");
    REQUIRE(M >= 0 && M < kMaxDim && I > 0 && I < kMaxDim / 2, FNI8_ERR_SHAPE,
            "M=%lld I=%lld out of range", (long long)M, (long long)I);
    REQUIRE(act == FNI8_ACT_SILU || act == FNI8_ACT_GELU_TANH, FNI8_ERR_SHAPE,
            "unknown activation %d", act);
    REQUIRE(ldx >= 2 * I && ldo >= I, FNI8_ERR_STRIDE, "ldx=%lld < 2I or ldo=%lld < I",
            (long long)ldx, (long long)ldo);
    REQUIRE(aligned(x, 2) && aligned(out, 2), FNI8_ERR_ALIGN, "x or out misaligned");
    int rc = check_device();
    if (rc) return rc;
    return fni8h::launch_act_and_mul((const uint16_t*)x, ldx, M, I, act, (uint16_t*)out, ldo,
                                     (hipStream_t)stream);
}

int fni8_act_and_mul_quant_f16(const void* x, int64_t ldx, int64_t M, int64_t I, int act,
                               int8_t* xq, int64_t ldq, float* xs, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(x && xq && xs, FNI8_ERR_NULL, "x, xq and xs are required");
    REQUIRE(M >= 0 && M < kMaxDim && I > 0 && I < kMaxDim / 2 && I % 4 == 0, FNI8_ERR_SHAPE,
            "M=%lld I=%lld out of range (I a multiple of 4)", (long long)M, (long long)I);
    REQUIRE(act == FNI8_ACT_SILU || act == FNI8_ACT_GELU_TANH, FNI8_ERR_SHAPE,
            "unknown activation %d", act);
    REQUIRE(ldx >= 2 * I && ldq >= I, FNI8_ERR_STRIDE, "ldx=%lld < 2I or ldq=%lld < I",
            (long long)ldx, (long long)ldq);
    REQUIRE(aligned(x, 2) && aligned(xs, 4), FNI8_ERR_ALIGN, "x or xs misaligned");
    int rc = check_device();
    if (rc) return rc;
    return fni8h::launch_act_and_mul_quant((const uint16_t*)x, ldx, M, I, act, xq, ldq, xs,
                                           nullptr, 0, (hipStream_t)stream);
}

int fni8_act_and_mul_quant_f16_ws(const void* x, int64_t ldx, int64_t M, int64_t I, int act,
                                  int8_t* xq, int64_t ldq, float* xs, void* workspace,
                                  int64_t workspace_bytes, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(x && xq && xs, FNI8_ERR_NULL, "x, xq and xs are required");
    REQUIRE(M >= 0 && M < kMaxDim && I > 0 && I < kMaxDim / 2 && I % 4 == 0, FNI8_ERR_SHAPE,
            "M=%lld I=%lld out of range (I a multiple of 4)", (long long)M, (long long)I);
    REQUIRE(act == FNI8_ACT_SILU || act == FNI8_ACT_GELU_TANH, FNI8_ERR_SHAPE,
            "unknown activation %d", act);
    REQUIRE(ldx >= 2 * I && ldq >= I, FNI8_ERR_STRIDE, "ldx=%lld < 2I or ldq=%lld < I",
            (long long)ldx, (long long)ldq);
    REQUIRE(aligned(x, 2) && aligned(xs, 4), FNI8_ERR_ALIGN, "x or xs misaligned");
    REQUIRE(workspace_bytes >= 0 && (!workspace || aligned(workspace, 256)), FNI8_ERR_ALIGN,
            "workspace must be 256-byte aligned with a size >= 0");
    int rc = check_device();
    if (rc) return rc;
    return fni8h::launch_act_and_mul_quant((const uint16_t*)x, ldx, M, I, act, xq, ldq, xs,
                                           static_cast<int8_t*>(workspace),
                                           workspace ? workspace_bytes : 0, (hipStream_t)stream);
}

int64_t fni8_act_and_mul_quant_workspace_bytes(int64_t M, int64_t I) {
    if (M < 0 || I <= 0 || M >= kMaxDim || I >= kMaxDim / 2) return 0;
    return fni8h::act_quant_workspace_bytes(M, I);
}

int fni8_rmsnorm_f16(const void* x, int64_t ldx, const void* residual, int64_t ldr,
                     const void* weight, float eps, int unit_offset, int64_t M, int64_t K,
                     void* out, int64_t ldo, void* residual_out, int64_t ldro, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(out, FNI8_ERR_NULL, "out is required");
    int rc = check_rmsnorm(x, ldx, residual, ldr, weight, eps, M, K, ldo, residual_out, ldro);
    if (rc) return rc;
    REQUIRE(aligned(out, 2), FNI8_ERR_ALIGN, "out misaligned");
    rc = check_device();
    if (rc) return rc;
    return fni8h::launch_rmsnorm((const uint16_t*)x, ldx, (const uint16_t*)residual, ldr,
                                 (const uint16_t*)weight, eps, unit_offset ? 1 : 0, M, K,
                                 (uint16_t*)out, ldo,
                                 residual ? (uint16_t*)residual_out : nullptr, ldro, nullptr, 0,
                                 nullptr, (hipStream_t)stream);
}

int fni8_rmsnorm_quant_f16(const void* x, int64_t ldx, const void* residual, int64_t ldr,
                           const void* weight, float eps, int unit_offset, int64_t M, int64_t K,
                           int8_t* xq, int64_t ldq, float* xs, void* residual_out,
                           int64_t ldro, void* stream) {
    fni8h::g_detail[0] = 0;
    REQUIRE(xq && xs, FNI8_ERR_NULL, "xq and xs are required");
    int rc = check_rmsnorm(x, ldx, residual, ldr, weight, eps, M, K, ldq, residual_out, ldro);
    if (rc) return rc;
    REQUIRE(K % 4 == 0, FNI8_ERR_SHAPE, "K=%lld is not a multiple of 4", (long long)K);
    REQUIRE(aligned(xs, 4), FNI8_ERR_ALIGN, "xs misaligned");
    rc = check_device();
    if (rc) return rc;
    return fni8h::launch_rmsnorm((const uint16_t*)x, ldx, (const uint16_t*)residual, ldr,
                                 (const uint16_t*)weight, eps, unit_offset ? 1 : 0, M, K, nullptr,
                                 0, residual ? (uint16_t*)residual_out : nullptr, ldro, xq, ldq,
                                 xs, (hipStream_t)stream);
}

}  // extern "C"
