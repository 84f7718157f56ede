/*
 * fni8amd: C ABI of the MI355X (gfx950) W8A8 linear kernels.
 *
 * The reference (Josephur/fni8-serve) reaches its int8 arithmetic through the
 * Python call `fni8.linear(x, qt, bias=...)` at fni8serve/layers/linear.py:69;
 * `fni8` is a closed CUDA wheel (v0.1.0-rc2) with no C interface of its own.
 * These entry points are what a binding of that call needs: plain device
 * pointers, sizes and a stream, no framework types.
 *
 * Conventions shared by every entry point:
 *   - Pointers are device pointers on the current HIP device; `stream` is a
 *     hipStream_t (NULL = the legacy default stream).  Work is enqueued on
 *     `stream`; nothing synchronises the host.
 *   - The library allocates no device memory; every buffer comes from the
 *     caller, so calls can be captured in a HIP graph.  Calls are reentrant.
 *     Mutable global state: the per-GPU scratch of
 *     fni8_linear_w8a8_f16_noalloc (below), which only that entry point uses,
 *     and the process-wide settings of the fni8_debug_* test hooks.
 *   - fp16 tensors are IEEE binary16 passed as `void*` / `uint16_t*`.
 *   - Weights follow the per_row_i8 QTensor layout (models/weights.py:18-25):
 *     data int8 [N, K] row-major (K contiguous), scale fp32 [N].
 *   - Arithmetic: per-token quantization s = max(amax, 1e-6) / 127 in fp32,
 *     q = clamp(rint(x / s), -127, 127) with correctly rounded division and
 *     ties to even; exact int32 accumulation; epilogue
 *     y = fp16(((float)acc * s_x[m]) * s_w[n] (+ bias[n])) with one rounding
 *     per operation.
 *   - Return 0 on success, a negative FNI8_ERR_* code otherwise.  Argument
 *     errors are detected before anything is launched.
 */
#ifndef FNI8AMD_H
#define FNI8AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
    FNI8_OK = 0,
    FNI8_ERR_NULL = -1,      /* a required pointer is NULL */
    FNI8_ERR_SHAPE = -2,     /* M, N, K, E, T or k out of range; K % 4 != 0 */
    FNI8_ERR_ALIGN = -3,     /* a pointer or stride breaks the alignment rule */
    FNI8_ERR_STRIDE = -4,    /* a leading dimension is smaller than the row */
    FNI8_ERR_LAUNCH = -5,    /* the HIP runtime reported an error */
    FNI8_ERR_DEVICE = -6     /* the current device is not gfx950 */
};

/* Human-readable text for an FNI8_ERR_* code. */
const char* fni8_strerror(int code);

/* Detail of the last error raised on the calling thread ("" if none). */
const char* fni8_last_error(void);

/* Library version string. */
const char* fni8_version(void);

/*
 * Optional set-up, no counterpart in the reference: checks every visible
 * gfx950 device and looks up, with that device current, the address of the
 * per-GPU scratch that fni8_linear_w8a8_f16_noalloc uses.  Every entry point
 * does the same for the current device on its first call there, so only a
 * caller whose first call on a device may happen under HIP graph capture needs
 * it (call it before capturing).  Restores the current device.
 */
int fni8_init(void);

/*
 * Per-token symmetric activation quantization: step 1 of `fni8.linear`
 * (replaces the quantize half of fni8.linear, fni8serve/layers/linear.py:69;
 * semantics linear.py:5-10).
 *   x   fp16 [M, K], row stride ldx elements (ldx >= K)
 *   xq  int8 [M, K], row stride ldq bytes (ldq >= K)
 *   xs  fp32 [M]: the per-row scale
 * K must be a multiple of 4 (the reference's quantizable-linear rule,
 * fni8serve/convert.py:128).
 */
int fni8_quantize_rowwise_f16(const void* x, int64_t M, int64_t K, int64_t ldx,
                              int8_t* xq, int64_t ldq, float* xs, void* stream);

/*
 * int8 x int8 -> int32 GEMM with the fused dequant epilogue: `gemm_w8a8`
 * (replaces the GEMM half of fni8.linear for per_row_i8 weights,
 * fni8serve/layers/linear.py:9 and :69).
 *   xq      int8 [M, K], row stride ldq bytes; xs fp32 [M]
 *   w       int8 [N, K] (row stride K); ws fp32 [N]
 *   bias    fp16 [N] or NULL
 *   y       fp16 [M, N], row stride ldy elements
 *   acc_out int32 [M, N] (row stride N) or NULL: the raw accumulators, for
 *           parity checks
 */
int fni8_gemm_w8a8(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                   const int8_t* w, const float* ws, int64_t N, const void* bias, void* y,
                   int64_t ldy, int32_t* acc_out, void* stream);

/*
 * fni8_gemm_w8a8 with a workspace (replaces the same GEMM half of
 * fni8serve/layers/linear.py:69 at prefill sizes): the same arithmetic and
 * outputs, bit for bit.  Where the output has too few 256-wide tiles to fill
 * the GPU (e.g. Qwen3-8B's down projection, K = 12288, at M = 512 and 2048) the
 * workgroups of one tile split K between them and hand their int32 partial
 * tiles over through `workspace`.
 *   workspace  device memory, 256-byte aligned, at least
 *              fni8_linear_workspace_bytes(M, N, K) bytes; any contents;
 *              NULL or too small = no split.  One workspace per stream.
 */
int fni8_gemm_w8a8_ws(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                      const int8_t* w, const float* ws, int64_t N, const void* bias, void* y,
                      int64_t ldy, int32_t* acc_out, void* workspace, int64_t workspace_bytes,
                      void* stream);

/*
 * The whole W8A8 linear, `fni8.linear(x, qt, bias)` for a per_row_i8 QTensor
 * (replaces fni8serve/layers/linear.py:69): quantize x per token, int8 GEMM
 * against w, dequant epilogue to fp16.
 *   x    fp16 [M, K], row stride ldx elements (covers the non-contiguous
 *        `hidden[:, -1]` input of fni8serve/layers/embedding.py:49-53)
 *   xq   int8 [M, K] and xs fp32 [M]: caller-provided buffers that receive the
 *        quantized activations and their scales
 *   y    fp16 [M, N], row stride ldy elements; acc_out as in fni8_gemm_w8a8
 */
int fni8_linear_w8a8_f16(const void* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                         const float* ws, int64_t N, const void* bias, void* y, int64_t ldy,
                         int8_t* xq, float* xs, int32_t* acc_out, void* stream);

/*
 * fni8_linear_w8a8_f16 with a workspace: the same call, arithmetic and
 * outputs (bit for bit), faster where the workspace helps (replaces
 * fni8serve/layers/linear.py:69).  At decode batch sizes -- 5 <= M <= 16 tokens
 * on QKV- and down-shaped weights, 5 <= M <= 8 on O-shaped ones -- one launch
 * instead of two: the per-token quantization runs once per XCD and reaches the
 * GEMM workgroups through that XCD's L2, and `workspace` holds the exchanged
 * rows.  At prefill sizes the GEMM may split K as fni8_gemm_w8a8_ws does.
 * Other shapes take the same launches as fni8_linear_w8a8_f16.
 *   workspace        device memory, 256-byte aligned, at least
 *                    fni8_linear_workspace_bytes(M, N, K) bytes; any contents
 *                    (nothing needs clearing, before the first call or
 *                    between calls); NULL or too small = the two-launch path
 *   Two calls that may run at the same time must not share a workspace (one
 *   workspace per stream), as they must not share xq / xs.
 */
int fni8_linear_w8a8_f16_ws(const void* x, int64_t ldx, int64_t M, int64_t K, const int8_t* w,
                            const float* ws, int64_t N, const void* bias, void* y, int64_t ldy,
                            int8_t* xq, float* xs, int32_t* acc_out, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * Workspace bytes fni8_linear_w8a8_f16_ws and fni8_gemm_w8a8_ws use for M
 * tokens, N outputs and K inputs (0: no workspace is used).
 *   M <= 16: 8 * (2304 + M * K rounded up to 256) where the one-launch path
 *     takes the shape (5 <= M <= 16 with 4096 < N < 16384 and K = 4096, or
 *     N <= 4096 and K = 12288; 5 <= M <= 8 with N <= 4096 and K = 4096), at
 *     most 8 * (2304 + 16 * 12288) = 1,591,296; fni8_gemm_w8a8_ws uses none.
 *   M > 64: where the prefill GEMM splits K (down-shaped weights, K = 12288,
 *     below M = 4096), 8 regions of one 128-byte flag per output tile and
 *     split (rounded up to 256 bytes) plus `split` - 1 int32 partial tiles per
 *     output tile -- 32 MiB + 256 KiB for [2048, 12288] x [4096, 12288],
 *     24 MiB + 256 KiB at M = 512, 12 MiB + 512 KiB at M = 256.
 */
int64_t fni8_linear_workspace_bytes(int64_t M, int64_t N, int64_t K);

/*
 * Test hook, no counterpart in the reference: the bound, in ticks of the
 * 100 MHz real-time counter, on the two waits for data handed over inside one
 * XCD -- a GEMM workgroup of the one-launch decode path waiting for its XCD's
 * quantized rows (it then quantizes them itself), and the owner of a split-K
 * prefill tile waiting for its partners' partial tiles (it then recomputes the
 * tile over the whole K range).  Default 10000 = 100 us; a negative value
 * restores it.  0 makes every wait that does not succeed at its first look take
 * the fallback, which must give the same bits.  Process-wide; affects later
 * launches.
 */
void fni8_debug_coop_wait_ticks(int64_t ticks);

/*
 * Test hook, no counterpart in the reference: forces the prefill GEMM's output
 * tile (bm x bn: 256x256, 256x192, 128x256, 256x128 or 64x128) and split-K factor
 * (1, 2 or 4; 1 for 256x192) on every later launch whose shape allows it
 * (K / 128 a multiple of the split, the tile count a multiple of 8 and a big
 * enough workspace when split > 1); other values restore the automatic choice.
 * The output is the same bits under every plan.  Process-wide.
 */
void fni8_debug_gemm_plan(int64_t bm, int64_t bn, int64_t split);

/*
 * fni8_linear_w8a8_f16 for callers that cannot allocate (code under HIP graph
 * capture, tight serving loops, harnesses that forbid allocation).  No
 * counterpart in the reference.  Same arithmetic and output as
 * fni8_linear_w8a8_f16 (without the accumulator output); the quantized
 * activations and their scales go to a scratch array inside the library
 * (48 MiB plus 256 KiB per GPU, resident until the process ends) instead of
 * caller buffers, and the call allocates nothing.
 *   Limits: M <= 65536 and M * K <= 48 MiB (every Qwen3-8B linear up to
 *   M = 4096); larger shapes return FNI8_ERR_SHAPE.
 *   Every call on a GPU shares that GPU's scratch: calls that overlap on one
 *   GPU (different streams without ordering, several host threads) race.
 */
int fni8_linear_w8a8_f16_noalloc(const void* x, int64_t ldx, int64_t M, int64_t K,
                                 const int8_t* w, const float* ws, int64_t N, const void* bias,
                                 void* y, int64_t ldy, void* stream);

/*
 * Routing sort for the grouped expert GEMM (replaces the per-expert
 * `mask = topi == e; mask.nonzero()` gathers of SparseMoE.forward,
 * fni8serve/models/moe.py:100-103).  A stable counting sort of the T*k
 * (token, slot) pairs by expert id: inside each expert's segment the rows are
 * in ascending token, then slot, order, as nonzero() returns them.
 *   topi       int32 [T, k] expert ids in [0, E)
 *   seg_off    int32 [E + 1]: segment offsets, seg_off[E] = T*k
 *   row_token  int32 [T*k]: token of each sorted row
 *   pos        int32 [T, k]: sorted row of each (token, slot)
 * Expert ids outside [0, E) are not detected on the device; they are skipped.
 */
int fni8_moe_sort(const int32_t* topi, int64_t T, int64_t k, int64_t E, int32_t* seg_off,
                  int32_t* row_token, int32_t* pos, void* stream);

/*
 * Grouped W8A8 GEMM over expert segments: all experts' `gemm_w8a8` calls of
 * one projection in one launch (replaces the expert loop's linears,
 * fni8serve/models/moe.py:104 via layers/mlp.py:39-40; the reference notes
 * the kernel as future work at moe.py:9-11).
 *   aq, as     int8 [rows, K] (row stride K) and fp32 [rows]: quantized
 *              activations
 *   row_index  int32 [R] or NULL: sorted row r reads activation row
 *              row_index[r] (the token gather); NULL reads row r
 *   w, ws      int8 [E, N, K] and fp32 [E, N]: stacked expert weights
 *   seg_off    int32 [E + 1] from fni8_moe_sort; R = seg_off[E] on the device,
 *              R_max bounds it (the launch is sized from R_max)
 *   bias       fp16 [E, N] or NULL
 *   y          fp16 [R_max, N] (rows >= R are not written); acc_out int32 [R_max, N] or NULL
 */
int fni8_gemm_w8a8_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                           int64_t R_max, int64_t K, const int8_t* w, const float* ws,
                           int64_t E, int64_t N, const int32_t* seg_off, const void* bias,
                           void* y, int32_t* acc_out, void* stream);

/*
 * Grouped W4A8 GEMM over expert segments: all per_group_i4 experts'
 * `gemm_w4a8` calls of one projection in one launch (replaces the expert
 * loop's linears on int4 experts, fni8serve/models/moe.py:104 via
 * layers/mlp.py:39-40; experts of any QTensor scheme, moe.py:56, and the
 * converter's per_group_i4 experts, convert.py:130-131).
 *   aq, as     int8 [rows, K] (row stride K, 16-byte aligned) and fp32 [rows]
 *   row_index  int32 [R] or NULL: sorted row r reads activation row
 *              row_index[r]; NULL reads row r
 *   w, ws      uint8 [E, N, K/2] (packed as in fni8_gemm_w4a8, 16-byte aligned)
 *              and fp32 [E, N, K/G]: stacked expert weights and group scales
 *   G          64, 128 or 256; K a multiple of 256; N < 2^21
 *   seg_off    int32 [E + 1] from fni8_moe_sort; R = seg_off[E] on the device,
 *              R_max bounds it
 *   bias       fp16 [E, N] or NULL
 *   y          fp16 [R_max, N] in sorted-row order (rows >= R are not written)
 * Per output element the arithmetic of fni8_gemm_w4a8.
 */
int fni8_gemm_w4a8_grouped(const int8_t* aq, const float* as, const int32_t* row_index,
                           int64_t R_max, int64_t K, const uint8_t* w, const float* ws,
                           int64_t E, int64_t N, int64_t G, const int32_t* seg_off,
                           const void* bias, void* y, void* stream);

/*
 * Weighted combine of expert outputs (replaces moe.py:105's
 * `out.index_add_(0, tok_idx, contrib * topw[tok_idx, slot])` over the
 * expert loop): out[t] = sum over the token's slots, in ascending expert id,
 * of fp16(y_sorted[pos[t, j]] * topw[t, j]), accumulated from +0 in fp16.
 *   y_sorted  fp16 [T*k, H]; topi int32 [T, k]; topw fp16 [T, k]; pos int32 [T, k]
 *   out       fp16 [T, H]
 */
int fni8_moe_combine_f16(const void* y_sorted, int64_t H, const int32_t* topi,
                         const void* topw, const int32_t* pos, int64_t T, int64_t k,
                         void* out, void* stream);

/*
 * W4A8 GEMM: int8 activations against per_group_i4 int4 weights, `gemm_w4a8`
 * (replaces the GEMM half of fni8.linear for int4 QTensors,
 * fni8serve/layers/linear.py:9 and :63-65; weight format
 * fni8serve/convert.py:69-79).
 *   xq        int8 [M, K], row stride ldq bytes (a multiple of 16, base 16-byte
 *             aligned); xs fp32 [M]
 *   w         uint8 [N, K/2]: code k of row n in byte k/2, low nibble for even
 *             k, 4-bit two's complement; 16-byte aligned
 *   ws        fp32 [N, K/G]: one scale per group of G consecutive k
 *   G         32, 64, 128 or 256, dividing K; K a multiple of 32
 *   bias      fp16 [N] or NULL; y fp16 [M, N], row stride ldy
 * Arithmetic: per group the exact int32 sum acc_g; accf = fma(acc_g, ws[n, g],
 * accf) in ascending g from +0; y = fp16(accf * xs[m] (+ bias[n])).
 */
int fni8_gemm_w4a8(const int8_t* xq, int64_t ldq, const float* xs, int64_t M, int64_t K,
                   const uint8_t* w, const float* ws, int64_t N, int64_t G, const void* bias,
                   void* y, int64_t ldy, void* stream);

/*
 * The whole W4A8 linear, `fni8.linear(x, qt, bias)` for a per_group_i4 int4
 * QTensor (replaces fni8serve/layers/linear.py:69 on that scheme): per-token
 * quantization of x as in fni8_quantize_rowwise_f16, then fni8_gemm_w4a8.
 *   x      fp16 [M, K], row stride ldx; xq int8 [M, K] (row stride K) and
 *          xs fp32 [M] receive the quantized activations
 */
int fni8_linear_w4a8_f16(const void* x, int64_t ldx, int64_t M, int64_t K, const uint8_t* w,
                         const float* ws, int64_t N, int64_t G, const void* bias, void* y,
                         int64_t ldy, int8_t* xq, float* xs, void* stream);

/* Router scoring functions of fni8_moe_route. */
enum {
    FNI8_SCORE_SOFTMAX = 0, /* softmax over all experts (Qwen, Hunyuan, MiniMax) */
    FNI8_SCORE_SIGMOID = 1  /* sigmoid per expert (GLM, DeepSeek, LFM2) */
};

/*
 * MoE router, one launch: scores, optional selection bias, optional
 * group-limited mask, top-k, weights (replaces the routing of
 * SparseMoE.forward, fni8serve/models/moe.py:62-97, and the torch.topk /
 * gather / renormalisation launches it makes; no host synchronisation, so an
 * MoE layer can be captured in a HIP graph).
 *   logits      fp32 [T, E] router logits, row stride ldl (>= E); E <= 1024
 *   scoring     FNI8_SCORE_SOFTMAX or FNI8_SCORE_SIGMOID
 *   bias        fp32 [E] added to the scores for selection only, or NULL
 *   groups      0, or the number of expert groups (<= 64, dividing E): only
 *               experts of the topk_group best groups (group score = max of
 *               the biased scores) are selectable
 *   k           experts per token, 1 <= k <= min(32, E)
 *   renorm      non-zero: weights divided by max(their sum, 1e-9)
 *   scale       routed scaling factor applied last
 *   topw        fp16 [T, k]: softmax -> the selected scores; sigmoid -> the
 *               selected unbiased scores; topi int32 [T, k], best first
 * Arithmetic is fp32 with one rounding per operation; softmax sums in a
 * fixed order, exp is the activations' Cody-Waite exp.  Top-k order: larger
 * score first, NaN above +inf, ties to the lower expert index, -0 as +0 (the
 * order torch.topk gives).
 */
int fni8_moe_route(const float* logits, int64_t T, int64_t E, int64_t ldl, int scoring,
                   const float* bias, int64_t groups, int64_t topk_group, int64_t k, int renorm,
                   float scale, void* topw, int32_t* topi, void* stream);

/* Gated activations of act_and_mul. */
enum {
    FNI8_ACT_SILU = 0,      /* "silu": g * sigmoid(g) */
    FNI8_ACT_GELU_TANH = 1  /* "gelu_tanh": 0.5 g (1 + tanh(sqrt(2/pi) (g + 0.044715 g^3))) */
};

/*
 * Arithmetic of the activations (fp32, one rounding per operation): the gate
 * is g * sigmoid(z), evaluated as g / (1 + exp(-z)) with z = g (silu) or
 * z = 2 sqrt(2/pi) (g + 0.044715 g^3) (gelu_tanh, the same value as the tanh
 * form); -z is clamped to [-86, 88] and exp is a Cody-Waite reduction with a
 * degree-7 Taylor polynomial (error below 2 ulp).  out = fp16(gate * up).
 */

/*
 * act_and_mul over a merged gate_up row: `fni8.act_and_mul(x, "silu" |
 * "gelu_tanh")` (replaces fni8serve/layers/activation.py:24 and :40).
 *   x    fp16 [M, 2I], row stride ldx elements: gate = x[:, :I], up = x[:, I:]
 *   act  FNI8_ACT_SILU or FNI8_ACT_GELU_TANH
 *   out  fp16 [M, I], row stride ldo elements (must not overlap x)
 */
int fni8_act_and_mul_f16(const void* x, int64_t ldx, int64_t M, int64_t I, int act, void* out,
                         int64_t ldo, void* stream);

/*
 * act_and_mul with the per-token quantization of the down projection fused
 * in: the int8 rows and scales are bit-identical to fni8_act_and_mul_f16
 * followed by fni8_quantize_rowwise_f16, without the fp16 [M, I] round trip
 * (replaces activation.py:24 and the quantize half of down_proj's
 * fni8.linear, fni8serve/layers/mlp.py:39-40 -> linear.py:69).  Feed xq/xs to
 * fni8_gemm_w8a8 or fni8_gemm_w8a8_grouped.
 *   xq   int8 [M, I], row stride ldq bytes; xs fp32 [M]
 * I must be a multiple of 4.
 */
int fni8_act_and_mul_quant_f16(const void* x, int64_t ldx, int64_t M, int64_t I, int act,
                               int8_t* xq, int64_t ldq, float* xs, void* stream);

/*
 * fni8_act_and_mul_quant_f16 with a workspace (same arithmetic and outputs, bit
 * for bit; replaces the same step, fni8serve/layers/mlp.py:39-40 -> linear.py:69).
 * For few rows (M <= 128) several workgroups share a row,
 * each activating a part of it, and exchange their partial row maxima through
 * `workspace` inside one XCD (a part that does not arrive in time is recomputed,
 * so the bits never depend on it).
 *   workspace  device memory, 256-byte aligned, at least
 *              fni8_act_and_mul_quant_workspace_bytes(M, I) bytes; any contents;
 *              NULL or too small = one workgroup per row.  One per stream.
 */
int fni8_act_and_mul_quant_f16_ws(const void* x, int64_t ldx, int64_t M, int64_t I, int act,
                                  int8_t* xq, int64_t ldq, float* xs, void* workspace,
                                  int64_t workspace_bytes, void* stream);

/*
 * Workspace bytes of fni8_act_and_mul_quant_f16_ws: 8 * (M rounded up to 8) *
 * G * 128, G = ceil(I / 2048) parts per row where 2 <= G <= 8 and M <= 128,
 * else 0 (e.g. 393,216 for M = 64, I = 12288).
 */
int64_t fni8_act_and_mul_quant_workspace_bytes(int64_t M, int64_t I);

/*
 * RMSNorm: `fni8.rmsnorm(x, weight, eps, residual=, unit_offset=)` (replaces
 * fni8serve/layers/norm.py:51-52; semantics of its eager form norm.py:37-58).
 *   h = residual ? fp16(x + residual) : x
 *   out = fp16((h * r) * w), r = 1 / sqrt(sum(h^2) / K + eps), w = weight or,
 *         with unit_offset, 1 + weight (Gemma), all in fp32
 * The sum of squares runs in a fixed order: 8-element chunks dealt round-robin
 * to 256 accumulators, a butterfly within each group of 64, then
 * (w0 + w1) + (w2 + w3).
 *   x, residual (or NULL)  fp16 [M, K], row strides ldx, ldr elements
 *   weight                 fp16 [K]
 *   out                    fp16 [M, K], row stride ldo
 *   residual_out           fp16 [M, K] (stride ldro) receiving h, or NULL;
 *                          ignored without residual
 * Outputs must not overlap inputs.
 */
int fni8_rmsnorm_f16(const void* x, int64_t ldx, const void* residual, int64_t ldr,
                     const void* weight, float eps, int unit_offset, int64_t M, int64_t K,
                     void* out, int64_t ldo, void* residual_out, int64_t ldro, void* stream);

/*
 * RMSNorm with the per-token quantization of the next linear (QKV, gate_up)
 * fused in: xq/xs are bit-identical to fni8_rmsnorm_f16 followed by
 * fni8_quantize_rowwise_f16 (replaces norm.py:51-52 and the quantize half of
 * the following fni8.linear, linear.py:69).
 *   xq int8 [M, K] (row stride ldq bytes), xs fp32 [M]; K a multiple of 4
 */
int fni8_rmsnorm_quant_f16(const void* x, int64_t ldx, const void* residual, int64_t ldr,
                           const void* weight, float eps, int unit_offset, int64_t M, int64_t K,
                           int8_t* xq, int64_t ldq, float* xs, void* residual_out,
                           int64_t ldro, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FNI8AMD_H */
