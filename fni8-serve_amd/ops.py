"""Tensor-level entry points over the C ABI (libfni8amd.so).

`linear(x, qt, bias=None)` is the drop-in for `fni8.linear`, the one call the
reference's W8A8 seam makes (fni8serve/layers/linear.py:69): per-token int8
quantization of x, the int8 GEMM against a per_row_i8 QTensor, and the fused
dequant epilogue to fp16.  The other functions expose the pieces (for the
grouped MoE path and for parity checks).

Every function launches on `torch.cuda.current_stream()` of the operands'
device, allocates its outputs and scratch from torch's caching allocator, and
never synchronises, so the calls can be captured in a HIP graph.  GPU tensors
are required: there is no CPU or PyTorch fallback here.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib
from .qtensor import QTensor

_f16 = torch.float16


def _stream(dev: torch.device) -> ctypes.c_void_p:
    return ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)


def _ptr(t: torch.Tensor | None):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _require_cuda(name: str, *ts):
    dev = None
    for t in ts:
        if t is None:
            continue
        if not t.is_cuda:
            raise ValueError(f"{name}: every tensor must be on the GPU (got {t.device})")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"{name}: tensors on different devices ({dev} vs {t.device})")
    return dev


def _rows(x: torch.Tensor, K: int):
    """View x[..., K] as 2-D rows with unit inner stride; returns (x2, ldx)."""
    if x.stride(-1) != 1:
        x = x.contiguous()
    x2 = x.reshape(-1, K)
    if x2.stride(1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < K):
        x2 = x2.contiguous()
    ldx = x2.stride(0) if x2.shape[0] > 1 else K
    return x2, ldx


def _check_weight(qt: QTensor, K: int):
    if qt.scheme != "per_row_i8":
        raise ValueError(f"W8A8 linear cannot use scheme {qt.scheme!r}")
    w, s = qt.data, qt.scale
    if w.dtype != torch.int8 or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("per_row_i8 data must be a contiguous int8 [N, K] tensor")
    if w.shape[1] != K:
        raise ValueError(f"in_features mismatch: x has K={K}, weight has {w.shape[1]}")
    if s is None or s.dtype != torch.float32 or s.numel() != w.shape[0] or not s.is_contiguous():
        raise ValueError("per_row_i8 scale must be a contiguous fp32 tensor with N entries")
    return w, s.reshape(-1)


def _check_bias(bias: torch.Tensor | None, N: int):
    if bias is None:
        return None
    if bias.dtype != _f16 or bias.numel() != N:
        raise ValueError("bias must be an fp16 tensor with N entries")
    return bias.reshape(-1).contiguous()


W4_GROUPS = (32, 64, 128, 256)


def _check_weight_i4(qt: QTensor, K: int):
    """per_group_i4 int4 weight (fni8serve/convert.py:69-79): packed uint8
    [N, K/2], fp32 scales [N, K/G]."""
    if qt.codebook != "int4":
        raise ValueError(f"the W4A8 kernel needs the int4 codebook (got {qt.codebook!r}); "
                         "NF4 weights take the dequantize path")
    w, s, G = qt.data, qt.scale, qt.group_size
    if w.dtype != torch.uint8 or w.dim() != 2 or not w.is_contiguous():
        raise ValueError("per_group_i4 data must be a contiguous uint8 [N, K/2] tensor")
    if 2 * w.shape[1] != K:
        raise ValueError(f"in_features mismatch: x has K={K}, weight packs {2 * w.shape[1]}")
    if G not in W4_GROUPS or K % G or K % 32:
        raise ValueError(f"group size {G} with K={K} not supported (G in {W4_GROUPS}, "
                         "dividing K; K a multiple of 32)")
    N = w.shape[0]
    if s is None or s.dtype != torch.float32 or s.numel() != N * (K // G) or not s.is_contiguous():
        raise ValueError("per_group_i4 scale must be a contiguous fp32 tensor of N * K/G entries")
    return w, s.reshape(N, K // G), G


def _linear_w4a8(x, qt, bias):
    K = x.shape[-1]
    w, ws, G = _check_weight_i4(qt, K)
    N = w.shape[0]
    bias = _check_bias(bias, N)
    dev = _require_cuda("linear", x, w, ws, bias)
    if x.dtype != _f16:
        raise ValueError(f"linear expects fp16 activations (got {x.dtype})")
    x2, ldx = _rows(x, K)
    M = x2.shape[0]
    y = torch.empty((*x.shape[:-1], N), dtype=_f16, device=dev)
    xq = torch.empty((M, K), dtype=torch.int8, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    if M:
        with torch.cuda.device(dev):
            _lib.call("fni8_linear_w4a8_f16", _ptr(x2), ldx, M, K, _ptr(w), _ptr(ws), N, G,
                      _ptr(bias), _ptr(y), N, _ptr(xq), _ptr(xs), _stream(dev))
    return y, xq, xs, None


def linear_with_intermediates(x: torch.Tensor, qt: QTensor, bias: torch.Tensor | None = None,
                              want_acc: bool = False):
    """`linear` that also returns the quantized activations, their scales and
    (if want_acc) the int32 accumulators: (y, xq [M, K], xs [M], acc [M, N] | None).
    For per_group_i4 weights the accumulators are per group and not returned."""
    if qt.scheme == "per_group_i4":
        return _linear_w4a8(x, qt, bias)
    K = x.shape[-1]
    w, ws = _check_weight(qt, K)
    N = w.shape[0]
    bias = _check_bias(bias, N)
    dev = _require_cuda("linear", x, w, ws, bias)
    if x.dtype != _f16:
        raise ValueError(f"linear expects fp16 activations (got {x.dtype})")
    x2, ldx = _rows(x, K)
    M = x2.shape[0]
    y = torch.empty((*x.shape[:-1], N), dtype=_f16, device=dev)
    xq = torch.empty((M, K), dtype=torch.int8, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    acc = torch.empty((M, N), dtype=torch.int32, device=dev) if want_acc else None
    if M == 0:
        return y, xq, xs, acc
    # 5..16 tokens on the narrower weights: the one-launch path exchanges the
    # quantized rows through a workspace; prefill shapes with too few output
    # tiles split K and exchange partial tiles through it.  It comes from the
    # caching allocator like every other buffer: torch hands a block back to the
    # same stream only, after the work queued on it, so no two calls that can
    # overlap share one; its contents never matter, so it is not cleared.
    nw = _lib.workspace_bytes(M, N, K)
    work = torch.empty(nw, dtype=torch.uint8, device=dev) if nw else None
    with torch.cuda.device(dev):
        _lib.call("fni8_linear_w8a8_f16_ws", _ptr(x2), ldx, M, K, _ptr(w), _ptr(ws), N,
                  _ptr(bias), _ptr(y), N, _ptr(xq), _ptr(xs), _ptr(acc), _ptr(work), nw,
                  _stream(dev))
    return y, xq, xs, acc


def linear(x: torch.Tensor, qt: QTensor, bias: torch.Tensor | None = None) -> torch.Tensor:
    """fni8.linear(x, qt, bias=None): x fp16 [..., K] on the GPU -> fp16 [..., N],
    for per_row_i8 (W8A8) and per_group_i4 int4 (W4A8) weights."""
    return linear_with_intermediates(x, qt, bias)[0]


def quantize_rowwise(x: torch.Tensor):
    """Per-token quantization of fp16 x [..., K] -> (xq int8 [M, K], xs fp32 [M])."""
    K = x.shape[-1]
    dev = _require_cuda("quantize_rowwise", x)
    if x.dtype != _f16:
        raise ValueError(f"quantize_rowwise expects fp16 (got {x.dtype})")
    x2, ldx = _rows(x, K)
    M = x2.shape[0]
    xq = torch.empty((M, K), dtype=torch.int8, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    if M:
        with torch.cuda.device(dev):
            _lib.call("fni8_quantize_rowwise_f16", _ptr(x2), M, K, ldx, _ptr(xq), K, _ptr(xs),
                      _stream(dev))
    return xq, xs


def gemm_w8a8(xq: torch.Tensor, xs: torch.Tensor, qt: QTensor, bias: torch.Tensor | None = None,
              want_acc: bool = False):
    """`gemm_w8a8` on already-quantized activations: xq int8 [M, K], xs fp32 [M]
    -> y fp16 [M, N] (and the int32 accumulators if want_acc)."""
    if xq.dtype != torch.int8 or xq.dim() != 2 or xq.stride(1) != 1:
        raise ValueError("xq must be int8 [M, K] with unit inner stride")
    M, K = xq.shape
    w, ws = _check_weight(qt, K)
    N = w.shape[0]
    bias = _check_bias(bias, N)
    if xs.dtype != torch.float32 or xs.numel() != M or not xs.is_contiguous():
        raise ValueError("xs must be a contiguous fp32 tensor with M entries")
    dev = _require_cuda("gemm_w8a8", xq, xs, w, ws, bias)
    y = torch.empty((M, N), dtype=_f16, device=dev)
    acc = torch.empty((M, N), dtype=torch.int32, device=dev) if want_acc else None
    if M:
        ldq = xq.stride(0) if M > 1 else K
        # split-K workspace for prefill shapes with too few output tiles
        nw = _lib.workspace_bytes(M, N, K)
        work = torch.empty(nw, dtype=torch.uint8, device=dev) if nw else None
        with torch.cuda.device(dev):
            _lib.call("fni8_gemm_w8a8_ws", _ptr(xq), ldq, _ptr(xs), M, K, _ptr(w), _ptr(ws), N,
                      _ptr(bias), _ptr(y), N, _ptr(acc), _ptr(work), nw, _stream(dev))
    return (y, acc) if want_acc else y


def gemm_w4a8(xq: torch.Tensor, xs: torch.Tensor, qt: QTensor,
              bias: torch.Tensor | None = None) -> torch.Tensor:
    """`gemm_w4a8` on already-quantized activations: xq int8 [M, K], xs fp32 [M]
    and a per_group_i4 int4 QTensor -> y fp16 [M, N]."""
    if xq.dtype != torch.int8 or xq.dim() != 2 or xq.stride(1) != 1:
        raise ValueError("xq must be int8 [M, K] with unit inner stride")
    M, K = xq.shape
    w, ws, G = _check_weight_i4(qt, K)
    N = w.shape[0]
    bias = _check_bias(bias, N)
    if xs.dtype != torch.float32 or xs.numel() != M or not xs.is_contiguous():
        raise ValueError("xs must be a contiguous fp32 tensor with M entries")
    dev = _require_cuda("gemm_w4a8", xq, xs, w, ws, bias)
    y = torch.empty((M, N), dtype=_f16, device=dev)
    if M:
        ldq = xq.stride(0) if M > 1 else K
        if ldq % 16 or xq.data_ptr() % 16:
            xq, ldq = xq.contiguous(), K
        with torch.cuda.device(dev):
            _lib.call("fni8_gemm_w4a8", _ptr(xq), ldq, _ptr(xs), M, K, _ptr(w), _ptr(ws), N, G,
                      _ptr(bias), _ptr(y), N, _stream(dev))
    return y


def gemm_quantized(xq: torch.Tensor, xs: torch.Tensor, qt: QTensor,
                   bias: torch.Tensor | None = None) -> torch.Tensor:
    """The GEMM of `linear` for either weight scheme on pre-quantized activations."""
    if qt.scheme == "per_group_i4":
        return gemm_w4a8(xq, xs, qt, bias)
    return gemm_w8a8(xq, xs, qt, bias)


def moe_sort(topi: torch.Tensor, num_experts: int):
    """Stable counting sort of routed (token, slot) pairs by expert.
    topi int [T, k] -> (seg_off int32 [E+1], row_token int32 [T*k], pos int32 [T, k])."""
    if topi.dim() != 2:
        raise ValueError("topi must be [T, k]")
    dev = _require_cuda("moe_sort", topi)
    topi = topi.to(torch.int32).contiguous()
    T, k = topi.shape
    seg_off = torch.empty((num_experts + 1,), dtype=torch.int32, device=dev)
    row_token = torch.empty((T * k,), dtype=torch.int32, device=dev)
    pos = torch.empty((T, k), dtype=torch.int32, device=dev)
    with torch.cuda.device(dev):
        _lib.call("fni8_moe_sort", _ptr(topi), T, k, num_experts, _ptr(seg_off), _ptr(row_token),
                  _ptr(pos), _stream(dev))
    return seg_off, row_token, pos


def gemm_w8a8_grouped(aq: torch.Tensor, as_: torch.Tensor, w: torch.Tensor, ws: torch.Tensor,
                      seg_off: torch.Tensor, rows: int, row_index: torch.Tensor | None = None,
                      bias: torch.Tensor | None = None, want_acc: bool = False):
    """Grouped W8A8 GEMM over expert segments.
    aq int8 [A, K], as_ fp32 [A]; w int8 [E, N, K]; ws fp32 [E, N]; seg_off int32 [E+1];
    row_index int32 [rows] or None -> y fp16 [rows, N] in sorted-row order."""
    if aq.dtype != torch.int8 or aq.dim() != 2 or not aq.is_contiguous():
        raise ValueError("aq must be a contiguous int8 [rows, K] tensor")
    if w.dtype != torch.int8 or w.dim() != 3 or not w.is_contiguous():
        raise ValueError("w must be a contiguous int8 [E, N, K] tensor")
    E, N, K = w.shape
    if aq.shape[1] != K:
        raise ValueError(f"in_features mismatch: {aq.shape[1]} vs {K}")
    if ws.dtype != torch.float32 or ws.shape != (E, N) or not ws.is_contiguous():
        raise ValueError("ws must be a contiguous fp32 [E, N] tensor")
    if as_.dtype != torch.float32 or as_.numel() != aq.shape[0] or not as_.is_contiguous():
        raise ValueError("as_ must be a contiguous fp32 tensor with one entry per row of aq")
    if seg_off.dtype != torch.int32 or seg_off.numel() != E + 1:
        raise ValueError("seg_off must be int32 [E+1]")
    if row_index is not None and (row_index.dtype != torch.int32 or row_index.numel() < rows):
        raise ValueError("row_index must be int32 with at least `rows` entries")
    if row_index is None and aq.shape[0] < rows:
        raise ValueError("aq has fewer rows than `rows`")
    if bias is not None and (bias.dtype != _f16 or bias.shape != (E, N)):
        raise ValueError("bias must be fp16 [E, N]")
    dev = _require_cuda("gemm_w8a8_grouped", aq, as_, w, ws, seg_off, row_index, bias)
    y = torch.empty((rows, N), dtype=_f16, device=dev)
    acc = torch.empty((rows, N), dtype=torch.int32, device=dev) if want_acc else None
    if rows:
        with torch.cuda.device(dev):
            _lib.call("fni8_gemm_w8a8_grouped", _ptr(aq), _ptr(as_), _ptr(row_index), rows, K,
                      _ptr(w), _ptr(ws), E, N, _ptr(seg_off), _ptr(bias), _ptr(y), _ptr(acc),
                      _stream(dev))
    return (y, acc) if want_acc else y


W4_GROUPED_GROUPS = (64, 128, 256)


def gemm_w4a8_grouped(aq: torch.Tensor, as_: torch.Tensor, w: torch.Tensor, ws: torch.Tensor,
                      G: int, seg_off: torch.Tensor, rows: int,
                      row_index: torch.Tensor | None = None,
                      bias: torch.Tensor | None = None) -> torch.Tensor:
    """Grouped W4A8 GEMM over expert segments (per_group_i4 int4 experts).
    aq int8 [A, K], as_ fp32 [A]; w uint8 [E, N, K/2]; ws fp32 [E, N, K/G];
    seg_off int32 [E+1]; row_index int32 [rows] or None -> y fp16 [rows, N] in
    sorted-row order.  G in (64, 128, 256), K a multiple of 256."""
    if aq.dtype != torch.int8 or aq.dim() != 2 or not aq.is_contiguous():
        raise ValueError("aq must be a contiguous int8 [rows, K] tensor")
    if w.dtype != torch.uint8 or w.dim() != 3 or not w.is_contiguous():
        raise ValueError("w must be a contiguous uint8 [E, N, K/2] tensor")
    E, N, Kh = w.shape
    K = 2 * Kh
    if aq.shape[1] != K:
        raise ValueError(f"in_features mismatch: {aq.shape[1]} vs {K}")
    if G not in W4_GROUPED_GROUPS or K % 256:
        raise ValueError(f"grouped W4A8 needs G in {W4_GROUPED_GROUPS} and K a multiple of 256 "
                         f"(G={G}, K={K})")
    if ws.dtype != torch.float32 or ws.shape != (E, N, K // G) or not ws.is_contiguous():
        raise ValueError("ws must be a contiguous fp32 [E, N, K/G] tensor")
    if as_.dtype != torch.float32 or as_.numel() != aq.shape[0] or not as_.is_contiguous():
        raise ValueError("as_ must be a contiguous fp32 tensor with one entry per row of aq")
    if seg_off.dtype != torch.int32 or seg_off.numel() != E + 1:
        raise ValueError("seg_off must be int32 [E+1]")
    if row_index is not None and (row_index.dtype != torch.int32 or row_index.numel() < rows):
        raise ValueError("row_index must be int32 with at least `rows` entries")
    if row_index is None and aq.shape[0] < rows:
        raise ValueError("aq has fewer rows than `rows`")
    if bias is not None and (bias.dtype != _f16 or bias.shape != (E, N)):
        raise ValueError("bias must be fp16 [E, N]")
    dev = _require_cuda("gemm_w4a8_grouped", aq, as_, w, ws, seg_off, row_index, bias)
    y = torch.empty((rows, N), dtype=_f16, device=dev)
    if rows:
        with torch.cuda.device(dev):
            _lib.call("fni8_gemm_w4a8_grouped", _ptr(aq), _ptr(as_), _ptr(row_index), rows, K,
                      _ptr(w), _ptr(ws), E, N, G, _ptr(seg_off), _ptr(bias), _ptr(y),
                      _stream(dev))
    return y


def moe_combine(y_sorted: torch.Tensor, topi: torch.Tensor, topw: torch.Tensor,
                pos: torch.Tensor) -> torch.Tensor:
    """out[t] = sum over slots (ascending expert id) of fp16(y_sorted[pos[t, j]] * topw[t, j]),
    accumulated in fp16 from zero, as the expert loop's index_add_ does."""
    T, k = topi.shape
    if y_sorted.dtype != _f16 or y_sorted.dim() != 2 or y_sorted.shape[0] < T * k:
        raise ValueError("y_sorted must be fp16 [T*k, H]")
    if topw.dtype != _f16 or topw.shape != (T, k):
        raise ValueError("topw must be fp16 [T, k]")
    dev = _require_cuda("moe_combine", y_sorted, topi, topw, pos)
    H = y_sorted.shape[1]
    y_sorted = y_sorted.contiguous()
    topi = topi.to(torch.int32).contiguous()
    topw = topw.contiguous()
    pos = pos.to(torch.int32).contiguous()
    out = torch.empty((T, H), dtype=_f16, device=dev)
    if T:
        with torch.cuda.device(dev):
            _lib.call("fni8_moe_combine_f16", _ptr(y_sorted), H, _ptr(topi), _ptr(topw), _ptr(pos),
                      T, k, _ptr(out), _stream(dev))
    return out


_ACTS = {"silu": 0, "gelu_tanh": 1}


def _act_code(act: str) -> int:
    try:
        return _ACTS[act]
    except KeyError:
        raise ValueError(f"unsupported fused activation {act!r} (silu, gelu_tanh)") from None


def _merged_rows(x: torch.Tensor, name: str):
    if x.dtype != _f16:
        raise ValueError(f"{name} expects fp16 (got {x.dtype})")
    if x.shape[-1] % 2:
        raise ValueError(f"{name}: last dimension {x.shape[-1]} is not 2 * intermediate")
    return _rows(x, x.shape[-1])


def act_and_mul(x: torch.Tensor, act: str = "silu") -> torch.Tensor:
    """fni8.act_and_mul(x, act): x fp16 [..., 2I] (gate | up) -> fp16 [..., I]
    (fni8serve/layers/activation.py:24, :40)."""
    dev = _require_cuda("act_and_mul", x)
    code = _act_code(act)
    x2, ldx = _merged_rows(x, "act_and_mul")
    M, I = x2.shape[0], x2.shape[1] // 2
    out = torch.empty((*x.shape[:-1], I), dtype=_f16, device=dev)
    if M and I:
        with torch.cuda.device(dev):
            _lib.call("fni8_act_and_mul_f16", _ptr(x2), ldx, M, I, code, _ptr(out), I,
                      _stream(dev))
    return out


def act_and_mul_quant(x: torch.Tensor, act: str = "silu"):
    """act_and_mul with the next linear's per-token quantization fused in:
    x fp16 [..., 2I] -> (xq int8 [M, I], xs fp32 [M]), bit-identical to
    quantize_rowwise(act_and_mul(x, act))."""
    dev = _require_cuda("act_and_mul_quant", x)
    code = _act_code(act)
    x2, ldx = _merged_rows(x, "act_and_mul_quant")
    M, I = x2.shape[0], x2.shape[1] // 2
    if I % 4:
        raise ValueError(f"act_and_mul_quant: intermediate size {I} is not a multiple of 4")
    xq = torch.empty((M, I), dtype=torch.int8, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    if M:
        # few rows: several workgroups share a row and exchange partial maxima
        # through a workspace (caching allocator; contents never matter)
        nw = int(_lib.load().fni8_act_and_mul_quant_workspace_bytes(M, I))
        work = torch.empty(nw, dtype=torch.uint8, device=dev) if nw else None
        with torch.cuda.device(dev):
            _lib.call("fni8_act_and_mul_quant_f16_ws", _ptr(x2), ldx, M, I, code, _ptr(xq), I,
                      _ptr(xs), _ptr(work), nw, _stream(dev))
    return xq, xs


def _norm_args(name, x, weight, residual):
    dev = _require_cuda(name, x, weight, residual)
    K = x.shape[-1]
    if x.dtype != _f16 or weight.dtype != _f16:
        raise ValueError(f"{name} expects fp16 x and weight (got {x.dtype}, {weight.dtype})")
    if weight.numel() != K:
        raise ValueError(f"{name}: weight has {weight.numel()} entries, x rows have {K}")
    if residual is not None and (residual.dtype != _f16 or residual.shape != x.shape):
        raise ValueError(f"{name}: residual must be fp16 with x's shape")
    x2, ldx = _rows(x, K)
    r2, ldr = (None, 0) if residual is None else _rows(residual, K)
    return dev, K, x2, ldx, r2, ldr, weight.contiguous()


def rmsnorm(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
            residual: torch.Tensor | None = None, unit_offset: bool = False):
    """fni8.rmsnorm(x, weight, eps, residual=, unit_offset=)
    (fni8serve/layers/norm.py:51-52): the normed fp16 tensor, or
    (normed, x + residual) when a residual is given."""
    dev, K, x2, ldx, r2, ldr, w = _norm_args("rmsnorm", x, weight, residual)
    M = x2.shape[0]
    out = torch.empty(x.shape, dtype=_f16, device=dev)
    new_res = None if residual is None else torch.empty(x.shape, dtype=_f16, device=dev)
    if M:
        with torch.cuda.device(dev):
            _lib.call("fni8_rmsnorm_f16", _ptr(x2), ldx, _ptr(r2), ldr, _ptr(w),
                      ctypes.c_float(eps), int(bool(unit_offset)), M, K, _ptr(out), K,
                      _ptr(new_res), K, _stream(dev))
    return out if residual is None else (out, new_res)


def rmsnorm_quant(x: torch.Tensor, weight: torch.Tensor, eps: float = 1e-6,
                  residual: torch.Tensor | None = None, unit_offset: bool = False):
    """rmsnorm with the next linear's per-token quantization fused in:
    (xq int8 [M, K], xs fp32 [M]), or (xq, xs, x + residual) with a residual;
    bit-identical to quantize_rowwise(rmsnorm(...))."""
    dev, K, x2, ldx, r2, ldr, w = _norm_args("rmsnorm_quant", x, weight, residual)
    if K % 4:
        raise ValueError(f"rmsnorm_quant: K={K} is not a multiple of 4")
    M = x2.shape[0]
    xq = torch.empty((M, K), dtype=torch.int8, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    new_res = None if residual is None else torch.empty(x.shape, dtype=_f16, device=dev)
    if M:
        with torch.cuda.device(dev):
            _lib.call("fni8_rmsnorm_quant_f16", _ptr(x2), ldx, _ptr(r2), ldr, _ptr(w),
                      ctypes.c_float(eps), int(bool(unit_offset)), M, K, _ptr(xq), K, _ptr(xs),
                      _ptr(new_res), K, _stream(dev))
    return (xq, xs) if residual is None else (xq, xs, new_res)


_SCORES = {"softmax": 0, "sigmoid": 1}


def moe_route(logits: torch.Tensor, top_k: int, scoring: str = "softmax",
              bias: torch.Tensor | None = None, num_groups: int | None = None,
              topk_group: int | None = None, renorm: bool = True, scale: float = 1.0):
    """Router of SparseMoE (fni8serve/models/moe.py:62-91) in one launch:
    logits fp32 [T, E] -> (topw fp16 [T, k], topi int32 [T, k]), best first."""
    dev = _require_cuda("moe_route", logits, bias)
    if logits.dtype != torch.float32 or logits.dim() != 2:
        raise ValueError("moe_route expects fp32 logits [T, E]")
    if scoring not in _SCORES:
        raise ValueError(f"unsupported scoring function {scoring!r} (softmax, sigmoid)")
    if logits.stride(1) != 1:
        logits = logits.contiguous()
    T, E = logits.shape
    if bias is not None:
        if bias.numel() != E:
            raise ValueError(f"bias has {bias.numel()} entries, expected {E}")
        bias = bias.reshape(-1).float().contiguous()
    groups = 0 if num_groups is None or topk_group is None else int(num_groups)
    tg = 0 if groups == 0 else int(topk_group)
    topw = torch.empty((T, top_k), dtype=_f16, device=dev)
    topi = torch.empty((T, top_k), dtype=torch.int32, device=dev)
    if T:
        ldl = logits.stride(0) if T > 1 else E
        with torch.cuda.device(dev):
            _lib.call("fni8_moe_route", _ptr(logits), T, E, ldl, _SCORES[scoring], _ptr(bias),
                      groups, tg, top_k, int(bool(renorm)), ctypes.c_float(scale), _ptr(topw),
                      _ptr(topi), _stream(dev))
    return topw, topi
