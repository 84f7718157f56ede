"""numpy front end of the C oracle (oracle/w8a8_oracle.c).

TEST INFRASTRUCTURE ONLY.  Every function takes and returns numpy arrays on
the host; fp16 arrays are `np.float16` (their bit patterns are what the C code
reads).  Reference citations for each step live beside the C functions.

parity pinning (how each function is checked, in tests/test_oracle.py):
  f32_to_f16 / f16_to_f32 -- all 65536 fp16 bit patterns round-trip; f32->f16
      agrees bit-for-bit with numpy's IEEE conversion on 2^24 patterns spanning
      every exponent, ties, subnormals, overflow.
  quant_rowwise_f16 -- hand-computed known answers (ties to even, clamp, zero
      row, outlier), invariants (max element -> +-127, sign symmetry,
      monotonicity, |x - q s| <= s/2), exhaustive sweep of all finite fp16
      values, row locality.
  gemm_i8 -- exact against float64 BLAS matmul (exact while K*127^2 < 2^53) and
      torch._int_mm.
  dequant_f16 -- fp64 closed form within one fp16 rounding; transposed scale
      indexing fails the check.
  moe_sort / grouped_w8a8_f16 / moe_combine_f16 -- brute force against the
      reference's per-expert loop restated with `nonzero` in numpy (moe.py:99-105).
  quant_identity_check -- not an oracle function: the exhaustive proof, over
      every fp16 (x, amax) pair, that the division-free quantization of the GPU
      decode kernel reproduces quant_rowwise_f16's division (quant_identity.c).
  exp_cw / act_f32 / act_and_mul_f16 (act_norm_oracle.c; tests/test_oracle_act_norm.py)
      -- float64 exp over a dense fp32 sweep (max error in ulp), the float64
      closed forms of silu and the tanh gelu over every fp16 gate, known
      answers, torch's eager fallback (F.silu(g) * u, F.gelu(g, "tanh") * u) and
      torch's fp32 forms.
  moe_route (route_oracle.c) -- float64 softmax / sigmoid, brute-force top-k by
      sorting (value desc, index asc), the reference's torch routing
      (fni8serve/models/moe.py:62-97) on the CPU: same experts, weights within
      1 fp16 ulp; known answers (ties, groups, NaN rows, renormalisation).
  gemm_w4a8 / linear_w4a8_f16 (w4a8_oracle.c) -- the group sums exact against
      numpy integer matmuls over codes packed by the reference's own formula
      (fni8serve/convert.py:72-73) and unpacked as fni8serve/layers/linear.py:32-40
      does; outputs against the float64 closed form within the fp32 fold's error
      bound; the reference's CPU fallback (dequantize, F.linear) by cosine; the
      ascending-group fold order on a case that exposes it.
  sumsq_fixed / rmsnorm_f16 -- math.fsum error bound, exact known answers,
      float64 closed form, torch's eager RMSNorm (fni8serve/layers/norm.py:37-58)
      and torch's fp16 residual add bit for bit, unit-offset identity.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_SO = os.path.join(_HERE, "_build", "liboracle_w8a8.so")
QUANT_EPS = np.float32(1e-6)

_lib = None


def _load():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(_SO):
        subprocess.run(["make", "-s", "-C", _HERE], check=True)
    lib = ctypes.CDLL(_SO)
    P, I = ctypes.c_void_p, ctypes.c_int64
    lib.oracle_f32_to_f16.restype = ctypes.c_uint16
    lib.oracle_f32_to_f16.argtypes = [ctypes.c_float]
    lib.oracle_f16_to_f32.restype = ctypes.c_float
    lib.oracle_f16_to_f32.argtypes = [ctypes.c_uint16]
    lib.oracle_f16_to_f32_n.argtypes = [P, P, I]
    lib.oracle_f32_to_f16_n.argtypes = [P, P, I]
    lib.oracle_quant_rowwise_f16.argtypes = [P, I, I, I, P, I, P]
    lib.oracle_gemm_i8.argtypes = [P, I, I, I, P, I, I, P, I]
    lib.oracle_dequant_f16.argtypes = [P, I, I, I, P, P, P, P, I]
    lib.oracle_linear_w8a8_f16.argtypes = [P, I, I, I, P, P, I, P, P, I, P, P, P]
    lib.oracle_moe_sort.restype = ctypes.c_int
    lib.oracle_moe_sort.argtypes = [P, I, I, I, P, P, P, P]
    lib.oracle_grouped_w8a8_f16.argtypes = [P, P, I, P, P, P, I, I, P, P, P, P]
    lib.oracle_moe_combine_f16.argtypes = [P, I, P, P, P, I, I, P]
    lib.oracle_quant_identity_check.argtypes = [ctypes.c_int, P]
    F, C = ctypes.c_float, ctypes.c_int
    lib.oracle_exp_cw.restype = F
    lib.oracle_exp_cw.argtypes = [F]
    lib.oracle_act_f32.restype = F
    lib.oracle_act_f32.argtypes = [F, C]
    lib.oracle_act_and_mul_f16.argtypes = [P, I, I, I, C, P, I]
    lib.oracle_act_and_mul_quant_f16.argtypes = [P, I, I, I, C, P, P, I, P]
    lib.oracle_exp_cw_n.argtypes = [P, P, I]
    lib.oracle_act_f32_n.argtypes = [P, P, I, C]
    lib.oracle_moe_route.argtypes = [P, I, I, I, C, P, I, I, I, C, F, P, P]
    lib.oracle_gemm_w4a8.argtypes = [P, P, I, I, P, P, I, I, P, P, P]
    lib.oracle_linear_w4a8_f16.argtypes = [P, I, I, P, P, I, I, P, P, P, P]
    lib.oracle_sumsq_fixed.restype = F
    lib.oracle_sumsq_fixed.argtypes = [P, I]
    lib.oracle_rmsnorm_f16.argtypes = [P, I, P, I, P, F, C, I, I, P, I, P, I, P]
    lib.oracle_rmsnorm_quant_f16.argtypes = [P, I, P, I, P, F, C, I, I, P, P, I, P, P, I, P]
    for fn in ("oracle_f16_to_f32_n", "oracle_f32_to_f16_n", "oracle_quant_rowwise_f16",
               "oracle_gemm_i8", "oracle_dequant_f16", "oracle_linear_w8a8_f16",
               "oracle_grouped_w8a8_f16", "oracle_moe_combine_f16",
               "oracle_quant_identity_check", "oracle_act_and_mul_f16",
               "oracle_act_and_mul_quant_f16", "oracle_rmsnorm_f16", "oracle_rmsnorm_quant_f16",
               "oracle_exp_cw_n", "oracle_act_f32_n", "oracle_moe_route", "oracle_gemm_w4a8",
               "oracle_linear_w4a8_f16"):
        getattr(lib, fn).restype = None
    _lib = lib
    return lib


def _p(a):
    return None if a is None else a.ctypes.data


def _c(a, dtype):
    return np.ascontiguousarray(a, dtype=dtype)


def f32_to_f16(f: np.ndarray) -> np.ndarray:
    f = _c(f, np.float32)
    out = np.empty(f.shape, np.uint16)
    _load().oracle_f32_to_f16_n(_p(f), _p(out), f.size)
    return out.view(np.float16)


def f16_to_f32(h: np.ndarray) -> np.ndarray:
    h = _c(np.asarray(h).view(np.uint16) if np.asarray(h).dtype == np.float16 else h, np.uint16)
    out = np.empty(h.shape, np.float32)
    _load().oracle_f16_to_f32_n(_p(h), _p(out), h.size)
    return out


def quant_rowwise_f16(x: np.ndarray):
    """x fp16 [M, K] -> (q int8 [M, K], s fp32 [M])."""
    x = _c(x, np.float16)
    M, K = x.shape
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    _load().oracle_quant_rowwise_f16(_p(x), M, K, K, _p(q), K, _p(s))
    return q, s


def gemm_i8(a: np.ndarray, w: np.ndarray) -> np.ndarray:
    """a int8 [M, K], w int8 [N, K] -> acc int32 [M, N]."""
    a = _c(a, np.int8)
    w = _c(w, np.int8)
    M, K = a.shape
    N = w.shape[0]
    assert w.shape[1] == K
    acc = np.empty((M, N), np.int32)
    _load().oracle_gemm_i8(_p(a), K, M, K, _p(w), K, N, _p(acc), N)
    return acc


def dequant_f16(acc, a_s, w_s, bias=None) -> np.ndarray:
    acc = _c(acc, np.int32)
    M, N = acc.shape
    a_s = _c(a_s, np.float32)
    w_s = _c(w_s, np.float32)
    b = None if bias is None else _c(bias, np.float16)
    y = np.empty((M, N), np.float16)
    _load().oracle_dequant_f16(_p(acc), N, M, N, _p(a_s), _p(w_s), _p(b), _p(y), N)
    return y


def linear_w8a8_f16(x, w, w_s, bias=None):
    """Whole W8A8 linear.  Returns (y fp16 [M, N], xq int8, xs fp32, acc int32)."""
    x = _c(x, np.float16)
    w = _c(w, np.int8)
    w_s = _c(w_s, np.float32)
    b = None if bias is None else _c(bias, np.float16)
    M, K = x.shape
    N = w.shape[0]
    y = np.empty((M, N), np.float16)
    xq = np.empty((M, K), np.int8)
    xs = np.empty((M,), np.float32)
    acc = np.empty((M, N), np.int32)
    _load().oracle_linear_w8a8_f16(_p(x), K, M, K, _p(w), _p(w_s), N, _p(b), _p(y), N,
                                   _p(xq), _p(xs), _p(acc))
    return y, xq, xs, acc


def moe_sort(topi: np.ndarray, E: int):
    """topi int [T, k] -> (seg_off [E+1], row_token [R], row_slot [R], pos [T, k])."""
    topi = _c(topi, np.int32)
    T, k = topi.shape
    seg = np.empty((E + 1,), np.int32)
    rt = np.empty((T * k,), np.int32)
    rs = np.empty((T * k,), np.int32)
    pos = np.empty((T, k), np.int32)
    rc = _load().oracle_moe_sort(_p(topi), T, k, E, _p(seg), _p(rt), _p(rs), _p(pos))
    if rc != 0:
        raise ValueError("expert id out of range")
    return seg, rt, rs, pos


def grouped_w8a8_f16(aq, a_s, w, w_s, seg_off, row_index=None, bias=None, want_acc=False):
    """aq int8 [rows, K], a_s fp32 [rows]; w int8 [E, N, K]; w_s fp32 [E, N];
    seg_off [E+1]; row_index [R] (gather) or None -> y fp16 [R, N] (, acc int32)."""
    aq = _c(aq, np.int8)
    a_s = _c(a_s, np.float32)
    w = _c(w, np.int8)
    w_s = _c(w_s, np.float32)
    seg_off = _c(seg_off, np.int32)
    E, N, K = w.shape
    R = int(seg_off[-1])
    ri = None if row_index is None else _c(row_index, np.int32)
    b = None if bias is None else _c(bias, np.float16)
    y = np.zeros((R, N), np.float16)
    acc = np.zeros((R, N), np.int32) if want_acc else None
    _load().oracle_grouped_w8a8_f16(_p(aq), _p(a_s), K, _p(ri), _p(w), _p(w_s), E, N,
                                    _p(seg_off), _p(b), _p(y), _p(acc))
    return (y, acc) if want_acc else y


def moe_combine_f16(y_sorted, topi, topw, pos):
    y_sorted = _c(y_sorted, np.float16)
    topi = _c(topi, np.int32)
    topw = _c(topw, np.float16)
    pos = _c(pos, np.int32)
    T, k = topi.shape
    H = y_sorted.shape[1]
    out = np.empty((T, H), np.float16)
    _load().oracle_moe_combine_f16(_p(y_sorted), H, _p(topi), _p(topw), _p(pos), T, k, _p(out))
    return out


def quant_identity_check(corrected: bool = True, magic_slip: bool = False):
    """(pairs, quotient mismatches for x != 0, rounded mismatches, int8 byte
    mismatches) of the division-free quantization against fl(x / s) over every
    fp16 (x, amax) pair with |x| <= amax (quant_identity.c).  corrected=False
    drops the FMA correction step; magic_slip=True rounds with 2^23 instead of
    1.5 * 2^23 (negative controls)."""
    out = np.zeros(4, np.int64)
    mode = 2 if magic_slip else (0 if corrected else 1)
    _load().oracle_quant_identity_check(mode, _p(out))
    return tuple(int(v) for v in out)


ACTS = {"silu": 0, "gelu_tanh": 1}


def exp_cw(x) -> np.ndarray:
    """The activations' fp32 exp (Cody-Waite reduction + degree-7 Taylor), x in [-86, 88]."""
    x = _c(x, np.float32)
    y = np.empty_like(x)
    _load().oracle_exp_cw_n(_p(x), _p(y), x.size)
    return y


def act_f32(g, act: str) -> np.ndarray:
    """The gate value act(g) in fp32 (silu or gelu_tanh), before the product with up."""
    g = _c(g, np.float32)
    y = np.empty_like(g)
    _load().oracle_act_f32_n(_p(g), _p(y), g.size, ACTS[act])
    return y


def act_and_mul_f16(x: np.ndarray, act: str) -> np.ndarray:
    """x fp16 [M, 2I] (gate | up) -> fp16 [M, I]."""
    x = _c(x, np.float16)
    M, I2 = x.shape
    I = I2 // 2
    out = np.empty((M, I), np.float16)
    _load().oracle_act_and_mul_f16(_p(x), I2, M, I, ACTS[act], _p(out), I)
    return out


def act_and_mul_quant_f16(x: np.ndarray, act: str):
    """x fp16 [M, 2I] -> (q int8 [M, I], s fp32 [M]): act_and_mul then quant_rowwise_f16."""
    x = _c(x, np.float16)
    M, I2 = x.shape
    I = I2 // 2
    tmp = np.empty((M, I), np.float16)
    q = np.empty((M, I), np.int8)
    s = np.empty((M,), np.float32)
    _load().oracle_act_and_mul_quant_f16(_p(x), I2, M, I, ACTS[act], _p(tmp), _p(q), I, _p(s))
    return q, s


def sumsq_fixed(h: np.ndarray) -> np.float32:
    """Sum of squares of one fp16 row in the RMSNorm kernels' fixed order."""
    h = _c(h, np.float16).reshape(-1)
    return np.float32(_load().oracle_sumsq_fixed(_p(h), h.size))


def rmsnorm_f16(x, weight, eps, residual=None, unit_offset=False):
    """x fp16 [M, K], weight fp16 [K] -> (out fp16 [M, K], x + residual fp16 or None)."""
    x = _c(x, np.float16)
    M, K = x.shape
    w = _c(weight, np.float16)
    r = None if residual is None else _c(residual, np.float16)
    out = np.empty((M, K), np.float16)
    ro = None if r is None else np.empty((M, K), np.float16)
    tmp = np.empty((K,), np.float16)
    _load().oracle_rmsnorm_f16(_p(x), K, _p(r), K, _p(w), float(np.float32(eps)),
                               int(bool(unit_offset)), M, K, _p(out), K, _p(ro), K, _p(tmp))
    return out, ro


def rmsnorm_quant_f16(x, weight, eps, residual=None, unit_offset=False):
    """-> (q int8 [M, K], s fp32 [M], x + residual fp16 or None): rmsnorm then quant."""
    x = _c(x, np.float16)
    M, K = x.shape
    w = _c(weight, np.float16)
    r = None if residual is None else _c(residual, np.float16)
    normed = np.empty((M, K), np.float16)
    q = np.empty((M, K), np.int8)
    s = np.empty((M,), np.float32)
    ro = None if r is None else np.empty((M, K), np.float16)
    tmp = np.empty((K,), np.float16)
    _load().oracle_rmsnorm_quant_f16(_p(x), K, _p(r), K, _p(w), float(np.float32(eps)),
                                     int(bool(unit_offset)), M, K, _p(normed), _p(q), K, _p(s),
                                     _p(ro), K, _p(tmp))
    return q, s, ro


SCORES = {"softmax": 0, "sigmoid": 1}


def moe_route(logits, k, scoring="softmax", bias=None, groups=0, topk_group=0, renorm=True,
              scale=1.0):
    """logits fp32 [T, E] -> (topw fp16 [T, k], topi int32 [T, k])."""
    lg = _c(logits, np.float32)
    T, E = lg.shape
    b = None if bias is None else _c(bias, np.float32)
    topw = np.empty((T, k), np.float16)
    topi = np.empty((T, k), np.int32)
    _load().oracle_moe_route(_p(lg), T, E, E, SCORES[scoring], _p(b), groups, topk_group, k,
                             int(bool(renorm)), float(np.float32(scale)), _p(topw), _p(topi))
    return topw, topi


def gemm_w4a8(xq, xs, w_packed, ws, group_size, bias=None, want_groups=False):
    """xq int8 [M, K], xs fp32 [M]; w_packed uint8 [N, K/2]; ws fp32 [N, K/G]
    -> y fp16 [M, N] (and the int32 group sums [M, N, K/G])."""
    xq = _c(xq, np.int8)
    xs = _c(xs, np.float32)
    w = _c(w_packed, np.uint8)
    ws = _c(ws, np.float32)
    M, K = xq.shape
    N = w.shape[0]
    b = None if bias is None else _c(bias, np.float16)
    y = np.empty((M, N), np.float16)
    ga = np.empty((M, N, K // group_size), np.int32) if want_groups else None
    _load().oracle_gemm_w4a8(_p(xq), _p(xs), M, K, _p(w), _p(ws), N, group_size, _p(b), _p(y),
                             _p(ga))
    return (y, ga) if want_groups else y


def linear_w4a8_f16(x, w_packed, ws, group_size, bias=None):
    """Whole W4A8 linear: returns (y fp16 [M, N], xq int8, xs fp32)."""
    x = _c(x, np.float16)
    w = _c(w_packed, np.uint8)
    ws = _c(ws, np.float32)
    M, K = x.shape
    N = w.shape[0]
    b = None if bias is None else _c(bias, np.float16)
    y = np.empty((M, N), np.float16)
    xq = np.empty((M, K), np.int8)
    xs = np.empty((M,), np.float32)
    _load().oracle_linear_w4a8_f16(_p(x), M, K, _p(w), _p(ws), N, group_size, _p(b), _p(y),
                                   _p(xq), _p(xs))
    return y, xq, xs
