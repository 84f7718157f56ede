"""Pins of the CPU oracle (oracle/w8a8_oracle.c) against what the mathematics and
independent implementations fix.  The reference ships no golden vectors for this
path (its tests draw torch.randn at run time), so each oracle function is checked
here by known answers worked by hand, invariants, brute force, exhaustive sweeps
and independent library routines, chosen so that a plausible slip (a dropped abs,
round-half-up instead of half-even, fp64 instead of fp32 division, a transposed
scale index, an unstable sort) fails at least one test."""
from fractions import Fraction

import numpy as np
import pytest
import torch

from oracle import oracle

RNG = np.random.default_rng(1234)


def f16(a):
    return np.asarray(a, dtype=np.float16)


# ---- fp16 <-> fp32 ---------------------------------------------------------

def test_f16_to_f32_exhaustive():
    h = np.arange(65536, dtype=np.uint16)
    got = oracle.f16_to_f32(h)
    ref = h.view(np.float16).astype(np.float32)
    same = (got.view(np.uint32) == ref.view(np.uint32)) | (np.isnan(got) & np.isnan(ref))
    assert same.all()


def test_f32_to_f16_against_numpy():
    bits = RNG.integers(0, 2 ** 32, size=1 << 21, dtype=np.uint64).astype(np.uint32)
    # plus every fp16 value, and the midpoints between neighbours (exact ties)
    h = np.arange(0, 0x7c00, dtype=np.uint32)
    lo = h.astype(np.uint16).view(np.float16).astype(np.float64)
    hi = (h + 1).astype(np.uint16).view(np.float16).astype(np.float64)
    mids = ((lo + hi) / 2).astype(np.float32)
    specials = np.array([65504, 65519.99, 65520, 65536, 1e-8, 2 ** -25, 2 ** -24, 2 ** -14,
                         -0.0, np.inf, -np.inf], dtype=np.float32)
    f = np.concatenate([bits.view(np.float32), mids, -mids, specials])
    with np.errstate(over="ignore"):
        ref = f.astype(np.float16)
    got = oracle.f32_to_f16(f)
    nan = np.isnan(f)
    assert np.array_equal(got.view(np.uint16)[~nan], ref.view(np.uint16)[~nan])
    assert np.isnan(got[nan]).all()


# ---- per-token quantization ------------------------------------------------

def test_quant_known_answers():
    # amax = 127 makes the scale exactly 1.0, so the quotients are the inputs and
    # the rounding is visible directly: ties go to even, never away from zero.
    x = f16([[127, 1, -2, 0.5, 1.5, 2.5, -2.5, 126.5, -0.5, 3.5, -126.5, 0]])
    q, s = oracle.quant_rowwise_f16(x)
    assert s[0] == np.float32(1.0)
    assert q[0].tolist() == [127, 1, -2, 0, 2, 2, -2, 126, 0, 4, -126, 0]


def test_quant_negative_max_and_outlier():
    x = f16([[-3, 1, 2, 0], [1000, 1, -1, 7]])
    q, s = oracle.quant_rowwise_f16(x)
    assert s[0] == np.float32(3) / np.float32(127)
    assert q[0, 0] == -127 and q[0, 2] == 85          # 2 / (3/127) = 84.67 -> 85
    assert s[1] == np.float32(1000) / np.float32(127)
    assert q[1].tolist() == [127, 0, 0, 1]             # 7 / 7.874 = 0.889 -> 1


def test_quant_zero_and_tiny_rows_use_eps():
    x = np.zeros((2, 16), np.float16)
    x[1, 3] = np.float16(6e-8)                         # subnormal fp16, below eps
    q, s = oracle.quant_rowwise_f16(x)
    eps_scale = np.float32(1e-6) / np.float32(127)
    assert s[0] == eps_scale and s[1] == eps_scale
    assert not q[0].any()
    # 6e-8 / (1e-6/127) = 7.6 -> 8
    assert q[1, 3] == 8 and q[1].sum() == 8


def test_quant_nonfinite_rows():
    x = np.ones((3, 8), np.float16)
    x[0, 2] = np.nan
    x[1, 5] = np.inf
    x[2, 0] = -np.inf
    q, s = oracle.quant_rowwise_f16(x)
    assert np.isnan(s[0]) and np.isinf(s[1]) and np.isinf(s[2])
    assert not q.any()                                 # x/NaN and x/inf quantize to 0


def test_quant_invariants_random_rows():
    x = (RNG.standard_normal((64, 1024)) * RNG.uniform(0.01, 300, (64, 1))).astype(np.float16)
    q, s = oracle.quant_rowwise_f16(x)
    xf = x.astype(np.float64)
    # the max-magnitude element maps to +-127
    arg = np.abs(xf).argmax(axis=1)
    assert np.array_equal(np.abs(q[np.arange(64), arg]), np.full(64, 127))
    # sign symmetry
    qn, sn = oracle.quant_rowwise_f16(-x)
    assert np.array_equal(qn, -q) and np.array_equal(sn, s)
    # monotone in x within a row
    order = np.argsort(xf, axis=1, kind="stable")
    assert (np.diff(np.take_along_axis(q.astype(np.int32), order, axis=1), axis=1) >= 0).all()
    # dequantization error within half a step; the slack is the fp32 rounding of
    # the quotient (|x/s| <= 127.5, ulp 2^-17), which can land exactly on a tie
    err = np.abs(xf - q * s[:, None].astype(np.float64))
    assert (err <= s[:, None] * (0.5 + 2 ** -16)).all()
    # row locality: a row's result does not depend on the other rows
    q1, s1 = oracle.quant_rowwise_f16(x[7:8])
    assert np.array_equal(q1[0], q[7]) and s1[0] == s[7]


def test_quant_exhaustive_fp16_against_exact_rationals():
    """Every finite fp16 value under one fixed scale (forced by a 65504 entry).
    Away from half-integer ties, rint(fl32(x / s)) equals the integer nearest the
    exact rational x / s; at exact ties it is the even neighbour."""
    h = np.arange(65536, dtype=np.uint16).view(np.float16)
    h = h[np.isfinite(h)]
    row = np.concatenate([[np.float16(65504)], h])
    q, s = oracle.quant_rowwise_f16(row[None, :])
    sc = Fraction(float(s[0]))
    assert s[0] == np.float32(65504) / np.float32(127)
    checked = 0
    for xv, qv in zip(row[1:].tolist(), q[0, 1:].tolist()):
        t = Fraction(xv) / sc
        fl = t.numerator // t.denominator
        frac = t - fl
        if abs(frac - Fraction(1, 2)) < Fraction(1, 1 << 16):
            continue                     # within fp32 rounding of a tie: fl32(x/s) decides
        nearest = fl + (1 if frac > Fraction(1, 2) else 0)
        nearest = max(-127, min(127, nearest))
        assert qv == nearest, (xv, qv, nearest)
        checked += 1
    assert checked > 60000


def test_quant_matches_numpy_fp32_restatement():
    """numpy's IEEE fp32 division and half-even rint, evaluated independently."""
    x = (RNG.standard_normal((32, 4096)) * 3).astype(np.float16)
    x[RNG.random(x.shape) < 0.01] *= 20
    q, s = oracle.quant_rowwise_f16(x)
    amax = np.abs(x.astype(np.float32)).max(axis=1)
    s_np = np.maximum(amax, np.float32(1e-6)) / np.float32(127)
    q_np = np.clip(np.rint(x.astype(np.float32) / s_np[:, None]), -127, 127).astype(np.int8)
    assert np.array_equal(s, s_np.astype(np.float32)) and np.array_equal(q, q_np)


def test_division_free_quant_identity_exhaustive():
    """The GPU kernels quantize with y = fl(1/s), t = fl(x*y),
    v = fma(fma(-t, s, x), y, t) instead of fl(x/s), and take the int8 as the low
    byte of v + 1.5 * 2^23.  Over every fp16 amax and every fp16 x with
    |x| <= amax (about 10^9 pairs) the quotient is the same bits for x != 0, the
    rounded integer is always the same, and so is the int8."""
    pairs, bad_quot, bad_int, bad_byte = oracle.quant_identity_check()
    assert pairs == 1007713280
    assert bad_quot == 0 and bad_int == 0 and bad_byte == 0


def test_division_free_quant_identity_check_detects_a_missing_correction():
    """Negative control: without the FMA correction (q = rint(fl(x * fl(1/s))))
    the same exhaustive sweep finds quotient and rounded-integer mismatches."""
    pairs, bad_quot, bad_int, bad_byte = oracle.quant_identity_check(corrected=False)
    assert pairs == 1007713280
    assert bad_quot > 0 and bad_int > 0 and bad_byte > 0


def test_magic_rounding_check_detects_a_wrong_constant():
    """Negative control: rounding with 2^23 instead of 1.5 * 2^23 (exact for
    v >= 0, wrong for negative v) is caught by the int8 comparison."""
    pairs, bad_quot, bad_int, bad_byte = oracle.quant_identity_check(magic_slip=True)
    assert pairs == 1007713280
    assert bad_quot == 0 and bad_int == 0 and bad_byte > 0


# ---- int8 GEMM -------------------------------------------------------------

@pytest.mark.parametrize("M,N,K", [(1, 64, 4096), (8, 300, 1024), (33, 17, 12288), (5, 7, 4)])
def test_gemm_exact_against_blas_and_int_mm(M, N, K):
    a = RNG.integers(-127, 128, (M, K), dtype=np.int8)
    w = RNG.integers(-127, 128, (N, K), dtype=np.int8)
    acc = oracle.gemm_i8(a, w)
    ref = a.astype(np.float64) @ w.astype(np.float64).T     # exact: |acc| < 2^53
    assert np.array_equal(acc, ref.astype(np.int64).astype(np.int32))
    if M >= 17 and K % 8 == 0 and N % 8 == 0:
        mm = torch._int_mm(torch.from_numpy(a), torch.from_numpy(w).T.contiguous())
        assert np.array_equal(acc, mm.numpy())


def test_gemm_extreme_magnitudes_do_not_overflow():
    K = 12288
    a = np.full((2, K), 127, np.int8)
    a[1] = -127
    w = np.full((3, K), -127, np.int8)
    w[1] = 127
    acc = oracle.gemm_i8(a, w)
    big = K * 127 * 127
    assert acc.tolist() == [[-big, big, -big], [big, -big, big]]


# ---- dequant epilogue ------------------------------------------------------

def test_dequant_against_fp64_closed_form():
    M, N = 5, 9                                   # M != N: a transposed index fails
    acc = RNG.integers(-2 ** 27, 2 ** 27, (M, N)).astype(np.int32)
    a_s = RNG.uniform(1e-4, 0.5, M).astype(np.float32)
    w_s = RNG.uniform(1e-4, 0.02, N).astype(np.float32)
    bias = RNG.standard_normal(N).astype(np.float16)
    for b in (None, bias):
        y = oracle.dequant_f16(acc, a_s, w_s, b)
        exact = acc.astype(np.float64) * a_s[:, None] * w_s[None, :]
        if b is not None:
            exact = exact + b.astype(np.float64)[None, :]
        fin = np.abs(exact) < 65504
        err = np.abs(y.astype(np.float64) - exact)[fin]
        assert (err <= np.abs(exact[fin]) * (2 ** -11 + 2 ** -21) + 2 ** -24).all()
        assert np.isinf(y[~fin]).all() or (~fin).sum() == 0


def test_dequant_matches_numpy_fp32_sequence():
    acc = RNG.integers(-2 ** 30, 2 ** 30, (7, 11)).astype(np.int32)
    a_s = RNG.uniform(1e-5, 1e-2, 7).astype(np.float32)
    w_s = RNG.uniform(1e-3, 2e-2, 11).astype(np.float32)
    bias = RNG.standard_normal(11).astype(np.float16)
    y = oracle.dequant_f16(acc, a_s, w_s, bias)
    v = (acc.astype(np.float32) * a_s[:, None]) * w_s[None, :] + bias.astype(np.float32)
    with np.errstate(over="ignore"):
        assert np.array_equal(y.view(np.uint16), v.astype(np.float16).view(np.uint16))


def test_linear_is_the_composition():
    x = (RNG.standard_normal((6, 256))).astype(np.float16)
    w = RNG.integers(-127, 128, (40, 256), dtype=np.int8)
    ws = RNG.uniform(0.001, 0.02, 40).astype(np.float32)
    y, xq, xs, acc = oracle.linear_w8a8_f16(x, w, ws)
    q2, s2 = oracle.quant_rowwise_f16(x)
    acc2 = oracle.gemm_i8(q2, w)
    assert np.array_equal(xq, q2) and np.array_equal(xs, s2) and np.array_equal(acc, acc2)
    assert np.array_equal(y.view(np.uint16), oracle.dequant_f16(acc2, s2, ws).view(np.uint16))


def test_reference_cosine_bar_holds_for_oracle():
    """The reference's own bar for the int8 path against the fp16 dequant fallback:
    cosine >= 0.99 (tests/test_smoke.py:68-80, M=16, K=512, N=256)."""
    from oracle.reference_cpu import reference_cpu_linear
    torch.manual_seed(0)
    w = torch.randn(256, 512)
    s = w.abs().amax(-1, keepdim=True) / 127
    q = torch.round(w / s).clamp_(-127, 127).to(torch.int8)
    x = torch.randn(16, 512).half()
    y, *_ = oracle.linear_w8a8_f16(x.numpy(), q.numpy(), s.squeeze(-1).numpy())
    ref = reference_cpu_linear(x.float(), q, s.squeeze(-1)).float()
    cos = torch.nn.functional.cosine_similarity(torch.from_numpy(y).float().flatten(),
                                                ref.flatten(), dim=0)
    assert cos.item() >= 0.99


# ---- MoE sort / grouped GEMM / combine -------------------------------------

def _topi(T, E, k, seed):
    g = np.random.default_rng(seed)
    return np.stack([g.permutation(E)[:k] for _ in range(T)]).astype(np.int32)


def test_moe_sort_matches_nonzero_order():
    T, E, k = 50, 12, 3
    topi = _topi(T, E, k, 1)
    seg, rt, rs, pos = oracle.moe_sort(topi, E)
    row = 0
    for e in range(E):
        tok, slot = np.nonzero(topi == e)      # moe.py:100-103 order
        assert seg[e] == row
        assert rt[row:row + len(tok)].tolist() == tok.tolist()
        assert rs[row:row + len(tok)].tolist() == slot.tolist()
        assert (pos[tok, slot] == np.arange(row, row + len(tok))).all()
        row += len(tok)
    assert seg[E] == T * k


def test_moe_sort_rejects_bad_ids():
    with pytest.raises(ValueError):
        oracle.moe_sort(np.array([[0, 5]], np.int32), 4)


def test_grouped_equals_per_expert_loop():
    T, E, k, K, N = 40, 6, 2, 128, 24
    topi = _topi(T, E, k, 2)
    x = RNG.standard_normal((T, K)).astype(np.float16)
    w = RNG.integers(-127, 128, (E, N, K), dtype=np.int8)
    ws = RNG.uniform(0.001, 0.02, (E, N)).astype(np.float32)
    seg, rt, _, _ = oracle.moe_sort(topi, E)
    aq, as_ = oracle.quant_rowwise_f16(x)
    y, acc = oracle.grouped_w8a8_f16(aq, as_, w, ws, seg, row_index=rt, want_acc=True)
    for e in range(E):
        tok, _ = np.nonzero(topi == e)
        ye, xqe, _, acce = oracle.linear_w8a8_f16(x[tok], w[e], ws[e])  # quantize after gather
        assert np.array_equal(acc[seg[e]:seg[e + 1]], acce)
        assert np.array_equal(y[seg[e]:seg[e + 1]].view(np.uint16), ye.view(np.uint16))


def test_combine_equals_index_add_loop():
    T, E, k, H = 30, 8, 3, 16
    topi = _topi(T, E, k, 3)
    topw = RNG.uniform(0, 1, (T, k)).astype(np.float16)
    _, _, _, pos = oracle.moe_sort(topi, E)
    y = (RNG.standard_normal((T * k, H)) * 4).astype(np.float16)
    out = oracle.moe_combine_f16(y, topi, topw, pos)
    ref = np.zeros((T, H), np.float16)
    for e in range(E):                               # moe.py:99-105
        tok, slot = np.nonzero(topi == e)
        contrib = y[pos[tok, slot]]
        prod = (contrib.astype(np.float32) * topw[tok, slot].astype(np.float32)[:, None]).astype(np.float16)
        ref[tok] = (ref[tok].astype(np.float32) + prod.astype(np.float32)).astype(np.float16)
    assert np.array_equal(out.view(np.uint16), ref.view(np.uint16))
