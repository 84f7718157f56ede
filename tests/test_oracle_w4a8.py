"""Pins the W4A8 oracle (oracle/w4a8_oracle.c).

The reference packs int4 weights with fni8serve/convert.py:72-73 and unpacks
them with fni8serve/layers/linear.py:32-40; its `gemm_w4a8` is closed.  The
oracle's integer part is checked exactly against numpy matmuls over codes
packed by the reference's formula; its fp32 fold against the float64 closed
form (error bound of one fma rounding per group plus the two output
roundings) and, on a constructed case, against a different order; the whole
linear against the reference's CPU fallback (dequantize the weight, F.linear)
with the reference's own cosine bar tightened to 0.999.
"""
import numpy as np
import pytest
import torch

from oracle import oracle as o


def _pack_reference(codes: np.ndarray) -> np.ndarray:
    """fni8serve/convert.py:72-73: ((c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4))."""
    c = codes.astype(np.int64)
    return ((c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4)).astype(np.uint8)


def _unpack_reference(packed: np.ndarray) -> np.ndarray:
    """fni8serve/layers/linear.py:33-40 for the int4 codebook."""
    p = packed.astype(np.int32)
    codes = np.stack([p & 0xF, (p >> 4) & 0xF], -1).reshape(p.shape[0], -1)
    return codes - 16 * (codes >= 8)


def _case(M, N, K, G, seed):
    rng = np.random.default_rng(seed)
    xq = rng.integers(-127, 128, size=(M, K)).astype(np.int8)
    xs = (rng.random(M) * 0.05 + 1e-3).astype(np.float32)
    codes = rng.integers(-8, 8, size=(N, K))
    ws = (rng.random((N, K // G)) * 0.02 + 1e-3).astype(np.float32)
    return xq, xs, codes, _pack_reference(codes), ws


def test_packing_round_trips_every_code():
    codes = np.array([list(range(-8, 8)) * 2], dtype=np.int64)
    assert np.array_equal(_unpack_reference(_pack_reference(codes)), codes)


@pytest.mark.parametrize("M,N,K,G", [(3, 17, 256, 32), (5, 64, 512, 64), (2, 40, 1024, 128),
                                     (4, 9, 768, 256), (1, 33, 4096, 128)])
def test_group_sums_are_exact(M, N, K, G):
    xq, xs, codes, packed, ws = _case(M, N, K, G, seed=M * N + K)
    _, ga = o.gemm_w4a8(xq, xs, packed, ws, G, want_groups=True)
    ref = np.einsum("mgk,ngk->mng", xq.astype(np.int64).reshape(M, K // G, G),
                    codes.reshape(N, K // G, G))
    assert np.array_equal(ga.astype(np.int64), ref)
    # extremes: every code -8 and every activation -127 (largest magnitude)
    ex_q = np.full((1, K), -127, np.int8)
    ex_w = _pack_reference(np.full((2, K), -8))
    _, ga = o.gemm_w4a8(ex_q, xs[:1], ex_w, ws[:2], G, want_groups=True)
    assert (ga == 127 * 8 * G).all()


@pytest.mark.parametrize("G", [32, 128])
def test_outputs_against_float64(G):
    M, N, K = 6, 48, 2048
    xq, xs, codes, packed, ws = _case(M, N, K, G, seed=G)
    bias = np.random.default_rng(1).standard_normal(N).astype(np.float16)
    y, ga = o.gemm_w4a8(xq, xs, packed, ws, G, bias=bias, want_groups=True)
    terms = ga.astype(np.float64) * ws.astype(np.float64)[None]          # [M, N, ng]
    exact = terms.sum(-1) * xs.astype(np.float64)[:, None] + bias.astype(np.float64)[None]
    # one fma rounding per group: |error| <= ng * 2^-24 * sum |partial sums|
    bound = (K // G) * 2.0 ** -24 * np.abs(np.cumsum(terms, -1)).sum(-1) * xs[:, None]
    ulp = np.spacing(np.abs(exact).astype(np.float16)).astype(np.float64)
    err = np.abs(y.astype(np.float64) - exact)
    assert (err <= ulp + bound + 2.0 ** -24 * np.abs(exact)).all()


def test_fold_runs_in_ascending_group_order():
    """Three groups whose scaled sums are +2^26, +1 and -2^26: ascending order
    rounds the +1 away (2^26 + 1 is not an fp32 value) and returns 0; any order
    that adds the +1 last returns 1."""
    K, G = 96, 32
    xq = np.zeros((1, K), np.int8)
    xq[0, 0] = 64
    xq[0, 32] = 1
    xq[0, 64] = 64
    codes = np.zeros((1, K), np.int64)
    codes[0, 0] = 1
    codes[0, 32] = 1
    codes[0, 64] = -1
    ws = np.float32([[2.0 ** 20, 1.0, 2.0 ** 20]])
    y, ga = o.gemm_w4a8(xq, np.float32([1.0]), _pack_reference(codes), ws, G, want_groups=True)
    assert list(ga[0, 0]) == [64, 1, -64]
    assert float(y[0, 0]) == 0.0


@pytest.mark.parametrize("G", [32, 128])
def test_linear_against_the_reference_cpu_fallback(G):
    """fni8serve/layers/linear.py:70-71 on the CPU: F.linear(x, _dequant_weight(qt))."""
    rng = np.random.default_rng(G)
    M, N, K = 8, 96, 1024
    x = rng.standard_normal((M, K)).astype(np.float16)
    codes = rng.integers(-8, 8, size=(N, K))
    ws = (rng.random((N, K // G)) * 0.02 + 1e-3).astype(np.float32)
    y, xq, xs = o.linear_w4a8_f16(x, _pack_reference(codes), ws, G)
    q2, s2 = o.quant_rowwise_f16(x)
    assert np.array_equal(xq, q2) and np.array_equal(xs, s2)
    w = (codes.reshape(N, K // G, G) * ws[:, :, None]).reshape(N, K)
    ref = torch.nn.functional.linear(torch.from_numpy(x).float(),
                                     torch.from_numpy(w).float().half().float()).numpy()
    a, b = y.astype(np.float64).ravel(), ref.astype(np.float64).ravel()
    cos = a @ b / np.sqrt((a @ a) * (b @ b))
    assert cos >= 0.999, cos
