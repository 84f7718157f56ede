"""GPU parity of the W8A8 linear (quantize, GEMM, epilogue) against the CPU oracle.

Bar: int8 activations, fp32 scales, int32 accumulators and fp16 outputs are
bit-identical to the oracle on the same seeded inputs.  The fp16 output's error
against the fp64 closed form is also bounded (one fp16 rounding plus fp32
rounding of the scale products).  At prefill sizes, where the oracle GEMM
would take minutes, every row's quantization is checked in full and the GEMM
on a sample of rows (each output row depends only on its own input row).
"""
import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

SEEDS = {"qkv": 1, "o": 2, "gate_up": 3, "down": 4}


def _f16bits(t):
    return t.cpu().numpy().view(np.uint16)


def _same_f32(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or (
        np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)]))


def _run(pkg, x, q, s, bias=None):
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y, xq, xs, acc = pkg.linear_with_intermediates(
        x.cuda(), qt, None if bias is None else bias.cuda(), want_acc=True)
    torch.cuda.synchronize()
    return y.cpu(), xq.cpu().numpy(), xs.cpu().numpy(), acc.cpu().numpy()


def _check_full(pkg, x, q, s, bias=None, tag=""):
    y, xq, xs, acc = _run(pkg, x, q, s, bias)
    yr, xqr, xsr, accr = oracle.linear_w8a8_f16(x.numpy(), q.numpy(), s.numpy(),
                                               None if bias is None else bias.numpy())
    assert np.array_equal(xq, xqr), f"{tag}: int8 activations differ"
    assert _same_f32(xs, xsr), f"{tag}: activation scales differ"
    assert np.array_equal(acc, accr), f"{tag}: int32 accumulators differ"
    assert np.array_equal(_f16bits(y), yr.view(np.uint16)), f"{tag}: fp16 outputs differ"
    # fp64 closed form of the epilogue from the exact accumulators
    exact = accr.astype(np.float64) * xsr[:, None].astype(np.float64) * s.numpy()[None, :].astype(np.float64)
    if bias is not None:
        exact = exact + bias.numpy().astype(np.float64)[None, :]
    yf = y.numpy().astype(np.float64)
    fin = np.isfinite(exact) & (np.abs(exact) < 65504)
    err = np.abs(yf[fin] - exact[fin])
    tol = np.abs(exact[fin]) * (2.0 ** -11 + 2.0 ** -22) + 2.0 ** -24
    assert np.all(err <= tol), f"{tag}: fp16 error beyond one rounding (max {err.max()})"
    rel = (err / np.maximum(np.abs(exact[fin]), 1e-30)).max() if err.size else 0.0
    print(f"{tag}: bit-exact; max abs err {err.max() if err.size else 0:.3g} "
          f"max rel err {rel:.3g}", flush=True)


@pytest.mark.parametrize("M", [1, 4, 16, 32, 64])
@pytest.mark.parametrize("name", ["qkv", "o", "gate_up", "down"])
def test_decode_linear_bitexact(pkg, wl, cuda, name, M):
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=100 + M)
    q, s = wl.weight_i8(N, K, seed=SEEDS[name])
    _check_full(pkg, x, q, s, tag=f"decode {name} M={M}")


def test_cpu_case_bitexact(pkg, wl, cuda):
    c = wl.CPU_CASE
    x = wl.activations(c["M"], c["K"], seed=7)
    q, s = wl.weight_i8(c["N"], c["K"], seed=8)
    _check_full(pkg, x, q, s, tag="qwen3-0.6b gate_up M=8")


@pytest.mark.parametrize("N,K", [(768, 2048), (16384, 512), (256, 12288)])
def test_decode_every_token_count_bitexact(pkg, wl, cuda, N, K):
    """Every token count from 1 to 64 through linear(): the fused-quantization
    kernels up to 4 tokens, the one- or two-launch paths up to 16, the MFMA
    GEMM's 16-, 32- and 64-token blocks above, on a generic, a wide (N >= 16384)
    and a long-K shape; every intermediate bit for bit against the oracle."""
    q, s = wl.weight_i8(N, K, seed=N + K)
    for M in range(1, 65):
        x = wl.activations(M, K, seed=31 * M + K)
        _check_full(pkg, x, q, s, tag=f"M={M} N={N} K={K}")


@pytest.mark.parametrize("M,N,K", [
    (3, 100, 256), (17, 48, 512), (33, 4096, 4096), (65, 256, 1024), (100, 640, 2048),
    (257, 384, 1024), (130, 130, 128), (8, 16, 64), (64, 1000, 192),
    (5, 64, 1028), (7, 33, 36), (70, 20, 100),     # K % 64 != 0: generic kernel
])
def test_ragged_shapes_bitexact(pkg, wl, cuda, M, N, K):
    x = wl.activations(M, K, seed=M * 7 + K)
    q, s = wl.weight_i8(N, K, seed=N + K)
    _check_full(pkg, x, q, s, tag=f"ragged M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [1, 16, 300])
def test_bias_bitexact(pkg, wl, cuda, M):
    N, K = 512, 1024
    x = wl.activations(M, K, seed=11)
    q, s = wl.weight_i8(N, K, seed=12)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(13)) * 3).half()
    _check_full(pkg, x, q, s, bias=bias, tag=f"bias M={M}")


@pytest.mark.parametrize("M", [512, 2048, 4096])
@pytest.mark.parametrize("name", ["qkv", "o", "gate_up", "down"])
def test_prefill_linear_rows(pkg, wl, cuda, name, M):
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=200 + M)
    q, s = wl.weight_i8(N, K, seed=10 + SEEDS[name])
    y, xq, xs, acc = _run(pkg, x, q, s)
    xqr, xsr = oracle.quant_rowwise_f16(x.numpy())
    assert np.array_equal(xq, xqr) and _same_f32(xs, xsr), "quantization differs"
    rng = np.random.default_rng(M)
    rows = np.unique(np.concatenate([[0, M - 1], rng.choice(M, 30, replace=False)]))
    accr = oracle.gemm_i8(xqr[rows], q.numpy())
    assert np.array_equal(acc[rows], accr), "int32 accumulators differ"
    yr = oracle.dequant_f16(accr, xsr[rows], s.numpy())
    assert np.array_equal(_f16bits(y)[rows], yr.view(np.uint16)), "fp16 outputs differ"
    print(f"prefill {name} M={M}: quant full + {len(rows)} GEMM rows bit-exact", flush=True)


def _sample_rows(M, seed, n=30):
    rng = np.random.default_rng(seed)
    return np.unique(np.concatenate([[0, M - 1], rng.choice(M, min(n, M), replace=False)]))


@pytest.mark.parametrize("M", [65, 512, 2048, 4096])
@pytest.mark.parametrize("name", ["qkv", "o", "gate_up", "down"])
def test_prefill_shipped_kernel_rows(pkg, wl, cuda, name, M):
    """`linear()` exactly as shipped: no accumulator output, so the kernel
    instantiation production and the benchmark run (not the parity-only one that
    also stores int32 accumulators).  fp16 outputs of sampled rows against the
    oracle, bit for bit."""
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=300 + M)
    q, s = wl.weight_i8(N, K, seed=20 + SEEDS[name])
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y = pkg.linear(x.cuda(), qt)
    torch.cuda.synchronize()
    xqr, xsr = oracle.quant_rowwise_f16(x.numpy())
    rows = _sample_rows(M, M + N)
    yr = oracle.dequant_f16(oracle.gemm_i8(xqr[rows], q.numpy()), xsr[rows], s.numpy())
    assert np.array_equal(_f16bits(y)[rows], yr.view(np.uint16)), f"{name} M={M}: fp16 outputs differ"


@pytest.mark.parametrize("name,M", [("o", 1), ("o", 2), ("o", 4), ("qkv", 4), ("o", 16),
                                    ("down", 16), ("qkv", 64), ("gate_up", 33)])
def test_decode_shipped_kernel_full(pkg, wl, cuda, name, M):
    """One decode shape per kernel family (fused GEMV, fused MFMA, quantize + MFMA
    decode GEMM) through `linear()` without accumulators, every output bit."""
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=400 + M)
    q, s = wl.weight_i8(N, K, seed=30 + SEEDS[name])
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y = pkg.linear(x.cuda(), qt)
    torch.cuda.synchronize()
    yr, _, _, _ = oracle.linear_w8a8_f16(x.numpy(), q.numpy(), s.numpy(), None)
    assert np.array_equal(_f16bits(y), yr.view(np.uint16))


def test_prefill_bias_shipped_kernel(pkg, wl, cuda):
    """Bias in the prefill epilogue, shipped instantiation, ragged M and N."""
    M, N, K = 700, 1000, 1024
    x = wl.activations(M, K, seed=41)
    q, s = wl.weight_i8(N, K, seed=42)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(43)) * 3).half()
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y = pkg.linear(x.cuda(), qt, bias.cuda())
    torch.cuda.synchronize()
    yr, _, _, _ = oracle.linear_w8a8_f16(x.numpy(), q.numpy(), s.numpy(), bias.numpy())
    assert np.array_equal(_f16bits(y), yr.view(np.uint16))


@pytest.mark.parametrize("want_acc", [False, True])
@pytest.mark.parametrize("M,N,K", [(4096, 4096, 1024), (600, 1003, 512)])
def test_tile_epilogue_special_values(pkg, cuda, M, N, K, want_acc):
    """The tile kernels' epilogue (the ping-pong kernel at 4096x4096, the 8-wave
    tile kernel at 600x1003: ragged columns, rows not 16-byte aligned) on scales chosen to push fp16 outputs to overflow
    (inf), into the subnormal range, to signed zeros (all-zero rows, zero and
    -0 column scales and bias) and to NaN (one NaN row scale): fp16 bits against
    the oracle's epilogue on sampled rows, NaN positions against NaN positions."""
    rng = np.random.default_rng(7000 + M)
    xq = rng.integers(-127, 128, size=(M, K), dtype=np.int8)
    xq[3] = 0
    xq[M - 2] = 0
    q = rng.integers(-127, 128, size=(N, K), dtype=np.int8)
    xs = (10.0 ** rng.uniform(-12, 2, size=M)).astype(np.float32)
    xs[rng.random(M) < 0.25] *= -1
    xs[3] = 1.0                # zero row: +0 * s, and -0 where s < 0 and bias is -0
    xs[5] = np.float32(1e3)    # |acc| ~1e5 -> overflow
    xs[6] = np.float32(1e-10)  # products in the fp16 subnormal range
    xs[7] = np.nan
    s = (10.0 ** rng.uniform(-6, 0, size=N)).astype(np.float32)
    s[rng.random(N) < 0.3] *= -1
    s[1] = 0.0
    s[2] = -0.0
    s[4] = np.float32(-1e-3)
    bias = (rng.standard_normal(N) * 1e-3).astype(np.float16)
    bias[rng.random(N) < 0.5] = 0
    bias[4] = np.float16(-0.0)
    qt = pkg.QTensor(torch.from_numpy(q).cuda(), torch.from_numpy(s).cuda(), scheme="per_row_i8")
    out = pkg.gemm_w8a8(torch.from_numpy(xq).cuda(), torch.from_numpy(xs).cuda(), qt,
                            torch.from_numpy(bias).cuda(), want_acc=want_acc)
    torch.cuda.synchronize()
    y, acc = out if want_acc else (out, None)
    rows = np.unique(np.concatenate([np.arange(0, 9), _sample_rows(M, M + N), [M - 2, M - 1]]))
    accr = oracle.gemm_i8(xq[rows], q)
    if want_acc:
        assert np.array_equal(acc.cpu().numpy()[rows], accr), "int32 accumulators differ"
    yr = oracle.dequant_f16(accr, xs[rows], s, bias).view(np.uint16)
    yb = _f16bits(y)[rows]
    nan_r = np.isnan(yr.view(np.float16))
    assert np.array_equal(np.isnan(yb.view(np.float16)), nan_r), "NaN positions differ"
    assert np.array_equal(yb[~nan_r], yr[~nan_r]), "fp16 outputs differ"
    yf = yr.view(np.float16)
    # the chosen scales really reach every special class
    assert np.isinf(yf).any() and nan_r.any()
    assert ((yf != 0) & (np.abs(yf.astype(np.float32)) < 2.0 ** -14)).any()
    assert (yr == 0x8000).any() and (yr == 0).any()


@pytest.mark.parametrize("want_acc", [False, True])
def test_prefill_tile_192_ragged(pkg, wl, cuda, want_acc):
    """The 256x192 prefill tile (chosen when it fills the CUs in fewer
    tile-rounds) with a partial last row tile (2000 = 7*256 + 208) and a
    partial last column tile (6080 = 31*192 + 128), with bias; both kernel
    instantiations (with and without the accumulator output), sampled rows
    including the last ones, against the oracle bit for bit."""
    M, N, K = 2000, 6080, 1024
    x = wl.activations(M, K, seed=61)
    q, s = wl.weight_i8(N, K, seed=62)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(63)) * 2).half()
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y, xq, xs, acc = pkg.linear_with_intermediates(x.cuda(), qt, bias.cuda(), want_acc=want_acc)
    torch.cuda.synchronize()
    xqr, xsr = oracle.quant_rowwise_f16(x.numpy())
    rows = np.unique(np.concatenate([_sample_rows(M, 64), np.arange(M - 50, M)]))
    accr = oracle.gemm_i8(xqr[rows], q.numpy())
    if want_acc:
        assert np.array_equal(acc.cpu().numpy()[rows], accr), "int32 accumulators differ"
    yr = oracle.dequant_f16(accr, xsr[rows], s.numpy(), bias.numpy())
    assert np.array_equal(_f16bits(y)[rows], yr.view(np.uint16)), "fp16 outputs differ"


def test_quant_exhaustive_fp16(pkg, cuda):
    """Every fp16 bit pattern, in rows of 1024 (rows with inf/NaN get an inf/NaN
    scale), plus the same values under one fixed large scale."""
    allv = np.arange(65536, dtype=np.uint16).view(np.float16).reshape(64, 1024)
    finite = np.arange(65536, dtype=np.uint16).view(np.float16)
    finite = finite[np.isfinite(finite)]
    pad = (-finite.size) % 1023
    f2 = np.concatenate([finite, np.zeros(pad, np.float16)]).reshape(-1, 1023)
    f2 = np.concatenate([np.full((f2.shape[0], 1), 65504, np.float16), f2], axis=1)
    for arr in (allv, f2):
        xq, xs = pkg.quantize_rowwise(torch.from_numpy(arr.copy()).cuda())
        torch.cuda.synchronize()
        qr, sr = oracle.quant_rowwise_f16(arr)
        assert np.array_equal(xq.cpu().numpy(), qr)
        assert _same_f32(xs.cpu().numpy(), sr)


def test_quant_special_rows(pkg, cuda):
    x = np.zeros((6, 256), np.float16)
    x[1, 3] = 1e-7                      # subnormal-only row -> eps scale
    x[2, :] = np.linspace(-3, 3, 256)
    x[2, 17] = np.inf
    x[3, :] = 1.0
    x[3, 5] = np.nan
    x[4, :] = np.float16(-65504)
    x[5, ::2] = 2.5
    x[5, 1::2] = -127
    xq, xs = pkg.quantize_rowwise(torch.from_numpy(x).cuda())
    qr, sr = oracle.quant_rowwise_f16(x)
    assert np.array_equal(xq.cpu().numpy(), qr)
    assert _same_f32(xs.cpu().numpy(), sr)


def test_strided_and_3d_inputs(pkg, wl, cuda):
    """hidden[:, -1] (row stride S*K, fni8serve/layers/embedding.py:49-53) and [B, S, K]."""
    B, S, K, N = 4, 5, 1024, 768
    h = wl.activations(B * S, K, seed=31).reshape(B, S, K)
    q, s = wl.weight_i8(N, K, seed=32)
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    hg = h.cuda()
    last = hg[:, -1]
    assert not last.is_contiguous()
    y = pkg.linear(last, qt)
    yr, *_ = oracle.linear_w8a8_f16(h[:, -1].contiguous().numpy(), q.numpy(), s.numpy())
    assert np.array_equal(_f16bits(y), yr.view(np.uint16))
    y3 = pkg.linear(hg, qt)
    assert y3.shape == (B, S, N)
    yr3, *_ = oracle.linear_w8a8_f16(h.reshape(-1, K).numpy(), q.numpy(), s.numpy())
    assert np.array_equal(_f16bits(y3).reshape(-1, N), yr3.view(np.uint16))


def test_empty_batch(pkg, cuda):
    qt = pkg.QTensor(torch.zeros(64, 128, dtype=torch.int8, device="cuda"),
                     torch.ones(64, device="cuda"), scheme="per_row_i8")
    y = pkg.linear(torch.zeros(0, 128, dtype=torch.float16, device="cuda"), qt)
    assert y.shape == (0, 64)


def test_module_matches_fp16_reference(pkg, cuda):
    """The reference's own bar (tests/test_smoke.py:68-80): cosine >= 0.99 between
    the int8 path and F.linear over the dequantized weight."""
    torch.manual_seed(0)
    w = torch.randn(256, 512)
    qw, sw = pkg.quantize_int8_rowwise(w)
    qt = pkg.QTensor(qw.cuda(), sw.squeeze(-1).float().cuda(), scheme="per_row_i8")
    lin = pkg.LinearW8A8(qt)
    x = torch.randn(16, 512, device="cuda", dtype=torch.float16)
    y = lin(x)
    ref = torch.nn.functional.linear(x, pkg._dequant_weight(qt).to(x.dtype))
    cos = torch.nn.functional.cosine_similarity(y.flatten().float(), ref.flatten().float(), dim=0)
    assert cos.item() >= 0.99 and torch.isfinite(y).all()


def test_graph_replay_matches_eager(pkg, wl, cuda):
    """Captured in a HIP graph, replayed with eager work in between: every replay
    equals the eager result bit-for-bit (tests/test_cuda_graph.py:72-90)."""
    qt = pkg.QTensor(*[t.cuda() for t in wl.weight_i8(4096, 4096, seed=41)], scheme="per_row_i8")
    qt2 = pkg.QTensor(*[t.cuda() for t in wl.weight_i8(1024, 4096, seed=42)], scheme="per_row_i8")
    xs_in = [wl.activations(m, 4096, seed=43 + m).cuda() for m in (8, 8, 8)]
    static_x = xs_in[0].clone()
    for _ in range(3):  # warm up on a side stream, as graph capture requires
        pkg.linear(pkg.linear(static_x, qt), qt2)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_y = pkg.linear(pkg.linear(static_x, qt), qt2)
    for xi in xs_in + [wl.activations(300, 4096, seed=50).cuda()[:8]]:
        static_x.copy_(xi)
        g.replay()
        eager = pkg.linear(pkg.linear(xi, qt), qt2)
        torch.cuda.synchronize()
        assert torch.equal(static_y, eager)


def test_repeat_runs_identical(pkg, wl, cuda):
    qt = pkg.QTensor(*[t.cuda() for t in wl.weight_i8(6144, 4096, seed=51)], scheme="per_row_i8")
    for M in (4, 512):
        x = wl.activations(M, 4096, seed=52).cuda()
        a = pkg.linear(x, qt)
        b = pkg.linear(x, qt)
        assert torch.equal(a, b)


def test_argument_errors_on_gpu(pkg, cuda):
    qt = pkg.QTensor(torch.zeros(32, 64, dtype=torch.int8, device="cuda"),
                     torch.ones(32, device="cuda"), scheme="per_row_i8")
    with pytest.raises(ValueError):
        pkg.linear(torch.zeros(2, 60, dtype=torch.float16, device="cuda"), qt)  # K mismatch
    with pytest.raises(ValueError):
        pkg.linear(torch.zeros(2, 64, dtype=torch.bfloat16, device="cuda"), qt)
    bad = pkg.QTensor(torch.zeros(32, 66, dtype=torch.int8, device="cuda"),
                      torch.ones(32, device="cuda"), scheme="per_row_i8")
    with pytest.raises(ValueError, match="multiple of 4"):
        pkg.linear(torch.zeros(2, 66, dtype=torch.float16, device="cuda"), bad)
