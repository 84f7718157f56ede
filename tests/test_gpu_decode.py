"""GPU parity of the decode path: for M <= 4 the single-launch linear with the
per-token quantization fused into the GEMM (the dot4 GEMV for M <= 2, the MFMA
kernel for M = 3..4 where K is one of its shapes, else the GEMV), and the same
GEMV on pre-quantized activations; for 4 < M <= 64 the quantize launch plus the
MFMA decode GEMM.

Bar: int8 activations, fp32 scales, int32 accumulators and fp16 outputs are
bit-identical to the CPU oracle on the same seeded inputs.  The fused kernel
quantizes without a per-element division (a correctly rounded reciprocal plus
one FMA correction); the exhaustive and special-value cases below check that it
still reproduces the oracle's division exactly.
"""
import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

SEEDS = {"qkv": 1, "o": 2, "gate_up": 3, "down": 4}


def _same_f32(a, b):
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return np.array_equal(a.view(np.uint32), b.view(np.uint32)) or (
        np.array_equal(np.isnan(a), np.isnan(b)) and np.array_equal(a[~np.isnan(a)], b[~np.isnan(b)]))


def _linear_full(pkg, x, q, s, bias=None, tag=""):
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y, xq, xs, acc = pkg.linear_with_intermediates(
        x.cuda(), qt, None if bias is None else bias.cuda(), want_acc=True)
    torch.cuda.synchronize()
    xn = x.contiguous().numpy() if isinstance(x, torch.Tensor) else x
    yr, xqr, xsr, accr = oracle.linear_w8a8_f16(xn, q.numpy(), s.numpy(),
                                               None if bias is None else bias.numpy())
    assert np.array_equal(xq.cpu().numpy(), xqr), f"{tag}: int8 activations differ"
    assert _same_f32(xs.cpu().numpy(), xsr), f"{tag}: activation scales differ"
    assert np.array_equal(acc.cpu().numpy(), accr), f"{tag}: int32 accumulators differ"
    assert np.array_equal(y.cpu().numpy().view(np.uint16), yr.view(np.uint16)), \
        f"{tag}: fp16 outputs differ"
    print(f"{tag}: bit-exact", flush=True)


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("name", ["qkv", "o", "gate_up", "down"])
def test_fused_decode_bitexact(pkg, wl, cuda, name, M):
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=400 + M)
    q, s = wl.weight_i8(N, K, seed=SEEDS[name] + 20)
    _linear_full(pkg, x, q, s, tag=f"fused decode {name} M={M}")


@pytest.mark.parametrize("M", [1, 2, 3, 4])
@pytest.mark.parametrize("name", ["qkv", "down"])
def test_prequantized_decode_gemm_bitexact(pkg, wl, cuda, name, M):
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=500 + M)
    q, s = wl.weight_i8(N, K, seed=SEEDS[name] + 30)
    xqr, xsr = oracle.quant_rowwise_f16(x.numpy())
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y, acc = pkg.gemm_w8a8(torch.from_numpy(xqr).cuda(), torch.from_numpy(xsr).cuda(), qt,
                           want_acc=True)
    torch.cuda.synchronize()
    accr = oracle.gemm_i8(xqr, q.numpy())
    assert np.array_equal(acc.cpu().numpy(), accr)
    yr = oracle.dequant_f16(accr, xsr, s.numpy())
    assert np.array_equal(y.cpu().numpy().view(np.uint16), yr.view(np.uint16))


@pytest.mark.parametrize("M,N,K", [
    (3, 100, 1024),    # 8 slabs: 2 per wave, 2-slab batches; N not a multiple of 16
    (2, 48, 256),      # 2 slabs: 8 waves do not divide them -> two-launch path
    (4, 130, 384),     # 3 slabs -> two-launch path
    (1, 16, 128),      # the smallest fused shape
    (4, 6144, 8192),   # long K: 8 waves
    (2, 4096, 12288),
    (3, 40, 64),       # K % 128 != 0 -> two-launch path
    (4, 72, 2048),     # MFMA fused, 4 waves x 4 slabs; N not a multiple of 16
    (3, 24, 3072),     # MFMA fused, 2 waves x 12 slabs
    (4, 520, 5120),    # MFMA fused, 2 waves x 20 slabs
    (4, 33, 1536),     # K not 512 * waves * PQ for any entry -> GEMV
])
def test_fused_ragged_bitexact(pkg, wl, cuda, M, N, K):
    x = wl.activations(M, K, seed=M * 13 + K)
    q, s = wl.weight_i8(N, K, seed=N + K + 1)
    _linear_full(pkg, x, q, s, tag=f"fused ragged M={M} N={N} K={K}")


@pytest.mark.parametrize("M", [1, 3])
def test_fused_bias_and_stride(pkg, wl, cuda, M):
    N, K = 640, 2048
    big = wl.activations(M, 3 * K, seed=61)
    x = big[:, K:2 * K]                  # row stride 3K, inner stride 1
    q, s = wl.weight_i8(N, K, seed=62)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(63)) * 2).half()
    _linear_full(pkg, x, q, s, bias=bias, tag=f"fused bias+stride M={M}")


def test_fused_special_rows(pkg, cuda):
    """Zero, subnormal-only, inf, NaN, -65504 and tie rows through the fused path."""
    K, N = 4096, 256
    rows = np.zeros((4, K), np.float16)
    rows[1, 7] = 6e-8                    # subnormal only -> eps scale
    rows[2, :] = np.linspace(-3, 3, K)
    rows[2, 99] = np.inf                 # inf row -> inf scale, q = 0
    rows[3, :] = np.float16(-65504)
    rows[3, ::3] = 2.5
    nan_rows = np.ones((2, K), np.float16)
    nan_rows[1, 1000] = np.nan
    rng = np.random.default_rng(5)
    q = torch.from_numpy(rng.integers(-127, 128, (N, K), dtype=np.int8))
    s = torch.from_numpy(rng.uniform(0.001, 0.02, N).astype(np.float16).astype(np.float32))
    for arr in (rows, nan_rows):
        qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
        y, xq, xs, acc = pkg.linear_with_intermediates(torch.from_numpy(arr).cuda(), qt,
                                                       want_acc=True)
        torch.cuda.synchronize()
        xqr, xsr = oracle.quant_rowwise_f16(arr)
        assert np.array_equal(xq.cpu().numpy(), xqr)
        assert _same_f32(xs.cpu().numpy(), xsr)
        accr = oracle.gemm_i8(xqr, q.numpy())
        assert np.array_equal(acc.cpu().numpy(), accr)
        yr = oracle.dequant_f16(accr, xsr, s.numpy())
        a, b = y.cpu().numpy(), yr
        assert np.array_equal(np.isnan(a), np.isnan(b))
        assert np.array_equal(a[~np.isnan(a)].view(np.uint16), b[~np.isnan(b)].view(np.uint16))


def test_fused_quant_exhaustive_fp16(pkg, cuda):
    """Every finite fp16 value, 8 rows of 8192 (each row led by +-65504 so the
    scale is the largest one), and every fp16 value again under per-row scales
    set by the row's own maximum: the fused quantization equals the oracle's."""
    finite = np.arange(65536, dtype=np.uint16).view(np.float16)
    finite = finite[np.isfinite(finite)]
    K = 8192
    perm = np.random.default_rng(9).permutation(finite.size)
    vals = finite[perm]
    pad = (-vals.size) % K
    arr = np.concatenate([vals, np.zeros(pad, np.float16)]).reshape(-1, K)
    # a second layout: sorted magnitudes, so rows have very different maxima
    arr2 = np.sort(np.abs(finite.astype(np.float32))).astype(np.float16)
    arr2 = np.concatenate([arr2, np.zeros((-arr2.size) % K, np.float16)]).reshape(-1, K)
    arr2 = arr2 * np.where(np.arange(K) % 2 == 0, 1, -1).astype(np.float16)
    N = 32
    q = torch.ones(N, K, dtype=torch.int8)
    s = torch.full((N,), 0.01)
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    for a in (arr, arr2):
        for r0 in range(0, a.shape[0], 4):
            blk = np.ascontiguousarray(a[r0:r0 + 4])
            y, xq, xs, acc = pkg.linear_with_intermediates(torch.from_numpy(blk).cuda(), qt,
                                                           want_acc=True)
            torch.cuda.synchronize()
            xqr, xsr = oracle.quant_rowwise_f16(blk)
            assert np.array_equal(xq.cpu().numpy(), xqr), f"rows {r0}.."
            assert _same_f32(xs.cpu().numpy(), xsr)
            assert np.array_equal(acc.cpu().numpy()[:, 0], xqr.astype(np.int64).sum(1))


@pytest.mark.parametrize("M", [2, 4])
def test_fused_graph_replay(pkg, wl, cuda, M):
    """The fused decode launch (GEMV at M=2, MFMA at M=4) captured in a HIP graph
    equals eager on every replay."""
    qt = pkg.QTensor(*[t.cuda() for t in wl.weight_i8(4096, 4096, seed=71)], scheme="per_row_i8")
    static_x = wl.activations(M, 4096, seed=72).cuda()
    for _ in range(3):
        pkg.linear(static_x, qt)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        static_y = pkg.linear(static_x, qt)
    for i in range(4):
        xi = wl.activations(M, 4096, seed=80 + i).cuda()
        static_x.copy_(xi)
        g.replay()
        eager = pkg.linear(xi, qt)
        torch.cuda.synchronize()
        assert torch.equal(static_y, eager)


# ---- 4 < M <= 64: quantize launch + MFMA decode GEMM -------------------------

@pytest.mark.parametrize("M", [5, 17, 33, 63])
@pytest.mark.parametrize("name", ["qkv", "o", "gate_up", "down"])
def test_mfma_decode_bitexact(pkg, wl, cuda, name, M):
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=600 + M)
    q, s = wl.weight_i8(N, K, seed=SEEDS[name] + 40)
    _linear_full(pkg, x, q, s, tag=f"mfma decode {name} M={M}")


@pytest.mark.parametrize("M,N,K", [
    (12, 48, 384),     # 3 slabs: one wave
    (20, 100, 256),    # 2 slabs: two waves; N not a multiple of 16
    (40, 70, 640),     # 5 slabs
    (64, 16, 1024),
    (9, 4096, 12288),
])
def test_mfma_decode_ragged_bitexact(pkg, wl, cuda, M, N, K):
    x = wl.activations(M, K, seed=M * 3 + K)
    q, s = wl.weight_i8(N, K, seed=N * 7 + K)
    _linear_full(pkg, x, q, s, tag=f"mfma ragged M={M} N={N} K={K}")


def test_mfma_decode_bias_and_stride(pkg, wl, cuda):
    M, N, K = 20, 640, 2048
    big = wl.activations(M, 2 * K, seed=91)
    x = big[:, K:]
    q, s = wl.weight_i8(N, K, seed=92)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(93)) * 2).half()
    _linear_full(pkg, x, q, s, bias=bias, tag="mfma bias+stride M=20")


@pytest.mark.parametrize("M", [3, 4, 16, 32, 64])
@pytest.mark.parametrize("N", [5000, 6150])
def test_24_row_workgroups_ragged_bitexact(pkg, wl, cuda, M, N):
    """Mid-width linears whose workgroup count fits the CUs better in 24-row
    workgroups (three 8-row load groups over two 16-row MFMA blocks; the last
    workgroup holds a partial load group), through the fused kernel (3-4 rows)
    and the MFMA decode GEMM (more rows), with bias; every element against the
    oracle."""
    K = 4096
    x = wl.activations(M, K, seed=M * 29 + N)
    q, s = wl.weight_i8(N, K, seed=N + M)
    bias = torch.from_numpy((np.random.default_rng(N + M).standard_normal(N) * 2).astype(np.float16))
    _linear_full(pkg, x, q, s, bias=bias, tag=f"24-row M={M} N={N}")


@pytest.mark.parametrize("M", [33, 64])
@pytest.mark.parametrize("N", [16400, 16431])
def test_48_row_workgroups_ragged_bitexact(pkg, wl, cuda, M, N):
    """Wide linears at 33..64 rows run 48-row workgroups (three 16-row MFMA
    blocks, six 8-row load groups).  N = 16400 leaves the last workgroup a
    whole MFMA block past N, N = 16431 a partial load group; every element
    against the oracle, with bias."""
    K = 4096
    x = wl.activations(M, K, seed=M * 31 + N)
    q, s = wl.weight_i8(N, K, seed=N + 2 * M)
    bias = torch.from_numpy((np.random.default_rng(N - M).standard_normal(N) * 2).astype(np.float16))
    _linear_full(pkg, x, q, s, bias=bias, tag=f"48-row M={M} N={N}")
