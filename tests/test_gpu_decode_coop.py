"""GPU parity of the one-launch decode linear for 5..16 tokens on QKV-, O- and
down-shaped weights (the quantization shared per XCD through a workspace,
fni8_linear_w8a8_f16_ws).

Bar: bit-identical int8 activations, fp32 scales, int32 accumulators and fp16
outputs against the CPU oracle, and against the two-launch path of
fni8_linear_w8a8_f16 on the same inputs.  The workspace needs no clearing, so
the tests reuse one workspace across calls with different activations and
token counts, replay a captured graph on new inputs, and force the bounded
wait's fallback (every workgroup then quantizes the rows itself): each must
still give the same bits."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@pytest.fixture(scope="module")
def lib(pkg):
    from importlib import import_module
    return import_module("fni8serve_amd._lib")


def _call(lib, x, qt, bias=None, work=None, acc=False):
    """fni8_linear_w8a8_f16_ws with `work` (None: fni8_linear_w8a8_f16, two launches)."""
    M, K = x.shape
    N = qt.data.shape[0]
    dev = x.device
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    xq = torch.empty((M, K), dtype=torch.int8, device=dev)
    xs = torch.empty((M,), dtype=torch.float32, device=dev)
    a = torch.empty((M, N), dtype=torch.int32, device=dev) if acc else None
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if work is None:
        lib.call("fni8_linear_w8a8_f16", _ptr(x), x.stride(0), M, K, _ptr(qt.data), _ptr(qt.scale),
                 N, _ptr(bias), _ptr(y), N, _ptr(xq), _ptr(xs), _ptr(a), st)
    else:
        lib.call("fni8_linear_w8a8_f16_ws", _ptr(x), x.stride(0), M, K, _ptr(qt.data),
                 _ptr(qt.scale), N, _ptr(bias), _ptr(y), N, _ptr(xq), _ptr(xs), _ptr(a),
                 _ptr(work), work.numel(), st)
    return y, xq, xs, a


def _bits(t):
    return t.view(torch.int16) if t.dtype == torch.float16 else (
        t.view(torch.int32) if t.dtype == torch.float32 else t)


def _same(a, b):
    return all(torch.equal(_bits(u), _bits(v)) for u, v in zip(a, b) if u is not None)


def _workspace(lib, M, N, K, dev):
    n = lib.workspace_bytes(M, N, K)
    assert n > 0, (M, N, K)
    return torch.empty(n, dtype=torch.uint8, device=dev)


def test_shapes_the_one_launch_path_takes(wl, lib):
    """QKV and down from 5 to 16 tokens, O from 5 to 8; gate_up and other token
    counts keep the two launches (no workspace)."""
    for name, (N, K) in wl.QWEN3_8B_LINEARS.items():
        for M in (1, 4, 5, 8, 9, 16, 17, 64):
            taken = name != "gate_up" and 5 <= M <= (8 if name == "o" else 16)
            assert (lib.workspace_bytes(M, N, K) > 0) == taken, (name, M)


@pytest.mark.parametrize("name,M", [("qkv", 5), ("qkv", 13), ("qkv", 16), ("o", 5), ("o", 8),
                                    ("down", 6), ("down", 11), ("down", 16)])
def test_one_launch_bitexact_against_oracle(pkg, wl, lib, cuda, name, M):
    print(f"coop oracle {name} M={M}", flush=True)
    N, K = wl.QWEN3_8B_LINEARS[name]
    x = wl.activations(M, K, seed=900 + M)
    q, s = wl.weight_i8(N, K, seed=910 + len(name))
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(920 + M)) * 2).half()
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y, xq, xs, acc = _call(lib, x.cuda(), qt, bias.cuda(), _workspace(lib, M, N, K, cuda),
                           acc=True)
    torch.cuda.synchronize()
    yr, xqr, xsr, accr = oracle.linear_w8a8_f16(x.numpy(), q.numpy(), s.numpy(), bias.numpy())
    assert np.array_equal(xq.cpu().numpy(), xqr)
    assert np.array_equal(xs.cpu().numpy().view(np.uint32), xsr.view(np.uint32))
    assert np.array_equal(acc.cpu().numpy(), accr)
    assert np.array_equal(y.cpu().numpy().view(np.uint16), yr.view(np.uint16))


@pytest.mark.parametrize("name", ["qkv", "o", "down"])
def test_one_launch_equals_two_launches_every_M(pkg, wl, lib, cuda, name):
    """Every token count the path takes (5..16), one shared workspace reused
    across all calls, against the two-launch path on the same inputs."""
    N, K = wl.QWEN3_8B_LINEARS[name]
    q, s = wl.weight_i8(N, K, seed=930 + len(name))
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    top = 8 if name == "o" else 16
    work = _workspace(lib, top, N, K, cuda)
    for M in range(5, top + 1):
        x = wl.activations(M, K, seed=940 + M).cuda()
        got = _call(lib, x, qt, None, work, acc=True)
        ref = _call(lib, x, qt, None, None, acc=True)
        torch.cuda.synchronize()
        assert _same(got, ref), f"{name} M={M}"
    print(f"coop vs two launches {name}: M=5..{top} bit-identical", flush=True)


def test_stale_workspace_never_leaks(pkg, wl, lib, cuda):
    """Back-to-back calls on one workspace whose activations differ only in
    value (same M, K), then with fewer tokens, then after the two-launch path
    wrote different rows: each call's output is its own."""
    N, K = wl.QWEN3_8B_LINEARS["qkv"]
    q, s = wl.weight_i8(N, K, seed=950)
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    work = _workspace(lib, 16, N, K, cuda)
    seq = [(16, 1), (16, 2), (16, 3), (8, 4), (12, 5), (5, 6), (16, 7)]
    outs = [_call(lib, wl.activations(M, K, seed=960 + sd).cuda(), qt, None, work) for M, sd in seq]
    torch.cuda.synchronize()
    for (M, sd), got in zip(seq, outs):
        ref = _call(lib, wl.activations(M, K, seed=960 + sd).cuda(), qt, None, None)
        torch.cuda.synchronize()
        assert _same(got, ref), f"M={M} seed={sd}"


def test_forced_fallback_gives_the_same_bits(pkg, wl, lib, cuda):
    """With the wait bound at 0, GEMM workgroups that do not find their rows at
    the first look quantize them themselves; the result does not change."""
    raw = lib.load()
    try:
        for name, M in (("o", 8), ("qkv", 9), ("down", 12), ("o", 5), ("qkv", 16)):
            N, K = wl.QWEN3_8B_LINEARS[name]
            q, s = wl.weight_i8(N, K, seed=970 + M)
            qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
            x = wl.activations(M, K, seed=980 + M).cuda()
            ref = _call(lib, x, qt, None, None, acc=True)
            raw.fni8_debug_coop_wait_ticks(0)
            got = _call(lib, x, qt, None, _workspace(lib, M, N, K, cuda), acc=True)
            raw.fni8_debug_coop_wait_ticks(-1)
            torch.cuda.synchronize()
            assert _same(got, ref), f"{name} M={M}"
    finally:
        raw.fni8_debug_coop_wait_ticks(-1)


def test_graph_replays_on_new_inputs(pkg, wl, cuda):
    """`linear()` at 8 and 12 tokens captured in one HIP graph (workspace from
    the graph's pool), replayed five times with new activations copied in
    between, the program's own eager work and synchronisations around each
    replay: every replay equals the eager two-launch result."""
    from importlib import import_module
    lib = import_module("fni8serve_amd._lib")
    shapes = {"o": 8, "down": 12}
    qts, xin = {}, {}
    for i, (name, M) in enumerate(shapes.items()):
        N, K = wl.QWEN3_8B_LINEARS[name]
        q, s = wl.weight_i8(N, K, seed=990 + i)
        qts[name] = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
        xin[name] = torch.empty((M, K), dtype=torch.float16, device=cuda)
        xin[name].copy_(wl.activations(M, K, seed=1000 + i).cuda())
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        for name in shapes:
            pkg.linear(xin[name], qts[name])
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = {name: pkg.linear(xin[name], qts[name]) for name in shapes}
    for rep in range(5):
        for i, (name, M) in enumerate(shapes.items()):
            N, K = wl.QWEN3_8B_LINEARS[name]
            xin[name].copy_(wl.activations(M, K, seed=1100 + 10 * rep + i).cuda())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name in shapes:
            ref = _call(lib, xin[name].clone(), qts[name], None, None)[0]
            torch.cuda.synchronize()
            assert torch.equal(outs[name].view(torch.int16), ref.view(torch.int16)), \
                f"replay {rep} {name}"


def test_nonfinite_and_zero_rows(pkg, wl, lib, cuda):
    """NaN, inf and all-zero token rows through the producers: their rows
    quantize to 0 (NaN/inf scale) or to 0 with the 1e-6 floor, as the oracle does."""
    N, K = wl.QWEN3_8B_LINEARS["qkv"]
    M = 12
    x = wl.activations(M, K, seed=1200)
    x[2, 7] = float("nan")
    x[5, 100] = float("inf")
    x[7] = 0
    x[9, :] = 1e-7
    q, s = wl.weight_i8(N, K, seed=1201)
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    y, xq, xs, acc = _call(lib, x.cuda(), qt, None, _workspace(lib, M, N, K, cuda), acc=True)
    torch.cuda.synchronize()
    yr, xqr, xsr, accr = oracle.linear_w8a8_f16(x.numpy(), q.numpy(), s.numpy(), None)
    assert np.array_equal(xq.cpu().numpy(), xqr)
    got_s, ref_s = xs.cpu().numpy(), xsr
    assert np.array_equal(np.isnan(got_s), np.isnan(ref_s))
    fin = ~np.isnan(ref_s)
    assert np.array_equal(got_s[fin].view(np.uint32), ref_s[fin].view(np.uint32))
    assert np.array_equal(acc.cpu().numpy(), accr)
    yb, yrb = y.cpu().numpy(), yr
    assert np.array_equal(np.isnan(yb), np.isnan(yrb))
    ok = ~np.isnan(yrb)
    assert np.array_equal(yb[ok].view(np.uint16), yrb[ok].view(np.uint16))


@pytest.mark.parametrize("N", [8, 100, 1000])
def test_small_and_ragged_N(pkg, wl, lib, cuda, N):
    """Few or partial GEMM workgroups (N = 8 is one 16-row workgroup; rows past N
    are loaded but never stored), and the strided activation rows of a slice."""
    K, M = 4096, 8
    base = wl.activations(M, 2 * K, seed=1300 + N).cuda()
    x = base[:, :K]          # row stride 2K
    q, s = wl.weight_i8(N, K, seed=1301 + N)
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    got = _call(lib, x, qt, None, _workspace(lib, M, N, K, cuda), acc=True)
    ref = _call(lib, x, qt, None, None, acc=True)
    torch.cuda.synchronize()
    assert _same(got, ref)

