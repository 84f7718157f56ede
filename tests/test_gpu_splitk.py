"""GPU parity of the prefill GEMM with K split over 2 or 4 workgroups per output
tile (fni8_gemm_w8a8_ws, and fni8_linear_w8a8_f16_ws at prefill sizes): the
workgroups of the first splits hand their int32 partial tiles over through the
workspace, and the tile's owner (the last split) adds them up -- or, if one
does not arrive within the wait bound, recomputes the whole tile -- and runs the
epilogue.

Bar: bit-identical int32 accumulators and fp16 outputs against the CPU oracle
(every output at the small ragged shape, sampled rows at Qwen3-8B's), and
against the unsplit GEMM on the same inputs under every tile and split, on both
of the owner's paths (merged, and recomputed with the wait bound forced to 0).
The workspace needs no clearing, so the tests fill it with garbage first, reuse
it across calls, and replay a captured graph on new inputs.  On a zeroed
workspace each tile's owner leaves a merge mark in the flag region of its XCD:
exactly one mark per tile proves that the split kernel ran and that the
hand-over took the merge path."""
import ctypes

import numpy as np
import pytest
import torch

from oracle import oracle

pytestmark = pytest.mark.gpu

SPLIT_PLANS = [(256, 256, 2), (256, 256, 4), (128, 256, 2), (128, 256, 4), (256, 128, 2),
               (256, 128, 4), (64, 128, 2), (64, 128, 4)]


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


@pytest.fixture(scope="module")
def lib(pkg):
    from importlib import import_module
    return import_module("fni8serve_amd._lib")


@pytest.fixture
def plan(lib):
    """Sets a forced plan for one test and restores the automatic choice after it."""
    def force(bm, bn, split):
        lib.load().fni8_debug_gemm_plan(bm, bn, split)
    yield force
    lib.load().fni8_debug_gemm_plan(0, 0, 0)


def _gemm(lib, xq, xs, q, s, bias=None, work=None, acc=False):
    """fni8_gemm_w8a8_ws (fni8_gemm_w8a8 when work is None)."""
    M, K = xq.shape
    N = q.shape[0]
    dev = xq.device
    y = torch.empty((M, N), dtype=torch.float16, device=dev)
    a = torch.empty((M, N), dtype=torch.int32, device=dev) if acc else None
    st = ctypes.c_void_p(torch.cuda.current_stream(dev).cuda_stream)
    if work is None:
        lib.call("fni8_gemm_w8a8", _ptr(xq), K, _ptr(xs), M, K, _ptr(q), _ptr(s), N, _ptr(bias),
                 _ptr(y), N, _ptr(a), st)
    else:
        lib.call("fni8_gemm_w8a8_ws", _ptr(xq), K, _ptr(xs), M, K, _ptr(q), _ptr(s), N,
                 _ptr(bias), _ptr(y), N, _ptr(a), _ptr(work), work.numel(), st)
    return y, a


def _tiles(M, N, bm, bn):
    return -(-M // bm) * -(-N // bn)


def _merge_marks(work, tiles, split):
    """Per tile, the owner's merge marks summed over the 8 XCD flag regions
    (region x, tile t, split s: 128-byte line (x*tiles + t)*split + s)."""
    f = work[:8 * tiles * split * 128].view(torch.int64).view(8, tiles, split, 16)
    return f[:, :, split - 1, 0].sum(dim=0).cpu().numpy()


def _stale(nbytes, seed, dev):
    """A workspace full of garbage, counters included."""
    g = torch.Generator().manual_seed(seed)
    return torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g).to(dev)


def _inputs(wl, M, N, K, seed):
    x = wl.activations(M, K, seed=seed)
    q, s = wl.weight_i8(N, K, seed=seed + 1)
    xq, xs = oracle.quant_rowwise_f16(x.numpy())
    return xq, xs, q, s


@pytest.mark.parametrize("bm,bn,split", SPLIT_PLANS)
def test_split_plans_bitexact_small(lib, plan, wl, cuda, bm, bn, split):
    """M = 500, N = 1000 (ragged in both, 8 to 64 tiles), K = 1024 (8 k-tiles:
    2 or 4 per split), with bias and accumulators: every output against the
    oracle, on a zeroed workspace (one merge mark per tile), then on a workspace
    of stale bytes, then with the wait bound at 0 (owners recompute)."""
    M, N, K = 500, 1000, 1024
    xq, xs, q, s = _inputs(wl, M, N, K, seed=1100 + 10 * split + bm // 128)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(5)) * 3).half()
    plan(bm, bn, split)
    nw = lib.workspace_bytes(M, N, K)
    tiles = _tiles(M, N, bm, bn)
    assert nw >= tiles * (split - 1) * bm * bn * 4, f"plan {bm}x{bn}/{split} not taken ({nw} B)"
    accr = oracle.gemm_i8(xq, q.numpy())
    yr = oracle.dequant_f16(accr, xs, s.numpy(), bias.numpy())
    raw = lib.load()
    for case in ("zeroed", "stale", "recompute"):
        work = torch.zeros(nw, dtype=torch.uint8, device=cuda) if case == "zeroed" \
            else _stale(nw, 7, cuda)
        if case == "recompute":
            raw.fni8_debug_coop_wait_ticks(0)
        try:
            y, a = _gemm(lib, torch.from_numpy(xq).to(cuda), torch.from_numpy(xs).to(cuda),
                         q.to(cuda), s.to(cuda), bias.to(cuda), work, acc=True)
            torch.cuda.synchronize()
        finally:
            raw.fni8_debug_coop_wait_ticks(-1)
        assert np.array_equal(a.cpu().numpy(), accr), f"{case}: int32 accumulators differ"
        assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16),
                              yr.view(np.uint16)), f"{case}: fp16 outputs differ"
        if case == "zeroed":
            marks = _merge_marks(work, tiles, split)
            assert np.all(marks == 1), f"merge marks per tile {marks}"


@pytest.mark.parametrize("bm,bn,split", SPLIT_PLANS)
def test_split_equals_unsplit_shipped_instantiation(lib, plan, wl, cuda, bm, bn, split):
    """No accumulator output (the instantiation production runs), no bias: the
    split plan against the unsplit GEMM, every output bit, on M = 1000,
    N = 1536, K = 4096; then a second call on the same workspace with other
    activations (its counters then hold the first call's tag)."""
    M, N, K = 1000, 1536, 4096
    if _tiles(M, N, bm, bn) % 8:
        M = 1024
    xq, xs, q, s = _inputs(wl, M, N, K, seed=1200 + 10 * split + bm // 128)
    qd, sd = q.to(cuda), s.to(cuda)
    plan(bm, bn, split)
    nw = lib.workspace_bytes(M, N, K)
    assert nw > 0
    work = _stale(nw, 8, cuda)
    for call in range(2):
        if call:
            xq = np.ascontiguousarray(np.roll(xq, 37, axis=0))
            xs = np.ascontiguousarray(np.roll(xs, 37))
        xqd, xsd = torch.from_numpy(xq).to(cuda), torch.from_numpy(xs).to(cuda)
        y, _ = _gemm(lib, xqd, xsd, qd, sd, work=work)
        torch.cuda.synchronize()
        plan(bm, bn, 1)
        yu, _ = _gemm(lib, xqd, xsd, qd, sd, work=work)
        torch.cuda.synchronize()
        plan(bm, bn, split)
        assert torch.equal(y.view(torch.int16), yu.view(torch.int16)), f"call {call}"
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(3).choice(M, 20)]))
    yr = oracle.dequant_f16(oracle.gemm_i8(xq[rows], q.numpy()), xs[rows], s.numpy())
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16)[rows],
                          yr.view(np.uint16))


def test_back_to_back_calls_share_a_workspace(lib, plan, wl, cuda):
    """Four split GEMMs issued back to back on one workspace (adjacent dispatches,
    whose tags differ only in their lowest bits), each on other activations:
    none may take the counters or partial tiles of the one before."""
    M, N, K = 512, 1024, 2048
    q, s = wl.weight_i8(N, K, seed=1350)
    qd, sd = q.to(cuda), s.to(cuda)
    xs_in = []
    for i in range(4):
        xq, xs = oracle.quant_rowwise_f16(wl.activations(M, K, seed=1351 + i).numpy())
        xs_in.append((torch.from_numpy(xq).to(cuda), torch.from_numpy(xs).to(cuda)))
    plan(256, 128, 2)
    nw = lib.workspace_bytes(M, N, K)
    assert nw > 0
    work = _stale(nw, 11, cuda)
    torch.cuda.synchronize()
    ys = [_gemm(lib, xq, xs, qd, sd, work=work)[0] for xq, xs in xs_in]
    torch.cuda.synchronize()
    for i, (xq, xs) in enumerate(xs_in):
        yu, _ = _gemm(lib, xq, xs, qd, sd)
        torch.cuda.synchronize()
        assert torch.equal(ys[i].view(torch.int16), yu.view(torch.int16)), f"call {i}"


@pytest.mark.parametrize("name,M", [("down", 256), ("down", 512), ("down", 1024), ("down", 2048)])
def test_qwen3_shapes_automatic_plan(lib, pkg, wl, cuda, name, M):
    """The automatic plan at Qwen3-8B prefill shapes where it splits K, through
    `gemm_w8a8` and `linear()` as shipped: sampled rows against the oracle and
    every output against the unsplit GEMM (no workspace)."""
    N, K = wl.QWEN3_8B_LINEARS[name]
    assert lib.workspace_bytes(M, N, K) > 0, "the automatic plan does not split this shape"
    x = wl.activations(M, K, seed=1300 + M)
    q, s = wl.weight_i8(N, K, seed=1301 + M)
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    xd = x.cuda()
    xq, xs = pkg.quantize_rowwise(xd)
    y = pkg.gemm_w8a8(xq, xs, qt)
    y_lin = pkg.linear(xd, qt)
    yu, _ = _gemm(lib, xq, xs, qt.data, qt.scale)
    torch.cuda.synchronize()
    assert torch.equal(y.view(torch.int16), yu.view(torch.int16)), "split != unsplit"
    assert torch.equal(y_lin.view(torch.int16), yu.view(torch.int16)), "linear() != unsplit"
    xqr, xsr = oracle.quant_rowwise_f16(x.numpy())
    rows = np.unique(np.concatenate([[0, M - 1], np.random.default_rng(M).choice(M, 24)]))
    yr = oracle.dequant_f16(oracle.gemm_i8(xqr[rows], q.numpy()), xsr[rows], s.numpy())
    assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16)[rows],
                          yr.view(np.uint16))


def test_linear_split_k_strided_bias_3d(pkg, wl, cuda):
    """`linear()` on down-shaped weights at prefill sizes, the split-K plan taken
    through the workspace: a [B, S, K] input whose rows are a strided view (every
    other token of a longer sequence), with bias.  Every output against the
    oracle; the same call on a contiguous copy gives the same bits."""
    N, K = wl.QWEN3_8B_LINEARS["down"]
    B, S = 2, 160          # M = 320 rows: the 64x128 / 256x128 split plans' range
    h = wl.activations(B * 2 * S, K, seed=1600).reshape(B, 2 * S, K)
    q, s = wl.weight_i8(N, K, seed=1601)
    bias = (torch.randn(N, generator=torch.Generator().manual_seed(1602)) * 2).half()
    qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
    hs = h.cuda()[:, ::2]                      # [B, S, K], token stride 2K
    assert not hs.is_contiguous()
    from importlib import import_module
    assert import_module("fni8serve_amd._lib").workspace_bytes(B * S, N, K) > 0
    y = pkg.linear(hs, qt, bias.cuda())
    yc = pkg.linear(hs.contiguous(), qt, bias.cuda())
    torch.cuda.synchronize()
    assert y.shape == (B, S, N)
    assert torch.equal(y.view(torch.int16), yc.view(torch.int16))
    yr, *_ = oracle.linear_w8a8_f16(h[:, ::2].reshape(-1, K).contiguous().numpy(), q.numpy(),
                                    s.numpy(), bias.numpy())
    assert np.array_equal(y.reshape(-1, N).cpu().view(torch.int16).numpy().view(np.uint16),
                          yr.view(np.uint16))


def test_workspace_too_small_falls_back(lib, plan, wl, cuda):
    """A workspace one byte short of the forced plan's: another plan runs (same
    bits).  A workspace smaller than every split plan's: the unsplit GEMM runs
    (same bits) and leaves the workspace untouched."""
    M, N, K = 512, 1024, 2048
    xq, xs, q, s = _inputs(wl, M, N, K, seed=1400)
    xqd, xsd, qd, sd = (torch.from_numpy(xq).to(cuda), torch.from_numpy(xs).to(cuda), q.to(cuda),
                        s.to(cuda))
    yr = oracle.dequant_f16(oracle.gemm_i8(xq, q.numpy()), xs, s.numpy())
    plan(256, 128, 2)
    nw = lib.workspace_bytes(M, N, K)
    assert nw > 0
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for size in (nw - 1, 1 << 20):   # the smallest split plan here needs 2 MiB
        work = torch.zeros(nw, dtype=torch.uint8, device=cuda)
        y = torch.empty((M, N), dtype=torch.float16, device=cuda)
        lib.call("fni8_gemm_w8a8_ws", _ptr(xqd), K, _ptr(xsd), M, K, _ptr(qd), _ptr(sd), N, None,
                 _ptr(y), N, None, _ptr(work), size, st)
        torch.cuda.synchronize()
        assert np.array_equal(y.cpu().view(torch.int16).numpy().view(np.uint16),
                              yr.view(np.uint16)), f"workspace of {size} bytes"
        if size == 1 << 20:
            assert int(work.sum().item()) == 0, "a too-small workspace was written"


def test_split_graph_replays_on_new_inputs(lib, pkg, wl, cuda):
    """down at M = 512 (automatic split plan) captured in a HIP graph with its
    workspace, replayed three times on new activations with eager work and
    synchronisations between replays: every replay equals the eager unsplit GEMM."""
    N, K = wl.QWEN3_8B_LINEARS["down"]
    M = 512
    nw = lib.workspace_bytes(M, N, K)
    assert nw > 0
    q, s = wl.weight_i8(N, K, seed=1500)
    qd, sd = q.cuda(), s.cuda()
    xq = torch.empty((M, K), dtype=torch.int8, device=cuda)
    xs = torch.empty((M,), dtype=torch.float32, device=cuda)
    work = _stale(nw, 9, cuda)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        _gemm(lib, xq.zero_(), xs.fill_(1.0), qd, sd, work=work)  # warm-up outside the capture
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        y, _ = _gemm(lib, xq, xs, qd, sd, work=work)
    for rep in range(3):
        xr = wl.activations(M, K, seed=1510 + rep).cuda()
        q2, s2 = pkg.quantize_rowwise(xr)
        xq.copy_(q2)
        xs.copy_(s2)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        yu, _ = _gemm(lib, xq, xs, qd, sd)
        torch.cuda.synchronize()
        assert torch.equal(y.view(torch.int16), yu.view(torch.int16)), f"replay {rep}"
