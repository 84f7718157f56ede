"""fni8_linear_w8a8_f16_noalloc -- the W8A8 linear that allocates nothing (its
quantized activations live in a scratch array inside the library) -- against
fni8_linear_w8a8_f16 on the same inputs, through the C ABI, bit for bit.  Calls
run back to back on one GPU, each smaller than the one before, so a call that
read the previous call's leftover scratch would show."""
import ctypes

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _ptr(t):
    return None if t is None else ctypes.c_void_p(t.data_ptr())


def _noalloc(lib, x, qt, bias=None):
    K = x.shape[-1]
    N = qt.data.shape[0]
    y = torch.empty((x.shape[0], N), dtype=torch.float16, device=x.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream(x.device).cuda_stream)
    lib.call("fni8_linear_w8a8_f16_noalloc", _ptr(x), x.stride(0), x.shape[0], K, _ptr(qt.data),
             _ptr(qt.scale), N, _ptr(bias), _ptr(y), N, stream)
    return y


def test_noalloc_matches_linear_calls_in_a_row(pkg, wl, cuda):
    from importlib import import_module
    lib = import_module("fni8serve_amd._lib")
    # down at 12 tokens and O at 8 take the one-launch path (its workspace in the scratch)
    cases = [("gate_up", 2048, False), ("down", 300, True), ("down", 12, False), ("o", 8, True),
             ("qkv", 4, True), ("o", 1, False)]
    for i, (name, M, with_bias) in enumerate(cases):
        N, K = wl.QWEN3_8B_LINEARS[name]
        x = wl.activations(M, K, seed=500 + i).cuda()
        q, s = wl.weight_i8(N, K, seed=600 + i)
        qt = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
        bias = (torch.randn(N, generator=torch.Generator().manual_seed(700 + i)) * 2).half().cuda() \
            if with_bias else None
        ref = pkg.linear(x, qt, bias)
        got = _noalloc(lib, x, qt, bias)
        torch.cuda.synchronize()
        assert torch.equal(got.view(torch.int16), ref.view(torch.int16)), f"call {i}: {name} M={M}"


def test_noalloc_rejects_sizes_beyond_the_scratch(pkg, wl, cuda):
    from importlib import import_module
    lib = import_module("fni8serve_amd._lib")
    K, N = 12288, 64
    M = (48 << 20) // K + 1   # one row past the 48 MiB of quantized activations
    x = torch.zeros((1, K), dtype=torch.float16, device=cuda)
    w = torch.zeros((N, K), dtype=torch.int8, device=cuda)
    ws = torch.ones(N, dtype=torch.float32, device=cuda)
    y = torch.empty((1, N), dtype=torch.float16, device=cuda)
    with pytest.raises(ValueError, match="no-allocation scratch"):
        lib.call("fni8_linear_w8a8_f16_noalloc", _ptr(x), K, M, K, _ptr(w), _ptr(ws), N, None,
                 _ptr(y), N, None)


def test_noalloc_captured_in_a_graph_replays_on_new_inputs(pkg, wl, cuda):
    """fni8_init first (the scratch address is looked up outside any capture),
    one eager call per shape (kernel attributes set outside the capture), then
    noalloc calls at 4, 8 and 12 tokens (the last two on the one-launch path)
    captured in one HIP graph and replayed
    three times on new activations, the program's own eager work and
    synchronisations between replays: every replay equals the eager linear()."""
    from importlib import import_module
    lib = import_module("fni8serve_amd._lib")
    lib.call("fni8_init")
    shapes = {"qkv": 4, "o": 8, "down": 12}
    qts, xin = {}, {}
    for i, (name, M) in enumerate(shapes.items()):
        N, K = wl.QWEN3_8B_LINEARS[name]
        q, s = wl.weight_i8(N, K, seed=800 + i)
        qts[name] = pkg.QTensor(q.cuda(), s.cuda(), scheme="per_row_i8")
        xin[name] = wl.activations(M, K, seed=810 + i).cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for name in shapes:
            _noalloc(lib, xin[name], qts[name])
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        outs = {name: _noalloc(lib, xin[name], qts[name]) for name in shapes}
    for rep in range(3):
        for i, (name, M) in enumerate(shapes.items()):
            N, K = wl.QWEN3_8B_LINEARS[name]
            xin[name].copy_(wl.activations(M, K, seed=820 + 10 * rep + i).cuda())
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        for name in shapes:
            ref = pkg.linear(xin[name], qts[name])
            torch.cuda.synchronize()
            assert torch.equal(outs[name].view(torch.int16), ref.view(torch.int16)), \
                f"replay {rep} {name}"
