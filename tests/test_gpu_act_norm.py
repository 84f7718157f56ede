"""GPU parity of act_and_mul and RMSNorm, alone and fused with the next
linear's quantization, against the oracle (oracle/act_norm_oracle.c): fp16
outputs bit for bit (any NaN equals any NaN), int8 rows and fp32 scales bit for
bit.  Shapes cover the register-resident kernels (1..16 chunks per lane), the
generic kernels (ragged or long rows, strided rows) and Qwen3-8B's sizes
(intermediate 12288, hidden 4096) at full size.  The fused MLP is checked
against the unfused chain, and the kernels against torch's fp32 forms with
the tolerance stated in the test.
"""
import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as o

pytestmark = pytest.mark.gpu


def _same_f16(a: np.ndarray, b: np.ndarray) -> bool:
    a = np.asarray(a, np.float16)
    b = np.asarray(b, np.float16)
    nan = np.isnan(a) & np.isnan(b)
    return bool(((a.view(np.uint16) == b.view(np.uint16)) | nan).all())


def _same_f32(a, b) -> bool:
    a = np.asarray(a, np.float32)
    b = np.asarray(b, np.float32)
    return bool(((a.view(np.uint32) == b.view(np.uint32)) | (np.isnan(a) & np.isnan(b))).all())


def _merged(M, I, seed, scale=3.0, specials=False):
    rng = np.random.default_rng(seed)
    x = (rng.standard_normal((M, 2 * I)) * scale).astype(np.float16)
    if specials and x.size >= 16:
        flat = x.reshape(-1)
        idx = rng.choice(flat.size, 16, replace=False)
        flat[idx] = np.float16([0.0, -0.0, 60000, -60000, 6e-8, -6e-8, 100, -100,
                                np.nan, 8.5, -9.25, 1e-4, -1e-4, 20, -20, 3])
    return x


ACT_SHAPES = [(1, 12288), (4, 12288), (16, 768), (3, 1536), (7, 3072), (2, 25600),
              (5, 1000), (3, 1004), (2, 40000), (64, 12288)]


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
@pytest.mark.parametrize("M,I", ACT_SHAPES)
def test_act_and_mul_bitexact(pkg, act, M, I):
    print(f"act_and_mul {act} M={M} I={I}", flush=True)
    x = _merged(M, I, seed=M * 7 + I, specials=True)
    got = pkg.act_and_mul(torch.from_numpy(x).cuda(), act).cpu().numpy()
    assert _same_f16(got, o.act_and_mul_f16(x, act))


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
@pytest.mark.parametrize("M,I", ACT_SHAPES)
def test_act_and_mul_quant_bitexact(pkg, act, M, I):
    print(f"act_and_mul_quant {act} M={M} I={I}", flush=True)
    x = _merged(M, I, seed=M * 11 + I, specials=(M % 2 == 1))
    xq, xs = pkg.act_and_mul_quant(torch.from_numpy(x).cuda(), act)
    q, s = o.act_and_mul_quant_f16(x, act)
    assert np.array_equal(xq.cpu().numpy(), q)
    assert _same_f32(xs.cpu().numpy(), s)


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
@pytest.mark.parametrize("M,I", [(1, 12288), (5, 12288), (64, 12288), (128, 12288), (33, 4112),
                                 (9, 3072)])
def test_act_quant_split_rows(pkg, act, M, I):
    """fni8_act_and_mul_quant_f16_ws for few rows: G workgroups share each row and
    exchange partial maxima through the workspace.  Against the oracle, bit for
    bit, on a zeroed workspace (then exactly one XCD region holds each part's
    flag: the split kernel ran), on a workspace of garbage, and with the wait
    bound at 0 (parts whose flag is not there at the first look are
    recomputed).  I = 4112 leaves the last part of a row shorter."""
    import ctypes
    from importlib import import_module
    lib = import_module("fni8serve_amd._lib")
    raw = lib.load()
    nw = int(raw.fni8_act_and_mul_quant_workspace_bytes(M, I))
    G = -(-I // 2048)
    assert nw == 8 * (-(-M // 8) * 8) * G * 128 and 2 <= G <= 8, (nw, G)
    x = _merged(M, I, seed=M * 13 + I, specials=(M % 2 == 1))
    q_ref, s_ref = o.act_and_mul_quant_f16(x, act)
    xd = torch.from_numpy(x).cuda()
    code = 0 if act == "silu" else 1
    st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    mpad = -(-M // 8) * 8
    for case in ("zeroed", "stale", "recompute"):
        if case == "zeroed":
            work = torch.zeros(nw, dtype=torch.uint8, device="cuda")
        else:
            work = torch.randint(0, 256, (nw,), dtype=torch.uint8,
                                 generator=torch.Generator().manual_seed(M)).cuda()
        xq = torch.empty((M, I), dtype=torch.int8, device="cuda")
        xs = torch.empty((M,), dtype=torch.float32, device="cuda")
        if case == "recompute":
            raw.fni8_debug_coop_wait_ticks(0)
        try:
            lib.call("fni8_act_and_mul_quant_f16_ws", ctypes.c_void_p(xd.data_ptr()), 2 * I, M,
                     I, code, ctypes.c_void_p(xq.data_ptr()), I, ctypes.c_void_p(xs.data_ptr()),
                     ctypes.c_void_p(work.data_ptr()), nw, st)
            torch.cuda.synchronize()
        finally:
            raw.fni8_debug_coop_wait_ticks(-1)
        assert np.array_equal(xq.cpu().numpy(), q_ref), case
        assert _same_f32(xs.cpu().numpy(), s_ref), case
        if case == "zeroed":
            flags = work.view(torch.int64).view(8, mpad, G, 16)[:, :M, :, 0].cpu().numpy()
            assert np.all((flags != 0).sum(axis=0) == 1), "one flag per (row, part)"


def test_act_kernels_full_size_prefill(pkg):
    """Qwen3-8B gate_up output at M = 2048 (100 MB): both kernels against the
    oracle, and the fused form against quantize_rowwise of the unfused one."""
    print("act full size M=2048 I=12288", flush=True)
    x = _merged(2048, 12288, seed=5)
    xd = torch.from_numpy(x).cuda()
    a = pkg.act_and_mul(xd, "silu")
    assert _same_f16(a.cpu().numpy(), o.act_and_mul_f16(x, "silu"))
    xq, xs = pkg.act_and_mul_quant(xd, "silu")
    q2, s2 = pkg.quantize_rowwise(a)
    assert torch.equal(xq, q2) and torch.equal(xs, s2)
    q, s = o.act_and_mul_quant_f16(x, "silu")
    assert np.array_equal(xq.cpu().numpy(), q) and _same_f32(xs.cpu().numpy(), s)


def test_act_strided_rows(pkg):
    """gate | up taken from a wider buffer (row stride > 2I) and a 3-D input."""
    base = _merged(6, 1040, seed=9)                 # [6, 2080]
    I = 1024
    xs_ = torch.from_numpy(base).cuda()[:, :2 * I]  # row stride 2080
    got = pkg.act_and_mul(xs_, "silu").cpu().numpy()
    assert _same_f16(got, o.act_and_mul_f16(base[:, :2 * I], "silu"))
    x3 = torch.from_numpy(_merged(8, 256, seed=10)).cuda().reshape(2, 4, 512)
    y3 = pkg.act_and_mul(x3, "gelu_tanh")
    assert y3.shape == (2, 4, 256)
    assert _same_f16(y3.reshape(8, 256).cpu().numpy(),
                     o.act_and_mul_f16(x3.reshape(8, 512).cpu().numpy(), "gelu_tanh"))


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
def test_act_against_torch_fp32(pkg, act):
    """The kernel against torch's fp32 form on the GPU, rounded once to fp16:
    within 1 fp16 ulp (plus, for gelu, torch's own |g u| 2^-23 cancellation
    error in 0.5 g (1 + tanh y)); max abs / rel error printed."""
    x = _merged(256, 4096, seed=12)
    xd = torch.from_numpy(x).cuda()
    got = pkg.act_and_mul(xd, act).double()
    g, u = xd.float().chunk(2, -1)
    ref = (F.silu(g) if act == "silu" else F.gelu(g, approximate="tanh")) * u
    ref16 = ref.half().double()
    err = (got - ref16).abs()
    ulp = torch.from_numpy(np.spacing(np.maximum(np.abs(ref16.cpu().numpy()), 2 ** -14)
                                      .astype(np.float16)).astype(np.float64)).cuda()
    cancel = 0.0 if act == "silu" else (g.double() * u.double()).abs() * 2.0 ** -23
    assert (err <= ulp + cancel).all()
    rel = (err / ref.double().abs().clamp_min(1e-3)).max().item()
    print(f"{act}: max abs err {err.max().item():.3g}, max rel err {rel:.3g} vs torch fp32")


NORM_CASES = [(1, 4096), (4, 4096), (64, 4096), (3, 2048), (5, 5120), (2, 8192), (3, 16384),
              (2, 32768), (2, 40000), (7, 1000), (3, 1002), (4, 128), (1, 12)]


@pytest.mark.parametrize("res", [False, True])
@pytest.mark.parametrize("unit", [False, True])
@pytest.mark.parametrize("M,K", NORM_CASES)
def test_rmsnorm_bitexact(pkg, M, K, res, unit):
    print(f"rmsnorm M={M} K={K} res={res} unit={unit}", flush=True)
    rng = np.random.default_rng(M * 13 + K + res + 2 * unit)
    x = (rng.standard_normal((M, K)) * rng.uniform(0.05, 30, (M, 1))).astype(np.float16)
    r = (rng.standard_normal((M, K)) * 2).astype(np.float16) if res else None
    w = (rng.uniform(0.3, 1.7, K) - (1.0 if unit else 0.0)).astype(np.float16)
    eps = 1e-6
    want, want_res = o.rmsnorm_f16(x, w, eps, residual=r, unit_offset=unit)
    xd, wd = torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda()
    rd = None if r is None else torch.from_numpy(r).cuda()
    got = pkg.rmsnorm(xd, wd, eps, residual=rd, unit_offset=unit)
    if res:
        got, got_res = got
        assert _same_f16(got_res.cpu().numpy(), want_res)
    assert _same_f16(got.cpu().numpy(), want)
    if K % 4 == 0:
        qs = pkg.rmsnorm_quant(xd, wd, eps, residual=rd, unit_offset=unit)
        q, s, qres = o.rmsnorm_quant_f16(x, w, eps, residual=r, unit_offset=unit)
        assert np.array_equal(qs[0].cpu().numpy(), q) and _same_f32(qs[1].cpu().numpy(), s)
        if res:
            assert _same_f16(qs[2].cpu().numpy(), qres)


def test_rmsnorm_full_size_and_special_rows(pkg):
    """Qwen3-8B hidden at M = 4096 with the residual add, plus rows that are
    zero, constant, subnormal, at the fp16 maximum's scale and NaN."""
    print("rmsnorm full size M=4096 K=4096", flush=True)
    rng = np.random.default_rng(21)
    M, K = 4096, 4096
    x = rng.standard_normal((M, K)).astype(np.float16)
    r = rng.standard_normal((M, K)).astype(np.float16)
    x[0] = 0
    r[0] = 0
    x[1] = 3.0
    r[1] = 0
    x[2] = np.float16(6e-8)
    r[2] = 0
    x[3] = 60000.0
    r[3] = 0
    x[4, 17] = np.nan
    w = rng.uniform(0.5, 1.5, K).astype(np.float16)
    want, want_res = o.rmsnorm_f16(x, w, 1e-6, residual=r)
    got, got_res = pkg.rmsnorm(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), 1e-6,
                               residual=torch.from_numpy(r).cuda())
    assert _same_f16(got_res.cpu().numpy(), want_res)
    assert _same_f16(got.cpu().numpy(), want)
    q, s, _ = o.rmsnorm_quant_f16(x, w, 1e-6, residual=r)
    gq, gs, _ = pkg.rmsnorm_quant(torch.from_numpy(x).cuda(), torch.from_numpy(w).cuda(), 1e-6,
                                  residual=torch.from_numpy(r).cuda())
    assert np.array_equal(gq.cpu().numpy(), q) and _same_f32(gs.cpu().numpy(), s)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
def test_rmsnorm_module_other_dtypes_take_eager_form(pkg, dt):
    """GPU inputs the fp16 kernel does not take (fp32, bf16) return the reference's
    eager result instead of raising (fni8serve/layers/norm.py:50-58)."""
    g = torch.Generator().manual_seed(21)
    x = torch.randn(8, 256, generator=g).to(dt)
    r = torch.randn(8, 256, generator=g).to(dt)
    w = (torch.rand(256, generator=g) + 0.5).to(dt)
    n = pkg.RMSNorm(256, eps=1e-6, weight=w.clone())
    ref = n._norm(x)
    ref_r = n._norm(x + r)
    n = n.cuda()
    got = n(x.cuda())
    got_r, h = n(x.cuda(), r.cuda())
    torch.cuda.synchronize()
    assert got.dtype == dt and got_r.dtype == dt
    tol = 1e-6 if dt == torch.float32 else 1e-2
    assert torch.allclose(got.cpu().float(), ref.float(), rtol=tol, atol=tol)
    assert torch.allclose(got_r.cpu().float(), ref_r.float(), rtol=tol, atol=tol)
    assert torch.equal(h.cpu(), x + r)


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("mod", ["silu", "gelu_pytorch_tanh", "gelu"])
def test_act_and_mul_module_other_dtypes_take_eager_form(pkg, dt, mod):
    """GPU inputs the fp16 kernel does not take (fp32, bf16) return the eager
    act(gate) * up in their own dtype instead of raising; the reference computes
    fp32 the same way (fni8serve/layers/activation.py:16-17, :26-27, :42-43)."""
    print(f"act_and_mul module {mod} {dt}", flush=True)
    from fni8serve_amd.layers import activation as act
    import torch.nn.functional as F
    g = torch.Generator().manual_seed(22)
    x = (torch.randn(6, 2 * 384, generator=g) * 3).to(dt)
    m = act.get_act_and_mul(mod)
    got = m(x.cuda())
    torch.cuda.synchronize()
    gate, up = x.float().chunk(2, dim=-1)
    appr = getattr(m, "approximate", None)
    ref = (F.silu(gate) if appr is None else F.gelu(gate, approximate=appr)) * up
    assert got.dtype == dt and got.shape == (6, 384)
    tol = 1e-5 if dt == torch.float32 else 2e-2
    assert torch.allclose(got.cpu().float(), ref, rtol=tol, atol=tol)


def test_rmsnorm_against_torch_fp32(pkg):
    """Against the reference's eager form evaluated by torch on the GPU in fp32
    (norm.py:37-43): within 1 fp16 ulp; max abs / rel error printed."""
    g = torch.Generator(device="cuda").manual_seed(3)
    x = torch.randn(512, 4096, device="cuda", generator=g).half()
    w = (torch.rand(4096, device="cuda", generator=g) + 0.5).half()
    got = pkg.rmsnorm(x, w, 1e-6).double()
    xf = x.float()
    ref = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-6) * w.float())
    ref16 = ref.half().double()
    err = (got - ref16).abs()
    ulp = torch.from_numpy(np.spacing(np.maximum(np.abs(ref16.cpu().numpy()), 2 ** -14)
                                      .astype(np.float16)).astype(np.float64)).cuda()
    assert (err <= ulp).all()
    print(f"rmsnorm: max abs err {err.max().item():.3g}, "
          f"max rel err {(err / ref.double().abs().clamp_min(1e-3)).max().item():.3g} vs torch fp32")


def test_fused_kernels_graph_replay(pkg):
    """The four kernels captured in one HIP graph and replayed three times, with
    eager work in between: every replay equals the eager result bit for bit."""
    g = torch.Generator(device="cuda").manual_seed(4)
    h = (torch.randn(16, 2 * 3072, device="cuda", generator=g) * 2).half()
    x = torch.randn(16, 4096, device="cuda", generator=g).half()
    r = torch.randn(16, 4096, device="cuda", generator=g).half()
    w = (torch.rand(4096, device="cuda", generator=g) + 0.5).half()

    def run():
        a = pkg.act_and_mul(h, "silu")
        q1, s1 = pkg.act_and_mul_quant(h, "gelu_tanh")
        n, nr = pkg.rmsnorm(x, w, 1e-6, residual=r)
        q2, s2, nr2 = pkg.rmsnorm_quant(x, w, 1e-5, residual=r, unit_offset=True)
        return a, q1, s1, n, nr, q2, s2, nr2

    eager = [t.clone() for t in run()]
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        run()
    torch.cuda.current_stream().wait_stream(s)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        outs = run()
    for rep in range(3):
        for t in outs:
            t.fill_(0) if t.dtype != torch.float16 else t.fill_(float("nan"))
        graph.replay()
        torch.cuda.synchronize()
        for e, t in zip(eager, outs):
            assert torch.equal(e, t), rep
        _ = (h.float() * 2).sum().item()  # eager work between replays


@pytest.mark.parametrize("act", ["silu", "gelu_tanh"])
@pytest.mark.parametrize("M", [1, 4, 5, 16, 64, 512])
def test_gated_mlp_fused_equals_unfused(pkg, act, M):
    """GatedMLP on the GPU (gate_up linear -> act_and_mul_quant -> int8 GEMM
    from 5 rows up) equals the unfused chain down_proj(act_fn(gate_up_proj(x)))
    bit for bit at Qwen3-8B's MLP shapes; the fused chain itself too at 1 and 4
    rows, where GatedMLP takes the unfused one."""
    print(f"gated mlp {act} M={M}", flush=True)
    from importlib import import_module
    wl = import_module("fni8serve_amd.workloads")
    g = torch.Generator(device="cuda").manual_seed(31)
    qts = []
    for N, K in ((24576, 4096), (4096, 12288)):  # weights at a trained model's scale
        q, s_ = pkg.quantize_int8_rowwise(torch.randn(N, K, device="cuda", generator=g) * 0.02)
        qts.append(pkg.QTensor(q, s_.squeeze(-1), scheme="per_row_i8"))
    mlp = pkg.GatedMLP(*qts, act="silu" if act == "silu" else "gelu_pytorch_tanh")
    x = wl.activations(M, 4096, seed=33, device="cpu").cuda()
    fused = mlp(x)
    unfused = mlp.down_proj(mlp.act_fn(mlp.gate_up_proj(x)))
    assert fused.shape == (M, 4096)
    assert torch.isfinite(fused).all()
    assert torch.equal(fused, unfused)
    h = mlp.gate_up_proj(x)
    chain = pkg.gemm_w8a8(*pkg.act_and_mul_quant(h, act), mlp.down_proj.weight)
    assert torch.equal(chain, unfused)
