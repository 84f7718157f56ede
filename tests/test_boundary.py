"""Host side of the drop-in boundary, on the CPU: the QTensor / LinearW8A8 /
GatedMLP / SparseMoE / LMHead contracts of the reference (fni8serve/layers and
fni8serve/models), the weight helpers, and the rule that GPU entry points never
fall back to the CPU."""
import os
import subprocess
import sys

import numpy as np
import pytest
import torch

from oracle.reference_cpu import reference_cpu_linear

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def _i8(pkg, out, in_, seed=0):
    """tests/test_layers.py:29-33's helper: fp16 weight, per-row int8 QTensor."""
    g = torch.Generator().manual_seed(seed)
    w = torch.randn(out, in_, generator=g).half()
    s = w.abs().amax(-1, keepdim=True).clamp_min(1e-6) / 127
    q = torch.round(w / s).clamp_(-127, 127).to(torch.int8)
    return pkg.QTensor(q, s.squeeze(-1).float(), scheme="per_row_i8"), (q.float() * s).half()


def _i4(pkg, out, in_, g):
    """tests/test_smoke.py:21-29's int4 packing."""
    w = torch.randn(out, in_)
    wg = w.reshape(out, in_ // g, g)
    s = wg.abs().amax(-1, keepdim=True) / 7
    c = torch.round(wg / s).clamp_(-7, 7).reshape(out, in_).to(torch.int64)
    u = (c & 0xF).to(torch.int32)
    packed = (u[:, 0::2] | (u[:, 1::2] << 4)).to(torch.uint8)
    return pkg.QTensor(packed, s.squeeze(-1).float(), scheme="per_group_i4", group_size=g,
                       codebook="int4"), c.float() * s.reshape(out, in_ // g).repeat_interleave(g, 1)


def test_qtensor_contract(pkg):
    qt, _ = _i8(pkg, 32, 64)
    assert qt.scheme == "per_row_i8" and qt.group_size is None and qt.codebook is None
    assert qt.data.shape == (32, 64) and qt.scale.shape == (32,)
    with pytest.raises(ValueError):
        pkg.QTensor(qt.data.float(), qt.scale, scheme="per_row_i8")
    with pytest.raises(ValueError):
        pkg.QTensor(qt.data, qt.scale[:5], scheme="per_row_i8")
    with pytest.raises(ValueError):
        pkg.QTensor(qt.data, qt.scale, scheme="per_col_i8")
    raw = pkg.QTensor(torch.ones(3), None, scheme="raw")
    assert raw.scale is None


def test_quantize_int8_rowwise_idiom(pkg):
    w = torch.randn(64, 128) * 3
    q, s = pkg.quantize_int8_rowwise(w)
    assert q.dtype == torch.int8 and s.shape == (64, 1) and s.dtype == torch.float32
    assert torch.equal(q.abs().amax(-1), torch.full((64,), 127, dtype=torch.int8))
    ref_s = w.abs().amax(-1, keepdim=True).clamp_min(1e-6) / 127
    assert torch.equal(s, ref_s)
    assert torch.equal(q, torch.round(w / ref_s).clamp(-127, 127).to(torch.int8))
    assert (w - q.float() * s).abs().le(s / 2 + 1e-6).all()


def test_to_qtensor_and_merge_are_exact(pkg):
    a, b, c = (torch.randn(n, 64) for n in (32, 8, 8))
    qa, qb, qc = (pkg.to_qtensor(t) for t in (a, b, c))
    assert pkg.to_qtensor(qa) is qa                                  # idempotent
    m = pkg.merge_qtensor([qa, qb, qc])
    assert torch.equal(m.data, torch.cat([qa.data, qb.data, qc.data]))
    assert torch.equal(m.scale, torch.cat([qa.scale, qb.scale, qc.scale]))
    sd = {"p.q_proj.weight": a, "p.k_proj.weight": b, "p.v_proj.weight": c,
          "p.gate_proj.weight": b, "p.up_proj.weight": c}
    assert pkg.qkv_weight(sd, "p").data.shape == (48, 64)
    assert pkg.gate_up_weight(sd, "p").data.shape == (16, 64)


def test_linear_attributes_and_cpu_fallback(pkg):
    qt, wdq = _i8(pkg, 96, 128)
    bias = torch.randn(96).half()
    lin = pkg.LinearW8A8(qt, bias)
    assert lin.in_features == 128 and lin.out_features == 96
    assert lin.weight is qt and lin.bias is bias
    x = torch.randn(5, 128).half()
    y = lin(x)                                           # CPU: reference fallback path
    ref = reference_cpu_linear(x, qt.data, qt.scale, bias)
    assert torch.equal(y, ref)
    assert torch.equal(pkg._dequant_weight(qt), wdq)


def test_linear_w4_cpu_seam(pkg):
    qt, wref = _i4(pkg, 64, 128, 32)
    lin = pkg.LinearW8A8(qt)
    assert lin.in_features == 128 and lin.out_features == 64
    y = lin(torch.randn(2, 128))
    assert y.shape == (2, 64) and torch.isfinite(y).all()
    assert torch.allclose(pkg._dequant_weight(qt).float(), wref, atol=1e-2)


def test_nf4_dequant_and_bad_scheme(pkg):
    codes = torch.arange(16, dtype=torch.int32).repeat(4, 1)       # [4, 16]
    packed = (codes[:, 0::2] | (codes[:, 1::2] << 4)).to(torch.uint8)
    qt = pkg.QTensor(packed, torch.ones(4, 1), scheme="per_group_i4", group_size=16, codebook="nf4")
    w = pkg._dequant_weight(qt)
    assert torch.allclose(w[0].float(), torch.tensor(pkg.NF4_CODEBOOK), atol=1e-3)
    with pytest.raises(ValueError):
        pkg._dequant_weight(pkg.QTensor(torch.ones(2, 2), None, scheme="raw"))


def test_gpu_entry_points_refuse_cpu_tensors(pkg):
    qt, _ = _i8(pkg, 16, 64)
    with pytest.raises(ValueError, match="GPU"):
        pkg.linear(torch.randn(2, 64).half(), qt)
    with pytest.raises(ValueError, match="GPU"):
        pkg.quantize_rowwise(torch.randn(2, 64).half())
    with pytest.raises(ValueError):
        pkg.linear(torch.randn(2, 64).half(), pkg.QTensor(torch.ones(2), None, scheme="raw"))


def test_gated_mlp_cpu_and_activations(pkg):
    gu, _ = _i8(pkg, 2 * 48, 64, 1)
    dn, _ = _i8(pkg, 64, 48, 2)
    mlp = pkg.GatedMLP(gu, dn, act="silu")
    assert mlp.hidden_size == 64 and mlp.intermediate_size == 48
    y = mlp(torch.randn(3, 64).half())
    assert y.shape == (3, 64)
    from importlib import import_module
    act = import_module("fni8serve_amd.layers.activation")
    x = torch.randn(4, 32)
    g, u = x.chunk(2, -1)
    assert torch.allclose(act.SiluAndMul()(x), torch.nn.functional.silu(g) * u)
    assert isinstance(act.get_act_and_mul("gelu_pytorch_tanh"), act.GeluAndMul)
    with pytest.raises(ValueError):
        act.get_act_and_mul("relu")
    assert act.fused_act(act.SiluAndMul()) == "silu"
    assert act.fused_act(act.GeluAndMul("tanh")) == "gelu_tanh"
    assert act.fused_act(act.GeluAndMul("none")) is None  # exact-erf gelu: eager only


def test_rmsnorm_cpu_is_the_reference_eager_form(pkg):
    """CPU tensors take norm.py:37-58's eager form: fp32 norm cast back, the
    residual added in the input dtype and returned alongside."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(3, 64, generator=g).half()
    r = torch.randn(3, 64, generator=g).half()
    w = (torch.rand(64, generator=g) + 0.5).half()
    n = pkg.RMSNorm(64, eps=1e-5, weight=w.clone())
    xf = x.float()
    want = (xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.float()).half()
    assert torch.equal(n(x), want)
    out, new_r = n(x, r)
    assert torch.equal(new_r, x + r)
    hf = (x + r).float()
    assert torch.equal(out, (hf * torch.rsqrt(hf.pow(2).mean(-1, keepdim=True) + 1e-5) * w.float()).half())
    gem = pkg.RMSNorm(64, add_unit_offset=True)
    assert torch.equal(gem.weight, torch.zeros(64, dtype=torch.float16))
    with pytest.raises(ValueError, match="GPU"):
        pkg.rmsnorm(x, w)
    with pytest.raises(ValueError, match="GPU"):
        pkg.act_and_mul(torch.randn(2, 8).half())


@pytest.mark.parametrize("dt", [torch.float32, torch.bfloat16, torch.float16])
def test_act_and_mul_modules_on_the_cpu_are_the_eager_form(pkg, dt):
    """CPU tensors of every dtype take act(gate) * up in their own dtype
    (fni8serve/layers/activation.py:26-27, :42-43); only GPU fp16 takes the kernel."""
    import torch.nn.functional as F
    from fni8serve_amd.layers import activation as act
    x = (torch.randn(3, 64, generator=torch.Generator().manual_seed(5)) * 2).to(dt)
    gate, up = x.chunk(2, dim=-1)
    assert torch.equal(act.SiluAndMul()(x), F.silu(gate) * up)
    assert torch.equal(act.GeluAndMul("tanh")(x), F.gelu(gate, approximate="tanh") * up)
    assert torch.equal(act.GeluAndMul("none")(x), F.gelu(gate) * up)
    assert not act._kernel_ok(x)


def _moe(pkg, E=4, H=64, I=32, k=2, **kw):
    g = torch.Generator().manual_seed(0)
    experts = [(pkg.to_qtensor(torch.randn(2 * I, H, generator=g) * 0.05),
                pkg.to_qtensor(torch.randn(H, I, generator=g) * 0.05)) for _ in range(E)]
    return pkg.SparseMoE(gate=torch.randn(E, H, generator=g) * 0.05, experts=experts, top_k=k, **kw)


def test_sparse_moe_cpu_loop_and_routing(pkg):
    moe = _moe(pkg)
    x = torch.randn(1, 5, 64)
    with torch.inference_mode():
        topw, topi = moe.route(x.reshape(-1, 64))
        assert topi.shape == (5, 2) and torch.allclose(topw.float().sum(-1), torch.ones(5))
        y = moe(x)
    assert y.shape == x.shape and torch.isfinite(y).all()
    assert moe.w_gate_up.shape == (4, 64, 64) and moe.w_down.shape == (4, 64, 32)


def test_sparse_moe_w4_experts_cpu_loop(pkg):
    """per_group_i4 experts build (no stacking) and run the reference's CPU loop
    through each expert's GatedMLP (dequantized int4 weights, linear.py:32-45)."""
    g = torch.Generator().manual_seed(3)
    E, H, I, G = 4, 64, 32, 32

    def w4(n, k):
        codes = torch.randint(-8, 8, (n, k), generator=g)
        packed = ((codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)).to(torch.uint8)
        return pkg.QTensor(packed, torch.rand(n, k // G, generator=g) * 0.02 + 1e-3,
                           scheme="per_group_i4", group_size=G, codebook="int4")
    experts = [(w4(2 * I, H), w4(H, I)) for _ in range(E)]
    moe = pkg.SparseMoE(gate=torch.randn(E, H, generator=g) * 0.05, experts=experts, top_k=2)
    assert not moe.grouped and len(moe.experts) == E
    x = torch.randn(1, 5, H)
    with torch.inference_mode():
        y = moe(x)
        topw, topi = moe.route(x.reshape(-1, H))
        want = torch.zeros(5, H)
        for e in range(E):
            tok, slot = (topi == e).nonzero(as_tuple=True)
            if tok.numel():
                want.index_add_(0, tok, moe.experts[e](x.reshape(-1, H)[tok]) * topw[tok, slot, None])
    assert torch.equal(y.reshape(5, H), want)


def test_sparse_moe_w4_experts_stack_for_the_grouped_kernel(pkg):
    """int4 experts of one layout (G in 64..256, K a multiple of 256) are stacked
    for the grouped W4A8 GEMM, with the per-expert modules as views of the
    stacks; other layouts keep their own modules.  On the CPU both run the
    reference loop and give the same output as modules built from the original
    QTensors."""
    g = torch.Generator().manual_seed(5)
    E, H, I = 4, 256, 256

    def w4(n, k, G, scale_dtype=torch.float32):
        codes = torch.randint(-8, 8, (n, k), generator=g)
        packed = ((codes[:, 0::2] & 0xF) | ((codes[:, 1::2] & 0xF) << 4)).to(torch.uint8)
        scale = (torch.rand(n, k // G, generator=g) * 0.02 + 1e-3).to(scale_dtype)
        return pkg.QTensor(packed, scale, scheme="per_group_i4", group_size=G, codebook="int4")

    gate = torch.randn(E, H, generator=g) * 0.05
    experts = [(w4(2 * I, H, 128), w4(H, I, 64)) for _ in range(E)]
    moe = pkg.SparseMoE(gate=gate, experts=experts, top_k=2)
    assert moe.grouped_w4 and not moe.grouped
    assert moe.w_gate_up.shape == (E, 2 * I, H // 2) and moe.w_gate_up.dtype == torch.uint8
    assert moe.s_gate_up.shape == (E, 2 * I, H // 128) and moe.s_down.shape == (E, H, I // 64)
    assert (moe.g_gate_up, moe.g_down) == (128, 64)
    assert moe.experts[1].gate_up_proj.weight.data.data_ptr() == moe.w_gate_up[1].data_ptr()
    x = torch.randn(1, 6, H)
    with torch.inference_mode():
        y = moe(x)
        ref = pkg.SparseMoE(gate=gate, experts=experts, top_k=2)
        ref.experts = torch.nn.ModuleList([pkg.GatedMLP(gu, dn) for gu, dn in experts])
        want = ref(x)
    assert torch.equal(y, want)
    # group size 32, mixed group sizes within a projection, or fp16 scales: not stacked
    for bad in ([(w4(2 * I, H, 32), w4(H, I, 32)) for _ in range(E)],
                [(w4(2 * I, H, 128 if e else 64), w4(H, I, 64)) for e in range(E)],
                [(w4(2 * I, H, 128, torch.float16), w4(H, I, 64)) for _ in range(E)]):
        m = pkg.SparseMoE(gate=gate, experts=bad, top_k=2)
        assert not m.grouped_w4 and not m.grouped and len(m.experts) == E


def test_sparse_moe_group_limited_routing(pkg):
    """tests/test_deepseek.py:207-265: with 2 groups of 2 experts and topk_group=1,
    every token's experts come from one group."""
    bias = torch.randn(4) * 0.1
    moe = _moe(pkg, scoring_func="sigmoid", e_score_correction_bias=bias,
               num_expert_groups=2, topk_group=1)
    with torch.inference_mode():
        _, topi = moe.route(torch.randn(8, 64))
    for row in topi.tolist():
        assert len({e // 2 for e in row}) == 1


def test_lm_head_cpu(pkg):
    qt, _ = _i8(pkg, 100, 64)
    head = pkg.LMHead(qt)
    h = torch.randn(2, 3, 64).half()
    assert head(h[:, -1]).shape == (2, 100)
    fp = pkg.LMHead(torch.randn(100, 64), logit_softcap=30.0)
    assert fp(torch.randn(2, 64)).abs().max() <= 30.0


def test_workload_formulas_match_the_measurement_plan(wl):
    # bytes = N*K + 4N + 2MK + 2MN; the QKV decode row reads 25.21 MB at M=1
    assert round(wl.linear_bytes(1, 6144, 4096) / 1e6, 2) == 25.21
    assert round(wl.linear_bytes(64, 24576, 4096) / 1e6, 2) == 104.43
    assert round(wl.linear_ops(4096, 24576, 4096) / 1e9, 1) == 824.6
    a = wl.activations(8, 64, seed=3)
    assert torch.equal(a, wl.activations(8, 64, seed=3)) and a.dtype == torch.float16
    q, s = wl.weight_i8(16, 64, seed=4)
    assert q.dtype == torch.int8 and int(q.min()) >= -127 and s.min() >= 0.001 and s.max() <= 0.02
    topw, topi = wl.route(wl.router_logits(32, 128, seed=5), 8)
    assert topi.shape == (32, 8) and topw.dtype == torch.float16


def test_bench_refuses_more_than_one_gpu():
    r = subprocess.run([sys.executable, os.path.join(ROOT, "bench.py"), "--gpus", "2"],
                       capture_output=True, text=True, timeout=120)
    assert r.returncode == 2 and "one GPU" in r.stderr


def test_moe_router_weight_cache_follows_the_parameter(pkg):
    """The fp32 router weight is cached; an in-place update of the parameter
    (its version changes) or a new tensor is picked up on the next call."""
    moe = _moe(pkg)
    xf = torch.randn(5, 64)
    w1, i1 = moe.route(xf)
    assert torch.equal(moe._gate_f32(), moe.gate.detach().float())
    with torch.no_grad():
        moe.gate.mul_(-1.0)
    w2, i2 = moe.route(xf)
    assert torch.equal(moe._gate_f32(), moe.gate.detach().float())
    assert not torch.equal(i1, i2)
    moe.gate = torch.nn.Parameter(torch.zeros_like(moe.gate))
    w3, i3 = moe.route(xf)
    assert torch.equal(moe._gate_f32(), torch.zeros_like(moe.gate, dtype=torch.float32))
    assert (w3 == 1.0 / moe.top_k).all()  # uniform scores, renormalised
