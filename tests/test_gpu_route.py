"""GPU parity of the MoE router (`fni8_moe_route`) and graph capture of a whole
SparseMoE layer.

The router against the oracle (oracle/route_oracle.c): experts bit for bit,
fp16 weights bit for bit (any NaN equals any NaN).  Against torch's routing of
the same logits on the GPU (fni8serve/models/moe.py:62-91 as written): same
experts, weights within one fp16 ulp, on rows without near-ties.  Then a
SparseMoE layer -- router GEMM, router kernel, sort, grouped GEMMs, fused
activation, combine, shared expert -- is captured in one HIP graph and
replayed on new inputs, each replay equal to the eager forward bit for bit;
the reference declines MoE layers for graph capture
(fni8serve/engine/cuda_graph.py:190-191).
"""
import numpy as np
import pytest
import torch

from oracle import oracle as o

pytestmark = pytest.mark.gpu

ROUTE_CASES = [
    dict(T=1, E=128, k=8, scoring="softmax"),
    dict(T=300, E=128, k=8, scoring="softmax"),
    dict(T=4096, E=128, k=8, scoring="softmax"),
    dict(T=300, E=64, k=2, scoring="softmax", renorm=False),
    dict(T=77, E=160, k=6, scoring="softmax", scale=2.5),
    dict(T=300, E=256, k=8, scoring="sigmoid", bias=True, groups=8, topk_group=4, scale=2.5),
    dict(T=300, E=256, k=8, scoring="sigmoid", bias=True),
    dict(T=50, E=512, k=10, scoring="softmax"),
    dict(T=33, E=1024, k=32, scoring="sigmoid", bias=True, groups=64, topk_group=7),
    dict(T=9, E=8, k=1, scoring="softmax"),
    dict(T=9, E=16, k=16, scoring="softmax"),
    dict(T=200, E=40, k=12, scoring="softmax", ties=True),
    dict(T=64, E=96, k=4, scoring="sigmoid", nan=True),
    dict(T=64, E=96, k=4, scoring="softmax", nan=True),
]


def _case_inputs(c):
    rng = np.random.default_rng(c["T"] * 3 + c["E"] + c["k"])
    if c.get("ties"):
        logits = rng.integers(-3, 4, size=(c["T"], c["E"])).astype(np.float32)
    else:
        logits = (rng.standard_normal((c["T"], c["E"])) * 2).astype(np.float32)
    if c.get("nan"):
        logits[::7, 5] = np.nan
    bias = (rng.standard_normal(c["E"]) * 0.1).astype(np.float32) if c.get("bias") else None
    return logits, bias


def _kw(c, bias):
    return dict(scoring=c["scoring"], bias=bias, groups=c.get("groups", 0),
                topk_group=c.get("topk_group", 0), renorm=c.get("renorm", True),
                scale=c.get("scale", 1.0))


@pytest.mark.parametrize("c", ROUTE_CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_route_bitexact(pkg, c):
    print(f"moe_route {c}", flush=True)
    logits, bias = _case_inputs(c)
    kw = _kw(c, bias)
    w, i = o.moe_route(logits, c["k"], **kw)
    gw, gi = pkg.ops.moe_route(torch.from_numpy(logits).cuda(), c["k"], kw["scoring"],
                               None if bias is None else torch.from_numpy(bias).cuda(),
                               kw["groups"] or None, kw["topk_group"] or None, kw["renorm"],
                               kw["scale"])
    assert np.array_equal(gi.cpu().numpy(), i)
    gw = gw.cpu().numpy()
    same = (gw.view(np.uint16) == w.view(np.uint16)) | (np.isnan(gw) & np.isnan(w))
    assert same.all()


def test_route_strided_logits(pkg):
    logits, _ = _case_inputs(dict(T=40, E=128, k=8))
    wide = np.zeros((40, 160), np.float32)
    wide[:, :128] = logits
    gw, gi = pkg.ops.moe_route(torch.from_numpy(wide).cuda()[:, :128], 8)
    w, i = o.moe_route(logits, 8)
    assert np.array_equal(gi.cpu().numpy(), i) and np.array_equal(gw.cpu().numpy(), w)


@pytest.mark.parametrize("scoring", ["softmax", "sigmoid"])
def test_route_against_torch_on_the_gpu(pkg, scoring):
    """The module's CPU routing chain (torch ops, moe.py:62-91) run on the GPU
    against the kernel: same experts on rows without near-ties (gap > 1e-6
    relative between consecutive selection scores up to k + 1), weights within
    one fp16 ulp."""
    torch.manual_seed(0)
    T, E, k = 2048, 128, 8
    logits = torch.randn(T, E, device="cuda") * 2
    bias = torch.randn(E, device="cuda") * 0.1 if scoring == "sigmoid" else None
    if scoring == "sigmoid":
        scores = torch.sigmoid(logits)
        sel = scores + bias
        _, ti = torch.topk(sel, k, dim=-1)
        tw = scores.gather(-1, ti)
    else:
        sel = torch.softmax(logits, dim=-1)
        tw, ti = torch.topk(sel, k, dim=-1)
    tw = (tw / tw.sum(-1, keepdim=True).clamp_min(1e-9)).half()
    gw, gi = pkg.ops.moe_route(logits, k, scoring, bias)
    srt = sel.sort(dim=-1, descending=True).values[:, :k + 1]
    gaps = (srt[:, :-1] - srt[:, 1:]).abs() / srt[:, :-1].abs().clamp_min(1e-30)
    clean = (gaps > 1e-6).all(dim=-1)
    assert clean.float().mean() > 0.97
    assert torch.equal(gi[clean].long(), ti[clean])
    a, b = gw[clean].double(), tw[clean].double()
    ulp = torch.from_numpy(np.spacing(np.abs(b.cpu().numpy()).astype(np.float16))
                           .astype(np.float64)).cuda()
    assert ((a - b).abs() <= ulp).all()


def _moe(pkg, E=128, H=2048, I=768, k=8, shared=False, scoring="softmax", seed=0, **kw):
    g = torch.Generator(device="cuda").manual_seed(seed)

    def qt(n, kk):
        q, s = pkg.quantize_int8_rowwise(torch.randn(n, kk, device="cuda", generator=g) * 0.02)
        return pkg.QTensor(q, s.squeeze(-1), scheme="per_row_i8")

    experts = [(qt(2 * I, H), qt(H, I)) for _ in range(E)]
    gate = (torch.randn(E, H, device="cuda", generator=g) * 0.05).half()
    extra = {}
    if shared:
        extra["shared_expert"] = (qt(2 * 2 * I, H), qt(H, 2 * I))
        extra["shared_expert_gate"] = (torch.randn(1, H, device="cuda", generator=g) * 0.05).half()
    if scoring == "sigmoid":
        extra["e_score_correction_bias"] = torch.randn(E, device="cuda", generator=g) * 0.1
        extra["num_expert_groups"] = 8
        extra["topk_group"] = 4
        extra["routed_scaling_factor"] = 2.5
    return pkg.SparseMoE(gate=gate, experts=experts, top_k=k, norm_topk_prob=True,
                         scoring_func=scoring, **extra, **kw)


@pytest.mark.parametrize("T", [1, 4, 16, 64])
@pytest.mark.parametrize("variant", ["softmax", "sigmoid_groups_shared"])
def test_sparse_moe_graph_capture(pkg, T, variant):
    """Qwen3-30B-A3B-shaped layer (128 experts, top-8, hidden 2048, expert
    intermediate 768); the second variant adds DeepSeek-style sigmoid scoring
    with a selection bias and group-limited top-k, and a gated shared expert."""
    print(f"moe graph capture T={T} {variant}", flush=True)
    sig = variant != "softmax"
    moe = _moe(pkg, shared=sig, scoring="sigmoid" if sig else "softmax", seed=T)
    g = torch.Generator(device="cuda").manual_seed(100 + T)
    x_static = (torch.randn(1, T, 2048, device="cuda", generator=g) * 0.5).half()
    with torch.inference_mode():
        eager0 = moe(x_static).clone()
        s = torch.cuda.Stream()
        s.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(s):
            for _ in range(2):
                moe(x_static)
        torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            y_static = moe(x_static)
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(y_static, eager0)
        for rep in range(3):
            x_new = (torch.randn(1, T, 2048, device="cuda", generator=g) * 0.5).half()
            x_static.copy_(x_new)
            y_static.fill_(float("nan"))
            graph.replay()
            torch.cuda.synchronize()
            want = moe(x_new)
            torch.cuda.synchronize()
            assert torch.isfinite(want).all()
            assert torch.equal(y_static, want), rep
