"""Pins the router oracle (oracle/route_oracle.c).

Against the reference's own routing, run by torch on the CPU in fp32 exactly
as fni8serve/models/moe.py:62-91 writes it: the same experts in the same
order and weights within one fp16 ulp, over softmax and sigmoid scoring, the
selection bias, group-limited top-k, renormalisation and scaling.  Against
what the mathematics fixes: a brute-force top-k (stable sort by value, then
index), float64 softmax, and known answers for ties, groups and NaN rows.
"""
import math

import numpy as np
import pytest
import torch
import torch.nn.functional as F

from oracle import oracle as o


def _torch_route(logits, k, scoring, bias, groups, topk_group, renorm, scale):
    """fni8serve/models/moe.py:62-91, verbatim in behaviour, fp32 on the CPU."""
    router_logits = torch.from_numpy(logits)
    if scoring == "sigmoid":
        scores = torch.sigmoid(router_logits)
        sel = scores + torch.from_numpy(bias) if bias is not None else scores
    else:
        scores = F.softmax(router_logits, dim=-1)
        sel = scores
    if groups:
        T = sel.shape[0]
        per = sel.shape[-1] // groups
        gs = sel.view(T, groups, per).amax(dim=-1)
        chosen = gs.topk(topk_group, dim=-1)[1]
        idx = (chosen.unsqueeze(-1) * per + torch.arange(per).view(1, 1, per)).reshape(T, -1)
        mask = torch.full_like(sel, float("-inf"))
        mask.scatter_(1, idx, 0.0)
        sel = sel + mask
    if scoring == "sigmoid":
        _, topi = torch.topk(sel, k, dim=-1)
        topw = scores.gather(-1, topi)
    else:
        topw, topi = torch.topk(sel, k, dim=-1)
    if renorm:
        topw = topw / topw.sum(dim=-1, keepdim=True).clamp_min(1e-9)
    return (topw * scale).half().numpy(), topi.numpy().astype(np.int32), sel.numpy()


CASES = [
    dict(E=128, k=8, scoring="softmax"),
    dict(E=64, k=2, scoring="softmax", renorm=False),
    dict(E=160, k=6, scoring="softmax", scale=2.5),
    dict(E=256, k=8, scoring="sigmoid", bias=True, groups=8, topk_group=4, scale=2.5),
    dict(E=256, k=8, scoring="sigmoid", bias=True),
    dict(E=512, k=10, scoring="softmax"),
    dict(E=1024, k=32, scoring="sigmoid", bias=True, groups=64, topk_group=7),
    dict(E=8, k=1, scoring="softmax"),
    dict(E=16, k=16, scoring="softmax"),
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "-".join(f"{k}{v}" for k, v in c.items()))
def test_route_matches_the_reference_torch_routing(case):
    rng = np.random.default_rng(case["E"] + case["k"])
    T, E, k = 300, case["E"], case["k"]
    logits = (rng.standard_normal((T, E)) * 2).astype(np.float32)
    bias = (rng.standard_normal(E) * 0.1).astype(np.float32) if case.get("bias") else None
    args = (case["scoring"], bias, case.get("groups", 0), case.get("topk_group", 0),
            case.get("renorm", True), case.get("scale", 1.0))
    w, i = o.moe_route(logits, k, *args[:1], bias=args[1], groups=args[2], topk_group=args[3],
                       renorm=args[4], scale=args[5])
    tw, ti, sel = _torch_route(logits, k, *args)
    # rows where two selection scores sit within 1e-6 of each other around the
    # cut may order differently under different fp32 roundings; none here
    srt = -np.sort(-sel, axis=1)
    kk = min(k + 1, E)
    gaps = np.abs(np.diff(srt[:, :kk], axis=1)) / np.maximum(np.abs(srt[:, :kk - 1]), 1e-30)
    clean = (gaps > 1e-6).all(axis=1)
    assert clean.mean() > 0.97
    assert np.array_equal(i[clean], ti[clean])
    ulp = np.spacing(np.abs(tw[clean]).astype(np.float16)).astype(np.float64)
    assert (np.abs(w[clean].astype(np.float64) - tw[clean].astype(np.float64)) <= ulp).all()


def test_route_topk_is_a_stable_sort_with_ties_and_nan():
    """Brute force: the experts, in order, of a stable descending sort of the
    scores (value, then index), with many exact ties (integer logits)."""
    rng = np.random.default_rng(7)
    logits = rng.integers(-3, 4, size=(200, 40)).astype(np.float32)
    w, i = o.moe_route(logits, 12, "softmax", renorm=False)
    p = np.exp(logits.astype(np.float64) - logits.max(1, keepdims=True))
    p /= p.sum(1, keepdims=True)
    for t in range(200):
        order = sorted(range(40), key=lambda e: (-logits[t, e], e))[:12]
        assert list(i[t]) == order
    # float64 softmax values, rounded to fp16, except within a hair of a tie
    ref = np.take_along_axis(p, i.astype(np.int64), 1).astype(np.float16)
    assert (w != ref).mean() < 1e-3
    # a NaN ranks first; a NaN logit makes the whole softmax row NaN
    x = np.float32([[0.0, 1.0, np.nan, 2.0]])
    w, i = o.moe_route(x, 2, "sigmoid", renorm=False)
    assert list(i[0]) == [2, 3] and np.isnan(w[0, 0])
    w, i = o.moe_route(x, 2, "softmax")
    assert list(i[0]) == [0, 1] and np.isnan(w).all()


def test_route_known_answers():
    # uniform logits: the first k experts, each 1/k after renormalisation
    w, i = o.moe_route(np.zeros((3, 64), np.float32), 8)
    assert (i == np.arange(8)).all() and (w == np.float16(0.125)).all()
    # -0 ranks with +0 (ties to the lower index)
    w, i = o.moe_route(np.float32([[-0.0, 0.0, -1.0]]), 2, "sigmoid", renorm=False)
    assert list(i[0]) == [0, 1]
    # renormalisation and scaling: two equal experts out of many -> 0.5 * 2.5
    x = np.full((1, 10), -20.0, np.float32)
    x[0, 3] = x[0, 7] = 5.0
    w, i = o.moe_route(x, 2, scale=2.5)
    assert list(i[0]) == [3, 7] and (w == np.float16(1.25)).all()
    # a sum below 1e-9 is divided by 1e-9 (clamp_min), not by itself
    w, i = o.moe_route(np.float32([[-30.0, -30.0, 10.0]]), 2, "sigmoid")
    assert list(i[0]) == [2, 0]


def test_route_groups_and_bias():
    """Group-limited selection: the best expert outside the chosen groups is
    never picked; bias steers selection, the weights stay unbiased."""
    x = np.full((1, 16), -5.0, np.float32)     # 4 groups of 4
    x[0, 0] = 3.0                              # group 0: max 3.0
    x[0, 5:8] = [2.9, 2.8, 2.7]                # group 1: max 2.9
    x[0, 8] = 2.95                             # group 2: max 2.95
    w, i = o.moe_route(x, 3, "sigmoid", groups=4, topk_group=2, renorm=False)
    assert list(i[0]) == [0, 8, 1]             # groups 0 and 2 only; then index order
    sig = 1 / (1 + np.exp(-x[0].astype(np.float64)))
    assert w[0, 0] == np.float16(sig[0]) and w[0, 1] == np.float16(sig[8])
    bias = np.zeros(16, np.float32)
    bias[12] = 10.0                            # group 3 wins through its bias
    w, i = o.moe_route(x, 1, "sigmoid", bias=bias, groups=4, topk_group=1, renorm=False)
    assert list(i[0]) == [12] and w[0, 0] == np.float16(sig[12])
    # k larger than the kept groups: the masked experts follow at -inf, lowest index first
    w, i = o.moe_route(x, 6, "softmax", groups=4, topk_group=1, renorm=False)
    assert list(i[0][:4]) == [0, 1, 2, 3] and list(i[0][4:]) == [4, 5]
    assert np.isneginf(w[0, 4:].astype(np.float32)).all()


def test_softmax_denominator_order():
    """The fixed order (64 accumulators by expert index, then a butterfly),
    restated in fp32 Python floats over the oracle's own exp values, on a row
    where it differs from left-to-right summation: the oracle's weight of the
    top expert is exactly fp16(1 / s) for the restated s."""
    E = 192
    x = np.full(E, -10.0, np.float32)
    x[0] = 10.0
    x[64] = 10.0
    x[100:140] = 9.0
    f32 = np.float32
    e = [f32(v) for v in o.exp_cw((x - f32(10.0)).astype(np.float32))]
    acc = [f32(0)] * 64
    for i in range(E):
        acc[i % 64] = f32(acc[i % 64] + e[i])
    for d in (32, 16, 8, 4, 2, 1):
        acc = [f32(acc[a] + acc[a ^ d]) for a in range(64)]
    seq = f32(0)
    for v in e:
        seq = f32(seq + v)
    assert acc[0] != seq  # the order is visible on this row
    w, i = o.moe_route(x[None], 2, renorm=False)
    assert list(i[0]) == [0, 64]
    assert w[0, 0] == np.float16(f32(e[0] / acc[0]))
