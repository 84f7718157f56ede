"""Restatements of the reference's own CPU code paths (test infrastructure only).

`reference_cpu_linear` is the only CPU implementation of `LinearW8A8` the
reference has (fni8serve/layers/linear.py:28-31 and :70-71): dequantize the
per_row_i8 weight to fp16 on every call, then `F.linear` in the activation
dtype.  It is not W8A8 arithmetic (no activation quantization, no int32
accumulator); the benchmark times it as the CPU baseline, and the tests use it
for the reference's own tolerance checks (cosine >= 0.99,
tests/test_smoke.py:68-80).

`reference_moe_loop` restates SparseMoE.forward's routing and expert loop
(fni8serve/models/moe.py:62-105, softmax scoring, no shared expert) with each
expert linear computed by the W8A8 oracle, so the grouped path can be checked
against the loop it replaces.
"""
from __future__ import annotations

import numpy as np
import torch
import torch.nn.functional as F

from . import oracle


def dequant_weight_per_row_i8(q: torch.Tensor, s: torch.Tensor) -> torch.Tensor:
    """linear.py:31: (qt.data.float() * qt.scale.unsqueeze(-1)).to(fp16)."""
    return (q.float() * s.unsqueeze(-1)).to(torch.float16)


def reference_cpu_linear(x: torch.Tensor, q: torch.Tensor, s: torch.Tensor,
                         bias: torch.Tensor | None = None) -> torch.Tensor:
    """linear.py:70-71: w = _dequant_weight(qt).to(x.dtype); F.linear(x, w, bias)."""
    w = dequant_weight_per_row_i8(q, s).to(x.dtype)
    return F.linear(x, w, bias)


def route_softmax_topk(x: torch.Tensor, gate: torch.Tensor, top_k: int,
                       norm_topk_prob: bool = True):
    """moe.py:65-95 (softmax scoring): fp32 router, softmax over all experts,
    top-k, renormalise, cast the weights to the activation dtype."""
    xf = x.reshape(-1, x.shape[-1])
    logits = F.linear(xf.float(), gate.float())
    scores = F.softmax(logits, dim=-1)
    topw, topi = torch.topk(scores, top_k, dim=-1)
    if norm_topk_prob:
        topw = topw / topw.sum(dim=-1, keepdim=True).clamp_min(1e-9)
    return topw.to(x.dtype), topi


def silu_and_mul_f16(h: np.ndarray) -> np.ndarray:
    """activation.py:25-26 on the CPU: silu(gate) * up in fp16 torch ops."""
    t = torch.from_numpy(np.ascontiguousarray(h, np.float16))
    g, u = t.chunk(2, dim=-1)
    return (F.silu(g) * u).numpy()


def reference_moe_loop(xf: np.ndarray, topi: np.ndarray, topw: np.ndarray,
                       gu_q, gu_s, dn_q, dn_s, act=silu_and_mul_f16) -> np.ndarray:
    """moe.py:97-105 with W8A8 oracle linears: for each expert e in order,
    gather its (token, slot) rows via nonzero, run gate_up -> act -> down,
    weight by topw and index_add into an fp16 zero tensor."""
    T, H = xf.shape
    out = np.zeros((T, H), np.float16)
    E = gu_q.shape[0]
    for e in range(E):
        mask = topi == e
        if not mask.any():
            continue
        tok_idx, slot = np.nonzero(mask)
        xe = xf[tok_idx]
        h1, *_ = oracle.linear_w8a8_f16(xe, gu_q[e], gu_s[e])
        a = act(h1)
        h2, *_ = oracle.linear_w8a8_f16(a, dn_q[e], dn_s[e])
        w = topw[tok_idx, slot].astype(np.float16)[:, None]
        contrib = (h2.astype(np.float32) * w.astype(np.float32)).astype(np.float16)
        cur = out[tok_idx].astype(np.float32) + contrib.astype(np.float32)
        out[tok_idx] = cur.astype(np.float16)
    return out
