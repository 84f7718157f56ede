"""Seeded synthetic inputs for the W8A8 linear workloads.

Shapes are the Qwen3-8B decoder linears and the Qwen3-30B-A3B-style expert
GEMMs; distributions follow the measurement plan of the hot path:
  x     fp16 ~ N(0, 1), each element an outlier with probability 0.01, scaled x20
  W     int8 uniform in [-127, 127]
  w_s   drawn in fp16 from U(0.001, 0.02), stored fp32 (exact)
  MoE   router logits N(0, 1) + a seeded Zipf-like bias -ln(1 + rank[e]),
        softmax over all experts, top-8, renormalised (fni8serve/models/moe.py:70-95)
Every generator takes an explicit seed and a device; generation on "cpu" is
bit-reproducible across runs, and the GPU gets copies of the same tensors.
"""
from __future__ import annotations

import torch

# Qwen3-8B decoder linears: name -> (N, K)
QWEN3_8B_LINEARS = {
    "qkv": (6144, 4096),      # 32 q heads + 8 kv heads x head_dim 128, fused
    "o": (4096, 4096),
    "gate_up": (24576, 4096),  # gate and up merged
    "down": (4096, 12288),
}
DECODE_M = (1, 4, 16, 64)
PREFILL_M = (512, 2048, 4096)
QWEN3_8B_LAYERS = 36

# Qwen3-0.6B MLP gate_up at M=8: the CPU-runnable single-linear case
CPU_CASE = {"M": 8, "N": 6144, "K": 1024}

# Qwen3-30B-A3B-style MoE
MOE = {"experts": 128, "top_k": 8, "hidden": 2048, "inter": 768}
MOE_T = (16, 256, 4096)

OUTLIER_P = 0.01
OUTLIER_SCALE = 20.0


def _gen(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activations(M: int, K: int, seed: int, device="cpu") -> torch.Tensor:
    g = _gen(seed, device)
    x = torch.randn(M, K, generator=g, device=device, dtype=torch.float32)
    outlier = torch.rand(M, K, generator=g, device=device) < OUTLIER_P
    x = torch.where(outlier, x * OUTLIER_SCALE, x)
    return x.to(torch.float16)


def weight_i8(N: int, K: int, seed: int, device="cpu"):
    """(data int8 [N, K], scale fp32 [N])."""
    g = _gen(seed, device)
    q = torch.randint(-127, 128, (N, K), generator=g, device=device, dtype=torch.int8)
    s = (torch.rand(N, generator=g, device=device) * 0.019 + 0.001).to(torch.float16).float()
    return q, s


def expert_weights(E: int, N: int, K: int, seed: int, device="cpu"):
    """Stacked (data int8 [E, N, K], scale fp32 [E, N])."""
    g = _gen(seed, device)
    q = torch.randint(-127, 128, (E, N, K), generator=g, device=device, dtype=torch.int8)
    s = (torch.rand(E, N, generator=g, device=device) * 0.019 + 0.001).to(torch.float16).float()
    return q, s


def router_logits(T: int, E: int, seed: int, device="cpu") -> torch.Tensor:
    g = _gen(seed, device)
    rank = torch.randperm(E, generator=g, device=device).float()
    bias = -torch.log1p(rank)
    return torch.randn(T, E, generator=g, device=device) + bias


def route(logits: torch.Tensor, top_k: int, dtype=torch.float16):
    """softmax over all experts -> top-k -> renormalise -> cast (moe.py:70-95)."""
    scores = torch.softmax(logits.float(), dim=-1)
    topw, topi = torch.topk(scores, top_k, dim=-1)
    topw = topw / topw.sum(dim=-1, keepdim=True).clamp_min(1e-9)
    return topw.to(dtype), topi


def linear_bytes(M: int, N: int, K: int, bias: bool = False) -> int:
    """Algorithmic HBM bytes of one W8A8 linear: W int8 + w_s fp32 + x fp16 in + y fp16 out."""
    return N * K + 4 * N + 2 * M * K + 2 * M * N + (2 * N if bias else 0)


def linear_ops(M: int, N: int, K: int) -> int:
    return 2 * M * N * K


def grouped_bytes(active_experts: int, R: int, N: int, K: int) -> int:
    """Algorithmic bytes of one grouped projection over R routed rows."""
    return active_experts * (N * K + 4 * N) + R * (2 * K + 2 * N)
