"""Gated MLP over two W8A8 linears (fni8serve/layers/mlp.py:22-48).

`GatedMLP(gate_up, down, *, act="silu", bias_gate_up=None, bias_down=None)`
computes down(act_and_mul(gate_up(x))) with gate/up merged into one
[2*intermediate, hidden] weight (mlp.py:39-40).  The activations restate
fni8serve/layers/activation.py:20-53 (SiluAndMul, GeluAndMul,
get_act_and_mul); they run as PyTorch elementwise ops between the two
linears.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..qtensor import QTensor
from .linear import LinearW8A8


class SiluAndMul(nn.Module):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: [..., 2*intermediate], first half gate, second half up."""
        gate, up = x.chunk(2, dim=-1)
        return F.silu(gate) * up


class GeluAndMul(nn.Module):
    """GeGLU; HF `hidden_act='gelu_pytorch_tanh'` is the tanh approximation."""

    def __init__(self, approximate: str = "tanh"):
        super().__init__()
        self.approximate = approximate

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        gate, up = x.chunk(2, dim=-1)
        return F.gelu(gate, approximate=self.approximate) * up


def get_act_and_mul(hidden_act: str) -> nn.Module:
    a = hidden_act.lower()
    if a == "silu":
        return SiluAndMul()
    if a in ("gelu_pytorch_tanh", "gelu_tanh"):
        return GeluAndMul("tanh")
    if a in ("gelu", "gelu_new"):
        return GeluAndMul("none")
    raise ValueError(f"unsupported gated activation {hidden_act!r}")


class GatedMLP(nn.Module):
    def __init__(self, gate_up: QTensor, down: QTensor, *, act: nn.Module | str = "silu",
                 bias_gate_up=None, bias_down=None):
        super().__init__()
        self.gate_up_proj = LinearW8A8(gate_up, bias_gate_up)
        self.down_proj = LinearW8A8(down, bias_down)
        self.act_fn = get_act_and_mul(act) if isinstance(act, str) else act
        self.hidden_size = self.down_proj.out_features
        self.intermediate_size = self.gate_up_proj.out_features // 2

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.down_proj(self.act_fn(self.gate_up_proj(x)))


class Qwen3MLP(GatedMLP):
    """Qwen3 dense MLP (SwiGLU)."""

    def __init__(self, gate_up: QTensor, down: QTensor, bias_gate_up=None, bias_down=None):
        super().__init__(gate_up, down, act=SiluAndMul(), bias_gate_up=bias_gate_up,
                         bias_down=bias_down)
