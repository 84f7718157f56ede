"""Gated MLP over two W8A8 linears (fni8serve/layers/mlp.py:22-48).

`GatedMLP(gate_up, down, *, act="silu", bias_gate_up=None, bias_down=None)`
computes down(act_and_mul(gate_up(x))) with gate/up merged into one
[2*intermediate, hidden] weight (mlp.py:39-40).  On the GPU, with int8
weights, a kernel activation (silu, tanh gelu) and at least FUSE_MIN_ROWS
rows, the activation and the down projection's per-token quantization run as
one launch (`ops.act_and_mul_quant`) feeding the int8 GEMM directly: the fp16
[M, intermediate] tensor never goes to HBM, and the result is bit-identical to
the unfused chain.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import ops
from ..qtensor import QTensor
from .activation import SiluAndMul, fused_act, get_act_and_mul
from .linear import LinearW8A8

# Rows from which the fused activation + quantization feeds the down projection.
# Below it the unfused chain is faster: up to 4 rows the down projection's
# linear() quantizes its own input inside the GEMM at almost no cost, while the
# fused kernel runs each row's activation (12288 exps for Qwen3-8B) on one
# workgroup (MI355X, Qwen3-8B down chain, unfused vs fused: 10.07 vs 11.66 us at
# 1 row, 12.54 vs 14.69 at 4; 15.81 vs 15.50 at 16, 26.73 vs 26.09 at 64).
FUSE_MIN_ROWS = 5


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
        act = fused_act(self.act_fn)
        rows = x.numel() // max(x.shape[-1], 1)
        if (act is not None and rows >= FUSE_MIN_ROWS and self.gate_up_proj._int8_ok(x)
                and self.down_proj._int8_ok(x)):
            h = self.gate_up_proj(x)
            xq, xs = ops.act_and_mul_quant(h, act)
            y = ops.gemm_quantized(xq, xs, self.down_proj.weight, self.down_proj.bias)
            return y.reshape(*x.shape[:-1], y.shape[-1])
        return self.down_proj(self.act_fn(self.gate_up_proj(x)))


class Qwen3MLP(GatedMLP):
    """Qwen3 dense MLP (SwiGLU)."""

    def __init__(self, gate_up: QTensor, down: QTensor, bias_gate_up=None, bias_down=None):
        super().__init__(gate_up, down, act=SiluAndMul(), bias_gate_up=bias_gate_up,
                         bias_down=bias_down)
