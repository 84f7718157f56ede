"""Gated activations over a merged gate_up output (fni8serve/layers/activation.py:20-53).

SiluAndMul (Qwen3) and GeluAndMul (Gemma, tanh form) split [..., 2I] into gate
and up and return act(gate) * up.  As in the reference (`_fused_ok`,
activation.py:16-17, :24, :40), a GPU fp16 tensor takes the fused kernel
(`ops.act_and_mul`, one launch).  Every other input takes the eager torch form
`act(gate) * up` in the input's own dtype: CPU tensors, the exact-erf gelu,
GPU fp32 (which the reference also computes eagerly) and GPU bf16 (which the
reference sends to its closed fused kernel; the kernel here is fp16-only, and
the bf16 result is torch's).  No input raises where the reference returns a
result.  `fused_act(module)` names the kernel activation a module computes, so
GatedMLP and SparseMoE can fuse it with the down projection's quantization.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from .. import ops


def _kernel_ok(x: torch.Tensor) -> bool:
    return x.is_cuda and x.dtype == torch.float16


class SiluAndMul(nn.Module):
    def forward(self, x: torch.Tensor) -> torch.Tensor:
        """x: [..., 2*intermediate], first half gate, second half up."""
        if _kernel_ok(x):
            return ops.act_and_mul(x, "silu")
        gate, up = x.chunk(2, dim=-1)
        return F.silu(gate) * up


class GeluAndMul(nn.Module):
    """GeGLU; HF `hidden_act='gelu_pytorch_tanh'` is the tanh approximation."""

    def __init__(self, approximate: str = "tanh"):
        super().__init__()
        self.approximate = approximate

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.approximate == "tanh" and _kernel_ok(x):
            return ops.act_and_mul(x, "gelu_tanh")
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


def fused_act(module: nn.Module) -> str | None:
    """The kernel activation ("silu" / "gelu_tanh") `module` computes, or None."""
    if type(module) is SiluAndMul:
        return "silu"
    if type(module) is GeluAndMul and module.approximate == "tanh":
        return "gelu_tanh"
    return None
