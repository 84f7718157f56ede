"""RMSNorm (fni8serve/layers/norm.py:21-58).

Same constructor and forward contract: `RMSNorm(dim, eps=1e-6, weight=None, *,
add_unit_offset=False)`; `forward(x, residual=None)` returns the normed tensor,
or `(normed, x + residual)` with a residual (the fused residual add).  A GPU
fp16 tensor with an fp16 weight takes the kernel (`ops.rmsnorm`, one launch);
every other input (CPU, or another dtype on the GPU) takes the reference's eager
fp32 form (norm.py:37-43, :56-58), so no input raises where the reference
returns a result.  `forward_quant` is the
fused form for a norm that feeds a W8A8 linear (QKV, gate_up): it returns the
linear's int8 input and per-token scales instead of the fp16 row.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import ops


class RMSNorm(nn.Module):
    def __init__(self, dim: int, eps: float = 1e-6, weight: torch.Tensor | None = None, *,
                 add_unit_offset: bool = False):
        super().__init__()
        self.eps = eps
        self.add_unit_offset = add_unit_offset
        if weight is None:
            weight = (torch.zeros(dim, dtype=torch.float16) if add_unit_offset
                      else torch.ones(dim, dtype=torch.float16))
        self.weight = nn.Parameter(weight)

    def _norm(self, x: torch.Tensor) -> torch.Tensor:
        dt = x.dtype
        xf = x.float()
        xf = xf * torch.rsqrt(xf.pow(2).mean(-1, keepdim=True) + self.eps)
        w = (1.0 + self.weight.float()) if self.add_unit_offset else self.weight.float()
        return (xf * w).to(dt)

    def forward(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        if x.is_cuda and x.dtype == torch.float16 and self.weight.dtype == torch.float16:
            return ops.rmsnorm(x, self.weight.detach(), self.eps, residual=residual,
                               unit_offset=self.add_unit_offset)
        if residual is None:
            return self._norm(x)
        x = x + residual
        return self._norm(x), x

    def forward_quant(self, x: torch.Tensor, residual: torch.Tensor | None = None):
        """(xq int8 [M, K], xs fp32 [M]) -- plus x + residual with a residual --
        bit-identical to quantizing forward(x, residual)'s normed output."""
        return ops.rmsnorm_quant(x, self.weight.detach(), self.eps, residual=residual,
                                 unit_offset=self.add_unit_offset)
