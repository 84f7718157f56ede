"""LMHead over a W8A8 linear (fni8serve/layers/embedding.py:34-53).

An int8 head is a LinearW8A8 with N = vocab.  Its input is often
`hidden[:, -1]`, a strided view whose rows are S*hidden elements apart; the
linear passes that row stride to the kernels instead of copying.
"""
from __future__ import annotations

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..qtensor import QTensor
from .linear import LinearW8A8


class LMHead(nn.Module):
    def __init__(self, weight: QTensor | torch.Tensor, logit_softcap: float | None = None):
        super().__init__()
        self.logit_softcap = logit_softcap
        if isinstance(weight, QTensor):
            self.proj = LinearW8A8(weight)
            self._fp16_w = None
        else:
            self.proj = None
            self.weight = nn.Parameter(weight)
            self._fp16_w = True

    def forward(self, hidden: torch.Tensor) -> torch.Tensor:
        logits = self.proj(hidden) if self.proj is not None else F.linear(hidden, self.weight)
        if self.logit_softcap:
            logits = self.logit_softcap * torch.tanh(logits.float() / self.logit_softcap)
        return logits
