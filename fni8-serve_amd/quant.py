"""Load-time per-row int8 weight quantization.

`quantize_int8_rowwise(w) -> (q int8 [N, K], s fp32 [N, 1])` stands in for
`fni8.quant.core.quantize_int8_rowwise`, which the reference calls when it
builds per_row_i8 QTensors (fni8serve/models/weights.py:24,
fni8serve/convert.py:65, tools/forge.py:139); callers squeeze the scale
(`s.squeeze(-1).float()`).  `fni8` is closed and absent, so the convention is
the reference's own Python quant idiom (tests/test_layers.py:31-32,
tests/test_smoke.py:16-17) evaluated in fp32:

    s = amax(|w_row|).clamp_min(1e-6) / 127 ;  q = round(w / s).clamp(-127, 127)

This runs once per weight at load or conversion time, on the weight's device,
and is not part of the timed path.
"""
from __future__ import annotations

import torch

QUANT_EPS = 1e-6


def quantize_int8_rowwise(w: torch.Tensor):
    if w.dim() != 2:
        raise ValueError("quantize_int8_rowwise expects a 2-D weight [out, in]")
    wf = w.float()
    s = wf.abs().amax(dim=-1, keepdim=True).clamp_min(QUANT_EPS) / 127.0
    q = torch.round(wf / s).clamp_(-127, 127).to(torch.int8)
    return q, s
