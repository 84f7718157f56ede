"""Weight helpers that build per_row_i8 QTensors (fni8serve/models/weights.py:18-49).

QKV and gate/up are merged on the output axis so the runtime issues fewer,
wider GEMMs: q/k/v -> QKV [6144, 4096] and gate/up -> [24576, 4096] at
Qwen3-8B shapes.  For already-quantized rows the int8 data and the per-row
scales are concatenated, which is exact because every output row keeps its
own scale.
"""
from __future__ import annotations

import torch

from ..qtensor import QTensor
from ..quant import quantize_int8_rowwise


def to_qtensor(w) -> QTensor:
    """fp16/fp32 weight [out, in] (in % 4 == 0) -> per_row_i8 QTensor; a QTensor
    passes through unchanged (weights.py:18-25)."""
    if isinstance(w, QTensor):
        return w
    q, s = quantize_int8_rowwise(w)
    return QTensor(q.contiguous(), s.squeeze(-1).float().contiguous(), scheme="per_row_i8")


def merge_qtensor(rows: list) -> QTensor:
    """Row-concatenate q/k/v (or gate/up) (weights.py:28-39)."""
    if isinstance(rows[0], QTensor):
        data = torch.cat([r.data for r in rows], dim=0)
        scale = torch.cat([r.scale for r in rows], dim=0)
        r0 = rows[0]
        return QTensor(data.contiguous(), scale.contiguous(), scheme=r0.scheme,
                       group_size=r0.group_size, codebook=r0.codebook)
    return to_qtensor(torch.cat(rows, dim=0))


def qkv_weight(sd: dict, prefix: str) -> QTensor:
    return merge_qtensor([sd[f"{prefix}.q_proj.weight"], sd[f"{prefix}.k_proj.weight"],
                          sd[f"{prefix}.v_proj.weight"]])


def gate_up_weight(sd: dict, prefix: str) -> QTensor:
    return merge_qtensor([sd[f"{prefix}.gate_proj.weight"], sd[f"{prefix}.up_proj.weight"]])
