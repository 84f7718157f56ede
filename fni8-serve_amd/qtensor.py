"""QTensor: the quantized-weight container the linear consumes.

Mirrors the constructor and attributes of `fni8.QTensor` as the reference uses
it (ctor at fni8serve/models/weights.py:25 and :35-36, tests/test_smoke.py:18,
:28-29; attributes read at fni8serve/layers/linear.py:30-44, :52-65):

    QTensor(data, scale, *, scheme, group_size=None, codebook=None)
    .data .scale .scheme .group_size .codebook

For scheme "per_row_i8" (the W8A8 path): data int8 [N, K] row-major, scale
fp32 [N].  "per_group_i4" packs two int4 codes per byte with a per-group
scale; "raw" carries an unquantized tensor and no scale
(fni8serve/convert.py:133).
"""
from __future__ import annotations

import torch

SCHEMES = ("per_row_i8", "per_group_i4", "raw")


class QTensor:
    __slots__ = ("data", "scale", "scheme", "group_size", "codebook")

    def __init__(self, data: torch.Tensor, scale: torch.Tensor | None, *, scheme: str,
                 group_size: int | None = None, codebook: str | None = None):
        if scheme not in SCHEMES:
            raise ValueError(f"unknown QTensor scheme {scheme!r}")
        if scheme == "per_row_i8":
            if data.dtype != torch.int8 or data.dim() != 2:
                raise ValueError("per_row_i8 data must be int8 [out, in]")
            if scale is None or scale.numel() != data.shape[0]:
                raise ValueError("per_row_i8 scale must have one entry per output row")
        self.data = data
        self.scale = scale
        self.scheme = scheme
        self.group_size = group_size
        self.codebook = codebook

    @property
    def shape(self):
        return self.data.shape

    @property
    def device(self):
        return self.data.device

    def to(self, device) -> "QTensor":
        return QTensor(self.data.to(device), None if self.scale is None else self.scale.to(device),
                       scheme=self.scheme, group_size=self.group_size, codebook=self.codebook)

    def cuda(self) -> "QTensor":
        return self.to("cuda")

    def __repr__(self) -> str:
        return (f"QTensor(scheme={self.scheme!r}, shape={tuple(self.data.shape)}, "
                f"device={self.data.device})")
