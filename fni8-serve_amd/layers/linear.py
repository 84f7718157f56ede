"""LinearW8A8: the reference's linear seam, on the gfx950 W8A8 kernels.

Same constructor, attributes and module-level helpers as
fni8serve/layers/linear.py:28-71:

    LinearW8A8(weight: QTensor, bias: Tensor | None = None)
    .weight .bias .out_features .in_features     (read by layers/mlp.py:36-37
                                                  and training/lora.py:17-37)
    _dequant_weight(qt)                          (linear.py:28-46)
    NF4_CODEBOOK                                 (linear.py:22-25)

forward(x) dispatch follows linear.py:58-71: a per_row_i8 (W8A8) or
per_group_i4 int4 (W4A8) weight with x on the GPU runs `ops.linear`
(per-token quant + int8 GEMM + fused epilogue); a CPU x runs the reference's
numerically-correct fp16 fallback (dequantize the weight, F.linear), which is
the reference's documented CPU behaviour.  On the GPU there is no fallback for
those schemes: a missing library raises.  NF4 weights take the dequant path on
either device, as in the reference (linear.py:11-12, :65).
"""
from __future__ import annotations

import torch
import torch.nn as nn

from .. import ops
from ..qtensor import QTensor

# The 16 NormalFloat-4 levels (Dettmers et al., QLoRA, 2023, Appendix E).
NF4_CODEBOOK = (
    -1.0, -0.6961928009986877, -0.5250730514526367, -0.39491748809814453,
    -0.28444138169288635, -0.18477343022823334, -0.09105003625154495, 0.0,
    0.07958029955625534, 0.16093020141124725, 0.24611230194568634, 0.33791524171829224,
    0.44070982933044434, 0.5626170039176941, 0.7229568362236023, 1.0,
)


def _dequant_weight(qt: QTensor) -> torch.Tensor:
    """Reconstruct an fp16 weight [out, in] from a QTensor (linear.py:28-46)."""
    if qt.scheme == "per_row_i8":
        return (qt.data.float() * qt.scale.unsqueeze(-1)).to(torch.float16)
    if qt.scheme == "per_group_i4":
        packed = qt.data.to(torch.int32)                       # [out, in // 2]
        lo = packed & 0xF
        hi = (packed >> 4) & 0xF
        codes = torch.stack([lo, hi], -1).reshape(qt.data.shape[0], -1)  # [out, in]
        if qt.codebook == "nf4":
            cb = torch.tensor(NF4_CODEBOOK, device=codes.device, dtype=torch.float32)
            vals = cb[codes.long()]
        else:  # signed int4, two's complement
            vals = codes.float() - 16.0 * (codes >= 8).float()
        g = qt.group_size
        out, in_ = vals.shape
        scale = qt.scale.reshape(out, in_ // g, 1)
        return (vals.reshape(out, in_ // g, g) * scale).reshape(out, in_).to(torch.float16)
    raise ValueError(f"LinearW8A8 cannot use scheme {qt.scheme!r}")


class LinearW8A8(nn.Module):
    def __init__(self, weight: QTensor, bias: torch.Tensor | None = None):
        super().__init__()
        self.weight = weight          # QTensor; a plain attribute, as in the reference
        self.bias = bias
        self.out_features = weight.data.shape[0]
        self.in_features = weight.data.shape[1] * (2 if weight.scheme == "per_group_i4" else 1)

    def _int8_ok(self, x: torch.Tensor) -> bool:
        """The int8 kernels run for GPU activations with per_row_i8 weights
        (W8A8) or per_group_i4 int4 weights (W4A8) -- linear.py:58-65."""
        if not x.is_cuda:
            return False
        qt = self.weight
        return qt.scheme == "per_row_i8" or (qt.scheme == "per_group_i4" and qt.codebook == "int4")

    # the reference's name for the same rule (linear.py:58)
    _dp4a_ok = _int8_ok

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self._int8_ok(x):
            return ops.linear(x, self.weight, bias=self.bias)
        qt = self.weight
        w = _dequant_weight(qt).to(x.dtype)    # reference fallback: CPU tensors, NF4
        return torch.nn.functional.linear(x, w, self.bias)
