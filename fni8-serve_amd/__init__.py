"""fni8serve_amd: the W8A8 linear path of fni8-serve, native to MI355X (gfx950).

Drop-in pieces for the reference's seam (fni8serve/layers/linear.py and its
callers):

    linear(x, qt, bias=None)      the `fni8.linear` call (linear.py:69), W8A8
                                  (per_row_i8) and W4A8 (per_group_i4 int4)
    QTensor                       the quantized-weight container
    quantize_int8_rowwise(w)      load-time per-row weight quantization
    act_and_mul(x, act), rmsnorm(x, w, eps, residual=, unit_offset=)
                                  the producers of the linears' inputs
                                  (activation.py:24, norm.py:51), and their
                                  forms fused with the next linear's
                                  quantization (act_and_mul_quant, rmsnorm_quant)
    LinearW8A8, GatedMLP, SparseMoE, LMHead, RMSNorm and the weight helpers
    save_fni8, FQWriter, FQReader the `.fni8` checkpoint container
    load_fni8_checkpoint, load_fni8_state_dict, checkpoint_info
                                  the loader (fni8serve/loader.py:19-69)

The arithmetic runs in libfni8amd.so (hand-written HIP kernels for gfx950,
C ABI in include/fni8amd.h); this package is the host side.  The directory is
named `fni8-serve_amd`; it is imported as `fni8serve_amd`.
"""
from .ops import (  # noqa: F401
    act_and_mul,
    act_and_mul_quant,
    gemm_quantized,
    gemm_w4a8,
    gemm_w8a8,
    gemm_w8a8_grouped,
    linear,
    linear_with_intermediates,
    moe_combine,
    moe_sort,
    quantize_rowwise,
    rmsnorm,
    rmsnorm_quant,
)
from .qtensor import QTensor  # noqa: F401
from .container import FQReader, FQWriter, save_fni8  # noqa: F401
from .loader import checkpoint_info, load_fni8_checkpoint, load_fni8_state_dict  # noqa: F401
from .quant import quantize_int8_rowwise  # noqa: F401
from .layers import (  # noqa: F401
    NF4_CODEBOOK,
    GatedMLP,
    GeluAndMul,
    RMSNorm,
    SiluAndMul,
    get_act_and_mul,
    LinearW8A8,
    LMHead,
    Qwen3MLP,
    SparseMoE,
    _dequant_weight,
    gate_up_weight,
    merge_qtensor,
    qkv_weight,
    to_qtensor,
)

__all__ = [
    "linear", "linear_with_intermediates", "quantize_rowwise", "gemm_w8a8", "gemm_w8a8_grouped",
    "moe_sort", "moe_combine", "QTensor", "quantize_int8_rowwise", "LinearW8A8", "GatedMLP",
    "Qwen3MLP", "SparseMoE", "LMHead", "NF4_CODEBOOK", "to_qtensor", "merge_qtensor",
    "qkv_weight", "gate_up_weight", "save_fni8", "FQWriter", "FQReader", "load_fni8_checkpoint",
    "load_fni8_state_dict", "checkpoint_info", "act_and_mul", "act_and_mul_quant", "rmsnorm",
    "rmsnorm_quant", "RMSNorm", "SiluAndMul", "GeluAndMul", "get_act_and_mul", "gemm_w4a8",
    "gemm_quantized",
]
