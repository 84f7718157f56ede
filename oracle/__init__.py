"""CPU oracle for the W8A8 linear path (test infrastructure only).

Only `tests/`, `__graft_entry__.smoke()` and the CPU-baseline leg of `bench.py`
may import this package, and only to check results or as the timed CPU baseline.
The product path (the `fni8serve_amd` package) never imports it.
"""
from .oracle import (  # noqa: F401
    QUANT_EPS,
    dequant_f16,
    f16_to_f32,
    f32_to_f16,
    gemm_i8,
    grouped_w8a8_f16,
    linear_w8a8_f16,
    moe_combine_f16,
    moe_sort,
    quant_rowwise_f16,
)
