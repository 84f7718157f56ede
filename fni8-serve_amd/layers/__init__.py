from .embedding import LMHead  # noqa: F401
from .linear import NF4_CODEBOOK, LinearW8A8, _dequant_weight  # noqa: F401
from .activation import GeluAndMul, SiluAndMul, get_act_and_mul  # noqa: F401
from .mlp import GatedMLP, Qwen3MLP  # noqa: F401
from .norm import RMSNorm  # noqa: F401
from .moe import SparseMoE  # noqa: F401
from .weights import gate_up_weight, merge_qtensor, qkv_weight, to_qtensor  # noqa: F401
