"""Public kernel surface, as the reference's ``kernels/__init__.py:1-6``."""

from .fused_decode_attn import (  # noqa: F401
    choose_waves,
    default_num_splits,
    fused_decode_attention,
    hip_available,
    pick_num_splits,
    plan_splits,
    triton_available,
)
from .fp16_decode_attn import fp16_decode_attention  # noqa: F401
