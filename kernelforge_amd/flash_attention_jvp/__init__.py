"""FlashAttention forward/JVP drop-in (mirrors flash_attention_jvp/__init__.py:3-15)
plus the fused single-pass ``flash_attention_fwd_jvp`` and the standalone
backward ``flash_attention_backward``."""

from .custom import (
    FlashAttentionFunction,
    flash_attention,
    flash_attention_backward,
    flash_attention_fwd_jvp,
    flash_attention_jvp,
    get_jvp_config,
)

__all__ = [
    "FlashAttentionFunction",
    "flash_attention",
    "flash_attention_backward",
    "flash_attention_jvp",
    "flash_attention_fwd_jvp",
    "get_jvp_config",
]
