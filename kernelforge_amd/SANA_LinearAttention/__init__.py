"""SANA ReLU linear attention drop-in (mirrors SANA_LinearAttention/__init__.py:3-26):
the attention factory ``qkv_attn_matmul``, the ``LiteLA`` / ``CustomLiteLA`` /
``JointLiteLA`` modules and the ``qkv_projection`` factory."""

from .custom import default_splits, linear_attention, qkv_attn_matmul
from .modules import CustomLiteLA, JointLiteLA, LiteLA, apply_rotary_emb, qkv_projection

__all__ = ["LiteLA", "CustomLiteLA", "JointLiteLA", "apply_rotary_emb", "qkv_attn_matmul", "qkv_projection",
           "linear_attention", "default_splits"]
