"""SANA ReLU linear attention drop-in (mirrors SANA_LinearAttention/__init__.py:3-26
for the attention hot path: ``qkv_attn_matmul``)."""

from .custom import default_splits, linear_attention, qkv_attn_matmul

__all__ = ["qkv_attn_matmul", "linear_attention", "default_splits"]
