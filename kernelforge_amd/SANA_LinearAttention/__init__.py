"""SANA ReLU linear attention drop-in (mirrors SANA_LinearAttention/__init__.py:3-26):
the attention factory ``qkv_attn_matmul``, the ``LiteLA`` / ``CustomLiteLA`` /
``JointLiteLA`` modules, their custom-operator, HIP-graph and single-shape
variants (``CustomOpJointLiteLA``, ``CUDAGraphJointLiteLA``,
``GroupedFull64QOutLiteLA``, ``optimized_joint_litela``) and the
``qkv_projection`` factory."""

from .custom import attn_matmul, check_status, default_splits, linear_attention, qkv_attn_matmul
from .modules import (CUDAGraphJointLiteLA, CustomLiteLA, CustomOpJointLiteLA, GroupedFull64QOutLiteLA,
                      JointLiteLA, LiteLA, apply_rotary_emb, optimized_joint_litela, qkv_projection)

__all__ = ["LiteLA", "CustomLiteLA", "apply_rotary_emb", "qkv_attn_matmul", "qkv_projection", "JointLiteLA",
           "CustomOpJointLiteLA", "CUDAGraphJointLiteLA", "optimized_joint_litela", "GroupedFull64QOutLiteLA",
           "linear_attention", "default_splits", "attn_matmul", "check_status"]
