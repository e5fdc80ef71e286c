"""RMSNorm drop-in (mirrors rmsnorm/__init__.py:1-4 of KernelForge)."""

from .custom import RMSNorm, original_tilelang_rms_norm, rms_norm, rms_norm_module_forward, rms_norm_tensor
from .custom import rms_norm as custom_rms_norm

__all__ = ["RMSNorm", "custom_rms_norm", "original_tilelang_rms_norm", "rms_norm", "rms_norm_module_forward",
           "rms_norm_tensor"]
