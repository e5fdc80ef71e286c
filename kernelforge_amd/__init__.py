"""kernelforge_amd: KernelForge's three operator hot paths as gfx950 HIP kernels.

Sub-packages mirror the reference packages' public APIs:

- ``kernelforge_amd.rmsnorm``              (rmsnorm/__init__.py)
- ``kernelforge_amd.SANA_LinearAttention`` (SANA_LinearAttention/__init__.py)
- ``kernelforge_amd.flash_attention_jvp``  (flash_attention_jvp/__init__.py)

All compute runs in ``libkernelforge_amd.so`` (C ABI in
``include/kernelforge_amd.h``), built by ``kernelforge_amd.build``.
"""

from . import _lib  # noqa: F401

__all__ = ["_lib"]
