"""ctypes binding of the kernelforge_amd C ABI (include/kernelforge_amd.h).

torch is imported before the shared library is opened, so the library binds
to the HIP runtime torch already loaded (both carry the SONAME
libamdhip64.so.7) and the stream handles torch hands out are valid in it.
The library must have been built (``python -m kernelforge_amd.build``); there
is no fallback implementation: a missing library raises immediately.
"""

from __future__ import annotations

import ctypes
import threading
from pathlib import Path

import torch

LIB_PATH = Path(__file__).resolve().parent / "libkernelforge_amd.so"
ABI_VERSION = 1

KF_F32, KF_F16, KF_BF16 = 0, 1, 2
KF_WEIGHT_NK, KF_WEIGHT_KN = 0, 1
TORCH_TO_KF = {torch.float32: KF_F32, torch.float16: KF_F16, torch.bfloat16: KF_BF16}

_c_void_p = ctypes.c_void_p
_i64 = ctypes.c_int64
_int = ctypes.c_int
_f32 = ctypes.c_float

# name -> (restype, argtypes); must list every function of include/kernelforge_amd.h.
SIGNATURES = {
    "kf_abi_version": (_int, []),
    "kf_status_string": (ctypes.c_char_p, [_int]),
    "kf_last_error": (ctypes.c_char_p, []),
    "kf_rmsnorm_fwd": (_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32, _int, _c_void_p]),
    "kf_rmsnorm_fwd_strided": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _f32, _int, _c_void_p]),
    "kf_rmsnorm_noweight_f32": (_int, [_c_void_p, _c_void_p, _i64, _i64, _f32, _c_void_p]),
    "kf_rmsnorm_fwd_mixed": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _f32, _int, _int, _int, _c_void_p]),
    "kf_rmsnorm_bwd_workspace_bytes": (_i64, [_i64, _i64]),
    "kf_rmsnorm_bwd": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _f32,
               _int, _int, _c_void_p]),
    "kf_linattn_default_splits": (_i64, [_i64, _i64, _i64, _i64]),
    "kf_linattn_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "kf_linattn_workspace_init": (_int, [_c_void_p, _i64, _c_void_p]),
    "kf_linattn_fwd": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int,
         _c_void_p],
    ),
    "kf_linattn_attn_matmul": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _c_void_p],
    ),
    "kf_linattn_check": (_int, [_c_void_p, _i64, _c_void_p]),
    "kf_linattn_noalloc_max_bytes": (_i64, []),
    "kf_linattn_fwd_noalloc": (
        _int, [_c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _c_void_p]),
    "kf_linattn_noalloc_check": (_int, [_c_void_p]),
    "kf_proj_gemm": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _int, _int, _c_void_p]),
    "kf_litela_fused_workspace_bytes": (_i64, [_i64, _i64, _i64]),
    "kf_litela_fused_attn": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _f32, _int,
               _c_void_p]),
    "kf_rope_packed": (_int, [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _int, _c_void_p]),
    "kf_fa_fwd": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _c_void_p],
    ),
    "kf_fa_jvp": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p,
         _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _c_void_p],
    ),
    "kf_fa_fwd_jvp": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p,
         _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _c_void_p],
    ),
    "kf_fa_bwd_workspace_bytes": (_i64, [_i64, _i64, _i64, _i64]),
    "kf_fa_bwd": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _c_void_p],
    ),
}

# Measurement kernels (kernelforge_amd/csrc/measure.hip: bench.py's copy and
# MFMA ceilings) and test entry points (a public entry point plus one per-call
# argument that forces a kernel choice or a limit; no global state): exported
# by the library, not part of the public header.
MEASURE_SIGNATURES = {
    "kfm_copy": (_int, [_c_void_p, _c_void_p, _i64, _int, _int, _c_void_p]),
    "kfm_copy_ex": (_int, [_c_void_p, _c_void_p, _i64, _int, _int, _int, _int, _c_void_p]),
    "kfm_mfma_bf16": (_int, [_c_void_p, _i64, _int, _c_void_p]),
    "kfm_litela_fused_attn_heads": (
        _int, [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _f32, _int,
               _int, _c_void_p]),
    "kfm_linattn_fwd_spin": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _i64,
         _c_void_p],
    ),
    "kfm_linattn_split_plan": (_int, [_i64, _i64, _i64, _i64, ctypes.POINTER(_i64)]),
    "kfm_fa_bwd_blocks": (
        _int,
        [_c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p, _c_void_p,
         _c_void_p, _c_void_p, _c_void_p, _c_void_p, _i64,
         _i64, _i64, _i64, _i64, _i64, _i64, _f32, _int, _int, _int, _c_void_p],
    ),
}

# Hardware probes (kernelforge_amd/csrc/probes/), in their own library.
PROBES_PATH = Path(__file__).resolve().parent / "libkernelforge_amd_probes.so"
PROBE_SIGNATURES = {
    "kfm_coissue": (_int, [_c_void_p, _c_void_p, _i64, _int, _int, _int, _int, _c_void_p]),
    "kfm_lds_rate": (_int, [_c_void_p, _c_void_p, _i64, _int, _int, _int, _c_void_p]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None
_probes: ctypes.CDLL | None = None


def load() -> ctypes.CDLL:
    """Open the shared library once and attach the ctypes signatures."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not LIB_PATH.exists():
                raise RuntimeError(
                    f"kernelforge_amd native library missing at {LIB_PATH}; "
                    "build it with `python -m kernelforge_amd.build`"
                )
            lib = ctypes.CDLL(str(LIB_PATH))
            for name, (res, args) in {**SIGNATURES, **MEASURE_SIGNATURES}.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            version = lib.kf_abi_version()
            if version != ABI_VERSION:
                raise RuntimeError(f"kernelforge_amd ABI mismatch: library {version}, python {ABI_VERSION}")
            _lib = lib
    return _lib


def load_probes() -> ctypes.CDLL:
    """Open the hardware-probe library (measurement only; bench.py --only)."""
    global _probes
    load()
    with _lock:
        if _probes is None:
            if not PROBES_PATH.exists():
                raise RuntimeError(f"probe library missing at {PROBES_PATH}; build with `python -m kernelforge_amd.build`")
            lib = ctypes.CDLL(str(PROBES_PATH))
            for name, (res, args) in PROBE_SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _probes = lib
    return _probes


def check(rc: int, what: str) -> None:
    """Raise RuntimeError carrying the library's message when rc != KF_OK."""
    if rc != 0:
        lib = load()
        status = lib.kf_status_string(rc).decode()
        msg = lib.kf_last_error().decode()
        raise RuntimeError(f"{what} failed with {status}: {msg}")


def stream_of(t: torch.Tensor) -> ctypes.c_void_p:
    """hipStream_t of torch's current stream on t's device."""
    return ctypes.c_void_p(torch.cuda.current_stream(t.device).cuda_stream)


def ptr(t: torch.Tensor | None) -> ctypes.c_void_p:
    return ctypes.c_void_p(0 if t is None else t.data_ptr())


def kf_dtype(dtype: torch.dtype) -> int:
    try:
        return TORCH_TO_KF[dtype]
    except KeyError:
        raise ValueError(f"unsupported dtype {dtype}") from None


def require_gpu(*tensors: torch.Tensor) -> None:
    """The kernels run on HIP devices only; CPU tensors are rejected, never computed."""
    for t in tensors:
        if t is not None and not t.is_cuda:
            raise ValueError("kernelforge_amd kernels require tensors on a HIP (cuda) device")
