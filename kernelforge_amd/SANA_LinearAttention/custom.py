"""SANA ReLU linear attention on gfx950 behind the reference factory API.

``qkv_attn_matmul(batch, heads, dim, seq_len, eps, dtype, output_dtype,
reduce_splits)`` returns ``run(qkv[B, N, 3, H*D]) -> out[B, N, H*D]`` like the
TileLang factory it replaces (SANA_LinearAttention/custom.py:340-388), with
the arithmetic of ``LiteLA.attn_matmul`` (SANA_LinearAttention/original.py:
99-117) in fp32: ``out = S relu(q) / (z . relu(q) + eps)`` with
``S = v^T relu(k)`` and ``z = sum relu(k)`` per (batch, head).

The HIP kernel (kernelforge_amd/csrc/linear_attn.hip) builds per-split
states on MFMA, lets the split workgroups of each (batch, head pair) meet at
a counter, sums their partials in a fixed order (deterministic) and
contracts the state with relu(q) on MFMA, all in one launch.  The counters
and partials live in a workspace kept per (device, stream): allocated zeroed
once, grown when a call needs more, and left with zero counters by every
call.
"""

from __future__ import annotations

import threading

import torch

from .. import _lib

THREADS = 128  # the reference's dim bound: 0 < dim <= 128 and 128 % dim == 0
DTYPES = {"float16": torch.float16, "bfloat16": torch.bfloat16, "float": torch.float32,
          "float32": torch.float32}
OUTPUT_DTYPES = ("float", "float16", "bfloat16")


def default_splits(batch: int, heads: int, dim: int, seq_len: int) -> int:
    """Sequence split count of the state producer for this shape."""
    return int(_lib.load().kf_linattn_default_splits(batch, heads, dim, seq_len))


_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}


def _workspace(device: torch.device, nbytes: int) -> torch.Tensor:
    """The zero-initialised workspace of the current stream on `device`, at
    least `nbytes` long (its control words are zero between calls)."""
    stream = torch.cuda.current_stream(device)
    key = (device.index if device.index is not None else torch.cuda.current_device(), stream.cuda_stream)
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is None or ws.numel() < nbytes:
            ws = torch.zeros(max(nbytes, 1 << 20), device=device, dtype=torch.uint8)
            _workspaces[key] = ws
    return ws


def linear_attention(qkv: torch.Tensor, heads: int, dim: int, eps: float = 1e-15,
                     output_dtype: torch.dtype = torch.float32, splits: int | None = None) -> torch.Tensor:
    """Shape-generic call: packed ``qkv[B, N, 3, heads*dim]`` -> ``out[B, N, heads*dim]``."""
    if qkv.dim() != 4 or qkv.shape[2] != 3 or qkv.shape[3] != heads * dim:
        raise ValueError(f"qkv must have shape [B, N, 3, {heads * dim}], got {tuple(qkv.shape)}")
    if qkv.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("qkv must be float16, bfloat16 or float32")
    _lib.require_gpu(qkv)
    lib = _lib.load()
    B, N = qkv.shape[0], qkv.shape[1]
    qkv = qkv.contiguous()
    out = torch.empty((B, N, heads * dim), device=qkv.device, dtype=output_dtype)
    if out.numel() == 0:
        return out
    if splits is None:
        splits = int(lib.kf_linattn_default_splits(B, heads, dim, N))
    ws_bytes = int(lib.kf_linattn_workspace_bytes(B, heads, dim, splits))
    ws = _workspace(qkv.device, ws_bytes)
    rc = lib.kf_linattn_fwd(_lib.ptr(qkv), _lib.ptr(out), _lib.ptr(ws), ws.numel(), B, N, heads, dim,
                            splits, float(eps), _lib.kf_dtype(qkv.dtype), _lib.kf_dtype(output_dtype),
                            _lib.stream_of(qkv))
    _lib.check(rc, "kf_linattn_fwd")
    return out


def qkv_attn_matmul(batch: int, heads: int, dim: int, seq_len: int, eps: float = 1e-15,
                    dtype: str = "bfloat16", output_dtype: str = "float", reduce_splits: bool = True):
    """Return ``run(qkv) -> out`` for one shape (SANA_LinearAttention/custom.py:340-388).

    ``reduce_splits`` selected the reference's 3-kernel or 2-kernel schedule;
    both compute the same values.  This build always combines the split
    partials inside its one fused launch, in a fixed order, so the flag is
    accepted for API compatibility only.
    """
    if dim <= 0 or dim > THREADS or THREADS % dim != 0:
        raise ValueError(f"dim must divide {THREADS} and be at most {THREADS}")
    if output_dtype not in OUTPUT_DTYPES:
        raise ValueError("output_dtype must be float, float16, or bfloat16")
    if dtype not in DTYPES:
        raise ValueError(f"dtype must be one of {sorted(DTYPES)}")
    in_dtype, out_dtype = DTYPES[dtype], DTYPES[output_dtype]
    expect = (batch, seq_len, 3, heads * dim)

    def run(qkv: torch.Tensor) -> torch.Tensor:
        if tuple(qkv.shape) != expect or qkv.dtype != in_dtype:
            raise ValueError(f"qkv must be {in_dtype} of shape {expect}, got {qkv.dtype} {tuple(qkv.shape)}")
        return linear_attention(qkv, heads, dim, eps, out_dtype)

    return run
