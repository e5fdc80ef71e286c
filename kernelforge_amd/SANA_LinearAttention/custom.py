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

``attn_matmul(q, k, v, eps)`` is ``LiteLA.attn_matmul`` itself (original.py:
99-117) on the same kernel: q ``[B, h, d, N]``, k ``[B, h, N, d]``, v ``[B, h,
d, N]`` -> fp32 ``[B, h, d, N]``.  When the three are the views that
``LiteLA.forward`` makes of one packed ``[B, N, 3, C]`` buffer (original.py:
122-134; also the reference's harness, test.py:53-57) the kernel reads that
buffer in place; other tensors are packed once.

The split workgroups of a group wait for each other with a bounded poll;
only other work holding the GPU's slots for about a second can make them
give up, and then they write NaN.  ``linear_attention(..., check=True)`` and
``check_status()`` read that condition back (they synchronise the stream).
"""

from __future__ import annotations

import ctypes
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


def _check_workspace(ws: torch.Tensor, stream) -> None:
    rc = _lib.load().kf_linattn_check(_lib.ptr(ws), ws.numel(), stream)
    _lib.check(rc, "kf_linattn_check")


def check_status(device: torch.device | int | None = None) -> None:
    """Raise RuntimeError if a linear-attention launch on ``device`` since the
    last check gave up waiting for its split workgroups (its outputs are NaN).

    Synchronises each stream that owns a workspace on the device; not for use
    under graph capture.  Clears the condition it reports.
    """
    dev = torch.device("cuda", device) if isinstance(device, int) else torch.device(device or "cuda")
    index = dev.index if dev.index is not None else torch.cuda.current_device()
    with _ws_lock:
        items = [(key, ws) for key, ws in _workspaces.items() if key[0] == index]
    for (_, stream_handle), ws in items:
        _check_workspace(ws, ctypes.c_void_p(stream_handle))


def _launch(kind: str, qkv: torch.Tensor, out: torch.Tensor, B: int, N: int, heads: int, dim: int, eps: float,
            splits: int | None, check: bool) -> None:
    lib = _lib.load()
    if splits is None:
        splits = int(lib.kf_linattn_default_splits(B, heads, dim, N))
    if splits < 1:
        raise ValueError(f"splits must be positive, got {splits}")
    # The library runs at most one split per 32-token tile (its smallest split
    # unit), so a larger request needs no larger workspace.
    ws_splits = min(splits, max(1, -(-N // 32)))
    ws_bytes = int(lib.kf_linattn_workspace_bytes(B, heads, dim, ws_splits))
    ws = _workspace(qkv.device, ws_bytes)
    stream = _lib.stream_of(qkv)
    if kind == "fwd":
        rc = lib.kf_linattn_fwd(_lib.ptr(qkv), _lib.ptr(out), _lib.ptr(ws), ws.numel(), B, N, heads, dim,
                                splits, float(eps), _lib.kf_dtype(qkv.dtype), _lib.kf_dtype(out.dtype), stream)
    else:
        rc = lib.kf_linattn_attn_matmul(_lib.ptr(qkv), _lib.ptr(out), _lib.ptr(ws), ws.numel(), B, N, heads, dim,
                                        splits, float(eps), _lib.kf_dtype(qkv.dtype), stream)
    _lib.check(rc, f"kf_linattn_{kind}")
    if check:
        _check_workspace(ws, stream)


def linear_attention(qkv: torch.Tensor, heads: int, dim: int, eps: float = 1e-15,
                     output_dtype: torch.dtype = torch.float32, splits: int | None = None,
                     check: bool = False) -> torch.Tensor:
    """Shape-generic call: packed ``qkv[B, N, 3, heads*dim]`` -> ``out[B, N, heads*dim]``.

    ``splits`` bounds the sequence splits (the library may run fewer: see
    kf_linattn_fwd); ``check=True`` synchronises and raises if the launch
    reported an incomplete result.
    """
    if qkv.dim() != 4 or qkv.shape[2] != 3 or qkv.shape[3] != heads * dim:
        raise ValueError(f"qkv must have shape [B, N, 3, {heads * dim}], got {tuple(qkv.shape)}")
    if qkv.dtype not in (torch.float16, torch.bfloat16, torch.float32):
        raise ValueError("qkv must be float16, bfloat16 or float32")
    _lib.require_gpu(qkv)
    B, N = qkv.shape[0], qkv.shape[1]
    qkv = qkv.contiguous()
    out = torch.empty((B, N, heads * dim), device=qkv.device, dtype=output_dtype)
    if out.numel() == 0:
        return out
    _launch("fwd", qkv, out, B, N, heads, dim, eps, splits, check)
    return out


def _same_strides(t: torch.Tensor, strides: tuple[int, ...]) -> bool:
    """Strides equal where they matter (dimensions of size 1 may carry any stride)."""
    return all(n == 1 or a == b for n, a, b in zip(t.shape, t.stride(), strides))


def packed_source(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor) -> torch.Tensor | None:
    """The packed ``qkv[B, N, 3, C]`` that q ``[B, h, d, N]``, k ``[B, h, N, d]``
    and v ``[B, h, d, N]`` are views of, as ``LiteLA.forward`` makes them
    (original.py:122-134), or None when they are not such views."""
    B, h, d, N = q.shape
    C = h * d
    if k.shape != (B, h, N, d) or v.shape != (B, h, d, N):
        return None
    if k.dtype != q.dtype or v.dtype != q.dtype or k.device != q.device or v.device != q.device:
        return None
    qv_strides = (N * 3 * C, d, 1, 3 * C)
    if not (_same_strides(q, qv_strides) and _same_strides(v, qv_strides)
            and _same_strides(k, (N * 3 * C, d, 3 * C, 1))):
        return None
    es = q.element_size()
    if k.data_ptr() != q.data_ptr() + C * es or v.data_ptr() != q.data_ptr() + 2 * C * es:
        return None
    if q.untyped_storage().data_ptr() != k.untyped_storage().data_ptr() or \
            q.untyped_storage().data_ptr() != v.untyped_storage().data_ptr():
        return None
    return q.as_strided((B, N, 3, C), (N * 3 * C, 3 * C, C, 1), q.storage_offset())


def attn_matmul(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, eps: float = 1e-15,
                splits: int | None = None, check: bool = False) -> torch.Tensor:
    """``LiteLA.attn_matmul`` (SANA_LinearAttention/original.py:99-117) on the HIP kernel.

    q ``[B, h, d, N]``, k ``[B, h, N, d]`` (already transposed, as forward
    passes it), v ``[B, h, d, N]`` -> fp32 ``[B, h, d, N]`` (contiguous), with
    ReLU on q and k, the ones-row denominator and eps, in fp32 arithmetic (the
    reference's ``fp32_attention`` semantics).  Views of one packed buffer are
    read in place; other inputs are packed once on the GPU.
    """
    if q.dim() != 4 or k.dim() != 4 or v.dim() != 4:
        raise ValueError("q, k, v must be [B, h, d, N], [B, h, N, d], [B, h, d, N]")
    B, h, d, N = q.shape
    if k.shape != (B, h, N, d) or v.shape != (B, h, d, N):
        raise ValueError(f"k must be [B, h, N, d] and v [B, h, d, N] for q {tuple(q.shape)}, "
                         f"got {tuple(k.shape)} and {tuple(v.shape)}")
    if q.dtype not in (torch.float16, torch.bfloat16, torch.float32) or k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share one dtype: float16, bfloat16 or float32")
    if d <= 0 or d > THREADS or THREADS % d:
        raise ValueError(f"head dim {d} must divide {THREADS}")
    _lib.require_gpu(q, k, v)
    out = torch.empty((B, h, d, N), device=q.device, dtype=torch.float32)
    if out.numel() == 0:
        return out
    qkv = packed_source(q, k, v)
    if qkv is None:
        C = h * d
        qkv = torch.empty((B, N, 3, C), device=q.device, dtype=q.dtype)
        qkv[:, :, 0].view(B, N, h, d).copy_(q.permute(0, 3, 1, 2))
        qkv[:, :, 1].view(B, N, h, d).copy_(k.permute(0, 2, 1, 3))
        qkv[:, :, 2].view(B, N, h, d).copy_(v.permute(0, 3, 1, 2))
    _launch("attn_matmul", qkv, out, B, N, h, d, eps, splits, check)
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
