"""FlashAttention forward and forward-mode AD (JVP) on gfx950.

Mirrors the public API of flash_attention_jvp/custom.py (KernelForge):

- ``flash_attention(q, k, v, *, softmax_scale, causal, return_lse)``   (:279-291)
- ``flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, ...)``          (:188-223)
- ``get_jvp_config(q, k, v, *, softmax_scale, causal)``                (:131-134)
- ``FlashAttentionFunction`` with ``setup_context``/``jvp`` so that
  ``torch.func.jvp`` and ``torch.autograd.forward_ad`` reach the JVP kernel
  (:226-276).

and adds the fused single-pass operator the reference describes but does not
implement (flash-attention-jvp-derivation.md:388-558):

- ``flash_attention_fwd_jvp(q, k, v, tq, tk, tv, *, softmax_scale, causal)``
  returning ``(out, lse, tangent)`` from one scan over the K/V tiles.

Every operator is a ``torch.library.custom_op`` with a fake implementation,
so torch.func transforms unwrap their tensors before the C ABI sees raw
pointers and torch.compile can trace them.  The standalone JVP is the
reference's ``kernelforge::flash_attention_jvp`` (same schema,
custom.py:137-157); the others live in ``kernelforge_amd::``.  Layouts
are ``[B, S, H, D]``; LSE is fp32 ``[B, Hq, Nq]`` in natural log.  Rows with no
valid key (bottom-right causal masks with Nq > Nk) give out = 0, tangent = 0
and LSE = +inf, the FlashAttention convention.

The backward pass (the reference delegates it to flash-attn's
``_flash_attn_backward``, custom.py:252-267) runs on the gfx950 backward
kernels (``kf_fa_bwd``): dQ per query tile, dK/dV per key tile with the query
heads of a GQA group summed in a fixed order, so gradients are deterministic.
"""

from __future__ import annotations

import math

import torch
from torch.autograd.function import once_differentiable

from .. import _lib

# Schedule values the reference accepts for explicit tile/pipeline arguments
# (flash_attention_jvp/custom.py:214-217), plus the gfx950 JVP kernel's own
# (_schedule below), so that ``flash_attention_jvp(..., **get_jvp_config(...))``
# is accepted too.
_ALLOWED = dict(block_m=(16, 32, 64, 128), block_n=(32, 64, 128), threads=(128, 256, 512),
                num_stages=(1, 2, 3))


def _schedule(head_dim: int) -> dict:
    """Tile of the gfx950 JVP kernel for a head dim.  Head dims up to 128 run
    128 query rows per workgroup (8 wavefronts x 16 rows, 512 threads) over
    64-key tiles; 136-256 run 64 rows (4 wavefronts, 256 threads) over 32-key
    tiles.  The K/V tiles are double-buffered in LDS in both (2 stages)."""
    if head_dim > 128:
        return dict(block_m=64, block_n=32, threads=256, num_stages=2)
    return dict(block_m=128, block_n=64, threads=512, num_stages=2)


def _validate_inputs(q, k, v, softmax_scale):
    """Shape/dtype/scale checks with the reference's messages (custom.py:160-174)."""
    if any(x.ndim != 4 for x in (q, k, v)):
        raise ValueError("q, k, v must have shape [batch, sequence, heads, dim]")
    if q.dtype not in (torch.float16, torch.bfloat16):
        raise ValueError("FlashAttention JVP supports float16 and bfloat16")
    if any(x.device != q.device or x.dtype != q.dtype for x in (k, v)):
        raise ValueError("q, k, v must use the same CUDA device and dtype")
    b, nq, h, d = q.shape
    if min(b, nq, h, d, k.shape[1], k.shape[2]) <= 0:
        raise ValueError("batch, sequence lengths, heads, and head dimension must be positive")
    if k.shape != v.shape or k.shape[0] != b or k.shape[-1] != d:
        raise ValueError("k and v must match, with the same batch and head dimension as q")
    if h % k.shape[2] or d % 8 or d > 256:
        raise ValueError("query heads must be divisible by KV heads; dim must be a multiple of 8 <= 256")
    scale = d ** -0.5 if softmax_scale is None else float(softmax_scale)
    if not math.isfinite(scale) or scale <= 0:
        raise ValueError("softmax_scale must be finite and positive")
    if not q.is_cuda:
        raise ValueError("q, k, v must use the same CUDA device and dtype")
    return scale


def _prepare_tangent(tangent, primal, name):
    """``None`` stays ``None`` (the kernels treat it as zero, skipping its products)."""
    if tangent is None:
        return None
    if tangent.shape != primal.shape or tangent.device != primal.device or tangent.dtype != primal.dtype:
        raise ValueError(f"{name} must have the same shape, device, and dtype as its primal")
    return tangent.contiguous()


def _dims(q, k):
    return q.shape[0], q.shape[1], k.shape[1], q.shape[2], k.shape[2], q.shape[3]


def _check_cached(q, out, lse):
    """The cached forward results: out like q, LSE fp32 [B, Hq, Nq] (custom.py:204-207)."""
    if out.shape != q.shape or out.dtype != q.dtype or out.device != q.device:
        raise ValueError("out must have q's shape, device, and dtype")
    if lse.shape != (q.shape[0], q.shape[2], q.shape[1]) or lse.dtype != torch.float32 or lse.device != q.device:
        raise ValueError("lse must be float32 [B, Hq, Nq] on q's device")


# ---------------------------------------------------------------------------
# Opaque operators (C ABI launches on the current stream).
# ---------------------------------------------------------------------------
@torch.library.custom_op("kernelforge_amd::flash_attention_fwd", mutates_args=(), device_types="cuda")
def _fwd_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float,
            causal: bool) -> tuple[torch.Tensor, torch.Tensor]:
    B, Nq, Nk, Hq, Hkv, D = _dims(q, k)
    out = torch.empty_like(q)
    lse = torch.empty((B, Hq, Nq), device=q.device, dtype=torch.float32)
    rc = _lib.load().kf_fa_fwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse),
                               B, Nq, Nk, Hq, Hkv, D, scale, int(causal), _lib.kf_dtype(q.dtype),
                               _lib.stream_of(q))
    _lib.check(rc, "kf_fa_fwd")
    return out, lse


@_fwd_op.register_fake
def _fwd_fake(q, k, v, scale, causal):
    return torch.empty_like(q), q.new_empty((q.shape[0], q.shape[2], q.shape[1]), dtype=torch.float32)


@torch.library.custom_op("kernelforge::flash_attention_jvp", mutates_args=(), device_types="cuda")
def _launch_jvp(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tq: torch.Tensor, tk: torch.Tensor,
                tv: torch.Tensor, out: torch.Tensor, lse: torch.Tensor, scale: float, causal: bool,
                block_m: int, block_n: int, threads: int, num_stages: int) -> torch.Tensor:
    """The reference's registered operator (flash_attention_jvp/custom.py:137-152),
    same name and schema, on the gfx950 JVP kernel (kf_fa_jvp).  The schedule
    arguments are accepted for schema compatibility; the kernel runs its own
    tile for the head dim.  A tangent with no elements stands for a zero
    tangent, whose products the kernel skips (the reference passes explicit
    zeros, which give the same result).  Every argument is checked here, so a
    direct ``torch.ops.kernelforge.flash_attention_jvp`` call gets the same
    ValueErrors as the Python wrapper, never an out-of-bounds launch."""
    _validate_inputs(q, k, v, scale)
    _check_cached(q, out, lse)
    tq, tk, tv = (None if t.numel() == 0 else _prepare_tangent(t, p, n)
                  for t, p, n in zip((tq, tk, tv), (q, k, v), ("tq", "tk", "tv")))
    q, k, v, out, lse = (x.contiguous() for x in (q, k, v, out, lse))
    B, Nq, Nk, Hq, Hkv, D = _dims(q, k)
    tout = torch.empty_like(out)
    rc = _lib.load().kf_fa_jvp(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(tq), _lib.ptr(tk),
                               _lib.ptr(tv), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(tout),
                               B, Nq, Nk, Hq, Hkv, D, scale, int(causal), _lib.kf_dtype(q.dtype),
                               _lib.stream_of(q))
    _lib.check(rc, "kf_fa_jvp")
    return tout


@_launch_jvp.register_fake
def _launch_jvp_fake(q, k, v, tq, tk, tv, out, lse, scale, causal, block_m, block_n, threads, num_stages):
    return torch.empty_like(out)


@torch.library.custom_op("kernelforge_amd::flash_attention_fwd_jvp", mutates_args=(), device_types="cuda")
def _fwd_jvp_op(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, tq: torch.Tensor | None,
                tk: torch.Tensor | None, tv: torch.Tensor | None, scale: float,
                causal: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, Nq, Nk, Hq, Hkv, D = _dims(q, k)
    out = torch.empty_like(q)
    tout = torch.empty_like(q)
    lse = torch.empty((B, Hq, Nq), device=q.device, dtype=torch.float32)
    rc = _lib.load().kf_fa_fwd_jvp(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(tq), _lib.ptr(tk),
                                   _lib.ptr(tv), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(tout),
                                   B, Nq, Nk, Hq, Hkv, D, scale, int(causal), _lib.kf_dtype(q.dtype),
                                   _lib.stream_of(q))
    _lib.check(rc, "kf_fa_fwd_jvp")
    return out, lse, tout


@_fwd_jvp_op.register_fake
def _fwd_jvp_fake(q, k, v, tq, tk, tv, scale, causal):
    lse = q.new_empty((q.shape[0], q.shape[2], q.shape[1]), dtype=torch.float32)
    return torch.empty_like(q), lse, torch.empty_like(q)


@torch.library.custom_op("kernelforge_amd::flash_attention_bwd", mutates_args=(), device_types="cuda")
def _bwd_op(dout: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, out: torch.Tensor,
            lse: torch.Tensor, scale: float, causal: bool) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    B, Nq, Nk, Hq, Hkv, D = _dims(q, k)
    lib = _lib.load()
    dq, dk, dv = (torch.empty_like(x, memory_format=torch.contiguous_format) for x in (q, k, v))
    ws_bytes = lib.kf_fa_bwd_workspace_bytes(B, Nq, Hq, D)
    if ws_bytes < 0:
        raise ValueError("flash attention backward: unsupported shape")
    ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)
    rc = lib.kf_fa_bwd(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(dout),
                       _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), ws_bytes,
                       B, Nq, Nk, Hq, Hkv, D, scale, int(causal), _lib.kf_dtype(q.dtype), _lib.stream_of(q))
    _lib.check(rc, "kf_fa_bwd")
    return dq, dk, dv


@_bwd_op.register_fake
def _bwd_fake(dout, q, k, v, out, lse, scale, causal):
    return torch.empty_like(q), torch.empty_like(k), torch.empty_like(v)


def flash_attention_backward(dout, q, k, v, out, lse, *, softmax_scale=None, causal=False):
    """``(dq, dk, dv)`` for the output cotangent ``dout`` from the forward's ``out`` and ``lse``.

    The standalone form of ``FlashAttentionFunction.backward`` (the reference
    calls flash-attn's ``_flash_attn_backward`` there, custom.py:252-267):
    P is recomputed from the natural-log LSE, no forward is launched.
    """
    scale = _validate_inputs(q, k, v, softmax_scale)
    for name, t in (("dout", dout), ("out", out)):
        if t.shape != q.shape or t.dtype != q.dtype or t.device != q.device:
            raise ValueError(f"{name} must have q's shape, device, and dtype")
    if lse.shape != (q.shape[0], q.shape[2], q.shape[1]) or lse.dtype != torch.float32 or lse.device != q.device:
        raise ValueError("lse must be float32 [B, Hq, Nq] on q's device")
    q, k, v, dout, out, lse = (x.contiguous() for x in (q, k, v, dout, out, lse))
    return _bwd_op(dout, q, k, v, out, lse, scale, bool(causal))


# ---------------------------------------------------------------------------
# Public API.
# ---------------------------------------------------------------------------
def get_jvp_config(q, k, v, *, softmax_scale=None, causal=False):
    """Return the schedule of the gfx950 JVP kernel for these inputs without launching anything.

    Same keys as the reference (custom.py:123-134), which returns its
    H20-tuned TileLang defaults; here the values are the tile the gfx950
    kernel runs for the head dim (one schedule per head-dim class, the same
    for causal and non-causal masks and every key length).
    """
    _validate_inputs(q, k, v, softmax_scale)
    return _schedule(q.shape[-1])


@torch.no_grad()
def flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, *, softmax_scale=None, causal=False,
                        block_m=64, block_n=None, threads=None, num_stages=None):
    """Standalone JVP from cached forward results, without a forward launch (custom.py:188-223).

    q/tq: [B, Nq, Hq, D]; k/tk/v/tv: [B, Nk, Hkv, D]; out: [B, Nq, Hq, D];
    lse: fp32 [B, Hq, Nq] in natural log, from the same primals, scale and mask.
    A ``None`` tangent denotes zero.  The result has q's dtype and out's shape.
    ``out`` enters as in the reference, tO = P tv + H v - rowsum(H) out, on
    every 128-row tile where rowsum(H) cannot amplify out's 16-bit rounding
    past a small fraction of the tolerance; the kernel's second launch redoes
    the other tiles (strongly peaked softmaxes) with O recomputed in fp32 from
    the same probabilities, without reading ``out``.  Schedule arguments are validated against the reference's accepted values
    (and the gfx950 kernel's own, as ``get_jvp_config`` reports them) and
    otherwise do not change the computation: the kernel runs one tile per
    head-dim class.  The launch goes through the registered operator
    ``torch.ops.kernelforge.flash_attention_jvp`` (the reference's schema).
    """
    scale = _validate_inputs(q, k, v, softmax_scale)
    _check_cached(q, out, lse)
    sched = _schedule(q.shape[-1])
    for key, val in (("block_m", block_m), ("block_n", block_n), ("threads", threads), ("num_stages", num_stages)):
        if val is not None:
            sched[key] = val
    if any(sched[key] not in _ALLOWED[key] for key in _ALLOWED):
        raise ValueError("unsupported tile/pipeline configuration")
    q, k, v = (x.contiguous() for x in (q, k, v))
    tq, tk, tv = (_prepare_tangent(t, p, n) for t, p, n in zip((tq, tk, tv), (q, k, v), ("tq", "tk", "tv")))
    empty = q.new_empty(0)
    tq, tk, tv = (empty if t is None else t for t in (tq, tk, tv))
    return torch.ops.kernelforge.flash_attention_jvp(q, k, v, tq, tk, tv, out.contiguous(), lse.contiguous(),
                                                     scale, bool(causal), sched["block_m"], sched["block_n"],
                                                     sched["threads"], sched["num_stages"])


@torch.no_grad()
def flash_attention_fwd_jvp(q, k, v, tq, tk, tv, *, softmax_scale=None, causal=False):
    """Fused single pass: ``(out, lse, tangent)`` with one scan over the K/V tiles.

    Implements the online recurrences of flash-attention-jvp-derivation.md:
    388-558 (states m, l, U, r, G per query row).  ``None`` tangents are zero.
    """
    scale = _validate_inputs(q, k, v, softmax_scale)
    q, k, v = (x.contiguous() for x in (q, k, v))
    tq, tk, tv = (_prepare_tangent(t, p, n) for t, p, n in zip((tq, tk, tv), (q, k, v), ("tq", "tk", "tv")))
    return _fwd_jvp_op(q, k, v, tq, tk, tv, scale, bool(causal))


class FlashAttentionFunction(torch.autograd.Function):
    """Forward on the HIP kernel plus a HIP JVP rule, with torch.func support (custom.py:226-276)."""

    @staticmethod
    def forward(q, k, v, softmax_scale, causal):
        scale = _validate_inputs(q, k, v, softmax_scale)
        out, lse = _fwd_op(q, k, v, scale, bool(causal))
        # LSE is an auxiliary output so setup_context can save it without a
        # second forward (required by torch.func transforms).
        return out, lse

    @staticmethod
    def setup_context(ctx, inputs, output):
        q, k, v, scale, causal = inputs
        out, lse = output
        ctx.softmax_scale = q.shape[-1] ** -0.5 if scale is None else float(scale)
        ctx.causal = causal
        ctx.set_materialize_grads(False)
        ctx.mark_non_differentiable(lse)
        ctx.save_for_backward(q, k, v, out, lse)
        ctx.save_for_forward(q, k, v, out, lse)

    @staticmethod
    @once_differentiable
    def backward(ctx, dout, dlse):
        # LSE is non-differentiable: its cotangent is ignored, as in the reference.
        if dout is None:
            return (None,) * 5
        q, k, v, out, lse = ctx.saved_tensors
        dq, dk, dv = flash_attention_backward(dout, q, k, v, out, lse, softmax_scale=ctx.softmax_scale,
                                              causal=ctx.causal)
        return dq, dk, dv, None, None

    @staticmethod
    def jvp(ctx, tq, tk, tv, tscale, tcausal):
        q, k, v, out, lse = ctx.saved_tensors
        tangent = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse,
                                      softmax_scale=ctx.softmax_scale, causal=ctx.causal)
        return tangent, None


def flash_attention(q, k, v, *, softmax_scale=None, causal=False, return_lse=False):
    """Attention forward on the HIP kernel with a HIP forward-mode AD rule (custom.py:279-291).

    Returns out, or (out, lse) with ``return_lse=True``; LSE is a
    non-differentiable natural-log auxiliary output for standalone JVP calls.
    Supports torch.autograd (backward on the HIP backward kernels), torch.func.jvp
    and torch.autograd.forward_ad.  First order only.
    """
    _validate_inputs(q, k, v, softmax_scale)
    out, lse = FlashAttentionFunction.apply(q.contiguous(), k.contiguous(), v.contiguous(),
                                            softmax_scale, bool(causal))
    return (out, lse) if return_lse else out
