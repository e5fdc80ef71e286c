"""SANA ReLU linear-attention CPU oracle -- TEST INFRASTRUCTURE ONLY.

Restates ``LiteLA.attn_matmul`` (SANA_LinearAttention/original.py:99-117) on
the packed-QKV layout of ``LiteLA.forward`` (:124-134) and of the reference
test (SANA_LinearAttention/test.py:53-57, 74-75).
"""

from __future__ import annotations

import torch

PAD_VAL = 1  # SANA_LinearAttention/original.py:68


def unpack_qkv(qkv: torch.Tensor, heads: int, dim: int):
    """Packed ``[B, N, 3, H*D]`` -> q ``[B,H,D,N]``, k ``[B,H,N,D]``, v ``[B,H,D,N]``.

    SANA_LinearAttention/test.py:53-57 / original.py:124-134: channel
    ``h*D + r`` of part j (0=q, 1=k, 2=v) is head h, feature r.
    """
    B, N, three, C = qkv.shape
    assert three == 3 and C == heads * dim
    q, k, v = qkv.unbind(2)
    q = q.transpose(-1, -2).reshape(B, heads, dim, N)
    k = k.transpose(-1, -2).reshape(B, heads, dim, N).transpose(-1, -2)
    v = v.transpose(-1, -2).reshape(B, heads, dim, N)
    return q, k, v


def attn_matmul(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, eps: float = 1e-15,
                fp32_attention: bool = True) -> torch.Tensor:
    """``LiteLA.attn_matmul`` (SANA_LinearAttention/original.py:100-117).

    q ``[B,h,d,N]``, k ``[B,h,N,d]``, v ``[B,h,d,N]`` -> fp32 ``[B,h,d,N]``.
    ``fp32_attention=True`` upcasts after the ReLU (:105-107), the north-star
    fp32 reference; ``False`` keeps the eager matmuls in the input dtype.
    """
    q = torch.relu(q)
    k = torch.relu(k)
    if fp32_attention:
        q, k, v = q.float(), k.float(), v.float()
    v = torch.nn.functional.pad(v, (0, 0, 0, 1), mode="constant", value=PAD_VAL)
    vk = torch.matmul(v, k)
    out = torch.matmul(vk, q)
    if out.dtype in (torch.float16, torch.bfloat16):
        out = out.float()
    return out[:, :, :-1] / (out[:, :, -1:] + eps)


def linear_attention(qkv: torch.Tensor, heads: int, dim: int, eps: float = 1e-15,
                     fp32_attention: bool = True) -> torch.Tensor:
    """Packed ``[B,N,3,H*D]`` -> fp32 ``[B,N,H*D]`` (SANA_LinearAttention/test.py:72-75)."""
    qkv = qkv.detach().cpu()
    B, N, _, C = qkv.shape
    q, k, v = unpack_qkv(qkv, heads, dim)
    out = attn_matmul(q, k, v, eps, fp32_attention)
    return out.reshape(B, C, N).permute(0, 2, 1).contiguous()


def linear_attention_split(qkv: torch.Tensor, heads: int, dim: int, splits: int,
                           eps: float = 1e-15) -> torch.Tensor:
    """fp64 split-state form: per-split partial ``[v;1] relu(k)`` summed in split order.

    This is the decomposition the HIP kernel uses (state partials per sequence
    split, reduced in a fixed order; SANA_LinearAttention/custom.py:88-165,
    238-337).  In fp64 it must equal ``linear_attention`` for every split count.
    """
    qkv = qkv.detach().cpu().double()
    B, N, _, C = qkv.shape
    q, k, v = unpack_qkv(qkv, heads, dim)
    q, k = torch.relu(q), torch.relu(k)
    v = torch.nn.functional.pad(v, (0, 0, 0, 1), value=PAD_VAL)
    split_len = -(-N // splits)
    state = torch.zeros(B, heads, dim + 1, dim, dtype=torch.float64)
    for s in range(splits):
        lo, hi = s * split_len, min(N, (s + 1) * split_len)
        if lo < hi:
            state = state + v[..., lo:hi] @ k[:, :, lo:hi]
    out = state @ q
    out = out[:, :, :-1] / (out[:, :, -1:] + eps)
    return out.reshape(B, C, N).permute(0, 2, 1).contiguous()


def apply_rotary_emb(x: torch.Tensor, freqs_cis, use_real: bool = True, use_real_unbind_dim: int = -1):
    """``apply_rotary_emb`` (SANA_LinearAttention/original.py:14-58), written
    as explicit complex-pair arithmetic.

    ``use_real``: ``freqs_cis = (cos, sin)``, each ``[S, D]``.  Channels
    (2i, 2i+1) form the complex value ``a + ib``; with ``use_real_unbind_dim
    = -2`` (SANA) x is ``[B, H, D, S]`` and the pairs run along dim -2, with -1
    x is ``[B, H, S, D]`` and they run along the last dim.  Per pair
    ``a' = a cos_{2i} - b sin_{2i}`` and ``b' = b cos_{2i+1} + a sin_{2i+1}``,
    each product and the sum rounded in fp32, the result rounded to x's
    dtype.  Otherwise ``freqs_cis`` is a complex ``[B or 1, S, D/2]`` tensor
    that multiplies the pairs of a ``[B, S, H, D]`` x.  fp64 inputs stay in fp64
    (the closed-form checks need exact arithmetic; the reference would round
    them to fp32).
    """
    ct = torch.float64 if x.dtype == torch.float64 else torch.float32
    if not use_real:
        xf = x.to(ct)
        z = torch.complex(xf[..., 0::2], xf[..., 1::2]) * freqs_cis.unsqueeze(2)
        return torch.stack((z.real, z.imag), dim=-1).flatten(-2).to(x.dtype)
    cos, sin = (t.to(x.device).to(ct) for t in freqs_cis)
    if use_real_unbind_dim == -2:
        cos, sin = cos.T, sin.T                       # [D, S], broadcast over [B, H]
        a, b = x[..., 0::2, :].to(ct), x[..., 1::2, :].to(ct)
        c0, c1, s0, s1 = cos[0::2], cos[1::2], sin[0::2], sin[1::2]
        dim = -2
    elif use_real_unbind_dim == -1:
        a, b = x[..., 0::2].to(ct), x[..., 1::2].to(ct)
        c0, c1, s0, s1 = cos[..., 0::2], cos[..., 1::2], sin[..., 0::2], sin[..., 1::2]
        dim = -1
    else:
        raise ValueError(f"`use_real_unbind_dim={use_real_unbind_dim}` but should be -1 or -2.")
    re = a * c0 + (-b) * s0
    im = b * c1 + a * s1
    return _interleave(re, im, dim).to(x.dtype)


def _interleave(re: torch.Tensor, im: torch.Tensor, dim: int) -> torch.Tensor:
    """Channels 2i <- re[i], 2i+1 <- im[i] along ``dim`` (-1 or -2)."""
    if dim == -1:
        return torch.stack((re, im), dim=-1).flatten(-2)
    return torch.stack((re, im), dim=-2).flatten(-3, -2)


def rope_packed(qkv: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor, heads: int) -> torch.Tensor:
    """q and k of a packed ``[B, N, 3, C]`` qkv rotated as LiteLA.forward does
    (SANA_LinearAttention/original.py:128-138): ``[B, h, D, N]`` views of q and
    k through ``apply_rotary_emb(.., use_real_unbind_dim=-2)``; v unchanged."""
    B, N, _, C = qkv.shape
    D = C // heads
    parts = []
    for j in range(2):
        x = qkv[:, :, j].transpose(-1, -2).reshape(B, heads, D, N)
        y = apply_rotary_emb(x, (cos, sin), use_real_unbind_dim=-2)
        parts.append(y.reshape(B, C, N).transpose(-1, -2))
    return torch.stack((parts[0], parts[1], qkv[:, :, 2]), dim=2)


def lite_la_forward(x: torch.Tensor, qkv_weight: torch.Tensor, qkv_bias, proj_weight: torch.Tensor,
                    proj_bias, heads: int, eps: float = 1e-15, q_norm_weight=None, k_norm_weight=None,
                    norm_eps: float = 1e-5, qkv_dtype=None, rotary_emb=None) -> torch.Tensor:
    """``LiteLA.forward`` (SANA_LinearAttention/original.py:119-145) on the CPU.

    ``qkv = x W^T (+ b)`` reshaped to ``[B, N, 3, C]`` (:122-123); the optional
    q/k RMSNorm over C (:91-94, 129-130, with the rounding points of
    ``oracle.rmsnorm.rmsnorm``); the fp32 linear attention of ``attn_matmul``
    (:99-117) on the packed layout (:132-134, 136); ``.to(dtype)`` and the
    output projection (:138-143).  ``qkv_dtype`` rounds the projected qkv the
    way a GEMM with a 16-bit output does (fp32 accumulation, one rounding).
    ``rotary_emb = (cos, sin)`` rotates q and k after the norm (:136-138).
    """
    from .rmsnorm import rmsnorm

    x = x.detach().cpu()
    dtype = x.dtype
    B, N, C = x.shape
    f = lambda t: None if t is None else t.detach().cpu().float()
    qkv = torch.nn.functional.linear(x.float(), f(qkv_weight), f(qkv_bias))
    qkv = qkv.to(qkv_dtype or dtype).reshape(B, N, 3, C)
    if q_norm_weight is not None:
        q = rmsnorm(qkv[:, :, 0], q_norm_weight.detach().cpu().to(qkv.dtype), norm_eps)
        k = rmsnorm(qkv[:, :, 1], k_norm_weight.detach().cpu().to(qkv.dtype), norm_eps)
        qkv = torch.stack((q, k, qkv[:, :, 2]), dim=2)
    if rotary_emb is not None:
        cos, sin = (t.detach().cpu() for t in rotary_emb)
        qkv = rope_packed(qkv, cos, sin, heads)
    out = linear_attention(qkv, heads, C // heads, eps).to(dtype)
    return torch.nn.functional.linear(out.float(), f(proj_weight), f(proj_bias))
