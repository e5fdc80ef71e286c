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
