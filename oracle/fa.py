"""FlashAttention forward / JVP CPU oracle -- TEST INFRASTRUCTURE ONLY.

Restates flash_attention_jvp/original.py:6-65 (dense attention, its
torch.func.jvp, and the dense JVP from cached O/LSE) and the fused online
recurrence of flash_attention_jvp/flash-attention-jvp-derivation.md:388-558.
Layout ``[B, S, H, D]``; LSE ``[B, H, Nq]`` in natural log.
"""

from __future__ import annotations

import math

import torch


def _mask(nq: int, nk: int, device=None) -> torch.Tensor:
    """Bottom-right causal validity ``col <= row + nk - nq`` (original.py:20-23)."""
    rows = torch.arange(nq, device=device)[:, None]
    cols = torch.arange(nk, device=device)[None, :]
    return cols <= rows + nk - nq


def attention(q, k, v, *, softmax_scale=None, causal=False):
    """Dense softmax attention, GQA by repeat_interleave (original.py:6-30).

    Low-precision inputs use fp32 intermediates; fp64 stays fp64.  Fully
    masked rows produce zeros, as native FlashAttention does (:25-29).
    """
    dtype = torch.float64 if q.dtype == torch.float64 else torch.float32
    qh, kh, vh = (x.to(dtype).transpose(1, 2) for x in (q, k, v))
    groups = q.shape[2] // k.shape[2]
    if groups > 1:
        kh, vh = (x.repeat_interleave(groups, dim=1) for x in (kh, vh))
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    scores = (qh @ kh.transpose(-1, -2)) * scale
    if causal:
        valid = _mask(q.shape[1], k.shape[1], q.device)
        scores = scores.masked_fill(~valid, -torch.inf)
        scores = torch.where(valid.any(dim=-1, keepdim=True), scores, 0.0)
    probabilities = scores.softmax(dim=-1)
    if causal:
        probabilities = probabilities.masked_fill(~valid, 0.0)
    return (probabilities @ vh).transpose(1, 2).to(q.dtype)


def attention_jvp(q, k, v, tq, tk, tv, *, softmax_scale=None, causal=False):
    """``(out, tangent)`` = torch.func.jvp of ``attention`` (original.py:33-39)."""
    tangents = tuple(torch.zeros_like(p) if t is None else t for p, t in zip((q, k, v), (tq, tk, tv)))
    return torch.func.jvp(
        lambda q, k, v: attention(q, k, v, softmax_scale=softmax_scale, causal=causal),
        (q, k, v), tangents,
    )


def attention_lse(q, k, *, softmax_scale=None, causal=False):
    """Natural-log LSE ``[B, Hq, Nq]`` of the scaled scores; +inf for rows with no valid key.

    The +inf convention is FlashAttention's for empty causal rows
    (flash_attention_jvp/custom.py:70-71 relies on it).
    """
    dtype = torch.float64 if q.dtype == torch.float64 else torch.float32
    qh, kh = (x.to(dtype).transpose(1, 2) for x in (q, k))
    groups = q.shape[2] // k.shape[2]
    if groups > 1:
        kh = kh.repeat_interleave(groups, dim=1)
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    scores = (qh @ kh.transpose(-1, -2)) * scale
    if causal:
        valid = _mask(q.shape[1], k.shape[1], q.device)
        scores = scores.masked_fill(~valid, -torch.inf)
    lse = torch.logsumexp(scores, dim=-1)
    return torch.where(torch.isneginf(lse), torch.full_like(lse, math.inf), lse)


@torch.no_grad()
def attention_jvp_from_forward(q, k, v, tq, tk, tv, out, lse, *, softmax_scale=None, causal=False):
    """Dense JVP from cached O/LSE (original.py:42-65), fp32 intermediates."""
    primals = (q, k, v)
    tangents = tuple(torch.zeros_like(p) if t is None else t for p, t in zip(primals, (tq, tk, tv)))
    qh, kh, vh, tqh, tkh, tvh = (x.float().transpose(1, 2) for x in (*primals, *tangents))
    groups = q.shape[2] // k.shape[2]
    if groups > 1:
        kh, vh, tkh, tvh = (x.repeat_interleave(groups, dim=1) for x in (kh, vh, tkh, tvh))
    scale = q.shape[-1] ** -0.5 if softmax_scale is None else softmax_scale
    probabilities = ((qh @ kh.transpose(-1, -2)) * scale - lse.float()[..., None]).exp()
    if causal:
        valid = _mask(q.shape[1], k.shape[1], q.device)
        probabilities = probabilities.masked_fill(~valid, 0.0)
    tscores = (tqh @ kh.transpose(-1, -2) + qh @ tkh.transpose(-1, -2)) * scale
    weighted = probabilities * tscores
    result = probabilities @ tvh + weighted @ vh - weighted.sum(-1, keepdim=True) * out.float().transpose(1, 2)
    return result.transpose(1, 2).to(q.dtype)


@torch.no_grad()
def fused_forward_jvp_tiled(q, k, v, tq, tk, tv, *, softmax_scale=None, causal=False, block_n=64):
    """Single-pass online recurrence for (O, LSE, tO) in fp64.

    flash-attention-jvp-derivation.md:519-558 (pseudocode) with the guards of
    :541-553: states m, l, U, r, G per query row; alpha = exp(m - m_ref);
    E = exp(S - m_ref); H = E * tS; O = U/l; tO = G/l - (r/l) O;
    LSE = m + log l.  Rows with no valid key get O = tO = 0 and LSE = +inf.
    """
    dt = torch.float64
    B, Nq, Hq, D = q.shape
    Nk, Hkv = k.shape[1], k.shape[2]
    groups = Hq // Hkv
    z = lambda t, p: torch.zeros_like(p, dtype=dt) if t is None else t.to(dt)  # noqa: E731
    qh, tqh = q.to(dt).transpose(1, 2), z(tq, q).transpose(1, 2)
    kh, vh = k.to(dt).transpose(1, 2), v.to(dt).transpose(1, 2)
    tkh, tvh = z(tk, k).transpose(1, 2), z(tv, v).transpose(1, 2)
    if groups > 1:
        kh, vh, tkh, tvh = (x.repeat_interleave(groups, dim=1) for x in (kh, vh, tkh, tvh))
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    m = torch.full((B, Hq, Nq, 1), -math.inf, dtype=dt)
    ell = torch.zeros((B, Hq, Nq, 1), dtype=dt)
    r = torch.zeros((B, Hq, Nq, 1), dtype=dt)
    U = torch.zeros((B, Hq, Nq, D), dtype=dt)
    G = torch.zeros((B, Hq, Nq, D), dtype=dt)
    valid_all = _mask(Nq, Nk) if causal else torch.ones(Nq, Nk, dtype=torch.bool)
    for j0 in range(0, Nk, block_n):
        j1 = min(Nk, j0 + block_n)
        kj, vj, tkj, tvj = (x[:, :, j0:j1] for x in (kh, vh, tkh, tvh))
        valid = valid_all[:, j0:j1]
        S = scale * (qh @ kj.transpose(-1, -2))
        tS = scale * (tqh @ kj.transpose(-1, -2) + qh @ tkj.transpose(-1, -2))
        S = S.masked_fill(~valid, -math.inf)
        m_new = torch.maximum(m, S.amax(-1, keepdim=True))
        m_ref = torch.where(torch.isfinite(m_new), m_new, torch.zeros_like(m_new))
        alpha = torch.exp(m - m_ref)
        E = torch.exp(S - m_ref)
        H = E * tS.masked_fill(~valid, 0.0)
        ell = alpha * ell + E.sum(-1, keepdim=True)
        U = alpha * U + E @ vj
        r = alpha * r + H.sum(-1, keepdim=True)
        G = alpha * G + H @ vj + E @ tvj
        m = m_new
    empty = ell == 0
    safe = torch.where(empty, torch.ones_like(ell), ell)
    O = torch.where(empty, 0.0, U / safe)
    tO = torch.where(empty, 0.0, G / safe - (r / safe) * O)
    lse = torch.where(empty, math.inf, m + torch.log(safe)).squeeze(-1)
    return O.transpose(1, 2), lse, tO.transpose(1, 2)
