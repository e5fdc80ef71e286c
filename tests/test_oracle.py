"""CPU tests that pin the oracle (no GPU).

Each oracle function is checked against the golden fixtures (pure-Python fp64
brute force with a different algorithm, tests/golden/make_golden.py) and
against what the mathematics fixes: closed forms, invariants, finite
differences.  The `test_mutation_*` tests plant a plausible mistake in a copy
of an oracle function and assert that the corresponding check fails, i.e.
that the check actually pins something.
"""

import json
import math
from pathlib import Path

import pytest
import torch

from oracle import fa as ofa
from oracle import rmsnorm as orms
from oracle import sana as osana

GOLDEN = Path(__file__).resolve().parent / "golden"


def load(name):
    return json.loads((GOLDEN / f"{name}_golden.json").read_text())


def t64(x):
    return torch.tensor(x, dtype=torch.float64)


# ---------------------------------------------------------------------------
# RMSNorm
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", load("rmsnorm"), ids=lambda c: f"{c['rows']}x{c['dim']}")
def test_rmsnorm_golden(case):
    x, w, y = t64(case["x"]), t64(case["w"]), t64(case["y"])
    torch.testing.assert_close(orms.rmsnorm_fp64(x, w, case["eps"]), y, rtol=1e-12, atol=0)
    out32 = orms.rmsnorm(x.float(), w.float(), case["eps"])
    torch.testing.assert_close(out32.double(), y, rtol=3e-7, atol=1e-30)
    outbf = orms.rmsnorm(x.bfloat16(), w.bfloat16(), case["eps"])
    # two bf16 roundings: |err| <= 2^-8 |y| * (1 + |w|) roughly; use 2 ulps
    assert ((outbf.double() - y).abs() <= 2.0 ** -7 * y.abs() + 1e-12).all()


def test_rmsnorm_unit_rms_and_scale_equivariance():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(16, 300, generator=g, dtype=torch.float64)
    y = orms.rmsnorm_fp64(x, torch.ones(300, dtype=torch.float64), 0.0)
    torch.testing.assert_close(y.pow(2).mean(-1).sqrt(), torch.ones(16, dtype=torch.float64))
    torch.testing.assert_close(orms.rmsnorm_fp64(7.5 * x, torch.ones(300, dtype=torch.float64), 0.0), y)
    # eps only matters relative to the mean square
    a = orms.rmsnorm_noweight(x.float(), 1e-12)
    torch.testing.assert_close(a.double(), y, rtol=1e-6, atol=1e-7)


@pytest.mark.parametrize("case", load("rmsnorm_bf16"), ids=lambda c: f"{c['rows']}x{c['dim']}")
def test_rmsnorm_bf16_two_rounding_points(case):
    """The oracle in bf16 reproduces the fixture's two rounding points bit for bit."""
    x = torch.tensor(case["x"], dtype=torch.float64).bfloat16()
    w = torch.tensor(case["w"], dtype=torch.float64).bfloat16()
    y = torch.tensor(case["y"], dtype=torch.float64).bfloat16()
    assert torch.equal(x.double(), torch.tensor(case["x"], dtype=torch.float64))  # exact in bf16
    out = orms.rmsnorm(x, w, case["eps"])
    assert out.dtype == torch.bfloat16
    assert torch.equal(out, y)


@pytest.mark.parametrize("case", load("rmsnorm_inv"), ids=lambda c: f"eps{c['eps']:.4g}dir{c['direction']}")
def test_rmsnorm_inverse_sqrt_is_correctly_rounded(case):
    """Rows where a one-ulp error of 1/sqrt(mean + eps) flips a bf16 output: the
    oracle gives the fixture's bits, and the same computation with inv moved
    one ulp in the recorded direction gives the fixture's ``y_off`` instead."""
    x = torch.tensor(case["x"], dtype=torch.float64).bfloat16()
    w = torch.tensor(case["w"], dtype=torch.float64).bfloat16()
    y = torch.tensor(case["y"], dtype=torch.float64).bfloat16()
    y_off = torch.tensor(case["y_off"], dtype=torch.float64).bfloat16()
    assert torch.equal(orms.rmsnorm(x, w, case["eps"]), y)
    xf = x.float()
    inv = 1.0 / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + case["eps"])
    off = torch.nextafter(inv, torch.full_like(inv, math.inf if case["direction"] > 0 else -math.inf))
    bad = ((xf * off).bfloat16().float() * w.float()).bfloat16()
    assert torch.equal(bad, y_off) and not torch.equal(bad, y)


def test_mutation_rmsnorm_single_rounding():
    """A restatement that rounds once (dropping the cast before the weight
    multiply, original.py:51) fails the double-rounding fixture."""
    def single_rounding(x, w, eps):
        xf = x.float()
        inv = 1.0 / torch.sqrt(xf.pow(2).mean(-1, keepdim=True) + eps)
        return (xf * inv * w.float()).to(x.dtype)

    failures = 0
    for case in load("rmsnorm_bf16"):
        x = torch.tensor(case["x"], dtype=torch.float64).bfloat16()
        w = torch.tensor(case["w"], dtype=torch.float64).bfloat16()
        y = torch.tensor(case["y"], dtype=torch.float64).bfloat16()
        y_single = torch.tensor(case["y_single"], dtype=torch.float64).bfloat16()
        bad = single_rounding(x, w, case["eps"])
        assert torch.equal(bad, y_single)
        failures += int(not torch.equal(bad, y))
    assert failures == len(load("rmsnorm_bf16"))


def test_rmsnorm_promotion_and_gradients():
    """bf16 x with an fp32 weight returns fp32 (torch promotion, original.py:52);
    the autograd gradients of the oracle agree with central differences of the
    fp64 formula."""
    g = torch.Generator().manual_seed(4)
    x = torch.randn(3, 40, generator=g).bfloat16()
    w = 1 + 0.1 * torch.randn(40, generator=g)
    y = orms.rmsnorm(x, w, 1e-6)
    assert y.dtype == torch.float32
    assert torch.equal(y, (orms.rmsnorm(x, torch.ones(40), 1e-6)) * w)
    x64 = torch.randn(3, 40, generator=g, dtype=torch.float64)
    w64 = 1 + 0.1 * torch.randn(40, generator=g, dtype=torch.float64)
    dy = torch.randn(3, 40, generator=g, dtype=torch.float64)
    dx, dw = orms.rmsnorm_grads(x64, w64, dy, 1e-6)
    e = 1e-6
    for i, j in ((0, 0), (1, 17), (2, 39)):
        d = torch.zeros_like(x64)
        d[i, j] = e
        fd = ((orms.rmsnorm_fp64(x64 + d, w64, 1e-6) - orms.rmsnorm_fp64(x64 - d, w64, 1e-6)) * dy).sum() / (2 * e)
        assert abs(float(fd) - float(dx[i, j])) < 1e-7
    for j in (0, 21):
        d = torch.zeros_like(w64)
        d[j] = e
        fd = ((orms.rmsnorm_fp64(x64, w64 + d, 1e-6) - orms.rmsnorm_fp64(x64, w64 - d, 1e-6)) * dy).sum() / (2 * e)
        assert abs(float(fd) - float(dw[j])) < 1e-7


def test_mutation_rmsnorm_mean_vs_sum():
    case = load("rmsnorm")[0]
    x, w, y = t64(case["x"]), t64(case["w"]), t64(case["y"])
    bad = x / torch.sqrt(x.pow(2).sum(-1, keepdim=True) + case["eps"]) * w  # sum instead of mean
    assert not torch.allclose(bad, y, rtol=1e-3)


# ---------------------------------------------------------------------------
# SANA linear attention
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("case", load("sana"), ids=lambda c: f"B{c['B']}N{c['N']}H{c['H']}D{c['D']}")
def test_sana_golden(case):
    qkv, ref = t64(case["qkv"]), t64(case["out"])
    H, D = case["H"], case["D"]
    out = osana.linear_attention(qkv.float(), H, D, case["eps"])
    torch.testing.assert_close(out.double(), ref, rtol=1e-5, atol=1e-6)
    for splits in (1, 2, 3, case["N"]):
        torch.testing.assert_close(osana.linear_attention_split(qkv, H, D, splits, case["eps"]), ref,
                                   rtol=1e-10, atol=1e-12)


def test_sana_invariants():
    g = torch.Generator().manual_seed(1)
    qkv = torch.randn(2, 50, 3, 4 * 8, generator=g, dtype=torch.float64)
    out = osana.linear_attention(qkv, 4, 8)
    # linear in v
    q2 = qkv.clone()
    q2[:, :, 2] *= -3.0
    torch.testing.assert_close(osana.linear_attention(q2, 4, 8), -3.0 * out)
    # relu(q) = 0 -> 0
    q3 = qkv.clone()
    q3[:, :, 0] = -q3[:, :, 0].abs()
    assert torch.count_nonzero(osana.linear_attention(q3, 4, 8)) == 0
    # v = const -> out = const wherever the denominator is non-zero
    q4 = qkv.clone()
    q4[:, :, 2] = 2.5
    o4 = osana.linear_attention(q4, 4, 8)
    # (rows whose relu(q) is all zero for a head have a zero denominator -> 0)
    live = (torch.relu(qkv[:, :, 0]).reshape(2, 50, 4, 8).sum(-1) > 0).repeat_interleave(8, dim=-1)
    torch.testing.assert_close(o4[live], torch.full_like(o4[live], 2.5))
    assert torch.count_nonzero(o4[~live]) == 0


def test_sana_eager_bf16_close_to_fp32():
    g = torch.Generator().manual_seed(2)
    qkv = torch.randn(1, 256, 3, 2 * 32, generator=g).bfloat16()
    a = osana.linear_attention(qkv, 2, 32, fp32_attention=True)
    b = osana.linear_attention(qkv, 2, 32, fp32_attention=False)
    torch.testing.assert_close(b, a, atol=2e-2, rtol=2e-2)


def test_mutation_sana_drop_ones_row_or_transpose():
    case = load("sana")[0]
    qkv, ref = t64(case["qkv"]), t64(case["out"])
    H, D = case["H"], case["D"]
    q, k, v = osana.unpack_qkv(qkv, H, D)
    q, k = torch.relu(q), torch.relu(k)
    # a PAD_VAL of 0 (dropped denominator) is caught
    vk = torch.nn.functional.pad(v, (0, 0, 0, 1), value=0.0) @ k
    out = vk @ q
    bad = (out[:, :, :-1] / (out[:, :, -1:] + 1e-15)).reshape(case["B"], H * D, -1).permute(0, 2, 1)
    assert not torch.allclose(bad, ref, rtol=1e-3)
    # a transposed state (S^T instead of S) is caught
    vk = torch.nn.functional.pad(v, (0, 0, 0, 1), value=1.0) @ k
    st = torch.cat([vk[:, :, :-1].transpose(-1, -2), vk[:, :, -1:]], dim=2)
    out = st @ q
    bad = (out[:, :, :-1] / (out[:, :, -1:] + 1e-15)).reshape(case["B"], H * D, -1).permute(0, 2, 1)
    assert not torch.allclose(bad, ref, rtol=1e-3)


def test_lite_la_forward_glue():
    """LiteLA.forward's glue (part order of the packed qkv, the q/k RMSNorm, the
    output projection) on top of the golden-pinned linear attention: with
    W_qkv = [I; 2I; 3I] the packed qkv is exactly (x, 2x, 3x), a proj of
    diag(d) + b scales and shifts the attention output per channel."""
    g = torch.Generator().manual_seed(5)
    B, N, H, D = 2, 40, 3, 8
    C = H * D
    x = torch.randn(B, N, C, generator=g, dtype=torch.float64).float()
    eye = torch.eye(C)
    w_qkv = torch.cat([eye, 2 * eye, 3 * eye])
    d = torch.rand(C, generator=g) + 0.5
    bias = torch.randn(C, generator=g)
    got = osana.lite_la_forward(x, w_qkv, None, torch.diag(d), bias, H, 1e-15)
    att = osana.linear_attention(torch.stack((x, 2 * x, 3 * x), dim=2), H, D)
    torch.testing.assert_close(got, att * d + bias, rtol=1e-6, atol=1e-6)
    # a swapped q/v order is caught
    swapped = osana.linear_attention(torch.stack((3 * x, 2 * x, x), dim=2), H, D)
    assert not torch.allclose(swapped * d + bias, got, rtol=1e-3)
    # qk_norm normalises q and k over C before the attention
    wq, wk = torch.rand(C, generator=g) + 0.5, torch.rand(C, generator=g) + 0.5
    got = osana.lite_la_forward(x, w_qkv, None, torch.diag(d), bias, H, 1e-15, wq, wk, 1e-5)
    qn = orms.rmsnorm(x, wq, 1e-5)
    kn = orms.rmsnorm(2 * x, wk, 1e-5)
    att = osana.linear_attention(torch.stack((qn, kn, 3 * x), dim=2), H, D)
    torch.testing.assert_close(got, att * d + bias, rtol=1e-6, atol=1e-6)



def _angles(S, D, g):
    """Per-token, per-pair angles: cos/sin [S, D] with equal values on 2i, 2i+1."""
    theta = torch.rand(S, D // 2, generator=g, dtype=torch.float64) * 6.0 - 3.0
    rep = theta.repeat_interleave(2, dim=-1)
    return theta, torch.cos(rep), torch.sin(rep)


def test_rotary_closed_forms():
    """apply_rotary_emb (SANA_LinearAttention/original.py:14-58) pinned by the
    mathematics: zero angle is the identity, a quarter turn maps (a, b) to
    (-b, a), equal pair angles are a complex multiplication by e^{i theta}
    (fp64), rotations preserve each pair's norm and compose additively, and the
    complex-frequency path agrees with the (cos, sin) path."""
    g = torch.Generator().manual_seed(11)
    B, H, D, S = 2, 3, 8, 7
    x = torch.randn(B, H, D, S, generator=g, dtype=torch.float64)   # SANA layout [B, H, D, S]
    one, zero = torch.ones(S, D, dtype=torch.float64), torch.zeros(S, D, dtype=torch.float64)
    assert torch.equal(osana.apply_rotary_emb(x, (one, zero), use_real_unbind_dim=-2), x)
    quarter = osana.apply_rotary_emb(x, (zero, one), use_real_unbind_dim=-2)
    assert torch.equal(quarter[:, :, 0::2], -x[:, :, 1::2]) and torch.equal(quarter[:, :, 1::2], x[:, :, 0::2])
    theta, cos, sin = _angles(S, D, g)
    got = osana.apply_rotary_emb(x, (cos, sin), use_real_unbind_dim=-2)
    z = torch.complex(x[:, :, 0::2], x[:, :, 1::2]) * torch.polar(torch.ones_like(theta), theta).T
    torch.testing.assert_close(got[:, :, 0::2], z.real, rtol=1e-12, atol=1e-12)
    torch.testing.assert_close(got[:, :, 1::2], z.imag, rtol=1e-12, atol=1e-12)
    norm = lambda t: t[:, :, 0::2] ** 2 + t[:, :, 1::2] ** 2
    torch.testing.assert_close(norm(got), norm(x), rtol=1e-12, atol=1e-12)
    theta2, cos2, sin2 = _angles(S, D, g)
    both = osana.apply_rotary_emb(got, (cos2, sin2), use_real_unbind_dim=-2)
    rep = (theta + theta2).repeat_interleave(2, dim=-1)
    direct = osana.apply_rotary_emb(x, (torch.cos(rep), torch.sin(rep)), use_real_unbind_dim=-2)
    torch.testing.assert_close(both, direct, rtol=1e-12, atol=1e-12)
    # the last-dim layout [B, H, S, D] is the same rotation, transposed
    last = osana.apply_rotary_emb(x.transpose(-1, -2), (cos, sin), use_real_unbind_dim=-1)
    torch.testing.assert_close(last, got.transpose(-1, -2), rtol=0, atol=0)
    # complex frequencies [1, S, D/2] on a [B, S, H, D] tensor
    xs = x.permute(0, 3, 1, 2)
    cplx = osana.apply_rotary_emb(xs, torch.polar(torch.ones_like(theta), theta)[None], use_real=False)
    torch.testing.assert_close(cplx, got.permute(0, 3, 1, 2), rtol=1e-12, atol=1e-12)


def test_rotary_packed_layout_and_rounding():
    """rope_packed rotates q and k of the packed [B, N, 3, C] qkv per head and
    leaves v alone; a quarter turn moves channel h*D + 2i of token n to
    h*D + 2i + 1 of the same token and head.  In 16 bits the result is the
    fp32 value rounded once (round to nearest even)."""
    B, N, H, D = 1, 4, 3, 8
    C = H * D
    qkv = torch.zeros(B, N, 3, C, dtype=torch.float64)
    qkv[0, 2, 0, 1 * D + 4] = 1.0      # q, token 2, head 1, pair 2 (real part)
    qkv[0, 1, 1, 2 * D + 7] = 2.0      # k, token 1, head 2, pair 3 (imaginary part)
    qkv[0, 3, 2, 5] = 3.0              # v is not rotated
    zero, one = torch.zeros(N, D, dtype=torch.float64), torch.ones(N, D, dtype=torch.float64)
    out = osana.rope_packed(qkv, zero, one, H)
    want = torch.zeros_like(qkv)
    want[0, 2, 0, 1 * D + 5] = 1.0     # (a, b) -> (-b, a): real 1 -> imaginary 1
    want[0, 1, 1, 2 * D + 6] = -2.0    # imaginary 2 -> real -2
    want[0, 3, 2, 5] = 3.0
    assert torch.equal(out, want)
    g = torch.Generator().manual_seed(3)
    x = torch.randn(2, 5, 3, C, generator=g).to(torch.bfloat16)
    _, cos, sin = _angles(5, D, g)
    got = osana.rope_packed(x, cos.float(), sin.float(), H)
    exact = osana.rope_packed(x.double(), cos.float().double(), sin.float().double(), H)
    # one rounding of a value computed with two fp32 products and one fp32 sum
    torch.testing.assert_close(got.double(), exact.to(torch.bfloat16).double(), rtol=2 ** -7, atol=1e-6)
    assert torch.equal(got[:, :, 2], x[:, :, 2])


def test_lite_la_forward_rotary():
    """LiteLA.forward applies the rotary embedding to q and k after the norm
    and before the attention (SANA_LinearAttention/original.py:129-138)."""
    g = torch.Generator().manual_seed(9)
    B, N, H, D = 1, 12, 2, 8
    C = H * D
    x = torch.randn(B, N, C, generator=g)
    eye = torch.eye(C)
    w_qkv = torch.cat([eye, 2 * eye, 3 * eye])
    _, cos, sin = _angles(N, D, g)
    got = osana.lite_la_forward(x, w_qkv, None, eye, None, H, 1e-15, rotary_emb=(cos.float(), sin.float()))
    qkv = osana.rope_packed(torch.stack((x, 2 * x, 3 * x), dim=2), cos.float(), sin.float(), H)
    torch.testing.assert_close(got, osana.linear_attention(qkv, H, D), rtol=1e-6, atol=1e-6)
    plain = osana.lite_la_forward(x, w_qkv, None, eye, None, H, 1e-15)
    assert not torch.allclose(got, plain, rtol=1e-3)

# ---------------------------------------------------------------------------
# FlashAttention forward / JVP
# ---------------------------------------------------------------------------
def _fa_tensors(case):
    def t(name):
        return t64(case[name])  # [B, S, H, D]
    return tuple(t(n) for n in ("q", "k", "v", "tq", "tk", "tv"))


FA_CASES = load("fa")


@pytest.mark.parametrize("case", FA_CASES, ids=lambda c: f"{c['Nq']}x{c['Nk']}H{c['Hq']}/{c['Hkv']}D{c['D']}c{int(c['causal'])}")
def test_fa_golden(case):
    q, k, v, tq, tk, tv = _fa_tensors(case)
    kw = dict(softmax_scale=case["scale"], causal=case["causal"])
    out, tout = ofa.attention_jvp(q, k, v, tq, tk, tv, **kw)
    torch.testing.assert_close(out, t64(case["out"]), rtol=1e-10, atol=1e-12)
    torch.testing.assert_close(tout, t64(case["tout"]), rtol=1e-10, atol=1e-12)
    lse = ofa.attention_lse(q, k, **kw)
    torch.testing.assert_close(lse, t64(case["lse"]), rtol=1e-12, atol=1e-12)
    dense = ofa.attention_jvp_from_forward(q, k, v, tq, tk, tv, out, lse, **kw)
    torch.testing.assert_close(dense.double(), t64(case["tout"]), rtol=1e-5, atol=1e-6)
    for bn in (1, 2, 3, 64):
        o2, l2, t2 = ofa.fused_forward_jvp_tiled(q, k, v, tq, tk, tv, block_n=bn, **kw)
        torch.testing.assert_close(o2, t64(case["out"]), rtol=1e-10, atol=1e-12)
        torch.testing.assert_close(t2, t64(case["tout"]), rtol=1e-10, atol=1e-12)
        torch.testing.assert_close(l2, t64(case["lse"]), rtol=1e-12, atol=1e-12)


def _rand(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float64)


@pytest.mark.parametrize("causal", (False, True))
def test_fa_finite_difference_and_tiled(causal):
    B, Nq, Nk, Hq, Hkv, D = 1, 9, 13, 4, 2, 16
    q, tq = _rand((B, Nq, Hq, D), 1), _rand((B, Nq, Hq, D), 2)
    k, v, tk, tv = (_rand((B, Nk, Hkv, D), s) for s in (3, 4, 5, 6))
    _, tout = ofa.attention_jvp(q, k, v, tq, tk, tv, causal=causal)
    eps = 1e-5
    plus = ofa.attention(q + eps * tq, k + eps * tk, v + eps * tv, causal=causal)
    minus = ofa.attention(q - eps * tq, k - eps * tk, v - eps * tv, causal=causal)
    torch.testing.assert_close(tout, (plus - minus) / (2 * eps), rtol=1e-6, atol=1e-8)
    for bn in (4, 5, 16):
        o, lse, t = ofa.fused_forward_jvp_tiled(q, k, v, tq, tk, tv, causal=causal, block_n=bn)
        torch.testing.assert_close(t, tout, rtol=1e-10, atol=1e-12)


def test_fa_consistency_checks():
    """Derivation section 11: uniform shift -> 0, value-only -> P tv, mass preservation."""
    B, N, H, D = 1, 11, 2, 8
    q, k, v, tv = (_rand((B, N, H, D), s) for s in (7, 8, 9, 10))
    zero = torch.zeros_like(q)
    _, t = ofa.attention_jvp(q, k, v, None, torch.ones_like(k) * 0.25, None)
    assert t.abs().max() < 1e-12
    out, t = ofa.attention_jvp(q, k, v, None, None, tv)
    torch.testing.assert_close(t, ofa.attention(q, k, tv))
    # mass preservation: with v = 1 the output is 1 for every tangent, so tO = 0
    ones = torch.ones_like(v)
    _, t = ofa.attention_jvp(q, k, ones, _rand(q.shape, 11), _rand(k.shape, 12), zero[:, :, :, :] * 0)
    assert t.abs().max() < 1e-12


def test_mutation_fa_wrong_sign_or_missing_correction():
    case = FA_CASES[0]
    q, k, v, tq, tk, tv = _fa_tensors(case)
    gamma = case["D"] ** -0.5
    qh, kh, vh, tqh, tkh, tvh = (x.transpose(1, 2) for x in (q, k, v, tq, tk, tv))
    grp = case["Hq"] // case["Hkv"]
    kh, vh, tkh, tvh = (x.repeat_interleave(grp, dim=1) for x in (kh, vh, tkh, tvh))
    p = (qh @ kh.transpose(-1, -2) * gamma).softmax(-1)
    ts = (tqh @ kh.transpose(-1, -2) + qh @ tkh.transpose(-1, -2)) * gamma
    ref = t64(case["tout"]).transpose(1, 2)
    missing = p @ tvh + (p * ts) @ vh  # no "- rowsum(H) O" term
    assert not torch.allclose(missing, ref, atol=1e-3)
    flipped = p @ tvh + (p * ts) @ vh + (p * ts).sum(-1, keepdim=True) * (p @ vh)
    assert not torch.allclose(flipped, ref, atol=1e-3)
    good = p @ tvh + (p * ts) @ vh - (p * ts).sum(-1, keepdim=True) * (p @ vh)
    torch.testing.assert_close(good, ref, rtol=1e-10, atol=1e-12)


def test_fa_empty_rows_convention():
    case = FA_CASES[2]  # Nq=5 > Nk=3 causal: rows 0..1 have no valid key
    q, k, v, tq, tk, tv = _fa_tensors(case)
    out, t = ofa.attention_jvp(q, k, v, tq, tk, tv, causal=True, softmax_scale=case["scale"])
    assert torch.count_nonzero(out[:, :2]) == 0 and torch.count_nonzero(t[:, :2]) == 0
    lse = ofa.attention_lse(q, k, causal=True, softmax_scale=case["scale"])
    assert torch.isinf(lse[:, :, :2]).all() and (lse[:, :, :2] > 0).all()
    assert math.isinf(case["lse"][0][0][0])
