"""FlashAttention forward / JVP parity on the GPU (HIP via the C ABI vs the CPU oracle).

Ports the forward and forward-mode parts of flash_attention_jvp/test.py:
the shape table (:25-38), standalone JVP (:68-84), the torch.func and
forward_ad interfaces (:87-123), missing/value-only tangents (:144-158), the
uniform score shift (:161-172), central finite differences (:175-185), input
validation (:194-209), pipeline tails and empty rows (:212-224), graph replay
with a mutated tangent (:227-243) and long keys (:246-257).  Assertions that
need the backward pass (flash-attn's, not implemented here) are left out.
Tolerances: bf16 3e-2/3e-2 and fp16 3e-3/1e-2 against a CPU fp64 oracle (the
reference's), and the north-star 2e-2/2e-2 against dense fp32 torch.func.jvp
at the BASELINE config.
"""

from unittest.mock import patch

import pytest
import torch

from kernelforge_amd.flash_attention_jvp import (
    flash_attention,
    flash_attention_fwd_jvp,
    flash_attention_jvp,
    get_jvp_config,
)
from oracle import fa as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = (torch.float16, torch.bfloat16)
# B, Nq, Nk, Hq, Hkv, D, causal, scale -- the reference's case table.
CASES = (
    (1, 7, 11, 2, 2, 8, False, None),
    (2, 33, 65, 4, 4, 24, False, 0.3),
    (1, 129, 131, 3, 3, 64, False, None),
    (1, 65, 65, 2, 2, 64, True, None),
    (1, 19, 71, 4, 2, 96, True, None),
    (1, 71, 19, 4, 1, 32, True, None),
    (1, 37, 91, 6, 2, 128, False, 0.2),
    (1, 9, 13, 2, 1, 256, False, None),
    (1, 1, 1, 2, 2, 64, True, None),
    (1, 17, 29, 2, 2, 16, False, 0.05),
    (1, 23, 37, 2, 2, 80, False, 0.15),
    (1, 999, 515, 2, 2, 64, False, None),
)
# Head dims above 128 (the 4-wavefront, 32-key-tile schedule): several key
# tiles, partial tiles, causal masks, GQA and padded head dims.
CASES_WIDE = (
    (1, 130, 97, 2, 1, 256, True, None),
    (2, 70, 45, 2, 2, 200, False, 0.1),
    (1, 64, 256, 1, 1, 136, False, None),
    (1, 200, 200, 4, 2, 256, False, None),
)


def make_inputs(case, dtype, *, noncontiguous=False, seed=2026):
    b, nq, nk, h, hk, d, _, _ = case
    g = torch.Generator().manual_seed(seed)
    shapes = ((b, nq, h, d), (b, nk, hk, d), (b, nk, hk, d))
    out = []
    for shape in (*shapes, *shapes):
        if noncontiguous:
            x = torch.randn((*shape[:-1], shape[-1] * 2), generator=g).to(dtype).to(DEV)[..., ::2]
        else:
            x = torch.randn(shape, generator=g).to(dtype).to(DEV)
        out.append(x)
    return tuple(out)


def tolerance(dtype):
    return {torch.float16: dict(atol=3e-3, rtol=1e-2), torch.bfloat16: dict(atol=3e-2, rtol=3e-2)}[dtype]


def double_reference(inputs):
    return tuple(None if x is None else x.detach().cpu().double() for x in inputs)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CASES + CASES_WIDE)
def test_standalone_jvp(case, dtype):
    q, k, v, tq, tk, tv = make_inputs(case, dtype)
    kwargs = dict(causal=case[-2], softmax_scale=case[-1])
    out, lse = flash_attention(q, k, v, return_lse=True, **kwargs)
    from kernelforge_amd.flash_attention_jvp import custom

    with patch.object(custom, "_fwd_op", side_effect=AssertionError("extra forward")):
        actual = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, **kwargs)
    ref_out, ref_tangent = orc.attention_jvp(*double_reference((q, k, v, tq, tk, tv)), **kwargs)
    torch.testing.assert_close(out.cpu().double(), ref_out, **tolerance(dtype))
    torch.testing.assert_close(actual.cpu().double(), ref_tangent, **tolerance(dtype))
    ref_lse = orc.attention_lse(*double_reference((q, k)), **kwargs)
    torch.testing.assert_close(lse.cpu().double(), ref_lse, atol=1e-3, rtol=1e-4)
    dense = orc.attention_jvp_from_forward(*(x.cpu() for x in (q, k, v, tq, tk, tv, out, lse)), **kwargs)
    torch.testing.assert_close(actual.cpu(), dense, **tolerance(dtype))
    assert actual.shape == out.shape and actual.dtype == dtype and torch.isfinite(actual).all()
    if kwargs["causal"] and q.shape[1] > k.shape[1]:
        assert torch.count_nonzero(actual[:, :q.shape[1] - k.shape[1]]) == 0
        assert torch.count_nonzero(out[:, :q.shape[1] - k.shape[1]]) == 0
        assert torch.isinf(lse[:, :, :q.shape[1] - k.shape[1]]).all()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CASES + CASES_WIDE)
def test_fused_forward_jvp(case, dtype):
    """The single-pass (O, LSE, tO) kernel against the fp64 oracle and the two-launch path."""
    q, k, v, tq, tk, tv = make_inputs(case, dtype)
    kwargs = dict(causal=case[-2], softmax_scale=case[-1])
    out, lse, tangent = flash_attention_fwd_jvp(q, k, v, tq, tk, tv, **kwargs)
    ref_out, ref_tangent = orc.attention_jvp(*double_reference((q, k, v, tq, tk, tv)), **kwargs)
    torch.testing.assert_close(out.cpu().double(), ref_out, **tolerance(dtype))
    torch.testing.assert_close(tangent.cpu().double(), ref_tangent, **tolerance(dtype))
    ref_lse = orc.attention_lse(*double_reference((q, k)), **kwargs)
    torch.testing.assert_close(lse.cpu().double(), ref_lse, atol=1e-3, rtol=1e-4)
    # The forward kernel normalises O by the fp32 sum of E, the fused one by
    # the sum of the 16-bit E its products consume: O agrees to two ulps, the
    # LSE (the same fp32 sum in both) bit for bit.
    out2, lse2 = flash_attention(q, k, v, return_lse=True, **kwargs)
    torch.testing.assert_close(out.float(), out2.float(), atol=1e-6, rtol=2 * torch.finfo(dtype).eps)
    torch.testing.assert_close(lse, lse2, atol=0, rtol=0)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
def test_autograd_interfaces(dtype, causal):
    case = (1, 67, 41, 4, 2, 64, causal, 0.17)
    inputs = make_inputs(case, dtype, noncontiguous=True)
    q, k, v, tq, tk, tv = inputs
    kwargs = dict(causal=causal, softmax_scale=case[-1])

    def fn(q, k, v):
        return flash_attention(q, k, v, **kwargs)

    def fn_with_lse(q, k, v):
        return flash_attention(q, k, v, return_lse=True, **kwargs)

    ref_out, ref_tangent = orc.attention_jvp(*double_reference(inputs), **kwargs)
    out, tangent = torch.func.jvp(fn, (q, k, v), (tq, tk, tv))
    torch.testing.assert_close(out.cpu().double(), ref_out, **tolerance(dtype))
    torch.testing.assert_close(tangent.cpu().double(), ref_tangent, **tolerance(dtype))
    (stats_out, lse), (stats_tangent, lse_tangent) = torch.func.jvp(fn_with_lse, (q, k, v), (tq, tk, tv))
    torch.testing.assert_close(stats_out, out, atol=0, rtol=0)
    torch.testing.assert_close(stats_tangent, tangent, atol=0, rtol=0)
    assert lse.shape == (q.shape[0], q.shape[2], q.shape[1]) and lse.dtype == torch.float32
    assert torch.count_nonzero(lse_tangent) == 0
    with torch.autograd.forward_ad.dual_level():
        duals = tuple(torch.autograd.forward_ad.make_dual(p, t) for p, t in zip((q, k, v), (tq, tk, tv)))
        primal, forward_tangent = torch.autograd.forward_ad.unpack_dual(fn(*duals))
        torch.testing.assert_close(primal, out, atol=0, rtol=0)
        torch.testing.assert_close(forward_tangent, tangent, atol=0, rtol=0)
        dual_stats_out, dual_lse = fn_with_lse(*duals)
        stats_primal, stats_forward_tangent = torch.autograd.forward_ad.unpack_dual(dual_stats_out)
        lse_primal, lse_forward_tangent = torch.autograd.forward_ad.unpack_dual(dual_lse)
        torch.testing.assert_close(stats_primal, primal, atol=0, rtol=0)
        torch.testing.assert_close(stats_forward_tangent, forward_tangent, atol=0, rtol=0)
        torch.testing.assert_close(lse_primal, lse, atol=0, rtol=0)
        assert lse_forward_tangent is None


@pytest.mark.parametrize("dtype", DTYPES)
def test_missing_and_value_only_tangents(dtype):
    case = (1, 35, 49, 2, 2, 64, False, None)
    q, k, v, tq, tk, tv = make_inputs(case, dtype)
    out, lse = flash_attention(q, k, v, return_lse=True)
    for tangents in ((None, None, None), (None, None, tv), (tq, None, None), (None, tk, None), (tq, tk, None)):
        actual = flash_attention_jvp(q, k, v, *tangents, out, lse)
        _, reference = orc.attention_jvp(*double_reference((q, k, v)), *double_reference(tangents))
        torch.testing.assert_close(actual.cpu().double(), reference, **tolerance(dtype))
        _, _, fused = flash_attention_fwd_jvp(q, k, v, *tangents)
        torch.testing.assert_close(fused.cpu().double(), reference, **tolerance(dtype))
    with torch.autograd.forward_ad.dual_level():
        dual_v = torch.autograd.forward_ad.make_dual(v, tv)
        _, actual = torch.autograd.forward_ad.unpack_dual(flash_attention(q, k, dual_v))
    expected = flash_attention_jvp(q, k, v, None, None, tv, out, lse)
    torch.testing.assert_close(actual, expected, atol=0, rtol=0)


@pytest.mark.parametrize("dtype", DTYPES)
def test_uniform_score_shift_and_tile_sizes(dtype):
    case = (1, 39, 73, 2, 2, 64, False, None)
    q, k, v, tq, tk, tv = make_inputs(case, dtype)
    tk = torch.ones_like(k) * 0.25  # q tk^T is constant across keys
    out, lse = flash_attention(q, k, v, return_lse=True)
    shifted = flash_attention_jvp(q, k, v, None, tk, None, out, lse)
    torch.testing.assert_close(shifted, torch.zeros_like(shifted), **tolerance(dtype))
    _, _, fused_shift = flash_attention_fwd_jvp(q, k, v, None, tk, None)
    torch.testing.assert_close(fused_shift, torch.zeros_like(fused_shift), **tolerance(dtype))
    _, reference = orc.attention_jvp(*double_reference((q, k, v, tq, tk, tv)))
    for bm, bn, threads in ((16, 32, 128), (32, 64, 128), (64, 128, 256)):
        actual = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, block_m=bm, block_n=bn, threads=threads)
        torch.testing.assert_close(actual.cpu().double(), reference, **tolerance(dtype))


def test_finite_difference():
    case = (1, 23, 31, 4, 2, 32, True, None)
    inputs = make_inputs(case, torch.float16)
    q, k, v, tq, tk, tv = inputs
    out, lse = flash_attention(q, k, v, causal=True, return_lse=True)
    actual = flash_attention_jvp(*inputs, out, lse, causal=True)
    primals, tangents = double_reference(inputs[:3]), double_reference(inputs[3:])
    eps = 1e-4
    plus = orc.attention(*(p + eps * t for p, t in zip(primals, tangents)), causal=True)
    minus = orc.attention(*(p - eps * t for p, t in zip(primals, tangents)), causal=True)
    torch.testing.assert_close(actual.cpu().double(), (plus - minus) / (2 * eps), **tolerance(q.dtype))


def test_input_validation():
    case = (1, 9, 13, 2, 2, 64, False, None)
    q, k, v, tq, tk, tv = make_inputs(case, torch.float16)
    out, lse = flash_attention(q, k, v, return_lse=True)
    with pytest.raises(ValueError, match="lse"):
        flash_attention_jvp(q, k, v, tq, tk, tv, out, lse.half())
    with pytest.raises(ValueError, match="tq"):
        flash_attention_jvp(q, k, v, tq[:, :-1], tk, tv, out, lse)
    with pytest.raises(ValueError, match="finite"):
        flash_attention(q, k, v, softmax_scale=float("nan"))
    with pytest.raises(ValueError, match="positive"):
        flash_attention(q, k, v, softmax_scale=0.0)
    with pytest.raises(ValueError, match="float16"):
        flash_attention(q.float(), k.float(), v.float())
    with pytest.raises(ValueError, match="pipeline"):
        flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, num_stages=4)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("stages", (2, 3))
def test_pipeline_tails_and_empty_rows(dtype, causal, stages):
    inputs = make_inputs((1, 193, 97, 4, 2, 64, causal, None), dtype)
    out, lse = flash_attention(*inputs[:3], causal=causal, return_lse=True)
    actual = flash_attention_jvp(*inputs, out, lse, causal=causal, block_m=32, block_n=32, threads=128,
                                 num_stages=stages)
    _, reference = orc.attention_jvp(*double_reference(inputs), causal=causal)
    torch.testing.assert_close(actual.cpu().double(), reference, **tolerance(dtype))
    if causal:
        assert torch.count_nonzero(actual[:, :96]) == 0


def test_graph_replay_with_updated_tangent():
    inputs = make_inputs((1, 67, 131, 4, 2, 64, True, None), torch.float16)
    out, lse = flash_attention(*inputs[:3], causal=True, return_lse=True)
    config = get_jvp_config(*inputs[:3], causal=True)
    actual = flash_attention_jvp(*inputs, out, lse, causal=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = flash_attention_jvp(*inputs, out, lse, causal=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(captured, actual, atol=0, rtol=0)
    inputs[5].add_(0.03125)
    expected = flash_attention_jvp(*inputs, out, lse, causal=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        torch.testing.assert_close(captured, expected, atol=0, rtol=0)
    assert get_jvp_config(*inputs[:3], causal=True) == config


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
def test_long_key_default_and_explicit_pipeline(dtype, causal):
    inputs = make_inputs((1, 5, 8192, 2, 1, 64, causal, None), dtype)
    out, lse = flash_attention(*inputs[:3], causal=causal, return_lse=True)
    config = get_jvp_config(*inputs[:3], causal=causal)
    assert set(config) == {"block_m", "block_n", "threads", "num_stages"}
    actual = flash_attention_jvp(*inputs, out, lse, causal=causal)
    explicit = flash_attention_jvp(*inputs, out, lse, causal=causal, num_stages=2)
    _, reference = orc.attention_jvp(*double_reference(inputs), causal=causal)
    torch.testing.assert_close(actual.cpu().double(), reference, **tolerance(dtype))
    torch.testing.assert_close(explicit.cpu().double(), reference, **tolerance(dtype))


def test_baseline_config_fused():
    """B=2, H=16, N=4096, D=128 bf16, scale 1/sqrt(D), non-causal.

    O, LSE and tO of the fused kernel against dense fp32 torch.func.jvp
    (north-star tolerance 2e-2 / 2e-2) on a subset of (batch, head) slices,
    plus size-independent properties over the whole output: agreement with
    the two-launch path, exact linearity in the tangents, finiteness.
    """
    case = (2, 4096, 4096, 16, 16, 128, False, None)
    q, k, v, tq, tk, tv = make_inputs(case, torch.bfloat16, seed=0)
    out, lse, tangent = flash_attention_fwd_jvp(q, k, v, tq, tk, tv)
    for b, h in ((0, 0), (1, 7), (1, 15)):
        sl = lambda x: x[b:b + 1, :, h:h + 1].cpu()  # noqa: E731
        ro, rt = orc.attention_jvp(*(sl(x) for x in (q, k, v, tq, tk, tv)))
        torch.testing.assert_close(sl(out).float(), ro.float(), atol=2e-2, rtol=2e-2)
        torch.testing.assert_close(sl(tangent).float(), rt.float(), atol=2e-2, rtol=2e-2)
        rl = orc.attention_lse(sl(q).float(), sl(k).float())
        torch.testing.assert_close(lse[b:b + 1, h:h + 1].cpu(), rl, atol=2e-3, rtol=1e-4)
    o2, l2 = flash_attention(q, k, v, return_lse=True)
    torch.testing.assert_close(out.float(), o2.float(), atol=1e-6, rtol=2 * torch.finfo(torch.bfloat16).eps)
    torch.testing.assert_close(lse, l2, atol=0, rtol=0)
    t2 = flash_attention_jvp(q, k, v, tq, tk, tv, o2, l2)
    torch.testing.assert_close(t2.float(), tangent.float(), atol=2e-2, rtol=2e-2)
    _, _, tangent2 = flash_attention_fwd_jvp(q, k, v, 2 * tq, 2 * tk, 2 * tv)
    assert torch.equal(tangent2, 2 * tangent)
    assert torch.isfinite(tangent).all() and torch.isfinite(out).all()


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("jump", (30.0, 140.0))
@pytest.mark.parametrize("d", (64, 256))
def test_scores_growing_past_first_tile(dtype, jump, d):
    """Keys after the first tile score `jump` log2 units above it.

    The forward kernels fix each row's exponent reference at the max of its
    first key tile; E = exp2(S - m) then grows to 2^jump.  bf16 holds 2^30 and
    2^140 overflows; fp16 overflows already at 2^16.  An overflow must send
    the workgroup to the rescaling scan and still give the oracle's result.
    """
    b, n, h = 1, 300, 2
    g = torch.Generator().manual_seed(11)
    q = torch.full((b, n, h, d), 2.0)
    k = 0.05 * torch.randn(b, n, h, d, generator=g)
    # q.k over the later keys: 2 * c * d; scaled by d^-0.5 and log2(e) -> jump.
    c = jump / (2.0 * d * d ** -0.5 * 1.4426950408889634)
    k[:, 64:] += c
    v, tq, tk, tv = (torch.randn(b, n, h, d, generator=g) for _ in range(4))
    inputs = tuple(x.to(dtype).to(DEV) for x in (q, k, v, tq, tk, tv))
    ref_out, ref_tangent = orc.attention_jvp(*double_reference(inputs))
    ref_lse = orc.attention_lse(*double_reference(inputs[:2]))
    out, lse, tangent = flash_attention_fwd_jvp(*inputs)
    out2, lse2 = flash_attention(*inputs[:3], return_lse=True)
    tangent2 = flash_attention_jvp(*inputs, out2, lse2)
    for o, t, l in ((out, tangent, lse), (out2, tangent2, lse2)):
        assert torch.isfinite(o).all() and torch.isfinite(t).all() and torch.isfinite(l).all()
        torch.testing.assert_close(o.cpu().double(), ref_out, **tolerance(dtype))
        torch.testing.assert_close(t.cpu().double(), ref_tangent, **tolerance(dtype))
        torch.testing.assert_close(l.cpu().double(), ref_lse, atol=1e-3, rtol=1e-4)
