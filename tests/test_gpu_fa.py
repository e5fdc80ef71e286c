"""FlashAttention forward and forward-mode AD on the GPU: the HIP kernels (through
the C ABI) against the CPU oracle.

The shapes are the reference's edge-case table (flash_attention_jvp/test.py:
25-38: partial tiles, padded head dims, bottom-right rectangular causal masks,
rows with no valid key, GQA and MQA) plus head dims above 128.  The properties
checked are those the reference's forward-mode tests pin (test.py:68-123,
144-257): the JVP from cached statistics without a second forward, the
torch.func / forward_ad rules, absent tangents, a score shift that is uniform
over keys, central differences, argument validation, masked rows, graph
replay with a changed tangent and long key sequences.  Tolerances: 3e-2/3e-2
(bf16) and 3e-3/1e-2 (fp16) against a CPU fp64 oracle, as the reference uses,
and the north-star 2e-2/2e-2 against dense fp32 torch.func.jvp at the
BASELINE config.
"""

from unittest.mock import patch

import pytest
import torch

from kernelforge_amd.flash_attention_jvp import (
    custom,
    flash_attention,
    flash_attention_fwd_jvp,
    flash_attention_jvp,
    get_jvp_config,
)
from oracle import fa as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = (torch.float16, torch.bfloat16)
# B, Nq, Nk, Hq, Hkv, D, causal, scale -- the reference's case table (test data).
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
BOUNDS = {torch.float16: dict(atol=3e-3, rtol=1e-2), torch.bfloat16: dict(atol=3e-2, rtol=3e-2)}


def seeded(case, dtype, *, strided=False, seed=2026):
    """q, k, v, tq, tk, tv drawn on the CPU from one seeded generator, then moved to
    the GPU.  ``strided`` gives every tensor a last-dimension stride of 2."""
    b, nq, nk, hq, hkv, d = case[:6]
    g = torch.Generator().manual_seed(seed)
    tensors = []
    for shape in [(b, nq, hq, d), (b, nk, hkv, d), (b, nk, hkv, d)] * 2:
        if strided:
            wide = torch.randn((*shape[:-1], 2 * shape[-1]), generator=g).to(dtype).to(DEV)
            tensors.append(wide[..., ::2])
        else:
            tensors.append(torch.randn(shape, generator=g).to(dtype).to(DEV))
    return tuple(tensors)


def on_cpu64(tensors):
    return tuple(None if t is None else t.detach().cpu().double() for t in tensors)


def close(actual, expected, dtype):
    torch.testing.assert_close(actual.detach().cpu().double(), expected, **BOUNDS[dtype])


def opts(case):
    return dict(causal=case[6], softmax_scale=case[7])


def empty_rows(case):
    """Query rows with no valid key under a bottom-right causal mask."""
    return max(0, case[1] - case[2]) if case[6] else 0


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CASES + CASES_WIDE)
def test_jvp_from_cached_statistics(case, dtype):
    """tO from the forward's O and LSE with no second forward launch."""
    q, k, v, tq, tk, tv = seeded(case, dtype)
    out, lse = flash_attention(q, k, v, return_lse=True, **opts(case))
    with patch.object(custom, "_fwd_op", side_effect=AssertionError("the JVP launched a forward")):
        tangent = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, **opts(case))
    ref_out, ref_tangent = orc.attention_jvp(*on_cpu64((q, k, v, tq, tk, tv)), **opts(case))
    close(out, ref_out, dtype)
    close(tangent, ref_tangent, dtype)
    torch.testing.assert_close(lse.cpu().double(), orc.attention_lse(*on_cpu64((q, k)), **opts(case)),
                               atol=1e-3, rtol=1e-4)
    # The reference's dense formula on the same cached statistics.
    dense = orc.attention_jvp_from_forward(*(t.cpu() for t in (q, k, v, tq, tk, tv, out, lse)), **opts(case))
    torch.testing.assert_close(tangent.cpu(), dense, **BOUNDS[dtype])
    assert tangent.dtype == dtype and tangent.shape == out.shape
    assert bool(torch.isfinite(tangent).all())
    n_empty = empty_rows(case)
    if n_empty:
        assert not out[:, :n_empty].any() and not tangent[:, :n_empty].any()
        assert bool(torch.isposinf(lse[:, :, :n_empty]).all())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CASES + CASES_WIDE)
def test_fused_single_pass(case, dtype):
    """(O, LSE, tO) from one scan against the fp64 oracle and the two-launch path."""
    q, k, v, tq, tk, tv = seeded(case, dtype)
    out, lse, tangent = flash_attention_fwd_jvp(q, k, v, tq, tk, tv, **opts(case))
    ref_out, ref_tangent = orc.attention_jvp(*on_cpu64((q, k, v, tq, tk, tv)), **opts(case))
    close(out, ref_out, dtype)
    close(tangent, ref_tangent, dtype)
    torch.testing.assert_close(lse.cpu().double(), orc.attention_lse(*on_cpu64((q, k)), **opts(case)),
                               atol=1e-3, rtol=1e-4)
    # The forward kernel divides by the fp32 sum of E, the fused one by the
    # sum of the 16-bit E its products use: O within two ulps, LSE (the same
    # fp32 sum) bit for bit.
    out_fwd, lse_fwd = flash_attention(q, k, v, return_lse=True, **opts(case))
    torch.testing.assert_close(out.float(), out_fwd.float(), atol=1e-6, rtol=2 * torch.finfo(dtype).eps)
    assert torch.equal(lse, lse_fwd)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
def test_func_jvp_and_forward_ad(dtype, causal):
    """torch.func.jvp and forward_ad dual numbers reach the same HIP JVP rule; the
    LSE output carries no tangent.  Inputs have a non-unit last stride."""
    case = (1, 67, 41, 4, 2, 64, causal, 0.17)
    primals_tangents = seeded(case, dtype, strided=True)
    primals, tangents = primals_tangents[:3], primals_tangents[3:]
    ref_out, ref_tangent = orc.attention_jvp(*on_cpu64(primals_tangents), **opts(case))

    def attend(*qkv):
        return flash_attention(*qkv, **opts(case))

    def attend_with_lse(*qkv):
        return flash_attention(*qkv, return_lse=True, **opts(case))

    out, tangent = torch.func.jvp(attend, primals, tangents)
    close(out, ref_out, dtype)
    close(tangent, ref_tangent, dtype)
    (out2, lse), (tangent2, lse_tangent) = torch.func.jvp(attend_with_lse, primals, tangents)
    assert torch.equal(out2, out) and torch.equal(tangent2, tangent)
    assert lse.dtype == torch.float32 and lse.shape == (1, 4, 67)
    assert not lse_tangent.any()

    fwd_ad = torch.autograd.forward_ad
    with fwd_ad.dual_level():
        duals = [fwd_ad.make_dual(p, t) for p, t in zip(primals, tangents)]
        p_out, t_out = fwd_ad.unpack_dual(attend(*duals))
        assert torch.equal(p_out, out) and torch.equal(t_out, tangent)
        dual_out, dual_lse = attend_with_lse(*duals)
        p2, t2 = fwd_ad.unpack_dual(dual_out)
        l2, lt2 = fwd_ad.unpack_dual(dual_lse)
        assert torch.equal(p2, out) and torch.equal(t2, tangent) and torch.equal(l2, lse)
        assert lt2 is None


@pytest.mark.parametrize("dtype", DTYPES)
def test_absent_tangents(dtype):
    """None tangents are zero: every subset agrees with the oracle, in both the
    standalone and the fused kernels, and a dual on v alone matches tv-only."""
    case = (1, 35, 49, 2, 2, 64, False, None)
    q, k, v, tq, tk, tv = seeded(case, dtype)
    out, lse = flash_attention(q, k, v, return_lse=True)
    subsets = ((None, None, None), (None, None, tv), (tq, None, None), (None, tk, None), (tq, tk, None))
    for tangents in subsets:
        _, expected = orc.attention_jvp(*on_cpu64((q, k, v) + tangents))
        close(flash_attention_jvp(q, k, v, *tangents, out, lse), expected, dtype)
        close(flash_attention_fwd_jvp(q, k, v, *tangents)[2], expected, dtype)
    fwd_ad = torch.autograd.forward_ad
    with fwd_ad.dual_level():
        _, only_v = fwd_ad.unpack_dual(flash_attention(q, k, fwd_ad.make_dual(v, tv)))
    assert torch.equal(only_v, flash_attention_jvp(q, k, v, None, None, tv, out, lse))


@pytest.mark.parametrize("dtype", DTYPES)
def test_jvp_reads_the_cached_output(dtype):
    """At scale 1/sqrt(D) the standalone JVP takes O from `out`, as the
    reference's kernel does: a shifted `out` moves tO by -rowsum(H) * shift,
    and the result follows the reference's dense formula for that `out`."""
    case = (1, 200, 300, 2, 2, 64, False, None)
    q, k, v, tq, tk, tv = seeded(case, dtype)
    out, lse = flash_attention(q, k, v, return_lse=True)
    shifted = (out.float() + 0.125).to(dtype)
    plain = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse)
    moved = flash_attention_jvp(q, k, v, tq, tk, tv, shifted, lse)
    assert not torch.equal(plain, moved)
    for cached, tangent in ((out, plain), (shifted, moved)):
        dense = orc.attention_jvp_from_forward(*(t.cpu() for t in (q, k, v, tq, tk, tv, cached, lse)))
        torch.testing.assert_close(tangent.cpu(), dense, **BOUNDS[dtype])


PEAKED = (
    (2, 64, 80, 2, 2, 32, False, 1.0),
    (1, 100, 150, 4, 2, 64, True, 0.6),   # GQA, bottom-right causal mask
    (1, 40, 300, 2, 1, 128, False, 0.35),  # MQA, several key tiles
)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", PEAKED)
def test_jvp_peaked_rows_recompute_the_output(case, dtype):
    """With scores this peaked most rows' rowsum(H)/l would amplify the cached
    O's rounding past the kernel's bound, so their tiles are redone with O
    recomputed from the same probabilities: tO no longer depends on `out` and
    stays within the tolerance of the fp64 oracle (the reference's formula
    with the cached O does not, on such rows)."""
    q, k, v, tq, tk, tv = seeded(case, dtype)
    out, lse = flash_attention(q, k, v, return_lse=True, **opts(case))
    nudged = (out.float() * (1 + 2 ** -6)).to(dtype)
    first = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, **opts(case))
    second = flash_attention_jvp(q, k, v, tq, tk, tv, nudged, lse, **opts(case))
    assert torch.equal(first, second)
    _, expected = orc.attention_jvp(*on_cpu64((q, k, v, tq, tk, tv)), **opts(case))
    close(first, expected, dtype)
    n_empty = empty_rows(case)
    if n_empty:
        assert not first[:, :n_empty].any()


@pytest.mark.parametrize("dtype", DTYPES)
def test_jvp_recompute_only_where_marked(dtype):
    """One launch with both kinds of 128-row tile: the first tile's queries are
    scaled up so its softmax is peaked (its rows are redone with O
    recomputed), the other two keep unit-normal queries (the cached O is
    used).  Every row matches the fp64 oracle; a shifted `out` moves only the
    rows of the cached-O tiles."""
    b, nq, nk, h, d = 1, 384, 256, 2, 64
    q, k, v, tq, tk, tv = seeded((b, nq, nk, h, h, d), dtype)
    q = q.clone()
    q[:, :128] = (q[:, :128].float() * 2).to(dtype)
    out, lse = flash_attention(q, k, v, return_lse=True)
    plain = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse)
    _, expected = orc.attention_jvp(*on_cpu64((q, k, v, tq, tk, tv)))
    close(plain, expected, dtype)
    shifted = flash_attention_jvp(q, k, v, tq, tk, tv, (out.float() + 0.125).to(dtype), lse)
    assert torch.equal(shifted[:, :128], plain[:, :128])
    assert not torch.equal(shifted[:, 128:], plain[:, 128:])


@pytest.mark.parametrize("dtype", DTYPES)
def test_uniform_score_shift_and_schedule_arguments(dtype):
    """A key tangent with q.tk the same for every key shifts all scores of a row
    by one constant: the softmax, hence O, does not move and tO = 0.  Explicit
    schedule arguments leave the result unchanged."""
    case = (1, 39, 73, 2, 2, 64, False, None)
    q, k, v, tq, tk, tv = seeded(case, dtype)
    constant_tk = torch.full_like(k, 0.25)
    out, lse = flash_attention(q, k, v, return_lse=True)
    zero = torch.zeros_like(q)
    torch.testing.assert_close(flash_attention_jvp(q, k, v, None, constant_tk, None, out, lse), zero,
                               **BOUNDS[dtype])
    torch.testing.assert_close(flash_attention_fwd_jvp(q, k, v, None, constant_tk, None)[2], zero,
                               **BOUNDS[dtype])
    default = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse)
    for bm, bn, threads in ((16, 32, 128), (32, 64, 128), (64, 128, 256), (128, 64, 512)):
        assert torch.equal(flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, block_m=bm, block_n=bn,
                                               threads=threads), default)
    _, expected = orc.attention_jvp(*on_cpu64((q, k, v, tq, tk, tv)))
    close(default, expected, dtype)


def test_central_difference():
    """tO against (f(x + e t) - f(x - e t)) / 2e of the fp64 dense attention."""
    case = (1, 23, 31, 4, 2, 32, True, None)
    primals_tangents = seeded(case, torch.float16)
    q, k, v = primals_tangents[:3]
    out, lse = flash_attention(q, k, v, causal=True, return_lse=True)
    tangent = flash_attention_jvp(*primals_tangents, out, lse, causal=True)
    p64, t64 = on_cpu64(primals_tangents[:3]), on_cpu64(primals_tangents[3:])
    e = 1e-4
    plus = orc.attention(*(p + e * t for p, t in zip(p64, t64)), causal=True)
    minus = orc.attention(*(p - e * t for p, t in zip(p64, t64)), causal=True)
    close(tangent, (plus - minus) / (2 * e), torch.float16)


def test_validation_messages():
    """The reference's ValueError message fragments (custom.py:160-217)."""
    q, k, v, tq, tk, tv = seeded((1, 9, 13, 2, 2, 64, False, None), torch.float16)
    out, lse = flash_attention(q, k, v, return_lse=True)
    bad_calls = {
        "lse": lambda: flash_attention_jvp(q, k, v, tq, tk, tv, out, lse.half()),
        "tq": lambda: flash_attention_jvp(q, k, v, tq[:, :-1], tk, tv, out, lse),
        "finite": lambda: flash_attention(q, k, v, softmax_scale=float("inf")),
        "positive": lambda: flash_attention(q, k, v, softmax_scale=-1.0),
        "float16": lambda: flash_attention(q.float(), k.float(), v.float()),
        "pipeline": lambda: flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, num_stages=5),
    }
    for fragment, call in bad_calls.items():
        with pytest.raises(ValueError, match=fragment):
            call()


def test_registered_operator_validates_direct_calls():
    """torch.ops.kernelforge.flash_attention_jvp called directly (bypassing the
    Python wrapper) checks its arguments before any launch, with the same
    messages; non-contiguous primals are copied, giving the wrapper's result."""
    q, k, v, tq, tk, tv = seeded((1, 9, 13, 2, 2, 64, False, None), torch.float16)
    out, lse = flash_attention(q, k, v, return_lse=True)
    op = torch.ops.kernelforge.flash_attention_jvp
    scale = 64 ** -0.5
    bad_calls = {
        "tq": lambda: op(q, k, v, tq[:, :-1], tk, tv, out, lse, scale, False, 64, 64, 128, 1),
        "tv": lambda: op(q, k, v, tq, tk, tv.float(), out, lse, scale, False, 64, 64, 128, 1),
        "out": lambda: op(q, k, v, tq, tk, tv, out[:, :-1], lse, scale, False, 64, 64, 128, 1),
        "lse": lambda: op(q, k, v, tq, tk, tv, out, lse[:, :1], scale, False, 64, 64, 128, 1),
        "must match": lambda: op(q, k[:, :-1], v, tq, tk, tv, out, lse, scale, False, 64, 64, 128, 1),
        "positive": lambda: op(q, k, v, tq, tk, tv, out, lse, -1.0, False, 64, 64, 128, 1),
    }
    for fragment, call in bad_calls.items():
        with pytest.raises(ValueError, match=fragment):
            call()
    expected = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse)
    qt = q.transpose(1, 2).contiguous().transpose(1, 2)  # same values, non-contiguous
    assert not qt.is_contiguous()
    assert torch.equal(op(qt, k, v, tq, tk, tv, out, lse, scale, False, 64, 64, 128, 1), expected)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
@pytest.mark.parametrize("stages", (1, 2, 3))
def test_masked_rows_and_partial_tiles(dtype, causal, stages):
    """Nq > Nk with a bottom-right mask: the first Nq - Nk rows see no key."""
    case = (1, 193, 97, 4, 2, 64, causal, None)
    primals_tangents = seeded(case, dtype)
    out, lse = flash_attention(*primals_tangents[:3], causal=causal, return_lse=True)
    tangent = flash_attention_jvp(*primals_tangents, out, lse, causal=causal, block_m=32, block_n=32,
                                  threads=128, num_stages=stages)
    close(tangent, orc.attention_jvp(*on_cpu64(primals_tangents), causal=causal)[1], dtype)
    if causal:
        assert not tangent[:, :96].any()


def test_graph_capture_replays():
    """A captured JVP replays bit-identically, and follows an in-place change of
    a tangent between replays."""
    case = (1, 67, 131, 4, 2, 64, True, None)
    primals_tangents = seeded(case, torch.float16)
    q, k, v, tq, tk, tv = primals_tangents
    out, lse = flash_attention(q, k, v, causal=True, return_lse=True)
    config = get_jvp_config(q, k, v, causal=True)
    eager = flash_attention_jvp(*primals_tangents, out, lse, causal=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        replayed = flash_attention_jvp(*primals_tangents, out, lse, causal=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
    tv.add_(0.03125)
    eager = flash_attention_jvp(*primals_tangents, out, lse, causal=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(replayed, eager)
    assert get_jvp_config(q, k, v, causal=True) == config


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
def test_long_key_sequence(dtype, causal):
    """Nk = 8192 keys for 5 query rows (MQA): the default and explicit schedules."""
    case = (1, 5, 8192, 2, 1, 64, causal, None)
    primals_tangents = seeded(case, dtype)
    out, lse = flash_attention(*primals_tangents[:3], causal=causal, return_lse=True)
    config = get_jvp_config(*primals_tangents[:3], causal=causal)
    assert config == dict(block_m=128, block_n=64, threads=512, num_stages=2)
    expected = orc.attention_jvp(*on_cpu64(primals_tangents), causal=causal)[1]
    close(flash_attention_jvp(*primals_tangents, out, lse, causal=causal), expected, dtype)
    close(flash_attention_jvp(*primals_tangents, out, lse, causal=causal, num_stages=1), expected, dtype)
    close(flash_attention_jvp(*primals_tangents, out, lse, causal=causal, **config), expected, dtype)


def test_reference_operator_schema():
    """torch.ops.kernelforge.flash_attention_jvp, called as the reference calls it
    (explicit zero tensors for absent tangents, schedule integers), equals the
    public function with None tangents."""
    case = (1, 48, 80, 4, 2, 128, True, None)
    q, k, v, tq, tk, tv = seeded(case, torch.bfloat16)
    out, lse = flash_attention(q, k, v, causal=True, return_lse=True)
    via_op = torch.ops.kernelforge.flash_attention_jvp(q, k, v, tq, torch.zeros_like(k), tv, out, lse,
                                                       128 ** -0.5, True, 64, 64, 128, 2)
    via_api = flash_attention_jvp(q, k, v, tq, None, tv, out, lse, causal=True)
    assert torch.equal(via_op, via_api)
    close(via_op, orc.attention_jvp(*on_cpu64((q, k, v, tq, None, tv)), causal=True)[1], torch.bfloat16)


def test_baseline_config_fused():
    """B=2, H=16, N=4096, D=128 bf16, scale 1/sqrt(D), non-causal.

    On every one of the 32 (batch, head) slices, against dense fp32
    torch.func.jvp (north-star tolerance 2e-2 / 2e-2; the oracle computes in
    fp32 on the fp32 values of the bf16 inputs): O, LSE and tO of the fused
    kernel, O and LSE of the forward, and tO of the standalone
    ``flash_attention_jvp`` (the reference's drop-in) from that forward's O
    and LSE.  Over the whole output: exact linearity in the tangents,
    finiteness.
    """
    case = (2, 4096, 4096, 16, 16, 128, False, None)
    q, k, v, tq, tk, tv = seeded(case, torch.bfloat16, seed=0)
    out, lse, tangent = flash_attention_fwd_jvp(q, k, v, tq, tk, tv)
    out_fwd, lse_fwd = flash_attention(q, k, v, return_lse=True)
    standalone = flash_attention_jvp(q, k, v, tq, tk, tv, out_fwd, lse_fwd)
    host = [t.cpu().float() for t in (q, k, v, tq, tk, tv, out, tangent, out_fwd, standalone)]
    lse_h, lse_fwd_h = lse.cpu(), lse_fwd.cpu()
    for b in range(2):
        for h in range(16):
            print(f"baseline FA slice b={b} h={h}", flush=True)
            qs, ks, vs, tqs, tks, tvs, o, t, o_fwd, t_sa = (x[b:b + 1, :, h:h + 1] for x in host)
            ref_out, ref_tangent = orc.attention_jvp(qs, ks, vs, tqs, tks, tvs)
            assert ref_out.dtype == torch.float32 and ref_tangent.dtype == torch.float32
            ref_lse = orc.attention_lse(qs, ks)
            for name, got, ref in (("fused O", o, ref_out), ("fused tO", t, ref_tangent),
                                   ("forward O", o_fwd, ref_out), ("standalone tO", t_sa, ref_tangent)):
                torch.testing.assert_close(got, ref, atol=2e-2, rtol=2e-2, msg=lambda m: f"{name} b={b} h={h}: {m}")
            for got in (lse_h, lse_fwd_h):
                torch.testing.assert_close(got[b:b + 1, h:h + 1], ref_lse, atol=2e-3, rtol=1e-4)
    torch.testing.assert_close(out.float(), out_fwd.float(), atol=1e-6, rtol=2 * torch.finfo(torch.bfloat16).eps)
    assert torch.equal(lse, lse_fwd)
    doubled = flash_attention_fwd_jvp(q, k, v, 2 * tq, 2 * tk, 2 * tv)[2]
    assert torch.equal(doubled, 2 * tangent)
    assert bool(torch.isfinite(tangent).all()) and bool(torch.isfinite(out).all())


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
    ref_out, ref_tangent = orc.attention_jvp(*on_cpu64(inputs))
    ref_lse = orc.attention_lse(*on_cpu64(inputs[:2]))
    out, lse, tangent = flash_attention_fwd_jvp(*inputs)
    out2, lse2 = flash_attention(*inputs[:3], return_lse=True)
    tangent2 = flash_attention_jvp(*inputs, out2, lse2)
    for o, t, l in ((out, tangent, lse), (out2, tangent2, lse2)):
        assert torch.isfinite(o).all() and torch.isfinite(t).all() and torch.isfinite(l).all()
        close(o, ref_out, dtype)
        close(t, ref_tangent, dtype)
        torch.testing.assert_close(l.cpu().double(), ref_lse, atol=1e-3, rtol=1e-4)
