"""FlashAttention backward parity on the GPU (HIP kf_fa_bwd via autograd vs the CPU oracle).

The reference gets its gradients from flash-attn's ``_flash_attn_backward``
(flash_attention_jvp/custom.py:252-267) and checks them in
flash_attention_jvp/test.py: ``test_autograd_interfaces`` (:124-140, gradients
of ``flash_attention`` with and without ``return_lse`` against CPU fp64
autograd of ``attention``) and ``test_finite_difference_and_duality``
(:186-191, <JVP(t), c> == <t, VJP(c)>).  Both are restated here, and the
gradient check is widened to the reference's whole shape table (partial
tiles, padded head dims, GQA/MQA, bottom-right causal masks with empty rows,
head dims up to 256).  Tolerances are the reference's: bf16 3e-2/3e-2 and fp16
3e-3/1e-2 against CPU fp64; 2e-2/2e-2 against fp32 torch autograd at the
BASELINE config shape (B=2, H=16, N=4096, D=128).
"""

import pytest
import torch

from kernelforge_amd import _lib
from kernelforge_amd.flash_attention_jvp import flash_attention, flash_attention_backward, flash_attention_jvp
from oracle import fa as orc

pytestmark = pytest.mark.gpu
DEV = "cuda"
DTYPES = (torch.float16, torch.bfloat16)
# B, Nq, Nk, Hq, Hkv, D, causal, scale: flash_attention_jvp/test.py:25-38 plus
# the head dims above 128.
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
    (1, 130, 97, 2, 1, 256, True, None),
    (2, 70, 45, 2, 2, 200, False, 0.1),
    (1, 64, 256, 1, 1, 136, False, None),
    (1, 200, 200, 4, 2, 256, False, None),
    (1, 300, 300, 8, 1, 128, True, None),
    # D = 128, no mask, whole tiles: the 32-key-wavefront dK/dV kernel (GQA, MQA).
    (1, 128, 256, 4, 2, 128, False, None),
    (2, 192, 128, 2, 2, 128, False, 0.1),
    (1, 64, 384, 3, 1, 128, False, None),
)


def tolerance(dtype):
    return {torch.float16: dict(atol=3e-3, rtol=1e-2), torch.bfloat16: dict(atol=3e-2, rtol=3e-2)}[dtype]


def make_inputs(case, dtype, *, noncontiguous=False, seed=2026):
    """q, k, v and an output cotangent, drawn on the CPU from a seeded generator."""
    b, nq, nk, h, hk, d, _, _ = case
    g = torch.Generator().manual_seed(seed)
    out = []
    for shape in ((b, nq, h, d), (b, nk, hk, d), (b, nk, hk, d), (b, nq, h, d)):
        if noncontiguous:
            x = torch.randn((*shape[:-1], shape[-1] * 2), generator=g).to(dtype).to(DEV)[..., ::2]
        else:
            x = torch.randn(shape, generator=g).to(dtype).to(DEV)
        out.append(x)
    return tuple(out)


def hip_grads(q, k, v, cot, **kwargs):
    prim = tuple(x.detach().clone().requires_grad_() for x in (q, k, v))
    out = flash_attention(*prim, **kwargs)
    return torch.autograd.grad(out, prim, cot)


def fp64_grads(q, k, v, cot, **kwargs):
    prim = tuple(x.detach().cpu().double().requires_grad_() for x in (q, k, v))
    ref = orc.attention(*prim, **kwargs)
    return torch.autograd.grad(ref, prim, cot.detach().cpu().double())


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", CASES)
def test_gradients_match_fp64(case, dtype):
    q, k, v, cot = make_inputs(case, dtype)
    kwargs = dict(causal=case[-2], softmax_scale=case[-1])
    grads = hip_grads(q, k, v, cot, **kwargs)
    for name, actual, ref, primal in zip(("dq", "dk", "dv"), grads, fp64_grads(q, k, v, cot, **kwargs), (q, k, v)):
        assert actual.shape == primal.shape and actual.dtype == dtype, name
        assert torch.isfinite(actual).all(), name
        torch.testing.assert_close(actual.cpu().double(), ref, **tolerance(dtype), msg=lambda m: f"{name}: {m}")


def bwd_blocks(dout, q, k, v, out, lse, blocks, causal=False, softmax_scale=None):
    """The backward launch with the dK/dV kernel's 16-key blocks per wavefront
    forced (1 or 2; head dims up to 128) through the library's per-call test
    entry point kfm_fa_bwd_blocks; otherwise as flash_attention_backward."""
    B, Nq, Hq, D = q.shape
    Nk, Hkv = k.shape[1], k.shape[2]
    scale = D ** -0.5 if softmax_scale is None else softmax_scale
    lib = _lib.load()
    dq, dk, dv = (torch.empty_like(x, memory_format=torch.contiguous_format) for x in (q, k, v))
    ws_bytes = lib.kf_fa_bwd_workspace_bytes(B, Nq, Hq, D)
    ws = torch.empty(max(ws_bytes, 1), device=q.device, dtype=torch.uint8)
    q, k, v, dout, out, lse = (x.contiguous() for x in (q, k, v, dout, out, lse))
    rc = lib.kfm_fa_bwd_blocks(_lib.ptr(q), _lib.ptr(k), _lib.ptr(v), _lib.ptr(out), _lib.ptr(lse), _lib.ptr(dout),
                               _lib.ptr(dq), _lib.ptr(dk), _lib.ptr(dv), _lib.ptr(ws), ws_bytes, B, Nq, Nk, Hq, Hkv,
                               D, scale, int(causal), _lib.kf_dtype(q.dtype), blocks, _lib.stream_of(q))
    _lib.check(rc, "kfm_fa_bwd_blocks")
    return dq, dk, dv


def grads_blocks(q, k, v, cot, blocks, **kwargs):
    """Forward, then the backward with `blocks` key blocks per dK/dV wavefront."""
    out, lse = flash_attention(q, k, v, return_lse=True, **kwargs)
    return bwd_blocks(cot, q, k, v, out, lse, blocks, **kwargs)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("case", [c for c in CASES if c[5] <= 128])
def test_dkdv_kernels_agree(case, dtype):
    """The two-block dK/dV kernel (32 keys per wavefront, V staged in LDS)
    against the one-block kernel and the fp64 oracle.  Per key both add the
    same products in the same order, so dK and dV agree exactly."""
    print(f"dkdv kernels case={case} dtype={dtype}", flush=True)
    q, k, v, cot = make_inputs(case, dtype, seed=7)
    kwargs = dict(causal=case[-2], softmax_scale=case[-1])
    one = grads_blocks(q, k, v, cot, 1, **kwargs)
    two = grads_blocks(q, k, v, cot, 2, **kwargs)
    ref = fp64_grads(q, k, v, cot, **kwargs)
    for name, a, b, r in zip(("dq", "dk", "dv"), one, two, ref):
        torch.testing.assert_close(b, a, atol=0, rtol=0, msg=lambda m: f"{name}: {m}")
        torch.testing.assert_close(b.cpu().double(), r, **tolerance(dtype), msg=lambda m: f"{name}: {m}")


@pytest.mark.parametrize("d", (32, 64, 128))
def test_dkdv_two_block_kernel_long_gqa(d):
    """Several multi-block workgroups per head (256 keys, 512 at D = 32) with a
    partial last one, GQA group of 4, causal and not: the multi-block kernel
    against the one-block kernel."""
    for causal in (False, True):
        case = (1, 700, 1100, 8, 2, d, causal, None)
        print(f"dkdv long case={case}", flush=True)
        q, k, v, cot = make_inputs(case, torch.bfloat16, seed=8)
        one = grads_blocks(q, k, v, cot, 1, causal=causal)
        two = grads_blocks(q, k, v, cot, 2, causal=causal)
        for a, b in zip(one, two):
            torch.testing.assert_close(b, a, atol=0, rtol=0)


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("causal", (False, True))
def test_autograd_interfaces_backward(dtype, causal):
    """flash_attention_jvp/test.py:124-140 on non-contiguous inputs."""
    case = (1, 67, 41, 4, 2, 64, causal, 0.17)
    q, k, v, cot = make_inputs(case, dtype, noncontiguous=True)
    kwargs = dict(causal=causal, softmax_scale=case[-1])
    prim = tuple(x.detach().requires_grad_() for x in (q, k, v))
    actual_grads = torch.autograd.grad(flash_attention(*prim, **kwargs), prim, cot)
    stats_out, lse = flash_attention(*prim, return_lse=True, **kwargs)
    assert not lse.requires_grad
    stats_grads = torch.autograd.grad(stats_out, prim, cot)
    reference = fp64_grads(q, k, v, cot, **kwargs)
    for actual, stats, ref in zip(actual_grads, stats_grads, reference):
        # No atomics: the two backward launches give identical bits.
        torch.testing.assert_close(stats, actual, atol=0, rtol=0)
        torch.testing.assert_close(actual.cpu().double(), ref, **tolerance(dtype))


def test_jvp_vjp_duality():
    """<JVP(t), c> == sum <t_x, VJP(c)_x> (flash_attention_jvp/test.py:186-191)."""
    g = torch.Generator().manual_seed(2026)
    shapes = ((1, 23, 4, 32), (1, 31, 2, 32), (1, 31, 2, 32))
    q, k, v, tq, tk, tv = (torch.randn(s, generator=g).half().to(DEV) for s in (*shapes, *shapes))
    out, lse = flash_attention(q, k, v, causal=True, return_lse=True)
    tangent = flash_attention_jvp(q, k, v, tq, tk, tv, out, lse, causal=True)
    cot = torch.randn(out.shape, generator=g).half().to(DEV)
    grads = hip_grads(q, k, v, cot, causal=True)
    lhs = (tangent.float() * cot.float()).sum()
    rhs = sum((gr.float() * t.float()).sum() for gr, t in zip(grads, (tq, tk, tv)))
    torch.testing.assert_close(lhs, rhs, atol=2e-2, rtol=1e-2)


@pytest.mark.parametrize("blocks", (1, 2))
@pytest.mark.parametrize("dtype", DTYPES)
def test_deterministic_and_standalone(dtype, blocks):
    """Repeated backward passes give identical bits (GQA group of 4 summed in a
    fixed order) with both dK/dV kernels, and the standalone entry point
    matches autograd."""
    case = (2, 150, 170, 8, 2, 64, False, None)
    q, k, v, cot = make_inputs(case, dtype)
    first = grads_blocks(q, k, v, cot, blocks)
    second = grads_blocks(q, k, v, cot, blocks)
    out, lse = flash_attention(q, k, v, return_lse=True)
    standalone = flash_attention_backward(cot, q, k, v, out, lse)
    autograd = hip_grads(q, k, v, cot)
    for a, b, c, d in zip(first, second, standalone, autograd):
        torch.testing.assert_close(b, a, atol=0, rtol=0)
        torch.testing.assert_close(c, d, atol=0, rtol=0)
    with pytest.raises(ValueError, match="lse"):
        flash_attention_backward(cot, q, k, v, out, lse.half())
    with pytest.raises(ValueError, match="dout"):
        flash_attention_backward(cot[:, :-1], q, k, v, out, lse)


def test_empty_rows_have_zero_dq():
    """Bottom-right causal with Nq > Nk: rows i < Nq - Nk see no key (LSE = +inf)
    and get dq = 0; keys still receive the gradients of the other rows."""
    case = (1, 71, 19, 4, 1, 32, True, None)
    q, k, v, cot = make_inputs(case, torch.bfloat16)
    dq, dk, dv = hip_grads(q, k, v, cot, causal=True)
    assert torch.count_nonzero(dq[:, : 71 - 19]) == 0
    assert torch.count_nonzero(dq[:, 71 - 19:]) > 0
    assert torch.isfinite(dk).all() and torch.isfinite(dv).all()


@pytest.mark.parametrize("causal", (False, True))
def test_baseline_config_backward(causal):
    """B=2, H=16, N=4096, D=128 bf16 against fp32 torch autograd on the GPU."""
    B, H, N, D = 2, 16, 4096, 128
    g = torch.Generator().manual_seed(0)
    q, k, v, cot = (torch.randn((B, N, H, D), generator=g).to(torch.bfloat16).to(DEV) for _ in range(4))
    grads = hip_grads(q, k, v, cot, causal=causal)
    prim = tuple(x.detach().float().requires_grad_() for x in (q, k, v))
    ref = torch.autograd.grad(orc.attention(*prim, causal=causal), prim, cot.float())
    for name, actual, r in zip(("dq", "dk", "dv"), grads, ref):
        torch.testing.assert_close(actual.float(), r, atol=2e-2, rtol=2e-2, msg=lambda m: f"{name}: {m}")
        assert ((actual.float() - r).norm() / r.norm()).item() < 1e-2


@pytest.mark.parametrize("blocks", (1, 2))
def test_backward_graph_replay(blocks):
    """The backward launches (dq and dkdv kernels, torch-allocated workspace)
    replay from a captured HIP graph with the eager result, also after the
    cotangent changes in place; the program's own eager work runs between
    replays.  Both dK/dV kernels."""
    case = (1, 70, 90, 4, 2, 64, True, None)
    q, k, v, cot = make_inputs(case, torch.bfloat16)
    out, lse = flash_attention(q, k, v, causal=True, return_lse=True)
    expected = bwd_blocks(cot, q, k, v, out, lse, blocks, causal=True)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = bwd_blocks(cot, q, k, v, out, lse, blocks, causal=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for c, e in zip(captured, expected):
            torch.testing.assert_close(c, e, atol=0, rtol=0)
        flash_attention(q, k, v)  # unrelated eager work between replays
    cot.mul_(0.5)
    expected = bwd_blocks(cot, q, k, v, out, lse, blocks, causal=True)
    for _ in range(3):
        graph.replay()
        torch.cuda.synchronize()
        for c, e in zip(captured, expected):
            torch.testing.assert_close(c, e, atol=0, rtol=0)
