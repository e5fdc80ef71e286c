"""SANA ReLU linear attention parity on the GPU (HIP via the C ABI vs the CPU oracle).

Mirrors SANA_LinearAttention/test.py:50-94 (packed qkv, custom vs eager) with
the north-star tolerance (2e-2 abs / 2e-2 rel in bf16 against an fp32
reference).  The outputs are O(1/sqrt(N)) in magnitude, so every case also
checks the relative Frobenius error, which a dropped term or a wrong index
would fail.
"""

import ctypes

import pytest
import torch

from kernelforge_amd.SANA_LinearAttention import default_splits, linear_attention, qkv_attn_matmul
from oracle import sana as orc
from tests._util import randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def rel_fro(a, b):
    a, b = a.double().cpu(), b.double().cpu()
    return float((a - b).norm() / b.norm().clamp_min(1e-30))


def check(out, ref, rel):
    torch.testing.assert_close(out.float().cpu(), ref.float(), atol=2e-2, rtol=2e-2)
    err = rel_fro(out, ref)
    assert err < rel, f"relative Frobenius error {err:.3g} >= {rel}"
    return err


@pytest.mark.parametrize("B,H,N", [(2, 70, 4096), (1, 70, 16384)])
@pytest.mark.parametrize("out_name", ["bfloat16", "float"])
def test_baseline_configs(B, H, N, out_name):
    """BASELINE configs 2 and 3: bf16 qkv ~ N(0,1), D = 32."""
    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=B * 7 + N)
    run = qkv_attn_matmul(B, H, 32, N, 1e-15, "bfloat16", out_name)
    out = run(qkv.to(DEV))
    assert out.shape == (B, N, H * 32)
    ref = orc.linear_attention(qkv, H, 32)
    err = check(out, ref, 1e-2 if out_name == "bfloat16" else 1e-4)
    print(f"B={B} H={H} N={N} out={out_name} rel_fro={err:.3g} max_abs={float((out.float().cpu()-ref).abs().max()):.3g}")


@pytest.mark.parametrize("N", [1024, 4096, 16384])
@pytest.mark.parametrize("C", [1152, 2240])
def test_reference_harness_sizes(N, C):
    """SANA_LinearAttention/test.py:50-94 at the sizes of its main()
    (test.py:182-190): batch 1, C = 1152 / 2240 (36 / 70 heads of 32), bf16 in
    and out, built with the reference's keyword arguments."""
    H = C // 32
    qkv = randn((1, N, 3, C), torch.bfloat16, seed=N + C)
    run = qkv_attn_matmul(1, H, 32, N, dtype="bfloat16", output_dtype="bfloat16")
    out = run(qkv.to(DEV))
    assert out.shape == (1, N, C) and out.dtype == torch.bfloat16
    check(out, orc.linear_attention(qkv, H, 32), 1e-2)


@pytest.mark.parametrize("B,H,N", [(1, 1, 1), (1, 2, 63), (1, 3, 65), (2, 5, 200), (3, 4, 1000),
                                   (1, 70, 2048), (2, 36, 1024)])
@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_ragged_shapes(B, H, N, dtype):
    qkv = randn((B, N, 3, H * 32), dtype, seed=N + H)
    out = linear_attention(qkv.to(DEV), H, 32, output_dtype=torch.float32)
    check(out, orc.linear_attention(qkv, H, 32), 1e-4)


@pytest.mark.parametrize("splits", [1, 2, 7, 13, 64])
def test_split_invariance(splits):
    """The split count changes only the fp32 summation order."""
    qkv = randn((1, 4096, 3, 8 * 32), torch.bfloat16, seed=11).to(DEV)
    base = linear_attention(qkv, 8, 32, output_dtype=torch.float32, splits=1)
    out = linear_attention(qkv, 8, 32, output_dtype=torch.float32, splits=splits)
    assert rel_fro(out, base) < 1e-5
    check(out, orc.linear_attention(qkv.cpu(), 8, 32), 1e-4)


@pytest.mark.parametrize("dim", [8, 16, 64, 128])
def test_generic_head_dims(dim):
    H = 256 // dim
    qkv = randn((2, 300, 3, H * dim), torch.bfloat16, seed=dim)
    out = linear_attention(qkv.to(DEV), H, dim, output_dtype=torch.float32)
    check(out, orc.linear_attention(qkv, H, dim), 1e-4)


def test_fp32_input():
    qkv = randn((1, 500, 3, 4 * 32), torch.float32, seed=3)
    run = qkv_attn_matmul(1, 4, 32, 500, 1e-15, "float", "float")
    check(run(qkv.to(DEV)), orc.linear_attention(qkv, 4, 32), 1e-5)


def test_deterministic_and_linear_in_v():
    """Two runs are bit-identical; doubling v doubles the output exactly."""
    B, H, N = 2, 70, 4096
    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=21).to(DEV)
    a = linear_attention(qkv, H, 32, output_dtype=torch.float32)
    b = linear_attention(qkv, H, 32, output_dtype=torch.float32)
    assert torch.equal(a, b)
    qkv2 = qkv.clone()
    qkv2[:, :, 2] *= 2
    c = linear_attention(qkv2, H, 32, output_dtype=torch.float32)
    assert torch.equal(c, 2 * a)


def test_negative_q_gives_zero():
    qkv = randn((1, 777, 3, 3 * 32), torch.bfloat16, seed=4)
    qkv[:, :, 0] = -qkv[:, :, 0].abs()
    out = linear_attention(qkv.to(DEV), 3, 32, output_dtype=torch.float32)
    assert torch.count_nonzero(out) == 0


def test_matches_eager_bf16_semantics():
    """The reference test compares against eager bf16 attn_matmul at 2e-2 (test.py:79-82)."""
    qkv = randn((1, 1024, 3, 36 * 32), torch.bfloat16, seed=5)
    out = qkv_attn_matmul(1, 36, 32, 1024, dtype="bfloat16", output_dtype="bfloat16")(qkv.to(DEV))
    eager = orc.linear_attention(qkv, 36, 32, fp32_attention=False)
    torch.testing.assert_close(out.float().cpu(), eager, atol=2e-2, rtol=2e-2)


def test_validation_and_splits():
    with pytest.raises(ValueError, match="dim"):
        qkv_attn_matmul(1, 2, 48, 16)
    with pytest.raises(ValueError, match="output_dtype"):
        qkv_attn_matmul(1, 2, 32, 16, output_dtype="int8")
    run = qkv_attn_matmul(1, 2, 32, 16)
    with pytest.raises(ValueError):
        run(torch.zeros(1, 17, 3, 64, device=DEV, dtype=torch.bfloat16))
    assert default_splits(2, 70, 32, 4096) >= 1


@pytest.mark.parametrize("dim", [32, 16])
def test_workspace_contract(dim):
    """A workspace is zeroed once (kf_linattn_workspace_init) and then serves
    calls of any shape it is large enough for: every call leaves its control
    words (the fused kernel's group counters) zero, and the error word that a
    timed-out group barrier would set stays zero.  An unaligned workspace is
    refused on the host."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    H = 256 // dim
    big = int(lib.kf_linattn_workspace_bytes(2, 16, dim, 13))
    ws = torch.empty(big + 256, device=DEV, dtype=torch.uint8)
    stream = _lib.stream_of(ws)
    _lib.check(lib.kf_linattn_workspace_init(_lib.ptr(ws), big, stream), "kf_linattn_workspace_init")
    for B, N, heads, splits in ((2, 1000, H, 13), (1, 333, 3, 5), (2, 4096, 16, 7), (1, 64, H, 1)):
        qkv = randn((B, N, 3, heads * dim), torch.bfloat16, seed=N).to(DEV)
        out = torch.empty(B, N, heads * dim, device=DEV, dtype=torch.float32)
        need = int(lib.kf_linattn_workspace_bytes(B, heads, dim, splits))
        assert need <= big
        for _ in range(2):
            rc = lib.kf_linattn_fwd(_lib.ptr(qkv), _lib.ptr(out), _lib.ptr(ws), big, B, N, heads, dim, splits,
                                    1e-15, _lib.KF_BF16, _lib.KF_F32, stream)
            _lib.check(rc, "kf_linattn_fwd")
        check(out, orc.linear_attention(qkv.cpu(), heads, dim), 1e-4)
        ctrl = ws[:256].view(torch.int32).cpu()
        assert not ctrl.any(), ctrl[:4]
    bad = ctypes.c_void_p(ws.data_ptr() + 16)
    rc = lib.kf_linattn_fwd(_lib.ptr(qkv), _lib.ptr(out), bad, big, 1, 64, H, dim, 1, 1e-15, _lib.KF_BF16,
                            _lib.KF_F32, stream)
    assert rc == 3 and b"aligned" in lib.kf_last_error()


def test_dirty_control_words_are_reported():
    """A workspace whose control words were never zeroed (filled with 0x7f
    here) breaks the contract: with workgroups numbered by index, the group
    counters then read above the member count, and the kernel reports it
    (error word 2, KF_E_INCOMPLETE from kf_linattn_check, NaN instead of a
    result) rather than reading incomplete partials silently.  The check
    clears the control words, and the next call is exact again."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    B, N, H, splits = 1, 1024, 4, 4
    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=23).to(DEV)
    need = int(lib.kf_linattn_workspace_bytes(B, H, 32, splits))
    ws = torch.full((need,), 0x7F, device=DEV, dtype=torch.uint8)
    stream = _lib.stream_of(ws)

    def call():
        out = torch.empty(B, N, H * 32, device=DEV, dtype=torch.float32)
        _lib.check(lib.kf_linattn_fwd(_lib.ptr(qkv), _lib.ptr(out), _lib.ptr(ws), need, B, N, H, 32, splits,
                                      1e-15, _lib.KF_BF16, _lib.KF_F32, stream), "kf_linattn_fwd")
        torch.cuda.synchronize()
        return out

    dirty = call()
    assert torch.isnan(dirty).any()
    rc = lib.kf_linattn_check(_lib.ptr(ws), need, stream)
    assert rc == 5 and b"not zero on entry" in lib.kf_last_error(), rc
    clean = call()
    assert lib.kf_linattn_check(_lib.ptr(ws), need, stream) == 0
    check(clean, orc.linear_attention(qkv.cpu(), H, 32), 1e-4)


def test_group_wait_give_up_writes_nan():
    """Failure handling of the fused kernel's group barrier, forced from the
    host: with the poll limit cut to two polls (the per-call test entry
    kfm_linattn_fwd_spin, which then also numbers the workgroups by ticket, so
    a group's members start one after another), members that arrive before
    the rest of their group stop waiting.  Each of them must set the workspace's error word and write
    NaN for its tokens; every other element must equal the normal result bit
    for bit.  The counters still return to zero, kf_linattn_check reports the
    condition (KF_E_INCOMPLETE) and clears it, and the next call is normal
    again.  Every wave exits normally (no fault, no hang)."""
    from kernelforge_amd import _lib

    lib = _lib.load()
    B, N, H, splits = 1, 2048, 4, 8
    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=21).to(DEV)
    need = int(lib.kf_linattn_workspace_bytes(B, H, 32, splits))
    ws = torch.zeros(need, device=DEV, dtype=torch.uint8)
    stream = _lib.stream_of(ws)

    def call(polls=0):
        out = torch.empty(B, N, H * 32, device=DEV, dtype=torch.float32)
        _lib.check(lib.kfm_linattn_fwd_spin(_lib.ptr(qkv), _lib.ptr(out), _lib.ptr(ws), need, B, N, H, 32, splits,
                                            1e-15, _lib.KF_BF16, _lib.KF_F32, polls, stream), "kfm_linattn_fwd_spin")
        torch.cuda.synchronize()
        return out

    ref = call()
    assert not torch.isnan(ref).any()
    assert lib.kf_linattn_check(_lib.ptr(ws), need, stream) == 0
    gave_up = False
    for _ in range(5):
        out = call(polls=2)
        ctrl = ws[:256].view(torch.int32).cpu()
        nan = torch.isnan(out)
        assert bool(nan.any()) == (int(ctrl[1]) == 1), (int(ctrl[1]), int(nan.sum()))
        assert torch.equal(out[~nan], ref[~nan])
        assert int(ctrl[0]) == 0  # the ticket counter returned to zero
        if nan.any():
            gave_up = True
            # whole token rows of a head pair: a member's split, both heads
            assert bool(nan.view(B, N, H // 2, 64).all(-1).eq(nan.view(B, N, H // 2, 64).any(-1)).all())
            rc = lib.kf_linattn_check(_lib.ptr(ws), need, stream)
            assert rc == 5 and b"stopped waiting" in lib.kf_last_error(), rc
            assert int(ws[:256].view(torch.int32).cpu()[1]) == 0  # cleared by the check
    assert gave_up, "no member stopped waiting at a two-poll limit"
    assert torch.equal(call(), ref)
    assert lib.kf_linattn_check(_lib.ptr(ws), need, stream) == 0


def test_check_status_through_python():
    """``linear_attention(check=True)`` and ``check_status`` on a normal call:
    they synchronise, find the error word clear and return."""
    from kernelforge_amd.SANA_LinearAttention import check_status

    qkv = randn((1, 1000, 3, 4 * 32), torch.bfloat16, seed=22).to(DEV)
    out = linear_attention(qkv, 4, 32, output_dtype=torch.float32, check=True)
    check_status()
    check_status(qkv.device)
    torch.testing.assert_close(out.cpu(), orc.linear_attention(qkv.cpu(), 4, 32), atol=2e-2, rtol=2e-2)


@pytest.mark.parametrize("out_dtype", (torch.float32, torch.bfloat16))
def test_splits_beyond_resident_capacity(out_dtype):
    """A split request larger than the fused kernel's resident capacity
    (256 workgroups of the fp32-output kernel on MI355X) is cut to it, so a
    group's workgroups are all resident together and none gives up: B=1,
    H=2, N=40000, splits=400 (313 splits of 128 tokens before the cut) match
    the fp32 oracle, hold no NaN, and the status check is clean."""
    B, N, H = 1, 40000, 2
    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=23)
    print(f"splits beyond capacity out={out_dtype}", flush=True)
    out = linear_attention(qkv.to(DEV), H, 32, output_dtype=out_dtype, splits=400, check=True)
    assert not torch.isnan(out).any()
    ref = orc.linear_attention(qkv, H, 32)
    torch.testing.assert_close(out.cpu().float(), ref, atol=2e-2, rtol=2e-2)
    rel = ((out.cpu().float() - ref).norm() / ref.norm()).item()
    assert rel < (1e-4 if out_dtype == torch.float32 else 1e-2), rel
    # any positive request gives a valid result, however large
    again = linear_attention(qkv.to(DEV), H, 32, output_dtype=out_dtype, splits=100000, check=True)
    torch.testing.assert_close(again.cpu().float(), ref, atol=2e-2, rtol=2e-2)


def test_ticket_numbering_beyond_residency():
    """A launch with more workgroups than the device holds at once (B=4,
    H=128: 256 head pairs x 4 splits = 1024 workgroups, above the 256-512
    slots of any output type) numbers its workgroups by ticket; it must match
    the oracle and, to fp32 summation order, the one-split launch (256
    workgroups, numbered by index)."""
    B, H, N = 4, 128, 1024
    print(f"ticket path B={B} H={H} N={N}", flush=True)
    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=31)
    ref = orc.linear_attention(qkv, H, 32)
    dev = qkv.to(DEV)
    one = linear_attention(dev, H, 32, output_dtype=torch.float32, splits=1, check=True)
    four = linear_attention(dev, H, 32, output_dtype=torch.float32, splits=4, check=True)
    assert rel_fro(four, one) < 1e-5
    check(four, ref, 1e-4)
    check(one, ref, 1e-4)


def test_graph_replay_and_streams():
    """The fused launch inside a HIP graph: replays after eager calls and
    between them give the eager bits each time (the counters return to zero
    after every replay), also from a second stream with its own workspace."""
    qkv = randn((2, 777, 3, 12 * 32), torch.bfloat16, seed=9).to(DEV)
    run = qkv_attn_matmul(2, 12, 32, 777, dtype="bfloat16", output_dtype="float")
    eager = run(qkv)
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        on_side = run(qkv)
    torch.cuda.current_stream().wait_stream(side)
    assert torch.equal(on_side, eager)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        captured = run(qkv)
    for _ in range(4):
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(captured, eager)
        assert torch.equal(run(qkv), eager)


def test_concurrent_launches_oversubscribe_the_device():
    """Four launches of config A's shape on four streams at once (4 x 210
    workgroups numbered by index, against 256 slots): every group's members
    must still meet, so each result equals its eager value bit for bit and
    no launch reports an incomplete wait."""
    from kernelforge_amd.SANA_LinearAttention import check_status

    qkvs = [randn((2, 4096, 3, 70 * 32), torch.bfloat16, seed=40 + i).to(DEV) for i in range(4)]
    eager = [linear_attention(x, 70, 32, output_dtype=torch.bfloat16, check=True) for x in qkvs]
    streams = [torch.cuda.Stream() for _ in qkvs]
    outs = [None] * len(qkvs)
    for rep in range(3):
        print(f"concurrent launches, round {rep}", flush=True)
        for s in streams:
            s.wait_stream(torch.cuda.current_stream())
        for i, (x, s) in enumerate(zip(qkvs, streams)):
            with torch.cuda.stream(s):
                outs[i] = linear_attention(x, 70, 32, output_dtype=torch.bfloat16)
        for s in streams:
            torch.cuda.current_stream().wait_stream(s)
        torch.cuda.synchronize()
        check_status()
        for o, e in zip(outs, eager):
            assert torch.equal(o, e)


def _views(qkv, heads, dim):
    """q, k, v as LiteLA.forward makes them from a packed buffer (original.py:122-134,
    k transposed as forward passes it to attn_matmul, :140)."""
    B, N, _, C = qkv.shape
    q, k, v = qkv.unbind(2)
    q = q.transpose(-1, -2).reshape(B, heads, dim, N)
    k = k.transpose(-1, -2).reshape(B, heads, dim, N).transpose(-1, -2)
    v = v.transpose(-1, -2).reshape(B, heads, dim, N)
    return q, k, v


@pytest.mark.parametrize("B,H,N", [(2, 70, 4096), (1, 3, 333), (2, 1, 129)])
def test_attn_matmul_on_forward_views(B, H, N):
    """LiteLA.attn_matmul(q, k, v) (original.py:99-117) on the views of one
    packed bf16 buffer, as LiteLA.forward and the reference's harness
    (test.py:53-57) build them: the kernel reads the buffer in place and
    writes fp32 [B, h, d, N] contiguous, so the harness's .view(B, C, N)
    works; values match the fp32 oracle's attn_matmul on the same views."""
    from kernelforge_amd.SANA_LinearAttention import LiteLA
    from kernelforge_amd.SANA_LinearAttention.custom import packed_source

    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=31 + N)
    qd = qkv.to(DEV)
    q, k, v = _views(qd, H, 32)
    assert packed_source(q, k, v) is not None
    module = LiteLA(H * 32, H * 32, heads=H, dim=32)
    out = module.attn_matmul(q, k, v)
    assert out.dtype == torch.float32 and out.shape == (B, H, 32, N) and out.is_contiguous()
    ref = orc.attn_matmul(*_views(qkv, H, 32))
    check(out, ref, 1e-4)
    # the harness's reshaping of the result (test.py:74-75)
    flat = out.view(B, H * 32, N).permute(0, 2, 1)
    check(flat, orc.linear_attention(qkv, H, 32), 1e-4)


@pytest.mark.parametrize("dtype,D", [(torch.bfloat16, 32), (torch.float16, 32), (torch.float32, 32),
                                     (torch.bfloat16, 16), (torch.bfloat16, 64)])
def test_attn_matmul_separate_tensors(dtype, D):
    """Separately allocated q, k, v of ragged sizes (not views of one buffer)
    are packed once and run on the same kernels: the MFMA kernel for 16-bit
    head dim 32, the VALU path otherwise (fp32 input, other head dims)."""
    from kernelforge_amd.SANA_LinearAttention import attn_matmul
    from kernelforge_amd.SANA_LinearAttention.custom import packed_source

    B, H, N = 2, 5, 517
    g = torch.Generator().manual_seed(41 + D)
    q = torch.randn(B, H, D, N, generator=g).to(dtype)
    k = torch.randn(B, H, N, D, generator=g).to(dtype)
    v = torch.randn(B, H, D, N, generator=g).to(dtype)
    qd, kd, vd = (t.to(DEV) for t in (q, k, v))
    assert packed_source(qd, kd, vd) is None
    out = attn_matmul(qd, kd, vd)
    assert out.dtype == torch.float32 and out.shape == (B, H, D, N) and out.is_contiguous()
    check(out, orc.attn_matmul(q, k, v), 1e-4)
    # a non-contiguous k (a transposed view of [B, h, d, N]) gives the same bits
    kt = kd.transpose(-1, -2).contiguous().transpose(-1, -2)
    assert torch.equal(attn_matmul(qd, kt, vd), out)


def test_attn_matmul_matches_the_packed_entry_point():
    """attn_matmul on forward's views and qkv_attn_matmul on the same packed
    buffer run the same kernel with the same splits: identical values, one
    transposed against the other."""
    from kernelforge_amd.SANA_LinearAttention import attn_matmul

    B, H, N = 2, 6, 1000
    qkv = randn((B, N, 3, H * 32), torch.bfloat16, seed=43).to(DEV)
    a = attn_matmul(*_views(qkv, H, 32))
    b = linear_attention(qkv, H, 32, output_dtype=torch.float32)
    assert torch.equal(a.view(B, H * 32, N).permute(0, 2, 1), b)
