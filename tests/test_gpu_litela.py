"""GPU parity of the LiteLA modules and the in-place strided RMSNorm (qk_norm).

Modules: SANA_LinearAttention/original.py:65-145 (LiteLA, with the rotary
embedding of :136-138), custom.py:391-454 (CustomLiteLA), custom.py:526-592
(JointLiteLA), custom.py:83-85 (qkv_projection), original.py:14-58
(apply_rotary_emb), custom.py:864-945 (CustomOpJointLiteLA,
CUDAGraphJointLiteLA, optimized_joint_litela) and custom.py:812-861
(GroupedFull64QOutLiteLA, checked at its one shape).  The custom-operator and
graph tests follow SANA_LinearAttention/test.py:120-150.  The oracle (oracle/sana.py:lite_la_forward) restates
original.py:119-145 on the CPU with the fp32 attention; the projected qkv is
rounded to the module dtype the way the GPU GEMM's 16-bit output is.
"""

import pytest
import torch

from kernelforge_amd.rmsnorm.custom import rms_norm_rows_
from kernelforge_amd import _lib
from kernelforge_amd.SANA_LinearAttention import (CUDAGraphJointLiteLA, CustomLiteLA, CustomOpJointLiteLA,
                                                  GroupedFull64QOutLiteLA, JointLiteLA, LiteLA, apply_rotary_emb,
                                                  optimized_joint_litela, qkv_projection)
from oracle import rmsnorm as orms
from oracle import sana as osana

pytestmark = pytest.mark.gpu
DEV = "cuda"


@pytest.fixture(autouse=True)
def _forward_only():
    """The modules are forward-only (no backward kernels): every test runs under
    no_grad, as the reference's tests run under inference_mode."""
    with torch.no_grad():
        yield


def test_modules_refuse_to_record_autograd():
    m = LiteLA(64, 64).to(DEV)
    x = torch.randn(1, 16, 64, device=DEV)
    with torch.enable_grad():
        with pytest.raises(RuntimeError, match="no backward"):
            m(x)
        m.requires_grad_(False)
        with pytest.raises(RuntimeError, match="no backward"):
            m(x.requires_grad_(True))
        y = m(x.detach())  # frozen module, plain input: allowed
    assert y.shape == (1, 16, 64) and not y.requires_grad


def _module_ref(m, x, qk_norm, rotary_emb=None):
    return osana.lite_la_forward(
        x.cpu(), m.qkv.weight, m.qkv.bias, m.proj.weight, m.proj.bias, m.heads, m.eps,
        m.q_norm.weight if qk_norm else None, m.k_norm.weight if qk_norm else None,
        m.q_norm.eps if qk_norm else 1e-5, qkv_dtype=x.dtype, rotary_emb=rotary_emb)


def _rope_tables(N, D, seed=4):
    """cos/sin [N, D] of per-pair angles (equal on channels 2i, 2i+1)."""
    g = torch.Generator().manual_seed(seed)
    theta = (torch.rand(N, D // 2, generator=g) * 6.0 - 3.0).repeat_interleave(2, dim=-1)
    return torch.cos(theta), torch.sin(theta)


def _close(got, ref, tol=2e-2):
    got = got.detach().cpu().float()
    torch.testing.assert_close(got, ref, atol=tol, rtol=tol)
    rel = float((got - ref).norm() / ref.norm())
    assert rel < 1e-2, rel


@pytest.mark.parametrize("qk_norm", (False, True))
@pytest.mark.parametrize("use_bias", (False, True))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_litela_matches_reference_forward(qk_norm, use_bias, dtype):
    torch.manual_seed(0)
    B, N, C = 2, 300, 8 * 32
    m = LiteLA(C, C, use_bias=use_bias, qk_norm=qk_norm).to(DEV, dtype)
    x = torch.randn(B, N, C, generator=torch.Generator().manual_seed(1)).to(dtype).to(DEV)
    _close(m(x), _module_ref(m, x, qk_norm))


def test_litela_fp32_and_head_dim_16():
    torch.manual_seed(0)
    m = LiteLA(96, 96, dim=16).to(DEV)
    assert (m.heads, m.dim) == (6, 16)
    x = torch.randn(1, 77, 96, generator=torch.Generator().manual_seed(2)).to(DEV)
    _close(m(x), _module_ref(m, x, False), tol=1e-4)


@pytest.mark.parametrize("dtype", (torch.float32, torch.bfloat16))
def test_litela_narrow_widths(dtype):
    """A module whose widths are not multiples of 8 (C = 12, three heads of
    4): both projections run on the GEMM through zero-padded operands, the
    attention on the VALU path; the forward matches the reference."""
    torch.manual_seed(0)
    m = LiteLA(12, 12, dim=4, use_bias=True).to(DEV, dtype)
    assert (m.heads, m.dim) == (3, 4)
    x = torch.randn(2, 50, 12, generator=torch.Generator().manual_seed(6)).to(dtype).to(DEV)
    _close(m(x), _module_ref(m, x, False), tol=1e-4 if dtype == torch.float32 else 2e-2)


@pytest.mark.parametrize("cls", (CustomLiteLA, JointLiteLA))
def test_custom_and_joint_modules(cls):
    torch.manual_seed(0)
    B, N, C = 1, 512, 1152  # SANA-1.6B width: 36 heads of 32
    m = cls(C, C, batch=B, seq_len=N, dtype=torch.bfloat16, qk_norm=True).to(DEV, torch.bfloat16)
    x = torch.randn(B, N, C, generator=torch.Generator().manual_seed(3)).to(torch.bfloat16).to(DEV)
    _close(m(x), _module_ref(m, x, True))
    with pytest.raises(ValueError, match="expected LiteLA input shape"):
        m(x[:, :-1])
    with pytest.raises(ValueError, match="expected LiteLA dtype"):
        m(x.float())
    rot = _rope_tables(N, 32)
    _close(m(x, rotary_emb=rot), _module_ref(m, x, True, rot))
    with pytest.raises(ValueError, match="rotary_emb"):
        m(x, rotary_emb=(torch.ones(1), torch.ones(1)))


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
def test_rope_packed_matches_oracle_bitwise(dtype):
    """kf_rope_packed against the oracle's rotation of the packed qkv: the same
    two fp32 products, one fp32 sum and one rounding, so identical bits."""
    B, N, H, D = 2, 37, 5, 32
    g = torch.Generator().manual_seed(7)
    qkv = torch.randn(B, N, 3, H * D, generator=g).to(dtype)
    cos, sin = _rope_tables(N, D)
    dev, dcos, dsin = qkv.to(DEV), cos.to(DEV), sin.to(DEV)  # kept alive across the launch
    rc = _lib.load().kf_rope_packed(_lib.ptr(dev), _lib.ptr(dcos), _lib.ptr(dsin), B, N, H, D,
                                    _lib.kf_dtype(dtype), _lib.stream_of(dev))
    _lib.check(rc, "kf_rope_packed")
    torch.testing.assert_close(dev.cpu(), osana.rope_packed(qkv, cos, sin, H), atol=0, rtol=0)


@pytest.mark.parametrize("qk_norm", (False, True))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_litela_rotary_matches_reference_forward(qk_norm, dtype):
    torch.manual_seed(0)
    B, N, C = 2, 300, 8 * 32
    m = LiteLA(C, C, qk_norm=qk_norm).to(DEV, dtype)
    x = torch.randn(B, N, C, generator=torch.Generator().manual_seed(1)).to(dtype).to(DEV)
    rot = _rope_tables(N, 32)
    out = m(x, rotary_emb=rot)
    _close(out, _module_ref(m, x, qk_norm, rot))
    assert not torch.allclose(out, m(x), atol=1e-2)


def test_apply_rotary_emb_helper():
    """The exported helper matches the oracle's apply_rotary_emb for both pair
    layouts and the complex form."""
    g = torch.Generator().manual_seed(8)
    x = torch.randn(2, 3, 32, 10, generator=g).to(torch.bfloat16)
    cos, sin = _rope_tables(10, 32)
    for dim, xx in ((-2, x), (-1, x.transpose(-1, -2).contiguous())):
        got = apply_rotary_emb(xx.to(DEV), (cos.to(DEV), sin.to(DEV)), use_real_unbind_dim=dim)
        torch.testing.assert_close(got.cpu(), osana.apply_rotary_emb(xx, (cos, sin), use_real_unbind_dim=dim),
                                   atol=0, rtol=0)
    theta = torch.rand(1, 10, 16, generator=g)
    freqs = torch.polar(torch.ones_like(theta), theta)
    xs = x.permute(0, 3, 1, 2).contiguous()
    got = apply_rotary_emb(xs.to(DEV), freqs.to(DEV), use_real=False)
    torch.testing.assert_close(got.cpu(), osana.apply_rotary_emb(xs, freqs, use_real=False), atol=1e-2, rtol=1e-2)


def test_module_validation():
    with pytest.raises(ValueError, match="unsupported attention dtype"):
        CustomLiteLA(64, 64, batch=1, seq_len=4, dtype=torch.int8)
    with pytest.raises(ValueError, match="JointLiteLA requires in_dim == out_dim"):
        JointLiteLA(64, 128, batch=1, seq_len=4, dtype=torch.bfloat16)
    m = LiteLA(64, 64).to(DEV)
    with pytest.raises(ValueError):
        m(torch.randn(2, 3, 65, device=DEV))
    with pytest.raises(ValueError):
        m(torch.randn(2, 3, 64))  # CPU input is rejected, never computed


def test_qkv_projection_factory():
    g = torch.Generator().manual_seed(4)
    B, N, C = 2, 64, 96
    x = torch.randn(B, N, C, generator=g).bfloat16()
    wt = (0.1 * torch.randn(C, 3 * C, generator=g)).bfloat16()
    kern = qkv_projection(B, N, C, "bfloat16")
    got = kern(x.to(DEV), wt.to(DEV)).cpu().float()
    ref = (x.float() @ wt.float()).bfloat16().float()
    torch.testing.assert_close(got, ref, atol=2e-2, rtol=2e-2)
    with pytest.raises(ValueError):
        kern(x.to(DEV), wt[:, :-1].to(DEV))


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
def test_rms_norm_rows_in_place_on_packed_parts(dtype):
    g = torch.Generator().manual_seed(6)
    B, N, C = 3, 50, 2240
    qkv = torch.randn(B, N, 3, C, generator=g).to(dtype)
    w = (1 + 0.1 * torch.randn(C, generator=g)).to(dtype)
    dq = qkv.to(DEV)
    rms_norm_rows_(dq[:, :, 0], w.to(DEV), 1e-5)
    got = dq.cpu()
    ref_q = orms.rmsnorm(qkv[:, :, 0], w, 1e-5)
    if dtype == torch.float32:
        torch.testing.assert_close(got[:, :, 0], ref_q, rtol=1e-5, atol=0)
    else:
        torch.testing.assert_close(got[:, :, 0].float(), ref_q.float(), atol=1e-2, rtol=2 ** -6)
    # the k and v parts are untouched
    assert torch.equal(got[:, :, 1:], qkv[:, :, 1:])


def test_rms_norm_rows_rejects_uneven_rows():
    x = torch.randn(4, 6, 16, device=DEV)[:, ::2]  # rows evenly spaced
    rms_norm_rows_(x, torch.ones(16, device=DEV))
    y = torch.randn(4, 6, 16, device=DEV)[:3, :5]  # row spacing jumps between dim 0 blocks
    with pytest.raises(ValueError):
        rms_norm_rows_(y, torch.ones(16, device=DEV))


def _joint_pair(cls, B, N, C, qk_norm, seed=0):
    torch.manual_seed(seed)
    ref = JointLiteLA(C, C, batch=B, seq_len=N, dtype=torch.bfloat16, qk_norm=qk_norm).to(DEV, torch.bfloat16)
    m = cls(C, C, batch=B, seq_len=N, dtype=torch.bfloat16, qk_norm=qk_norm).to(DEV, torch.bfloat16)
    m.load_state_dict(ref.state_dict())
    return ref, m


@pytest.mark.parametrize("qk_norm", (False, True))
def test_custom_op_joint_litela(qk_norm):
    B, N, C = 2, 256, 8 * 32
    ref, m = _joint_pair(CustomOpJointLiteLA, B, N, C, qk_norm)
    x = torch.randn(B, N, C, generator=torch.Generator().manual_seed(5)).to(torch.bfloat16).to(DEV)
    with torch.inference_mode():
        want = ref(x)
        got = m(x)
        # Dynamo traces the module as one opaque operator (no graph break).
        compiled = torch.compile(m, backend="aot_eager", fullgraph=True)(x)
    assert torch.equal(got, want)
    assert torch.equal(compiled, want)
    _close(got, _module_ref(ref, x, qk_norm))
    # rotary_emb takes the JointLiteLA path
    rot = _rope_tables(N, 32)
    with torch.inference_mode():
        assert torch.equal(m(x, rotary_emb=rot), ref(x, rotary_emb=rot))
    with pytest.raises(ValueError, match="expected LiteLA input shape"):
        m(x[:, :-1])


def test_cuda_graph_joint_litela():
    B, N, C = 1, 512, 1152
    ref, _ = _joint_pair(JointLiteLA, B, N, C, False)
    g = CUDAGraphJointLiteLA(ref)
    gen = torch.Generator().manual_seed(6)
    xs = [torch.randn(B, N, C, generator=gen).to(torch.bfloat16).to(DEV) for _ in range(3)]
    replays = []
    for x in xs + xs[:1]:
        out = g(x).clone()
        torch.cuda.synchronize()
        with torch.inference_mode():
            eager = ref(x)  # eager work between replays
        torch.cuda.synchronize()
        _close(out, eager.cpu().float(), tol=1e-2)
        replays.append(out)
    # the same input replays to the same bits
    assert torch.equal(replays[0], replays[3])
    _close(replays[1], _module_ref(ref, xs[1], False))


def test_grouped_full64_module_and_selector():
    B, N, C = 1, 1024, 1152
    m = optimized_joint_litela(C, C, batch=B, seq_len=N, dtype=torch.bfloat16, heads=36, dim=32)
    assert type(m) is GroupedFull64QOutLiteLA
    m = m.to(DEV, torch.bfloat16)
    x = torch.randn(B, N, C, generator=torch.Generator().manual_seed(7)).to(torch.bfloat16).to(DEV)
    with torch.inference_mode():
        got = m(x)
    _close(got, _module_ref(m, x, False))
    with pytest.raises(ValueError, match="rotary_emb=None"):
        m(x, rotary_emb=_rope_tables(N, 32))


@pytest.mark.parametrize("use_bias", (False, True))
@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_fused_projection_path_matches_reference(use_bias, dtype):
    """LiteLA with the fused projection + attention kernels forced
    (fused_projection=True) against the oracle and the unfused module path."""
    torch.manual_seed(0)
    B, N, C = 2, 300, 6 * 32
    m = LiteLA(C, C, use_bias=use_bias).to(DEV, dtype)
    x = torch.randn(B, N, C, generator=torch.Generator().manual_seed(8)).to(dtype).to(DEV)
    m.fused_projection = True
    fused = m(x)
    m.fused_projection = False
    unfused = m(x)
    _close(fused, _module_ref(m, x, False))
    _close(fused, unfused.cpu().float(), tol=1e-2)


def test_fused_projection_path_in_a_graph():
    """The fused path captured in a HIP graph: replays with eager work between
    them match the eager result."""
    B, N, C = 1, 512, 1152
    ref, _ = _joint_pair(JointLiteLA, B, N, C, False)
    ref.fused_projection = True
    g = CUDAGraphJointLiteLA(ref)
    gen = torch.Generator().manual_seed(9)
    xs = [torch.randn(B, N, C, generator=gen).to(torch.bfloat16).to(DEV) for _ in range(2)]
    for x in xs + xs:
        out = g(x).clone()
        torch.cuda.synchronize()
        with torch.inference_mode():
            eager = ref(x)
        torch.cuda.synchronize()
        assert torch.equal(out, eager)


# SANA_LinearAttention/test.py:97-153 (test_end_to_end) at the sizes of its
# main() (test.py:182-190): batch 1, sequence lengths 1024 / 4096 / 16384,
# channels 1152 / 2240, head dim 32, bf16 (optimized_joint_litela); fp16 runs
# JointLiteLA, as there, here at the shortest length.
END_TO_END = ([pytest.param(torch.bfloat16, n, c, id=f"bf16-{n}-{c}") for n in (1024, 4096, 16384) for c in (1152, 2240)]
              + [pytest.param(torch.float16, 1024, c, id=f"fp16-1024-{c}") for c in (1152, 2240)])


@pytest.mark.parametrize("dtype,seq_len,channels", END_TO_END)
def test_end_to_end_reference_sizes(dtype, seq_len, channels):
    """The eager module, the shape-specialised module, the opaque custom
    operator traced with fullgraph=True and the HIP graph wrapper, each against
    the CPU oracle at the reference's 2e-2 (plus the relative-norm bound)."""
    torch._dynamo.reset()
    torch.manual_seed(0)
    B, heads = 1, channels // 32
    kw = dict(heads=heads, dim=32, qk_norm=False)
    original = LiteLA(channels, channels, **kw).to(DEV, dtype)
    custom_cls = optimized_joint_litela if dtype == torch.bfloat16 else JointLiteLA
    custom = custom_cls(channels, channels, batch=B, seq_len=seq_len, dtype=dtype, **kw).to(DEV, dtype)
    custom.load_state_dict(original.state_dict())
    custom_op = CustomOpJointLiteLA(channels, channels, batch=B, seq_len=seq_len, dtype=dtype, **kw).to(DEV, dtype)
    custom_op.load_state_dict(original.state_dict())
    x = torch.randn(B, seq_len, channels, generator=torch.Generator().manual_seed(9)).to(dtype).to(DEV)
    with torch.inference_mode():
        eager = original(x).clone()
        actual = custom(x).clone()
        op_out = torch.compile(custom_op, backend="aot_eager", fullgraph=True)(x).clone()
    graph_out = CUDAGraphJointLiteLA(custom)(x).clone()
    ref = _module_ref(original, x, False)
    for got in (eager, actual, op_out, graph_out):
        _close(got, ref)
    # The operator runs the same per-shape pipeline as the eager module, and
    # the graph replays the module it captured: both bit for bit.
    assert torch.equal(op_out, eager)
    assert torch.equal(graph_out, actual)
