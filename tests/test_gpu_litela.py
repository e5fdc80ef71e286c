"""GPU parity of the LiteLA modules and the in-place strided RMSNorm (qk_norm).

Modules: SANA_LinearAttention/original.py:65-145 (LiteLA), custom.py:391-454
(CustomLiteLA), custom.py:526-592 (JointLiteLA), custom.py:83-85
(qkv_projection).  The oracle (oracle/sana.py:lite_la_forward) restates
original.py:119-145 on the CPU with the fp32 attention; the projected qkv is
rounded to the module dtype the way the GPU GEMM's 16-bit output is.
"""

import pytest
import torch

from kernelforge_amd.rmsnorm.custom import rms_norm_rows_
from kernelforge_amd.SANA_LinearAttention import CustomLiteLA, JointLiteLA, LiteLA, qkv_projection
from oracle import rmsnorm as orms
from oracle import sana as osana

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _module_ref(m, x, qk_norm):
    return osana.lite_la_forward(
        x.cpu(), m.qkv.weight, m.qkv.bias, m.proj.weight, m.proj.bias, m.heads, m.eps,
        m.q_norm.weight if qk_norm else None, m.k_norm.weight if qk_norm else None,
        m.q_norm.eps if qk_norm else 1e-5, qkv_dtype=x.dtype)


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
    with pytest.raises(NotImplementedError):
        m(x, rotary_emb=(torch.ones(1), torch.ones(1)))


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
