"""CPU tests of the Python host layer: argument validation with the reference's
message fragments (flash_attention_jvp/test.py:194-209; SANA_LinearAttention/
custom.py:350-353; rmsnorm factory dtypes), no GPU needed and no CPU fallback
(CPU tensors are rejected, never computed)."""

import pytest
import torch

from kernelforge_amd.flash_attention_jvp import custom as fa
from kernelforge_amd.rmsnorm import custom_rms_norm, rms_norm_tensor
from kernelforge_amd.SANA_LinearAttention import qkv_attn_matmul


def qkv(b=1, nq=9, nk=13, h=2, hk=2, d=64, dtype=torch.float16):
    return (torch.zeros(b, nq, h, d, dtype=dtype), torch.zeros(b, nk, hk, d, dtype=dtype),
            torch.zeros(b, nk, hk, d, dtype=dtype))


def test_fa_validation_messages():
    q, k, v = qkv()
    with pytest.raises(ValueError, match="finite"):
        fa._validate_inputs(q, k, v, float("nan"))
    with pytest.raises(ValueError, match="positive"):
        fa._validate_inputs(q, k, v, 0.0)
    with pytest.raises(ValueError, match="float16"):
        fa._validate_inputs(q.float(), k.float(), v.float(), None)
    with pytest.raises(ValueError, match="multiple of 8"):
        fa._validate_inputs(*qkv(d=12), None)
    with pytest.raises(ValueError, match="divisible"):
        fa._validate_inputs(*qkv(h=3, hk=2), None)
    with pytest.raises(ValueError, match="shape"):
        fa._validate_inputs(q[0], k, v, None)
    with pytest.raises(ValueError, match="CUDA"):
        fa._validate_inputs(q, k, v, None)  # valid but on the CPU: rejected, never computed
    with pytest.raises(ValueError, match="tq"):
        fa._prepare_tangent(q[:, :-1], q, "tq")
    assert fa._prepare_tangent(None, q, "tq") is None


def test_fa_cpu_tensors_are_rejected_not_computed():
    q, k, v = qkv()
    with pytest.raises(ValueError, match="CUDA"):
        fa.flash_attention(q, k, v)
    with pytest.raises(ValueError, match="CUDA"):
        fa.flash_attention_fwd_jvp(q, k, v, None, None, None)
    lse = torch.zeros(1, 2, 9)
    with pytest.raises(ValueError, match="CUDA"):
        fa.flash_attention_backward(q, q, k, v, q, lse)


def test_sana_factory_validation():
    with pytest.raises(ValueError, match="dim"):
        qkv_attn_matmul(1, 2, 48, 16)
    with pytest.raises(ValueError, match="dim"):
        qkv_attn_matmul(1, 2, 256, 16)
    with pytest.raises(ValueError, match="output_dtype"):
        qkv_attn_matmul(1, 2, 32, 16, output_dtype="float64")
    run = qkv_attn_matmul(1, 2, 32, 16, dtype="bfloat16")
    with pytest.raises(ValueError):
        run(torch.zeros(1, 16, 3, 64, dtype=torch.float16))
    with pytest.raises(ValueError, match="device"):
        run(torch.zeros(1, 16, 3, 64, dtype=torch.bfloat16))


def test_rmsnorm_factory_validation():
    with pytest.raises(ValueError, match="dtype"):
        custom_rms_norm(1, 4, 64, 1e-6, "int8")
    k = custom_rms_norm(1, 4, 64, 1e-6, "bfloat16")
    with pytest.raises(ValueError):
        k(torch.zeros(1, 4, 32, dtype=torch.bfloat16), torch.ones(32, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="device"):
        k(torch.zeros(1, 4, 64, dtype=torch.bfloat16), torch.ones(64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="device"):
        rms_norm_tensor(torch.zeros(3, 8), torch.ones(8))


def test_fake_impls_for_tracing():
    """The custom ops carry fake implementations (shape inference without a device)."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    with FakeTensorMode():
        q = torch.empty(1, 9, 2, 64, dtype=torch.bfloat16)
        k = torch.empty(1, 13, 2, 64, dtype=torch.bfloat16)
        out, lse = fa._fwd_fake(q, k, k, 0.1, False)
        assert out.shape == q.shape and lse.shape == (1, 2, 9) and lse.dtype == torch.float32
        o, l2, t = fa._fwd_jvp_fake(q, k, k, None, None, None, 0.1, True)
        assert t.shape == q.shape
        dq, dk, dv = fa._bwd_fake(q, q, k, k, q, lse, 0.1, False)
        assert dq.shape == q.shape and dk.shape == k.shape and dv.shape == k.shape


def test_litela_variants_on_the_host():
    """Module selection and constructor checks of the LiteLA variants
    (SANA_LinearAttention/custom.py:812-868); the joint custom operator has a
    fake implementation for tracing."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    from kernelforge_amd.SANA_LinearAttention import (CustomOpJointLiteLA, GroupedFull64QOutLiteLA, JointLiteLA,
                                                      optimized_joint_litela)
    from kernelforge_amd.SANA_LinearAttention import modules

    kw = dict(batch=1, seq_len=1024, dtype=torch.bfloat16)
    assert type(optimized_joint_litela(1152, 1152, heads=36, **kw)) is GroupedFull64QOutLiteLA
    assert type(optimized_joint_litela(256, 256, batch=2, seq_len=64, dtype=torch.bfloat16)) is JointLiteLA
    for bad in (dict(kw, batch=2), dict(kw, dtype=torch.float16), dict(kw, qk_norm=True),
                dict(kw, use_bias=True), dict(kw, heads=18)):
        with pytest.raises(ValueError, match="GroupedFull64QOutLiteLA requires"):
            GroupedFull64QOutLiteLA(1152, 1152, **bad)
    m = CustomOpJointLiteLA(256, 256, batch=2, seq_len=64, dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="device"):
        m(torch.zeros(2, 64, 256, dtype=torch.bfloat16))
    with FakeTensorMode():
        x = torch.empty(2, 64, 256, dtype=torch.bfloat16)
        w = torch.empty(768, 256, dtype=torch.bfloat16)
        pw = torch.empty(256, 256, dtype=torch.bfloat16)
        y = modules._joint_litela_op_fake(x, w, None, pw, None, None, None, 8, 32, 1e-15, 1e-5)
        assert y.shape == (2, 64, 256) and y.dtype == torch.bfloat16


def test_reference_jvp_operator_schema():
    """kernelforge::flash_attention_jvp is registered with the reference's schema
    (flash_attention_jvp/custom.py:137-157) and has a fake implementation."""
    from torch._subclasses.fake_tensor import FakeTensorMode

    op = torch.ops.kernelforge.flash_attention_jvp.default
    schema = op._schema
    names = [a.name for a in schema.arguments]
    assert names == ["q", "k", "v", "tq", "tk", "tv", "out", "lse", "scale", "causal", "block_m", "block_n",
                     "threads", "num_stages"]
    types = [str(a.type) for a in schema.arguments]
    assert types == ["Tensor"] * 8 + ["float", "bool", "int", "int", "int", "int"]
    assert [str(r.type) for r in schema.returns] == ["Tensor"]
    with FakeTensorMode():
        q = torch.empty(1, 9, 2, 64, dtype=torch.bfloat16)
        k = torch.empty(1, 13, 2, 64, dtype=torch.bfloat16)
        lse = torch.empty(1, 2, 9, dtype=torch.float32)
        t = op(q, k, k, q, k, k, q, lse, 0.125, False, 64, 64, 128, 2)
        assert t.shape == q.shape and t.dtype == q.dtype


def test_jvp_schedule_reports_the_kernel_tile():
    assert fa._schedule(64) == dict(block_m=128, block_n=64, threads=512, num_stages=2)
    assert fa._schedule(128) == dict(block_m=128, block_n=64, threads=512, num_stages=2)
    assert fa._schedule(136) == dict(block_m=64, block_n=32, threads=256, num_stages=2)
    assert fa._schedule(256) == dict(block_m=64, block_n=32, threads=256, num_stages=2)
    for key, values in fa._ALLOWED.items():
        for d in (64, 256):
            assert fa._schedule(d)[key] in values


def test_rmsnorm_module_host_side():
    """The module keeps the reference's fp32 parameter (rmsnorm/original.py:25) and
    rejects CPU tensors instead of computing them."""
    from kernelforge_amd.rmsnorm import RMSNorm

    m = RMSNorm(64, scale_factor=2.0)
    assert m.weight.dtype == torch.float32 and bool((m.weight == 2.0).all())
    with pytest.raises(ValueError, match="device"):
        m(torch.zeros(3, 64, dtype=torch.bfloat16))
    with pytest.raises(ValueError, match="shape"):
        m(torch.zeros(3, 32))
