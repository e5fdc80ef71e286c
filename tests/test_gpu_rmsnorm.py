"""RMSNorm parity on the GPU: HIP kernel (through the C ABI) vs the CPU oracle.

Mirrors rmsnorm/test.py:26-63 (seeded inputs, custom vs torch module) with
fp32 within 1e-5 relative, bf16 within 1e-2
absolute plus one bf16 ulp for summation-order rounding flips.
"""

import pytest
import torch

from kernelforge_amd.rmsnorm import RMSNorm, custom_rms_norm, original_tilelang_rms_norm
from oracle import rmsnorm as orc
from tests._util import bf16_flip_check, randn

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(rows, dim, dtype, seed=0):
    g = torch.Generator().manual_seed(seed)
    x = randn((rows, dim), dtype, gen=g)
    w = randn((dim,), dtype, gen=g, mean=1.0, std=0.1)
    return x, w


def test_cpu_oracle_config_fp32():
    """fp32 [4096, 4096], w ~ N(1, 0.1), eps 1e-6, seed 0 -> 1e-5 rel."""
    x, w = _inputs(4096, 4096, torch.float32)
    kern = custom_rms_norm(1, 4096, 4096, 1e-6, "float32")
    y = kern(x[None].to(DEV), w.to(DEV))[0].cpu()
    ref = orc.rmsnorm(x, w, 1e-6)
    torch.testing.assert_close(y, ref, rtol=1e-5, atol=0)


@pytest.mark.parametrize("hidden", [2048, 4096, 8192])
def test_bf16_llm_sweep(hidden):
    """bf16 [16384, hidden] -> 1e-2 abs (+1 ulp flips)."""
    x, w = _inputs(16384, hidden, torch.bfloat16, seed=hidden)
    y = custom_rms_norm(1, 16384, hidden, 1e-6, "bfloat16")(x[None].to(DEV), w.to(DEV))[0]
    ref = orc.rmsnorm(x, w, 1e-6)
    err, n_diff = bf16_flip_check(y, ref)
    print(f"hidden={hidden} max_abs_err={err:.3g} differing={n_diff}")
    # Against the unrounded fp64 formula the error is bounded by the two roundings.
    exact = orc.rmsnorm_fp64(x, w, 1e-6)
    assert float((y.cpu().double() - exact).abs().max()) < 0.07


@pytest.mark.parametrize("dtype", [torch.float32, torch.float16, torch.bfloat16])
@pytest.mark.parametrize("rows,dim", [(1, 8), (3, 7), (5, 100), (17, 1000), (9, 1536), (4, 6144),
                                      (2, 12288), (3, 16384), (2, 20000), (33, 128), (64, 512)])
def test_shapes_and_dtypes(rows, dim, dtype):
    x, w = _inputs(rows, dim, dtype, seed=rows * 131 + dim)
    y = custom_rms_norm(1, rows, dim, 1e-6, str(dtype).removeprefix("torch."))(
        x[None].to(DEV), w.to(DEV))[0]
    ref = orc.rmsnorm(x, w, 1e-6)
    if dtype == torch.float32:
        torch.testing.assert_close(y.cpu(), ref, rtol=1e-5, atol=0)
    elif dtype == torch.bfloat16:
        bf16_flip_check(y, ref, max_flip_frac=2e-2)
    else:
        torch.testing.assert_close(y.cpu().float(), ref.float(), atol=1e-3, rtol=2.0 ** -10)


def test_unaligned_views_and_empty():
    x, w = _inputs(7, 257, torch.bfloat16)
    xd = x.to(DEV)
    # A view whose data pointer is not 16-byte aligned takes the generic path.
    sub = xd[:, 1:]
    y = RMSNorm(256).to(DEV, torch.bfloat16)
    y.weight.data.copy_(w[1:].to(DEV))
    out = y(sub)
    bf16_flip_check(out, orc.rmsnorm(x[:, 1:], w[1:]), max_flip_frac=2e-2)
    empty = custom_rms_norm(1, 0, 64, 1e-6, "bfloat16")(torch.empty(1, 0, 64, device=DEV,
                                                                    dtype=torch.bfloat16),
                                                        torch.ones(64, device=DEV, dtype=torch.bfloat16))
    assert empty.shape == (1, 0, 64)


def test_module_matches_factory():
    x, w = _inputs(64, 1024, torch.bfloat16, seed=3)
    m = RMSNorm(1024).to(DEV, torch.bfloat16)
    m.weight.data.copy_(w.to(DEV))
    a = m(x.to(DEV).view(2, 32, 1024))
    b = custom_rms_norm(2, 32, 1024, 1e-6, "bfloat16")(x.to(DEV).view(2, 32, 1024), w.to(DEV))
    torch.testing.assert_close(a, b, atol=0, rtol=0)


def test_original_tilelang_equivalent():
    a = randn((33, 700), torch.float32, seed=5)
    b = original_tilelang_rms_norm(a.to(DEV), 1).cpu()
    torch.testing.assert_close(b, orc.rmsnorm_noweight(a), rtol=1e-5, atol=0)


def test_weight_one_gives_unit_rms():
    """Closed form: with weight = 1 every row has RMS 1 (up to eps and rounding)."""
    x = randn((128, 4096), torch.float32, seed=9) * 3.0
    y = custom_rms_norm(1, 128, 4096, 0.0, "float32")(x[None].to(DEV), torch.ones(4096, device=DEV))[0]
    rms = y.double().pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms.cpu(), torch.ones(128, dtype=torch.float64), atol=1e-5, rtol=0)


def test_shape_validation():
    k = custom_rms_norm(1, 4, 64, 1e-6, "bfloat16")
    with pytest.raises(ValueError):
        k(torch.zeros(1, 4, 32, device=DEV, dtype=torch.bfloat16),
          torch.ones(32, device=DEV, dtype=torch.bfloat16))
