"""RMSNorm parity on the GPU: HIP kernel (through the C ABI) vs the CPU oracle.

Mirrors rmsnorm/test.py:26-63 (seeded inputs, custom vs torch module) with
fp32 within 1e-5 relative; bf16 bit-identical to
the oracle except for at most 1e-5 of the elements plus a Poisson margin
(tests/_util.py::bf16_flip_check), each within two bf16 ulps
(summation-order flips of the first rounding point; measured 5.5e-6).  The module (rmsnorm/original.py:9-52) is checked with its
default fp32 weight on bf16 input (an fp32 result by torch's promotion) and
through its gradients.
"""

import pytest
import torch

import json
from pathlib import Path

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
    # Summation-order flips only (see bf16_flip_check); the precision of inv
    # itself is pinned bit for bit by test_inverse_sqrt_sensitive_rows.
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
        bf16_flip_check(y, ref)
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
    bf16_flip_check(out, orc.rmsnorm(x[:, 1:], w[1:]))
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


def test_reference_harness_defaults():
    """rmsnorm/test.py:26-63 as its main() runs it: bf16 x [8, 512, 1024] and a
    N(0, 1) weight, the module cast to bf16 with that weight, the two-scan fp32
    export times the weight, and the factory kernel; the latter two within
    2e-2 of the module, and the module against the CPU oracle."""
    g = torch.Generator().manual_seed(0)
    x = torch.randn(8, 512, 1024, generator=g).to(torch.bfloat16)
    w = torch.randn(1024, generator=g).to(torch.bfloat16)
    xd, wd = x.to(DEV), w.to(DEV)
    module = RMSNorm(1024).to(DEV, torch.bfloat16)
    module.weight.data.copy_(wd)
    with torch.inference_mode():
        reference = module(xd)
    assert reference.dtype == torch.bfloat16
    original = original_tilelang_rms_norm(xd.reshape(-1, 1024).float(), 1).reshape_as(xd) * wd
    custom = custom_rms_norm(8, 512, 1024, module.eps, "bfloat16")(xd, wd)
    torch.testing.assert_close(original, reference.float(), rtol=2e-2, atol=2e-2)
    torch.testing.assert_close(custom.float(), reference.float(), rtol=2e-2, atol=2e-2)
    assert torch.equal(custom, reference)
    bf16_flip_check(reference.cpu().reshape(-1, 1024), orc.rmsnorm(x.reshape(-1, 1024), w, module.eps))


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


def test_inverse_sqrt_sensitive_rows():
    """Rows whose bf16 output flips if inv = 1/sqrt(mean + eps) is one fp32 ulp
    off (tests/golden/rmsnorm_inv_golden.json; exact sums of squares, so the
    summation order cannot matter): bit for bit.  An approximate reciprocal
    square root (v_rsq_f32) would miss some of them."""
    cases = json.loads((Path(__file__).resolve().parent / "golden" / "rmsnorm_inv_golden.json").read_text())
    for case in cases:
        x = torch.tensor(case["x"], dtype=torch.float64).bfloat16()
        w = torch.tensor(case["w"], dtype=torch.float64).bfloat16()
        y = torch.tensor(case["y"], dtype=torch.float64).bfloat16()
        out = custom_rms_norm(1, 1, case["dim"], case["eps"], "bfloat16")(x[None].to(DEV), w.to(DEV))[0]
        assert torch.equal(out.cpu(), y), case["eps"]


def test_double_rounding_fixture():
    """The pure-Python fixture with both bf16 rounding points (tests/golden,
    rmsnorm_bf16_golden.json): bit for bit, and not the single-rounding values."""
    cases = json.loads((Path(__file__).resolve().parent / "golden" / "rmsnorm_bf16_golden.json").read_text())
    for case in cases:
        x = torch.tensor(case["x"], dtype=torch.float64).bfloat16()
        w = torch.tensor(case["w"], dtype=torch.float64).bfloat16()
        y = torch.tensor(case["y"], dtype=torch.float64).bfloat16()
        single = torch.tensor(case["y_single"], dtype=torch.float64).bfloat16()
        out = custom_rms_norm(1, case["rows"], case["dim"], case["eps"], "bfloat16")(x[None].to(DEV), w.to(DEV))[0]
        assert torch.equal(out.cpu(), y)
        assert not torch.equal(out.cpu(), single)


@pytest.mark.parametrize("xdtype", [torch.bfloat16, torch.float16])
def test_default_module_promotes_to_fp32(xdtype):
    """RMSNorm(4096) keeps an fp32 weight (original.py:25); on 16-bit input the
    reference's `output * self.weight` returns fp32 (original.py:51-52)."""
    g = torch.Generator().manual_seed(21)
    x = randn((512, 4096), xdtype, gen=g)
    m = RMSNorm(4096).to(DEV)
    with torch.no_grad():
        m.weight.copy_((1 + 0.1 * torch.randn(4096, generator=g)).to(DEV))
    y = m(x.to(DEV))
    assert y.dtype == torch.float32
    ref = orc.rmsnorm(x, m.weight.detach().cpu(), 1e-6)
    assert ref.dtype == torch.float32
    # fp32 result of a 16-bit first rounding: equal except for summation-order
    # flips of that rounding (one 16-bit ulp of n, times |w|), whose rate is
    # ~2^-16 per element for bf16 and ~2^-13 for fp16 (finer grid).
    diff = (y.cpu() - ref).abs()
    ulp = 2.0 ** -7 if xdtype == torch.bfloat16 else 2.0 ** -10
    lam = (1e-5 if xdtype == torch.bfloat16 else 2e-4) * diff.numel()
    assert int((diff > 0).sum()) <= lam + 4 * lam ** 0.5 + 3
    assert bool((diff <= ulp * ref.abs() * 1.01 + 1e-30).all())
    torch.testing.assert_close(y.cpu(), ref, atol=1e-2, rtol=0)


@pytest.mark.parametrize("xdtype,wdtype", [(torch.bfloat16, torch.float32), (torch.float32, torch.float32),
                                           (torch.bfloat16, torch.bfloat16), (torch.float32, torch.bfloat16)])
@pytest.mark.parametrize("rows,dim", [(64, 1024), (7, 300), (2048, 4096)])
def test_module_gradients(xdtype, wdtype, rows, dim):
    """Gradients of the module (HIP backward kernel) against the reference
    module's autograd in fp64 on the CPU (oracle.rmsnorm.rmsnorm_grads)."""
    g = torch.Generator().manual_seed(rows + dim)
    x = randn((rows, dim), xdtype, gen=g)
    w = (1 + 0.1 * torch.randn(dim, generator=g)).to(wdtype)
    dy = randn((rows, dim), torch.promote_types(xdtype, wdtype), gen=g)
    m = RMSNorm(dim).to(DEV, wdtype)
    with torch.no_grad():
        m.weight.copy_(w.to(DEV))
    xd = x.to(DEV).requires_grad_(True)
    y = m(xd)
    y.backward(dy.to(DEV))
    dx_ref, dw_ref = orc.rmsnorm_grads(x.double(), w.double(), dy.double(), 1e-6)
    assert xd.grad.dtype == xdtype and m.weight.grad.dtype == wdtype
    tol = dict(atol=2e-2, rtol=2e-2) if torch.bfloat16 in (xdtype, wdtype) else dict(atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(xd.grad.cpu().double(), dx_ref, **tol)
    # dw sums `rows` products: scale the absolute bound with sqrt(rows).
    torch.testing.assert_close(m.weight.grad.cpu().double(), dw_ref, atol=tol["atol"] * rows ** 0.5,
                               rtol=tol["rtol"])
    # deterministic: a second backward gives the same bits
    xd2 = x.to(DEV).requires_grad_(True)
    m.weight.grad = None
    m(xd2).backward(dy.to(DEV))
    assert torch.equal(xd2.grad, xd.grad)
    dw1 = m.weight.grad.clone()
    m.weight.grad = None
    m(x.to(DEV).requires_grad_(True)).backward(dy.to(DEV))
    assert torch.equal(m.weight.grad, dw1)


def test_module_gradients_through_a_residual_block():
    """A pre-norm residual block: gradients reach x through both paths and the
    weight through the norm (the module is not detached)."""
    g = torch.Generator().manual_seed(5)
    x = randn((32, 256), torch.float32, gen=g).to(DEV).requires_grad_(True)
    m = RMSNorm(256).to(DEV)
    lin = torch.nn.Linear(256, 256).to(DEV)
    (x + lin(m(x))).square().sum().backward()
    assert m.weight.grad is not None and bool(m.weight.grad.abs().sum() > 0)
    x_ref = x.detach().cpu().double().requires_grad_(True)
    w_ref = m.weight.detach().cpu().double().requires_grad_(True)
    lin_ref = torch.nn.Linear(256, 256).double()
    lin_ref.load_state_dict({k: v.detach().cpu().double() for k, v in lin.state_dict().items()})
    normed = x_ref * torch.rsqrt(x_ref.pow(2).mean(-1, keepdim=True) + 1e-6) * w_ref
    (x_ref + lin_ref(normed)).square().sum().backward()
    torch.testing.assert_close(x.grad.cpu().double(), x_ref.grad, atol=1e-3, rtol=1e-3)
    torch.testing.assert_close(m.weight.grad.cpu().double(), w_ref.grad, atol=1e-3, rtol=1e-3)


@pytest.mark.parametrize("dtype", (torch.float32, torch.bfloat16, torch.float16))
def test_norm_method(dtype):
    """``RMSNorm._norm(x)`` (rmsnorm/original.py:27-38) on the HIP kernel:
    ``x * rsqrt(mean(x^2, -1) + eps)`` in x's dtype.  fp32: within 1e-5 of the
    fp64 closed form; 16-bit: within one rounding of it (2^-8 relative for
    bf16, 2^-11 for fp16), since the kernel computes in fp32 and rounds
    once.  The rows also have unit RMS, and forward equals
    ``_norm(x.float()).type_as(x) * weight`` (original.py:51-52)."""
    g = torch.Generator().manual_seed(5)
    x = (3 * torch.randn(37, 1000, generator=g)).to(dtype)
    m = RMSNorm(1000, scale_factor=1.0, eps=1e-6).to(DEV)
    with torch.no_grad():
        m.weight.copy_(1 + 0.1 * torch.randn(1000, generator=g))
    got = m._norm(x.to(DEV))
    assert got.dtype == dtype and got.shape == x.shape
    xd = x.double()
    closed = xd * torch.rsqrt(xd.pow(2).mean(-1, keepdim=True) + 1e-6)
    rel = {torch.float32: 1e-5, torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11}[dtype]
    torch.testing.assert_close(got.cpu().double(), closed, rtol=rel, atol=1e-30)
    rms = got.cpu().double().pow(2).mean(-1).sqrt()
    torch.testing.assert_close(rms, torch.ones_like(rms), rtol=4 * rel, atol=0)
    composed = m._norm(x.to(DEV).float()).type_as(x.to(DEV)) * m.weight
    # equal up to a summation-order flip of the 16-bit rounding point
    torch.testing.assert_close(composed, m(x.to(DEV)), rtol=2.0 ** -7, atol=0)
    # differentiable in x, like the reference's torch expression
    xg = x.to(DEV).float().requires_grad_()
    m._norm(xg).sum().backward()
    xr = x.float().requires_grad_()
    (xr * torch.rsqrt(xr.pow(2).mean(-1, keepdim=True) + 1e-6)).sum().backward()
    torch.testing.assert_close(xg.grad.cpu(), xr.grad, rtol=1e-4, atol=1e-5)
