"""GPU parity of the SANA projection GEMM (kf_proj_gemm; the reference's
_qkv_projection and _output_projection, SANA_LinearAttention/custom.py:23-85 and
:457-523).

The reference computes ``Cast(dtype, sum_k x*W (fp32 fragment) + float(bias))``.
Two checks pin that without trusting any GPU library:

- integer-valued inputs, small enough that every fp32 partial sum is exact in
  any order: the result must equal the fp64 product rounded once to the
  dtype, bit for bit (a wrong index, a dropped or doubled K chunk, a stale LDS
  stage or a second rounding all change bits);
- random inputs: |y - y64| <= K 2^-24 sum_k |x||w| (worst-case fp32
  accumulation in any order) + half an ulp of the dtype (the one rounding),
  against the fp64 product.
"""

import ctypes

import pytest
import torch

from kernelforge_amd import _lib
from kernelforge_amd.SANA_LinearAttention.projection import (linear, linear_t, output_projection,
                                                              qkv_projection)

pytestmark = pytest.mark.gpu
DEV = "cuda"
UNIT_ROUNDOFF = {torch.bfloat16: 2.0 ** -8, torch.float16: 2.0 ** -11, torch.float32: 2.0 ** -24}


def _ints(shape, lo, hi, seed, dtype):
    g = torch.Generator().manual_seed(seed)
    return torch.randint(lo, hi + 1, shape, generator=g).to(dtype)


def _ref64(x, w, b=None):
    y = x.double() @ w.double().T
    return y if b is None else y + b.double()


def _bound(x, w, y64, dtype):
    k = x.shape[-1]
    acc = k * 2.0 ** -24 * (x.double().abs() @ w.double().abs().T)
    return acc + UNIT_ROUNDOFF[dtype] * y64.abs() + 2.0 ** -24 * (y64.abs() + 1e-30) + 6e-8


SHAPES = [  # (M, N, K): full tiles, ragged rows/columns, a K tail of one chunk, tiny
    (512, 512, 256),
    (300, 264, 1160),
    (1, 8, 8),
    (777, 1152, 1152),
    (96, 288, 96),
]


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("layout", ("nk", "kn"))
@pytest.mark.parametrize("bias", (False, True))
def test_integer_inputs_round_once_bit_exact(dtype, layout, bias):
    for i, (M, N, K) in enumerate(SHAPES):
        print(f"proj int case dtype={dtype} layout={layout} bias={bias} M={M} N={N} K={K}", flush=True)
        x = _ints((M, K), -3, 3, 10 + i, dtype)
        w = _ints((N, K), -3, 3, 20 + i, dtype)
        b = _ints((N,), -50, 50, 30 + i, dtype) if bias else None
        xd, bd = x.to(DEV), (b.to(DEV) if bias else None)
        if layout == "nk":
            y = linear(xd, w.to(DEV), bd)
        else:
            y = linear_t(xd, w.T.contiguous().to(DEV), bd)
        torch.cuda.synchronize()
        expect = _ref64(x, w, b).to(dtype)
        assert torch.equal(y.cpu(), expect), (M, N, K)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_every_tile_width(dtype):
    """The launch picks the output-tile width (320, 256, 224, 192, 160 or 128
    channels) from the shape; on a 256-CU MI355X these shapes select each of
    them (8192x6720 -> 320, 16384x2048 -> 256, 4096x6720 -> 224,
    8192x1536 -> 192, 2048x4480 -> 160, 300x264 -> 128; 320 and 256 store the
    output tile in two row bands).  K = 72 adds a one-chunk K tail."""
    K = 72
    shapes = ((8192, 6720), (16384, 2048), (4096, 6720), (8192, 1536), (2048, 4480), (300, 264))
    for i, (M, N) in enumerate(shapes):
        print(f"proj width case dtype={dtype} M={M} N={N} K={K}", flush=True)
        x = _ints((M, K), -3, 3, 40 + i, dtype)
        w = _ints((N, K), -3, 3, 50 + i, dtype)
        b = _ints((N,), -50, 50, 60 + i, dtype)
        y = linear(x.to(DEV), w.to(DEV), b.to(DEV)).cpu()
        assert torch.equal(y, _ref64(x, w, b).to(dtype)), (M, N)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
@pytest.mark.parametrize("layout", ("nk", "kn"))
def test_wide_tiles_ragged_and_banded(dtype, layout):
    """The wide tiles (320 and 256 channels) store their output through LDS in
    two (fp32: four) row bands; these shapes select them with a partial last
    row tile and a partial last column tile (16-bit nn.Linear layout:
    7999x2216 -> 320, 8000x1992 -> 256; fp32 or WeightT: 16000x2040 -> 256)."""
    K = 72
    if dtype != torch.float32 and layout == "nk":
        shapes = ((7999, 2216), (8000, 1992))
    else:
        shapes = ((16000, 2040),)
    for i, (M, N) in enumerate(shapes):
        print(f"proj wide case dtype={dtype} layout={layout} M={M} N={N} K={K}", flush=True)
        x = _ints((M, K), -3, 3, 70 + i, dtype)
        w = _ints((N, K), -3, 3, 80 + i, dtype)
        b = _ints((N,), -50, 50, 90 + i, dtype)
        xd, bd = x.to(DEV), b.to(DEV)
        if layout == "nk":
            y = linear(xd, w.to(DEV), bd)
        else:
            y = linear_t(xd, w.T.contiguous().to(DEV), bd)
        assert torch.equal(y.cpu(), _ref64(x, w, b).to(dtype)), (M, N)


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
def test_random_inputs_within_the_accumulation_bound(dtype):
    for M, N, K in ((1024, 6720, 2240), (333, 2240, 2240), (64, 3456, 1152)):
        print(f"proj random case dtype={dtype} M={M} N={N} K={K}", flush=True)
        g = torch.Generator().manual_seed(M + N + K)
        x = torch.randn(M, K, generator=g).to(dtype)
        w = (torch.randn(N, K, generator=g) / K ** 0.5).to(dtype)
        b = torch.randn(N, generator=g).to(dtype)
        y = linear(x.to(DEV), w.to(DEV), b.to(DEV)).cpu().double()
        y64 = _ref64(x, w, b)
        err = (y - y64).abs()
        bound = _bound(x, w, y64, dtype)
        assert bool((err <= bound).all()), float((err - bound).max())
        # The bound is tight enough to see one dropped 8-element K chunk.
        dropped = _ref64(x[:, 8:], w[:, 8:], b)
        assert bool(((dropped - y64).abs() > bound).any())


@pytest.mark.parametrize("n_out,bias", ((6720, False), (2240, True)))
def test_config_a_random_rows_within_the_accumulation_bound(n_out, bias):
    """Both config-A projections (x [8192, 2240] bf16, 320-wide tiles) on
    random inputs: 64 rows spread over every row tile, all columns, against
    the fp64 product and the accumulation bound."""
    M, K = 8192, 2240
    dtype = torch.bfloat16
    print(f"proj config A random rows N={n_out} bias={bias}", flush=True)
    g = torch.Generator().manual_seed(n_out)
    x = torch.randn(M, K, generator=g).to(dtype)
    w = (torch.randn(n_out, K, generator=g) / K ** 0.5).to(dtype)
    b = torch.randn(n_out, generator=g).to(dtype) if bias else None
    y = linear(x.to(DEV), w.to(DEV), b.to(DEV) if bias else None).cpu().double()
    rows = torch.randperm(M, generator=g)[:64]
    y64 = _ref64(x[rows], w, b)
    err = (y[rows] - y64).abs()
    bound = _bound(x[rows], w, y64, dtype)
    assert bool((err <= bound).all()), float((err - bound).max())


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16, torch.float32))
def test_weight_layouts_agree_bitwise(dtype):
    """The [N, K] and the prepacked [K, N] weight feed the same operands to the
    same MFMA sequence: identical bits."""
    g = torch.Generator().manual_seed(5)
    M, N, K = 700, 1400, 1160
    x = torch.randn(M, K, generator=g).to(dtype).to(DEV)
    w = torch.randn(N, K, generator=g).to(dtype).to(DEV)
    b = torch.randn(N, generator=g).to(dtype).to(DEV)
    assert torch.equal(linear(x, w, b), linear_t(x, w.T.contiguous(), b))


@pytest.mark.parametrize("ldy_pad", (12, 8))
def test_strided_rows_and_untouched_padding(ldy_pad):
    """ldx > K with NaN padding beyond K (never read) and ldy > N (padding
    columns never written), through the C ABI.  A row stride of 8 extra
    elements keeps output rows 16-byte aligned (the LDS-staged output path),
    12 does not (per-lane stores)."""
    lib = _lib.load()
    M, N, K, ldx, ldy = 300, 264, 520, 520 + 24, 264 + ldy_pad
    x = _ints((M, ldx), -3, 3, 1, torch.bfloat16)
    x[:, K:] = float("nan")
    w = _ints((N, K), -3, 3, 2, torch.bfloat16)
    xd, wd = x.to(DEV), w.to(DEV)
    y = torch.full((M, ldy), 7.0, dtype=torch.bfloat16, device=DEV)
    rc = lib.kf_proj_gemm(_lib.ptr(xd), _lib.ptr(wd), None, _lib.ptr(y), M, N, K, ldx, ldy, _lib.KF_WEIGHT_NK,
                          _lib.KF_BF16, _lib.stream_of(xd))
    _lib.check(rc, "kf_proj_gemm")
    y = y.cpu()
    assert torch.equal(y[:, :N], _ref64(x[:, :K], w).to(torch.bfloat16))
    assert bool((y[:, N:] == 7.0).all())


def test_strided_input_view():
    """linear() on a column slice of a wider buffer uses its row stride."""
    g = torch.Generator().manual_seed(9)
    big = torch.randn(2, 130, 3 * 256, generator=g).to(torch.bfloat16).to(DEV)
    w = (torch.randn(512, 256, generator=g) / 16).to(torch.bfloat16).to(DEV)
    view = big[:, :, 256:512]
    assert torch.equal(linear(view, w), linear(view.contiguous(), w))


def test_reference_factories():
    """qkv_projection / output_projection keep the reference's call signatures
    (WeightT layouts, shape and dtype checks) and match linear()."""
    B, N, C = 2, 200, 256
    g = torch.Generator().manual_seed(3)
    x = torch.randn(B, N, C, generator=g).to(torch.bfloat16).to(DEV)
    w_qkv = (torch.randn(3 * C, C, generator=g) / 16).to(torch.bfloat16).to(DEV)
    w_out = (torch.randn(C, C, generator=g) / 16).to(torch.bfloat16).to(DEV)
    b_out = torch.randn(C, generator=g).to(torch.bfloat16).to(DEV)
    qkv = qkv_projection(B, N, C, "bfloat16")(x, w_qkv.t().contiguous())
    assert qkv.shape == (B, N, 3 * C) and torch.equal(qkv, linear(x, w_qkv))
    y = output_projection(B, N, C, "bfloat16")(x, w_out.t().contiguous(), b_out)
    assert torch.equal(y, linear(x, w_out, b_out))
    with pytest.raises(ValueError, match="WeightT"):
        qkv_projection(B, N, C, "bfloat16")(x, w_qkv)
    with pytest.raises(ValueError, match="X must be"):
        output_projection(B, N, C, "bfloat16")(x[:, 1:], w_out, b_out)


def test_host_rejections():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    assert lib.kf_proj_gemm(null, null, null, null, 4, 12, 16, 16, 12, 0, _lib.KF_BF16, null) == 1
    assert b"multiples of 8" in lib.kf_last_error()
    assert lib.kf_proj_gemm(null, null, null, null, 0, 16, 16, 16, 16, 0, _lib.KF_BF16, null) == 0


@pytest.mark.parametrize("k,n", [(12, 16), (16, 12), (4, 36), (13, 7)])
def test_ragged_widths_run_padded(k, n):
    """Widths that are not multiples of 8 (the kernel's C ABI refuses them)
    run on the same kernel through zero-padded copies: integer-valued inputs
    give the exact product bit for bit, in both weight layouts, with a bias."""
    g = torch.Generator().manual_seed(k * 100 + n)
    x = torch.randint(-3, 4, (2, 37, k), generator=g).to(torch.bfloat16)
    w = torch.randint(-3, 4, (n, k), generator=g).to(torch.bfloat16)
    b = torch.randint(-3, 4, (n,), generator=g).to(torch.bfloat16)
    exact = (x.double() @ w.double().T + b.double()).to(torch.bfloat16)
    got = linear(x.to(DEV), w.to(DEV), b.to(DEV))
    assert got.shape == (2, 37, n) and got.is_contiguous()
    assert torch.equal(got.cpu(), exact)
    assert torch.equal(linear_t(x.to(DEV), w.t().contiguous().to(DEV), b.to(DEV)).cpu(), exact)
