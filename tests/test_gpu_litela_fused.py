"""GPU parity of the fused LiteLA projection + attention (kf_litela_fused_attn;
the general-shape form of SANA_LinearAttention/custom.py:606-809).

Checks, on shapes with ragged token tiles (N % 256 != 0), head counts that are
not a multiple of the 4-head tile, several batches, bias and both 16-bit types:
- against the unfused HIP path (projection GEMM into the packed qkv, then the
  linear-attention kernel): the same q/k/v values, so the outputs differ only
  by the fp32 summation order of the state (bf16 flips at most);
- against the fp32 oracle (oracle/sana.py: the projection in fp64/fp32 rounded
  to the dtype, then attn_matmul) at the north-star tolerance;
- determinism: identical bits on a repeat call (fixed-order reduction), also
  after the workspace served another shape.
"""

import pytest
import torch

from kernelforge_amd import _lib
from kernelforge_amd.SANA_LinearAttention.custom import linear_attention
from kernelforge_amd.SANA_LinearAttention.fused import litela_fused_attention
from kernelforge_amd.SANA_LinearAttention.projection import linear
from oracle import sana as osana

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _inputs(B, N, H, dtype, bias, seed):
    g = torch.Generator().manual_seed(seed)
    C = 32 * H
    x = torch.randn(B, N, C, generator=g).to(dtype)
    w = (torch.randn(3 * C, C, generator=g) / C ** 0.5).to(dtype)
    b = (0.5 * torch.randn(3 * C, generator=g)).to(dtype) if bias else None
    return x, w, b


CASES = [  # B, N, H
    (1, 256, 4),
    (2, 300, 6),
    (3, 77, 9),
    (1, 1024, 36),
    (2, 4096, 70),
]


@pytest.fixture(params=(3, 4), ids=("3heads", "4heads"))
def heads_per_group(request):
    """Both workgroup shapes (3 or 4 heads per tile), forced per call."""
    return request.param


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
@pytest.mark.parametrize("bias", (False, True))
def test_fused_matches_unfused_hip_path(dtype, bias, heads_per_group):
    for i, (B, N, H) in enumerate(CASES):
        print(f"fused case B={B} N={N} H={H} dtype={dtype} bias={bias} hg={heads_per_group}", flush=True)
        x, w, b = _inputs(B, N, H, dtype, bias, 10 + i)
        xd, wd = x.to(DEV), w.to(DEV)
        bd = None if b is None else b.to(DEV)
        got = litela_fused_attention(xd, wd, bd, H, heads_per_group=heads_per_group)
        qkv = linear(xd, wd, bd).reshape(B, N, 3, 32 * H)
        ref = linear_attention(qkv, H, 32, 1e-15, dtype)
        torch.cuda.synchronize()
        diff = (got.float() - ref.float()).abs()
        tol = 2e-2 * ref.float().abs() + 1e-3
        assert bool((diff <= tol).all()), float((diff - tol).max())
        # Identical q/k/v; only the state's summation order differs.
        frac = float((got != ref).float().mean())
        assert frac < 0.02, frac


@pytest.mark.parametrize("dtype", (torch.bfloat16, torch.float16))
def test_fused_matches_the_oracle(dtype, heads_per_group):
    for i, (B, N, H) in enumerate(CASES[:4]):
        x, w, b = _inputs(B, N, H, dtype, True, 30 + i)
        got = litela_fused_attention(x.to(DEV), w.to(DEV), b.to(DEV), H,
                                     heads_per_group=heads_per_group).cpu().float()
        C = 32 * H
        qkv = (torch.nn.functional.linear(x.double(), w.double(), b.double()).to(dtype)).reshape(B, N, 3, C)
        expect = osana.linear_attention(qkv, H, 32)
        torch.testing.assert_close(got, expect, atol=2e-2, rtol=2e-2)


def test_determinism_and_workspace_reuse(heads_per_group):
    B, N, H = 2, 300, 6
    x, w, b = _inputs(B, N, H, torch.bfloat16, True, 5)
    xd, wd, bd = x.to(DEV), w.to(DEV), b.to(DEV)
    hg = dict(heads_per_group=heads_per_group)
    first = litela_fused_attention(xd, wd, bd, H, **hg)
    second = litela_fused_attention(xd, wd, bd, H, **hg)
    # another shape through the same workspace in between
    x2, w2, _ = _inputs(1, 513, 5, torch.bfloat16, False, 6)
    litela_fused_attention(x2.to(DEV), w2.to(DEV), None, 5, **hg)
    third = litela_fused_attention(xd, wd, bd, H, **hg)
    torch.cuda.synchronize()
    assert torch.equal(first, second) and torch.equal(first, third)


def test_fused_rejects_on_the_host():
    x = torch.zeros(1, 16, 64, device=DEV, dtype=torch.float32)
    w = torch.zeros(192, 64, device=DEV, dtype=torch.float32)
    with pytest.raises(ValueError, match="bfloat16 or float16"):
        litela_fused_attention(x, w, None, 2)
    with pytest.raises(ValueError, match="heads"):
        litela_fused_attention(x.bfloat16(), w.bfloat16(), None, 4)
    lib = _lib.load()
    rc = lib.kf_litela_fused_attn(None, None, None, None, None, 0, 1, 16, 2, 64, 1e-15, _lib.KF_BF16, None)
    assert rc == 2 and b"head dim must be 32" in lib.kf_last_error()
