"""kf_linattn_fwd_noalloc through the C ABI: the same results as kf_linattn_fwd
with a caller workspace, from a static device scratch array and without any
allocation in the library.

Two calls in a row, the second with a smaller input (the scratch keeps the
first call's contents), each compared bit for bit with kf_linattn_fwd at the
same split count and with the fp32 oracle at the north-star tolerance; then
an oversized request, which must fail on the host with KF_E_WORKSPACE.
"""

import ctypes

import pytest
import torch

from kernelforge_amd import _lib
from oracle import sana as osana

pytestmark = pytest.mark.gpu
DEV = "cuda"


def _run_both(B, N, H, D, in_dtype, out_dtype, seed):
    lib = _lib.load()
    g = torch.Generator().manual_seed(seed)
    qkv = torch.randn(B, N, 3, H * D, generator=g).to(in_dtype)
    qkv_d = qkv.to(DEV)
    splits = int(lib.kf_linattn_default_splits(B, H, D, N))
    ws_bytes = int(lib.kf_linattn_workspace_bytes(B, H, D, splits))
    assert ws_bytes <= lib.kf_linattn_noalloc_max_bytes()
    ws = torch.zeros(ws_bytes, device=DEV, dtype=torch.uint8)  # control words start at zero
    ref_out = torch.empty(B, N, H * D, device=DEV, dtype=out_dtype)
    out = torch.full((B, N, H * D), float("nan"), device=DEV, dtype=out_dtype)
    kin, kout = _lib.kf_dtype(in_dtype), _lib.kf_dtype(out_dtype)
    stream = _lib.stream_of(qkv_d)
    print(f"noalloc case B={B} N={N} H={H} D={D} splits={splits}", flush=True)
    _lib.check(lib.kf_linattn_fwd(_lib.ptr(qkv_d), _lib.ptr(ref_out), _lib.ptr(ws), ws_bytes, B, N, H, D,
                                  splits, 1e-15, kin, kout, stream), "kf_linattn_fwd")
    _lib.check(lib.kf_linattn_fwd_noalloc(_lib.ptr(qkv_d), _lib.ptr(out), B, N, H, D, splits, 1e-15, kin,
                                          kout, stream), "kf_linattn_fwd_noalloc")
    torch.cuda.synchronize()
    return qkv, out, ref_out


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_twice(out_dtype):
    # First call: BASELINE config A's shape; second call: a smaller, ragged one.
    for B, N, H, D, seed in ((2, 4096, 70, 32, 1), (1, 300, 8, 32, 2)):
        qkv, out, ref_out = _run_both(B, N, H, D, torch.bfloat16, out_dtype, seed)
        assert torch.equal(out, ref_out)
        if N <= 300:
            expect = osana.linear_attention(qkv, H, D)
            torch.testing.assert_close(out.cpu().float(), expect, atol=2e-2, rtol=2e-2)


def test_noalloc_allocates_nothing_and_checks_clean():
    """A warm kf_linattn_fwd_noalloc call leaves the device's free memory
    unchanged (no allocation by the library or by torch), and
    kf_linattn_noalloc_check finds the scratch's error word clear."""
    lib = _lib.load()
    B, N, H, D = 1, 2048, 16, 32
    g = torch.Generator().manual_seed(4)
    qkv = torch.randn(B, N, 3, H * D, generator=g).to(torch.bfloat16).to(DEV)
    out = torch.empty(B, N, H * D, device=DEV, dtype=torch.bfloat16)
    stream = _lib.stream_of(qkv)

    def call():
        _lib.check(lib.kf_linattn_fwd_noalloc(_lib.ptr(qkv), _lib.ptr(out), B, N, H, D, 0, 1e-15, _lib.KF_BF16,
                                              _lib.KF_BF16, stream), "kf_linattn_fwd_noalloc")

    call()  # warm: resolves the scratch address and loads the kernels
    torch.cuda.synchronize()
    free_before, _ = torch.cuda.mem_get_info()
    for _ in range(3):
        call()
    torch.cuda.synchronize()
    free_after, _ = torch.cuda.mem_get_info()
    assert free_after == free_before, (free_before, free_after)
    assert lib.kf_linattn_noalloc_check(stream) == 0
    torch.testing.assert_close(out.cpu().float(), osana.linear_attention(qkv.cpu(), H, D), atol=2e-2, rtol=2e-2)


def test_noalloc_generic_head_dim():
    # The VALU path (head dim 64) shares the scratch the same way.
    qkv, out, ref_out = _run_both(1, 200, 4, 64, torch.float16, torch.float32, 3)
    assert torch.equal(out, ref_out)
    torch.testing.assert_close(out.cpu(), osana.linear_attention(qkv, 4, 64), atol=2e-2, rtol=2e-2)


def test_noalloc_rejects_oversized_requests_before_device_work():
    lib = _lib.load()
    null = ctypes.c_void_p(0)
    B, N, H, D = 64, 4096, 70, 32
    splits = int(lib.kf_linattn_default_splits(B, H, D, N))
    assert lib.kf_linattn_workspace_bytes(B, H, D, splits) > lib.kf_linattn_noalloc_max_bytes()
    rc = lib.kf_linattn_fwd_noalloc(null, null, B, N, H, D, splits, 1e-15, _lib.KF_BF16, _lib.KF_BF16, null)
    assert rc == 3  # KF_E_WORKSPACE
    assert b"static scratch" in lib.kf_last_error()
    # invalid arguments are refused before the scratch is touched
    assert lib.kf_linattn_fwd_noalloc(null, null, 1, 64, 2, 48, 1, 1e-15, _lib.KF_BF16, _lib.KF_BF16, null) == 1
    assert b"dim" in lib.kf_last_error()
