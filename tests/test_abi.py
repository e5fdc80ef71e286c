"""CPU tests of the C ABI boundary (no GPU, no kernel launches).

The shared library must load, export every function include/kernelforge_amd.h
declares, match the ctypes signature table, and reject invalid arguments on
the host with the documented status codes before touching a device.
"""

import ctypes
import re
from pathlib import Path

import pytest

from kernelforge_amd import _lib

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "kernelforge_amd.h"


@pytest.fixture(scope="module")
def lib():
    if not _lib.LIB_PATH.exists():
        from kernelforge_amd.build import build_library

        build_library()
    return _lib.load()


def declared_functions():
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    decls = {}
    for m in re.finditer(r"\b(?:int|int64_t|const char\*)\s+(kf_\w+)\s*\(([^)]*)\)\s*;", text):
        args = [a for a in m.group(2).replace("\n", " ").split(",") if a.strip() and a.strip() != "void"]
        decls[m.group(1)] = len(args)
    return decls


def test_header_declares_the_abi():
    decls = declared_functions()
    assert {"kf_rmsnorm_fwd", "kf_linattn_fwd", "kf_fa_fwd", "kf_fa_jvp", "kf_fa_fwd_jvp", "kf_fa_bwd"} <= set(decls)


def test_every_declared_symbol_is_exported_and_bound(lib):
    decls = declared_functions()
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name, nargs in decls.items():
        assert hasattr(raw, name), f"{name} not exported"
        assert name in _lib.SIGNATURES, f"{name} missing from the ctypes table"
        assert len(_lib.SIGNATURES[name][1]) == nargs, f"{name}: arity mismatch"
    assert set(_lib.SIGNATURES) == set(decls)


def test_measurement_entry_points_are_exported_outside_the_header(lib):
    """The measurement and test hooks (kfm_*) are exported and bound but not
    part of the public ABI, and reject bad arguments on the host."""
    decls = declared_functions()
    raw = ctypes.CDLL(str(_lib.LIB_PATH))
    for name in _lib.MEASURE_SIGNATURES:
        assert name.startswith("kfm_") and hasattr(raw, name), name
        assert name not in decls
    KF_E_INVALID = 1
    bwd_args = (None,) * 9 + (None, 0, 1, 4, 4, 2, 2, 64, 0.1, 0, _lib.KF_BF16)
    for bad in (-1, 3):
        assert lib.kfm_fa_bwd_blocks(*bwd_args, bad, None) == KF_E_INVALID
    assert lib.kfm_litela_fused_attn_heads(None, None, None, None, None, 0, 1, 16, 2, 32, 1e-15, _lib.KF_BF16, 5,
                                           None) == KF_E_INVALID
    assert lib.kfm_copy(None, None, 15, 1, 64, None) == KF_E_INVALID
    assert lib.kfm_copy(None, None, 16, 1, 128, None) == KF_E_INVALID
    assert lib.kfm_copy_ex(None, None, 16, 1, 64, 4, 0, None) == KF_E_INVALID
    assert lib.kfm_copy_ex(None, None, 16, 1, 64, 0, 65537, None) == KF_E_INVALID
    assert lib.kfm_copy_ex(None, None, 0, 1, 1024, 3, 65536, None) == 0
    # no test entry point keeps global state: the old setter hooks are gone
    for gone in ("kfm_fa_bwd_key_blocks", "kfm_litela_fused_heads", "kfm_linattn_spin_limit", "kfm_coissue",
                 "kfm_lds_rate"):
        assert not hasattr(raw, gone), gone


def test_probe_library_is_separate(lib):
    """The issue-rate probes live in their own library, not in the product's."""
    if not _lib.PROBES_PATH.exists():
        pytest.skip("probe library not built")
    probes = _lib.load_probes()
    assert probes.kfm_coissue(None, None, 4, 1, 0, 0, 2, None) == 1
    assert probes.kfm_lds_rate(None, None, 1, 0, 1, 0, None) == 1


def split_plan(lib, n, splits, align, max_members):
    plan = (ctypes.c_int64 * 2)()
    assert lib.kfm_linattn_split_plan(n, splits, align, max_members, plan) == 0
    return plan[0], plan[1]


def test_linattn_split_plan_arithmetic(lib):
    """The split plan behind kf_linattn_fwd: the request is cut to the
    sequence length and to the fused kernel's resident capacity, then every
    split takes whole tiles; the effective count never exceeds the cut
    request, the splits cover the sequence, and none is empty."""
    # the regression case: N = 40000, 400 requested, 256 resident workgroups
    assert split_plan(lib, 40000, 400, 128, 256) == (256, 157)
    # without the cut the 400 requests give 313 members, more than 256 slots
    assert split_plan(lib, 40000, 400, 128, 1 << 20) == (128, 313)
    assert split_plan(lib, 4096, 3, 128, 256) == (1408, 3)
    assert split_plan(lib, 16384, 7, 128, 256) == (2432, 7)
    assert split_plan(lib, 5, 64, 128, 256) == (128, 1)
    assert split_plan(lib, 1000, 1, 32, 65535) == (1024, 1)
    for n in (1, 127, 128, 129, 4096, 40000, 1 << 20):
        for req in (1, 2, 3, 7, 64, 255, 256, 257, 400, 100000):
            for cap in (1, 7, 256, 512):
                length, eff = split_plan(lib, n, req, 128, cap)
                assert length % 128 == 0 and length > 0
                assert 1 <= eff <= min(req, cap, n)
                assert (eff - 1) * length < n <= eff * length  # covered, last split non-empty
    assert lib.kfm_linattn_split_plan(0, 1, 128, 1, (ctypes.c_int64 * 2)()) == 1


def test_version_and_status_strings(lib):
    assert lib.kf_abi_version() == _lib.ABI_VERSION == 1
    assert lib.kf_status_string(0) == b"KF_OK"
    assert lib.kf_status_string(3) == b"KF_E_WORKSPACE"
    assert lib.kf_status_string(5) == b"KF_E_INCOMPLETE"
    assert lib.kf_status_string(99) == b"KF_E_UNKNOWN"


def test_host_side_validation_needs_no_device(lib):
    null = ctypes.c_void_p(0)
    # empty problems succeed without a launch
    assert lib.kf_rmsnorm_fwd(null, null, null, 0, 64, 1e-6, _lib.KF_BF16, null) == 0
    # invalid shapes / dtypes are rejected with a message
    assert lib.kf_rmsnorm_fwd(null, null, null, 4, 0, 1e-6, _lib.KF_BF16, null) == 1
    assert b"bad shape" in lib.kf_last_error()
    assert lib.kf_rmsnorm_fwd(null, null, null, 4, 64, 1e-6, 7, null) == 1
    assert lib.kf_linattn_fwd(null, null, null, 0, 1, 8, 2, 48, 1, 1e-15, _lib.KF_BF16, _lib.KF_F32, null) == 1
    assert b"dim" in lib.kf_last_error()
    assert lib.kf_linattn_fwd(null, null, null, 0, 0, 8, 2, 32, 1, 1e-15, _lib.KF_BF16, _lib.KF_F32, null) == 0
    # the no-allocation entry point validates before it resolves its scratch
    assert lib.kf_linattn_fwd_noalloc(null, null, 1, 8, 2, 48, 1, 1e-15, _lib.KF_BF16, _lib.KF_F32, null) == 1
    assert b"dim" in lib.kf_last_error()
    assert lib.kf_linattn_attn_matmul(null, null, null, 0, 1, 8, 2, 32, 1, 1e-15, 9, null) == 1
    assert lib.kf_linattn_check(null, 0, null) == 3
    assert lib.kf_fa_fwd(null, null, null, null, null, 1, 4, 4, 2, 2, 12, 0.3, 0, _lib.KF_BF16, null) == 1
    assert b"multiple of 8" in lib.kf_last_error()
    assert lib.kf_fa_fwd(null, null, null, null, null, 1, 4, 4, 3, 2, 64, 0.3, 0, _lib.KF_BF16, null) == 1
    assert lib.kf_fa_fwd_jvp(null, null, null, null, null, null, null, null, null,
                             1, 4, 4, 2, 2, 64, -1.0, 0, _lib.KF_BF16, null) == 1
    assert b"scale" in lib.kf_last_error()
    assert lib.kf_fa_jvp(null, null, null, null, null, null, null, null, null,
                         1, 4, 4, 2, 2, 64, 0.1, 0, _lib.KF_F32, null) == 1
    bwd_args = (null,) * 9
    assert lib.kf_fa_bwd(*bwd_args, null, 0, 1, 4, 4, 3, 2, 64, 0.1, 0, _lib.KF_BF16, null) == 1
    assert b"multiple of Hkv" in lib.kf_last_error()
    assert lib.kf_fa_bwd(*bwd_args, null, 0, 1, 4, 4, 2, 2, 264, 0.1, 0, _lib.KF_BF16, null) == 1
    # a workspace smaller than kf_fa_bwd_workspace_bytes is refused before any launch
    need = lib.kf_fa_bwd_workspace_bytes(1, 4, 2, 64)
    assert lib.kf_fa_bwd(*bwd_args, null, need - 1, 1, 4, 4, 2, 2, 64, 0.1, 0, _lib.KF_BF16, null) == 3
    assert lib.kf_fa_bwd(*bwd_args, null, 0, 0, 4, 4, 2, 2, 64, 0.1, 0, _lib.KF_BF16, null) == 0


def test_workspace_size_formula(lib):
    # fp32 partials [B, H, splits, D+1, D] plus the reduced state [B, H, D+1, D]
    for B, H, D, S in ((2, 70, 32, 15), (1, 1, 8, 1), (3, 4, 128, 7)):
        assert lib.kf_linattn_workspace_bytes(B, H, D, S) >= 4 * B * H * (D + 1) * D * (S + 1)
    assert lib.kf_linattn_workspace_bytes(1, 1, 48, 1) == 0
    # fp32 [LSE*log2e, Delta] per (batch, head, row), rows padded to the query tile
    assert lib.kf_fa_bwd_workspace_bytes(2, 1000, 16, 128) == 8 * 2 * 16 * 1024
    assert lib.kf_fa_bwd_workspace_bytes(1, 65, 3, 256) == 8 * 3 * 128
    assert lib.kf_fa_bwd_workspace_bytes(1, 0, 3, 64) == 0
    assert lib.kf_fa_bwd_workspace_bytes(1, 8, 3, 264) == -1
