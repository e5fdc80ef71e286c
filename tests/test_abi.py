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
    for bad in (-1, 3):
        assert lib.kfm_fa_bwd_key_blocks(bad) == KF_E_INVALID
    assert lib.kfm_fa_bwd_key_blocks(0) == 0  # the per-shape choice (the default)
    assert lib.kfm_copy(None, None, 15, 1, None) == KF_E_INVALID
    assert lib.kfm_coissue(None, None, 4, 1, 0, 0, 2, None) == KF_E_INVALID
    assert lib.kfm_lds_rate(None, None, 1, 0, 1, 0, None) == KF_E_INVALID


def test_version_and_status_strings(lib):
    assert lib.kf_abi_version() == _lib.ABI_VERSION == 1
    assert lib.kf_status_string(0) == b"KF_OK"
    assert lib.kf_status_string(3) == b"KF_E_WORKSPACE"
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
