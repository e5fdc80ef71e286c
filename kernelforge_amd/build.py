"""Build libkernelforge_amd.so in-tree with hipcc for gfx950.

Every HIP/C++ source directly under ``csrc/`` is compiled to an object (in
parallel) and linked into ``kernelforge_amd/libkernelforge_amd.so``.  The
library has a plain C ABI (``include/kernelforge_amd.h``); Python reaches it
through ctypes (``kernelforge_amd/_lib.py``), so no torch headers are
compiled.  The hardware probes under ``csrc/probes/`` (measurement code that
bench.py runs on request) go into a library of their own,
``kernelforge_amd/libkernelforge_amd_probes.so``.

Run ``python -m kernelforge_amd.build`` (or ``__graft_entry__.build()``).
"""

from __future__ import annotations

import concurrent.futures
import os
import shutil
import subprocess
import sys
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
INCLUDE = PKG_DIR.parent / "include"
LIB_NAME = "libkernelforge_amd.so"
LIB_PATH = PKG_DIR / LIB_NAME
PROBES_PATH = PKG_DIR / "libkernelforge_amd_probes.so"
OBJ_DIR = PKG_DIR / "_build"

ARCH = "gfx950"
# Packed FP32 VALU ops are disabled for every HIP translation unit: the
# compiler then never forms v_pk_{add,mul,fma}_f32 from scalar float code.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    "-Wall",
    "-Wno-unused-function",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    f"-I{INCLUDE}",
]


def _hipcc() -> str:
    for cand in (os.environ.get("HIPCC"), shutil.which("hipcc"), "/opt/rocm/bin/hipcc"):
        if cand and Path(cand).exists():
            return cand
    raise RuntimeError("hipcc not found: the HIP toolchain is required to build kernelforge_amd")


def _sources() -> list[Path]:
    return sorted(p for p in CSRC.iterdir() if p.suffix in (".hip", ".cpp"))


def _probe_sources() -> list[Path]:
    return sorted(p for p in (CSRC / "probes").iterdir() if p.suffix == ".hip")


def _compile(hipcc: str, src: Path, verbose: bool) -> Path:
    obj = OBJ_DIR / (("probe_" if src.parent.name == "probes" else "") + src.stem + ".o")
    cmd = [hipcc, *HIPCC_FLAGS, "-c", str(src), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src.name}:\n{res.stdout}\n{res.stderr}")
    # The host pass does not know the packed-fp32 feature flag; drop that noise.
    noise = ("packed-fp32-ops", "is not a recognized feature", "warnings generated")
    warn = "\n".join(l for l in res.stderr.splitlines() if l.strip() and not any(n in l for n in noise))
    if verbose and warn:
        print(warn, file=sys.stderr)
    return obj


def _link(hipcc: str, objs: list[Path], path: Path, verbose: bool) -> None:
    tmp = path.with_suffix(".so.tmp")
    cmd = [hipcc, f"--offload-arch={ARCH}", "-shared", "-fPIC", *map(str, objs), "-o", str(tmp)]
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"link failed:\n{res.stdout}\n{res.stderr}")
    os.replace(tmp, path)


def build_library(verbose: bool = False, jobs: int | None = None) -> Path:
    """Compile every source in csrc/ and link the product library, then the
    probes library (csrc/probes/ plus the error-reporting object); return the
    product library's path."""
    hipcc = _hipcc()
    OBJ_DIR.mkdir(exist_ok=True)
    sources = _sources()
    probes = _probe_sources()
    everything = sources + probes
    jobs = jobs or min(len(everything), max(1, min(os.cpu_count() or 1, 16)))
    with concurrent.futures.ThreadPoolExecutor(max_workers=jobs) as pool:
        objs = list(pool.map(lambda s: _compile(hipcc, s, verbose), everything))
    main_objs, probe_objs = objs[:len(sources)], objs[len(sources):]
    _link(hipcc, main_objs, LIB_PATH, verbose)
    abi_obj = [o for o, src in zip(main_objs, sources) if src.name == "abi.cpp"]
    _link(hipcc, probe_objs + abi_obj, PROBES_PATH, verbose)
    return LIB_PATH


if __name__ == "__main__":
    path = build_library(verbose="-v" in sys.argv)
    print(path)
