"""Compile ``csrc/*.hip`` into ``libfluxbin_amd.so`` for gfx950 with hipcc.

One shared library, ``extern "C"`` entry points only (``include/fluxbin_amd.h``);
Python reaches it through ctypes (``_lib.py``).  Run ``python -m
marlin_style_fluxbin_amd.build`` or ``__graft_entry__.build()``.
"""
from __future__ import annotations

import os
import shutil
import subprocess
import sys
from pathlib import Path

PACKAGE = Path(__file__).resolve().parent
CSRC = PACKAGE / "csrc"
LIBRARY = PACKAGE / "libfluxbin_amd.so"
ARCH = os.environ.get("FLUXBIN_OFFLOAD_ARCH", "gfx950")

# Packed fp32 ops are disabled for every HIP translation unit.
HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    "-fPIC",
    f"--offload-arch={ARCH}",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-munsafe-fp-atomics",
    "-Wno-unused-command-line-argument",
]


def hipcc() -> str:
    for candidate in (os.environ.get("HIPCC"), "/opt/rocm/bin/hipcc", shutil.which("hipcc")):
        if candidate and Path(candidate).exists():
            return candidate
    raise RuntimeError("hipcc not found: the HIP extension cannot be built")


def sources() -> list[Path]:
    """Translation units; the W3 instantiations are split by activation-row block
    so they compile in parallel."""
    return sorted(CSRC.glob("*.hip"), key=lambda p: (p.name != "capi.hip", p.name))


def compile_units() -> list[Path]:
    """The translation units hipcc compiles; w3_lut.hip holds kernel templates only
    and is included by its instantiation units, not compiled alone."""
    return [s for s in sources() if s.name != "w3_lut.hip"]


def _compile(source: Path, obj: Path, verbose: bool) -> subprocess.CompletedProcess:
    cmd = [hipcc(), *HIPCC_FLAGS, "-c", "-I", str(PACKAGE.parent / "include"),
           str(source), "-o", str(obj)]
    if verbose:
        print(" ".join(cmd), flush=True)
    return subprocess.run(cmd, capture_output=True, text=True)


def build(verbose: bool = False, jobs: int | None = None) -> Path:
    """Always recompile (the build check must compile every time it is called)."""
    from concurrent.futures import ThreadPoolExecutor

    units = compile_units()
    objdir = PACKAGE / "_build"
    objdir.mkdir(exist_ok=True)
    objects = [objdir / (s.stem + ".o") for s in units]
    jobs = jobs or min(len(units), os.cpu_count() or 4, 16)
    with ThreadPoolExecutor(max_workers=jobs) as pool:
        results = list(pool.map(lambda so: _compile(*so, verbose), zip(units, objects)))
    for source, result in zip(units, results):
        if result.returncode != 0:
            sys.stderr.write(result.stdout + result.stderr)
            raise RuntimeError(f"hipcc failed on {source.name}")
    tmp = LIBRARY.with_suffix(".so.tmp")
    link = [hipcc(), *HIPCC_FLAGS, "-shared", *map(str, objects), "-o", str(tmp)]
    result = subprocess.run(link, capture_output=True, text=True)
    if result.returncode != 0:
        sys.stderr.write(result.stdout + result.stderr)
        raise RuntimeError("hipcc failed linking libfluxbin_amd.so")
    os.replace(tmp, LIBRARY)
    return LIBRARY


if __name__ == "__main__":
    path = build(verbose=True)
    print(f"built {path}")
