"""The C-ABI library loads and exports exactly what include/fluxbin_amd.h declares.

CPU-only: argument validation returns FX_EINVAL before any device call, so no
kernel is launched here.
"""
import ctypes
import re
from pathlib import Path

import pytest

from marlin_style_fluxbin_amd import _lib

HEADER = Path(__file__).resolve().parents[1] / "include" / "fluxbin_amd.h"


def declared_functions():
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(fx_[a-z0-9_]+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    lib = _lib.library()
    names = declared_functions()
    assert "fx_w3_gemv" in names and "fx_w3_restore" in names
    for name in names:
        assert hasattr(lib, name), name
    assert set(names) == set(_lib.SIGNATURES), "ctypes signature table out of sync with the header"
    assert lib.fx_abi_version() == _lib.ABI_VERSION


def test_invalid_arguments_fail_closed_without_launching():
    lib = _lib.library()
    rc = lib.fx_w3_gemv(None, 2, None, None, 2, None, None, None, 0, None, 1, 64, 256, 0, None)
    assert rc == 1
    assert "non-null" in lib.fx_last_error().decode()
    dummy = ctypes.c_void_p(4096)
    rc = lib.fx_w3_gemv(dummy, 2, dummy, dummy, 2, None, None, None, 0, dummy, 1, 64, 100, 0, None)
    assert rc == 1 and "multiple of 128" in lib.fx_last_error().decode()
    rc = lib.fx_w3_gemv(dummy, 2, ctypes.c_void_p(4097), dummy, 2, None, None, None, 0, dummy, 1, 64, 256, 0, None)
    assert rc == 1 and "aligned" in lib.fx_last_error().decode()
    rc = lib.fx_w3_gemv(dummy, 2, dummy, dummy, 1, None, None, None, 0, dummy, 1, 64, 256, 1, None)
    assert rc == 1 and "bf16 scales" in lib.fx_last_error().decode()
    rc = lib.fx_w3_m1_out(dummy, 2, dummy, dummy, 2, None, None, None, dummy, 1, 64, 256, 1, 300, 0, None)
    assert rc == 1 and "row_tile" in lib.fx_last_error().decode()
    # MFMA workspace: fp32 partials [splits, mb, O] only when K is split over workgroups
    assert lib.fx_w3_gemv_config_workspace_bytes(1, 4096, 4096, 8, 1, 32, 1) == 0
    assert lib.fx_w3_gemv_config_workspace_bytes(1, 64, 384, 4, 1, 4, 2) == 0
    assert lib.fx_w3_gemv_config_workspace_bytes(1, 4096, 4096, 8, 1, 16, 2) == 2 * 4096 * 4
    assert lib.fx_w3_gemv_config_workspace_bytes(3, 4096, 4096, 8, 1, 8, 1) == 4 * 2 * 4096 * 4
    rc = lib.fx_w3_gemv(dummy, 2, dummy, dummy, 2, None, None, None, 0, dummy, 1, 65536, 32768 * 4, 0, None)
    assert rc == 1 and "2 GiB" in lib.fx_last_error().decode()
    rc = lib.fx_w3_gemv_config(dummy, 2, dummy, dummy, 2, None, None, dummy, 1 << 20, dummy, 1, 64, 256, 3, 1, 4, 1, None)
    assert rc == 1 and "waves" in lib.fx_last_error().decode()


def test_check_raises_runtime_error_with_message():
    lib = _lib.library()
    rc = lib.fx_w3_finish(None, None, 2, 1, 1, 1, None)
    with pytest.raises(RuntimeError, match="non-null"):
        _lib.check(rc, "fx_w3_finish")


def test_plain_c_caller(tmp_path):
    """The header compiles as C99 and as C++, and a C program linked against the
    library calls it (host-only calls: ABI version, workspace query, fail-closed
    argument checks)."""
    import shutil
    import subprocess

    gcc = shutil.which("gcc")
    if gcc is None:
        pytest.skip("no gcc")
    root = HEADER.parents[1]
    libdir = root / "marlin_style_fluxbin_amd"
    exe = tmp_path / "caller"
    subprocess.run([gcc, "-std=c99", "-Wall", "-Wextra", "-Werror", "-I", str(root / "include"),
                    str(root / "tests" / "c_abi" / "caller.c"), "-L", str(libdir), "-lfluxbin_amd",
                    f"-Wl,-rpath,{libdir}", "-o", str(exe)], check=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, run.stdout + run.stderr
    assert f"abi {_lib.ABI_VERSION}" in run.stdout
    assert f"workspace {_lib.library().fx_w3_gemv_workspace_bytes(1, 4096, 4096)}" in run.stdout
    gxx = shutil.which("g++")
    if gxx is not None:  # the extern "C" block keeps the names unmangled for C++ callers
        src = tmp_path / "probe.cc"
        src.write_text('#include "fluxbin_amd.h"\nint main() { return fx_abi_version() > 0 ? 0 : 1; }\n')
        subprocess.run([gxx, "-Wall", "-Werror", "-I", str(root / "include"), str(src), "-L", str(libdir),
                        "-lfluxbin_amd", f"-Wl,-rpath,{libdir}", "-o", str(tmp_path / "probe")], check=True)
        assert subprocess.run([str(tmp_path / "probe")], timeout=120).returncode == 0
