"""The C ABI from plain C: tests/c_caller.c compiled as C99 with -Wall
-Werror against include/fdattn.h, linked against the built library, and run
(no GPU needed: queries, a host-side argument error, and one decode through
the host-core entry point checked against double-precision attention)."""

from __future__ import annotations

import shutil
import subprocess
from pathlib import Path

import pytest

from vllm_fastdecoder_amd import _lib

ROOT = Path(__file__).resolve().parents[1]


def test_plain_c_caller_builds_links_and_runs(tmp_path):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    lib_dir = _lib.LIB_PATH.parent
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    exe = tmp_path / "c_caller"
    rocm_lib = "/opt/rocm/lib"
    cmd = [cc, "-std=c99", "-Wall", "-Wextra", "-Werror", f"-DEXPECTED_ABI={_lib.ABI_VERSION}",
           "-I", str(ROOT / "include"), str(ROOT / "tests" / "c_caller.c"), "-o", str(exe),
           f"-L{lib_dir}", "-lfdattn", f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath-link,{rocm_lib}",
           "-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, f"check {run.returncode} failed: {run.stdout}{run.stderr}"
    assert "c caller ok" in run.stdout
