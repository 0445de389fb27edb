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
    exe = _build(tmp_path, gpu=False)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, f"check {run.returncode} failed: {run.stdout}{run.stderr}"
    assert "c caller ok" in run.stdout


def _build(tmp_path, gpu: bool):
    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    if not _lib.LIB_PATH.exists():
        pytest.skip("library not built")
    lib_dir = _lib.LIB_PATH.parent
    rocm = Path("/opt/rocm")
    exe = tmp_path / ("c_caller_gpu" if gpu else "c_caller")
    cmd = [cc, "-std=c99", "-Wall", "-Wextra", "-Werror", f"-DEXPECTED_ABI={_lib.ABI_VERSION}",
           "-I", str(ROOT / "include")]
    if gpu:
        cmd += ["-DWITH_GPU", "-D__HIP_PLATFORM_AMD__", "-I", str(rocm / "include")]
    cmd += [str(ROOT / "tests" / "c_caller.c"), "-o", str(exe), f"-L{lib_dir}", "-lfdattn",
            f"-Wl,-rpath,{lib_dir}", f"-Wl,-rpath-link,{rocm / 'lib'}"]
    if gpu:
        cmd += [f"-L{rocm / 'lib'}", "-lamdhip64", f"-Wl,-rpath,{rocm / 'lib'}"]
    cmd += ["-lm"]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-3000:]
    return exe


@pytest.mark.gpu
def test_plain_c_caller_on_the_gpu(gpu, tmp_path):
    """The same C caller with its GPU section: device copies through the HIP
    runtime API (C), fd_paged_decode_partial on fp32 KV in 16-token blocks
    (the tiled fp32 kernel), and a whole hybrid split step (the host share
    queued behind q's copy, the fused launch over both tiers, the merge of
    the pinned host partial), each checked against double-precision
    attention; the hybrid step twice, by separate calls and with
    fd_hybrid_share_start, bit-identical."""
    exe = _build(tmp_path, gpu=True)
    run = subprocess.run([str(exe)], capture_output=True, text=True, timeout=120)
    assert run.returncode == 0, f"check {run.returncode} failed: {run.stdout}{run.stderr}"
    assert "c caller ok" in run.stdout
