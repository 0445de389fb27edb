"""Builds libfdattn.so, the gfx950 HIP library behind the split decode path.

The library is compiled in-tree with hipcc (no JIT cache), so the built
shared object sits next to this file and ships with the package. Every HIP
source under csrc/ is compiled for gfx950 only; the host-only C++ sources
(the host-core decode of the host tier) are compiled with the system C++
compiler and linked into the same library.
"""

from __future__ import annotations

import os
import subprocess
import tempfile
from concurrent.futures import ThreadPoolExecutor
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parent
CSRC = PKG_DIR / "csrc"
LIB_NAME = "libfdattn.so"
LIB_PATH = PKG_DIR / LIB_NAME
ARCH = "gfx950"

HIPCC_FLAGS = [
    "-O3",
    "-std=c++17",
    f"--offload-arch={ARCH}",
    "-fPIC",
    # keep packed-fp32 VALU ops out of the generated code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall",
    "-Wno-unused-function",
]


# Per-source additions. decode_mm.hip: MFMA accumulators in VGPRs. With the
# default heuristic its P.V accumulators live in AGPRs, and the rarely taken
# rescale branch of every block makes the compiler copy all 32 of them to
# VGPRs and back on the common path too (64 v_accvgpr moves per block); in
# VGPRs the kernel needs 154 registers and no AGPRs.
SOURCE_FLAGS = {
    "decode_mm.hip": ["-mllvm", "-amdgpu-mfma-vgpr-form"],
}

CXX_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-pthread", "-Wall", "-Wno-unused-function"]


def sources() -> list[Path]:
    return sorted(CSRC.glob("*.hip"))


def host_sources() -> list[Path]:
    return sorted(CSRC.glob("*.cpp"))


def cxx() -> str:
    return os.environ.get("CXX", "g++")


def hipcc() -> str:
    rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
    cand = Path(rocm) / "bin" / "hipcc"
    return str(cand) if cand.exists() else "hipcc"


def _run(cmd: list[str], verbose: bool) -> None:
    if verbose:
        print(" ".join(cmd), flush=True)
    res = subprocess.run(cmd, capture_output=True, text=True)
    if res.returncode != 0:
        raise RuntimeError(f"{cmd[0]} failed ({res.returncode}):\n{res.stderr}")
    if verbose and res.stderr:
        # hipcc's host pass warns about the device-only target feature
        lines = [ln for ln in res.stderr.splitlines() if "packed-fp32-ops" not in ln]
        if lines:
            print("\n".join(lines))


def build(verbose: bool = False, out: Path | None = None) -> Path:
    """Compiles every csrc/*.hip (one hipcc per source, in parallel) and links
    them into one shared library. Always rebuilds."""
    out = out or LIB_PATH
    tmp = out.with_suffix(".so.tmp")
    srcs = sources()
    hsrcs = host_sources()
    jobs = max(1, min(len(srcs) + len(hsrcs),
                      int(os.environ.get("MAX_JOBS", os.cpu_count() or 1))))
    with tempfile.TemporaryDirectory(prefix="fdattn_build_") as d:
        objs = [Path(d) / (src.stem + ".o") for src in srcs]
        hobjs = [Path(d) / (src.stem + ".host.o") for src in hsrcs]
        cmds = [[hipcc(), *HIPCC_FLAGS, *SOURCE_FLAGS.get(src.name, []), "-c", str(src), "-o",
                 str(obj)] for src, obj in zip(srcs, objs)]
        cmds += [[cxx(), *CXX_FLAGS, "-c", str(src), "-o", str(obj)]
                 for src, obj in zip(hsrcs, hobjs)]
        with ThreadPoolExecutor(max_workers=jobs) as pool:
            for f in [pool.submit(_run, c, verbose) for c in cmds]:
                f.result()
        _run([hipcc(), f"--offload-arch={ARCH}", "-fPIC", "-shared", "-pthread",
              *map(str, objs + hobjs), "-o", str(tmp)], verbose)
    os.replace(tmp, out)
    return out


if __name__ == "__main__":
    print(build(verbose=True))
