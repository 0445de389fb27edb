"""The matrix-core kernels' gfx950 code reads no MFMA result sooner after a
branch than the compiler allows on straight-line paths (see isa_hazards.py:
a conditional branch between the scores MFMAs and their scaling once left a
path 1-5 wait states long, against 8 on straight-line code, and the kernel
read stale scores). And the cross-lane butterflies built on
v_permlane16_swap / v_permlane32_swap with one value as both operands
(fd_common.h xor_pair) are really emitted: an LLVM fold of such a swap into
a copy of its operand has been seen once, and would leave each lane-row's
partial sums unmerged. Compiles the tiled decode kernels to assembly with
the library's own flags; no GPU needed."""

from __future__ import annotations

import shutil
import subprocess
from collections import defaultdict
from concurrent.futures import ThreadPoolExecutor

import pytest

from tests import isa_hazards
from vllm_fastdecoder_amd import build

SOURCES = ["decode_mm.hip", "decode_mfma.hip"]
SWAP_SOURCES = ["decode_valu.hip", "decode_mm.hip", "decode_mfma.hip", "decode_f32.hip"]


def _asm(src: str, tmp_path) -> str:
    out = tmp_path / (src + ".s")
    cmd = [build.hipcc(), *build.HIPCC_FLAGS, *build.SOURCE_FLAGS.get(src, []),
           "--cuda-device-only", "-S", str(build.CSRC / src), "-o", str(out)]
    res = subprocess.run(cmd, capture_output=True, text=True)
    assert res.returncode == 0, res.stderr[-2000:]
    return out.read_text()


@pytest.fixture(scope="module")
def asm(tmp_path_factory):
    if shutil.which(build.hipcc()) is None:
        pytest.skip("hipcc not available")
    tmp = tmp_path_factory.mktemp("isa")
    srcs = sorted(set(SOURCES) | set(SWAP_SOURCES))
    with ThreadPoolExecutor(max_workers=len(srcs)) as pool:
        texts = list(pool.map(lambda s: _asm(s, tmp), srcs))
    return dict(zip(srcs, texts))


@pytest.mark.parametrize("src", SOURCES)
def test_no_mfma_result_read_early_across_a_branch(asm, src):
    gaps = [g for name, ins, labels in isa_hazards.kernels(asm[src])
            for g in isa_hazards.mfma_read_gaps(name, ins, labels)]
    assert gaps, "no MFMA result reads found: the parser no longer matches the assembly"
    straight = defaultdict(lambda: 1 << 30)
    for g in gaps:
        if not g.via_branch:
            straight[g.mfma] = min(straight[g.mfma], g.wait_states)
    short = [g for g in gaps if g.via_branch and g.mfma in straight
             and g.wait_states < straight[g.mfma]]
    assert not short, "\n".join(
        f"{g.kernel}: {g.mfma} read by {g.reader} after {g.wait_states} wait states across "
        f"a branch (straight-line minimum {straight[g.mfma]})" for g in short[:10])


@pytest.mark.parametrize("src", SWAP_SOURCES)
def test_lane_swap_butterflies_are_emitted(asm, src):
    """Every tiled decode kernel merges its lane-rows (or the score rows of a
    block) with xor_sum / xor_max, whose last step at any head size is a
    32-lane v_permlane32_swap; a kernel without one has had the swap folded."""
    names = [name for name, _, _ in isa_hazards.kernels(asm[src]) if "decode" in name]
    assert names, "no decode kernels found in the assembly"
    missing = []
    for name, ins, _ in isa_hazards.kernels(asm[src]):
        if "decode" in name and not any(op.startswith("v_permlane32_swap") for op, _ in ins):
            missing.append(name)
    assert not missing, f"{len(missing)} kernels without v_permlane32_swap, e.g. {missing[:3]}"
