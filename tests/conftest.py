"""pytest configuration: the `gpu` marker, repo-root imports, library build.

Tests marked `gpu` need an MI355X; the rest run on any CPU. The HIP library
is built in-tree by __graft_entry__.build(); tests only build it when no
library exists yet (a machine that received a built tree uses that one).
"""

from __future__ import annotations

import sys
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]
if str(ROOT) not in sys.path:
    sys.path.insert(0, str(ROOT))


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs a ROCm GPU (MI355X)")


@pytest.fixture(scope="session", autouse=True)
def _libraries():
    from vllm_fastdecoder_amd import build as fdbuild

    if not fdbuild.LIB_PATH.exists():
        fdbuild.build()
    import oracle

    if not oracle.LIB_PATH.exists():
        oracle.build()
    yield


@pytest.fixture
def gpu():
    import torch

    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    return torch.device("cuda", 0)
