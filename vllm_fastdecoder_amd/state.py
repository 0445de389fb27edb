"""Worker-side state: the host KV tier in pinned, GPU-mapped memory.

Mirrors fastdecode/state.py:16-134 and fastdecode/config.py:20-59. The
difference that matters: the reference allocates the host tier as pageable
`torch.zeros` and stages q/k/v/o/lse through pinned buffers every layer;
here the tier itself is pinned and mapped (pinned.pinned_zeros), so the
decode and cache-write kernels reach it directly and no staging copy or
host-side compute exists. `PinnedStaging` is kept for callers that still
move data through host buffers.
"""

from __future__ import annotations

import logging
import os
import time
from dataclasses import dataclass, field

import torch

from .pinned import pinned_empty, pinned_zeros

logger = logging.getLogger("fastdecode")

ENV_CPU_BLOCKS = "FASTDECODE_CPU_BLOCKS"
ENV_CPU_KV_GB = "FASTDECODE_CPU_KV_GB"


def enabled() -> bool:
    """A host tier is configured (config.py:25)."""
    return bool(os.environ.get(ENV_CPU_BLOCKS) or os.environ.get(ENV_CPU_KV_GB))


def resolve_num_cpu_blocks(per_block_bytes: int) -> int:
    """Host-tier blocks from FASTDECODE_CPU_BLOCKS, else FASTDECODE_CPU_KV_GB
    GiB divided by the bytes one block takes over all layers (config.py:41-59)."""
    blocks = os.environ.get(ENV_CPU_BLOCKS)
    if blocks:
        return max(0, int(blocks))
    gb = os.environ.get(ENV_CPU_KV_GB)
    if gb:
        return max(0, int(float(gb) * (1 << 30)) // per_block_bytes)
    return 0


@dataclass
class HostKVStore:
    """The G+C block split: ids [0, G) in HBM, [G, G + C) here at id - G.
    Per layer, K and V are [C, KVH, BS, D] in pinned mapped memory."""

    num_gpu_blocks: int
    num_cpu_blocks: int
    block_size: int
    num_kv_heads: int
    head_size: int
    dtype: torch.dtype
    k: dict[str, torch.Tensor] = field(default_factory=dict)
    v: dict[str, torch.Tensor] = field(default_factory=dict)
    steps: int = 0

    @property
    def shape(self) -> tuple[int, int, int, int]:
        return (self.num_cpu_blocks, self.num_kv_heads, self.block_size, self.head_size)

    def add_layer(self, name: str) -> None:
        # zero-filled (not just allocated) so the pages are committed now
        self.k[name] = pinned_zeros(self.shape, self.dtype)
        self.v[name] = pinned_zeros(self.shape, self.dtype)


# CpuKVStore is the reference's name for the same object (state.py:16).
CpuKVStore = HostKVStore

STORE: HostKVStore | None = None


def ensure_store(num_gpu_blocks: int | None, num_cpu_blocks: int, block_size: int,
                 num_kv_heads: int, head_size: int, dtype: torch.dtype,
                 layer_names: list[str]) -> HostKVStore | None:
    """Create (idempotently) the worker's host tier (state.py:32-90, without
    the vLLM config objects): nothing when G is unknown yet (profiling-time
    builders) or when no host blocks are configured."""
    global STORE
    if num_gpu_blocks is None:
        return STORE
    if num_cpu_blocks <= 0:
        STORE = None
        return None
    if (STORE is not None and STORE.num_gpu_blocks == num_gpu_blocks
            and STORE.num_cpu_blocks == num_cpu_blocks and STORE.block_size == block_size
            and STORE.num_kv_heads == num_kv_heads and STORE.head_size == head_size
            and STORE.dtype == dtype and all(n in STORE.k for n in layer_names)):
        return STORE
    store = HostKVStore(int(num_gpu_blocks), int(num_cpu_blocks), block_size, num_kv_heads,
                        head_size, dtype)
    t0 = time.time()
    for name in layer_names:
        store.add_layer(name)
    elt = torch.empty((), dtype=dtype).element_size()
    gib = 2 * len(layer_names) * num_cpu_blocks * num_kv_heads * block_size * head_size * elt / (1 << 30)
    logger.info("FastDecode: %d GPU blocks + %d host blocks (block_size=%d, %.2f GiB pinned "
                "host KV for %d layers, allocated in %.1fs)", num_gpu_blocks, num_cpu_blocks,
                block_size, gib, len(layer_names), time.time() - t0)
    STORE = store
    return store


class PinnedStaging:
    """Grow-only pinned host buffers (state.py:93-124)."""

    def __init__(self) -> None:
        self._bufs: dict[str, torch.Tensor] = {}

    def get(self, name: str, shape: tuple[int, ...], dtype: torch.dtype) -> torch.Tensor:
        numel = 1
        for s in shape:
            numel *= int(s)
        buf = self._bufs.get(name)
        if buf is None or buf.dtype != dtype or buf.numel() < numel:
            cap = max(numel, 1, 2 * (buf.numel() if buf is not None else 0))
            buf = pinned_empty((cap,), dtype)
            self._bufs[name] = buf
        return buf[:numel].view(shape)


_STAGING: PinnedStaging | None = None


def staging() -> PinnedStaging:
    global _STAGING
    if _STAGING is None:
        _STAGING = PinnedStaging()
    return _STAGING
