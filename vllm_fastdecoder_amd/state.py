"""Worker-side state: the host KV tier in pinned, GPU-mapped memory.

Mirrors fastdecode/state.py:16-90, with the tier sized from the same
environment (config.py). The difference that matters: the reference
allocates the host tier as pageable `torch.zeros` and stages q/k/v/o/lse
through pinned buffers every layer (state.py:93-134); here the tier itself
is pinned and mapped (pinned.pinned_zeros), so the decode and cache-write
kernels reach it directly and no per-layer staging exists (the hybrid
split's few small buffers live in ops).
"""

from __future__ import annotations

import logging
import time
from dataclasses import dataclass, field

import torch

from . import config
from .pinned import pinned_zeros

logger = logging.getLogger("fastdecode")


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


def ensure_host_store(num_gpu_blocks: int | None, num_cpu_blocks: int, block_size: int,
                      num_kv_heads: int, head_size: int, dtype: torch.dtype,
                      layer_names: list[str]) -> HostKVStore | None:
    """Create (idempotently) the worker's host tier from explicit geometry:
    nothing when G is unknown yet (profiling-time builders), none when no
    host blocks are configured; rebuilt when the geometry or the layers
    change. ensure_store below resolves the geometry as the reference does."""
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
    from . import _lib

    lib = _lib.load_lib()  # loaded now so a missing library fails at start-up
    logger.warning("FastDecode: %d GPU blocks + %d host blocks (block_size=%d, %.2f GiB pinned "
                   "host KV for %d layers, allocated in %.1fs). Host-core kernel: %d-bit "
                   "vectors, threads=%d", num_gpu_blocks, num_cpu_blocks, block_size, gib,
                   len(layer_names), time.time() - t0, lib.fd_host_decode_isa(),
                   lib.fd_host_decode_threads())
    STORE = store
    return store


def ensure_store(vllm_config, spec, layer_names: list[str]) -> HostKVStore | None:
    """The reference's entry point (state.py:32-90), called from the metadata
    builder's constructor: no-op unless FASTDECODE_CPU_BLOCKS /
    FASTDECODE_CPU_KV_GB is set; G from vllm_config.cache_config.num_gpu_blocks
    (None while memory is being profiled: nothing happens); C from the
    environment over the spec's page size and the layer count; the spec
    validated (full attention, unquantised) before anything is allocated.
    Returns the store (the reference returns None)."""
    global STORE
    if not config.enabled():
        return None
    num_gpu = vllm_config.cache_config.num_gpu_blocks
    if num_gpu is None:
        return STORE
    num_cpu = config.resolve_num_cpu_blocks_from_spec(spec, len(layer_names))
    if num_cpu <= 0:
        STORE = None
        return None
    config.validate_spec(spec)
    return ensure_host_store(int(num_gpu), num_cpu, spec.block_size, spec.num_kv_heads,
                             spec.head_size, spec.dtype, layer_names)
