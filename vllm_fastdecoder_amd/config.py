"""Environment-driven configuration of the host tier (fastdecode/config.py).

The same variables as the reference, read by both the engine-side scheduler
and the worker, so they must be set in the environment that launches the
engine:

FASTDECODE_CPU_BLOCKS   number of extra KV blocks held in host memory, or
FASTDECODE_CPU_KV_GB    the same as GiB of host memory (ignored when
                        FASTDECODE_CPU_BLOCKS is set)
FASTDECODE_CPU_THREADS  worker threads of the host-core decode kernel
                        (read by the library, fd_host_decode_threads)
FASTDECODE_STATS        "1" logs the per-step split of requests and host-tier
                        tokens every 50 steps

The spec checks follow fastdecode/config.py:62-81. vLLM's spec classes are
used when vLLM is importable; otherwise a spec is checked by its attributes
(sliding_window, kv_quant_mode, head_size_v), so plain objects of the same
shape work too.
"""

from __future__ import annotations

import os

ENV_CPU_BLOCKS = "FASTDECODE_CPU_BLOCKS"
ENV_CPU_KV_GB = "FASTDECODE_CPU_KV_GB"
ENV_STATS = "FASTDECODE_STATS"


def enabled() -> bool:
    """A host tier is configured (config.py:25-26)."""
    return bool(os.environ.get(ENV_CPU_BLOCKS) or os.environ.get(ENV_CPU_KV_GB))


def stats_enabled() -> bool:
    return os.environ.get(ENV_STATS, "0") not in ("", "0", "false", "False")


def kv_bytes_per_block(kv_cache_config) -> int:
    """Bytes one KV block takes over all layers, K and V (config.py:33-38)."""
    return sum(group.kv_cache_spec.page_size_bytes * len(group.layer_names)
               for group in kv_cache_config.kv_cache_groups)


def _resolve(per_block_bytes: int) -> int:
    blocks = os.environ.get(ENV_CPU_BLOCKS)
    if blocks:
        return max(0, int(blocks))
    gb = os.environ.get(ENV_CPU_KV_GB)
    if gb:
        if per_block_bytes <= 0:
            raise ValueError("FastDecode: a KV block of 0 bytes cannot size the host tier")
        return max(0, int(float(gb) * (1 << 30)) // per_block_bytes)
    return 0


def resolve_num_cpu_blocks(kv_cache_config) -> int:
    """Host-tier blocks, engine side (the whole KV cache config)."""
    return _resolve(kv_bytes_per_block(kv_cache_config))


def resolve_num_cpu_blocks_from_spec(spec, num_layers: int) -> int:
    """Host-tier blocks, worker side (one group's spec and its layer count);
    agrees with resolve_num_cpu_blocks for single-group models."""
    return _resolve(spec.page_size_bytes * num_layers)


def validate_kv_cache_config(kv_cache_config) -> None:
    """Exactly one full-attention KV cache group (config.py:62-70)."""
    groups = kv_cache_config.kv_cache_groups
    if len(groups) != 1:
        raise NotImplementedError(
            f"FastDecode supports models with a single KV cache group, got {len(groups)} "
            "(hybrid / sliding-window / MLA models are out of scope).")
    validate_spec(groups[0].kv_cache_spec)


def _vllm_spec_types():
    try:
        from vllm.v1.kv_cache_interface import FullAttentionSpec, KVQuantMode
    except Exception:  # vLLM absent: check by attributes
        return None
    return FullAttentionSpec, KVQuantMode


def validate_spec(spec) -> None:
    """Full attention, unquantised KV, equal K and V head sizes
    (config.py:73-81); NotImplementedError otherwise."""
    types = _vllm_spec_types()
    if types is not None:
        full, quant = types
        if not isinstance(spec, full) or spec.sliding_window is not None:
            raise NotImplementedError(f"FastDecode needs full attention, got {type(spec).__name__}")
        if spec.kv_quant_mode != quant.NONE:
            raise NotImplementedError("FastDecode does not support quantized KV cache")
    else:
        if getattr(spec, "sliding_window", None) is not None:
            raise NotImplementedError(f"FastDecode needs full attention, got {type(spec).__name__}")
        mode = getattr(spec, "kv_quant_mode", None)
        if mode is not None and getattr(mode, "name", mode) not in ("NONE", "none"):
            raise NotImplementedError("FastDecode does not support quantized KV cache")
    if getattr(spec, "head_size_v", spec.head_size) != spec.head_size:
        raise NotImplementedError("FastDecode needs head_size_v == head_size")
