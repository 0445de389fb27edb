"""MI355X-native split decode attention for vllm_fastdecode's G+C KV tiers.

Hot path (HIP kernels in libfdattn.so, C ABI in include/fdattn.h):
  * paged partial decode attention over a block subset -> (out, lse);
  * log-sum-exp merge of the HBM-tier and host-tier partials;
  * reshape_and_cache slot-mapping writes into either tier.

Python surface (mirrors the reference plugin's modules):
  ops      decode_attn / store_kv (cpu_ops extension ABI), paged_decode,
           merge_attn_states, reshape_and_cache (backend.OPS primitives)
  plan     build_host_plan / to_device (per-step execution plan)
  state    HostKVStore over pinned host memory, ensure_store
  config   FASTDECODE_CPU_BLOCKS / FASTDECODE_CPU_KV_GB sizing, spec checks
  backend  HipOps seam and the _forward_split orchestration
"""

from ._lib import FdError, load_lib  # noqa: F401

__all__ = ["FdError", "load_lib"]
