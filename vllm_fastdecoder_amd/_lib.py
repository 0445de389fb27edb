"""ctypes binding of libfdattn.so (the C ABI declared in include/fdattn.h).

`load_lib()` mirrors the reference's extension loader (fastdecode/cpu_ops.py:
17-46): a process-wide singleton behind a double-checked lock. The library is
never compiled here; `build()` in build.py (or `__graft_entry__.build()`)
produces it in-tree. A missing or stale library raises instead of falling
back to anything else.
"""

from __future__ import annotations

import ctypes
import threading
from ctypes import POINTER, c_char_p, c_double, c_float, c_int, c_int32, c_int64, c_size_t, c_void_p

from .build import LIB_PATH

FD_F16, FD_BF16, FD_F32 = 0, 1, 2
FD_OK = 0
FD_ERR_INVALID, FD_ERR_RANGE, FD_ERR_WORKSPACE, FD_ERR_HIP, FD_ERR_UNSUPPORTED = 1, 2, 3, 4, 5
FD_ERR_RESOURCE = 6
ABI_VERSION = 12
NOALLOC_SCRATCH_BYTES = 32 << 20  # FD_NOALLOC_SCRATCH_BYTES of include/fdattn.h


# Kernel families of fd_decode_plan_info (include/fdattn.h).
FD_KERNEL_NAMES = {0: "generic", 1: "valu", 2: "mfma", 3: "mm", 4: "f32"}


class FdDecodePlan(ctypes.Structure):
    _fields_ = [
        ("kernel", c_int32),
        ("heads_per_task", c_int32),
        ("passes", c_int32),
        ("split_blocks", c_int32),
        ("max_splits", c_int32),
        ("wg_cap", c_int32),
        ("wave_blocks", c_int32),
    ]


class FdKvTier(ctypes.Structure):
    """struct fd_kv_tier of include/fdattn.h: one KV tier of fd_split_decode."""

    _fields_ = [
        ("k_cache", c_void_p),
        ("v_cache", c_void_p),
        ("stride_block", c_int64),
        ("stride_head", c_int64),
        ("stride_token", c_int64),
        ("num_blocks", c_int64),
        ("block_table", c_void_p),
        ("bt_stride", c_int64),
        ("bt_width", c_int32),
        ("lens", c_void_p),
    ]


# name -> (restype, argtypes); the order follows include/fdattn.h
SIGNATURES: dict[str, tuple] = {
    "fd_last_error": (c_char_p, []),
    "fd_abi_version": (c_int, []),
    "fd_paged_decode_partial": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # q, q strides
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # kv strides block/head/token
            c_int64,                               # num_blocks
            c_void_p, c_int64, c_int32,            # block_table, bt_stride, bt_width
            c_void_p, c_void_p,                    # lens, row_order
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_int64, c_int64, c_int32,   # out, strides, out_dtype
            c_void_p, c_int64,                     # lse, lse_stride_head
            c_void_p, c_size_t,                    # workspace
            c_void_p,                              # stream
        ],
    ),
    "fd_paged_decode_partial_hint": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # q, q strides
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # kv strides block/head/token
            c_int64,                               # num_blocks
            c_void_p, c_int64, c_int32,            # block_table, bt_stride, bt_width
            c_void_p, c_void_p,                    # lens, row_order
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_int64, c_int64, c_int32,   # out, strides, out_dtype
            c_void_p, c_int64,                     # lse, lse_stride_head
            c_void_p, c_size_t,                    # workspace
            c_void_p,                              # stream
            c_int64,                               # total_tokens
        ],
    ),
    "fd_paged_decode_timeline": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # q, q strides
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # kv strides block/head/token
            c_int64,                               # num_blocks
            c_void_p, c_int64, c_int32,            # block_table, bt_stride, bt_width
            c_void_p, c_void_p,                    # lens, row_order
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_int64, c_int64, c_int32,   # out, strides, out_dtype
            c_void_p, c_int64,                     # lse, lse_stride_head
            c_void_p, c_size_t,                    # workspace
            c_void_p,                              # stream
            c_void_p, c_int64,                     # timeline, timeline_workgroups
        ],
    ),
    "fd_paged_decode_workspace_size": (
        c_int,
        [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32, POINTER(c_size_t)],
    ),
    "fd_decode_plan_info": (
        c_int,
        [c_int32, c_int32, c_int32, c_int32, c_int32, c_int32,  # n, H, KVH, D, BS, bt_width
         c_int32, c_int32, c_int32,                             # kv_dtype, aligned, host_tier
         c_int64,                                               # total_tokens
         POINTER(FdDecodePlan)],
    ),
    "fd_paged_decode_partial_noalloc": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # q, q strides
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # kv strides block/head/token
            c_int64,                               # num_blocks
            c_void_p, c_int64, c_int32,            # block_table, bt_stride, bt_width
            c_void_p, c_void_p,                    # lens, row_order
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_int64, c_int64, c_int32,   # out, strides, out_dtype
            c_void_p, c_int64,                     # lse, lse_stride_head
            c_void_p,                              # stream
        ],
    ),
    "fd_split_decode": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # q, q strides
            POINTER(FdKvTier), POINTER(FdKvTier),  # hbm tier, host tier
            c_void_p,                              # row_order
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_int64, c_int64, c_int32,   # out, strides, out_dtype
            c_void_p, c_int64,                     # lse, lse_stride_head
            c_void_p, c_size_t,                    # workspace
            c_void_p,                              # stream
        ],
    ),
    "fd_plan_tiers": (
        c_int,
        [
            c_void_p, c_int64, c_int32,            # block_table, bt_stride, bt_width
            c_void_p, c_int32,                     # seq_lens, n_rows
            c_int32, c_int64, c_int32,             # G, C, block_size
            c_void_p, c_void_p, c_int64, c_int32,  # gpu/cpu tables, out stride, width
            c_void_p, c_void_p,                    # gpu_lens, cpu_lens
            c_void_p, c_int32,                     # slot_mapping, n_tokens
            c_void_p, c_void_p,                    # gpu / host slot mappings
            c_void_p,                              # error_count
            c_void_p,                              # stream
        ],
    ),
    "fd_merge_attn_states": (
        c_int,
        [
            c_void_p, c_int64, c_int64, c_int32,   # out
            c_void_p, c_int64, c_int64, c_int32,   # o_a
            c_void_p, c_int64,                     # lse_a
            c_void_p, c_int64, c_int64, c_int32,   # o_b
            c_void_p, c_int64,                     # lse_b
            c_void_p, c_int64,                     # out_lse
            c_int32, c_int32, c_int32,             # n, H, D
            c_void_p,                              # stream
        ],
    ),
    "fd_reshape_and_cache": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # key
            c_void_p, c_int64, c_int64,            # value
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # cache strides block/token/head
            c_int64,                               # num_blocks
            c_void_p, c_int32,                     # slot_mapping, num_tokens
            c_int32, c_int32, c_int32,             # KVH, D, block_size
            c_int32, c_void_p, c_void_p,           # dtype, error_count, write_gate
            c_void_p,                              # stream
        ],
    ),
    "fd_check_slots": (c_int, [c_void_p, c_int64, c_int64, POINTER(c_int64)]),
    "fd_host_alloc": (c_int, [c_size_t, POINTER(c_void_p)]),
    "fd_host_free": (c_int, [c_void_p]),
    "fd_host_device_pointer": (c_int, [c_void_p, POINTER(c_void_p)]),
    "fd_host_decode_partial": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # q, q strides
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # kv strides block/head/token
            c_int64,                               # num_blocks
            c_void_p, c_int64, c_int32,            # block_table, bt_stride, bt_width
            c_void_p,                              # lens
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_int64, c_int64, c_int32,   # out, strides, out_dtype
            c_void_p, c_int64,                     # lse, lse_stride_head
            c_int32,                               # num_threads
        ],
    ),
    "fd_host_decode_partial_start": (
        c_int,
        [
            c_void_p,                              # ready_event
            c_void_p, c_int64, c_int64,            # q, q strides
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # kv strides block/head/token
            c_int64,                               # num_blocks
            c_void_p, c_int64, c_int32,            # block_table, bt_stride, bt_width
            c_void_p,                              # lens
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_int64, c_int64, c_int32,   # out, strides, out_dtype
            c_void_p, c_int64,                     # lse, lse_stride_head
            c_int32, POINTER(c_int64),             # num_threads, call
        ],
    ),
    "fd_host_decode_wait": (c_int, [c_int64, POINTER(c_double)]),
    "fd_host_decode_threads": (c_int, []),
    "fd_host_decode_isa": (c_int, []),
    "fd_host_stream_read": (c_int, [c_void_p, c_size_t, c_int32, POINTER(ctypes.c_uint64)]),
    "fd_host_set_threads": (c_int, [c_int32]),
    "fd_share_host_blocks": (
        c_int,
        [
            c_void_p, c_int64, c_int32,            # host_bt, bt_stride, bt_width
            c_void_p, c_int32, c_int32, c_double,  # host_lens, n, block_size, cpu_fraction
            c_void_p, c_void_p, c_int64, c_void_p,  # gpu_lens, cpu_bt, cpu_bt_stride, cpu_lens
            POINTER(c_int32),                      # cpu_width
        ],
    ),
    "fd_hybrid_share_start": (
        c_int,
        [
            c_void_p, c_void_p, c_void_p, c_void_p,  # stream, ready_event, q, q_host
            c_void_p, c_int64, c_int32,            # host_bt, bt_stride, bt_width
            c_void_p, c_double,                    # host_lens, cpu_fraction
            c_void_p, c_void_p, c_int64, c_void_p,  # gpu_lens, cpu_bt, cpu_bt_stride, cpu_lens
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # kv strides block/head/token
            c_int64,                               # num_blocks
            c_int32, c_int32, c_int32, c_int32,    # n, H, KVH, D
            c_int32, c_float, c_int32,             # block_size, scale, kv_dtype
            c_void_p, c_void_p,                    # out, lse
            c_int32, POINTER(c_int64),             # num_threads, call
        ],
    ),
    "fd_host_store_kv": (
        c_int,
        [
            c_void_p, c_int64, c_int64,            # k, strides token/head
            c_void_p, c_int64, c_int64,            # v, strides token/head
            c_void_p, c_void_p,                    # k_cache, v_cache
            c_int64, c_int64, c_int64,             # cache strides block/head/token
            c_int64,                               # num_blocks
            c_void_p, c_int64,                     # slots, m
            c_int32, c_int32, c_int32, c_int32,    # KVH, D, BS, dtype
        ],
    ),
    "fd_stream_copy": (c_int, [c_void_p, c_void_p, c_size_t, c_void_p]),
}

_LIB = None
_LOCK = threading.Lock()


class FdError(RuntimeError):
    """A libfdattn call returned a non-zero status (RuntimeError, like the
    reference's TORCH_CHECK failures)."""

    def __init__(self, status: int, msg: str):
        super().__init__(f"libfdattn error {status}: {msg}")
        self.status = status


def load_lib():
    global _LIB
    if _LIB is not None:
        return _LIB
    with _LOCK:
        if _LIB is not None:
            return _LIB
        if not LIB_PATH.exists():
            raise RuntimeError(
                f"{LIB_PATH} is missing: build it first (python -m vllm_fastdecoder_amd.build "
                "or __graft_entry__.build()); there is no fallback path"
            )
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        if lib.fd_abi_version() != ABI_VERSION:
            raise RuntimeError(f"{LIB_PATH} has ABI {lib.fd_abi_version()}, expected {ABI_VERSION}")
        _LIB = lib
        return _LIB


def check(status: int) -> None:
    if status != FD_OK:
        msg = load_lib().fd_last_error()
        raise FdError(status, msg.decode() if msg else "")
