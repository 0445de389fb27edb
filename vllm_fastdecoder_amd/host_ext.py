"""The reference's CPU extension, on this library's host-core kernels.

The reference builds a pybind11 module from fastdecode/csrc/cpu_attn.cpp
(exports at :531-537) and loads it through cpu_ops.load_ext
(fastdecode/cpu_ops.py:21-46). This module has the same five functions with
the same arguments, checks and errors, over host (CPU) tensors, computed by
libfdattn's host-core code (fd_host_decode_partial, fd_host_store_kv):

  decode_attn(q, k_cache, v_cache, block_table, lens, scale, out, lse)
  store_kv(k, v, slots, k_cache, v_cache)
  set_num_threads(n) / get_num_threads() / has_avx2()

`load_ext()` returns the module itself, so pointing the reference's
`cpu_ops.load_ext` at it swaps the kernels without touching its backend.
Beyond the reference, `out` may also be float32 (the partial before its cast)
and the host-core kernel needs AVX2/FMA/F16C (has_avx2() reports it; calls
raise otherwise).
"""

from __future__ import annotations

import os
import sys

import torch

from . import _lib, ops

_DT = {torch.float16: _lib.FD_F16, torch.bfloat16: _lib.FD_BF16, torch.float32: _lib.FD_F32}


def _check_cpu_contig(t: torch.Tensor, name: str) -> None:
    # cpu_attn.cpp:433-436
    if t.device.type != "cpu":
        raise RuntimeError(f"{name} must be a CPU tensor")
    if not t.is_contiguous():
        raise RuntimeError(f"{name} must be contiguous")


def decode_attn(q, k_cache, v_cache, block_table, lens, scale, out, lse) -> None:
    """Partial decode attention over each row's listed host-tier blocks
    (cpu_attn.cpp:456-489): out [n, H, D] (q's dtype, or float32), lse [H, n]
    float32; a row with lens <= 0 gives out = 0, lse = -inf."""
    for t, name in ((q, "q"), (k_cache, "k_cache"), (v_cache, "v_cache"),
                    (block_table, "block_table"), (lens, "lens"), (out, "out"), (lse, "lse")):
        _check_cpu_contig(t, name)
    if not (q.dim() == 3 and k_cache.dim() == 4 and v_cache.shape == k_cache.shape):
        raise RuntimeError("q must be [n, H, D] and k_cache/v_cache [C, KVH, BS, D]")
    if block_table.dtype != torch.int32 or lens.dtype != torch.int32:
        raise RuntimeError("block_table and lens must be int32")
    if lse.dtype != torch.float32:
        raise RuntimeError("lse must be float32")
    if q.dtype != k_cache.dtype or (out.dtype != q.dtype and out.dtype != torch.float32):
        raise RuntimeError("q, the caches and out must share a dtype (or out float32)")
    n, H, D = q.shape
    KVH = k_cache.shape[1]
    if k_cache.shape[3] != D:
        raise RuntimeError("head size mismatch")
    if H % KVH != 0:
        raise RuntimeError("num_heads must be a multiple of num_kv_heads")
    if not (block_table.dim() == 2 and block_table.shape[0] == n and lens.shape[0] == n):
        raise RuntimeError("block_table must be [n, W] and lens [n]")
    if out.shape != q.shape or tuple(lse.shape) != (H, n):
        raise RuntimeError("out must be [n, H, D] and lse [H, n]")
    if n == 0:
        return
    ops.host_decode_attn(q, k_cache, v_cache, block_table, lens, float(scale), out, lse)


def store_kv(k, v, slots, k_cache, v_cache) -> None:
    """Host-tier slot write (cpu_attn.cpp:491-517): every slot is checked
    against the cache's capacity before any write."""
    for t, name in ((k, "k"), (v, "v"), (slots, "slots"), (k_cache, "k_cache"),
                    (v_cache, "v_cache")):
        _check_cpu_contig(t, name)
    if slots.dtype != torch.int64:
        raise RuntimeError("slots must be int64")
    if k.dtype != k_cache.dtype or v.dtype != k.dtype or v_cache.dtype != k_cache.dtype:
        raise RuntimeError("k, v and the caches must share a dtype")
    m = k.shape[0]
    if m == 0:
        return
    if k.dtype not in _DT:
        raise RuntimeError(f"store_kv: unsupported dtype {k.dtype}")
    C, KVH, BS, D = k_cache.shape
    if not (k.dim() == 3 and k.shape[1] == KVH and k.shape[2] == D and v.shape == k.shape
            and v_cache.shape == k_cache.shape and slots.shape == (m,)):
        raise RuntimeError("k, v must be [m, KVH, D] and slots [m] for [C, KVH, BS, D] caches")
    _lib.check(
        _lib.load_lib().fd_host_store_kv(
            k.data_ptr(), k.stride(0), k.stride(1), v.data_ptr(), v.stride(0), v.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
            C, slots.data_ptr(), m, KVH, D, BS, _DT[k.dtype],
        )
    )


def set_num_threads(n: int) -> None:
    """Worker count of the host-core kernels for this process (n <= 0: the
    default, one per CPU of the affinity mask; cpu_attn.cpp:521)."""
    _lib.check(_lib.load_lib().fd_host_set_threads(int(n)))


def get_num_threads() -> int:
    return int(_lib.load_lib().fd_host_decode_threads())


def has_avx2() -> bool:
    """Whether this CPU runs the host-core kernel (AVX2, FMA and F16C)."""
    return _lib.load_lib().fd_host_decode_isa() >= 256


def load_ext(verbose: bool = False):
    """cpu_ops.load_ext's contract (cpu_ops.py:21-46): the loaded module, with
    FASTDECODE_CPU_THREADS applied. Nothing is compiled at run time; the
    library is built in-tree ahead of time."""
    _lib.load_lib()
    nt = os.environ.get("FASTDECODE_CPU_THREADS")
    if nt:
        set_num_threads(int(nt))
    return sys.modules[__name__]
