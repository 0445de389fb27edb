"""Pinned, GPU-mapped host memory for the host KV tier.

The reference keeps its host tier in pageable `torch.zeros` tensors and moves
every per-layer transfer through pinned staging buffers (fastdecode/state.py:
66-71, 93-124). Here the tier itself lives in hipHostMalloc'd memory mapped
into the GPU's address space, so the decode and cache-write kernels read and
write it in place over the host link: no staging copy, no host-side compute.

`pinned_empty` returns an ordinary CPU tensor over such an allocation;
`device_ptr` translates any view of it to the address the GPU uses.
"""

from __future__ import annotations

import bisect
import ctypes
import threading
import weakref

import torch

from . import _lib

_REG_LOCK = threading.Lock()
_STARTS: list[int] = []          # sorted host start addresses
_RANGES: dict[int, tuple[int, int]] = {}  # host start -> (nbytes, device start)
# blocks whose last view died while a stream capture was under way: freeing
# waits for the device, which a capture forbids, so they are freed by the
# next allocation or free_deferred() outside capture
_DEFERRED: list[int] = []


def _capturing() -> bool:
    try:
        return torch.cuda.is_available() and torch.cuda.is_current_stream_capturing()
    except RuntimeError:
        return False


def free_deferred() -> None:
    """Frees the blocks released during a stream capture (no-op inside one)."""
    if _capturing():
        return
    with _REG_LOCK:
        todo = list(_DEFERRED)
        _DEFERRED.clear()
    for host in todo:
        _free(host)


def _free(host: int) -> None:
    lib = _lib.load_lib()
    if lib.fd_host_free(ctypes.c_void_p(host)) != _lib.FD_OK and \
            b"block kept" in (lib.fd_last_error() or b""):
        with _REG_LOCK:  # a wait failed and the block was kept: retry later
            _DEFERRED.append(host)


class _Allocation:
    """Owns one fd_host_alloc block; freed when the last tensor view dies."""

    def __init__(self, nbytes: int):
        free_deferred()
        lib = _lib.load_lib()
        host = ctypes.c_void_p()
        _lib.check(lib.fd_host_alloc(nbytes, ctypes.byref(host)))
        dev = ctypes.c_void_p()
        try:
            _lib.check(lib.fd_host_device_pointer(host, ctypes.byref(dev)))
        except Exception:
            lib.fd_host_free(host)
            raise
        self.host = int(host.value)
        self.dev = int(dev.value)
        self.nbytes = nbytes
        with _REG_LOCK:
            bisect.insort(_STARTS, self.host)
            _RANGES[self.host] = (nbytes, self.dev)

    def release(self) -> None:
        with _REG_LOCK:
            if self.host in _RANGES:
                del _RANGES[self.host]
                _STARTS.remove(self.host)
            if _capturing():
                _DEFERRED.append(self.host)
                return
        _free(self.host)


def pinned_empty(shape, dtype: torch.dtype, zero: bool = False) -> torch.Tensor:
    """CPU tensor backed by pinned host memory that the GPU can address."""
    numel = 1
    for s in shape:
        numel *= int(s)
    elt = torch.empty((), dtype=dtype).element_size()
    nbytes = max(numel * elt, 16)
    alloc = _Allocation(nbytes)
    buf = (ctypes.c_uint8 * nbytes).from_address(alloc.host)
    flat = torch.frombuffer(buf, dtype=torch.uint8)
    t = flat[: numel * elt].view(dtype).view(tuple(int(s) for s in shape))
    # free the block once the tensor (and so the ctypes buffer) is gone
    weakref.finalize(buf, alloc.release)
    if zero:
        t.zero_()
    return t


def pinned_zeros(shape, dtype: torch.dtype) -> torch.Tensor:
    return pinned_empty(shape, dtype, zero=True)


def device_ptr(t: torch.Tensor) -> int:
    """GPU address of a tensor: its data pointer if it lives on the GPU, the
    mapped address if it is a view of pinned host memory. Pageable host
    memory is rejected (the kernels cannot reach it)."""
    if t.is_cuda:
        return t.data_ptr()
    p = t.data_ptr()
    with _REG_LOCK:
        k = bisect.bisect_right(_STARTS, p) - 1
        if k >= 0:
            start = _STARTS[k]
            nbytes, dev = _RANGES[start]
            end = p + max(t.numel(), 1) * t.element_size()
            if p + 0 >= start and end <= start + nbytes:
                return dev + (p - start)
    if t.numel() > 0 and t.is_pinned():
        # pinned by torch's own host allocator
        dev = ctypes.c_void_p()
        _lib.check(_lib.load_lib().fd_host_device_pointer(ctypes.c_void_p(p), ctypes.byref(dev)))
        return int(dev.value)
    raise RuntimeError(
        "host-tier tensor must live in pinned memory (vllm_fastdecoder_amd.pinned.pinned_empty "
        "or pin_memory=True); the GPU cannot read pageable memory"
    )
