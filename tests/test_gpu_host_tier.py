"""Pinned host-tier blocks on the GPU: fd_host_free waits for the work still
queued on the tier's device before the block goes (the tier lives as long as
the worker, fastdecode/state.py:66-71; here its memory is read in place by
kernels, so a free must not overtake them)."""

from __future__ import annotations

import ctypes

import pytest
import torch

from vllm_fastdecoder_amd import _lib

pytestmark = pytest.mark.gpu


def test_free_after_use_waits_for_the_reader(gpu):
    """A 256 MiB block read over the link by a copy kernel (several ms) and
    freed right after the launch, with no synchronisation: the copy's result
    is whole, so the free waited for it. A second free of the same block is
    an argument error."""
    lib = _lib.load_lib()
    nbytes = 256 << 20
    host = ctypes.c_void_p()
    assert lib.fd_host_alloc(nbytes, ctypes.byref(host)) == _lib.FD_OK
    freed = False
    try:
        src = torch.frombuffer((ctypes.c_uint8 * nbytes).from_address(host.value),
                               dtype=torch.uint8)
        pattern = torch.arange(nbytes // 4, dtype=torch.int32).view(torch.uint8)
        src.copy_(pattern)
        dev = ctypes.c_void_p()
        assert lib.fd_host_device_pointer(host, ctypes.byref(dev)) == _lib.FD_OK
        dst = torch.zeros(nbytes, dtype=torch.uint8, device=gpu)
        torch.cuda.synchronize()
        stream = torch.cuda.current_stream(gpu)
        for _ in range(3):  # ~15 ms of reads queued
            assert lib.fd_stream_copy(ctypes.c_void_p(dst.data_ptr()), dev, nbytes,
                                      ctypes.c_void_p(stream.cuda_stream)) == _lib.FD_OK
        del src
        assert lib.fd_host_free(host) == _lib.FD_OK
        freed = True
        assert stream.query(), "fd_host_free returned before the tier's readers finished"
        assert torch.equal(dst.cpu(), pattern)
        assert lib.fd_host_free(host) == _lib.FD_ERR_INVALID
    finally:
        if not freed:
            torch.cuda.synchronize()
            lib.fd_host_free(host)
