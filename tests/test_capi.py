"""CPU checks of the C ABI (no GPU compute): the library loads, exports every
function include/fdattn.h declares, and its host-side argument validation
rejects bad calls before any launch (the TORCH_CHECK contract of
fastdecode/csrc/cpu_attn.cpp:433-477 and the slot rule of :506-510)."""

from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

from vllm_fastdecoder_amd import _lib

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "fdattn.h"


def declared_functions() -> list[str]:
    text = re.sub(r"/\*.*?\*/", "", HEADER.read_text(), flags=re.S)
    return sorted(set(re.findall(r"\b(fd_\w+)\s*\(", text)))


def test_header_declares_the_bound_signatures():
    assert declared_functions() == sorted(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.load_lib()
    for name in declared_functions():
        assert hasattr(lib, name), name
    assert lib.fd_abi_version() == _lib.ABI_VERSION


def test_check_slots_host_rule():
    lib = _lib.load_lib()
    good = (ctypes.c_int64 * 4)(0, 5, 31, 17)
    assert lib.fd_check_slots(good, 4, 32, None) == _lib.FD_OK
    bad = (ctypes.c_int64 * 4)(0, 5, 32, 17)
    first = ctypes.c_int64(-1)
    assert lib.fd_check_slots(bad, 4, 32, ctypes.byref(first)) == _lib.FD_ERR_RANGE
    assert first.value == 2
    assert b"out of range" in lib.fd_last_error()
    neg = (ctypes.c_int64 * 1)(-1)
    assert lib.fd_check_slots(neg, 1, 32, None) == _lib.FD_ERR_RANGE


def test_workspace_size_query():
    lib = _lib.load_lib()
    size = ctypes.c_size_t()
    # vicuna-7b shape (128 sequences, 32/32 heads, width 128 blocks): one
    # workgroup covers a whole row, no split partials
    assert lib.fd_paged_decode_workspace_size(128, 32, 32, 128, 16, 128, ctypes.byref(size)) == 0
    assert size.value == 0
    # 16k-token rows (1024 blocks) are split into tasks of at most 256 blocks:
    # 4 fp32 partials (out [D] + lse) per (sequence, head)
    assert lib.fd_paged_decode_workspace_size(128, 32, 32, 128, 16, 1024, ctypes.byref(size)) == 0
    parts = 128 * 32 * 4
    assert size.value >= parts * 128 * 4 + parts * 4
    # a head size the tiled kernel does not take needs no workspace
    assert lib.fd_paged_decode_workspace_size(7, 8, 8, 72, 16, 6, ctypes.byref(size)) == 0
    assert size.value == 0
    assert lib.fd_paged_decode_workspace_size(-1, 8, 8, 64, 16, 6, ctypes.byref(size)) != 0


def _decode(lib, **over):
    """fd_paged_decode_partial with plausible pointers (never dereferenced:
    every call here must be rejected by host validation)."""
    a = dict(q=16, qss=8 * 64, qsh=64, k=32, v=48, sb=4 * 16 * 64, sh=16 * 64, st=64, nblk=10,
             bt=64, bts=4, btw=4, lens=80, n=2, H=8, KVH=4, D=64, BS=16, scale=0.125, dt=0,
             out=96, oss=8 * 64, osh=64, odt=0, lse=112, lsh=2, ws=None, wsb=0)
    a.update(over)
    return lib.fd_paged_decode_partial(
        a["q"], a["qss"], a["qsh"], a["k"], a["v"], a["sb"], a["sh"], a["st"], a["nblk"],
        a["bt"], a["bts"], a["btw"], a["lens"], None, a["n"], a["H"], a["KVH"], a["D"], a["BS"],
        a["scale"], a["dt"], a["out"], a["oss"], a["osh"], a["odt"], a["lse"], a["lsh"],
        a["ws"], a["wsb"], None)


@pytest.mark.parametrize(
    "over,code",
    [
        (dict(H=6, KVH=4), _lib.FD_ERR_INVALID),          # H % KVH != 0
        (dict(n=-1), _lib.FD_ERR_INVALID),
        (dict(D=1024), _lib.FD_ERR_UNSUPPORTED),
        (dict(dt=7), _lib.FD_ERR_INVALID),
        (dict(odt=1), _lib.FD_ERR_INVALID),                # out bf16 with fp16 KV
        (dict(q=None), _lib.FD_ERR_INVALID),
        (dict(bts=2), _lib.FD_ERR_INVALID),                # row stride < width
        (dict(scale=float("nan")), _lib.FD_ERR_INVALID),
        (dict(BS=0), _lib.FD_ERR_INVALID),
        # a wide table splits rows, and the split partials need workspace
        (dict(ws=None, wsb=0, btw=256, bts=256), _lib.FD_ERR_WORKSPACE),
    ],
)
def test_decode_rejects_bad_arguments_on_host(over, code):
    lib = _lib.load_lib()
    assert _decode(lib, **over) == code
    assert lib.fd_last_error()


def test_decode_n_zero_is_a_no_op():
    assert _decode(_lib.load_lib(), n=0) == _lib.FD_OK


def test_merge_and_cache_write_reject_bad_arguments():
    lib = _lib.load_lib()
    assert lib.fd_merge_attn_states(16, 64, 64, 9, 16, 64, 64, 0, 16, 1, 16, 64, 64, 0, 16, 1,
                                    None, 0, 1, 1, 64, None) == _lib.FD_ERR_INVALID
    assert lib.fd_merge_attn_states(None, 64, 64, 0, 16, 64, 64, 0, 16, 1, 16, 64, 64, 0, 16, 1,
                                    None, 0, 1, 1, 64, None) == _lib.FD_ERR_INVALID
    assert lib.fd_merge_attn_states(None, 64, 64, 0, None, 64, 64, 0, None, 1, None, 64, 64, 0,
                                    None, 1, None, 0, 0, 1, 64, None) == _lib.FD_OK  # empty
    assert lib.fd_reshape_and_cache(16, 64, 64, 16, 64, 64, 16, 16, 1, 1, 1, 4, None, 3, 1, 64,
                                     16, 0, None, None, None) == _lib.FD_ERR_INVALID
    assert lib.fd_reshape_and_cache(16, 64, 64, 16, 64, 64, 16, 16, 1, 1, 1, 4, 16, 3, 0, 64,
                                    16, 0, None, None, None) == _lib.FD_ERR_INVALID
    # the write gate must be another counter than the one the launch adds to
    assert lib.fd_reshape_and_cache(16, 64, 64, 16, 64, 64, 16, 16, 1, 1, 1, 4, 16, 3, 1, 64,
                                    16, 0, 32, 32, None) == _lib.FD_ERR_INVALID
    assert b"write_gate" in lib.fd_last_error()
    assert lib.fd_stream_copy(16, 16, 17, None) == _lib.FD_ERR_INVALID
    assert lib.fd_host_device_pointer(None, None) == _lib.FD_ERR_INVALID


def _tier(**over):
    t = dict(k=32, v=48, sb=4 * 16 * 64, sh=16 * 64, st=64, nblk=10, bt=64, bts=4, btw=4, lens=80)
    t.update(over)
    return _lib.FdKvTier(t["k"], t["v"], t["sb"], t["sh"], t["st"], t["nblk"], t["bt"], t["bts"],
                         t["btw"], t["lens"])


def _split(lib, hbm=None, host=None, **over):
    """fd_split_decode with plausible pointers (never dereferenced: every call
    here must be rejected by host validation, or be a no-op)."""
    a = dict(q=16, qss=8 * 64, qsh=64, n=2, H=8, KVH=4, D=64, BS=16, scale=0.125, dt=0,
             out=96, oss=8 * 64, osh=64, odt=0, lse=112, lsh=2, ws=None, wsb=0)
    a.update(over)
    th = hbm if hbm is not None else _tier()
    tc = host if host is not None else _tier()
    return lib.fd_split_decode(
        a["q"], a["qss"], a["qsh"], ctypes.byref(th), ctypes.byref(tc), None, a["n"], a["H"],
        a["KVH"], a["D"], a["BS"], a["scale"], a["dt"], a["out"], a["oss"], a["osh"], a["odt"],
        a["lse"], a["lsh"], a["ws"], a["wsb"], None)


@pytest.mark.parametrize(
    "tiers,over,code",
    [
        (dict(host=_tier(bts=2)), {}, _lib.FD_ERR_INVALID),       # host row stride < width
        (dict(host=_tier(lens=None)), {}, _lib.FD_ERR_INVALID),   # host lens missing
        (dict(hbm=_tier(k=None)), {}, _lib.FD_ERR_INVALID),       # hbm cache missing
        (dict(host=_tier(nblk=-1)), {}, _lib.FD_ERR_INVALID),
        ({}, dict(H=6, KVH=4), _lib.FD_ERR_INVALID),
        ({}, dict(odt=1), _lib.FD_ERR_INVALID),
        # the two tables together are what a task splits over: 128 + 128 blocks
        # of 2 rows split, and the split partials need workspace
        (dict(hbm=_tier(btw=128, bts=128), host=_tier(btw=128, bts=128)), {},
         _lib.FD_ERR_WORKSPACE),
    ],
)
def test_split_decode_rejects_bad_arguments_on_host(tiers, over, code):
    lib = _lib.load_lib()
    assert _split(lib, **tiers, **over) == code
    assert lib.fd_last_error()


def test_split_decode_null_descriptor_and_n_zero():
    lib = _lib.load_lib()
    t = _tier()
    assert lib.fd_split_decode(16, 512, 64, None, ctypes.byref(t), None, 2, 8, 4, 64, 16, 0.125,
                               0, 96, 512, 64, 0, 112, 2, None, 0, None) == _lib.FD_ERR_INVALID
    # n == 0: nothing to do, even with NULL tier pointers
    assert _split(lib, hbm=_tier(k=None, lens=None), host=_tier(bt=None), n=0) == _lib.FD_OK


def test_host_entry_points_reject_bad_arguments():
    """fd_share_host_blocks / fd_host_store_kv / fd_host_set_threads through the
    C ABI: every invalid call returns a status and writes nothing."""
    import ctypes

    import torch

    lib = _lib.load_lib()
    bt = torch.tensor([[1, 2], [3, 4]], dtype=torch.int32)
    lens = torch.tensor([20, 5], dtype=torch.int32)
    gl = torch.full((2,), -7, dtype=torch.int32)
    cl = torch.full((2,), -7, dtype=torch.int32)
    cbt = torch.full((2, 2), -7, dtype=torch.int32)
    wc = ctypes.c_int32(-1)

    def share(frac, stride=2, cstride=2, n=2, bs=16, bt_ptr=bt.data_ptr()):
        return lib.fd_share_host_blocks(bt_ptr, stride, 2, lens.data_ptr(), n, bs, frac,
                                        gl.data_ptr(), cbt.data_ptr(), cstride, cl.data_ptr(),
                                        ctypes.byref(wc))

    for bad in (share(1.5), share(-0.1), share(float("nan")), share(0.5, stride=1),
                share(0.5, cstride=1), share(0.5, bs=0), share(0.5, n=-1), share(0.5, bt_ptr=None)):
        assert bad == _lib.FD_ERR_INVALID
    assert torch.all(gl == -7) and torch.all(cbt == -7) and wc.value == -1
    assert share(0.5) == _lib.FD_OK
    assert gl.tolist() == [16, 0] and cl.tolist() == [4, 5] and wc.value == 1
    assert cbt[:, :1].tolist() == [[2], [3]] and int(cbt[0, 1]) == 0

    kc = torch.zeros(2, 1, 16, 8, dtype=torch.float16)
    k = torch.ones(1, 1, 8, dtype=torch.float16)
    slots = torch.tensor([5], dtype=torch.int64)

    def store(dtype=_lib.FD_F16, m=1, kvh=1, ptr=k.data_ptr()):
        return lib.fd_host_store_kv(ptr, 8, 8, ptr, 8, 8, kc.data_ptr(), kc.data_ptr(),
                                    kc.stride(0), kc.stride(1), kc.stride(2), 2,
                                    slots.data_ptr(), m, kvh, 8, 16, dtype)

    assert store(dtype=7) == _lib.FD_ERR_INVALID
    assert store(m=-1) == _lib.FD_ERR_INVALID
    assert store(kvh=0) == _lib.FD_ERR_INVALID
    assert store(ptr=None) == _lib.FD_ERR_INVALID
    assert store(m=0, ptr=None) == _lib.FD_OK  # nothing to write
    assert not kc.any()
    assert store() == _lib.FD_OK and kc[0, 0, 5].tolist() == [1.0] * 8
    assert lib.fd_host_set_threads(0) == _lib.FD_OK


def test_host_free_takes_only_its_own_blocks():
    """fd_host_free: NULL is a no-op; a pointer fd_host_alloc did not make is
    rejected with FD_ERR_INVALID before any device is waited for or touched
    (the block registry is checked first; no GPU needed)."""
    lib = _lib.load_lib()
    assert lib.fd_host_free(None) == _lib.FD_OK
    buf = (ctypes.c_uint8 * 64)()
    assert lib.fd_host_free(ctypes.cast(buf, ctypes.c_void_p)) == _lib.FD_ERR_INVALID
    assert b"not allocated by fd_host_alloc" in lib.fd_last_error()


def test_missing_library_raises_instead_of_falling_back(monkeypatch, tmp_path):
    """Without the built library every entry point raises: there is no
    CPU or PyTorch path behind the kernels."""
    from vllm_fastdecoder_amd import ops

    monkeypatch.setattr(_lib, "_LIB", None)
    monkeypatch.setattr(_lib, "LIB_PATH", tmp_path / "libfdattn.so")
    with pytest.raises(RuntimeError, match="missing.*no fallback"):
        _lib.load_lib()
    monkeypatch.setattr(ops, "_WS_SIZES", {})
    with pytest.raises(RuntimeError, match="missing"):
        ops.workspace_bytes(3, 8, 8, 64, 16, 5)
