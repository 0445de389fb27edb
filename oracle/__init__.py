"""CPU oracle for the split decode-attention path.

TEST INFRASTRUCTURE ONLY. Only tests/, __graft_entry__.smoke() and the CPU
baseline leg of bench.py import this package, and only as the checker (or
as the timed CPU baseline). The product package never imports it.

Contents:
  * ctypes bindings of liboracle.so (fd_oracle.c): the float64 closed form of
    the partial, the fp32 two-pass restatement of the reference's CPU
    kernel, the float64 merge and the slot-mapping write;
  * `ref_ext()`: the reference's own cpu_attn.cpp extension, compiled by
    oracle/Makefile into oracle/_ref (None when that build is absent);
  * `plan_oracle`: numpy restatement of the per-step block selection.

Parity status of each function is stated in plan_oracle.py and fd_oracle.c
and checked by tests/test_oracle.py.
"""

from __future__ import annotations

import ctypes
import importlib
import subprocess
import sys
from ctypes import c_double, c_float, c_int, c_int32, c_int64, c_void_p
from pathlib import Path

import torch

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "liboracle.so"
REF_DIR = HERE / "_ref"

_DT = {torch.float16: 0, torch.bfloat16: 1, torch.float32: 2}
_LIB = None
_REF = False  # False = not looked up yet


def build(verbose: bool = False) -> None:
    """make -C oracle (liboracle.so, plus _ref/ when the reference is present)."""
    res = subprocess.run(["make", "-C", str(HERE), "all"], capture_output=True, text=True)
    if verbose:
        print(res.stdout, res.stderr)
    if res.returncode != 0:
        raise RuntimeError(f"oracle build failed:\n{res.stdout}\n{res.stderr}")


def lib():
    global _LIB
    if _LIB is None:
        if not LIB_PATH.exists():
            build()
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_decode_attn_f64.restype = c_int
        L.oracle_decode_attn_f64.argtypes = [
            c_void_p, c_int64, c_int64, c_void_p, c_void_p, c_int64, c_int64, c_int64,
            c_int64, c_void_p, c_int64, c_int32, c_void_p, c_int, c_int, c_int, c_int, c_int,
            c_double, c_int, c_void_p, c_void_p, c_int,
        ]
        L.oracle_decode_attn_cpu_f32.restype = None
        L.oracle_decode_attn_cpu_f32.argtypes = [
            c_void_p, c_void_p, c_void_p, c_void_p, c_void_p, c_int, c_int, c_int, c_int, c_int,
            c_int, c_float, c_int, c_void_p, c_void_p, c_int,
        ]
        L.oracle_merge_f64.restype = None
        L.oracle_merge_f64.argtypes = [
            c_void_p, c_int, c_void_p, c_void_p, c_int, c_void_p, c_int, c_int, c_int,
            c_void_p, c_void_p,
        ]
        L.oracle_cache_write.restype = c_int
        L.oracle_cache_write.argtypes = [
            c_void_p, c_int64, c_int64, c_void_p, c_int64, c_int64, c_void_p, c_void_p,
            c_int64, c_int64, c_int64, c_int64, c_void_p, c_int, c_int, c_int, c_int, c_int,
            c_int, ctypes.POINTER(c_int64),
        ]
        L.oracle_num_threads.restype = c_int
        _LIB = L
    return _LIB


def ref_ext():
    """The reference's compiled cpu_attn.cpp extension, or None."""
    global _REF
    if _REF is False:
        _REF = None
        if any(REF_DIR.glob("fastdecode_cpu_ref*.so")):
            if str(REF_DIR) not in sys.path:
                sys.path.insert(0, str(REF_DIR))
            try:
                _REF = importlib.import_module("fastdecode_cpu_ref")
            except ImportError:
                _REF = None
    return _REF


def _cpu(t: torch.Tensor) -> torch.Tensor:
    return t.detach().to("cpu")


HOST_DIMS = (0, 1, 2)  # [C, KVH, BS, D]: block, head, token dims
VLLM_DIMS = (0, 2, 1)  # [B, BS, KVH, D]


def decode_attn_f64(q, k_cache, v_cache, dims, block_table, lens, scale, threads: int = 0):
    """float64 closed-form partial (cpu_ops.py:54-81 semantics) over 4-D caches
    whose (block, kv head, token) dimensions are `dims` (head_size last).
    Returns (out [n,H,D] f64, lse [H,n] f64, status) on the CPU; status 2
    flags a range error (those rows are NaN)."""
    q = _cpu(q).contiguous()
    k = _cpu(k_cache)
    v = _cpu(v_cache)
    assert k.shape == v.shape and k.stride(3) == 1 and v.stride(3) == 1
    if k.stride() != v.stride():
        k, v = k.contiguous(), v.contiguous()
    bt = _cpu(block_table).to(torch.int32).contiguous()
    ln = _cpu(lens).to(torch.int32).contiguous()
    n, H, D = q.shape
    sb, sh, st_ = (k.stride(d) for d in dims)
    num_blocks, KVH, BS = (k.shape[d] for d in dims)
    out = torch.empty(n, H, D, dtype=torch.float64)
    lse = torch.empty(H, n, dtype=torch.float64)
    st = lib().oracle_decode_attn_f64(
        q.data_ptr(), q.stride(0), q.stride(1), k.data_ptr(), v.data_ptr(), sb, sh, st_,
        num_blocks, bt.data_ptr(), bt.stride(0), bt.shape[1], ln.data_ptr(), n, H, KVH, D, BS,
        float(scale), _DT[q.dtype], out.data_ptr(), lse.data_ptr(), threads)
    return out, lse, st


def decode_attn_host_layout_f64(q, k_cache, v_cache, block_table, lens, scale):
    """Same, for the reference's host-tier layout [C, KVH, BS, D]."""
    out, lse, _ = decode_attn_f64(q, k_cache, v_cache, HOST_DIMS, block_table, lens, scale)
    return out, lse


def decode_attn_cpu_f32(q, k_cache, v_cache, block_table, lens, scale, out, lse,
                        threads: int = 0) -> None:
    """fp32 two-pass CPU kernel (restatement of cpu_attn.cpp:298-411);
    contiguous [C, KVH, BS, D] caches; out float32 [n,H,D], lse float32 [H,n]."""
    C, KVH, BS, D = k_cache.shape
    n, H, _ = q.shape
    for t in (q, k_cache, v_cache, block_table, lens, out, lse):
        assert t.is_contiguous() and not t.is_cuda
    assert out.dtype == torch.float32 and lse.dtype == torch.float32
    lib().oracle_decode_attn_cpu_f32(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
        lens.data_ptr(), n, H, KVH, D, BS, block_table.shape[1], float(scale), _DT[q.dtype],
        out.data_ptr(), lse.data_ptr(), threads)


_DT_MERGE = {**_DT, torch.float64: 3}


def merge_f64(o_a, lse_a, o_b, lse_b):
    """float64 LSE merge (cpu_ops.py:93-113) of partials in fp16/bf16/fp32 or
    float64 (the oracle's own). Returns (out [n,H,D], lse [H,n])."""
    o_a = _cpu(o_a).contiguous()
    o_b = _cpu(o_b).contiguous()
    la = _cpu(lse_a).double().contiguous()
    lb = _cpu(lse_b).double().contiguous()
    n, H, D = o_a.shape
    out = torch.empty(n, H, D, dtype=torch.float64)
    olse = torch.empty(H, n, dtype=torch.float64)
    lib().oracle_merge_f64(o_a.data_ptr(), _DT_MERGE[o_a.dtype], la.data_ptr(), o_b.data_ptr(),
                           _DT_MERGE[o_b.dtype], lb.data_ptr(), n, H, D, out.data_ptr(),
                           olse.data_ptr())
    return out, olse


def cache_write(key, value, k_cache, v_cache, strides_btg, num_blocks, block_size, slots,
                check_all: bool):
    """Byte-exact slot write into CPU copies of the caches (modified in place).
    Returns (status, n_out_of_range); status 2 = rejected before any write."""
    key = _cpu(key)
    value = _cpu(value)
    slots = _cpu(slots).to(torch.int64).contiguous()
    assert not k_cache.is_cuda and not v_cache.is_cuda
    T, KVH, D = key.shape
    oor = c_int64(0)
    st = lib().oracle_cache_write(
        key.data_ptr(), key.stride(0), key.stride(1), value.data_ptr(), value.stride(0),
        value.stride(1), k_cache.data_ptr(), v_cache.data_ptr(), strides_btg[0],
        strides_btg[1], strides_btg[2], num_blocks, slots.data_ptr(), T, KVH, D, block_size,
        key.element_size(), int(check_all), ctypes.byref(oor))
    return st, int(oor.value)
