"""GPU check of the allocation-free decode entry point
(fd_paged_decode_partial_noalloc) through the C ABI.

Its results must be bit-identical to fd_paged_decode_partial's with a
caller-allocated workspace (same kernels, same task split), on two calls in a
row, the second smaller, at shapes whose rows are long enough to split into
several tasks (so the split partials go through the library's device scratch
and the combine kernel). Both calls use long rows of a grouped-query and an
MHA shape; each result is also checked against the float64 oracle.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

import oracle
from tests import cases
from vllm_fastdecoder_amd import _lib

pytestmark = pytest.mark.gpu


def _workspace_bytes(n, H, KVH, D, BS, W):
    size = ctypes.c_size_t()
    _lib.check(_lib.load_lib().fd_paged_decode_workspace_size(n, H, KVH, D, BS, W,
                                                              ctypes.byref(size)))
    return int(size.value)


def _call(noalloc, q, kc, vc, bt, lens, scale, out, lse, ws=None):
    """One decode through the C ABI on torch's current stream; the caches are
    [C, KVH, BS, D] in HBM."""
    lib = _lib.load_lib()
    C, KVH, BS, D = kc.shape
    n, H, _ = q.shape
    stream = torch.cuda.current_stream(q.device).cuda_stream
    head = (q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
            kc.stride(0), kc.stride(1), kc.stride(2), C, bt.data_ptr(), bt.stride(0),
            bt.shape[1], lens.data_ptr(), None, n, H, KVH, D, BS, float(scale),
            {torch.float16: _lib.FD_F16, torch.bfloat16: _lib.FD_BF16,
             torch.float32: _lib.FD_F32}[q.dtype],
            out.data_ptr(), out.stride(0), out.stride(1), _lib.FD_F32,
            lse.data_ptr(), lse.stride(0))
    if noalloc:
        rc = lib.fd_paged_decode_partial_noalloc(*head, stream)
    else:
        rc = lib.fd_paged_decode_partial(*head, ws.data_ptr(), ws.numel(), stream)
    _lib.check(rc)


def _case(n, H, KVH, D, dtype, lo, hi, seed, dev):
    """n rows of lo..hi tokens over a pool holding every row's blocks."""
    BS = 16
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=g, dtype=torch.int32)
    nb = (lens + BS - 1) // BS
    W = int(nb.max())
    C = int(nb.sum())
    perm = torch.randperm(C, generator=g).to(torch.int32)
    bt = torch.zeros(n, W, dtype=torch.int32)
    pos = 0
    for i in range(n):
        bt[i, : nb[i]] = perm[pos : pos + nb[i]]
        pos += int(nb[i])
    q = torch.randn(n, H, D, generator=g).to(dtype)
    kc = torch.randn(C, KVH, BS, D, generator=g).to(dtype)
    vc = torch.randn(C, KVH, BS, D, generator=g).to(dtype)
    return q, kc, vc, bt, lens


@pytest.mark.parametrize("H,KVH,dtype", [(32, 8, torch.bfloat16), (32, 32, torch.float16),
                                         (16, 2, torch.float32)])
def test_noalloc_matches_workspace_entry_point(gpu, H, KVH, dtype):
    D = 128
    scale = 1.0 / math.sqrt(D)
    # two calls in a row on one stream, the second with fewer and shorter rows
    shapes = [(4, 6000, 9000, 11), (2, 2000, 4000, 12)]
    for n, lo, hi, seed in shapes:
        q, kc, vc, bt, lens = _case(n, H, KVH, D, dtype, lo, hi, seed, gpu)
        need = _workspace_bytes(n, H, KVH, D, 16, bt.shape[1])
        print(f"noalloc: H={H} KVH={KVH} {dtype} n={n} W={bt.shape[1]} workspace={need}",
              flush=True)
        assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES, need  # rows split into tasks
        qd, kd, vd = q.to(gpu), kc.to(gpu), vc.to(gpu)
        btd, ld = bt.to(gpu), lens.to(gpu)
        ws = torch.empty(need, dtype=torch.uint8, device=gpu)
        outs = []
        for noalloc in (False, True):
            out = torch.full((n, H, D), 7.0, device=gpu)
            lse = torch.full((H, n), 7.0, device=gpu)
            _call(noalloc, qd, kd, vd, btd, ld, scale, out, lse, ws)
            outs.append((out, lse))
        torch.cuda.synchronize()
        (o_ws, l_ws), (o_na, l_na) = outs
        assert torch.equal(o_na, o_ws)
        assert torch.equal(l_na, l_ws)
        ref_o, ref_l = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
        assert float((o_na.double().cpu() - ref_o).abs().max()) <= 2e-3
        rel = (l_na.double().cpu() - ref_l).abs() / ref_l.abs().clamp(min=1)
        assert float(rel.max()) <= 1e-4


def test_noalloc_rejects_sizes_beyond_its_scratch(gpu):
    """A shape whose split workspace exceeds the scratch is refused before
    anything is written."""
    n, H, KVH, D, BS = 64, 64, 64, 128, 16
    W = 1 << 14  # 256k-token rows: many split partials per (sequence, head)
    need = _workspace_bytes(n, H, KVH, D, BS, W)
    assert need > _lib.NOALLOC_SCRATCH_BYTES
    q = torch.zeros(n, H, D, dtype=torch.float16, device=gpu)
    kc = torch.zeros(1, KVH, BS, D, dtype=torch.float16, device=gpu)
    bt = torch.zeros(n, W, dtype=torch.int32, device=gpu)
    lens = torch.ones(n, dtype=torch.int32, device=gpu)
    out = torch.full((n, H, D), 7.0, device=gpu)
    lse = torch.full((H, n), 7.0, device=gpu)
    with pytest.raises(_lib.FdError) as e:
        _call(True, q, kc, kc, bt, lens, 0.1, out, lse)
    assert e.value.status == _lib.FD_ERR_WORKSPACE
    assert "scratch" in str(e.value)
    torch.cuda.synchronize()
    assert torch.all(out == 7.0) and torch.all(lse == 7.0)


@pytest.mark.parametrize("H,KVH,dtype", [(32, 8, torch.bfloat16), (32, 32, torch.float16)])
def test_noalloc_in_a_graph_matches_eager(gpu, H, KVH, dtype):
    """The entry point's use case: code under HIP graph capture. One eager
    call first (the device's scratch address and launch settings are looked
    up then), then the same call captured in a torch.cuda.CUDAGraph on a side
    stream, for a shape whose rows split (the scratch holds split partials).
    Each replay, with new queries and eager GPU work in between, is
    bit-identical to an eager call on the same inputs."""
    D = 128
    n = 3
    scale = 1.0 / math.sqrt(D)
    q, kc, vc, bt, lens = _case(n, H, KVH, D, dtype, 5000, 8000, 21, gpu)
    need = _workspace_bytes(n, H, KVH, D, 16, bt.shape[1])
    assert 0 < need <= _lib.NOALLOC_SCRATCH_BYTES, need
    qd, kd, vd = q.to(gpu), kc.to(gpu), vc.to(gpu)
    btd, ld = bt.to(gpu), lens.to(gpu)
    out = torch.empty((n, H, D), device=gpu)
    lse = torch.empty((H, n), device=gpu)
    _call(True, qd, kd, vd, btd, ld, scale, out, lse)
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=gpu)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        _call(True, qd, kd, vd, btd, ld, scale, out, lse)
    gen = torch.Generator(device=gpu).manual_seed(3)
    x = torch.randn(256, 256, device=gpu)
    for r in range(3):
        qd.copy_(torch.randn(qd.shape, generator=gen, device=gpu).to(dtype))
        g.replay()
        torch.cuda.synchronize()
        got = (out.clone(), lse.clone())
        x = torch.tanh(x @ x) * 0.5  # eager work between the replay and the check
        _call(True, qd, kd, vd, btd, ld, scale, out, lse)
        torch.cuda.synchronize()
        assert torch.equal(got[0], out) and torch.equal(got[1], lse), f"replay {r}"
    assert torch.isfinite(x).all()
    del g
