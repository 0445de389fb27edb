"""Parity of the host-core partial decode (fd_host_decode_partial /
ops.host_decode_attn) against the float64 oracle. Runs on the CPU.

The host cores compute the reference's decode_attn (fastdecode/csrc/
cpu_attn.cpp:298-411) over host-memory caches, so the tolerances are the GPU
partial's:
  * fp32 output: max |out - oracle| <= 2e-3 (16-bit KV, fp32 accumulation);
  * output in the KV dtype: fp16 2e-3, bf16 1.6e-2 (atol and rtol, the
    reference's tests/test_cpu_kernel.py:53), fp32 KV 1e-5;
  * lse: |lse - oracle| <= 1e-4 * max(1, |oracle|);
  * empty rows: out exactly 0, lse exactly -inf; range errors: NaN rows.
Work items are independent, so results are bit-identical for every thread
count.
"""

from __future__ import annotations

import ctypes
import math

import pytest
import torch

import oracle
from tests import cases
from vllm_fastdecoder_amd import _lib, ops

OUT_TOL_16BIT = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}


@pytest.fixture(params=["widest", "avx512", "avx2"])
def isa(request, monkeypatch):
    """Each case on every kernel body this CPU runs: the widest (AVX-512 with
    bf16 pair dot products where the CPU has them), plain AVX-512, AVX2."""
    lib = _lib.load_lib()
    monkeypatch.delenv("FASTDECODE_CPU_ISA", raising=False)
    widest = lib.fd_host_decode_isa()
    if request.param == "avx2":
        monkeypatch.setenv("FASTDECODE_CPU_ISA", "avx2")
        assert lib.fd_host_decode_isa() == 256
    elif request.param == "avx512":
        if widest != 512:
            pytest.skip("no AVX-512 on this CPU")
        monkeypatch.setenv("FASTDECODE_CPU_ISA", "avx512")
        assert lib.fd_host_decode_isa() == 512
    else:
        assert widest in (256, 512)
    return request.param


def run(q, kc, vc, bt, lens, scale, out_dtype, threads=0):
    n, H, D = q.shape
    out = torch.full((n, H, D), 7.0, dtype=out_dtype)
    lse = torch.full((H, n), 7.0, dtype=torch.float32)
    ops.host_decode_attn(q, kc, vc, bt, lens, scale, out, lse, num_threads=threads)
    return out, lse


def check(out, lse, ref_out, ref_lse, lens, kv_dtype):
    nz = lens > 0
    o = out.double()
    if out.dtype == torch.float32 and kv_dtype != torch.float32:
        err = float((o[nz] - ref_out[nz]).abs().max()) if nz.any() else 0.0
        assert err <= 2e-3, err
    else:
        tol = OUT_TOL_16BIT[kv_dtype]
        if nz.any():
            err = float(((o[nz] - ref_out[nz]).abs() - tol * ref_out[nz].abs()).max())
            assert err <= tol, err
    if nz.any():
        lerr = (lse.double()[:, nz] - ref_lse[:, nz]).abs() / ref_lse[:, nz].abs().clamp(min=1.0)
        assert float(lerr.max()) <= 1e-4, float(lerr.max())
    assert torch.all(out[~nz] == 0)
    assert torch.all(torch.isneginf(lse[:, ~nz]))


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,KVH", [(8, 8), (8, 2), (4, 1), (6, 2), (12, 2), (16, 1), (7, 1)])
@pytest.mark.parametrize("D", [64, 128, 72, 20])
def test_host_decode_matches_oracle(dtype, H, KVH, D, isa):
    """The reference's kernel grid (tests/test_cpu_kernel.py:38-57), plus
    query-head groups that are not powers of two or exceed 8 (several passes
    over the KV) and head sizes that are not multiples of 8 or 16."""
    n, BS, C = 7, 16, 64
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len=93, seed=D + H)
    lens[3] = 0
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    for out_dtype in (dtype, torch.float32):
        out, lse = run(q, kc, vc, bt, lens, scale, out_dtype)
        check(out, lse, ref_out, ref_lse, lens, dtype)


@pytest.mark.parametrize("BS", [1, 4, 8, 32])
def test_host_decode_block_sizes(BS, isa):
    dtype = torch.bfloat16
    q, kc, vc, bt, lens = cases.rand_case(5, 8, 2, 128, BS, 200, dtype, max_len=150, seed=BS)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, 0.09)
    out, lse = run(q, kc, vc, bt, lens, 0.09, torch.float32)
    check(out, lse, ref_out, ref_lse, lens, dtype)


def test_host_decode_large_scores(isa):
    """q x 300: the running max keeps every value finite
    (test_cpu_kernel.py:60-72)."""
    for dtype, D in ((torch.float32, 64), (torch.float16, 128)):
        q, kc, vc, bt, lens = cases.rand_case(2, 4, 4, D, 16, 8, torch.float32, 40, 0)
        q = (q * 300.0).to(dtype)
        kc, vc = kc.to(dtype), vc.to(dtype)
        ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, 1.0)
        out, lse = run(q, kc, vc, bt, lens, 1.0, torch.float32)
        assert torch.isfinite(out).all() and torch.isfinite(lse).all()
        assert float((out.double() - ref_out).abs().max()) <= (1e-3 if dtype == torch.float16
                                                               else 1e-4)
        assert float((lse.double() - ref_lse).abs().max()) <= 1e-3 * float(ref_lse.abs().max())


def test_host_decode_matches_reference_cpu_kernel_restatement():
    """Against the oracle's fp32 two-pass restatement of cpu_attn.cpp:298-411
    on the correctness workload shape (n=8, 32/32 heads, D=128, fp16)."""
    w = cases.WORKLOADS["correctness"]
    lens, bt, pool = cases.draw_lens_and_tables(w)
    k, v, _ = cases.kv_pool(w, pool, "host", "cpu")
    q = cases.queries(w, "cpu")
    n, H, D = q.shape
    ref_o = torch.empty(n, H, D)
    ref_l = torch.empty(H, n)
    oracle.decode_attn_cpu_f32(q, k, v, bt.contiguous(), lens, w.scale, ref_o, ref_l)
    out, lse = run(q, k, v, bt, lens, w.scale, torch.float32)
    assert float((out - ref_o).abs().max()) <= 2e-3
    assert float(((lse - ref_l).abs() / ref_l.abs().clamp(min=1)).max()) <= 1e-4


def test_host_decode_thread_counts_bit_identical(isa):
    q, kc, vc, bt, lens = cases.rand_case(23, 8, 2, 128, 16, 300, torch.float16, 400, 9)
    base = run(q, kc, vc, bt, lens, 0.1, torch.float32, threads=1)
    for t in (2, 3, 8, 64):
        o, l = run(q, kc, vc, bt, lens, 0.1, torch.float32, threads=t)
        assert torch.equal(o, base[0]) and torch.equal(l, base[1]), t
    assert _lib.load_lib().fd_host_decode_threads() >= 1


@pytest.mark.parametrize("H,KVH", [(32, 32), (12, 6), (32, 8)])
def test_host_decode_head_groups_bit_identical(H, KVH, isa):
    """A work item covers a group of adjacent kv heads of one row, the more
    the fewer workers there are (9 rows: every kv head at 1 thread, down to
    one kv head at 64), with a shorter last group when the group size does not
    divide KVH. Every grouping gives the same bits and the oracle's values,
    and a row with a block id outside the cache is NaN in every head."""
    n, D, BS, C = 9, 64, 16, 120
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, torch.float16, 200, KVH)
    lens[2] = 0
    lens[5] = max(int(lens[5]), 40)
    bad = bt.clone()
    bad[5, 1] = C + 3
    base = run(q, kc, vc, bad, lens, 0.125, torch.float32, threads=1)
    for t in (2, 3, 4, 8, 16, 64):
        o, l = run(q, kc, vc, bad, lens, 0.125, torch.float32, threads=t)
        assert torch.equal(o.nan_to_num(9.0), base[0].nan_to_num(9.0)), t
        assert torch.equal(l.nan_to_num(9.0), base[1].nan_to_num(9.0)), t
    ok = torch.ones(n, dtype=torch.bool)
    ok[5] = False
    assert torch.isnan(base[0][5]).all() and torch.isnan(base[1][:, 5]).all()
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q[ok], kc, vc, bt[ok], lens[ok], 0.125)
    check(base[0][ok], base[1][:, ok], ref_out, ref_lse, lens[ok], torch.float16)


def test_host_decode_strided_views_and_padded_table(isa):
    """q and out as head-major views, the table padded with junk past each
    row's blocks (never read), the caches as halves of one buffer."""
    n, H, KVH, D, BS, C = 6, 8, 4, 64, 16, 40
    q0, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, torch.float16, 120, 4)
    kv = torch.stack([kc, vc], dim=0)  # [2, C, KVH, BS, D]
    qbuf = torch.zeros(H, n, D, dtype=torch.float16)
    qbuf.copy_(q0.transpose(0, 1))
    q = qbuf.transpose(0, 1)  # strides (D, n*D, 1)
    btp = torch.randint(-(10**6), 10**6, (n, bt.shape[1] + 5), dtype=torch.int32)
    for i in range(n):
        nb = (int(lens[i]) + BS - 1) // BS
        btp[i, :nb] = bt[i, :nb]
    obuf = torch.zeros(H, n, D, dtype=torch.float32)
    out = obuf.transpose(0, 1)
    lse = torch.empty(H, n)
    ops.host_decode_attn(q, kv[0], kv[1], btp, lens, 0.125, out, lse)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q0, kc, vc, bt, lens, 0.125)
    check(out, lse, ref_out, ref_lse, lens, torch.float16)


def test_host_decode_range_errors_give_nan_rows(isa):
    n, H, KVH, D, BS, C = 4, 4, 2, 64, 16, 20
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, torch.bfloat16, 64, 1)
    lens = torch.tensor([64, 30, 17, 5], dtype=torch.int32)
    bt = torch.tensor([[0, 1, 2, 3], [4, C, 0, 0], [6, 7, 0, 0], [-1, 0, 0, 0]], dtype=torch.int32)
    bad_lens = lens.clone()
    bad_lens[2] = 4 * BS + 1  # past the table
    out, lse = run(q, kc, vc, bt, bad_lens, 0.1, torch.bfloat16)
    ok = torch.tensor([True, False, False, False])
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q[ok], kc, vc, bt[ok], lens[ok], 0.1)
    check(out[ok], lse[:, ok], ref_out, ref_lse, lens[ok], torch.bfloat16)
    assert torch.isnan(out[~ok]).all() and torch.isnan(lse[:, ~ok]).all()


def test_host_decode_rejects_bad_arguments():
    q, kc, vc, bt, lens = cases.rand_case(2, 4, 2, 64, 16, 8, torch.float16, 30, 0)
    out = torch.empty(2, 4, 64)
    lse = torch.empty(4, 2)
    with pytest.raises(RuntimeError, match="host memory"):
        ops.host_decode_attn(q.to("meta"), kc, vc, bt, lens, 0.1, out, lse)
    with pytest.raises(RuntimeError, match="share a dtype"):
        ops.host_decode_attn(q.float(), kc, vc, bt, lens, 0.1, out, lse)
    with pytest.raises(RuntimeError, match="int32"):
        ops.host_decode_attn(q, kc, vc, bt.long(), lens, 0.1, out, lse)
    lib = _lib.load_lib()
    st = lib.fd_host_decode_partial(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
        kc.stride(0), kc.stride(1), kc.stride(2), 8, bt.data_ptr(), bt.stride(0), bt.shape[1],
        lens.data_ptr(), 2, 3, 2, 64, 16, 0.1, _lib.FD_F16, out.data_ptr(), out.stride(0),
        out.stride(1), _lib.FD_F32, lse.data_ptr(), 2, 0)
    assert st == _lib.FD_ERR_INVALID and b"bad sizes" in lib.fd_last_error()
    st = lib.fd_host_decode_partial(
        q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
        kc.stride(0), kc.stride(1), kc.stride(2), 8, bt.data_ptr(), bt.stride(0), bt.shape[1],
        lens.data_ptr(), 2, 4, 2, 64, 16, 0.1, _lib.FD_F16, out.data_ptr(), out.stride(0),
        out.stride(1), _lib.FD_BF16, lse.data_ptr(), 2, 0)
    assert st == _lib.FD_ERR_INVALID and b"out dtype" in lib.fd_last_error()
    # n == 0 is a no-op even with NULL buffers
    assert lib.fd_host_decode_partial(None, 0, 0, None, None, 0, 0, 0, 0, None, 0, 0, None, 0, 4,
                                      2, 64, 16, 0.1, _lib.FD_F16, None, 0, 0, _lib.FD_F16,
                                      None, 0, 0) == _lib.FD_OK


def _child_decode(conn, args):
    q, kc, vc, bt, lens = args
    out, lse = run(q, kc, vc, bt, lens, 0.1, torch.float32, threads=4)
    conn.send((out.numpy().copy(), lse.numpy().copy()))  # by value, not shared memory
    conn.close()


def test_host_decode_in_a_forked_child():
    """A child forked after the parent used the worker pool gets its own pool
    (the parent's threads do not exist in the child): same results, no hang."""
    import multiprocessing as mp

    args = cases.rand_case(11, 8, 2, 64, 16, 60, torch.float16, 150, 3)
    parent = run(*args[:5], 0.1, torch.float32, threads=4)
    ctx = mp.get_context("fork")
    rd, wr = ctx.Pipe(duplex=False)
    proc = ctx.Process(target=_child_decode, args=(wr, args))
    proc.start()
    wr.close()
    try:
        assert rd.poll(120), "forked child did not answer"
        child = tuple(torch.from_numpy(x) for x in rd.recv())
    finally:
        proc.join(30)
        if proc.is_alive():
            proc.kill()
    assert proc.exitcode == 0
    assert torch.equal(child[0], parent[0]) and torch.equal(child[1], parent[1])


def test_host_stream_read_checksum_and_arguments():
    """fd_host_stream_read (the host-DRAM read-rate probe): the checksum is the
    XOR of the buffer's 64-bit words, whatever the thread count and whether
    the size is a whole number of its 1 MiB chunks or of the four interleaved
    streams each chunk is read as (odd line counts per stream, lines past the
    streams); bad sizes, unaligned sources and too many threads are argument
    errors."""
    import numpy as np

    from vllm_fastdecoder_amd import _lib, ops

    g = torch.Generator().manual_seed(3)
    for nbytes in (64, 320, 576, 704, 832, 4096, (1 << 20) - 64, (2 << 20) + 13 * 64,
                   (3 << 20) + 192):
        words = torch.randint(-(2 ** 62), 2 ** 62, (nbytes // 8,), generator=g, dtype=torch.int64)
        want = int(np.bitwise_xor.reduce(words.numpy().view(np.uint64)))
        for threads in (1, 3, 0):
            assert ops.host_stream_read(words, threads) == want
    lib = _lib.load_lib()
    buf = torch.zeros(1024, dtype=torch.int64)
    out = ctypes.c_uint64(7)
    assert lib.fd_host_stream_read(buf.data_ptr(), 100, 1, ctypes.byref(out)) == _lib.FD_ERR_INVALID
    assert lib.fd_host_stream_read(buf.data_ptr() + 8, 64, 1, ctypes.byref(out)) == \
        _lib.FD_ERR_INVALID
    assert lib.fd_host_stream_read(buf.data_ptr(), 64, 1 << 20, ctypes.byref(out)) == \
        _lib.FD_ERR_INVALID
    assert lib.fd_host_stream_read(None, 0, 1, ctypes.byref(out)) == _lib.FD_OK and out.value == 0


def test_host_decode_start_matches_the_synchronous_call(isa):
    """fd_host_decode_partial_start / fd_host_decode_wait: queued calls run in
    order on the library's runner thread and give the synchronous call's bits;
    the wait returns the call's own time."""
    cases_ = [cases.rand_case(9, 8, 2, 128, 16, 80, torch.float16, 300, s) for s in (1, 2, 3)]
    want = [run(*c[:5], 0.1, torch.float32) for c in cases_]
    outs, calls = [], []
    for c in cases_:
        q, kc, vc, bt, lens = c
        out = torch.full((9, 8, 128), 7.0)
        lse = torch.full((8, 9), 7.0)
        calls.append(ops.host_decode_start(q, kc, vc, bt, lens, 0.1, out, lse))
        outs.append((out, lse))
    for call, (out, lse), (wo, wl) in zip(calls, outs, want):
        assert call.wait() >= 0.0
        assert torch.equal(out, wo) and torch.equal(lse, wl)
    assert calls[0].wait() == 0.0  # a second wait of the Python handle is a no-op


def test_host_decode_start_checks_before_queueing():
    """Bad arguments are refused at start (nothing queued); an id that is not
    pending is refused by the wait; a call's range errors still give NaN rows."""
    lib = _lib.load_lib()
    q, kc, vc, bt, lens = cases.rand_case(2, 4, 2, 64, 16, 8, torch.float16, 30, 0)
    out = torch.empty(2, 4, 64)
    lse = torch.empty(4, 2)
    call = ctypes.c_int64(-1)
    st = lib.fd_host_decode_partial_start(
        None, q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
        kc.stride(0), kc.stride(1), kc.stride(2), 8, bt.data_ptr(), bt.stride(0), bt.shape[1],
        lens.data_ptr(), 2, 3, 2, 64, 16, 0.1, _lib.FD_F16, out.data_ptr(), out.stride(0),
        out.stride(1), _lib.FD_F32, lse.data_ptr(), 2, 0, ctypes.byref(call))
    assert st == _lib.FD_ERR_INVALID and b"bad sizes" in lib.fd_last_error()
    assert call.value == -1
    with pytest.raises(RuntimeError, match="share a dtype"):
        ops.host_decode_start(q.float(), kc, vc, bt, lens, 0.1, out, lse)
    secs = ctypes.c_double()
    assert lib.fd_host_decode_wait(10**12, ctypes.byref(secs)) == _lib.FD_ERR_INVALID
    assert b"no pending call" in lib.fd_last_error()
    st = lib.fd_host_decode_partial_start(
        None, q.data_ptr(), q.stride(0), q.stride(1), kc.data_ptr(), vc.data_ptr(),
        kc.stride(0), kc.stride(1), kc.stride(2), 8, bt.data_ptr(), bt.stride(0), bt.shape[1],
        lens.data_ptr(), 2, 4, 2, 64, 16, 0.1, _lib.FD_F16, out.data_ptr(), out.stride(0),
        out.stride(1), _lib.FD_F32, lse.data_ptr(), 2, 0, ctypes.byref(call))
    assert st == _lib.FD_OK and call.value > 0
    assert lib.fd_host_decode_wait(call.value, None) == _lib.FD_OK
    assert lib.fd_host_decode_wait(call.value, None) == _lib.FD_ERR_INVALID  # waited already
    bad = bt.clone()
    bad[1, 0] = 8 + 5
    o2, l2 = torch.empty(2, 4, 64), torch.empty(4, 2)
    ops.host_decode_start(q, kc, vc, bad, lens, 0.1, o2, l2).wait()
    assert torch.isnan(o2[1]).all() and torch.isnan(l2[:, 1]).all()
    assert torch.isfinite(o2[0]).all()


def test_hybrid_share_start_checks_before_any_work():
    """fd_hybrid_share_start refuses bad arguments before it enqueues the copy
    of q or queues a call (nothing written, *call 0), and n = 0 does nothing.
    None of these paths reaches the GPU."""
    lib = _lib.load_lib()
    q, kc, vc, bt, lens = cases.rand_case(2, 4, 2, 64, 16, 8, torch.float16, 30, 0)
    W = bt.shape[1]
    q_host = torch.empty_like(q)
    gl = torch.full((2,), -7, dtype=torch.int32)
    cl = torch.full((2,), -7, dtype=torch.int32)
    cbt = torch.full((2, W), -7, dtype=torch.int32)
    out = torch.full((2, 4, 64), -7.0)
    lse = torch.full((4, 2), -7.0)
    fake = ctypes.c_void_p(0x1000)  # a stream / event / GPU q no path below may touch

    def start(n=2, H=4, frac=0.5, cbt_stride=W, event=fake, threads=0, call=True):
        c = ctypes.c_int64(-1)
        st = lib.fd_hybrid_share_start(
            fake, event, fake, q_host.data_ptr(), bt.data_ptr(), bt.stride(0), W,
            lens.data_ptr(), frac, gl.data_ptr(), cbt.data_ptr(), cbt_stride, cl.data_ptr(),
            kc.data_ptr(), vc.data_ptr(), kc.stride(0), kc.stride(1), kc.stride(2), 8,
            n, H, 2, 64, 16, 0.1, _lib.FD_F16, out.data_ptr(), lse.data_ptr(), threads,
            ctypes.byref(c) if call else None)
        return st, c.value

    assert start(call=False)[0] == _lib.FD_ERR_INVALID
    assert b"call is NULL" in lib.fd_last_error()
    for kw, msg in ((dict(H=3), b"bad sizes"), (dict(frac=1.5), b"cpu_fraction"),
                    (dict(frac=float("nan")), b"cpu_fraction"),
                    (dict(cbt_stride=W - 1), b"bt_stride < bt_width"),
                    (dict(event=None), b"NULL pointer"),
                    (dict(threads=1025), b"bad sizes")):
        st, c = start(**kw)
        assert st == _lib.FD_ERR_INVALID and msg in lib.fd_last_error(), kw
        assert c == 0
    assert start(n=0) == (_lib.FD_OK, 0)
    for t in (gl, cl, cbt):
        assert (t == -7).all()
    assert (out == -7).all() and (lse == -7).all()


def _child_start(conn, args):
    q, kc, vc, bt, lens = args
    out = torch.empty(q.shape, dtype=torch.float32)
    lse = torch.empty(q.shape[1], q.shape[0])
    ops.host_decode_start(q, kc, vc, bt, lens, 0.1, out, lse, num_threads=4).wait()
    conn.send((out.numpy().copy(), lse.numpy().copy()))
    conn.close()


def test_host_decode_start_in_a_forked_child():
    """A child forked after the parent used the runner thread gets its own."""
    import multiprocessing as mp

    args = cases.rand_case(11, 8, 2, 64, 16, 60, torch.float16, 150, 5)
    out = torch.empty(11, 8, 64)
    lse = torch.empty(8, 11)
    ops.host_decode_start(*args, 0.1, out, lse, num_threads=4).wait()
    ctx = mp.get_context("fork")
    rd, wr = ctx.Pipe(duplex=False)
    proc = ctx.Process(target=_child_start, args=(wr, args))
    proc.start()
    wr.close()
    try:
        assert rd.poll(120), "forked child did not answer"
        child = tuple(torch.from_numpy(x) for x in rd.recv())
    finally:
        proc.join(30)
        if proc.is_alive():
            proc.kill()
    assert proc.exitcode == 0
    assert torch.equal(child[0], out) and torch.equal(child[1], lse)
