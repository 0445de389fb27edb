"""The decode path captured in a HIP graph (torch.cuda.CUDAGraph), as a
serving engine captures its decode step: the paged partial in vLLM's layout,
the same with rows split into tasks (combine kernel + workspace), and the
fused two-tier launch over a pinned host tier. Each graph is replayed several
times with new queries, with eager GPU work and synchronisations between the
replays, and every replay is checked bit-exactly against an eager call on
the same inputs (the same kernels in the same order)."""

from __future__ import annotations

import pytest
import torch

from tests import cases
from tests.test_gpu_split_fused import two_tier_case
from vllm_fastdecoder_amd import ops

pytestmark = pytest.mark.gpu


def _replays(gpu, q, step, outs, n_replays=4, ws_bytes=0):
    """Capture step() (which writes outs), then replay with fresh q values
    and compare each replay with an eager step() on the same q. The capture
    stream's split workspace (ws_bytes) is reserved before capture, so the
    captured launches allocate nothing."""
    step()  # warm-up: launch settings (and the eager stream's workspace) exist
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=gpu)
    ops.reserve_workspace(side, ws_bytes)
    before = {k: v for k, v in ops.WORKSPACE._bufs.items()}
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        step()
    # no workspace was allocated or replaced under capture
    assert {k: v.data_ptr() for k, v in ops.WORKSPACE._bufs.items()} == \
        {k: v.data_ptr() for k, v in before.items()}
    gen = torch.Generator(device=gpu).manual_seed(5)
    x = torch.randn(512, 512, device=gpu)
    for r in range(n_replays):
        q.copy_(torch.randn(q.shape, generator=gen, device=gpu).to(q.dtype))
        g.replay()
        torch.cuda.synchronize()
        got = [o.clone() for o in outs]
        for _ in range(3):  # the program's own eager work between replays
            x = torch.tanh(x @ x) * 0.5
        step()  # eager on the same q
        torch.cuda.synchronize()
        for a, b in zip(got, outs):
            assert torch.equal(a, b), f"replay {r} differs from the eager call"
    assert torch.isfinite(x).all()
    del g
    ops.release_workspace(side)


@pytest.mark.parametrize("split", ["0", "2"])
def test_paged_decode_in_a_graph(gpu, split, monkeypatch):
    monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
    w = cases.Workload("graph", 12, 32, 8, 128, 16, torch.bfloat16, 1, 700, None, 13)
    lens, bt, pool = cases.draw_lens_and_tables(w)
    lens[3] = 0
    kc, vc, _kv = cases.kv_pool(w, pool, "vllm", gpu)
    q = cases.queries(w, gpu)
    bt_d, lens_d = bt.to(gpu), lens.to(gpu)
    out = torch.empty(w.n, w.H, w.D, dtype=torch.float32, device=gpu)
    lse = torch.empty(w.H, w.n, dtype=torch.float32, device=gpu)

    def step():
        ops.paged_decode(q, kc, vc, bt_d, lens_d, w.scale, out=out, lse=lse)

    # an upper bound over the kernels this shape may take; forced 2-block
    # tasks always split these rows
    ws = ops.workspace_bytes(w.n, w.H, w.KVH, w.D, w.BS, bt.shape[1])
    assert ws > 0 or split != "2"
    _replays(gpu, q, step, [out, lse], ws_bytes=ws)


def test_paged_decode_with_token_total_in_a_graph(gpu):
    """The token-total hint in a graph: rows of uneven length on the
    matrix-core kernel take the slot fill's split tasks and the combine; each
    replay matches an eager call bit for bit."""
    w = cases.Workload("graph", 128, 8, 1, 128, 16, torch.bfloat16, 1024, 4096, None, 17)
    lens, bt, pool = cases.draw_lens_and_tables(w)
    total = int(lens.sum())
    info = ops.decode_plan_info(w.n, w.H, w.KVH, w.D, w.BS, bt.shape[1], w.dtype,
                                total_tokens=total)
    assert info["max_splits"] > 1, info
    kc, vc, _kv = cases.kv_pool(w, pool, "vllm", gpu)
    q = cases.queries(w, gpu)
    bt_d, lens_d = bt.to(gpu), lens.to(gpu)
    out = torch.empty(w.n, w.H, w.D, dtype=torch.float32, device=gpu)
    lse = torch.empty(w.H, w.n, dtype=torch.float32, device=gpu)

    def step():
        ops.paged_decode(q, kc, vc, bt_d, lens_d, w.scale, out=out, lse=lse, total_tokens=total)

    ws = ops.workspace_bytes(w.n, w.H, w.KVH, w.D, w.BS, bt.shape[1])
    _replays(gpu, q, step, [out, lse], ws_bytes=ws)


def test_fused_split_in_a_graph(gpu):
    c = two_tier_case(10, 32, 32, 128, torch.float16, seed=17, dev=gpu)
    q = c["q"].to(gpu)
    n, H, D = q.shape
    bt_g, len_g = c["bt_g"].to(gpu), c["len_g"].to(gpu)
    bt_c, len_c = c["bt_c"].to(gpu), c["len_c"].to(gpu)
    out = torch.empty(n, H, D, dtype=torch.float16, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)

    def step():
        ops.split_decode(q, c["kv"][..., :D], c["kv"][..., D:], bt_g, len_g, c["hk"], c["hv"],
                         bt_c, len_c, c["scale"], out=out, lse=lse)

    _replays(gpu, q, step, [out, lse],
             ws_bytes=ops.workspace_bytes(n, H, 32, D, 16, bt_g.shape[1] + bt_c.shape[1]))


def test_reserved_workspace_outlives_growth_and_eviction(gpu, monkeypatch):
    """A graph captured with a reserved workspace keeps its buffer's address.
    After capture, a larger eager call on the capture stream grows that
    stream's workspace, and workspaces of 20 more streams push it past the
    LRU limit; then fresh allocations take whatever memory was freed and are
    filled with a marker. Every replay still matches an eager call bit for
    bit and leaves the marker tensors untouched: the reserved buffer was
    neither freed nor reused."""
    monkeypatch.setenv("FD_SPLIT_BLOCKS", "2")  # rows always split: the workspace is used
    w = cases.Workload("graph", 12, 32, 8, 128, 16, torch.bfloat16, 64, 700, None, 19)
    lens, bt, pool = cases.draw_lens_and_tables(w)
    kc, vc, _kv = cases.kv_pool(w, pool, "vllm", gpu)
    q = cases.queries(w, gpu)
    bt_d, lens_d = bt.to(gpu), lens.to(gpu)
    out = torch.empty(w.n, w.H, w.D, dtype=torch.float32, device=gpu)
    lse = torch.empty(w.H, w.n, dtype=torch.float32, device=gpu)

    def step():
        ops.paged_decode(q, kc, vc, bt_d, lens_d, w.scale, out=out, lse=lse)

    ws = ops.workspace_bytes(w.n, w.H, w.KVH, w.D, w.BS, bt.shape[1])
    assert ws > 0
    step()
    torch.cuda.synchronize()
    side = torch.cuda.Stream(device=gpu)
    reserved = ops.reserve_workspace(side, ws)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g, stream=side):
        step()
    # growth: a call with 4x the rows on the capture stream needs a larger workspace
    big_n = 4 * w.n
    big_q = cases.queries(cases.Workload("graph", big_n, 32, 8, 128, 16, torch.bfloat16, 64,
                                         700, None, 19), gpu)
    big_bt = bt_d.repeat(4, 1)
    big_lens = lens_d.repeat(4)
    assert ops.workspace_bytes(big_n, w.H, w.KVH, w.D, w.BS, bt.shape[1]) > reserved.numel()
    with torch.cuda.stream(side):
        ops.paged_decode(big_q, kc, vc, big_bt, big_lens, w.scale)
    side.synchronize()
    key = (gpu.index or 0, side.cuda_stream)
    assert ops.WORKSPACE._bufs[key].data_ptr() != reserved.data_ptr()  # it grew
    # eviction pressure: more streams than the workspace keeps
    streams = [torch.cuda.Stream(device=gpu) for _ in range(ops.WORKSPACE.max_streams + 4)]
    for s in streams:
        ops.WORKSPACE.get(gpu, reserved.numel(), stream=s.cuda_stream)
    assert key in ops.WORKSPACE._bufs  # a reserved stream is never evicted
    ptr = reserved.data_ptr()
    del reserved
    torch.cuda.synchronize()
    # fresh allocations of the reserved buffer's size on its stream would reuse
    # it if it had been freed (the caching allocator keeps freed blocks per stream)
    with torch.cuda.stream(side):
        markers = [torch.full((ws,), 77, dtype=torch.uint8, device=gpu) for _ in range(8)]
    side.synchronize()
    assert all(m.data_ptr() != ptr for m in markers)
    gen = torch.Generator(device=gpu).manual_seed(9)
    for r in range(3):
        q.copy_(torch.randn(q.shape, generator=gen, device=gpu).to(q.dtype))
        g.replay()
        torch.cuda.synchronize()
        got = (out.clone(), lse.clone())
        step()
        torch.cuda.synchronize()
        assert torch.equal(got[0], out) and torch.equal(got[1], lse), f"replay {r}"
        assert all(bool((m == 77).all()) for m in markers), f"replay {r} wrote into freed memory"
    del g
    ops.release_workspace(side)
    for s in streams:
        ops.WORKSPACE.release(gpu, s.cuda_stream)
