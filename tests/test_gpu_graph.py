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
    before = dict(ops.WORKSPACE._bufs)
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
