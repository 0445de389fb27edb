"""GPU parity of the hybrid split decode (ops.hybrid_split_decode): the host
tier shared between the GPU's fused launch and the host cores, the two fp32
partials LSE-merged on the GPU.

Checked against the float64 oracle (merge of the two tiers' float64 partials,
as in test_gpu_split_fused) for host-core shares from 0 (all on the GPU) to 1
(the reference's division: the host cores compute the whole host-tier
partial, fastdecode/backend.py:343-351). Bars: fp32 out max-abs <= 2e-3, lse
<= 1e-4 relative; 16-bit out fp16 2e-3 / bf16 1.6e-2; empty rows exactly 0 /
-inf. Host-tier KV written on the stream by the GPU just before the call is
seen by the host cores.
"""

from __future__ import annotations

import pytest
import torch

from tests.test_gpu_split_fused import TOL16, oracle_merged, two_tier_case
from vllm_fastdecoder_amd import ops

pytestmark = pytest.mark.gpu


def run_hybrid(c, dev, frac, out_dtype=torch.float32, threads=0):
    q = c["q"].to(dev)
    n, H, D = q.shape
    out = torch.empty(n, H, D, dtype=out_dtype, device=dev)
    lse = torch.empty(H, n, dtype=torch.float32, device=dev)
    ops.hybrid_split_decode(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"],
                            c["hk"], c["hv"], c["bt_c"], c["len_c"], c["scale"], frac,
                            out=out, lse=lse, num_threads=threads)
    torch.cuda.synchronize()
    return out, lse


def check(out, lse, ref_o, ref_l, lens, tol=2e-3):
    nz = lens > 0
    o = out.double().cpu()
    assert float((o[nz] - ref_o[nz]).abs().max()) <= tol
    rel = (lse.double().cpu()[:, nz] - ref_l[:, nz]).abs() / ref_l[:, nz].abs().clamp(min=1)
    assert float(rel.max()) <= 1e-4
    assert torch.all(out.cpu()[~nz] == 0)
    assert torch.all(torch.isneginf(lse.cpu()[:, ~nz]))


@pytest.mark.parametrize("frac", [0.0, 0.3, 0.65, 1.0])
@pytest.mark.parametrize("H,KVH,D,dtype", [(32, 32, 128, torch.float16),
                                           (32, 8, 128, torch.bfloat16),
                                           (16, 2, 64, torch.float16),
                                           (8, 8, 256, torch.bfloat16)])
def test_hybrid_matches_oracle(gpu, frac, H, KVH, D, dtype):
    c = two_tier_case(12, H, KVH, D, dtype, seed=H + D + int(frac * 10), dev=gpu)
    ref_o, ref_l = oracle_merged(c)
    out, lse = run_hybrid(c, gpu, frac)
    check(out, lse, ref_o, ref_l, c["lens"])


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_hybrid_16bit_out_and_interleaved_tiers(gpu, dtype):
    """Output in the KV dtype; tiers interleaved, each ending in a partial
    block."""
    c = two_tier_case(9, 16, 4, 128, dtype, seed=77, dev=gpu, gpu_first=False)
    ref_o, ref_l = oracle_merged(c)
    out, lse = run_hybrid(c, gpu, 0.5, out_dtype=dtype)
    tol = TOL16[dtype]
    nz = c["lens"] > 0
    err = (out.double().cpu()[nz] - ref_o[nz]).abs() - tol * ref_o[nz].abs()
    assert float(err.max()) <= tol
    rel = (lse.double().cpu()[:, nz] - ref_l[:, nz]).abs() / ref_l[:, nz].abs().clamp(min=1)
    assert float(rel.max()) <= 1e-4


def test_hybrid_close_to_fused(gpu):
    """Same inputs through the fused launch alone: the merge of two fp32
    partials differs from the single-pass result by summation order only."""
    from tests.test_gpu_split_fused import run_fused

    c = two_tier_case(16, 32, 8, 128, torch.bfloat16, seed=5, dev=gpu)
    o_f, l_f = run_fused(c, gpu)
    nz = (c["lens"] > 0).to(gpu)
    for frac in (0.4, 0.9):
        o_h, l_h = run_hybrid(c, gpu, frac, threads=3)
        assert float((o_h - o_f).abs().max()) <= 2e-5
        assert float((l_h[:, nz] - l_f[:, nz]).abs().max()) <= 2e-5
        assert torch.equal(l_h[:, ~nz], l_f[:, ~nz])  # empty rows: -inf in both


def test_back_to_back_steps_over_both_staging_sets(gpu):
    """Five hybrid steps without a synchronisation between them: the pinned
    staging alternates between two sets, so each step reuses the set of the
    step before last, whose merge may still be queued; row counts change
    between steps (the sets' cached views are rebuilt, then reused). Every
    step's output matches its own oracle, and a step started on the set of a
    step still in flight is refused."""
    cases = [two_tier_case(n, 16, 4, 64, torch.float16, seed=40 + k, dev=gpu)
             for k, n in enumerate((10, 10, 7, 12, 10))]
    outs = []
    for c in cases:
        q = c["q"].to(gpu)
        n, H, D = q.shape
        out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
        lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
        h = ops.hybrid_split_begin(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"],
                                   c["hk"], c["hv"], c["bt_c"], c["len_c"], c["scale"], 0.6,
                                   out=out, lse=lse, num_threads=4)
        if c is cases[1]:
            with pytest.raises(RuntimeError, match="already in flight"):
                ops.hybrid_split_begin(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"],
                                       c["len_g"], c["hk"], c["hv"], c["bt_c"], c["len_c"],
                                       c["scale"], 0.6)
        h.finish()
        outs.append((out, lse))
    torch.cuda.synchronize()
    for c, (out, lse) in zip(cases, outs):
        ref_o, ref_l = oracle_merged(c)
        check(out, lse, ref_o, ref_l, c["lens"])


def test_a_refused_step_leaves_the_next_one_working(gpu):
    """A host row needing more blocks than its table holds is refused by the
    library after q's copy was enqueued: begin() raises, queues no host call,
    frees its staging set, and the next steps (on both sets) run normally."""
    c = two_tier_case(6, 8, 2, 64, torch.float16, seed=31, dev=gpu)
    q = c["q"].to(gpu)
    D = q.shape[2]
    bad_lens = c["len_c"].clone()
    bad_lens[3] = c["bt_c"].shape[1] * 16 + 1
    args = (q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"], c["hk"], c["hv"],
            c["bt_c"])
    with pytest.raises(RuntimeError, match="needs .* blocks"):
        ops.hybrid_split_begin(*args, bad_lens, c["scale"], 0.5)
    ref_o, ref_l = oracle_merged(c)
    for _ in range(3):
        out, lse = run_hybrid(c, gpu, 0.5)
        check(out, lse, ref_o, ref_l, c["lens"])


@pytest.mark.parametrize("width", [0, 3])
def test_hybrid_with_an_empty_host_tier(gpu, width):
    """No row has host-tier tokens (a zero-width host table, or zero lengths
    in a padded one): the host cores' share is all empty rows, and the step
    equals the HBM-tier partial alone."""
    c = two_tier_case(8, 16, 4, 64, torch.float16, seed=21, dev=gpu, special=False)
    q = c["q"].to(gpu)
    n, H, D = q.shape
    nb_g = (c["len_g"] + 15) // 16
    len_g = nb_g * 16  # whole HBM blocks: the HBM tier holds every token here
    c["len_g"] = len_g.to(torch.int32)
    c["len_c"] = torch.zeros(n, dtype=torch.int32)
    c["bt_c"] = torch.zeros(n, width, dtype=torch.int32)
    out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    for frac in (0.0, 0.5, 1.0):
        ops.hybrid_split_decode(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"],
                                c["hk"], c["hv"], c["bt_c"], c["len_c"], c["scale"], frac,
                                out=out, lse=lse)
        ref_o, ref_l = ops.paged_decode(q, c["kv"][..., :D], c["kv"][..., D:],
                                        c["bt_g"].to(gpu), c["len_g"].to(gpu), c["scale"],
                                        out=torch.empty_like(out))
        torch.cuda.synchronize()
        nz = c["len_g"] > 0
        assert float((out[nz.to(gpu)] - ref_o[nz.to(gpu)]).abs().max()) <= 2e-5, frac
        assert float((lse[:, nz.to(gpu)] - ref_l[:, nz.to(gpu)]).abs().max()) <= 2e-5, frac
        assert torch.all(out[~nz.to(gpu)] == 0) and torch.all(torch.isneginf(lse[:, ~nz.to(gpu)]))


def test_hybrid_sees_kv_written_by_the_gpu(gpu):
    """The step's new token is written into the pinned host tier by the GPU
    (reshape_and_cache on the stream) and then read by the host cores."""
    c = two_tier_case(6, 8, 2, 64, torch.float16, seed=3, dev=gpu, special=False)
    BS, D = 16, 64
    q = c["q"]
    n = q.shape[0]
    g = torch.Generator().manual_seed(11)
    k_new = torch.randn(n, 2, D, generator=g).to(torch.float16)
    v_new = torch.randn(n, 2, D, generator=g).to(torch.float16)
    slots = torch.full((n,), -1, dtype=torch.int64)
    for i in range(n):
        lc = int(c["len_c"][i])
        if lc:
            blk = int(c["bt_c"][i, (lc - 1) // BS])
            slots[i] = blk * BS + (lc - 1) % BS
    ops.reshape_and_cache(k_new.to(gpu), v_new.to(gpu), c["hk"].transpose(1, 2),
                          c["hv"].transpose(1, 2), slots.to(gpu))
    out, lse = run_hybrid(c, gpu, 1.0)  # the host cores read every host block
    for i in range(n):  # the oracle sees the same writes
        if slots[i] >= 0:
            b, t = divmod(int(slots[i]), BS)
            assert torch.equal(c["hk"][b, :, t], k_new[i]) and torch.equal(c["hv"][b, :, t], v_new[i])
    ref_o, ref_l = oracle_merged(c)
    check(out, lse, ref_o, ref_l, c["lens"])


def test_backend_uses_the_hybrid_only_above_its_host_bytes_threshold(gpu, monkeypatch):
    """SplitDecodeImpl's default ("auto" share) sends a layer's host tier to
    the host cores only when it holds at least hybrid_min_host_bytes of KV;
    below that the fused GPU launch reads it. Both give the reference output."""
    from types import SimpleNamespace

    from tests.test_gpu_forward import REQS16, TOL, _PrefillOps, build_tiers
    from vllm_fastdecoder_amd import backend, plan, state

    monkeypatch.setattr(backend, "OPS", _PrefillOps)
    calls = []
    real_begin = ops.hybrid_split_begin

    def spy(*a, **k):
        calls.append(a[10])  # the share
        return real_begin(*a, **k)

    monkeypatch.setattr(ops, "hybrid_split_begin", spy)
    G, C, H, KVH, D, BS, dtype = 24, 40, 8, 2, 128, 16, torch.float16
    for threshold, expect_hybrid in ((1 << 40, False), (0, True)):
        sc = build_tiers(REQS16, G, C, H, KVH, D, BS, dtype, 1, gpu)
        hp = plan.build_host_plan(sc.qsl, sc.seq, sc.bt, sc.slots, G, C, BS)
        dp = plan.to_device(hp, sc.bt.to(gpu), gpu)
        state.STORE = state.HostKVStore(G, C, BS, KVH, D, dtype, k={"l0": sc.host_k},
                                        v={"l0": sc.host_v})
        impl = backend.SplitDecodeImpl(H, KVH, D, sc.scale, hybrid_min_host_bytes=threshold)
        assert impl.cpu_fraction == "auto"
        calls.clear()
        out = torch.full_like(sc.query, float("nan"))
        impl._forward_split(SimpleNamespace(layer_name="l0", _k_scale=None, _v_scale=None),
                            sc.query, sc.key, sc.value, sc.kv_cache, dp, out)
        torch.cuda.synchronize()
        assert (len(calls) == 1) == expect_hybrid
        if expect_hybrid:
            assert calls[0] == plan.ShareTuner().fraction  # the tuner's starting share
        assert float((out.double().cpu() - sc.ref).abs().max()) <= TOL[dtype]
    state.STORE = None


def test_two_micro_batches_interleaved_with_other_gpu_work(gpu):
    """Micro-batch overlap with the begin / finish halves: begin(A), enqueue
    other GPU work, finish(A), begin(B), other work, finish(B). One hybrid
    split in flight per device; a second begin before finish is refused.
    Both micro-batches give the oracle's result."""
    ca = two_tier_case(10, 16, 4, 128, torch.float16, seed=21, dev=gpu)
    cb = two_tier_case(7, 16, 4, 128, torch.float16, seed=22, dev=gpu)
    x = torch.randn(2048, 2048, device=gpu)
    outs = []
    for c in (ca, cb):
        q = c["q"].to(gpu)
        n, H, D = q.shape
        out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
        lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
        h = ops.hybrid_split_begin(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"],
                                   c["hk"], c["hv"], c["bt_c"], c["len_c"], c["scale"], 0.6,
                                   out=out, lse=lse)
        with pytest.raises(RuntimeError, match="in flight"):
            ops.hybrid_split_begin(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"],
                                   c["hk"], c["hv"], c["bt_c"], c["len_c"], c["scale"], 0.6)
        for _ in range(4):  # the other micro-batch's GPU work
            x = torch.tanh(x @ x) * 0.01
        h.finish()
        outs.append((out, lse))
    torch.cuda.synchronize()
    assert torch.isfinite(x).all()
    for c, (out, lse) in zip((ca, cb), outs):
        ref_o, ref_l = oracle_merged(c)
        check(out, lse, ref_o, ref_l, c["lens"])


def test_hybrid_with_device_hbm_tables(gpu):
    """The HBM tier's table and lengths already on the GPU (no host-side row
    order then) give the oracle's result, as do host copies of them."""
    c = two_tier_case(10, 16, 4, 128, torch.float16, seed=31, dev=gpu)
    ref_o, ref_l = oracle_merged(c)
    q = c["q"].to(gpu)
    n, H, D = q.shape
    for dev_tables in (True, False):
        bt_g = c["bt_g"].to(gpu) if dev_tables else c["bt_g"]
        len_g = c["len_g"].to(gpu) if dev_tables else c["len_g"]
        out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
        lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
        ops.hybrid_split_decode(q, c["kv"][..., :D], c["kv"][..., D:], bt_g, len_g, c["hk"],
                                c["hv"], c["bt_c"], c["len_c"], c["scale"], 0.5, out=out, lse=lse)
        torch.cuda.synchronize()
        check(out, lse, ref_o, ref_l, c["lens"])


def test_cancel_frees_the_device_for_the_next_split(gpu):
    """A split abandoned between begin and finish (the caller's step failed)
    is cancelled: the next begin on the device is accepted and correct;
    cancel after finish is a no-op."""
    c = two_tier_case(6, 8, 2, 64, torch.float16, seed=41, dev=gpu)
    q = c["q"].to(gpu)
    n, H, D = q.shape
    args = (q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"], c["hk"], c["hv"],
            c["bt_c"], c["len_c"], c["scale"], 0.5)
    h = ops.hybrid_split_begin(*args)
    h.cancel()
    out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    h2 = ops.hybrid_split_begin(*args, out=out, lse=lse)
    h2.finish()
    h2.cancel()
    torch.cuda.synchronize()
    ref_o, ref_l = oracle_merged(c)
    check(out, lse, ref_o, ref_l, c["lens"])


def test_failed_begin_leaves_the_device_usable(gpu):
    """begin raising part-way (here: an HBM table of the wrong dtype, refused
    by the GPU launch's checks after q's copy to the host was enqueued) frees
    the staging and re-raises; the next split is correct."""
    c = two_tier_case(6, 8, 2, 64, torch.float16, seed=43, dev=gpu)
    q = c["q"].to(gpu)
    n, H, D = q.shape
    with pytest.raises(RuntimeError, match="int32"):
        ops.hybrid_split_begin(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"].long(),
                               c["len_g"], c["hk"], c["hv"], c["bt_c"], c["len_c"], c["scale"],
                               0.5)
    out, lse = run_hybrid(c, gpu, 0.5)
    ref_o, ref_l = oracle_merged(c)
    check(out, lse, ref_o, ref_l, c["lens"])


@pytest.mark.parametrize("given", [True, False])
def test_finish_on_another_stream_than_begin(gpu, given):
    """begin on a side stream, finish (and the merge) on the default stream,
    then a second split at once: each split is correct, and the second one's
    reuse of the pinned staging waits for the first one's copies on both
    streams. given=False: begin allocates out / lse itself (on the side
    stream), and they stay valid for the finishing stream's work."""
    c = two_tier_case(6, 8, 2, 64, torch.float16, seed=47, dev=gpu)
    q = c["q"].to(gpu)
    n, H, D = q.shape
    args = (q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"], c["len_g"], c["hk"], c["hv"],
            c["bt_c"], c["len_c"], c["scale"], 0.5)
    ref_o, ref_l = oracle_merged(c)
    side = torch.cuda.Stream(device=gpu)
    side.wait_stream(torch.cuda.current_stream(gpu))
    outs = []
    for _ in range(2):
        out = torch.empty(n, H, D, dtype=torch.float32, device=gpu) if given else None
        lse = torch.empty(H, n, dtype=torch.float32, device=gpu) if given else None
        with torch.cuda.stream(side):
            h = ops.hybrid_split_begin(*args, out=out, lse=lse)
        torch.cuda.current_stream(gpu).wait_stream(side)
        out, lse = h.finish()
        # fp32 copies on the finishing stream (begin's out is in q's dtype)
        outs.append((out.float(), lse.clone()))
        del h, out, lse
        # new work on begin's stream while the merge may still be pending
        with torch.cuda.stream(side):
            junk = torch.full((n, H, D), 3.0, dtype=q.dtype, device=gpu)
            junk += 1
    torch.cuda.synchronize()
    nz = c["lens"] > 0
    for out, lse in outs:
        if given:
            check(out, lse, ref_o, ref_l, c["lens"])
            continue
        # out in q's dtype: the reference's 16-bit bar
        tol = TOL16[q.dtype]
        err = (out.double().cpu()[nz] - ref_o[nz]).abs() - tol * ref_o[nz].abs()
        assert float(err.max()) <= tol
        rel = (lse.double().cpu()[:, nz] - ref_l[:, nz]).abs() / ref_l[:, nz].abs().clamp(min=1)
        assert float(rel.max()) <= 1e-4
        assert torch.all(out.cpu()[~nz] == 0)


def test_host_call_waits_for_its_event(gpu):
    """ops.host_decode_start with a ready event: q is copied to pinned memory
    behind a slow GPU kernel on the stream and the event recorded after the
    copy; the queued host call waits for it, so it reads the copied q (the
    synchronous call on the same q gives the same bits). An event that was
    never recorded is refused."""
    from tests import cases
    from vllm_fastdecoder_amd.pinned import pinned_empty

    q, kc, vc, bt, lens = cases.rand_case(10, 8, 2, 128, 16, 90, torch.float16, 300, 21)
    q_dev = q.to(gpu)
    q_host = pinned_empty(tuple(q.shape), q.dtype)
    q_host.zero_()
    stream = torch.cuda.current_stream(gpu)
    busy = torch.randn(4096, 4096, device=gpu)
    for _ in range(20):  # keep the stream busy for a while before the copy
        busy = (busy @ busy) * 1e-4
    q_host.copy_(q_dev, non_blocking=True)
    ready = torch.cuda.Event()
    ready.record(stream)
    out = torch.empty(10, 8, 128)
    lse = torch.empty(8, 10)
    call = ops.host_decode_start(q_host, kc, vc, bt, lens, 0.1, out, lse, ready=ready)
    call.wait()
    ref_o = torch.empty(10, 8, 128)
    ref_l = torch.empty(8, 10)
    ops.host_decode_attn(q, kc, vc, bt, lens, 0.1, ref_o, ref_l)
    assert torch.equal(out, ref_o) and torch.equal(lse, ref_l)
    with pytest.raises(RuntimeError, match="never recorded"):
        ops.host_decode_start(q_host, kc, vc, bt, lens, 0.1, out, lse, ready=torch.cuda.Event())
