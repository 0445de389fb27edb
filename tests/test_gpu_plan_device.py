"""GPU tests of the device-side tier split (fd_plan_tiers / ops.plan_tiers) and
of a step planned on the GPU (backend.build_device_step +
SplitDecodeImpl._forward_device).

Block selection is bit-exact work: every table, length and slot is compared
exactly with
  * the plan oracle (the row-by-row restatement of fastdecode/plan.py:82-199):
    its S rows' per-tier tables and lengths, its P rows' lengths, its HBM and
    host slot mappings;
  * invariants read off each scenario itself: each tier's table lists the
    row's ids of that tier in sequence order then zeros, the two tiers'
    token counts add up to the row's length.
"""

from __future__ import annotations

import random
from types import SimpleNamespace

import pytest
import torch

from oracle.plan_oracle import plan_oracle
from tests.test_gpu_forward import REQS16, _PrefillOps, build_tiers, TOL
from tests.test_plan import random_reqs, scenario
from vllm_fastdecoder_amd import backend, ops, plan, state

pytestmark = pytest.mark.gpu


def _tier_tokens(ctx, ql, blocks, G, BS):
    L = ctx + ql
    nb = len(blocks)
    g = c = 0
    for j, b in enumerate(blocks):
        ntok = BS if j < nb - 1 else L - (nb - 1) * BS
        if b < G:
            g += ntok
        else:
            c += ntok
    return g, c


@pytest.mark.parametrize("seed", range(30))
def test_plan_tiers_bit_exact(gpu, seed):
    rng = random.Random(5000 + seed)
    BS = rng.choice([4, 16])
    G = rng.randint(5, 60)
    C = rng.randint(5, 80)
    reqs = random_reqs(rng, G, C, BS, rng.randint(1, 14))
    if not reqs:
        return
    qsl, seq, bt, slots = scenario(reqs, BS, junk_seed=seed, G_C=G + C, slot_pad=rng.randint(0, 5))
    n_tok = int(qsl[-1])
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    gb, cb, gl, cl, gs, hs = ops.plan_tiers(bt.to(gpu), seq, slots[:n_tok].to(gpu), G, C, BS,
                                            error_count=err)
    gb, cb, gl, cl, gs, hs = (t.cpu() for t in (gb, cb, gl, cl, gs, hs))
    W = bt.shape[1]
    assert int(err.item()) == 0
    # every row, from the scenario itself
    for r, (ctx, ql, blocks) in enumerate(reqs):
        hbm = [b for b in blocks if b < G]
        host = [b - G for b in blocks if b >= G]
        assert gb[r].tolist() == hbm + [0] * (W - len(hbm)), r
        assert cb[r].tolist() == host + [0] * (W - len(host)), r
        assert (int(gl[r]), int(cl[r])) == _tier_tokens(ctx, ql, blocks, G, BS), r
    # the plan oracle, where it plans (a step touching the host tier)
    ref = plan_oracle(qsl.tolist(), seq.tolist(), bt.tolist(), slots.tolist(), G, C, BS)
    sl = slots[:n_tok]
    assert gs.tolist() == torch.where(sl >= G * BS, -1, sl).tolist()
    assert hs.tolist() == torch.where(sl >= G * BS, sl - G * BS, -1).tolist()
    if ref is None:
        return
    assert gs.tolist() == ref["gpu_slot_mapping"] and hs.tolist() == ref["host_slot_mapping"]
    row_of_tok = {int(qsl[r]): r for r in range(len(reqs))}
    for j, tok in enumerate(ref["s_tok"]):
        r = row_of_tok[tok]
        ng, nc = ref["s_gpu_lens"][j], ref["s_cpu_lens"][j]
        assert (int(gl[r]), int(cl[r])) == (ng, nc)
        kg = (ng + BS - 1) // BS
        kc = (nc + BS - 1) // BS
        assert gb[r, :kg].tolist() == ref["s_gpu_bt"][j][:kg]
        assert cb[r, :kc].tolist() == ref["s_cpu_bt"][j][:kc]
    for j, r in enumerate(ref["p_req"]):
        assert int(gl[r]) == ref["p_seqlens"][j] and int(cl[r]) == 0


def test_plan_tiers_counts_capacity_and_length_errors(gpu):
    """A host id past G + C and a length past the table are counted; the
    latter row's HBM length is poisoned so decode writes NaN for it."""
    G, C, BS = 8, 4, 16
    bt = torch.tensor([[1, 9, 2, 0], [3, G + C + 1, 0, 0], [4, 5, 6, 7]], dtype=torch.int32)
    seq = torch.tensor([40, 20, 4 * BS + 1], dtype=torch.int32)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    gb, cb, gl, cl, _, _ = ops.plan_tiers(bt.to(gpu), seq, torch.zeros(0, dtype=torch.int64,
                                                                       device=gpu), G, C, BS,
                                          error_count=err)
    assert int(err.item()) == 2
    # row 0: ids 1 (HBM, 16 tokens), 9 (host, 16), 2 (HBM, 8); row 1: 3 (HBM, 16), 13 (host, 4)
    assert gl.tolist()[:2] == [24, 16] and cl.tolist()[:2] == [16, 4]
    assert cb[1, 0].item() == C + 1  # kept (the decode kernels flag it as out of the tier)
    assert int(gl[2]) > 4 * BS       # past its table: decode turns the row into NaN


@pytest.mark.parametrize("H,KVH", [(4, 4), (8, 2)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_forward_device_matches_host_planned_step(gpu, H, KVH, dtype, monkeypatch):
    """The REQS16 step (decodes touching either or both tiers, fresh
    prefills) planned on the GPU gives the reference output and, row for
    row, the host-planned step's output; the KV lands bit-exact in both
    tiers."""
    monkeypatch.setattr(backend, "OPS", _PrefillOps)
    G, C, BS, D = 24, 40, 16, 128
    outs = []
    for device_planned in (True, False):
        sc = build_tiers(REQS16, G, C, H, KVH, D, BS, dtype, 1, gpu)
        state.STORE = state.HostKVStore(G, C, BS, KVH, D, dtype, k={"l0": sc.host_k},
                                        v={"l0": sc.host_v})
        impl = backend.SplitDecodeImpl(H, KVH, D, sc.scale)
        layer = SimpleNamespace(layer_name="l0", _k_scale=None, _v_scale=None)
        out = torch.full_like(sc.query, float("nan"))
        R = sc.bt.shape[0]
        if device_planned:
            ds = backend.build_device_step(sc.qsl, sc.seq, sc.bt.to(gpu), sc.slots.to(gpu), R,
                                           state.STORE, gpu)
            assert ds is not None and ds.n_dec > 0 and ds.n_f_tok > 0
            impl._forward_device(layer, sc.query, sc.key, sc.value, sc.kv_cache, ds, out)
            assert int(ds.errors.item()) == 0
        else:
            dp = backend.build_split_plan(sc.qsl, sc.seq, sc.bt.to(gpu), sc.slots.to(gpu), R,
                                          state.STORE, gpu)
            impl._forward_split(layer, sc.query, sc.key, sc.value, sc.kv_cache, dp, out)
        torch.cuda.synchronize()
        assert float((out.double().cpu() - sc.ref).abs().max()) <= TOL[dtype]
        phys = sc.phys.cpu()
        assert torch.equal(phys[..., :D], sc.ref_k[:G]) and torch.equal(phys[..., D:], sc.ref_v[:G])
        assert torch.equal(sc.host_k.transpose(1, 2), sc.ref_k[G:])
        assert torch.equal(sc.host_v.transpose(1, 2), sc.ref_v[G:])
        outs.append(out)
    state.STORE = None
    assert float((outs[0] - outs[1]).abs().max()) <= 1e-2 * (1 if dtype == torch.float16 else 4)


def test_build_device_step_declines_chunked_continuations(gpu):
    """A prefill extending prior context needs the host's tier check
    (plan.py:142-149): the device planner hands such a step back (None)."""
    store = state.HostKVStore(10, 20, 4, 2, 64, torch.float16)
    reqs = [(8, 4, [1, 2, 3]), (3, 1, [11])]
    qsl, seq, bt, slots = scenario(reqs, 4)
    assert backend.build_device_step(qsl, seq, bt.to(gpu), slots.to(gpu), 2, store, gpu) is None
    assert backend.build_device_step(qsl, seq, bt.to(gpu), slots.to(gpu), 2, None, gpu) is None


def test_device_planned_decode_step_never_waits_for_the_gpu(gpu, monkeypatch):
    """A decode step planned on the GPU makes no synchronising call: torch's
    sync debug mode raises on the synchronising operations it knows
    (device-to-host copies, .item(), blocking waits; torch calls the mode a
    prototype that may not see every one)."""
    monkeypatch.setattr(backend, "OPS", backend.HipOps)
    G, C, BS, H, KVH, D, dtype = 24, 40, 16, 8, 2, 128, torch.float16
    reqs = [r for r in REQS16 if r[1] == 1]
    sc = build_tiers(reqs, G, C, H, KVH, D, BS, dtype, 2, gpu)
    state.STORE = state.HostKVStore(G, C, BS, KVH, D, dtype, k={"l0": sc.host_k},
                                    v={"l0": sc.host_v})
    impl = backend.SplitDecodeImpl(H, KVH, D, sc.scale)
    layer = SimpleNamespace(layer_name="l0", _k_scale=None, _v_scale=None)
    out = torch.full_like(sc.query, float("nan"))
    bt_d, slots_d = sc.bt.to(gpu), sc.slots.to(gpu)
    impl._forward_device(layer, sc.query, sc.key, sc.value, sc.kv_cache,
                         backend.build_device_step(sc.qsl, sc.seq, bt_d, slots_d, len(reqs),
                                                   state.STORE, gpu), out)  # warm-up
    torch.cuda.synchronize()
    torch.cuda.set_sync_debug_mode("error")
    try:
        ds = backend.build_device_step(sc.qsl, sc.seq, bt_d, slots_d, len(reqs), state.STORE, gpu)
        impl._forward_device(layer, sc.query, sc.key, sc.value, sc.kv_cache, ds, out)
    finally:
        torch.cuda.set_sync_debug_mode(0)
    torch.cuda.synchronize()
    state.STORE = None
    assert float((out.double().cpu() - sc.ref).abs().max()) <= TOL[dtype]


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_forward_device_hybrid(gpu, dtype, monkeypatch):
    """device_step_hybrid: the decode rows' host tier shared with the host
    cores in a GPU-planned step (one copy of their tables per step, reused by
    every layer); the reference output, and the tables fetched once across
    two layers."""
    monkeypatch.setattr(backend, "OPS", _PrefillOps)
    G, C, BS, H, KVH, D = 24, 40, 16, 8, 2, 128
    sc = build_tiers(REQS16, G, C, H, KVH, D, BS, dtype, 1, gpu)
    state.STORE = state.HostKVStore(G, C, BS, KVH, D, dtype, k={"l0": sc.host_k, "l1": sc.host_k},
                                    v={"l0": sc.host_v, "l1": sc.host_v})
    impl = backend.SplitDecodeImpl(H, KVH, D, sc.scale, device_step_hybrid=True,
                                   hybrid_min_host_bytes=0)
    calls = []
    real_begin = ops.hybrid_split_begin
    monkeypatch.setattr(ops, "hybrid_split_begin",
                        lambda *a, **k: calls.append(1) or real_begin(*a, **k))
    R = sc.bt.shape[0]
    ds = backend.build_device_step(sc.qsl, sc.seq, sc.bt.to(gpu), sc.slots.to(gpu), R,
                                   state.STORE, gpu)
    assert ds is not None and ds.n_dec > 0
    out = torch.full_like(sc.query, float("nan"))
    impl._forward_device(SimpleNamespace(layer_name="l0", _k_scale=None, _v_scale=None),
                         sc.query, sc.key, sc.value, sc.kv_cache, ds, out)
    fetched = ds._host
    assert fetched is not None and len(calls) == 1
    # a second layer of the same step reuses the fetched tables (its KV
    # writes land on the same slots with the same values)
    out2 = torch.full_like(sc.query, float("nan"))
    impl._forward_device(SimpleNamespace(layer_name="l1", _k_scale=None, _v_scale=None),
                         sc.query, sc.key, sc.value, sc.kv_cache, ds, out2)
    assert ds._host is fetched and len(calls) == 2
    torch.cuda.synchronize()
    state.STORE = None
    for o in (out, out2):
        assert float((o.double().cpu() - sc.ref).abs().max()) <= TOL[dtype]


@pytest.mark.parametrize("fault", ["host_slot", "host_block_id"])
def test_device_planned_step_with_a_bad_host_id_writes_nothing_and_raises(gpu, monkeypatch,
                                                                          fault):
    """A step planned on the GPU with one host slot past the host tier, or one
    host block id past it (the reference's planner raises for the latter,
    plan.py:133-137, and store_kv checks every slot before any write,
    cpu_attn.cpp:506-510): neither tier receives any of the step's KV, the
    step's own check and the next step's builder raise the planner's
    RuntimeError, and once raised the error does not come back."""
    monkeypatch.setattr(backend, "OPS", _PrefillOps)
    G, C, BS, H, KVH, D, dtype = 24, 40, 16, 8, 2, 128, torch.float16
    sc = build_tiers(REQS16, G, C, H, KVH, D, BS, dtype, 5, gpu)
    state.STORE = state.HostKVStore(G, C, BS, KVH, D, dtype, k={"l0": sc.host_k},
                                    v={"l0": sc.host_v})
    bt, slots = sc.bt.clone(), sc.slots.clone()
    if fault == "host_slot":
        slots[0] = (G + C) * BS + 3  # row 0's new token, past the host tier
    else:
        bt[5, 2] = G + C + 7  # row 5's third block (a host block), past the host tier
    phys0, hk0, hv0 = sc.phys.clone(), sc.host_k.clone(), sc.host_v.clone()
    impl = backend.SplitDecodeImpl(H, KVH, D, sc.scale)
    layer = SimpleNamespace(layer_name="l0", _k_scale=None, _v_scale=None)
    R = bt.shape[0]
    out = torch.full_like(sc.query, float("nan"))
    ds = backend.build_device_step(sc.qsl, sc.seq, bt.to(gpu), slots.to(gpu), R, state.STORE, gpu)
    impl._forward_device(layer, sc.query, sc.key, sc.value, sc.kv_cache, ds, out)
    torch.cuda.synchronize()
    assert int(ds.errors.item()) == 1
    assert torch.equal(sc.phys, phys0)
    assert torch.equal(sc.host_k, hk0) and torch.equal(sc.host_v, hv0)
    with pytest.raises(RuntimeError, match="beyond GPU\\+CPU capacity"):
        ds.check_errors()
    with pytest.raises(RuntimeError, match="beyond GPU\\+CPU capacity"):
        backend.build_device_step(sc.qsl, sc.seq, bt.to(gpu), slots.to(gpu), R, state.STORE,
                                  gpu)
    # that second build was refused before planning: nothing is pending now,
    # and a good step runs and checks clean
    backend.raise_step_errors(wait=True)
    ds = backend.build_device_step(sc.qsl, sc.seq, sc.bt.to(gpu), sc.slots.to(gpu), R,
                                   state.STORE, gpu)
    out = torch.full_like(sc.query, float("nan"))
    impl._forward_device(layer, sc.query, sc.key, sc.value, sc.kv_cache, ds, out)
    torch.cuda.synchronize()
    ds.check_errors()
    backend.raise_step_errors(wait=True)
    state.STORE = None
    assert float((out.double().cpu() - sc.ref).abs().max()) <= TOL[dtype]
    phys = sc.phys.cpu()
    assert torch.equal(phys[..., :D], sc.ref_k[:G]) and torch.equal(phys[..., D:], sc.ref_v[:G])
    assert torch.equal(sc.host_k.transpose(1, 2), sc.ref_k[G:])
