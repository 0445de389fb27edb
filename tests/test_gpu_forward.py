"""GPU tests of the split path end to end: planner -> device plan ->
_forward_split (HBM-tier KV write, pinned host-tier KV write, both partials,
merge) against attention over one unified cache.

Follows the reference's own forward tests (tests/test_plan_and_forward.py:
123-256, 345-385): the prefill forms of OPS.fa (P and F rows, not on the
decode path) are served by a float32 torch stand-in defined here, the decode
partial by the library's HIP kernel. Tolerances: output 3e-3 max-abs for fp16
(2e-3 attention error + fp16 rounding), 2e-2 for bf16, 1e-4 for fp32; both
tiers bit-exact against the unified reference cache afterwards.
"""

from __future__ import annotations

import math
from types import SimpleNamespace

import pytest
import torch

from tests.test_plan import KATS, scenario
from vllm_fastdecoder_amd import backend, plan, state
from vllm_fastdecoder_amd.pinned import pinned_zeros

pytestmark = pytest.mark.gpu


def _attend_ref(q, k, v, scale, causal):
    """float64 attention; q [Lq,H,D], k/v [Lk,KVH,D] -> [Lq,H,D]."""
    H, KVH = q.shape[1], k.shape[1]
    k = k.double().repeat_interleave(H // KVH, dim=1)
    v = v.double().repeat_interleave(H // KVH, dim=1)
    s = torch.einsum("qhd,khd->hqk", q.double(), k) * scale
    if causal:
        Lq, Lk = q.shape[0], k.shape[0]
        mask = torch.arange(Lk)[None, :] > (torch.arange(Lq)[:, None] + (Lk - Lq))
        s = s.masked_fill(mask[None], float("-inf"))
    return torch.einsum("hqk,khd->qhd", torch.softmax(s, dim=-1), v)


class _PrefillOps(backend.HipOps):
    """HIP decode partial + a float32 stand-in for the prefill forms of fa."""

    @staticmethod
    def fa(q, k, v, cu_seqlens_q=None, max_seqlen_q=1, seqused_k=None, max_seqlen_k=None,
           softmax_scale=None, causal=False, block_table=None, cu_seqlens_k=None,
           return_softmax_lse=False, **kw):
        if max_seqlen_q == 1 and block_table is not None and not causal:
            return backend.HipOps.fa(q=q, k=k, v=v, cu_seqlens_q=cu_seqlens_q, max_seqlen_q=1,
                                     seqused_k=seqused_k, softmax_scale=softmax_scale,
                                     block_table=block_table,
                                     return_softmax_lse=return_softmax_lse, **kw)
        outs = []
        n = cu_seqlens_q.numel() - 1
        for b in range(n):
            q0, q1 = int(cu_seqlens_q[b]), int(cu_seqlens_q[b + 1])
            if block_table is not None:
                L = int(seqused_k[b])
                bs = k.shape[1]
                blks = block_table[b, : (L + bs - 1) // bs].long()
                kk = k[blks].reshape(-1, k.shape[2], k.shape[3])[:L]
                vv = v[blks].reshape(-1, v.shape[2], v.shape[3])[:L]
            else:
                k0, k1 = int(cu_seqlens_k[b]), int(cu_seqlens_k[b + 1])
                kk, vv = k[k0:k1], v[k0:k1]
            outs.append(_attend_ref(q[q0:q1].cpu(), kk.cpu(), vv.cpu(), softmax_scale, causal))
        return torch.cat(outs).to(q.dtype).to(q.device)


@pytest.fixture
def prefill_ops(monkeypatch):
    monkeypatch.setattr(backend, "OPS", _PrefillOps)
    yield
    state.STORE = None


def build_tiers(reqs, G, C, H, KVH, D, BS, dtype, seed, dev):
    """Unified logical cache over ids [0, G+C), this step's q/k/v, the
    reference output, and the two tiers in their real layouts."""
    g = torch.Generator().manual_seed(seed)
    uk = torch.randn(G + C, BS, KVH, D, generator=g).to(dtype)
    uv = torch.randn(G + C, BS, KVH, D, generator=g).to(dtype)
    qsl, seq, bt, slots = scenario(reqs, BS)
    T = int(qsl[-1])
    query = torch.randn(T, H, D, generator=g).to(dtype)
    key = torch.randn(T, KVH, D, generator=g).to(dtype)
    value = torch.randn(T, KVH, D, generator=g).to(dtype)
    rk, rv = uk.clone(), uv.clone()
    for t, s in enumerate(slots.tolist()):
        rk[s // BS, s % BS] = key[t]
        rv[s // BS, s % BS] = value[t]
    scale = 1.0 / math.sqrt(D)
    ref = torch.zeros(T, H, D, dtype=torch.float64)
    for i, (ctx, ql, blocks) in enumerate(reqs):
        L = ctx + ql
        kk = rk[torch.tensor(blocks)].reshape(-1, KVH, D)[:L]
        vv = rv[torch.tensor(blocks)].reshape(-1, KVH, D)[:L]
        ref[qsl[i]: qsl[i + 1]] = _attend_ref(query[qsl[i]: qsl[i + 1]], kk, vv, scale, True)
    phys = torch.empty(G, BS, KVH, 2 * D, dtype=dtype)
    phys[..., :D] = uk[:G]
    phys[..., D:] = uv[:G]
    phys = phys.to(dev)
    kv_cache = phys.permute(0, 2, 1, 3)  # logical [B, KVH, BS, 2D]
    host_k = pinned_zeros((C, KVH, BS, D), dtype)
    host_v = pinned_zeros((C, KVH, BS, D), dtype)
    host_k.copy_(uk[G:].transpose(1, 2))
    host_v.copy_(uv[G:].transpose(1, 2))
    return SimpleNamespace(qsl=qsl, seq=seq, bt=bt, slots=slots, query=query.to(dev),
                           key=key.to(dev), value=value.to(dev), ref=ref, ref_k=rk, ref_v=rv,
                           phys=phys, kv_cache=kv_cache, host_k=host_k, host_v=host_v, scale=scale)


TOL = {torch.float16: 3e-3, torch.bfloat16: 2e-2, torch.float32: 1e-4}

# BS=16 requests over a G+C = 24+40 id space: S with the last block on the
# host, P, F touching the host, S with no HBM tokens, S with an HBM block in
# the middle, single-token S, long S rows (tiled kernel, several blocks)
REQS16 = [
    (40, 1, [1, 2, 30]),
    (20, 1, [3, 4]),
    (0, 24, [31, 5]),
    (0, 9, [6]),
    (15, 1, [32]),
    (50, 1, [33, 7, 34, 8]),
    (0, 1, [35]),
    (150, 1, [9, 10, 36, 37, 11, 38, 39, 40, 12, 41]),
]


@pytest.mark.parametrize("mode", ["fused", "two_partials", "hybrid"])
@pytest.mark.parametrize("case", ["reqs4", "reqs16"])
@pytest.mark.parametrize("H,KVH", [(4, 4), (8, 2)])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_forward_split_matches_unified_attention(gpu, prefill_ops, case, H, KVH, dtype, mode):
    """S rows through the fused launch (default), the reference's two
    partials + merge, or the fused launch with 60% of each row's host blocks
    on the host cores; P and F rows as in the reference."""
    if case == "reqs4":
        reqs, G, C, BS, D = KATS["classification"]["reqs"], 10, 20, 4, 64
    else:
        reqs, G, C, BS, D = REQS16, 24, 40, 16, 128
    sc = build_tiers(reqs, G, C, H, KVH, D, BS, dtype, 1, gpu)
    hp = plan.build_host_plan(sc.qsl, sc.seq, sc.bt, sc.slots, G, C, BS)
    dp = plan.to_device(hp, sc.bt.to(gpu), gpu)
    state.STORE = state.HostKVStore(G, C, BS, KVH, D, dtype, k={"l0": sc.host_k}, v={"l0": sc.host_v})
    impl = backend.SplitDecodeImpl(H, KVH, D, sc.scale, fused_split=mode != "two_partials",
                                   cpu_fraction=0.6 if mode == "hybrid" else 0.0,
                                   hybrid_min_host_bytes=0)
    layer = SimpleNamespace(layer_name="l0", _k_scale=None, _v_scale=None)
    output = torch.full_like(sc.query, float("nan"))
    impl._forward_split(layer, sc.query, sc.key, sc.value, sc.kv_cache, dp, output)
    torch.cuda.synchronize()
    err = float((output.double().cpu() - sc.ref).abs().max())
    assert err <= TOL[dtype], err
    # both tiers hold exactly the unified reference cache
    phys = sc.phys.cpu()
    assert torch.equal(phys[..., :D], sc.ref_k[:G]) and torch.equal(phys[..., D:], sc.ref_v[:G])
    assert torch.equal(sc.host_k.transpose(1, 2), sc.ref_k[G:])
    assert torch.equal(sc.host_v.transpose(1, 2), sc.ref_v[G:])


def test_builder_then_forward_with_runner_padding(gpu, prefill_ops):
    """build_split_plan on runner-style inputs: a wider device block table,
    a slot mapping padded with -1, padded q/k/v rows
    (tests/test_plan_and_forward.py:345-385)."""
    G, C, H, KVH, D, BS, dtype = 24, 40, 8, 2, 128, 16, torch.float16
    sc = build_tiers(REQS16, G, C, H, KVH, D, BS, dtype, 3, gpu)
    state.STORE = state.HostKVStore(G, C, BS, KVH, D, dtype, k={"l0": sc.host_k}, v={"l0": sc.host_v})
    R, T = sc.bt.shape[0], int(sc.qsl[-1])
    bt_wide = torch.zeros(R + 2, 64, dtype=torch.int32)
    bt_wide[:R, : sc.bt.shape[1]] = sc.bt
    slot_pad = torch.full((T + 5,), -1, dtype=torch.int64)
    slot_pad[:T] = sc.slots
    dp = backend.build_split_plan(sc.qsl, sc.seq, bt_wide.to(gpu), slot_pad.to(gpu), R,
                                  state.STORE, gpu)
    assert isinstance(dp, plan.DevicePlan)
    pad = 5
    q = torch.cat([sc.query, torch.zeros(pad, H, D, dtype=dtype, device=gpu)])
    k = torch.cat([sc.key, torch.zeros(pad, KVH, D, dtype=dtype, device=gpu)])
    v = torch.cat([sc.value, torch.zeros(pad, KVH, D, dtype=dtype, device=gpu)])
    out = torch.full_like(q, float("nan"))
    backend.SplitDecodeImpl(H, KVH, D, sc.scale)._forward_split(
        SimpleNamespace(layer_name="l0", _k_scale=None, _v_scale=None), q, k, v, sc.kv_cache, dp, out)
    torch.cuda.synchronize()
    assert float((out[:T].double().cpu() - sc.ref).abs().max()) <= TOL[dtype]


def test_plan_none_when_no_host_tier_touched(gpu):
    store = state.HostKVStore(10, 5, 4, 2, 64, torch.float16)
    qsl, seq, bt, slots = scenario(KATS["all_gpu"]["reqs"], 4)
    assert backend.build_split_plan(qsl, seq, bt.to(gpu), slots.to(gpu), 2, store, gpu) is None
    assert backend.build_split_plan(qsl, seq, bt.to(gpu), slots.to(gpu), 2, None, gpu) is None


def test_hipops_fa_rejects_prefill_forms(gpu):
    q = torch.zeros(3, 4, 64, dtype=torch.float16, device=gpu)
    with pytest.raises(NotImplementedError):
        backend.HipOps.fa(q=q, k=q, v=q, cu_seqlens_q=torch.tensor([0, 3]), max_seqlen_q=3,
                          softmax_scale=0.1, causal=True)


@pytest.mark.parametrize("fused,planner,cpu_fraction",
                         [(True, "host", 0.0), (False, "host", 0.0), (True, "device", 0.0),
                          (True, "host", 0.6), (True, "host", "auto"),
                          (True, "device", "auto")])
def test_continuous_batching_simulation(gpu, fused, planner, cpu_fraction):
    """The config of the reference's GPU self-test at vicuna-7b head shapes:
    300 decode steps, G=256 HBM blocks, C=2048 host blocks, Poisson(4)
    arrivals, prompts U[64,512], outputs U[32,512], GPU-first allocation with
    block reuse; every step checked against monolithic attention over one
    G+C pool written with the same KV, and every slot written bit-exact. S
    rows through the fused launch and through two partials + merge, with the
    step planned on the host (one device-to-host copy per step, as in the
    reference) or on the GPU (none); and the fused launch with 60% of each
    row's host blocks reduced by the host cores (hybrid split), or the share
    balanced online, with either planner."""
    from tests.simulate import run_simulation

    stats = run_simulation(steps=300, seed=4, device=gpu, fused=fused, planner=planner,
                           cpu_fraction=cpu_fraction)
    print({k: v for k, v in stats.items() if k != "failures"})
    assert stats["failures"] == [], stats["failures"][:5]
    assert stats["rows_vs_f64"] >= stats["decode_rows"] // 20  # every row of every 10th step
    assert stats["decode_rows"] > 1000
    if planner == "device":
        assert stats["device_planned_steps"] > 250
    else:
        assert stats["split_steps"] > 100
    assert stats["max_err_vs_mono"] <= 2e-3
    assert stats["max_err_vs_f64"] <= 2e-3


@pytest.mark.parametrize("planner,cpu_fraction", [("host", 0.0), ("device", 0.0), ("host", "auto")])
def test_continuous_batching_simulation_32_token_blocks(gpu, planner, cpu_fraction):
    """The same simulation with vLLM cache blocks of 32 tokens: planning, the
    slot writes of both tiers, the fused launch (blocks as two 16-token
    tiles) and the hybrid split, every step against the monolithic oracle."""
    from tests.simulate import run_simulation

    stats = run_simulation(steps=120, seed=7, device=gpu, BS=32, G=128, C=1024, planner=planner,
                           cpu_fraction=cpu_fraction)
    print({k: v for k, v in stats.items() if k != "failures"})
    assert stats["failures"] == [], stats["failures"][:5]
    assert stats["rows_vs_f64"] >= stats["decode_rows"] // 20  # every row of every 10th step
    assert stats["decode_rows"] > 300
    assert stats["max_err_vs_mono"] <= 2e-3
    assert stats["max_err_vs_f64"] <= 2e-3


@pytest.mark.parametrize("H,KVH,dtype", [(32, 8, torch.bfloat16), (40, 8, torch.float16)])
@pytest.mark.parametrize("cpu_fraction", [0.0, "auto"])
def test_continuous_batching_simulation_grouped_heads(gpu, H, KVH, dtype, cpu_fraction):
    """The simulation at grouped-query head shapes (Llama-3's 4 and a 5-head
    group), through the fused launch and the hybrid split."""
    from tests.simulate import run_simulation

    tol = 2e-3 if dtype == torch.float16 else 1.6e-2  # 16-bit output of the split path
    stats = run_simulation(steps=120, seed=11, device=gpu, H=H, KVH=KVH, dtype=dtype,
                           cpu_fraction=cpu_fraction, tol=tol)
    print({k: v for k, v in stats.items() if k != "failures"})
    assert stats["failures"] == [], stats["failures"][:5]
    assert stats["rows_vs_f64"] >= stats["decode_rows"] // 20  # every row of every 10th step
    assert stats["decode_rows"] > 300
    assert stats["max_err_vs_mono"] <= tol
