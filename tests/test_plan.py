"""CPU tests of the per-step planner (block selection must be bit-exact).

* the reference planner's known answers (tests/test_plan_and_forward.py:199-227,
  transcribed into tests/golden/plan_kats.json) for both the product planner
  and the oracle;
* product vs oracle on every field for seeded random scenarios, including
  junk past each row's blocks and padded slot mappings (the runner's padding,
  tests/test_plan_and_forward.py:345-385; scripts/gpu_selftest.py:174-182);
* invariants neither implementation is used to compute: per-tier token
  counts add to the sequence length, each compacted table lists exactly the
  tier's block ids in sequence order then zeros, HBM widths are multiples of
  16, every slot lands in exactly one tier.
"""

from __future__ import annotations

import json
import random
from pathlib import Path

import pytest
import torch

from oracle.plan_oracle import PlanError, plan_oracle
from vllm_fastdecoder_amd import plan

KATS = json.loads((Path(__file__).resolve().parent / "golden" / "plan_kats.json").read_text())


def scenario(reqs, BS, junk_seed=None, G_C=None, slot_pad=0):
    """reqs: (ctx_len, q_len, block_ids) -> qsl, seq_lens, block_table, slots."""
    W = max(len(b) for _, _, b in reqs) if reqs else 1
    rng = random.Random(junk_seed)
    bt = torch.zeros(len(reqs), W, dtype=torch.int32)
    qsl, seq, slots = [0], [], []
    for i, (ctx, ql, blocks) in enumerate(reqs):
        L = ctx + ql
        assert len(blocks) == (L + BS - 1) // BS
        bt[i, : len(blocks)] = torch.tensor(blocks, dtype=torch.int32) if blocks else bt[i, :0]
        if junk_seed is not None:
            for c in range(len(blocks), W):
                bt[i, c] = rng.randrange(G_C)
        for p in range(ctx, L):
            slots.append(blocks[p // BS] * BS + p % BS)
        qsl.append(qsl[-1] + ql)
        seq.append(L)
    slots = slots + [-1] * slot_pad
    return (torch.tensor(qsl, dtype=torch.int32), torch.tensor(seq, dtype=torch.int32), bt,
            torch.tensor(slots, dtype=torch.int64))


def as_lists(hp: plan.HostPlan) -> dict:
    out = {}
    for k, v in hp.__dict__.items():
        out[k] = v.tolist() if isinstance(v, torch.Tensor) else v
    return out


def test_kat_classification():
    k = KATS["classification"]
    BS = KATS["block_size"]
    qsl, seq, bt, slots = scenario(k["reqs"], BS)
    e = k["expect"]
    hp = plan.build_host_plan(qsl, seq, bt, slots, k["G"], k["C"], BS)
    ref = plan_oracle(qsl.tolist(), seq.tolist(), bt.tolist(), slots.tolist(), k["G"], k["C"], BS)
    for got in (as_lists(hp), ref):
        assert got["p_req"] == e["p_req"]
        assert got["s_tok"] == e["s_tok"]
        assert got["f_cu"] == e["f_cu"]
        assert got["s_gpu_lens"] == e["s_gpu_lens"]
        assert got["s_cpu_lens"] == e["s_cpu_lens"]
        assert got["s_gpu_bt"][2][0] == e["s_gpu_bt_2_0"]
        assert got["s_cpu_bt"][2][:2] == e["s_cpu_bt_2_first2"]
    host = slots >= k["G"] * BS
    assert torch.equal(hp.gpu_slot_mapping[host], torch.full((int(host.sum()),), -1))
    assert torch.equal(hp.cpu_w_slot, slots[host] - k["G"] * BS)


def test_kat_none_when_all_gpu():
    k = KATS["all_gpu"]
    qsl, seq, bt, slots = scenario(k["reqs"], KATS["block_size"])
    assert plan.build_host_plan(qsl, seq, bt, slots, k["G"], k["C"], KATS["block_size"]) is None
    assert plan_oracle(qsl.tolist(), seq.tolist(), bt.tolist(), slots.tolist(), k["G"], k["C"],
                       KATS["block_size"]) is None


def test_kat_rejects_chunked_continuation_on_host_tier():
    k = KATS["chunked_continuation"]
    qsl, seq, bt, slots = scenario(k["reqs"], KATS["block_size"])
    with pytest.raises(NotImplementedError):
        plan.build_host_plan(qsl, seq, bt, slots, k["G"], k["C"], KATS["block_size"])
    with pytest.raises(NotImplementedError):
        plan_oracle(qsl.tolist(), seq.tolist(), bt.tolist(), slots.tolist(), k["G"], k["C"],
                    KATS["block_size"])


def test_rejects_block_beyond_capacity():
    qsl, seq, bt, slots = scenario([(4, 1, [1, 40])], 4)
    with pytest.raises(RuntimeError):
        plan.build_host_plan(qsl, seq, bt, slots, 10, 20, 4)
    with pytest.raises(PlanError):
        plan_oracle(qsl.tolist(), seq.tolist(), bt.tolist(), slots.tolist(), 10, 20, 4)


def random_reqs(rng: random.Random, G: int, C: int, BS: int, R: int):
    ids = list(range(1, G + C))
    rng.shuffle(ids)
    reqs = []
    for _ in range(R):
        kind = rng.random()
        if kind < 0.55:
            ctx, ql = rng.randint(0, 60), 1           # decode
        elif kind < 0.8:
            ctx, ql = 0, rng.randint(1, 40)           # fresh prefill
        elif kind < 0.9:
            ctx, ql = rng.randint(1, 30), 0           # inactive this step
        else:
            ctx, ql = rng.randint(1, 30), 1
        L = ctx + ql
        nb = (L + BS - 1) // BS
        if len(ids) < nb:
            break
        if rng.random() < 0.3:  # all in HBM
            blocks = [b for b in ids if b < G][:nb]
            if len(blocks) < nb:
                blocks = ids[:nb]
        else:
            blocks = ids[:nb]
        for b in blocks:
            ids.remove(b)
        if ql > 1 and ctx > 0:
            continue
        reqs.append((ctx, ql, blocks))
    return reqs


@pytest.mark.parametrize("seed", range(40))
def test_planner_matches_oracle_and_invariants(seed):
    rng = random.Random(seed)
    BS = rng.choice([4, 16])
    G = rng.randint(5, 60)
    C = rng.randint(5, 80)
    reqs = random_reqs(rng, G, C, BS, rng.randint(1, 12))
    if not reqs:
        return
    qsl, seq, bt, slots = scenario(reqs, BS, junk_seed=seed, G_C=G + C, slot_pad=rng.randint(0, 5))
    try:
        hp = plan.build_host_plan(qsl, seq, bt, slots, G, C, BS)
    except NotImplementedError:
        with pytest.raises(NotImplementedError):
            plan_oracle(qsl.tolist(), seq.tolist(), bt.tolist(), slots.tolist(), G, C, BS)
        return
    ref = plan_oracle(qsl.tolist(), seq.tolist(), bt.tolist(), slots.tolist(), G, C, BS)
    if hp is None:
        assert ref is None
        return
    got = as_lists(hp)
    for key, val in ref.items():
        if key == "classes":
            continue
        assert got[key] == val, key
    # dtypes of the reference's HostPlan (fastdecode/plan.py:26-62)
    for name in ("gpu_slot_mapping", "cpu_w_tok", "cpu_w_slot", "p_tok", "p_req", "s_tok", "f_tok"):
        assert getattr(hp, name).dtype == torch.int64, name
    for name in ("p_cu", "p_seqlens", "s_gpu_bt", "s_gpu_lens", "s_cpu_bt", "s_cpu_lens", "f_cu"):
        assert getattr(hp, name).dtype == torch.int32, name

    # invariants, from the scenario itself
    s_rows = [i for i, (ctx, ql, b) in enumerate(reqs) if ql == 1 and any(x >= G for x in b)]
    assert hp.s_tok.tolist() == [int(qsl[i]) for i in s_rows]
    assert hp.s_gpu_bt.shape[1] % 16 == 0
    for j, i in enumerate(s_rows):
        ctx, ql, blocks = reqs[i]
        assert int(hp.s_gpu_lens[j]) + int(hp.s_cpu_lens[j]) == ctx + ql
        hbm = [b for b in blocks if b < G]
        host = [b - G for b in blocks if b >= G]
        row_g = hp.s_gpu_bt[j].tolist()
        row_c = hp.s_cpu_bt[j].tolist()
        assert row_g[: len(hbm)] == hbm and all(x == 0 for x in row_g[len(hbm):])
        assert row_c[: len(host)] == host and all(x == 0 for x in row_c[len(host):])
    n_tok = int(qsl[-1])
    for t in range(n_tok):
        s = int(slots[t])
        g, h = int(hp.gpu_slot_mapping[t]), int(hp.host_slot_mapping[t])
        assert (g == s and h == -1) if s < G * BS else (g == -1 and h == s - G * BS)


def test_to_device_shapes_on_cpu():
    k = KATS["classification"]
    qsl, seq, bt, slots = scenario(k["reqs"], KATS["block_size"])
    hp = plan.build_host_plan(qsl, seq, bt, slots, k["G"], k["C"], KATS["block_size"])
    dp = plan.to_device(hp, bt, "cpu")
    assert dp.s_gpu_rows.tolist() == [0, 2]  # S rows holding HBM tokens
    assert dp.s_gpu_cu.tolist() == [0, 1, 2]
    assert torch.all(dp.s_gpu_lens > 0)
    assert dp.p_bt.shape == (2, bt.shape[1])
    assert torch.equal(dp.s_gpu_bt_all, hp.s_gpu_bt) and torch.equal(dp.s_cpu_lens, hp.s_cpu_lens)
