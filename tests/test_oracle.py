"""CPU checks that pin the oracle before it is trusted as the GPU checker.

Each oracle function is checked against something it did not produce:
  * the reference's own cpu_attn.cpp, compiled from its source into
    oracle/_ref (decode_attn, store_kv), on the reference's test grid;
  * golden fixtures written from that build (tests/golden/), so the check
    also holds where the reference tree is absent;
  * closed forms: one token (out = v, lse = s), identical keys
    (out = mean V, lse = s + log L), brute-force pure-Python attention;
  * invariants: split + merge == monolithic for any block partition, block
    order inside a row is irrelevant only through the softmax, the merge's
    empty conventions (tests/test_cpu_kernel.py:99-147);
  * planted mistakes (in the oracle, on the CPU) that the same comparisons
    must reject, so each check is shown to be sensitive.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests import cases

GOLDEN = Path(__file__).resolve().parent / "golden"


def _ref_or_skip():
    ext = oracle.ref_ext()
    if ext is None:
        pytest.skip("reference build (oracle/_ref) not present")
    return ext


# ------------------------------------------------------------------ decode


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,KVH", [(8, 8), (8, 2), (4, 1)])
@pytest.mark.parametrize("D", [64, 128, 72])
def test_oracle_matches_reference_build(dtype, H, KVH, D):
    """Float64 oracle vs the reference kernel on its own test grid and
    tolerances (tests/test_cpu_kernel.py:38-57)."""
    ext = _ref_or_skip()
    n, BS, C = 7, 16, 64
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len=93, seed=D + H)
    lens[3] = 0
    scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    lse = torch.empty(H, n, dtype=torch.float32)
    ext.decode_attn(q, kc, vc, bt, lens, scale, out, lse)
    o_ref, l_ref = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    nz = lens > 0
    tol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}[dtype]
    torch.testing.assert_close(out[nz].double(), o_ref[nz], atol=tol, rtol=tol)
    torch.testing.assert_close(lse[:, nz].double(), l_ref[:, nz], atol=1e-4, rtol=1e-5)
    assert torch.all(o_ref[~nz] == 0) and torch.all(torch.isneginf(l_ref[:, ~nz]))


def test_oracle_large_scores():
    """q x 300 with unit scale stays finite (tests/test_cpu_kernel.py:60-72)."""
    ext = _ref_or_skip()
    n, H, KVH, D, BS, C = 2, 4, 4, 64, 16, 8
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, torch.float32, 40, 0)
    q = q * 300.0
    out = torch.empty_like(q)
    lse = torch.empty(H, n, dtype=torch.float32)
    ext.decode_attn(q, kc, vc, bt, lens, 1.0, out, lse)
    o_ref, l_ref = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, 1.0)
    assert torch.isfinite(o_ref).all() and torch.isfinite(l_ref).all()
    torch.testing.assert_close(out.double(), o_ref, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(lse.double(), l_ref, atol=1e-3, rtol=1e-6)


def test_port_matches_reference_build():
    """The fp32 two-pass restatement (the CPU baseline fallback) agrees with the
    reference kernel on the correctness workload."""
    ext = _ref_or_skip()
    w = cases.WORKLOADS["correctness"]
    lens, bt, pool = cases.draw_lens_and_tables(w)
    k, v, _ = cases.kv_pool(w, pool, "host", "cpu")
    q = cases.queries(w, "cpu")
    out = torch.empty_like(q)
    lse = torch.empty(w.H, w.n)
    ext.decode_attn(q, k, v, bt, lens, w.scale, out, lse)
    out32 = torch.empty(w.n, w.H, w.D)
    lse32 = torch.empty(w.H, w.n)
    oracle.decode_attn_cpu_f32(q, k, v, bt, lens, w.scale, out32, lse32)
    torch.testing.assert_close(out32.half().float(), out.float(), atol=2e-3, rtol=2e-3)
    torch.testing.assert_close(lse32, lse, atol=1e-4, rtol=1e-5)


def test_oracle_matches_golden_fixture():
    """Outputs of the reference build stored under tests/golden (written by
    tests/golden/make_golden.py), regenerated inputs checked by checksum."""
    data = np.load(GOLDEN / "ref_decode_attn.npz")
    for name in sorted({k.split("__")[0] for k in data.files}):
        meta = data[f"{name}__meta"]
        n, H, KVH, D, BS, C, max_len, seed, dt_code, empty_row = (int(x) for x in meta)
        dtype = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32}[dt_code]
        q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len, seed)
        if empty_row >= 0:
            lens[empty_row] = 0
        digest = cases.tensor_digest(q, kc, vc, bt, lens)
        assert digest == str(data[f"{name}__digest"]), f"{name}: generator drift"
        scale = 1.0 / math.sqrt(D)
        o_ref, l_ref = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
        out = torch.from_numpy(data[f"{name}__out"]).double()
        lse = torch.from_numpy(data[f"{name}__lse"]).double()
        nz = lens > 0
        tol = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-5}[dtype]
        torch.testing.assert_close(out[nz], o_ref[nz], atol=tol, rtol=tol)
        torch.testing.assert_close(lse[:, nz], l_ref[:, nz], atol=1e-4, rtol=1e-5)


def _brute(q, kc, vc, bt, lens, scale):
    """Pure-Python softmax attention over the listed tokens (tiny cases)."""
    n, H, D = q.shape
    _, KVH, BS, _ = kc.shape
    G = H // KVH
    out = [[[0.0] * D for _ in range(H)] for _ in range(n)]
    lse = [[float("-inf")] * n for _ in range(H)]
    for i in range(n):
        L = int(lens[i])
        for h in range(H):
            if L == 0:
                continue
            kh = h // G
            s = []
            for t in range(L):
                b = int(bt[i, t // BS])
                krow = kc[b, kh, t % BS].tolist()
                s.append(scale * sum(a * c for a, c in zip(q[i, h].tolist(), krow)))
            m = max(s)
            z = sum(math.exp(x - m) for x in s)
            lse[h][i] = m + math.log(z)
            for t in range(L):
                b = int(bt[i, t // BS])
                vrow = vc[b, kh, t % BS].tolist()
                p = math.exp(s[t] - m) / z
                for d in range(D):
                    out[i][h][d] += p * vrow[d]
    return torch.tensor(out, dtype=torch.float64), torch.tensor(lse, dtype=torch.float64)


def test_oracle_matches_brute_force():
    q, kc, vc, bt, lens = cases.rand_case(3, 4, 2, 8, 4, 6, torch.float32, 9, 17)
    o, l = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, 0.37)
    ob, lb = _brute(q.double(), kc.double(), vc.double(), bt, lens, 0.37)
    torch.testing.assert_close(o, ob, atol=1e-12, rtol=1e-12)
    torch.testing.assert_close(l, lb, atol=1e-12, rtol=1e-12)


def test_oracle_closed_forms():
    """One token: out = v, lse = scale q.k. Identical keys: out = mean(V) and
    lse = scale q.k + log L."""
    g = torch.Generator().manual_seed(2)
    D, BS, H = 16, 4, 2
    q = torch.randn(2, H, D, generator=g)
    kc = torch.randn(3, 1, BS, D, generator=g)
    vc = torch.randn(3, 1, BS, D, generator=g)
    bt = torch.tensor([[2, 0, 1], [1, 2, 0]], dtype=torch.int32)
    lens = torch.tensor([1, 0], dtype=torch.int32)
    o, l = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, 0.5)
    for h in range(H):
        torch.testing.assert_close(o[0, h], vc[2, 0, 0].double())
        assert abs(float(l[h, 0]) - 0.5 * float(q[0, h].double() @ kc[2, 0, 0].double())) < 1e-12
    assert torch.all(o[1] == 0) and torch.all(torch.isneginf(l[:, 1]))
    kc_same = kc.clone()
    kc_same[:, 0] = kc[0, 0, 0]  # every token has the same key
    lens = torch.tensor([11, 7], dtype=torch.int32)
    o, l = oracle.decode_attn_host_layout_f64(q, kc_same, vc, bt, lens, 0.5)
    for i in range(2):
        L = int(lens[i])
        rows = torch.stack([vc[int(bt[i, t // BS]), 0, t % BS] for t in range(L)]).double()
        for h in range(H):
            torch.testing.assert_close(o[i, h], rows.mean(0))
            s = 0.5 * float(q[i, h].double() @ kc[0, 0, 0].double())
            assert abs(float(l[h, i]) - (s + math.log(L))) < 1e-10


def test_oracle_strided_layout_equals_host_layout():
    """The generic-stride reader sees vLLM's [B, BS, KVH, 2D] view and the
    host layout [C, KVH, BS, D] of the same cache identically."""
    q, kc, vc, bt, lens = cases.rand_case(4, 8, 2, 32, 16, 12, torch.float16, 70, 9)
    kv = torch.empty(12, 16, 2, 64, dtype=torch.float16)
    kv[..., :32] = kc.transpose(1, 2)
    kv[..., 32:] = vc.transpose(1, 2)
    o1, l1 = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, 0.2)
    o2, l2, st = oracle.decode_attn_f64(q, kv[..., :32], kv[..., 32:], oracle.VLLM_DIMS, bt, lens, 0.2)
    assert st == 0
    assert torch.equal(o1, o2) and torch.equal(l1, l2)


def test_oracle_range_error_flagged():
    q, kc, vc, bt, lens = cases.rand_case(3, 4, 4, 16, 16, 8, torch.float16, 40, 3)
    lens[:] = torch.tensor([40, 20, 5], dtype=torch.int32)
    bt[1, 1] = 99
    o, l, st = oracle.decode_attn_f64(q, kc, vc, oracle.HOST_DIMS, bt, lens, 0.25)
    assert st == 2
    assert torch.isnan(o[1]).all() and torch.isfinite(o[0]).all() and torch.isfinite(o[2]).all()


# ------------------------------------------------------------------ merge


def _split_even_odd(bt, lens, BS):
    n, W = bt.shape
    bt_a = torch.zeros_like(bt)
    bt_b = torch.zeros_like(bt)
    la = torch.zeros_like(lens)
    lb = torch.zeros_like(lens)
    for i in range(n):
        L = int(lens[i])
        nb = (L + BS - 1) // BS
        a = b = 0
        for j in range(nb):
            ntok = BS if j < nb - 1 else L - (nb - 1) * BS
            if j % 2 == 0:
                bt_a[i, a] = bt[i, j]
                a += 1
                la[i] += ntok
            else:
                bt_b[i, b] = bt[i, j]
                b += 1
                lb[i] += ntok
    return bt_a, la, bt_b, lb


def test_split_and_merge_equals_monolithic():
    """Core invariant (tests/test_cpu_kernel.py:99-138): the LSE merge of the
    partials over any block partition equals attention over all blocks."""
    q, kc, vc, bt, lens = cases.rand_case(5, 8, 2, 128, 16, 64, torch.float16, 80, 7)
    lens.clamp_(min=1)
    scale = 128 ** -0.5
    full, full_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    bt_a, la, bt_b, lb = _split_even_odd(bt, lens, 16)
    oa, lsa = oracle.decode_attn_host_layout_f64(q, kc, vc, bt_a, la, scale)
    ob, lsb = oracle.decode_attn_host_layout_f64(q, kc, vc, bt_b, lb, scale)
    merged, mlse = oracle.merge_f64(oa.float(), lsa.float(), ob.float(), lsb.float())
    torch.testing.assert_close(merged, full, atol=1e-6, rtol=0)
    torch.testing.assert_close(mlse, full_lse, atol=1e-5, rtol=0)
    # float64 partials merge to the float64 whole up to float64 rounding
    merged, mlse = oracle.merge_f64(oa, lsa, ob, lsb)
    torch.testing.assert_close(merged, full, atol=1e-12, rtol=0)
    torch.testing.assert_close(mlse, full_lse, atol=1e-12, rtol=0)
    # planted mistake: merging with unnormalised weights must be caught
    wrong = oa.double() * torch.exp(lsa.double()).t().unsqueeze(-1) + ob.double() * torch.exp(lsb.double()).t().unsqueeze(-1)
    assert float((wrong - full).abs().max()) > 2e-3


def test_merge_empty_conventions():
    """+inf (FlashAttention's empty) and -inf mean empty; both empty gives 0
    (cpu_ops.py:100-113, tests/test_cpu_kernel.py:141-147)."""
    o_a = torch.zeros(3, 2, 8)
    lse_a = torch.full((2, 3), float("inf"))
    o_b = torch.randn(3, 2, 8, generator=torch.Generator().manual_seed(0))
    lse_b = torch.randn(2, 3, generator=torch.Generator().manual_seed(1))
    out, olse = oracle.merge_f64(o_a, lse_a, o_b, lse_b)
    torch.testing.assert_close(out, o_b.double())
    torch.testing.assert_close(olse, lse_b.double())
    out, olse = oracle.merge_f64(o_b, torch.full((2, 3), float("-inf")), o_b,
                                 torch.full((2, 3), float("inf")))
    assert torch.all(out == 0) and torch.all(torch.isneginf(olse))


def test_merge_two_point_closed_form():
    """Two partials with lse difference d: weights 1/(1+e^-d), 1/(1+e^d)."""
    o_a = torch.ones(1, 1, 4)
    o_b = -torch.ones(1, 1, 4)
    for d in (0.0, 1.0, -3.5, 40.0):
        out, _ = oracle.merge_f64(o_a, torch.tensor([[d]]), o_b, torch.tensor([[0.0]]))
        wa = 1.0 / (1.0 + math.exp(-d))
        assert abs(float(out[0, 0, 0]) - (wa - (1 - wa))) < 1e-12


# ------------------------------------------------------------------ slot write


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_cache_write_matches_reference_store_kv(dtype):
    """Bit-exact against the reference's store_kv (tests/test_cpu_kernel.py:75-88)."""
    ext = _ref_or_skip()
    C, KVH, BS, D, m = 10, 4, 16, 128, 37
    g = torch.Generator().manual_seed(1)
    kc = torch.zeros(C, KVH, BS, D, dtype=dtype)
    vc = torch.zeros_like(kc)
    k = torch.randn(m, KVH, D, generator=g).to(dtype)
    v = torch.randn(m, KVH, D, generator=g).to(dtype)
    slots = torch.randperm(C * BS, generator=g)[:m].to(torch.int64)
    kc2, vc2 = kc.clone(), vc.clone()
    ext.store_kv(k, v, slots, kc, vc)
    st, _ = oracle.cache_write(k, v, kc2, vc2, (kc2.stride(0), kc2.stride(2), kc2.stride(1)), C, BS,
                               slots, check_all=True)
    assert st == 0
    assert torch.equal(kc, kc2) and torch.equal(vc, vc2)


def test_cache_write_range_rules():
    """store_kv: any slot past the tier rejects the whole call before writing
    (cpu_attn.cpp:506-510); reshape_and_cache: slot < 0 skipped, slots past
    the cache skipped and counted."""
    kc = torch.zeros(2, 1, 16, 8, dtype=torch.float16)
    vc = torch.zeros_like(kc)
    k = torch.ones(2, 1, 8, dtype=torch.float16)
    st, _ = oracle.cache_write(k, k, kc, vc, (kc.stride(0), kc.stride(2), kc.stride(1)), 2, 16,
                               torch.tensor([3, 32]), check_all=True)
    assert st == 2 and torch.all(kc == 0)
    ext = oracle.ref_ext()
    if ext is not None:
        with pytest.raises(RuntimeError):
            ext.store_kv(k, k, torch.tensor([3, 32], dtype=torch.int64), kc, vc)
        assert torch.all(kc == 0)
    st, oor = oracle.cache_write(k, k, kc, vc, (kc.stride(0), kc.stride(2), kc.stride(1)), 2, 16,
                                 torch.tensor([-1, 40]), check_all=False)
    assert st == 0 and oor == 1 and torch.all(kc == 0)
    # reference stand-in semantics (tests/test_plan_and_forward.py:88-95)
    st, oor = oracle.cache_write(k, k, kc, vc, (kc.stride(0), kc.stride(2), kc.stride(1)), 2, 16,
                                 torch.tensor([-1, 17]), check_all=False)
    assert torch.all(kc[1, 0, 1] == 1) and int((kc != 0).sum()) == 8
