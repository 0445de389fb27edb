"""GPU parity of the grouped-query kernel with both products on the matrix
cores (decode_mm.hip: groups of 4 to 16 query heads per kv head in one pass
of one 16-column group, larger groups in tasks of two or four column groups
(four up to D = 64) and passes of those; head sizes 32 to 128 in steps of 16;
the default for those shapes in HBM) against the float64 oracle.

Bars as in test_gpu_decode: fp32 out max-abs <= 2e-3; out in the KV dtype
fp16 2e-3 / bf16 1.6e-2 (atol and rtol); lse 1e-4 relative; empty rows
exactly 0 / -inf; a range error poisons only its own row. Besides the
reference's kind of inputs (N(0,1)), the cases stress what this kernel adds:
p fed to the matrix cores as two 16-bit parts (long rows, scores spread over
a wide range so most weights are tiny, fp16 and bf16), the lazily raised
running max (scores growing along the row), and the merge of 16 head columns
across the task's waves and across split tasks.
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from tests import cases
from tests.test_gpu_decode import (GQA_LENS, OUT_TOL_16BIT, assert_lse_close, assert_out_close,
                                   run_host_layout)
from vllm_fastdecoder_amd import ops

pytestmark = pytest.mark.gpu

LENS = GQA_LENS + [700, 333]


def _case(H, KVH, D, dtype, seed, lens=LENS, C=160):
    n = len(lens)
    q, kc, vc, bt, ln = cases.rand_case(n, H, KVH, D, 16, C, dtype,
                                        max_len=max(lens), seed=seed)
    ln[:] = torch.tensor(lens, dtype=torch.int32)
    # disjoint blocks for these lengths (rand_case laid its table out for its
    # own random lengths, reusing blocks once the cache was used up)
    nbs = [(L + 15) // 16 for L in lens]
    assert sum(nbs) <= C
    perm = torch.randperm(C, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    bt.zero_()
    pos = 0
    for i, nb in enumerate(nbs):
        bt[i, :nb] = perm[pos: pos + nb]
        pos += nb
    return q, kc, vc, bt, ln


def _check(out, lse, ref_out, ref_lse, lens, dtype, gpu):
    nz = lens > 0
    if out.dtype == torch.float32:
        assert_out_close(out, ref_out, 2e-3, mask=nz)
    else:
        tol = OUT_TOL_16BIT[dtype]
        assert_out_close(out, ref_out, tol, tol, mask=nz)
    assert_lse_close(lse, ref_lse, mask=nz)
    assert torch.all(out[~nz.to(gpu)] == 0)
    assert torch.all(torch.isneginf(lse[:, ~nz.to(gpu)]))


@pytest.mark.parametrize("G", [4, 5, 8, 12, 16, 20, 32, 36, 48, 71])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mm_kernel_matches_oracle(gpu, G, D, dtype, monkeypatch):
    """Host layout and vLLM's layout; whole rows, forced 2-block splits
    (split partials of 16 columns, the combine kernel) and the model's own
    choice; fp32 and 16-bit outputs. Groups past 16 heads take two or four
    column groups per task (20, 32: two; 36, 48, 71 at D = 64: four, with 28 /
    16 / 57 spare columns in the last pass; 36, 48, 71 at D = 128: passes of
    two)."""
    KVH = 2
    H = G * KVH
    q, kc, vc, bt, lens = _case(H, KVH, D, dtype, seed=G * D)
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    for split in ("0", "2", "16"):
        monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
        for out_dtype in (torch.float32, dtype):
            out, lse = run_host_layout(q, kc, vc, bt, lens, scale, out_dtype, gpu)
            _check(out, lse, ref_out, ref_lse, lens, dtype, gpu)
        o_v = torch.empty(len(LENS), H, D, dtype=torch.float32, device=gpu)
        o_v, l_v = ops.paged_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt.to(gpu),
                                    lens.to(gpu), scale, out=o_v)
        torch.cuda.synchronize()
        _check(o_v, l_v, ref_out, ref_lse, lens, dtype, gpu)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("kind", ["large", "spread", "rising"])
def test_mm_kernel_extreme_scores(gpu, dtype, kind):
    """Scores far from N(0,1): q x 300 (logits in the hundreds); q x 12 over
    2,000-token rows, so nearly every weight is tiny next to the largest
    (the case where a single 16-bit p would lose the most); K rows scaled up
    along the row, so the running max is raised again and again. Groups of 8
    at D = 128 and of 40 at D = 64 (four column groups per task, each with its
    own running max)."""
    for G, KVH, D in ((8, 2, 128), (40, 1, 64)):
        _extreme_case(gpu, dtype, kind, G, KVH, D)


def _extreme_case(gpu, dtype, kind, G, KVH, D):
    H = G * KVH
    lens = [2000, 1500, 17, 0, 1, 640]
    q, kc, vc, bt, ln = _case(H, KVH, D, torch.float32, seed=77, lens=lens, C=320)
    if kind == "large":
        q = q * 300.0
    elif kind == "spread":
        q = q * 12.0
    else:  # rising: block b's K scaled by 1 + b/8 in table order of each row
        kc = kc.clone()
        for i, L in enumerate(lens):
            for j in range((L + 15) // 16):
                kc[bt[i, j]] *= 1.0 + j / 8.0
    q, kc, vc = q.to(dtype), kc.to(dtype), vc.to(dtype)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, ln, 1.0 / math.sqrt(D))
    out, lse = run_host_layout(q, kc, vc, bt, ln, 1.0 / math.sqrt(D), torch.float32, gpu)
    nz = (ln > 0).to(gpu)
    assert torch.isfinite(out[nz]).all() and torch.isfinite(lse[:, nz]).all()
    _check(out, lse, ref_out, ref_lse, ln, dtype, gpu)


@pytest.mark.parametrize("G,D", [(16, 128), (48, 64)])
def test_mm_kernel_range_errors_poison_only_their_rows(gpu, G, D):
    KVH = 2
    H = G * KVH
    q, kc, vc, bt, lens = _case(H, KVH, D, torch.bfloat16, seed=5)
    lens[:4] = torch.tensor([64, 40, 33, 17], dtype=torch.int32)
    C = kc.shape[0]
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    bt_bad = bt.clone()
    bt_bad[1, 1] = C + 5  # past the cache
    lens_bad = lens.clone()
    lens_bad[2] = bt.shape[1] * 16 + 1  # beyond the table
    out, lse = run_host_layout(q, kc, vc, bt_bad, lens_bad, scale, torch.float32, gpu)
    assert torch.isnan(out[1]).all() and torch.isnan(lse[:, 1]).all()
    assert torch.isnan(out[2]).all() and torch.isnan(lse[:, 2]).all()
    ok = torch.ones(len(lens), dtype=torch.bool)
    ok[1] = ok[2] = False
    ok &= lens > 0
    assert_out_close(out, ref_out, 2e-3, mask=ok)
    assert_lse_close(lse, ref_lse, mask=ok)


@pytest.mark.parametrize("G", [8, 16, 48])
def test_mm_kernel_two_tiers_in_hbm(gpu, G):
    """The fused two-tier launch on this kernel: both tiers in HBM (a tier in
    pinned host memory takes the VALU kernel), each row's blocks split
    between them, against the oracle over the row's blocks as one list."""
    KVH, D, dtype = 2, 128, torch.bfloat16
    H = G * KVH
    lens = [700, 300, 1, 0, 17, 64]
    n = len(lens)
    q, kc, vc, bt, ln = _case(H, KVH, D, dtype, seed=G, lens=lens, C=160)
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, ln, scale)
    # tier 0: each row's first k blocks in vLLM's layout; tier 1: the rest in
    # the host layout (both in HBM); tier-relative tables
    W = bt.shape[1]
    bt0 = torch.zeros(n, W, dtype=torch.int32)
    bt1 = torch.zeros(n, W, dtype=torch.int32)
    l0 = torch.zeros(n, dtype=torch.int32)
    l1 = torch.zeros(n, dtype=torch.int32)
    for i, L in enumerate(lens):
        nb = (L + 15) // 16
        k = nb // 2
        bt0[i, :k] = bt[i, :k]
        bt1[i, : nb - k] = bt[i, k:nb]
        l0[i] = 16 * k
        l1[i] = L - 16 * k
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.split_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt0.to(gpu), l0.to(gpu), kc.to(gpu),
                     vc.to(gpu), bt1.to(gpu), l1.to(gpu), scale, out=out, lse=lse)
    torch.cuda.synchronize()
    _check(out, lse, ref_out, ref_lse, ln, dtype, gpu)


def test_mm_kernel_row_order_bit_identical(gpu):
    """Results do not depend on the scheduling order of the rows."""
    G, KVH, D = 12, 2, 64
    H = G * KVH
    q, kc, vc, bt, lens = _case(H, KVH, D, torch.float16, seed=9)
    qd, kd, vd, btd, ld = q.to(gpu), kc.to(gpu), vc.to(gpu), bt.to(gpu), lens.to(gpu)
    outs = []
    for order in (None, ops.longest_first(lens), torch.arange(len(LENS) - 1, -1, -1,
                                                               dtype=torch.int32)):
        out = torch.empty(len(LENS), H, D, dtype=torch.float32, device=gpu)
        lse = torch.empty(H, len(LENS), dtype=torch.float32, device=gpu)
        ops.decode_attn(qd, kd, vd, btd, ld, 0.125, out, lse,
                        row_order=None if order is None else order.to(gpu))
        torch.cuda.synchronize()
        outs.append((out, lse))
    for out, lse in outs[1:]:
        assert torch.equal(out, outs[0][0]) and torch.equal(lse, outs[0][1])


@pytest.mark.parametrize("G", [1, 2, 3])
@pytest.mark.parametrize("D", [64, 128])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mm_kernel_forced_on_small_groups(gpu, G, D, dtype, monkeypatch):
    """FD_DECODE_KERNEL=mm on groups the planner gives the VALU kernel: 1-3
    real heads in the 16 columns (the rest repeat the last head, unwritten);
    whole rows and forced 2-block splits."""
    monkeypatch.setenv("FD_DECODE_KERNEL", "mm")
    KVH = 4
    H = G * KVH
    q, kc, vc, bt, lens = _case(H, KVH, D, dtype, seed=100 + G * D)
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    for split in ("0", "2"):
        monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
        for out_dtype in (torch.float32, dtype):
            out, lse = run_host_layout(q, kc, vc, bt, lens, scale, out_dtype, gpu)
            _check(out, lse, ref_out, ref_lse, lens, dtype, gpu)


@pytest.mark.parametrize("D", [32, 48, 80, 96, 112])
@pytest.mark.parametrize("G", [4, 8, 20, 40])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_mm_kernel_head_sizes_between(gpu, D, G, dtype, monkeypatch):
    """Head sizes that are multiples of 16 but not of 32 (the last q.K step
    masked past D) or not powers of two (V chunks spread over whole 64-lane
    loads): host layout and vLLM's, whole rows and forced 2-block splits,
    fp32 and 16-bit outputs."""
    KVH = 2
    H = G * KVH
    q, kc, vc, bt, lens = _case(H, KVH, D, dtype, seed=G * D + 1)
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    for split in ("0", "2"):
        monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
        for out_dtype in (torch.float32, dtype):
            out, lse = run_host_layout(q, kc, vc, bt, lens, scale, out_dtype, gpu)
            _check(out, lse, ref_out, ref_lse, lens, dtype, gpu)
        o_v = torch.empty(len(LENS), H, D, dtype=torch.float32, device=gpu)
        o_v, l_v = ops.paged_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt.to(gpu),
                                    lens.to(gpu), scale, out=o_v)
        torch.cuda.synchronize()
        _check(o_v, l_v, ref_out, ref_lse, lens, dtype, gpu)


@pytest.mark.parametrize("D,G", [(80, 8), (96, 8), (112, 8), (96, 36), (48, 40), (64, 71)])
def test_mm_kernel_head_sizes_between_two_tiers(gpu, D, G):
    """The fused two-tier launch at those head sizes (both tiers in HBM), and
    with two or four column groups per task (36 at D = 96: passes of 32; 40 at
    D = 48 and 71 at D = 64: tasks of 64)."""
    KVH, dtype = 2, torch.bfloat16
    H = G * KVH
    lens = [700, 300, 1, 0, 17, 64]
    n = len(lens)
    q, kc, vc, bt, ln = _case(H, KVH, D, dtype, seed=D, lens=lens, C=160)
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, ln, scale)
    W = bt.shape[1]
    bt0 = torch.zeros(n, W, dtype=torch.int32)
    bt1 = torch.zeros(n, W, dtype=torch.int32)
    l0 = torch.zeros(n, dtype=torch.int32)
    l1 = torch.zeros(n, dtype=torch.int32)
    for i, L in enumerate(lens):
        nb = (L + 15) // 16
        k = nb // 2
        bt0[i, :k] = bt[i, :k]
        bt1[i, : nb - k] = bt[i, k:nb]
        l0[i] = 16 * k
        l1[i] = L - 16 * k
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.split_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt0.to(gpu), l0.to(gpu), kc.to(gpu),
                     vc.to(gpu), bt1.to(gpu), l1.to(gpu), scale, out=out, lse=lse)
    torch.cuda.synchronize()
    _check(out, lse, ref_out, ref_lse, ln, dtype, gpu)


def test_large_mha_launches_take_the_matrix_core_kernel(gpu, monkeypatch):
    """MHA at D = 128 takes this kernel once there are >= 8 tasks per CU and
    rows that may reach 1,024 tokens; smaller launches, short rows, other
    head sizes and G = 2 stay on the VALU kernel."""
    monkeypatch.delenv("FD_DECODE_KERNEL", raising=False)
    monkeypatch.delenv("FD_SPLIT_BLOCKS", raising=False)
    cus = torch.cuda.get_device_properties(gpu).multi_processor_count
    n_big = 8 * cus // 32  # tasks = n x 32 kv heads = 8 per CU

    def kernel(n, H, KVH, D, W):
        return ops.decode_plan_info(n, H, KVH, D, 16, W, torch.float16)["kernel"]

    assert kernel(128, 32, 32, 128, 128) == "mm"          # the vicuna-7b shape
    assert kernel(n_big, 32, 32, 128, 64) == "mm"
    assert kernel(n_big - 1, 32, 32, 128, 64) == "valu"   # fewer tasks
    assert kernel(n_big, 32, 32, 128, 63) == "valu"       # rows up to 1,008 tokens
    assert kernel(128, 32, 32, 96, 128) == "valu"
    assert kernel(128, 32, 16, 128, 128) == "valu"        # G = 2
    assert kernel(8, 32, 32, 128, 64) == "valu"           # the small batch
