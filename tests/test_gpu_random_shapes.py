"""Seeded random shapes across the planner's whole dispatch table against the
float64 oracle: head counts (MHA, GQA with groups of 2-71 heads, one kv
head), head sizes (multiples of 8 up to 256, including the sizes the tiled
kernels build and the ones they run in a larger build), cache blocks of 16-64
tokens, fp16 / bf16 / fp32, forced task sizes from 1 block to whole rows,
16-bit and fp32 outputs, both cache layouts. Each case states the kernel the
planner chose, so a failure names the dispatch path. Same bars as
test_gpu_decode and test_gpu_decode_f32: fp32 out 2e-3 for 16-bit KV and
5e-5 for fp32 KV; 16-bit out at the reference's tolerances; lse 1e-4
relative; empty rows exactly 0 / -inf.
"""

from __future__ import annotations

import math

import numpy as np
import pytest
import torch

import oracle
from tests import cases
from tests.test_gpu_decode import OUT_TOL_16BIT, assert_lse_close, assert_out_close
from vllm_fastdecoder_amd import ops

pytestmark = pytest.mark.gpu

N_CASES = 64
HEADS = [(8, 8), (32, 32), (16, 8), (12, 4), (24, 8), (32, 8), (40, 8), (28, 4), (64, 8),
         (32, 2), (48, 2), (40, 1), (71, 1), (16, 1), (96, 2)]
HEAD_SIZES = [32, 48, 64, 72, 80, 96, 112, 128, 160, 192, 256]
BLOCK_SIZES = [16, 16, 16, 32, 64]
DTYPES = [torch.float16, torch.bfloat16, torch.float32]
SPLITS = ["0", "0", "1", "3", "16"]


def _draw(i):
    r = np.random.default_rng(1000 + i)
    H, KVH = HEADS[r.integers(len(HEADS))]
    D = int(HEAD_SIZES[r.integers(len(HEAD_SIZES))])
    BS = int(BLOCK_SIZES[r.integers(len(BLOCK_SIZES))])
    dtype = DTYPES[r.integers(len(DTYPES))]
    n = int(r.integers(1, 7))
    lens = [int(x) for x in r.integers(0, 700, n)]
    lens[0] = int(r.integers(1, 1200))
    split = SPLITS[r.integers(len(SPLITS))]
    out16 = bool(r.integers(2)) and dtype != torch.float32
    layout = "vllm" if r.integers(2) else "host"
    return H, KVH, D, BS, dtype, lens, split, out16, layout


@pytest.mark.parametrize("i", range(N_CASES))
def test_random_shape_matches_oracle(gpu, i, monkeypatch):
    H, KVH, D, BS, dtype, lens_l, split, out16, layout = _draw(i)
    n = len(lens_l)
    nbs = [(L + BS - 1) // BS for L in lens_l]
    C = sum(nbs) + 2
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len=max(lens_l),
                                          seed=i)
    lens[:] = torch.tensor(lens_l, dtype=torch.int32)
    perm = torch.randperm(C, generator=torch.Generator().manual_seed(i)).to(torch.int32)
    bt.zero_()
    pos = 0
    for r, nb in enumerate(nbs):
        bt[r, :nb] = perm[pos: pos + nb]
        pos += nb
    scale = 1.0 / math.sqrt(D)
    monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
    info = ops.decode_plan_info(n, H, KVH, D, BS, bt.shape[1], dtype)
    what = (f"case {i}: H={H} KVH={KVH} D={D} BS={BS} {dtype} lens={lens_l} split={split} "
            f"out16={out16} layout={layout} plan={info}")
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    out_dtype = dtype if out16 else torch.float32
    out = torch.empty(n, H, D, dtype=out_dtype, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    if layout == "host":
        ops.decode_attn(q.to(gpu), kc.to(gpu), vc.to(gpu), bt.to(gpu), lens.to(gpu), scale, out,
                        lse)
    else:
        kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
        ops.paged_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt.to(gpu), lens.to(gpu), scale,
                         out=out, lse=lse)
    torch.cuda.synchronize()
    nz = lens > 0
    try:
        if out16:
            tol = OUT_TOL_16BIT[dtype]
            assert_out_close(out, ref_out, tol, tol, mask=nz)
        else:
            assert_out_close(out, ref_out, 5e-5 if dtype == torch.float32 else 2e-3, mask=nz)
        assert_lse_close(lse, ref_lse, mask=nz)
        assert torch.all(out[~nz.to(gpu)] == 0), "empty rows: out not 0"
        assert torch.all(torch.isneginf(lse[:, ~nz.to(gpu)])), "empty rows: lse not -inf"
    except AssertionError as e:
        raise AssertionError(f"{what}: {e}") from None


@pytest.mark.parametrize("i", range(32))
def test_random_two_tier_split_matches_oracle(gpu, i, monkeypatch):
    """The fused two-tier launch on random shapes: each row's first k blocks
    (k drawn from 0 to all of them) in an HBM tier in vLLM's layout, the rest in
    a host-layout tier, in HBM or (every third case) in pinned host memory read
    zero-copy, against the oracle over the row's blocks as one list."""
    from vllm_fastdecoder_amd.pinned import pinned_empty

    H, KVH, D, BS, dtype, lens_l, split, out16, _ = _draw(500 + i)
    r = np.random.default_rng(2000 + i)
    n = len(lens_l)
    nbs = [(L + BS - 1) // BS for L in lens_l]
    C = sum(nbs) + 2
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len=max(lens_l),
                                          seed=500 + i)
    lens[:] = torch.tensor(lens_l, dtype=torch.int32)
    perm = torch.randperm(C, generator=torch.Generator().manual_seed(500 + i)).to(torch.int32)
    bt.zero_()
    pos = 0
    for row, nb in enumerate(nbs):
        bt[row, :nb] = perm[pos: pos + nb]
        pos += nb
    W = bt.shape[1]
    bt0 = torch.zeros(n, W, dtype=torch.int32)
    bt1 = torch.zeros(n, W, dtype=torch.int32)
    l0 = torch.zeros(n, dtype=torch.int32)
    l1 = torch.zeros(n, dtype=torch.int32)
    for row, (L, nb) in enumerate(zip(lens_l, nbs)):
        k = int(r.integers(0, nb + 1))
        bt0[row, :k] = bt[row, :k]
        bt1[row, : nb - k] = bt[row, k:nb]
        l0[row] = L if k == nb else k * BS
        l1[row] = L - int(l0[row])
    pinned = i % 3 == 0
    scale = 1.0 / math.sqrt(D)
    monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
    what = (f"case {i}: H={H} KVH={KVH} D={D} BS={BS} {dtype} lens={lens_l} split={split} "
            f"out16={out16} pinned={pinned} l0={l0.tolist()}")
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    if pinned:
        hk = pinned_empty(kc.shape, kc.dtype)
        hv = pinned_empty(vc.shape, vc.dtype)
        hk.copy_(kc)
        hv.copy_(vc)
    else:
        hk, hv = kc.to(gpu), vc.to(gpu)
    out_dtype = dtype if out16 else torch.float32
    out = torch.empty(n, H, D, dtype=out_dtype, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.split_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt0.to(gpu), l0.to(gpu), hk, hv,
                     bt1.to(gpu), l1.to(gpu), scale, out=out, lse=lse)
    torch.cuda.synchronize()
    nz = lens > 0
    try:
        if out16:
            tol = OUT_TOL_16BIT[dtype]
            assert_out_close(out, ref_out, tol, tol, mask=nz)
        else:
            assert_out_close(out, ref_out, 5e-5 if dtype == torch.float32 else 2e-3, mask=nz)
        assert_lse_close(lse, ref_lse, mask=nz)
        assert torch.all(out[~nz.to(gpu)] == 0), "empty rows: out not 0"
        assert torch.all(torch.isneginf(lse[:, ~nz.to(gpu)])), "empty rows: lse not -inf"
    except AssertionError as e:
        raise AssertionError(f"{what}: {e}") from None


@pytest.mark.parametrize("i", range(32))
def test_random_shape_with_token_total_matches_oracle(gpu, i):
    """paged_decode given the rows' token total (the planner's hint for rows
    of uneven length), on random shapes in vLLM's layout: the true total in
    even cases, a wrong one (1 token, or ten times the table) in odd ones. A
    total steers only the task sizes: every case matches the oracle."""
    H, KVH, D, BS, dtype, lens_l, _, out16, _ = _draw(300 + i)
    n = len(lens_l)
    nbs = [(L + BS - 1) // BS for L in lens_l]
    C = sum(nbs) + 2
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len=max(lens_l),
                                          seed=300 + i)
    lens[:] = torch.tensor(lens_l, dtype=torch.int32)
    perm = torch.randperm(C, generator=torch.Generator().manual_seed(300 + i)).to(torch.int32)
    bt.zero_()
    pos = 0
    for r, nb in enumerate(nbs):
        bt[r, :nb] = perm[pos: pos + nb]
        pos += nb
    total = sum(lens_l) if i % 2 == 0 else (1 if i % 4 == 1 else 10 * n * bt.shape[1] * BS)
    scale = 1.0 / math.sqrt(D)
    info = ops.decode_plan_info(n, H, KVH, D, BS, bt.shape[1], dtype, total_tokens=total)
    what = (f"case {i}: H={H} KVH={KVH} D={D} BS={BS} {dtype} lens={lens_l} total={total} "
            f"out16={out16} plan={info}")
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    out_dtype = dtype if out16 else torch.float32
    out = torch.empty(n, H, D, dtype=out_dtype, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.paged_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt.to(gpu), lens.to(gpu), scale,
                     out=out, lse=lse, total_tokens=total)
    torch.cuda.synchronize()
    nz = lens > 0
    try:
        if out16:
            tol = OUT_TOL_16BIT[dtype]
            assert_out_close(out, ref_out, tol, tol, mask=nz)
        else:
            assert_out_close(out, ref_out, 5e-5 if dtype == torch.float32 else 2e-3, mask=nz)
        assert_lse_close(lse, ref_lse, mask=nz)
        assert torch.all(out[~nz.to(gpu)] == 0), "empty rows: out not 0"
        assert torch.all(torch.isneginf(lse[:, ~nz.to(gpu)])), "empty rows: lse not -inf"
    except AssertionError as e:
        raise AssertionError(f"{what}: {e}") from None


def _split_case(name, cus):
    """(n, H, KVH, D, dtype, full rows, hinted, expected split_blocks) of the
    planner's row-splitting rules at 64-block tables of 16 tokens."""
    return {
        # 2.25 full rows per CU, total given: half rows (32 of 64 blocks)
        "half_rows": (cus * 9 // 4, 4, 1, 128, torch.bfloat16, True, True, 32),
        # the same at D = 64, whose rules need all but equal rows
        "half_rows_d64": (cus * 9 // 8, 14, 2, 64, torch.bfloat16, True, True, 32),
        "quarter_rows_d64": (cus * 5 // 8, 14, 2, 64, torch.float16, True, True, 16),
        # 1.06 rows per CU, no total: quarter rows on the matrix-core kernel
        "quarter_rows_mm": (cus + cus // 16, 4, 1, 128, torch.bfloat16, False, False, 16),
        # 1.1 MHA rows per CU: quarter rows on the VALU kernel
        "quarter_rows_valu": (cus // 32 + 1, 32, 32, 128, torch.float16, False, False, 16),
        # one row per CU of mixed length, total given: the slot fill
        "slot_fill": (cus, 4, 1, 128, torch.bfloat16, False, True, 16),
    }[name]


@pytest.mark.parametrize("name", ["half_rows", "half_rows_d64", "quarter_rows_d64",
                                  "quarter_rows_mm", "quarter_rows_valu", "slot_fill"])
def test_row_splitting_plans_match_oracle(gpu, name):
    """The launches whose rows the planner cuts by row count and fill (half
    rows, quarter rows, the slot fill) at the row counts that trigger them on
    this device, run through paged_decode in vLLM's layout, with the plan
    asserted and the output checked against the oracle (fp32 out, 2e-3)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n, H, KVH, D, dtype, full, hinted, want_sb = _split_case(name, cus)
    BS, W = 16, 64
    C = n * W + 2
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len=W * BS, seed=77)
    if full:
        lens[:] = W * BS
    else:
        lens[2:] = torch.randint(1, W * BS + 1, (n - 2,),
                                 generator=torch.Generator().manual_seed(78), dtype=torch.int32)
    perm = torch.randperm(C, generator=torch.Generator().manual_seed(79)).to(torch.int32)
    bt.zero_()
    pos = 0
    for r in range(n):
        nb = (int(lens[r]) + BS - 1) // BS
        bt[r, :nb] = perm[pos: pos + nb]
        pos += nb
    total = int(lens.sum()) if hinted else None
    info = ops.decode_plan_info(n, H, KVH, D, BS, W, dtype, total_tokens=total)
    what = f"{name}: n={n} H={H} KVH={KVH} D={D} {dtype} total={total} plan={info}"
    print(what, flush=True)
    assert info["split_blocks"] == want_sb and info["max_splits"] == W // want_sb, what
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.paged_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt.to(gpu), lens.to(gpu), scale,
                     out=out, lse=lse, total_tokens=total)
    torch.cuda.synchronize()
    try:
        assert_out_close(out, ref_out, 2e-3)
        assert_lse_close(lse, ref_lse)
    except AssertionError as e:
        raise AssertionError(f"{what}: {e}") from None
