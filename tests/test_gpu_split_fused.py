"""GPU parity of the fused split decode (fd_split_decode / ops.split_decode):
both tiers of a row in one launch against

  * the float64 oracle: monolithic attention over all of the row's blocks
    when only the row's last block is partial (the GPU-first allocation of
    the reference), else the float64 merge of the two tiers' float64 partials;
  * the reference's own contract on the same inputs: HBM-tier partial +
    host-tier partial + merge_attn_states (fastdecode/backend.py:293-356),
    here run with this library's kernels.

Bars: fp32 out max-abs <= 2e-3 and lse <= 1e-4 relative against the oracle;
16-bit out the reference's own 16-bit tolerances (fp16 2e-3, bf16 1.6e-2);
fused vs two-partials-and-merge within 2e-5 (fp32 summation order only);
empty rows exactly 0 / -inf; a bad table entry or length turns only its row
into NaN.
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from vllm_fastdecoder_amd import ops
from vllm_fastdecoder_amd.pinned import pinned_zeros

pytestmark = pytest.mark.gpu

TOL16 = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}


def two_tier_case(n, H, KVH, D, dtype, seed, dev, G=512, C=512, lo=128, hi=1024,
                  gpu_first=True, special=True, BS=16):
    """Rows of lens ~ U[lo, hi]; row i's first k_i blocks (k_i ~ U[0, nb_i])
    come from the HBM tier (ids < G), the rest from the pinned host tier.
    gpu_first=False interleaves the tiers and then gives each tier's last
    block a random token count, so both tiers of a row end in a partial block
    (the fused entry allows it; only the per-tier oracle covers it). special:
    row 0 all on the host, row 1 all in HBM, row 2 empty. BS: tokens per
    cache block."""
    g = torch.Generator().manual_seed(seed)
    lens = torch.randint(lo, hi + 1, (n,), generator=g, dtype=torch.int32)
    if special:
        lens[2] = 0
    nb = (lens + BS - 1) // BS
    k_split = torch.stack([torch.randint(0, int(x) + 1, (1,), generator=g)[0] for x in nb])
    if special:
        k_split[0] = 0
        k_split[1] = nb[1]
    W = max(1, int(nb.max()))
    gpu_perm = torch.randperm(G, generator=g)
    host_perm = torch.randperm(C, generator=g)
    q = torch.randn(n, H, D, generator=g).to(dtype)
    pool_k = torch.randn(G + C, KVH, BS, D, generator=g).to(dtype)  # unified ids [0, G+C)
    pool_v = torch.randn(G + C, KVH, BS, D, generator=g).to(dtype)
    full_bt = torch.zeros(n, W, dtype=torch.int32)
    bt_g = torch.zeros(n, W, dtype=torch.int32)
    bt_c = torch.zeros(n, W, dtype=torch.int32)
    len_g = torch.zeros(n, dtype=torch.int32)
    len_c = torch.zeros(n, dtype=torch.int32)
    pg = pc = 0
    for i in range(n):
        L, nbi, k = int(lens[i]), int(nb[i]), int(k_split[i])
        last = L - (nbi - 1) * BS
        ng = nc = 0
        for j in range(nbi):
            on_gpu = j < k if gpu_first else (j % 2 == 0 and ng < k) or nc >= nbi - k
            ntok = BS if j < nbi - 1 else last
            if on_gpu:
                bid = int(gpu_perm[pg % G]); pg += 1
                bt_g[i, ng] = bid
                ng += 1
                full_bt[i, j] = bid
                len_g[i] += ntok
            else:
                bid = int(host_perm[pc % C]); pc += 1
                bt_c[i, nc] = bid
                nc += 1
                full_bt[i, j] = G + bid
                len_c[i] += ntok
        if not gpu_first:
            for cnt, ln in ((ng, len_g), (nc, len_c)):
                if cnt:
                    ln[i] = BS * (cnt - 1) + int(torch.randint(1, BS + 1, (1,), generator=g))
    kv = torch.empty(G, BS, KVH, 2 * D, dtype=dtype)
    kv[..., :D] = pool_k[:G].transpose(1, 2)
    kv[..., D:] = pool_v[:G].transpose(1, 2)
    kv = kv.to(dev)
    hk = pinned_zeros((C, KVH, BS, D), dtype)
    hv = pinned_zeros((C, KVH, BS, D), dtype)
    hk.copy_(pool_k[G:])
    hv.copy_(pool_v[G:])
    return dict(q=q, lens=lens, full_bt=full_bt, pool_k=pool_k, pool_v=pool_v, kv=kv, hk=hk,
                hv=hv, bt_g=bt_g, bt_c=bt_c, len_g=len_g, len_c=len_c, G=G, scale=1 / math.sqrt(D))


def run_fused(c, dev, out_dtype=torch.float32, row_order=None, tiers=None):
    t = tiers or c
    q = c["q"].to(dev)
    n, H, D = q.shape
    out = torch.empty(n, H, D, dtype=out_dtype, device=dev)
    lse = torch.empty(H, n, dtype=torch.float32, device=dev)
    ops.split_decode(q, c["kv"][..., :D], c["kv"][..., D:], t["bt_g"].to(dev), t["len_g"].to(dev),
                     c["hk"], c["hv"], t["bt_c"].to(dev), t["len_c"].to(dev), c["scale"],
                     out=out, lse=lse, row_order=row_order)
    torch.cuda.synchronize()
    return out, lse


def run_two_partials(c, dev):
    q = c["q"].to(dev)
    n, H, D = q.shape
    o_g = torch.empty(n, H, D, dtype=torch.float32, device=dev)
    l_g = torch.empty(H, n, dtype=torch.float32, device=dev)
    ops.paged_decode(q, c["kv"][..., :D], c["kv"][..., D:], c["bt_g"].to(dev), c["len_g"].to(dev),
                     c["scale"], out=o_g, lse=l_g)
    o_c = torch.empty_like(o_g)
    l_c = torch.empty_like(l_g)
    ops.decode_attn(q, c["hk"], c["hv"], c["bt_c"].to(dev), c["len_c"].to(dev), c["scale"], o_c, l_c)
    merged = torch.empty_like(o_g)
    mlse = torch.empty_like(l_g)
    ops.merge_attn_states(merged, o_g, l_g, o_c, l_c, out_lse=mlse)
    torch.cuda.synchronize()
    return merged, mlse


def oracle_merged(c):
    """float64 merge of the two tiers' float64 partials (any block layout)."""
    D = c["q"].shape[2]
    kv = c["kv"].cpu()
    og, lg, st = oracle.decode_attn_f64(c["q"], kv[..., :D], kv[..., D:], oracle.VLLM_DIMS,
                                        c["bt_g"], c["len_g"], c["scale"])
    assert st == 0
    oc, lc = oracle.decode_attn_host_layout_f64(c["q"], c["hk"], c["hv"], c["bt_c"], c["len_c"],
                                                c["scale"])
    return oracle.merge_f64(og, lg, oc, lc)


def check_vs_oracle(out, lse, ref, ref_lse, nonempty):
    err = float((out.double().cpu()[nonempty] - ref[nonempty]).abs().max())
    assert err <= 2e-3, f"out err {err:.3g}"
    lerr = (lse.double().cpu()[:, nonempty] - ref_lse[:, nonempty]).abs()
    rel = float((lerr / ref_lse[:, nonempty].abs().clamp(min=1.0)).max())
    assert rel <= 1e-4, f"lse rel err {rel:.3g}"


@pytest.mark.parametrize("kernel", ["default", "valu"])
@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H,KVH", [(32, 32), (32, 8), (16, 2), (64, 8)])
def test_fused_equals_monolithic_and_two_partials(gpu, kernel, dtype, H, KVH, monkeypatch):
    """GPU-first rows (config "GPU/host split + LSE merge" of the correctness
    shape, G = 512): fused == monolithic attention over all blocks ==
    two partials + merge."""
    if kernel == "valu":
        monkeypatch.setenv("FD_DECODE_KERNEL", "valu")
    c = two_tier_case(8, H, KVH, 128, dtype, seed=H + KVH, dev=gpu)
    out, lse = run_fused(c, gpu)
    ref, ref_lse = oracle.decode_attn_host_layout_f64(c["q"], c["pool_k"], c["pool_v"],
                                                      c["full_bt"], c["lens"], c["scale"])
    nz = c["lens"] > 0
    check_vs_oracle(out, lse, ref, ref_lse, nz)
    # the HBM tier's K + V loads (V after K in vLLM's cache) against separate
    # K and V loads: bit-identical
    monkeypatch.setenv("FD_KV_ADJ", "0")
    out_sep, lse_sep = run_fused(c, gpu)
    monkeypatch.delenv("FD_KV_ADJ")
    assert torch.equal(out, out_sep) and torch.equal(lse, lse_sep)
    assert torch.all(out[~nz.to(gpu)] == 0) and torch.all(torch.isneginf(lse[:, ~nz.to(gpu)]))
    merged, mlse = run_two_partials(c, gpu)
    assert float((out - merged)[nz.to(gpu)].abs().max()) <= 2e-5
    assert float((lse - mlse)[:, nz.to(gpu)].abs().max()) <= 2e-5 * float(mlse[:, nz.to(gpu)].abs().max())
    out16, lse16 = run_fused(c, gpu, out_dtype=dtype)
    tol = TOL16[dtype]
    err16 = ((out16.double().cpu() - ref).abs() - tol * ref.abs())[nz]
    assert float(err16.max()) <= tol
    assert torch.equal(lse16, lse)


@pytest.mark.parametrize("D", [64, 256])
@pytest.mark.parametrize("H,KVH", [(8, 8), (16, 2), (32, 4)])
def test_fused_head_sizes_and_interleaved_tiers(gpu, D, H, KVH):
    """Tiers interleaved within a row, so each tier may end in a partial
    block; checked against the float64 merge of float64 per-tier partials."""
    c = two_tier_case(8, H, KVH, D, torch.bfloat16, seed=D + H, dev=gpu, lo=1, hi=700,
                      gpu_first=False)
    out, lse = run_fused(c, gpu)
    ref, ref_lse = oracle_merged(c)
    nz = c["lens"] > 0
    check_vs_oracle(out, lse, ref, ref_lse, nz)


@pytest.mark.parametrize("split", ["1", "2", "5", "64"])
def test_fused_split_tasks_and_row_order(gpu, split, monkeypatch):
    """Rows split into tasks across the tier boundary (forced split sizes),
    any row order: same result within the fp32 bar and bit-identical across
    orders."""
    monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
    c = two_tier_case(12, 16, 4, 128, torch.float16, seed=7, dev=gpu, gpu_first=False, lo=1)
    ref, ref_lse = oracle_merged(c)
    nz = c["lens"] > 0
    res = []
    for order in (None, ops.longest_first(c["len_g"] + c["len_c"]),
                  torch.randperm(12, generator=torch.Generator().manual_seed(3)).to(torch.int32)):
        out, lse = run_fused(c, gpu, row_order=order)
        check_vs_oracle(out, lse, ref, ref_lse, nz)
        res.append((out, lse))
    for out, lse in res[1:]:
        assert torch.equal(out, res[0][0]) and torch.equal(lse, res[0][1])


def test_fused_generic_kernel(gpu):
    """Head size 72 (no tiled kernel) and fp32 KV: the generic kernel's two-tier
    walk against the oracle."""
    for D, dtype in ((72, torch.float16), (64, torch.float32)):
        c = two_tier_case(6, 8, 2, D, dtype, seed=D, dev=gpu, lo=1, hi=300, gpu_first=False)
        out, lse = run_fused(c, gpu)
        ref, ref_lse = oracle_merged(c)
        nz = c["lens"] > 0
        tol = 2e-3 if dtype != torch.float32 else 1e-5
        assert float((out.double().cpu()[nz] - ref[nz]).abs().max()) <= tol
        rel = ((lse.double().cpu() - ref_lse).abs() / ref_lse.abs().clamp(min=1.0))[:, nz]
        assert float(rel.max()) <= 1e-4


def test_fused_range_errors_poison_only_their_rows(gpu):
    """A host-tier table entry past the host cache, or a host length beyond the
    host table, turns that row into NaN; the other rows are unaffected."""
    c = two_tier_case(6, 16, 4, 128, torch.float16, seed=11, dev=gpu, special=False)
    ref, ref_lse = oracle_merged(c)
    bad = dict(c)
    bt_c = c["bt_c"].clone()
    len_c = c["len_c"].clone()
    rows = [i for i in range(6) if int(c["len_c"][i]) > 0]
    r1, r2 = rows[0], rows[1]
    bt_c[r1, 0] = c["hk"].shape[0] + 3
    len_c[r2] = bt_c.shape[1] * 16 + 1
    bad.update(bt_c=bt_c, len_c=len_c)
    out, lse = run_fused(c, gpu, tiers=bad)
    for r in (r1, r2):
        assert torch.isnan(out[r]).all() and torch.isnan(lse[:, r]).all()
    ok = torch.ones(6, dtype=torch.bool)
    ok[r1] = ok[r2] = False
    check_vs_oracle(out, lse, ref, ref_lse, ok)


def test_fused_with_a_zero_width_tier(gpu):
    """Every row in one tier: the other tier's table has no columns (and its
    lengths are 0). The fused launch equals the oracle of the tier that holds
    the rows; a row given tokens in the empty tier is a range error (NaN)."""
    for hbm_only in (True, False):
        c = two_tier_case(5, 16, 4, 64, torch.float16, seed=12 + hbm_only, dev=gpu,
                          special=False)
        n = c["q"].shape[0]
        t = dict(c)
        if hbm_only:  # whole-block HBM rows: give each its host blocks' count in HBM ids
            t["len_g"] = ((c["len_g"] + 15) // 16 * 16).to(torch.int32)
            t["len_c"] = torch.zeros(n, dtype=torch.int32)
            t["bt_c"] = torch.zeros(n, 0, dtype=torch.int32)
        else:
            t["len_g"] = torch.zeros(n, dtype=torch.int32)
            t["bt_g"] = torch.zeros(n, 0, dtype=torch.int32)
        out, lse = run_fused(c, gpu, tiers=t)
        ref, ref_lse = oracle_merged(dict(c, **{k: t[k] for k in ("len_g", "len_c")},
                                          bt_g=t["bt_g"] if t["bt_g"].shape[1] else
                                          torch.zeros(n, 1, dtype=torch.int32),
                                          bt_c=t["bt_c"] if t["bt_c"].shape[1] else
                                          torch.zeros(n, 1, dtype=torch.int32)))
        nz = (t["len_g"] + t["len_c"]) > 0
        check_vs_oracle(out, lse, ref, ref_lse, nz)
        assert torch.all(out.cpu()[~nz] == 0) and torch.all(torch.isneginf(lse.cpu()[:, ~nz]))
        bad = dict(t)
        key = "len_c" if hbm_only else "len_g"
        bad[key] = t[key].clone()
        bad[key][1] = 3
        out, lse = run_fused(c, gpu, tiers=bad)
        assert torch.isnan(out[1]).all() and torch.isnan(lse[:, 1]).all()


def test_fused_rejects_mismatched_tiers(gpu):
    c = two_tier_case(2, 8, 8, 64, torch.float16, seed=1, dev=gpu, hi=200, special=False)
    q = c["q"].to(gpu)
    with pytest.raises(RuntimeError):
        ops.split_decode(q, c["kv"][..., :64], c["kv"][..., 64:], c["bt_g"].to(gpu),
                         c["len_g"].to(gpu), c["hk"][:, :4], c["hv"][:, :4], c["bt_c"].to(gpu),
                         c["len_c"].to(gpu), 0.1)  # host tier with 4 kv heads, HBM with 8


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fused_second_tier_in_hbm(gpu, dtype):
    """Both tiers in device memory: the grouped-query launch stays on the
    matrix-core kernel (a launch that reads pinned host memory takes the VALU
    kernel instead); same oracle bars."""
    c = two_tier_case(8, 32, 8, 128, dtype, seed=31, dev=gpu)
    dev_tiers = dict(c, hk=c["hk"].to(gpu), hv=c["hv"].to(gpu))
    out, lse = run_fused(dev_tiers, gpu)
    ref, ref_lse = oracle.decode_attn_host_layout_f64(c["q"], c["pool_k"], c["pool_v"],
                                                      c["full_bt"], c["lens"], c["scale"])
    nz = c["lens"] > 0
    check_vs_oracle(out, lse, ref, ref_lse, nz)
    out_h, lse_h = run_fused(c, gpu)  # the same step reading the pinned host tier
    assert float((out - out_h)[nz.to(gpu)].abs().max()) <= 2e-5


@pytest.mark.parametrize("kernel", ["default", "valu"])
@pytest.mark.parametrize("H,KVH,dtype", [(32, 32, torch.float16), (32, 8, torch.bfloat16)])
def test_fused_long_rows(gpu, kernel, H, KVH, dtype, monkeypatch):
    """Rows of 6k-9k tokens (375-563 blocks, past one 256-block task) with
    their blocks divided at random between the tiers: the launch model's
    splits cross the tier boundary and the combine kernel merges them."""
    if kernel == "valu":
        monkeypatch.setenv("FD_DECODE_KERNEL", "valu")
    c = two_tier_case(5, H, KVH, 128, dtype, seed=H + KVH + 1, dev=gpu, G=2000, C=2600,
                      lo=6000, hi=9000)
    out, lse = run_fused(c, gpu)
    ref, ref_lse = oracle_merged(c)
    nz = c["lens"] > 0
    check_vs_oracle(out, lse, ref, ref_lse, nz)
    assert torch.all(out[~nz.to(gpu)] == 0) and torch.all(torch.isneginf(lse[:, ~nz.to(gpu)]))


@pytest.mark.parametrize("kernel", ["default", "valu"])
@pytest.mark.parametrize("H,KVH", [(32, 2), (40, 8), (28, 4)])
def test_fused_any_head_group(gpu, kernel, H, KVH, monkeypatch):
    """Fused two-tier launch with 16 (passes of 8), 5 and 7 (8-slot kernel)
    query heads per kv head; the host tier lies in pinned memory, so the
    default is the VALU kernel too (the matrix-core kernels' two-tier form is
    covered by tests/test_gpu_decode_mm.py with both tiers in HBM)."""
    if kernel == "valu":
        monkeypatch.setenv("FD_DECODE_KERNEL", "valu")
    c = two_tier_case(9, H, KVH, 128, torch.bfloat16, seed=61 + H, dev=gpu)
    out, lse = run_fused(c, gpu)
    ref, ref_lse = oracle_merged(c)
    nz = c["lens"] > 0
    check_vs_oracle(out, lse, ref, ref_lse, nz)
    assert torch.all(out[~nz.to(gpu)] == 0) and torch.all(torch.isneginf(lse[:, ~nz.to(gpu)]))


@pytest.mark.parametrize("D", [80, 96])
def test_fused_head_sizes_between_kernels(gpu, D):
    """Fused two-tier launch at head sizes run in the next larger kernel."""
    c = two_tier_case(9, 16, 4, D, torch.float16, seed=D, dev=gpu)
    out, lse = run_fused(c, gpu)
    ref, ref_lse = oracle_merged(c)
    nz = c["lens"] > 0
    check_vs_oracle(out, lse, ref, ref_lse, nz)
    assert torch.all(out[~nz.to(gpu)] == 0) and torch.all(torch.isneginf(lse[:, ~nz.to(gpu)]))


@pytest.mark.parametrize("BS", [32, 64])
@pytest.mark.parametrize("H,KVH,dtype", [(32, 32, torch.float16), (32, 8, torch.bfloat16)])
def test_fused_larger_cache_blocks(gpu, BS, H, KVH, dtype):
    """Cache blocks of 32 and 64 tokens (2 and 4 tiles of 16 to the kernels),
    tiers interleaved so both end in partial blocks."""
    c = two_tier_case(9, H, KVH, 128, dtype, seed=BS + H, dev=gpu, BS=BS, G=256, C=256,
                      gpu_first=False)
    out, lse = run_fused(c, gpu)
    ref, ref_lse = oracle_merged(c)
    nz = c["lens"] > 0
    check_vs_oracle(out, lse, ref, ref_lse, nz)
