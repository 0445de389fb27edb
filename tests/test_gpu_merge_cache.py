"""GPU parity of the LSE merge and the slot-mapping cache write.

Merge: against the float64 oracle merge (rule of cpu_ops.py:93-113), max-abs
2e-3 for fp32 output, the reference's 16-bit tolerances otherwise; merged lse
1e-4 relative. Split + merge against monolithic attention (the core
invariant, tests/test_cpu_kernel.py:99-138) at the same tolerance.
Cache write: bit-exact against the oracle scatter.
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from vllm_fastdecoder_amd import ops
from vllm_fastdecoder_amd.pinned import pinned_zeros

pytestmark = pytest.mark.gpu


def _partials(n, H, D, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    o_a = torch.randn(n, H, D, generator=g).to(dtype)
    o_b = torch.randn(n, H, D, generator=g).to(dtype)
    lse_a = torch.randn(H, n, generator=g) * 3
    lse_b = torch.randn(H, n, generator=g) * 3
    # conventions: +inf and -inf mean "empty"; both empty in column 0
    if n >= 4:
        lse_a[:, 0] = float("-inf")
        lse_b[:, 0] = float("inf")
        lse_a[:, 1] = float("inf")   # FA's empty: take b alone
        lse_b[:, 2] = float("-inf")  # take a alone
        lse_a[0, 3] = 80.0           # large gap
    return o_a.to(dev), lse_a.to(dev), o_b.to(dev), lse_b.to(dev)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("D", [128, 64, 72, 5])
def test_merge_matches_oracle(gpu, dtype, D):
    n, H = 9, 8
    o_a, lse_a, o_b, lse_b = _partials(n, H, D, dtype, D, gpu)
    ref, ref_lse = oracle.merge_f64(o_a, lse_a, o_b, lse_b)
    for out_dtype in (dtype, torch.float32):
        out = torch.full((n, H, D), float("nan"), dtype=out_dtype, device=gpu)
        olse = torch.empty(H, n, dtype=torch.float32, device=gpu)
        ops.merge_attn_states(out, o_a, lse_a, o_b, lse_b, out_lse=olse)
        torch.cuda.synchronize()
        tol = 2e-3 if out_dtype == torch.float32 else {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}[dtype]
        err = (out.double().cpu() - ref).abs() - (0 if out_dtype == torch.float32 else tol) * ref.abs()
        assert float(err.max()) <= tol
        assert torch.all(out[0] == 0)  # both empty -> 0 (cpu_ops.py:104-110)
        fin = torch.isfinite(ref_lse)
        assert torch.isneginf(olse[:, 0]).all()
        lerr = (olse.double().cpu()[fin] - ref_lse[fin]).abs() / ref_lse[fin].abs().clamp(min=1)
        assert float(lerr.max()) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.float32])
def test_merge_reads_a_pinned_host_partial(gpu, dtype):
    """o_b / lse_b in pinned host memory (the host cores' partial of the hybrid
    split, read zero-copy over the link): the same bits as from HBM; pageable
    host memory is refused."""
    n, H, D = 9, 8, 128
    o_a, lse_a, o_b, lse_b = _partials(n, H, D, dtype, D, gpu)
    out_dev = torch.empty(n, H, D, dtype=dtype, device=gpu)
    lse_dev = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.merge_attn_states(out_dev, o_a, lse_a, o_b, lse_b, out_lse=lse_dev)
    o_h = torch.empty(o_b.shape, dtype=o_b.dtype, pin_memory=True)
    l_h = torch.empty(lse_b.shape, dtype=torch.float32, pin_memory=True)
    o_h.copy_(o_b)
    l_h.copy_(lse_b)
    out = torch.full_like(out_dev, float("nan"))
    olse = torch.empty_like(lse_dev)
    ops.merge_attn_states(out, o_a, lse_a, o_h, l_h, out_lse=olse)
    torch.cuda.synchronize()
    assert torch.equal(out.cpu(), out_dev.cpu()) and torch.equal(olse.cpu(), lse_dev.cpu())
    with pytest.raises(RuntimeError, match="pinned memory"):
        ops.merge_attn_states(out, o_a, lse_a, o_b.cpu(), lse_b.cpu())


def test_merge_fa_empty_convention(gpu):
    """+inf LSE is empty: merge returns the other partial (test_cpu_kernel.py:141-147)."""
    o_a = torch.zeros(3, 2, 8, device=gpu)
    lse_a = torch.full((2, 3), float("inf"), device=gpu)
    o_b = torch.randn(3, 2, 8, device=gpu)
    lse_b = torch.randn(2, 3, device=gpu)
    out = torch.empty_like(o_b)
    ops.merge_attn_states(out, o_a, lse_a, o_b, lse_b)
    torch.cuda.synchronize()
    torch.testing.assert_close(out, o_b)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
@pytest.mark.parametrize("H,KVH", [(32, 32), (8, 2)])
def test_split_tiers_merge_equals_monolithic(gpu, dtype, H, KVH):
    """GPU/host split of the correctness workload (ids < G=512 are the HBM tier,
    >= G the host tier read zero-copy from pinned memory): each row's first k
    blocks (k ~ U[0, nb]) from the GPU tier and the rest from the host tier.
    Merged partials must equal monolithic attention over all blocks."""
    D, BS, n, G, C = 128, 16, 8, 512, 512
    g = torch.Generator().manual_seed(1)
    lens = torch.randint(128, 1025, (n,), generator=g, dtype=torch.int32)
    nb = (lens + BS - 1) // BS
    k_split = torch.stack([torch.randint(0, int(x) + 1, (1,), generator=g)[0] for x in nb])
    k_split[0] = 0           # GPU partial empty
    k_split[1] = nb[1]       # host partial empty
    W = int(nb.max())
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
        for j in range(nbi):
            ntok = BS if j < nbi - 1 else last
            if j < k:
                bid = int(gpu_perm[pg % G]); pg += 1
                bt_g[i, j] = bid
                full_bt[i, j] = bid
                len_g[i] += ntok
            else:
                bid = int(host_perm[pc % C]); pc += 1
                bt_c[i, j - k] = bid
                full_bt[i, j] = G + bid
                len_c[i] += ntok
    # the GPU tier in vLLM's layout, the host tier pinned in the host layout
    kv = torch.empty(G, BS, KVH, 2 * D, dtype=dtype)
    kv[..., :D] = pool_k[:G].transpose(1, 2)
    kv[..., D:] = pool_v[:G].transpose(1, 2)
    kv = kv.to(gpu)
    hk = pinned_zeros((C, KVH, BS, D), dtype)
    hv = pinned_zeros((C, KVH, BS, D), dtype)
    hk.copy_(pool_k[G:])
    hv.copy_(pool_v[G:])
    qd = q.to(gpu)
    scale = 1 / math.sqrt(D)
    o_g, l_g = ops.paged_decode(qd, kv[..., :D], kv[..., D:], bt_g.to(gpu), len_g.to(gpu), scale)
    o_c = torch.empty_like(qd)
    l_c = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.decode_attn(qd, hk, hv, bt_c.to(gpu), len_c.to(gpu), scale, o_c, l_c)
    merged = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    mlse = torch.empty(H, n, dtype=torch.float32, device=gpu)
    ops.merge_attn_states(merged, o_g, l_g, o_c, l_c, out_lse=mlse)
    # fp32 partials: the merged output then meets the fp32 bar
    o_g32 = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    ops.paged_decode(qd, kv[..., :D], kv[..., D:], bt_g.to(gpu), len_g.to(gpu), scale, out=o_g32, lse=l_g)
    o_c32 = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
    ops.decode_attn(qd, hk, hv, bt_c.to(gpu), len_c.to(gpu), scale, o_c32, l_c)
    merged32 = torch.empty_like(merged)
    ops.merge_attn_states(merged32, o_g32, l_g, o_c32, l_c)
    torch.cuda.synchronize()
    ref, ref_lse = oracle.decode_attn_host_layout_f64(q, pool_k, pool_v, full_bt, lens, scale)
    tol16 = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2}[dtype]
    assert float(((merged.double().cpu() - ref).abs() - tol16 * ref.abs()).max()) <= tol16
    assert float((merged32.double().cpu() - ref).abs().max()) <= 2e-3
    assert float(((mlse.double().cpu() - ref_lse).abs() / ref_lse.abs().clamp(min=1)).max()) <= 1e-4


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_reshape_and_cache_bit_exact(gpu, dtype):
    """vLLM-layout write of strided (fused-qkv) rows with padding slots -1 and
    one slot past the cache (skipped and counted)."""
    B, BS, KVH, D, H = 12, 16, 4, 128, 8
    T = 37
    g = torch.Generator().manual_seed(3)
    qkv = torch.randn(T, (H + 2 * KVH) * D, generator=g).to(dtype)
    _, key, value = qkv.split([H * D, KVH * D, KVH * D], dim=-1)
    key = key.view(T, KVH, D)
    value = value.view(T, KVH, D)
    slots = torch.randperm(B * BS, generator=g)[:T].to(torch.int64)
    slots[5] = -1
    slots[9] = -1
    slots[11] = B * BS + 3
    kv = torch.randn(B, BS, KVH, 2 * D, generator=g).to(dtype)  # garbage-filled
    kv_ref = kv.clone()
    st, oor = oracle.cache_write(key, value, kv_ref[..., :D], kv_ref[..., D:],
                                 (kv_ref.stride(0), kv_ref.stride(1), kv_ref.stride(2)),
                                 B, BS, slots, check_all=False)
    assert st == 0 and oor == 1
    kvd = kv.to(gpu)
    err = torch.zeros(1, dtype=torch.int32, device=gpu)
    ops.reshape_and_cache(key.to(gpu), value.to(gpu), kvd[..., :D], kvd[..., D:], slots.to(gpu),
                          "auto", None, None, error_count=err)
    torch.cuda.synchronize()
    assert torch.equal(kvd.cpu(), kv_ref)
    assert int(err.item()) == 1


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_store_kv_host_tier_bit_exact(gpu, dtype):
    """Host-tier write into pinned memory (test_cpu_kernel.py:75-88 shapes)."""
    C, KVH, BS, D, m = 10, 4, 16, 128, 37
    g = torch.Generator().manual_seed(1)
    k = torch.randn(m, KVH, D, generator=g).to(dtype)
    v = torch.randn(m, KVH, D, generator=g).to(dtype)
    slots = torch.randperm(C * BS, generator=g)[:m].to(torch.int64)
    kc = pinned_zeros((C, KVH, BS, D), dtype)
    vc = pinned_zeros((C, KVH, BS, D), dtype)
    kc_ref = torch.zeros(C, KVH, BS, D, dtype=dtype)
    vc_ref = torch.zeros_like(kc_ref)
    st, _ = oracle.cache_write(k, v, kc_ref, vc_ref, (kc_ref.stride(0), kc_ref.stride(2), kc_ref.stride(1)),
                               C, BS, slots, check_all=True)
    assert st == 0
    ops.store_kv(k.to(gpu), v.to(gpu), slots, kc, vc)
    torch.cuda.synchronize()
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref)
    # the reference's own kernel agrees (when its build is present)
    ext = oracle.ref_ext()
    if ext is not None:
        kc2 = torch.zeros_like(kc_ref)
        vc2 = torch.zeros_like(vc_ref)
        ext.store_kv(k, v, slots, kc2, vc2)
        assert torch.equal(kc2, kc_ref) and torch.equal(vc2, vc_ref)


def test_store_kv_rejects_out_of_range(gpu):
    """Any slot past the tier -> RuntimeError and nothing written
    (test_cpu_kernel.py:91-96, cpu_attn.cpp:506-510)."""
    kc = pinned_zeros((2, 1, 16, 64), torch.float16)
    vc = pinned_zeros((2, 1, 16, 64), torch.float16)
    k = torch.ones(2, 1, 64, dtype=torch.float16, device=gpu)
    for slots in (torch.tensor([3, 32], dtype=torch.int64), torch.tensor([3, 32], dtype=torch.int64, device=gpu)):
        with pytest.raises(RuntimeError):
            ops.store_kv(k, k, slots, kc, vc)
    torch.cuda.synchronize()
    assert torch.all(kc == 0) and torch.all(vc == 0)


def test_ensure_store_rebuilds_when_the_geometry_changes(gpu, monkeypatch):
    """ensure_store (state.py:32-90) returns the existing host tier for the
    same geometry and builds a new one, of the new shape and dtype, when any
    of it changes."""
    from vllm_fastdecoder_amd import state

    monkeypatch.setattr(state, "STORE", None)
    names = ["l0", "l1"]
    s1 = state.ensure_host_store(8, 4, 16, 2, 64, torch.float16, names)
    assert state.ensure_host_store(8, 4, 16, 2, 64, torch.float16, names) is s1
    for args, shape, dtype in (((8, 4, 32, 2, 64, torch.float16), (4, 2, 32, 64), torch.float16),
                               ((8, 4, 16, 2, 64, torch.bfloat16), (4, 2, 16, 64), torch.bfloat16),
                               ((8, 4, 16, 2, 128, torch.float16), (4, 2, 16, 128), torch.float16)):
        s = state.ensure_host_store(*args, names)
        assert s is not s1 and s.k["l1"].shape == shape and s.v["l0"].dtype == dtype
        assert int(s.k["l0"].abs().sum()) == 0
        s1 = s
    assert state.ensure_host_store(8, 0, 16, 2, 64, torch.float16, names) is None
