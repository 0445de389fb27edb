"""The reference's CPU-extension surface on the host-core kernels
(vllm_fastdecoder_amd.host_ext), checked the way the reference checks its
own extension (tests/test_cpu_kernel.py) plus its golden outputs. CPU only.

  * decode_attn on the reference's kernel grid and large scores against the
    float64 oracle (fp16 2e-3, bf16 1.6e-2 atol and rtol; fp32 1e-4), and
    against the golden outputs of the reference's own build
    (tests/golden/ref_decode_attn.npz);
  * store_kv bit-exact against the oracle's slot write, and rejecting an
    out-of-range slot before writing anything;
  * the thread controls and has_avx2;
  * split + merge of two host-core partials == attention over all blocks.
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest
import torch

import oracle
from tests import cases
from vllm_fastdecoder_amd import host_ext

GOLDEN = Path(__file__).resolve().parent / "golden"
TOL = {torch.float16: 2e-3, torch.bfloat16: 1.6e-2, torch.float32: 1e-4}


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
@pytest.mark.parametrize("H,KVH", [(8, 8), (8, 2), (4, 1)])
@pytest.mark.parametrize("D", [64, 128, 72])
def test_decode_attn_matches_oracle(dtype, H, KVH, D):
    """tests/test_cpu_kernel.py:38-57: out in q's dtype, as the reference
    requires."""
    ext = host_ext.load_ext()
    n, BS, C = 7, 16, 64
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len=93, seed=D + H)
    lens[3] = 0
    scale = 1.0 / math.sqrt(D)
    out = torch.empty_like(q)
    lse = torch.empty(H, n, dtype=torch.float32)
    ext.decode_attn(q, kc, vc, bt, lens, scale, out, lse)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    nz = lens > 0
    tol = TOL[dtype]
    torch.testing.assert_close(out.double()[nz], ref_out[nz], atol=tol, rtol=tol)
    torch.testing.assert_close(lse.double()[:, nz], ref_lse[:, nz], atol=1e-4, rtol=1e-5)
    assert torch.all(out[~nz] == 0) and torch.all(torch.isneginf(lse[:, ~nz]))


def test_decode_attn_large_scores():
    """tests/test_cpu_kernel.py:60-72."""
    ext = host_ext.load_ext()
    n, H, KVH, D, BS, C = 2, 4, 4, 64, 16, 8
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, torch.float32, 40, 0)
    q = q * 300.0
    out = torch.empty_like(q)
    lse = torch.empty(H, n, dtype=torch.float32)
    ext.decode_attn(q, kc, vc, bt, lens, 1.0, out, lse)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, 1.0)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    torch.testing.assert_close(out.double(), ref_out, atol=1e-4, rtol=1e-4)
    torch.testing.assert_close(lse.double(), ref_lse, atol=1e-3, rtol=1e-6)


def test_decode_attn_matches_reference_build_golden_outputs():
    """The golden outputs of the reference's own cpu_attn.cpp build on its
    test grid (inputs regenerated from the same seeds; the digest guards the
    generator)."""
    data = np.load(GOLDEN / "ref_decode_attn.npz")
    names = sorted({k.split("__")[0] for k in data.files})
    assert names
    for name in names:
        meta = data[f"{name}__meta"]
        n, H, KVH, D, BS, C, max_len, seed, dt_code, empty_row = (int(x) for x in meta)
        dtype = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32}[dt_code]
        q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, dtype, max_len, seed)
        if empty_row >= 0:
            lens[empty_row] = 0
        assert cases.tensor_digest(q, kc, vc, bt, lens) == str(data[f"{name}__digest"])
        out = torch.empty_like(q)
        lse = torch.empty(H, n, dtype=torch.float32)
        host_ext.decode_attn(q, kc, vc, bt, lens, 1.0 / math.sqrt(D), out, lse)
        g_out = torch.from_numpy(data[f"{name}__out"]).double()
        g_lse = torch.from_numpy(data[f"{name}__lse"]).double()
        nz = lens > 0
        # two fp32 kernels, each within the 16-bit bar of float64: twice the bar
        tol = 2 * TOL[dtype]
        torch.testing.assert_close(out.double()[nz], g_out[nz], atol=tol, rtol=tol)
        torch.testing.assert_close(lse.double()[:, nz], g_lse[:, nz], atol=2e-4, rtol=1e-5)


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16, torch.float32])
def test_store_kv_matches_oracle(dtype):
    """tests/test_cpu_kernel.py:75-88, bit-exact."""
    ext = host_ext.load_ext()
    C, KVH, BS, D, m = 10, 4, 16, 128, 37
    g = torch.Generator().manual_seed(1)
    kc = torch.zeros(C, KVH, BS, D, dtype=dtype)
    vc = torch.zeros_like(kc)
    kc_ref, vc_ref = kc.clone(), vc.clone()
    k = torch.randn(m, KVH, D, generator=g).to(dtype)
    v = torch.randn(m, KVH, D, generator=g).to(dtype)
    slots = torch.randperm(C * BS, generator=g)[:m].to(torch.int64)
    ext.store_kv(k, v, slots, kc, vc)
    st, _ = oracle.cache_write(k, v, kc_ref, vc_ref, (kc_ref.stride(0), kc_ref.stride(2),
                                                      kc_ref.stride(1)), C, BS, slots, True)
    assert st == 0
    assert torch.equal(kc, kc_ref) and torch.equal(vc, vc_ref)


def test_store_kv_rejects_out_of_range_before_writing():
    """tests/test_cpu_kernel.py:91-96; and nothing is written when any slot
    is bad (cpu_attn.cpp:506-510)."""
    ext = host_ext.load_ext()
    kc = torch.zeros(2, 1, 16, 64, dtype=torch.float16)
    k = torch.ones(1, 1, 64, dtype=torch.float16)
    with pytest.raises(RuntimeError, match="out of range"):
        ext.store_kv(k, k, torch.tensor([32], dtype=torch.int64), kc, kc.clone())
    k2 = torch.ones(2, 1, 64, dtype=torch.float16)
    vc = kc.clone()
    for bad in (-1, 32):
        with pytest.raises(RuntimeError, match="out of range"):
            ext.store_kv(k2, k2, torch.tensor([3, bad], dtype=torch.int64), kc, vc)
        assert not kc.any() and not vc.any()
    with pytest.raises(RuntimeError, match="int64"):
        ext.store_kv(k, k, torch.tensor([3], dtype=torch.int32), kc, vc)
    k_strided = torch.ones(2, 1, 128, dtype=torch.float16)[..., ::2]
    with pytest.raises(RuntimeError, match="contiguous"):
        ext.store_kv(k_strided, k_strided, torch.tensor([3, 4], dtype=torch.int64), kc, vc)


def test_thread_controls_and_isa():
    ext = host_ext.load_ext()
    default = ext.get_num_threads()
    assert default >= 1
    try:
        ext.set_num_threads(3)
        assert ext.get_num_threads() == 3
        q, kc, vc, bt, lens = cases.rand_case(9, 8, 2, 64, 16, 40, torch.float16, 120, 2)
        o3 = torch.empty_like(q)
        l3 = torch.empty(8, 9)
        ext.decode_attn(q, kc, vc, bt, lens, 0.1, o3, l3)
        ext.set_num_threads(1)
        o1 = torch.empty_like(q)
        l1 = torch.empty(8, 9)
        ext.decode_attn(q, kc, vc, bt, lens, 0.1, o1, l1)
        assert torch.equal(o1, o3) and torch.equal(l1, l3)
        with pytest.raises(RuntimeError, match="at most 1024"):
            ext.set_num_threads(1025)
        assert ext.get_num_threads() == 1  # a refused count changes nothing
    finally:
        ext.set_num_threads(0)
    assert ext.get_num_threads() == default
    assert ext.has_avx2() is True


def test_decode_attn_rejects_like_the_reference():
    ext = host_ext.load_ext()
    q, kc, vc, bt, lens = cases.rand_case(2, 4, 2, 64, 16, 8, torch.float16, 30, 0)
    out = torch.empty_like(q)
    lse = torch.empty(4, 2)
    with pytest.raises(RuntimeError, match="contiguous"):
        ext.decode_attn(q.transpose(0, 1).contiguous().transpose(0, 1), kc, vc, bt, lens, 0.1,
                        out, lse)
    with pytest.raises(RuntimeError, match="int32"):
        ext.decode_attn(q, kc, vc, bt.long(), lens, 0.1, out, lse)
    with pytest.raises(RuntimeError, match="multiple"):
        ext.decode_attn(q[:, :3].contiguous(), kc, vc, bt, lens, 0.1, out[:, :3].contiguous(),
                        lse[:3].contiguous())
    with pytest.raises(RuntimeError, match="share a dtype"):
        ext.decode_attn(q, kc, vc, bt, lens, 0.1, out.to(torch.bfloat16), lse)


def test_split_and_merge_equals_full_attention():
    """tests/test_cpu_kernel.py:99-147's invariant on the host-core kernel:
    two partials over a split of each row's blocks, LSE-merged by the float64
    oracle, equal the partial over all blocks."""
    n, H, KVH, D, BS, C = 6, 8, 2, 128, 16, 64
    q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, torch.bfloat16, 200, 7)
    lens[1] = 40
    nb = (lens + BS - 1) // BS
    cut = nb // 2
    bt_a = torch.zeros_like(bt)
    bt_b = torch.zeros_like(bt)
    len_a = torch.zeros_like(lens)
    len_b = torch.zeros_like(lens)
    for i in range(n):
        c, k = int(cut[i]), int(nb[i])
        bt_a[i, :c] = bt[i, :c]
        bt_b[i, :k - c] = bt[i, c:k]
        len_a[i] = c * BS
        len_b[i] = int(lens[i]) - c * BS
    parts = []
    for t, ln in ((bt_a, len_a), (bt_b, len_b)):
        o = torch.empty(n, H, D)
        l = torch.empty(H, n)
        host_ext.decode_attn(q, kc, vc, t, ln, 0.09, o, l)
        parts.append((o, l))
    merged, mlse = oracle.merge_f64(parts[0][0], parts[0][1], parts[1][0], parts[1][1])
    full = torch.empty(n, H, D)
    flse = torch.empty(H, n)
    host_ext.decode_attn(q, kc, vc, bt, lens, 0.09, full, flse)
    torch.testing.assert_close(merged.float(), full, atol=2e-5, rtol=2e-5)
    torch.testing.assert_close(mlse.float(), flse, atol=2e-5, rtol=1e-6)
