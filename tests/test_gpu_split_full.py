"""GPU parity of the split run at the full headline shapes.

The layout of the split run (tests/cases.split_tiers): every row of the
workload (n=128, 32/32 heads, fp16, L ~ U[256, 2048] for vicuna-7b; n=256,
32/8 heads, bf16, L ~ U[1024, 4096] for Llama-3-8B) keeps its first 40 % of
blocks in HBM in vLLM's [B, BS, KVH, 2D] layout and its last ceil(0.6 * nb)
blocks in pinned host memory [C, KVH, BS, D], read by the GPU zero-copy.

The reference's split step is three calls: the GPU-tier partial, the
host-tier partial and the LSE merge (fastdecode/backend.py:293-356; the same
check in scripts/gpu_selftest.py:215-239). Each way the library runs that step
is compared, on every row, with the float64 oracle of monolithic attention
over the row's blocks of both tiers as one list:
  * the three calls (paged_decode + decode_attn + merge_attn_states);
  * the fused single launch (split_decode);
  * the hybrid split (host cores + GPU) at a fixed host-core share of 0.8,
    and at the share ShareTuner settles on after warm-up steps.
Bars: fp32 out max-abs <= 2e-3, lse <= 1e-4 relative.
"""

from __future__ import annotations

import pytest
import torch

import oracle
from tests import cases
from vllm_fastdecoder_amd import ops
from vllm_fastdecoder_amd.plan import ShareTuner

pytestmark = pytest.mark.gpu


def monolithic_oracle(w, q, t, lens):
    """float64 attention over each row's HBM blocks followed by its host
    blocks, as one pool [G + C, KVH, BS, D] (the HBM tier's blocks first)."""
    D = w.D
    kv = t["kv"].cpu()
    G, C = t["G"], t["C"]
    k = torch.cat([kv[:G, ..., :D].permute(0, 2, 1, 3), t["hk"][:C]]).contiguous()
    v = torch.cat([kv[:G, ..., D:].permute(0, 2, 1, 3), t["hv"][:C]]).contiguous()
    del kv
    nbg = (t["len_g"] + w.BS - 1) // w.BS
    nbc = (t["len_c"] + w.BS - 1) // w.BS
    W = int((nbg + nbc).max())
    uni = torch.zeros(w.n, W, dtype=torch.int32)
    for i in range(w.n):
        a, b = int(nbg[i]), int(nbc[i])
        uni[i, :a] = t["bt_g"][i, :a]
        uni[i, a:a + b] = t["bt_c"][i, :b] + G
    assert torch.equal(t["len_g"] + t["len_c"], lens)
    return oracle.decode_attn_host_layout_f64(q.cpu(), k, v, uni, lens, w.scale)


def check(name, out, lse, ref_o, ref_l):
    err = float((out.double().cpu() - ref_o).abs().max())
    rel = float(((lse.double().cpu() - ref_l).abs() / ref_l.abs().clamp(min=1)).max())
    print(f"  {name}: max|out err| {err:.2e}, max lse rel err {rel:.2e}", flush=True)
    assert err <= 2e-3, name
    assert rel <= 1e-4, name


@pytest.mark.parametrize("name", ["vicuna7b", "llama3_8b"])
def test_split_run_full_size_matches_oracle(gpu, name):
    w = cases.WORKLOADS[name]
    print(f"split run {name}: n={w.n}, {w.H}/{w.KVH} heads, {w.dtype}", flush=True)
    lens, bt, _ = cases.draw_lens_and_tables(w)
    t = cases.split_tiers(w, lens, bt, gpu)
    q = cases.queries(w, gpu)
    kc_g, vc_g, hk, hv = t["kc_g"], t["vc_g"], t["hk"], t["hv"]
    bt_g, bt_c, len_g, len_c = t["bt_g"], t["bt_c"], t["len_g"], t["len_c"]
    assert int((len_c > 0).sum()) == w.n  # every row reads the host tier
    bt_g_d, bt_c_d = bt_g.to(gpu), bt_c.to(gpu)
    len_g_d, len_c_d = len_g.to(gpu), len_c.to(gpu)
    n, H, D = w.n, w.H, w.D

    def f32(*shape):
        return torch.empty(*shape, dtype=torch.float32, device=gpu)

    results = {}
    # the reference's three calls: GPU-tier partial, host-tier partial, merge
    o_g, l_g = ops.paged_decode(q, kc_g, vc_g, bt_g_d, len_g_d, w.scale, out=f32(n, H, D))
    o_c, l_c = f32(n, H, D), f32(H, n)
    ops.decode_attn(q, hk, hv, bt_c_d, len_c_d, w.scale, o_c, l_c)
    merged, m_lse = f32(n, H, D), f32(H, n)
    ops.merge_attn_states(merged, o_g, l_g, o_c, l_c, out_lse=m_lse)
    results["three calls"] = (merged, m_lse)
    # one fused launch over both tiers
    results["fused"] = ops.split_decode(q, kc_g, vc_g, bt_g_d, len_g_d, hk, hv, bt_c_d, len_c_d,
                                        w.scale, out=f32(n, H, D), lse=f32(H, n))
    # hybrid at a fixed host-core share
    results["hybrid 0.8"] = ops.hybrid_split_decode(q, kc_g, vc_g, bt_g_d, len_g, hk, hv, bt_c,
                                                    len_c, w.scale, 0.8, out=f32(n, H, D),
                                                    lse=f32(H, n))
    # hybrid at the share the online balance settles on
    tuner = ShareTuner()
    h_out, h_lse = f32(n, H, D), f32(H, n)
    for _ in range(40):
        h = ops.hybrid_split_begin(q, kc_g, vc_g, bt_g_d, len_g, hk, hv, bt_c, len_c, w.scale,
                                   tuner.fraction, out=h_out, lse=h_lse)
        h.finish()
        tuner.update(h.gpu_finished_first)
    frac = tuner.fraction
    results[f"hybrid auto ({frac:.2f})"] = ops.hybrid_split_decode(
        q, kc_g, vc_g, bt_g_d, len_g, hk, hv, bt_c, len_c, w.scale, frac, out=f32(n, H, D),
        lse=f32(H, n))
    torch.cuda.synchronize()
    ref_o, ref_l = monolithic_oracle(w, q, t, lens)
    for mode, (out, lse) in results.items():
        check(mode, out, lse, ref_o, ref_l)
