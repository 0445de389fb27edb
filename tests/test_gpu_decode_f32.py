"""GPU parity of the fp32-KV tiled kernel (decode_f32.hip) against the
float64 oracle: the reference's third dtype (fastdecode/csrc/cpu_attn.cpp:
439-448; its own tests run fp32 too, tests/test_cpu_kernel.py:38-57).

Bars: out max-abs <= 5e-5 (fp32 arithmetic throughout, inputs ~N(0,1)),
lse relative <= 1e-5; empty rows exactly 0 / -inf; a range error poisons
only its own row. Cases: head sizes 64 / 128 / 256 and between them (72, 96,
in the next larger kernel with idle lanes); groups of 1, 2, 3, 4, 8, 12 and
20 (passes of 8 at D <= 128, of 4 above); host layout and vLLM's; whole
rows, forced 2-block splits and the model's choice; cache blocks of 32 and
64 tokens; two tiers in one launch; pinned host memory read zero-copy;
large scores.
"""

from __future__ import annotations

import math

import pytest
import torch

import oracle
from tests import cases
from tests.test_gpu_decode import GQA_LENS, run_host_layout
from vllm_fastdecoder_amd import ops
from vllm_fastdecoder_amd.pinned import pinned_empty

pytestmark = pytest.mark.gpu

OUT_TOL = 5e-5
LSE_TOL = 1e-5
LENS = GQA_LENS + [700, 333]


def _case(H, KVH, D, seed, lens=LENS, BS=16, C=None):
    n = len(lens)
    nbs = [(L + BS - 1) // BS for L in lens]
    C = C or sum(nbs) + 4
    q, kc, vc, bt, ln = cases.rand_case(n, H, KVH, D, BS, C, torch.float32,
                                        max_len=max(lens), seed=seed)
    ln[:] = torch.tensor(lens, dtype=torch.int32)
    perm = torch.randperm(C, generator=torch.Generator().manual_seed(seed)).to(torch.int32)
    bt.zero_()
    pos = 0
    for i, nb in enumerate(nbs):  # disjoint blocks for these lengths
        bt[i, :nb] = perm[pos: pos + nb]
        pos += nb
    return q, kc, vc, bt, ln


def _check(out, lse, ref_out, ref_lse, lens, gpu):
    nz = lens > 0
    o = out.double().cpu()[nz]
    err = float((o - ref_out[nz]).abs().max()) if bool(nz.any()) else 0.0
    assert err <= OUT_TOL, f"out err {err:.3g}"
    lr = lse.double().cpu()[:, nz]
    rl = ref_lse[:, nz]
    lerr = float(((lr - rl).abs() / rl.abs().clamp(min=1.0)).max()) if bool(nz.any()) else 0.0
    assert lerr <= LSE_TOL, f"lse rel err {lerr:.3g}"
    assert torch.all(out[~nz.to(gpu)] == 0)
    assert torch.all(torch.isneginf(lse[:, ~nz.to(gpu)]))


@pytest.mark.parametrize("D", [64, 128, 256, 72, 96])
@pytest.mark.parametrize("H,KVH", [(8, 8), (8, 4), (12, 4), (16, 4), (16, 2), (24, 2), (40, 2)])
def test_f32_kernel_matches_oracle(gpu, D, H, KVH, monkeypatch):
    q, kc, vc, bt, lens = _case(H, KVH, D, seed=D + 7 * H + KVH)
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, lens, scale)
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    for split in ("0", "2", "16"):
        monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
        out, lse = run_host_layout(q, kc, vc, bt, lens, scale, torch.float32, gpu)
        _check(out, lse, ref_out, ref_lse, lens, gpu)
        o_v, l_v = ops.paged_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt.to(gpu),
                                    lens.to(gpu), scale)
        torch.cuda.synchronize()
        _check(o_v, l_v, ref_out, ref_lse, lens, gpu)


@pytest.mark.parametrize("BS", [32, 64])
def test_f32_kernel_larger_cache_blocks(gpu, BS, monkeypatch):
    lens = [0, 1, BS - 1, BS, BS + 1, 3 * BS + 5, 7, 2 * BS, 900]
    q, kc, vc, bt, ln = _case(16, 4, 128, seed=BS, lens=lens, BS=BS)
    scale = 1.0 / math.sqrt(128)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, ln, scale)
    for split in ("0", "2"):
        monkeypatch.setenv("FD_SPLIT_BLOCKS", split)
        out, lse = run_host_layout(q, kc, vc, bt, ln, scale, torch.float32, gpu)
        _check(out, lse, ref_out, ref_lse, ln, gpu)


@pytest.mark.parametrize("H,KVH", [(8, 8), (16, 4)])
def test_f32_two_tiers_one_launch(gpu, H, KVH):
    """Each row's blocks split between an HBM tier (vLLM's layout) and a
    pinned host tier (host layout) read zero-copy, in one launch, against the
    oracle over the row's blocks as one list."""
    D = 128
    lens = [700, 300, 1, 0, 17, 64, 1500]
    n = len(lens)
    q, kc, vc, bt, ln = _case(H, KVH, D, seed=H, lens=lens)
    scale = 1.0 / math.sqrt(D)
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, ln, scale)
    W = bt.shape[1]
    bt0 = torch.zeros(n, W, dtype=torch.int32)
    bt1 = torch.zeros(n, W, dtype=torch.int32)
    l0 = torch.zeros(n, dtype=torch.int32)
    l1 = torch.zeros(n, dtype=torch.int32)
    for i, L in enumerate(lens):
        nb = (L + 15) // 16
        k = (2 * nb) // 5
        bt0[i, :k] = bt[i, :k]
        bt1[i, : nb - k] = bt[i, k:nb]
        l0[i] = 16 * k
        l1[i] = L - 16 * k
    kv = torch.cat([kc.transpose(1, 2), vc.transpose(1, 2)], dim=-1).contiguous().to(gpu)
    hk = pinned_empty(kc.shape, kc.dtype)
    hv = pinned_empty(vc.shape, vc.dtype)
    hk.copy_(kc)
    hv.copy_(vc)
    for k_host, v_host in ((hk, hv), (kc.to(gpu), vc.to(gpu))):
        out = torch.empty(n, H, D, dtype=torch.float32, device=gpu)
        lse = torch.empty(H, n, dtype=torch.float32, device=gpu)
        ops.split_decode(q.to(gpu), kv[..., :D], kv[..., D:], bt0.to(gpu), l0.to(gpu), k_host,
                         v_host, bt1.to(gpu), l1.to(gpu), scale, out=out, lse=lse)
        torch.cuda.synchronize()
        _check(out, lse, ref_out, ref_lse, ln, gpu)


def test_f32_large_scores_and_range_errors(gpu):
    """q x 300 stays finite and matches the oracle; a table entry past the
    cache or a length past the table poisons only its own row."""
    H, KVH, D = 8, 2, 128
    lens = [64, 40, 33, 17, 500]
    q, kc, vc, bt, ln = _case(H, KVH, D, seed=3, lens=lens)
    q = q * 300.0
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, ln, 1.0)
    out, lse = run_host_layout(q, kc, vc, bt, ln, 1.0, torch.float32, gpu)
    assert torch.isfinite(out).all() and torch.isfinite(lse).all()
    # scores in the thousands: the lse bar is relative, the weights stay exact
    _check(out, lse, ref_out, ref_lse, ln, gpu)
    bt_bad = bt.clone()
    bt_bad[1, 1] = kc.shape[0] + 5
    ln_bad = ln.clone()
    ln_bad[2] = bt.shape[1] * 16 + 1
    out, lse = run_host_layout(q, kc, vc, bt_bad, ln_bad, 1.0, torch.float32, gpu)
    assert torch.isnan(out[1]).all() and torch.isnan(lse[:, 1]).all()
    assert torch.isnan(out[2]).all() and torch.isnan(lse[:, 2]).all()
    ok = torch.tensor([True, False, False, True, True])
    o = out.double().cpu()[ok]
    assert float((o - ref_out[ok]).abs().max()) <= OUT_TOL


def test_f32_takes_the_tiled_kernel_when_aligned(gpu):
    """An aligned fp32 launch and the same call with an unaligned head
    stride (the generic kernel) agree with the oracle; the aligned one takes
    the tiled kernel, so its long rows also split (workspace needed)."""
    H, KVH, D = 8, 8, 64
    q, kc, vc, bt, ln = _case(H, KVH, D, seed=11)
    scale = 0.125
    ref_out, ref_lse = oracle.decode_attn_host_layout_f64(q, kc, vc, bt, ln, scale)
    out, lse = run_host_layout(q, kc, vc, bt, ln, scale, torch.float32, gpu)
    _check(out, lse, ref_out, ref_lse, ln, gpu)
    # q with a padded head stride of 68 floats (not a multiple of 8): generic
    qp = torch.zeros(q.shape[0], H, 68)
    qp[..., :D] = q
    qv = qp.to(gpu)[..., :D]
    out2 = torch.empty(q.shape[0], H, D, dtype=torch.float32, device=gpu)
    lse2 = torch.empty(H, q.shape[0], dtype=torch.float32, device=gpu)
    ops.decode_attn(qv, kc.to(gpu), vc.to(gpu), bt.to(gpu), ln.to(gpu), scale, out2, lse2)
    torch.cuda.synchronize()
    _check(out2, lse2, ref_out, ref_lse, ln, gpu)
