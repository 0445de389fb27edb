"""CPU test of the OPS seam a maintainer installs in the reference plugin
(backend.make_ops, the INTEGRATION snippet for fastdecode/backend.py:42-64).

The reference calls OPS.fa in three forms (fastdecode/backend.py:305-340):
the S rows' paged decode (one query token per row, block table, not causal),
the P rows' causal prefill over the paged cache, and the F rows' prefill over
this step's q/k/v with no block table. Only the first may reach this
library's paged decode; the other two must reach FlashAttention unchanged.
Here FlashAttention is a recording stub and the HIP decode a recording
stand-in (no GPU), and the P/F calls are driven through the orchestration's
own prefill step (SplitDecodeImpl._prefill_rows) on the reference's
classification KAT scenario.
"""

from __future__ import annotations

import torch

from tests.test_plan import KATS, scenario
from vllm_fastdecoder_amd import backend, plan


class _Recorder:
    def __init__(self):
        self.calls = []

    def fa(self, **kw):
        self.calls.append(kw)
        q = kw["q"]
        return torch.zeros_like(q)


def test_decode_form_goes_to_hip_and_prefill_forms_to_flash_attention(monkeypatch):
    stub = _Recorder()
    hip_calls = []

    def fake_paged_decode(q, k, v, block_table, seqused_k, softmax_scale, out=None,
                          row_order=None, max_seqlen_k=None, total_tokens=None):
        hip_calls.append((q.shape, block_table.shape, max_seqlen_k))
        return torch.zeros_like(q), torch.zeros(q.shape[1], q.shape[0])

    monkeypatch.setattr(backend.ops, "paged_decode", fake_paged_decode)
    OPS = backend.make_ops(prefill_fa=stub.fa)
    H, KVH, D, BS, B = 4, 2, 64, 16, 6
    q1 = torch.zeros(3, H, D)
    kc = torch.zeros(B, BS, KVH, D)
    bt = torch.zeros(3, 2, dtype=torch.int32)
    lens = torch.tensor([5, 0, 17], dtype=torch.int32)
    # S rows: the decode call of backend.py:306-314 (with its extra FA kwargs)
    o, lse = OPS.fa(q=q1, k=kc, v=kc, cu_seqlens_q=torch.arange(4, dtype=torch.int32),
                    max_seqlen_q=1, seqused_k=lens, max_seqlen_k=17, softmax_scale=0.125,
                    causal=False, block_table=bt, softcap=0.0, return_softmax_lse=True,
                    num_splits=1, fa_version=2)
    assert len(hip_calls) == 1 and not stub.calls
    assert hip_calls[0][2] == 17  # max_seqlen_k reaches the decode (it narrows the table)
    # P rows: causal prefill over the paged cache (backend.py:317-327)
    OPS.fa(q=torch.zeros(7, H, D), k=kc, v=kc, cu_seqlens_q=torch.tensor([0, 4, 7]),
           max_seqlen_q=4, seqused_k=torch.tensor([20, 9]), max_seqlen_k=20,
           softmax_scale=0.125, causal=True, block_table=bt[:2], softcap=0.0, fa_version=2)
    # a P batch of single-token requests is still causal: it stays on FlashAttention
    OPS.fa(q=torch.zeros(2, H, D), k=kc, v=kc, cu_seqlens_q=torch.tensor([0, 1, 2]),
           max_seqlen_q=1, seqused_k=torch.tensor([20, 9]), max_seqlen_k=20,
           softmax_scale=0.125, causal=True, block_table=bt[:2], softcap=0.0, fa_version=2)
    # F rows: prefill over this step's q/k/v, no block table (backend.py:328-340)
    kf = torch.zeros(9, KVH, D)
    OPS.fa(q=torch.zeros(9, H, D), k=kf, v=kf, cu_seqlens_q=torch.tensor([0, 9]),
           cu_seqlens_k=torch.tensor([0, 9]), max_seqlen_q=9, max_seqlen_k=9,
           softmax_scale=0.125, causal=True, softcap=0.0, fa_version=2)
    assert len(hip_calls) == 1 and len(stub.calls) == 3
    assert stub.calls[0]["block_table"] is not None and stub.calls[0]["causal"]
    assert "block_table" not in stub.calls[2] and "cu_seqlens_k" in stub.calls[2]
    # a decode call with a soft-cap is not this library's: FlashAttention gets it
    OPS.fa(q=q1, k=kc, v=kc, cu_seqlens_q=torch.arange(4, dtype=torch.int32), max_seqlen_q=1,
           seqused_k=lens, max_seqlen_k=17, softmax_scale=0.125, causal=False, block_table=bt,
           softcap=30.0, return_softmax_lse=True)
    assert len(hip_calls) == 1 and len(stub.calls) == 4
    # the rest of the seam is this library's
    assert OPS.reshape_and_cache is backend.HipOps.reshape_and_cache
    assert OPS.merge is backend.HipOps.merge and OPS.split_decode is backend.HipOps.split_decode


def test_prefill_rows_of_a_step_reach_flash_attention(monkeypatch):
    """The P and F rows of the reference's classification KAT
    (tests/test_plan_and_forward.py:199-227) go through the orchestration's
    prefill step to the stub, with the reference's arguments."""
    stub = _Recorder()
    monkeypatch.setattr(backend, "OPS", backend.make_ops(prefill_fa=stub.fa))
    reqs, G, C, BS, D = KATS["classification"]["reqs"], 10, 20, 4, 64
    H, KVH = 4, 2
    qsl, seq, bt, slots = scenario(reqs, BS)
    hp = plan.build_host_plan(qsl, seq, bt, slots, G, C, BS)
    dp = plan.to_device(hp, bt, "cpu")
    assert hp.n_p_tok > 0 and hp.n_f_tok > 0
    T = int(qsl[-1])
    query = torch.randn(T, H, D)
    key = torch.randn(T, KVH, D)
    value = torch.randn(T, KVH, D)
    kv_cache = torch.zeros(G, KVH, BS, 2 * D)
    key_cache, value_cache = kv_cache.transpose(1, 2).split(D, dim=-1)
    out = torch.full((T, H, D), float("nan"))
    impl = backend.SplitDecodeImpl(H, KVH, D, 0.125, cpu_fraction=0.0)
    impl._prefill_rows(query, key, value, key_cache, value_cache, dp, out)
    assert len(stub.calls) == 2
    p, f = stub.calls
    assert p["causal"] and p["block_table"] is not None and p["q"].shape[0] == hp.n_p_tok
    assert torch.equal(p["seqused_k"], dp.p_seqlens)
    assert f["causal"] and f.get("block_table") is None and f["q"].shape[0] == hp.n_f_tok
    assert torch.equal(f["cu_seqlens_q"], dp.f_cu) and torch.equal(f["cu_seqlens_k"], dp.f_cu)
    # the stub's rows were written into the step's output at the P and F tokens
    assert torch.all(out[dp.p_tok] == 0) and torch.all(out[dp.f_tok] == 0)
