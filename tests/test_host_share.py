"""plan.share_host_blocks: the division of each row's host-tier blocks
between the GPU and the host cores (host logic, CPU only).

Invariants checked on random tables: the GPU's leading blocks followed by the
host cores' trailing blocks are exactly the row's block list; the two token
counts add up to the row's; the GPU's count covers whole blocks whenever the
host cores have any; the host cores get floor(nb * f + 1/2) blocks; f = 1 is
the reference's division (every host block on the host cores) and f = 0
leaves everything to the GPU.
"""

from __future__ import annotations

import math
import random

import pytest
import torch

from vllm_fastdecoder_amd.plan import share_host_blocks


def _random_rows(rng, n, BS, W):
    lens = torch.tensor([rng.choice([0, 1, BS, rng.randint(1, W * BS)]) for _ in range(n)],
                        dtype=torch.int32)
    bt = torch.randint(-5, 10**6, (n, W), dtype=torch.int32)  # junk past each row's blocks
    return bt, lens


@pytest.mark.parametrize("seed", range(20))
def test_share_invariants(seed):
    rng = random.Random(seed)
    BS = rng.choice([1, 4, 16])
    n, W = rng.randint(1, 30), rng.randint(1, 40)
    bt, lens = _random_rows(rng, n, BS, W)
    f = rng.choice([0.0, 1.0, rng.random()])
    s = share_host_blocks(bt, lens, BS, f)
    assert s.gpu_lens.dtype == s.cpu_lens.dtype == s.cpu_bt.dtype == torch.int32
    for r in range(n):
        L = int(lens[r])
        nb = (L + BS - 1) // BS
        gl, cl = int(s.gpu_lens[r]), int(s.cpu_lens[r])
        assert gl + cl == L
        kc = (cl + BS - 1) // BS
        assert kc == min(nb, math.floor(nb * f + 0.5))
        if cl:
            assert gl % BS == 0
        kg = gl // BS if cl else (gl + BS - 1) // BS
        assert kg + kc == nb
        assert bt[r, :kg].tolist() + s.cpu_bt[r, :kc].tolist() == bt[r, :nb].tolist()
        assert torch.all(s.cpu_bt[r, kc:] == 0)


def test_share_extremes_are_the_reference_split_and_the_gpu_only_split():
    bt = torch.tensor([[5, 6, 7, 8], [1, 2, 0, 0], [3, 0, 0, 0], [0, 0, 0, 0]], dtype=torch.int32)
    lens = torch.tensor([50, 17, 3, 0], dtype=torch.int32)
    s1 = share_host_blocks(bt, lens, 16, 1.0)
    assert s1.gpu_lens.tolist() == [0, 0, 0, 0] and s1.cpu_lens.tolist() == [50, 17, 3, 0]
    assert s1.cpu_bt[:, :4].tolist() == [[5, 6, 7, 8], [1, 2, 0, 0], [3, 0, 0, 0], [0, 0, 0, 0]]
    s0 = share_host_blocks(bt, lens, 16, 0.0)
    assert s0.gpu_lens.tolist() == [50, 17, 3, 0] and s0.cpu_lens.tolist() == [0, 0, 0, 0]
    sh = share_host_blocks(bt, lens, 16, 0.5)
    assert sh.gpu_lens.tolist() == [32, 16, 0, 0] and sh.cpu_lens.tolist() == [18, 1, 3, 0]
    assert sh.cpu_bt.tolist() == [[7, 8], [2, 0], [3, 0], [0, 0]]


def test_share_rejects_fractions_outside_unit_interval():
    bt = torch.zeros(1, 1, dtype=torch.int32)
    with pytest.raises(ValueError):
        share_host_blocks(bt, torch.ones(1, dtype=torch.int32), 16, 1.5)
    s = share_host_blocks(bt[:0], torch.zeros(0, dtype=torch.int32), 16, 0.5)
    assert s.gpu_lens.numel() == 0 and s.cpu_bt.shape[0] == 0


def test_share_tuner_converges_to_the_balanced_fraction():
    """A modelled step: the host cores take f * B bytes at rate c, the GPU
    (1 - f) * B at rate g; whoever finishes first is reported. The tuner
    settles within one step of the balance point c / (c + g) and stays
    there."""
    from vllm_fastdecoder_amd.plan import ShareTuner

    for c, g in ((175.0, 55.6), (40.0, 55.6), (300.0, 20.0)):
        t = ShareTuner(start=0.5, step=0.01)
        seen = []
        for _ in range(200):
            f = t.fraction
            t.update(gpu_finished_first=(1 - f) / g < f / c)
            seen.append(t.fraction)
        star = c / (c + g)
        assert all(abs(x - star) <= 0.011 for x in seen[-50:]), (c, g, seen[-5:])


def test_share_tuner_bounds_and_backend_validation():
    from vllm_fastdecoder_amd import backend
    from vllm_fastdecoder_amd.plan import ShareTuner

    t = ShareTuner(start=0.06, step=0.05, lo=0.05, hi=1.0)
    assert t.update(True) == 0.05 and t.update(True) == 0.05
    t = ShareTuner(start=0.99, step=0.05)
    assert t.update(False) == 1.0
    with pytest.raises(ValueError):
        ShareTuner(start=2.0)
    assert backend.SplitDecodeImpl(4, 4, 64, 0.1, cpu_fraction="auto")._host_share() == 0.85
    assert backend.SplitDecodeImpl(4, 4, 64, 0.1, cpu_fraction=0.3)._host_share() == 0.3
    for bad in (1.5, -0.1, "fast"):
        with pytest.raises(ValueError):
            backend.SplitDecodeImpl(4, 4, 64, 0.1, cpu_fraction=bad)


def test_share_rejects_rows_past_their_table_and_handles_empty_tables():
    bt = torch.tensor([[1, 2], [3, 4]], dtype=torch.int32)
    with pytest.raises(RuntimeError, match="needs 3 blocks"):
        share_host_blocks(bt, torch.tensor([16, 33], dtype=torch.int32), 16, 0.5)
    s = share_host_blocks(torch.zeros(3, 0, dtype=torch.int32), torch.zeros(3, dtype=torch.int32),
                          16, 0.7)
    assert s.gpu_lens.tolist() == [0, 0, 0] and s.cpu_lens.tolist() == [0, 0, 0]
    # negative lengths count as empty rows
    s = share_host_blocks(bt, torch.tensor([-5, 20], dtype=torch.int32), 16, 1.0)
    assert s.gpu_lens.tolist() == [0, 0] and s.cpu_lens.tolist() == [0, 20]
    assert s.cpu_bt[1].tolist() == [3, 4]


def test_share_tuner_ignores_a_step_without_a_finishing_order():
    from vllm_fastdecoder_amd.plan import ShareTuner

    t = ShareTuner(start=0.5, step=0.01)
    assert t.update(None) == 0.5
    assert t.update(True) == pytest.approx(0.49)
    assert t.update(False) == pytest.approx(0.5)
