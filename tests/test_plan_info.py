"""The planner's kernel choice through fd_decode_plan_info (no GPU needed:
without a device the CU count is unknown, so the large-MHA rule, which needs
it, is checked by tests/test_gpu_decode_mm.py)."""

from __future__ import annotations

import math

import pytest
import torch

from vllm_fastdecoder_amd import _lib, ops

F16, BF16, F32 = torch.float16, torch.bfloat16, torch.float32


def plan(n, H, KVH, D, W, dtype=BF16, BS=16, **kw):
    return ops.decode_plan_info(n, H, KVH, D, BS, W, dtype, **kw)


@pytest.fixture(autouse=True)
def _no_overrides(monkeypatch):
    monkeypatch.delenv("FD_DECODE_KERNEL", raising=False)
    monkeypatch.delenv("FD_SPLIT_BLOCKS", raising=False)
    monkeypatch.delenv("FD_WAVE_BLOCKS", raising=False)


@pytest.mark.parametrize("H,KVH,D,kernel,slots,passes", [
    (32, 32, 128, "valu", 1, 1),    # MHA (small launch)
    (32, 16, 128, "valu", 2, 1),    # G = 2
    (24, 8, 128, "valu", 4, 1),     # G = 3: 4-slot VALU kernel
    (32, 8, 128, "mm", 16, 1),      # G = 4: both products on the matrix cores
    (64, 8, 128, "mm", 16, 1),      # G = 8
    (64, 2, 128, "mm", 32, 1),      # G = 32: two groups of 16 columns per task
    (48, 1, 128, "mm", 32, 2),      # G = 48 at D = 128: passes of 32
    (96, 2, 64, "mm", 64, 1),       # G = 48 at D = 64: four groups of 16
    (71, 1, 64, "mm", 64, 2),       # multi-query, 71 heads: passes of 64
    (32, 8, 64, "mm", 16, 1),
    (32, 8, 32, "mm", 16, 1),       # D a multiple of 32: groups of 4
    (32, 8, 96, "mm", 16, 1),
    (32, 8, 48, "valu", 4, 1),      # half-empty last q.K step: groups of 4 stay on the VALU
    (32, 8, 80, "valu", 4, 1),
    (32, 8, 112, "valu", 4, 1),
    (40, 8, 112, "mm", 16, 1),      # groups of 5 take it
    (64, 8, 80, "mm", 16, 1),
    (32, 8, 256, "mfma", 4, 1),     # D = 256: q.K-only matrix-core kernel
    (64, 8, 256, "mfma", 8, 1),
    (32, 8, 72, "valu", 4, 1),      # not a multiple of 16: VALU in its 128 build
    (32, 8, 160, "valu", 4, 1),
])
def test_16bit_kernel_choice(H, KVH, D, kernel, slots, passes):
    p = plan(128, H, KVH, D, 128)
    assert (p["kernel"], p["heads_per_task"], p["passes"]) == (kernel, slots, passes), p


@pytest.mark.parametrize("H,KVH,D,slots,passes", [
    (32, 32, 128, 1, 1), (32, 8, 128, 4, 1), (64, 8, 128, 8, 1), (64, 8, 256, 4, 2),
    (96, 4, 64, 8, 3),
])
def test_fp32_takes_its_own_kernel(H, KVH, D, slots, passes):
    p = plan(64, H, KVH, D, 64, dtype=F32)
    assert (p["kernel"], p["heads_per_task"], p["passes"]) == ("f32", slots, passes), p


def test_host_tier_and_unaligned_launches():
    # a tier in pinned host memory: 16-bit launches leave the matrix cores
    assert plan(128, 64, 8, 128, 128, host_tier=True)["kernel"] == "valu"
    assert plan(128, 64, 8, 128, 128, dtype=F32, host_tier=True)["kernel"] == "f32"
    # layouts the tiled kernels cannot take
    assert plan(128, 32, 8, 128, 128, aligned=False)["kernel"] == "generic"
    assert plan(8, 8, 8, 128, 8, BS=8)["kernel"] == "generic"      # block size not 16 m
    assert plan(8, 8, 8, 100, 8)["kernel"] == "generic"             # D not a multiple of 8
    assert plan(8, 8, 8, 512, 8)["kernel"] == "generic"             # D > 256
    assert plan(8, 8, 8, 128, 8, BS=64)["kernel"] == "valu"         # 4 tiles per block


def test_forced_kernels(monkeypatch):
    monkeypatch.setenv("FD_DECODE_KERNEL", "valu")
    assert plan(128, 64, 8, 128, 128)["kernel"] == "valu"
    monkeypatch.setenv("FD_DECODE_KERNEL", "mfma")
    assert plan(128, 64, 8, 128, 128)["kernel"] == "mfma"
    assert plan(128, 64, 8, 96, 128)["kernel"] == "valu"            # not built for 96
    monkeypatch.setenv("FD_DECODE_KERNEL", "mm")
    assert plan(8, 32, 32, 128, 64)["kernel"] == "mm"
    assert plan(8, 32, 32, 256, 64)["kernel"] == "valu"             # not built for 256


def test_task_split_follows_the_override(monkeypatch):
    monkeypatch.setenv("FD_SPLIT_BLOCKS", "16")
    p = plan(4, 32, 8, 128, 100)
    assert p["split_blocks"] == 16 and p["max_splits"] == 7 and not p["capped"]
    monkeypatch.setenv("FD_SPLIT_BLOCKS", "64")
    p = plan(4, 32, 8, 128, 100, BS=32)  # 100 blocks of 32 tokens = 200 tiles
    assert p["split_blocks"] == 64 and p["max_splits"] == 4 and p["capped"]


def test_tuning_variables_match_whole_names(monkeypatch):
    """The planner reads its tuning variables in one pass over the
    environment: each counts under its exact name only, and a longer name
    sharing its prefix, or the name without FD_, changes nothing."""
    base = plan(4, 32, 8, 128, 100)
    for name in ("FD_SPLIT_BLOCKSX", "FD_SPLIT_BLOCK", "SPLIT_BLOCKS", "XFD_SPLIT_BLOCKS"):
        monkeypatch.setenv(name, "16")
    monkeypatch.setenv("FD_DECODE_KERNEL_", "mfma")
    monkeypatch.setenv("FD_WG_CAPS", "1")
    assert plan(4, 32, 8, 128, 100) == base
    monkeypatch.setenv("FD_WG_CAP", "1")
    monkeypatch.setenv("FD_WAVE_BLOCKS", "5")
    p = plan(4, 32, 8, 128, 100)
    assert p["wg_cap"] == 1 and p["capped"] and p["wave_blocks"] == 5
    monkeypatch.setenv("FD_WG_CAP", "")      # empty: no cap from the variable
    monkeypatch.setenv("FD_WAVE_BLOCKS", "-3")  # negative: every wave works
    p = plan(4, 32, 8, 128, 100)
    assert p["wg_cap"] == base["wg_cap"] and p["wave_blocks"] == 0


def test_task_size_follows_the_block_bytes():
    """The launch-time model takes a workgroup's stream rate as proportional to
    a block's K + V bytes below 8 KiB (D = 128 at 16 bits), so at D = 64 the
    same rows are cut into tasks half as long, and a small multi-query launch
    (71 heads over one kv head) splits its rows. Measured (batch 32-128, 1-4k
    tokens, bf16) these are the best fixed sizes."""
    assert plan(64, 14, 2, 64, 256)["split_blocks"] == 64
    assert plan(64, 14, 2, 128, 256)["split_blocks"] == 128
    assert plan(128, 14, 2, 64, 256)["split_blocks"] == 128
    assert plan(32, 71, 1, 64, 256)["split_blocks"] < 256
    # D = 128 at 16 bits, fp32 at D = 64 (8 KiB blocks) and larger blocks: unchanged
    assert plan(128, 32, 8, 128, 128)["split_blocks"] == 256
    assert plan(64, 14, 2, 64, 256, dtype=F32)["split_blocks"] == \
        plan(64, 14, 2, 128, 256)["split_blocks"]


def test_bad_arguments_raise():
    with pytest.raises(_lib.FdError):
        plan(8, 30, 8, 128, 8)           # H not a multiple of KVH
    with pytest.raises(_lib.FdError):
        ops.decode_plan_info(8, 32, 8, 128, 16, -1, BF16)


def test_token_total_without_a_device_keeps_the_plan():
    """Without a GPU (no CU count) the token total changes nothing; a negative
    total is an argument error."""
    if torch.cuda.is_available():
        pytest.skip("planner sees a device here")
    a = ops.decode_plan_info(256, 8, 1, 128, 16, 256, torch.bfloat16)
    b = ops.decode_plan_info(256, 8, 1, 128, 16, 256, torch.bfloat16, total_tokens=650_000)
    assert a == b
    with pytest.raises(Exception):
        ops.decode_plan_info(256, 8, 1, 128, 16, 256, torch.bfloat16, total_tokens=-1)


@pytest.mark.gpu
def test_token_total_steers_uneven_rows_to_the_slot_fill(gpu):
    """On the device: 8 query heads over 1 kv head, batch 256, a 256-block
    table. Rows filling 62 % of it on average take 64-block tasks at the
    kernel's own three workgroups per CU (the slot fill); rows filling all of
    it, or an unknown total, keep the model's whole-row tasks under the
    two-per-CU cap. Other kernel families ignore the total."""
    full = 256 * 256 * 16
    base = ops.decode_plan_info(256, 8, 1, 128, 16, 256, torch.bfloat16)
    assert base["split_blocks"] == 256 and base["max_splits"] == 1 and base["wg_cap"] == 2
    uneven = ops.decode_plan_info(256, 8, 1, 128, 16, 256, torch.bfloat16,
                                  total_tokens=int(0.62 * full))
    assert uneven["kernel"] == "mm" and uneven["split_blocks"] == 64
    assert uneven["max_splits"] == 4 and uneven["wg_cap"] == 0
    assert ops.decode_plan_info(256, 8, 1, 128, 16, 256, torch.bfloat16, total_tokens=full) == base
    mha = ops.decode_plan_info(16, 32, 32, 128, 16, 256, torch.bfloat16)
    assert ops.decode_plan_info(16, 32, 32, 128, 16, 256, torch.bfloat16,
                                total_tokens=int(0.5 * 16 * 256 * 16)) == mha
    # the workspace query covers any total
    need = ops.workspace_bytes(256, 8, 1, 128, 16, 256)
    assert need >= 256 * 8 * 4 * 128 * 4


@pytest.mark.gpu
def test_quarter_rows_just_past_one_row_per_cu(gpu):
    """On the device: a little more than one (sequence, kv head) row per CU
    (1.0-1.3) at D = 128 takes tasks of a quarter of the table width at three
    workgroups per CU, on the matrix-core and the VALU kernel alike; one row
    per CU, 1.4 rows per CU and D = 64 keep the model's whole rows."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    one = ops.decode_plan_info(cus, 8, 1, 128, 16, 256, torch.bfloat16)
    assert one["split_blocks"] == 256 and one["wg_cap"] == 2
    past = ops.decode_plan_info(cus + cus // 16, 8, 1, 128, 16, 256, torch.bfloat16)
    assert past["kernel"] == "mm" and past["split_blocks"] == 64 and past["max_splits"] == 4
    assert past["wg_cap"] in (0, 3)
    narrow = ops.decode_plan_info(cus + cus // 16, 8, 1, 128, 16, 128, torch.bfloat16)
    assert narrow["split_blocks"] == 32
    mha = ops.decode_plan_info(cus // 32 + 1, 32, 32, 128, 16, 256, torch.float16)
    assert mha["kernel"] == "valu" and mha["split_blocks"] == 64 and mha["wg_cap"] == 3
    far = ops.decode_plan_info(cus * 14 // 10, 8, 1, 128, 16, 256, torch.bfloat16)
    assert far["split_blocks"] == 256
    d64 = ops.decode_plan_info((cus + cus // 16) // 2, 14, 2, 64, 16, 256, torch.bfloat16)
    assert not (d64["split_blocks"] == 64 and d64["max_splits"] == 4 and d64["wg_cap"] in (0, 3))


@pytest.mark.gpu
def test_working_waves_by_row_length_on_small_launches(gpu):
    """On the device: launches of at most one task per CU on the VALU kernel at
    D = 128 give each task's waves a quarter of the longest task's tiles
    (table width, or the task size when rows split); one task more than the
    CUs, another kernel or another head size keeps every wave working."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    at = ops.decode_plan_info(cus // 32, 32, 32, 128, 16, 64, torch.float16)
    assert at["kernel"] == "valu" and at["max_splits"] == 1 and at["wave_blocks"] == 16, at
    g2 = ops.decode_plan_info(cus // 16, 32, 16, 128, 16, 50, torch.bfloat16)
    assert g2["kernel"] == "valu" and g2["wave_blocks"] == 13, g2
    big_bs = ops.decode_plan_info(cus // 32, 32, 32, 128, 32, 64, torch.float16)
    if big_bs["max_splits"] == 1:
        assert big_bs["wave_blocks"] == 32, big_bs  # 128 tiles of 16 tokens
    over = ops.decode_plan_info(cus // 32 + 1, 32, 32, 128, 16, 64, torch.float16)
    assert over["wave_blocks"] == 0, over
    for other in (ops.decode_plan_info(cus // 32, 32, 32, 64, 16, 64, torch.float16),
                  ops.decode_plan_info(cus // 32, 32, 8, 128, 16, 64, torch.bfloat16),
                  ops.decode_plan_info(cus // 32, 32, 32, 128, 16, 64, torch.float32)):
        assert other["wave_blocks"] == 0, other
    # batch 1 with rows longer than one task: the task size sets the tiles per wave
    split = ops.decode_plan_info(1, 32, 32, 128, 16, 1024, torch.float16)
    if split["max_splits"] * 32 <= cus:
        assert split["wave_blocks"] == (min(split["split_blocks"], 1024) + 3) // 4, split


@pytest.mark.gpu
def test_half_rows_for_full_rows_past_two_per_cu(gpu):
    """On the device: 2.0-2.6 rows per CU at D = 128 take half-row tasks when
    the token total shows the rows full (mean fill 0.8 or more); rows of
    mixed length, or no total, keep whole rows."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    n = cus * 9 // 4
    full = n * 256 * 16
    whole = ops.decode_plan_info(n, 8, 1, 128, 16, 256, torch.bfloat16)
    assert whole["split_blocks"] == 256
    half = ops.decode_plan_info(n, 8, 1, 128, 16, 256, torch.bfloat16, total_tokens=full)
    assert half["split_blocks"] == 128 and half["max_splits"] == 2
    mixed = ops.decode_plan_info(n, 8, 1, 128, 16, 256, torch.bfloat16,
                                 total_tokens=int(0.6 * full))
    assert mixed["split_blocks"] == 256


@pytest.mark.gpu
def test_workspace_covers_every_total(gpu):
    """The workspace query (which takes no total) covers what a total makes of
    a plan: half rows on the VALU kernel for full MHA rows, the slot fill on
    the matrix-core kernel for uneven ones."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for n, H, KVH, total_share, dt in ((cus * 17 // 256, 32, 32, 1.0, torch.float16),
                                        (cus * 9 // 4, 8, 1, 1.0, torch.bfloat16),
                                        (cus // 2, 8, 1, 0.6, torch.bfloat16)):
        total = int(total_share * n * 256 * 16)
        plan = ops.decode_plan_info(n, H, KVH, 128, 16, 256, dt, total_tokens=total)
        need = n * H * plan["max_splits"] * (128 + 1) * 4 if plan["max_splits"] > 1 else 0
        assert ops.workspace_bytes(n, H, KVH, 128, 16, 256) >= need, (n, H, KVH, plan)


@pytest.mark.gpu
def test_d64_rows_split_only_when_the_total_shows_them_full(gpu):
    """On the device at D = 64: 1.25 and 2.25 (sequence, kv head) rows per CU
    take quarter and half rows when the token total shows the rows all but
    full (mean fill 0.95 or more); a mean fill of 0.85, or no total, keeps
    the model's plan."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    for n, sb, splits in ((cus * 5 // 8, 64, 4), (cus * 9 // 8, 128, 2)):
        full = n * 256 * 16
        base = ops.decode_plan_info(n, 14, 2, 64, 16, 256, torch.bfloat16)
        split = ops.decode_plan_info(n, 14, 2, 64, 16, 256, torch.bfloat16, total_tokens=full)
        assert split["split_blocks"] == sb and split["max_splits"] == splits, (n, split)
        mixed = ops.decode_plan_info(n, 14, 2, 64, 16, 256, torch.bfloat16,
                                     total_tokens=int(0.85 * full))
        assert mixed == base, (n, mixed, base)


@pytest.mark.gpu
def test_every_window_boundary_from_both_sides(gpu):
    """Each window of the planner's cut table (decode_partial.hip, "row
    cuts") just inside and just outside each of its bounds, on a 256-block
    table (4096 tokens): rows per CU 1.0 / 1.3 (quarter rows at D = 128 and
    64), 2.0 / 2.6 (half rows), 1.5 (slot fill); mean fill 0.8 (half rows on
    one side, slot fill on the other) and 0.95 (D = 64). Inside a quarter
    window tasks are 64 blocks (4 per row), inside a half window 128 (2 per
    row); outside, the model's whole rows (or, at D = 64, the plan without a
    total)."""
    cus = torch.cuda.get_device_properties(0).multi_processor_count
    W = 256

    def plan(n, H, KVH, D, fill=None, below=False):
        total = None
        if fill is not None:
            cap = n * W * 16
            total = math.floor(fill * cap) - 1 if below else math.ceil(fill * cap)
        return ops.decode_plan_info(n, H, KVH, D, 16, W, torch.bfloat16, total_tokens=total)

    def cut(p):
        return (p["split_blocks"], p["max_splits"])

    def rows_n(kvh, lo10, hi10):
        """Sequence counts just outside and just inside each side of the
        window lo10 / 10 < rows per CU <= hi10 / 10 (rows = n * kvh)."""
        ns = [n for n in range(1, 4 * cus) if n * kvh * 10 > lo10 * cus and
              n * kvh * 10 <= hi10 * cus]
        first, last = ns[0], ns[-1]
        return first - 1, first, last, last + 1

    # quarter rows at D = 128 (8 query heads on 1 kv head: the matrix-core kernel), any fill
    out_lo, in_lo, in_hi, out_hi = rows_n(1, 10, 13)
    for n in (in_lo, in_hi):
        assert cut(plan(n, 8, 1, 128)) == (64, 4), n
    for n in (out_lo, out_hi):
        assert cut(plan(n, 8, 1, 128)) == (256, 1), n
    # ... and on the VALU kernel (MHA, 32 kv heads)
    out_lo, in_lo, in_hi, out_hi = rows_n(32, 10, 13)
    assert cut(plan(in_lo, 32, 32, 128)) == (64, 4) and cut(plan(in_hi, 32, 32, 128)) == (64, 4)
    assert plan(out_hi, 32, 32, 128)["split_blocks"] != 64
    # quarter rows at D = 64 (14 query heads on 2 kv heads): fill 0.95 or more
    out_lo, in_lo, in_hi, out_hi = rows_n(2, 10, 13)
    for n in (in_lo, in_hi):
        assert cut(plan(n, 14, 2, 64, 0.95)) == (64, 4), n
        assert plan(n, 14, 2, 64, 0.95, below=True) == plan(n, 14, 2, 64), n
    for n in (out_lo, out_hi):
        assert plan(n, 14, 2, 64, 1.0) == plan(n, 14, 2, 64), n
    # half rows at D = 128: fill 0.8 or more
    out_lo, in_lo, in_hi, out_hi = rows_n(1, 20, 26)
    for n in (in_lo, in_hi):
        assert cut(plan(n, 8, 1, 128, 0.8)) == (128, 2), n
        assert cut(plan(n, 8, 1, 128, 0.8, below=True)) == (256, 1), n
    for n in (out_lo, out_hi):
        assert cut(plan(n, 8, 1, 128, 1.0)) == (256, 1), n
    # half rows at D = 64: fill 0.95 or more
    out_lo, in_lo, in_hi, out_hi = rows_n(2, 20, 26)
    for n in (in_lo, in_hi):
        assert cut(plan(n, 14, 2, 64, 0.95)) == (128, 2), n
        assert plan(n, 14, 2, 64, 0.95, below=True) == plan(n, 14, 2, 64), n
    for n in (out_lo, out_hi):
        assert plan(n, 14, 2, 64, 1.0) == plan(n, 14, 2, 64), n
    # slot fill: fill below 0.8, at most 1.5 rows per CU, on the matrix-core kernel
    _, _, in_hi, out_hi = rows_n(1, 0, 15)
    base = plan(in_hi, 8, 1, 128)
    assert plan(in_hi, 8, 1, 128, 0.6)["max_splits"] > 1
    assert plan(in_hi, 8, 1, 128, 0.8, below=True)["max_splits"] > 1
    assert plan(in_hi, 8, 1, 128, 0.8) == base
    assert plan(out_hi, 8, 1, 128, 0.6) == plan(out_hi, 8, 1, 128)
    half_cu = cus // 2
    assert plan(half_cu, 8, 1, 128, 0.8, below=True)["max_splits"] > 1
    assert plan(half_cu, 8, 1, 128, 0.8) == plan(half_cu, 8, 1, 128)
