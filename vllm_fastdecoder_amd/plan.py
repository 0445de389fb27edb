"""Per-step execution plan of the split decode path (host side).

Block ids `< G` live in the HBM tier, ids `>= G` in the pinned host tier at
`id - G` (fastdecode/plan.py:3-4). Every active request falls in one class
(plan.py:6-10):

  P  all of its blocks in HBM                 -> ordinary paged attention
  S  a decode (one query token) touching the  -> HBM-tier partial + host-tier
     host tier                                   partial, LSE-merged
  F  a fresh prefill (no prior context)        -> attention over this step's
     touching the host tier                      q/k/v only

A request with prior context, more than one query token and host blocks (a
chunked-prefill continuation or prefix hit) is rejected (plan.py:142-149).

`build_host_plan` returns the same `HostPlan` fields, dtypes and values as
the reference's planner (fastdecode/plan.py:26-199): stable per-tier block
compaction, HBM tables zero-padded to a multiple of 16 columns, tier token
counts from the tokens held by each block, host slots masked to -1 in the
HBM slot mapping and rebased by `G * block_size` for the host tier. Beyond
the reference it also returns `host_slot_mapping`: the whole step's slot
mapping rebased to the host tier with HBM slots masked to -1, so one
cache-write kernel can write the host tier in place (no gather, no staging).

`to_device` mirrors fastdecode/plan.py:202-245.
"""

from __future__ import annotations

from dataclasses import dataclass

import numpy as np

import torch

GPU_TABLE_PAD = 16  # HBM-tier tables are padded to a multiple of 16 columns (plan.py:171,195-201)


@dataclass
class HostPlan:
    n_tok: int
    # KV writes
    gpu_slot_mapping: torch.Tensor  # [n_tok] int64, host-tier slots replaced by -1
    cpu_w_tok: torch.Tensor  # [nw] int64 token rows whose KV goes to the host tier
    cpu_w_slot: torch.Tensor  # [nw] int64 host-tier-relative slot ids
    # P
    p_tok: torch.Tensor  # [nP_tok] int64
    p_cu: torch.Tensor  # [nP + 1] int32
    p_seqlens: torch.Tensor  # [nP] int32
    p_req: torch.Tensor  # [nP] int64 rows of the block table
    p_max_q: int
    p_max_k: int
    # S
    s_tok: torch.Tensor  # [nS] int64
    s_gpu_bt: torch.Tensor  # [nS, Wg] int32 (HBM-tier block ids, compacted)
    s_gpu_lens: torch.Tensor  # [nS] int32
    s_max_gpu_len: int
    s_gpu_tokens: int  # sum of s_gpu_lens (the decode launch's token-total hint)
    s_cpu_bt: torch.Tensor  # [nS, Wc] int32 (host-tier-relative ids, compacted)
    s_cpu_lens: torch.Tensor  # [nS] int32
    # F
    f_tok: torch.Tensor  # [nF_tok] int64
    f_cu: torch.Tensor  # [nF + 1] int32
    f_max: int
    # (no counterpart in the reference) the step's slots rebased to the host
    # tier, HBM slots -> -1
    host_slot_mapping: torch.Tensor | None = None  # [n_tok] int64

    @property
    def n_s(self) -> int:
        return int(self.s_tok.numel())

    @property
    def n_p_tok(self) -> int:
        return int(self.p_tok.numel())

    @property
    def n_f_tok(self) -> int:
        return int(self.f_tok.numel())


# The planner's array work is numpy: single-threaded and cheap for a step's
# few hundred rows. torch's parallel CPU operators would leave their OpenMP
# team spinning on the host cores that the hybrid split's host share uses
# next. Results are torch tensors, as in the reference.


def _token_runs(starts: np.ndarray, counts: np.ndarray) -> np.ndarray:
    """The token indices start .. start + count - 1 of every run, in order."""
    counts = counts.astype(np.int64)
    total = int(counts.sum()) if counts.size else 0
    if total == 0:
        return np.zeros(0, dtype=np.int64)
    run = np.repeat(np.arange(counts.size), counts)
    first = np.cumsum(counts) - counts  # position of each run's first token
    return starts.astype(np.int64)[run] + (np.arange(total) - first[run])


def _offsets(counts: np.ndarray) -> np.ndarray:
    """[0, c0, c0 + c1, ...] as int32."""
    out = np.zeros(counts.size + 1, dtype=np.int32)
    if counts.size:
        out[1:] = np.cumsum(counts.astype(np.int64)).astype(np.int32)
    return out


def compact_rows(table, keep, subtract: int, pad_to: int = 1) -> torch.Tensor:
    """Per row, the kept entries moved to the front in their original order,
    minus `subtract`; every other entry 0. Width: the largest kept count
    (at least 1) rounded up to `pad_to` (fastdecode/plan.py:82-100). numpy
    or torch CPU arrays in, an int32 torch tensor out."""
    table = np.asarray(table)
    keep = np.asarray(keep, dtype=bool)
    rows, width_in = table.shape
    if table.size == 0:
        return torch.zeros(rows, pad_to, dtype=torch.int32)
    per_row = keep.sum(1)
    width = max(1, int(per_row.max()))
    width = -(-width // pad_to) * pad_to
    vals = table[keep].astype(np.int64) - subtract  # row-major: stable inside each row
    row = np.repeat(np.arange(rows, dtype=np.int64), per_row)
    pos = np.arange(vals.size, dtype=np.int64) - np.repeat(np.cumsum(per_row) - per_row, per_row)
    out = np.zeros(rows * width, dtype=np.int32)
    out[row * width + pos] = vals
    return torch.from_numpy(out.reshape(rows, width))


def build_host_plan(
    query_start_loc: torch.Tensor,  # [R + 1] (cpu)
    seq_lens: torch.Tensor,  # [R] (cpu), context + this step's tokens
    block_table: torch.Tensor,  # [R, W] int32 (cpu), W >= ceil(max seq / bs)
    slot_mapping: torch.Tensor,  # [>= n_tok] int64 (cpu)
    num_gpu_blocks: int,
    num_cpu_blocks: int,
    block_size: int,
) -> HostPlan | None:
    G, bs = int(num_gpu_blocks), int(block_size)
    qsl = query_start_loc.numpy().astype(np.int64)
    lens = seq_lens.numpy().astype(np.int64)
    qlen = qsl[1:] - qsl[:-1]
    prior = lens - qlen
    n_tok = int(qsl[-1]) if qsl.size else 0
    slots = slot_mapping.numpy()[:n_tok].astype(np.int64)

    R, W = block_table.shape
    col = np.arange(W, dtype=np.int64)
    # tokens held by column c of each row: bs for full blocks, the remainder
    # for the last one, 0 past the row's blocks
    held = np.clip(lens[:, None] - col[None, :] * bs, 0, bs)
    used = held > 0
    ids = block_table.numpy().astype(np.int64)
    in_host = used & (ids >= G)
    in_hbm = used & (ids < G)
    touches_host = in_host.any(1)
    host_slot = slots >= G * bs

    if not bool(touches_host.any()) and not bool(host_slot.any()):
        return None  # everything in HBM this step: plain paged attention

    if int(np.max(ids, where=in_host, initial=-1)) >= G + int(num_cpu_blocks):
        raise RuntimeError(
            "FastDecode: block id beyond GPU+CPU capacity; engine and worker "
            "disagree on FASTDECODE_CPU_BLOCKS / FASTDECODE_CPU_KV_GB"
        )

    active = qlen > 0
    is_s = active & touches_host & (qlen == 1)
    is_f = active & touches_host & (qlen > 1) & (prior == 0)
    if bool((active & touches_host & (qlen > 1) & (prior > 0)).any()):
        raise NotImplementedError(
            "FastDecode: a request with prior context is being extended by >1 token "
            "while part of its KV is on the CPU (chunked prefill or prefix-cache hit). "
            "Run with enable_prefix_caching=False and "
            "max_num_batched_tokens >= max_model_len."
        )
    is_p = active & ~touches_host

    gpu_slot_mapping = np.where(host_slot, -1, slots)
    host_slot_mapping = np.where(host_slot, slots - G * bs, -1)
    cpu_w_tok = np.nonzero(host_slot)[0]
    cpu_w_slot = slots[cpu_w_tok] - G * bs

    p_req = np.nonzero(is_p)[0]
    p_q = qlen[p_req]
    p_seqlens = lens[p_req].astype(np.int32)

    s_req = np.nonzero(is_s)[0]
    s_held = held[s_req]
    s_gpu_lens = (s_held * in_hbm[s_req]).sum(1).astype(np.int32)
    s_cpu_lens = (s_held * in_host[s_req]).sum(1).astype(np.int32)

    f_req = np.nonzero(is_f)[0]
    f_q = qlen[f_req]

    def t(a: np.ndarray) -> torch.Tensor:
        return torch.from_numpy(np.ascontiguousarray(a))

    return HostPlan(
        n_tok=n_tok,
        gpu_slot_mapping=t(gpu_slot_mapping.astype(np.int64)),
        cpu_w_tok=t(cpu_w_tok.astype(np.int64)),
        cpu_w_slot=t(cpu_w_slot.astype(np.int64)),
        p_tok=t(_token_runs(qsl[p_req], p_q)),
        p_cu=t(_offsets(p_q)),
        p_seqlens=t(p_seqlens),
        p_req=t(p_req.astype(np.int64)),
        p_max_q=int(p_q.max()) if p_q.size else 0,
        p_max_k=int(p_seqlens.max()) if p_seqlens.size else 0,
        s_tok=t(qsl[s_req]),
        s_gpu_bt=compact_rows(ids[s_req], in_hbm[s_req], 0, pad_to=GPU_TABLE_PAD),
        s_gpu_lens=t(s_gpu_lens),
        s_max_gpu_len=int(s_gpu_lens.max()) if s_gpu_lens.size else 0,
        s_gpu_tokens=int(s_gpu_lens.sum()),
        s_cpu_bt=compact_rows(ids[s_req], in_host[s_req], G),
        s_cpu_lens=t(s_cpu_lens),
        f_tok=t(_token_runs(qsl[f_req], f_q)),
        f_cu=t(_offsets(f_q)),
        f_max=int(f_q.max()) if f_q.size else 0,
        host_slot_mapping=t(host_slot_mapping.astype(np.int64)),
    )


@dataclass
class DevicePlan:
    """HostPlan with the tensors the GPU needs moved to the device
    (fastdecode/plan.py:202-221)."""

    host: HostPlan
    gpu_slot_mapping: torch.Tensor
    cpu_w_tok: torch.Tensor
    p_tok: torch.Tensor
    p_cu: torch.Tensor
    p_seqlens: torch.Tensor
    p_bt: torch.Tensor  # [nP, W] int32 rows of the batch block table
    s_tok: torch.Tensor
    # the S rows that hold HBM tokens (the reference hands only these to
    # FlashAttention; the HIP kernel here also accepts empty rows)
    s_gpu_rows: torch.Tensor  # [nG] int64, indices into the S rows
    s_gpu_cu: torch.Tensor  # arange(nG + 1) int32
    s_gpu_bt: torch.Tensor  # [nG, Wg] int32
    s_gpu_lens: torch.Tensor  # [nG] int32, all > 0
    f_tok: torch.Tensor
    f_cu: torch.Tensor
    # (no counterpart in the reference) every S row's tables on the device,
    # and the host-tier writes
    s_gpu_bt_all: torch.Tensor | None = None  # [nS, Wg] int32
    s_gpu_lens_all: torch.Tensor | None = None  # [nS] int32
    s_cpu_bt: torch.Tensor | None = None  # [nS, Wc] int32
    s_cpu_lens: torch.Tensor | None = None  # [nS] int32
    host_slot_mapping: torch.Tensor | None = None  # [n_tok] int64
    # scheduling order of the S rows for each tier's partial: longest first
    s_gpu_order: torch.Tensor | None = None  # [nS] int32
    s_cpu_order: torch.Tensor | None = None  # [nS] int32
    s_order: torch.Tensor | None = None  # [nS] int32, by both tiers' tokens (fused path)


def longest_first(lens: torch.Tensor) -> torch.Tensor:
    """int32 row permutation by decreasing length (stable)."""
    return torch.argsort(lens.to(torch.int64), descending=True, stable=True).to(torch.int32)


def to_device(hp: HostPlan, block_table_dev: torch.Tensor, device) -> DevicePlan:
    def d(t: torch.Tensor) -> torch.Tensor:
        return t.to(device, non_blocking=False)

    g_rows = (hp.s_gpu_lens > 0).nonzero().flatten()
    return DevicePlan(
        host=hp,
        gpu_slot_mapping=d(hp.gpu_slot_mapping),
        cpu_w_tok=d(hp.cpu_w_tok),
        p_tok=d(hp.p_tok),
        p_cu=d(hp.p_cu),
        p_seqlens=d(hp.p_seqlens),
        p_bt=(block_table_dev.index_select(0, d(hp.p_req)) if hp.p_req.numel()
              else block_table_dev[:0]),
        s_tok=d(hp.s_tok),
        s_gpu_rows=d(g_rows),
        s_gpu_cu=torch.arange(g_rows.numel() + 1, dtype=torch.int32, device=device),
        s_gpu_bt=d(hp.s_gpu_bt[g_rows]),
        s_gpu_lens=d(hp.s_gpu_lens[g_rows]),
        f_tok=d(hp.f_tok),
        f_cu=d(hp.f_cu),
        s_gpu_bt_all=d(hp.s_gpu_bt),
        s_gpu_lens_all=d(hp.s_gpu_lens),
        s_cpu_bt=d(hp.s_cpu_bt),
        s_cpu_lens=d(hp.s_cpu_lens),
        host_slot_mapping=d(hp.host_slot_mapping) if hp.host_slot_mapping is not None else None,
        s_gpu_order=d(longest_first(hp.s_gpu_lens)),
        s_cpu_order=d(longest_first(hp.s_cpu_lens)),
        s_order=d(longest_first(hp.s_gpu_lens + hp.s_cpu_lens)),
    )


@dataclass
class HostShare:
    """How one step's host-tier blocks are divided between the GPU (reading
    them over the link) and the host cores (reading their own DRAM)."""

    gpu_lens: torch.Tensor  # [n] int32 host-tier tokens the GPU reads: whole leading blocks
    cpu_bt: torch.Tensor  # [n, Wc] int32 the host cores' blocks: each row's trailing ones
    cpu_lens: torch.Tensor  # [n] int32


def share_host_blocks(host_bt: torch.Tensor, host_lens: torch.Tensor, block_size: int,
                      cpu_fraction: float) -> HostShare:
    """Gives the last round(cpu_fraction * nb) of each row's nb host-tier
    blocks (the partial last block among them; halves round up) to the host cores and the
    leading ones to the GPU. cpu_fraction 1 is the reference's split (the
    host cores compute the whole host-tier partial, fastdecode/backend.py:
    343-351); 0 leaves everything to the GPU. The GPU keeps its rows' table
    (its length covers only whole leading blocks); the host cores get each
    row's trailing ids shifted to column 0, zero padded. CPU tensors in and
    out."""
    if not 0.0 <= cpu_fraction <= 1.0:
        raise ValueError(f"cpu_fraction must be in [0, 1], got {cpu_fraction}")
    # one pass of host code in the library (fd_share_host_blocks): this runs
    # once per layer right before the host cores' share, so it stays cheap and
    # single-threaded (torch's parallel CPU operators leave their OpenMP team
    # spinning on the very cores that share needs)
    import ctypes

    from . import _lib

    bt = host_bt.contiguous() if host_bt.stride(-1) != 1 else host_bt
    lens = host_lens
    if lens.dtype != torch.int32 or not lens.is_contiguous():
        lens = lens.to(torch.int32).contiguous()
    n, W = bt.shape
    both = torch.empty(2, n, dtype=torch.int32)  # gpu_lens, cpu_lens
    gpu_lens, cpu_lens = both[0], both[1]
    cpu_bt = (torch.empty if W else torch.zeros)(n, max(W, 1), dtype=torch.int32)
    wc = ctypes.c_int32(0)
    _lib.check(_lib.load_lib().fd_share_host_blocks(
        bt.data_ptr(), bt.stride(0) if n else W, W, lens.data_ptr(), n, block_size,
        float(cpu_fraction), gpu_lens.data_ptr(), cpu_bt.data_ptr(), cpu_bt.stride(0),
        cpu_lens.data_ptr(), ctypes.byref(wc)))
    return HostShare(gpu_lens, cpu_bt[:, :max(wc.value, 1)], cpu_lens)


class ShareTuner:
    """Online balance of share_host_blocks' cpu_fraction between the host
    cores and the GPU. After each hybrid step, `update(gpu_finished_first)`
    moves the fraction one step toward the side that finished last: if the
    GPU's launch was already complete when the host cores finished, the host
    cores were the bottleneck and get less; otherwise more. The fraction
    settles where both finish together and then alternates within one step of
    it. No counterpart in the reference (its host cores take every host
    block)."""

    # start: near where the share settles at the vicuna-7b split shape on a
    # 16-core host (0.86-0.89: the host cores read their DRAM about seven
    # times as fast as the GPU reads the tier over PCIe)
    def __init__(self, start: float = 0.85, step: float = 0.01, lo: float = 0.05,
                 hi: float = 1.0) -> None:
        if not lo <= start <= hi:
            raise ValueError("start must lie in [lo, hi]")
        self.fraction = start
        self.step = step
        self.lo, self.hi = lo, hi

    def update(self, gpu_finished_first: bool | None) -> float:
        if gpu_finished_first is None:  # no finishing order seen (a split with no rows)
            return self.fraction
        delta = -self.step if gpu_finished_first else self.step
        self.fraction = min(self.hi, max(self.lo, self.fraction + delta))
        return self.fraction
