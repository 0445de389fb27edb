"""Seeded synthetic decode-attention workloads: the shapes the library is
measured on (bench.py) and tested at full size (tests/).

  "correctness"  n=8, 32/32 heads, D=128, BS=16, fp16, pool 1024 blocks,
                 L ~ U[128, 1024]
  "vicuna7b"     n=128, 32/32 heads, D=128, BS=16, fp16, L ~ U[256, 2048],
                 pool = sum of the rows' blocks
  "llama3_8b"    n=256, 32/8 heads (GQA 4), D=128, BS=16, bf16,
                 L ~ U[1024, 4096], pool = sum of the rows' blocks

Large pools are drawn on the GPU with a seeded generator (CPU draws of
gigabytes would take minutes); everything else is drawn on the CPU.
"""

from __future__ import annotations

import math
from dataclasses import dataclass

import torch


@dataclass
class Workload:
    name: str
    n: int
    H: int
    KVH: int
    D: int
    BS: int
    dtype: torch.dtype
    lo: int
    hi: int
    pool: int | None  # fixed pool size, or None = sum of the rows' blocks
    seed: int

    @property
    def scale(self) -> float:
        return 1.0 / math.sqrt(self.D)


WORKLOADS = {
    "correctness": Workload("correctness", 8, 32, 32, 128, 16, torch.float16, 128, 1024, 1024, 0),
    "vicuna7b": Workload("vicuna7b", 128, 32, 32, 128, 16, torch.float16, 256, 2048, None, 2),
    "llama3_8b": Workload("llama3_8b", 256, 32, 8, 128, 16, torch.bfloat16, 1024, 4096, None, 3),
}


def draw_lens_and_tables(w: Workload):
    """lens [n] int32 and a block table [n, W] int32 (W = ceil(hi / BS)); each
    row's blocks are distinct ids of the pool. Returns (lens, bt, pool)."""
    g = torch.Generator().manual_seed(w.seed)
    lens = torch.randint(w.lo, w.hi + 1, (w.n,), generator=g, dtype=torch.int32)
    nb = (lens + w.BS - 1) // w.BS
    W = (w.hi + w.BS - 1) // w.BS
    pool = w.pool if w.pool is not None else int(nb.sum())
    bt = torch.zeros(w.n, W, dtype=torch.int32)
    if w.pool is None:
        perm = torch.randperm(pool, generator=g).to(torch.int32)
        pos = 0
        for i in range(w.n):
            k = int(nb[i])
            bt[i, :k] = perm[pos : pos + k]
            pos += k
    else:
        for i in range(w.n):
            k = int(nb[i])
            bt[i, :k] = torch.randperm(pool, generator=g)[:k].to(torch.int32)
    return lens, bt, pool


def kv_pool(w: Workload, pool: int, layout: str, device, seed_offset: int = 0):
    """K and V caches of `pool` blocks with N(0,1) values.

    layout "host": separate [pool, KVH, BS, D] tensors (the reference's host
    tier). layout "vllm": one [pool, BS, KVH, 2D] tensor whose K / V halves
    are returned as [pool, BS, KVH, D] views (vLLM's HBM tier).
    """
    g = torch.Generator(device=device).manual_seed(1000 + w.seed + seed_offset)
    if layout == "host":
        k = torch.randn(pool, w.KVH, w.BS, w.D, generator=g, device=device, dtype=torch.float32).to(w.dtype)
        v = torch.randn(pool, w.KVH, w.BS, w.D, generator=g, device=device, dtype=torch.float32).to(w.dtype)
        return k, v, None
    if layout == "vllm":
        kv = torch.empty(pool, w.BS, w.KVH, 2 * w.D, dtype=w.dtype, device=device)
        # fill in slabs to bound the fp32 temporary
        step = max(1, (1 << 28) // (w.BS * w.KVH * 2 * w.D))
        for s in range(0, pool, step):
            e = min(pool, s + step)
            kv[s:e] = torch.randn(e - s, w.BS, w.KVH, 2 * w.D, generator=g, device=device).to(w.dtype)
        return kv[..., : w.D], kv[..., w.D :], kv
    raise ValueError(layout)


def split_tiers(w: Workload, lens: torch.Tensor, bt: torch.Tensor, dev):
    """The split-run layout of a workload: the last ceil(0.6 * nb) blocks of
    each row in pinned host memory [C, KVH, BS, D], the rest in the HBM
    tier's vLLM layout [G, BS, KVH, 2D], each tier's table compacted in
    sequence order (the planner's s_gpu_bt / s_cpu_bt) and its token counts
    (HBM blocks are whole; the host tier holds the partial last block). A
    row's blocks in each tier are scattered: consecutive runs of a seeded
    random permutation of that tier's ids, as the all-HBM run draws them and
    as an allocator that reuses freed blocks hands them out. Data N(0,1),
    seeded. bt only gives the table width."""
    from vllm_fastdecoder_amd.pinned import pinned_empty

    nb = (lens + w.BS - 1) // w.BS
    n_host = torch.ceil(nb.double() * 0.6).to(torch.int32)
    n_hbm = nb - n_host
    W = bt.shape[1]
    bt_g = torch.zeros(w.n, W, dtype=torch.int32)
    bt_c = torch.zeros(w.n, W, dtype=torch.int32)
    len_g = (n_hbm * w.BS).to(torch.int32)
    len_c = (lens - len_g).to(torch.int32)
    G = int(n_hbm.sum())
    C = int(n_host.sum())
    g = torch.Generator().manual_seed(7000 + w.seed)
    perm_g = torch.randperm(max(G, 1), generator=g).to(torch.int32)
    perm_c = torch.randperm(max(C, 1), generator=g).to(torch.int32)
    pg = pc = 0
    for i in range(w.n):
        a, b = int(n_hbm[i]), int(n_host[i])
        bt_g[i, :a] = perm_g[pg : pg + a]
        bt_c[i, :b] = perm_c[pc : pc + b]
        pg += a
        pc += b
    kc_g, vc_g, kv = kv_pool(w, max(G, 1), "vllm", dev)
    hk = pinned_empty((max(C, 1), w.KVH, w.BS, w.D), w.dtype)
    hv = pinned_empty((max(C, 1), w.KVH, w.BS, w.D), w.dtype)
    # fill the host tier in slabs (N(0,1), seeded)
    gen = torch.Generator(device=dev).manual_seed(4242)
    slab = 2048
    for t in (hk, hv):
        for s in range(0, C, slab):
            e = min(C, s + slab)
            t[s:e].copy_(torch.randn(e - s, w.KVH, w.BS, w.D, generator=gen,
                                     device=dev).to(w.dtype).cpu())
    return dict(bt_g=bt_g, bt_c=bt_c, len_g=len_g, len_c=len_c, G=G, C=C, kc_g=kc_g, vc_g=vc_g,
                kv=kv, hk=hk, hv=hv)


def queries(w: Workload, device) -> torch.Tensor:
    g = torch.Generator().manual_seed(500 + w.seed)
    return torch.randn(w.n, w.H, w.D, generator=g).to(w.dtype).to(device)


def kv_bytes(lens: torch.Tensor, KVH: int, D: int, elt: int) -> int:
    """Algorithmic K+V bytes of one partial: 2 * KVH * D * elt per token."""
    return int(lens.clamp(min=0).sum()) * 2 * KVH * D * elt
