"""Seeded input generators shared by the tests, the smoke check and bench.py.

`rand_case` follows the reference's test generator _rand_case
(tests/test_cpu_kernel.py:14-35): q, K pool, V pool drawn as fp32 N(0,1) from
one seeded CPU generator and cast, lens uniform with lens[0] = max_len and
lens[1] = 1, and each row's blocks a slice of a random permutation of the pool
(a fresh permutation when the current one runs out).

The headline shapes' workloads (Workload, WORKLOADS, draw_lens_and_tables,
kv_pool, split_tiers, queries, kv_bytes) live in vllm_fastdecoder_amd.workloads,
which bench.py uses too; they are re-exported here.
"""

from __future__ import annotations

import torch

from vllm_fastdecoder_amd.workloads import (  # noqa: F401  (re-exported)
    WORKLOADS,
    Workload,
    draw_lens_and_tables,
    kv_bytes,
    kv_pool,
    queries,
    split_tiers,
)


def rand_case(n, H, KVH, D, BS, C, dtype, max_len, seed):
    g = torch.Generator().manual_seed(seed)
    q = torch.randn(n, H, D, generator=g).to(dtype)
    k_cache = torch.randn(C, KVH, BS, D, generator=g).to(dtype)
    v_cache = torch.randn(C, KVH, BS, D, generator=g).to(dtype)
    lens = torch.randint(0, max_len + 1, (n,), generator=g, dtype=torch.int32)
    lens[0] = max_len
    if n > 1:
        lens[1] = 1
    W = (max_len + BS - 1) // BS
    perm = torch.randperm(C, generator=g)
    bt = torch.zeros(n, W, dtype=torch.int32)
    pos = 0
    for i in range(n):
        nb = (int(lens[i]) + BS - 1) // BS
        if pos + nb > C:
            perm = torch.randperm(C, generator=g)
            pos = 0
        bt[i, :nb] = perm[pos : pos + nb].to(torch.int32)
        pos += nb
    return q, k_cache, v_cache, bt, lens


def tensor_digest(*tensors: torch.Tensor) -> str:
    """sha256 over the raw bytes of CPU tensors (detects generator drift)."""
    import hashlib

    h = hashlib.sha256()
    for t in tensors:
        t = t.detach().cpu().contiguous()
        h.update(str(t.dtype).encode())
        h.update(str(tuple(t.shape)).encode())
        h.update(t.view(torch.uint8).numpy().tobytes() if t.numel() else b"")
    return h.hexdigest()


