"""Writes tests/golden/ref_decode_attn.npz: outputs of the reference's own
host-tier kernel (fastdecode/csrc/cpu_attn.cpp decode_attn, compiled from its
source by oracle/Makefile into oracle/_ref) on seeded cases of its test grid
(tests/test_cpu_kernel.py:38-57 shapes).

Inputs are not stored: tests regenerate them with tests.cases.rand_case and
compare a sha256 digest, so only the small outputs are committed.

    python tests/golden/make_golden.py
"""

from __future__ import annotations

import math
import sys
from pathlib import Path

import numpy as np
import torch

ROOT = Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))

import oracle  # noqa: E402
from tests import cases  # noqa: E402

CASES = [
    # name, n, H, KVH, D, BS, C, max_len, seed, dtype code, empty row
    ("f16_h8_kv2_d128", 7, 8, 2, 128, 16, 64, 93, 136, 0, 3),
    ("bf16_h4_kv1_d64", 7, 4, 1, 64, 16, 64, 93, 68, 1, 3),
    ("f32_h8_kv8_d72", 7, 8, 8, 72, 16, 64, 93, 80, 2, 3),
    ("f16_h32_kv32_d128_long", 3, 32, 32, 128, 16, 96, 500, 5, 0, -1),
    ("bf16_h32_kv8_d128", 4, 32, 8, 128, 16, 64, 300, 6, 1, 2),
]
DT = {0: torch.float16, 1: torch.bfloat16, 2: torch.float32}


def main() -> None:
    oracle.build()
    ext = oracle.ref_ext()
    if ext is None:
        raise SystemExit("reference build missing (needs /root/reference)")
    arrays = {}
    for name, n, H, KVH, D, BS, C, max_len, seed, dt, empty in CASES:
        q, kc, vc, bt, lens = cases.rand_case(n, H, KVH, D, BS, C, DT[dt], max_len, seed)
        if empty >= 0:
            lens[empty] = 0
        out = torch.empty_like(q)
        lse = torch.empty(H, n, dtype=torch.float32)
        ext.decode_attn(q, kc, vc, bt, lens, 1.0 / math.sqrt(D), out, lse)
        arrays[f"{name}__meta"] = np.array([n, H, KVH, D, BS, C, max_len, seed, dt, empty], np.int64)
        arrays[f"{name}__digest"] = np.array(cases.tensor_digest(q, kc, vc, bt, lens))
        arrays[f"{name}__out"] = out.float().numpy()
        arrays[f"{name}__lse"] = lse.numpy()
    dst = Path(__file__).resolve().parent / "ref_decode_attn.npz"
    np.savez_compressed(dst, **arrays)
    print(f"wrote {dst} ({dst.stat().st_size} bytes)")


if __name__ == "__main__":
    main()
