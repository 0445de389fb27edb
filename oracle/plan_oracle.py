"""Plain-Python restatement of the reference's per-step planner
(fastdecode/plan.py:103-199, with _compact :82-100, _ranges :65-72, _cu :75-79).

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py). Row-by-row loops over
Python ints; returns a dict of lists so comparisons are exact.

Pinned by the reference's planner known-answer tests
(tests/test_plan_and_forward.py:199-227), transcribed as data into
tests/golden/plan_kats.json, and by invariants checked in tests/test_plan.py
(per-tier token counts add up to the sequence length, the compacted tables
hold exactly the tier's ids in sequence order, padding is zero and the HBM
width a multiple of 16, every slot lands in exactly one tier).
"""

from __future__ import annotations


class PlanError(Exception):
    pass


def plan_oracle(qsl, seq_lens, block_table, slots, G, C, bs):
    """qsl [R+1], seq_lens [R], block_table [R][W], slots [>= n_tok]: lists of
    ints. Returns None (no host tier involved) or a dict of lists."""
    R = len(seq_lens)
    W = len(block_table[0]) if R else 0
    n_tok = qsl[-1] if qsl else 0
    slots = list(slots[:n_tok])

    rows = []
    any_host_block = False
    max_host_id = -1
    for r in range(R):
        L = seq_lens[r]
        nb = (L + bs - 1) // bs if L > 0 else 0
        blocks = []
        for c in range(min(nb, W)):
            b = block_table[r][c]
            ntok = bs if c < nb - 1 else L - (nb - 1) * bs
            blocks.append((b, ntok))
        host = [(b, t) for b, t in blocks if b >= G]
        if host:
            any_host_block = True
            max_host_id = max(max_host_id, max(b for b, _ in host))
        rows.append((blocks, host))

    host_slot = [s >= G * bs for s in slots]
    if not any_host_block and not any(host_slot):
        return None
    if any_host_block and max_host_id >= G + C:
        raise PlanError("block id beyond capacity")

    cls = []
    for r in range(R):
        ql = qsl[r + 1] - qsl[r]
        prior = seq_lens[r] - ql
        touches = bool(rows[r][1])
        if ql <= 0:
            cls.append("-")
        elif not touches:
            cls.append("P")
        elif ql == 1:
            cls.append("S")
        elif prior == 0:
            cls.append("F")
        else:
            raise NotImplementedError("chunked continuation touching the host tier")

    out = {
        "n_tok": n_tok,
        "gpu_slot_mapping": [-1 if h else s for s, h in zip(slots, host_slot)],
        "host_slot_mapping": [s - G * bs if h else -1 for s, h in zip(slots, host_slot)],
        "cpu_w_tok": [j for j, h in enumerate(host_slot) if h],
        "cpu_w_slot": [s - G * bs for s, h in zip(slots, host_slot) if h],
    }

    p_req = [r for r in range(R) if cls[r] == "P"]
    out["p_req"] = p_req
    out["p_tok"] = [t for r in p_req for t in range(qsl[r], qsl[r + 1])]
    out["p_cu"] = [0]
    for r in p_req:
        out["p_cu"].append(out["p_cu"][-1] + qsl[r + 1] - qsl[r])
    out["p_seqlens"] = [seq_lens[r] for r in p_req]
    out["p_max_q"] = max((qsl[r + 1] - qsl[r] for r in p_req), default=0)
    out["p_max_k"] = max(out["p_seqlens"], default=0)

    s_req = [r for r in range(R) if cls[r] == "S"]
    out["s_tok"] = [qsl[r] for r in s_req]
    gpu_lists, cpu_lists = [], []
    for r in s_req:
        blocks = rows[r][0]
        gpu_lists.append([(b, t) for b, t in blocks if b < G])
        cpu_lists.append([(b - G, t) for b, t in blocks if b >= G])
    out["s_gpu_lens"] = [sum(t for _, t in lst) for lst in gpu_lists]
    out["s_cpu_lens"] = [sum(t for _, t in lst) for lst in cpu_lists]
    out["s_max_gpu_len"] = max(out["s_gpu_lens"], default=0)

    def table(lists, pad_to):
        if not lists or W == 0:
            return [[0] * pad_to for _ in lists]
        width = max(1, max(len(lst) for lst in lists))
        width = ((width + pad_to - 1) // pad_to) * pad_to
        return [[b for b, _ in lst] + [0] * (width - len(lst)) for lst in lists]

    out["s_gpu_bt"] = table(gpu_lists, 16)
    out["s_cpu_bt"] = table(cpu_lists, 1)

    f_req = [r for r in range(R) if cls[r] == "F"]
    out["f_tok"] = [t for r in f_req for t in range(qsl[r], qsl[r + 1])]
    out["f_cu"] = [0]
    for r in f_req:
        out["f_cu"].append(out["f_cu"][-1] + qsl[r + 1] - qsl[r])
    out["f_max"] = max((qsl[r + 1] - qsl[r] for r in f_req), default=0)
    out["classes"] = cls
    return out
