"""Wait states between a matrix-core instruction and the first read of its
result, over every control-flow path of a kernel's gfx950 assembly.

A VALU (or memory) instruction that reads an MFMA's destination registers
must issue enough cycles after the MFMA; the compiler pads straight-line
code with s_nop for that. Across a conditional branch its count has been
found short: in the two-column-group decode_mm_kernel the scores MFMA of the
second group reached the v_mul that scales them after 1-5 wait states on the
path that skips the short-block masking (8 on every straight-line path), and
the kernel read stale scores. This module measures, for each MFMA, the
fewest wait states before a read of its result along any path, counting one
per instruction and k + 1 per s_nop k, separately for paths that take a
branch and for straight-line ones.
"""

from __future__ import annotations

import re
from dataclasses import dataclass

_REG = re.compile(r"\b([va])\[(\d+):(\d+)\]|\b([va])(\d+)\b")
_STORES = ("global_store", "buffer_store", "ds_write", "ds_store", "scratch_store", "flat_store")


def _regs(text: str) -> set:
    out = set()
    for m in _REG.finditer(text):
        if m.group(1):
            out.update((m.group(1), r) for r in range(int(m.group(2)), int(m.group(3)) + 1))
        else:
            out.add((m.group(4), int(m.group(5))))
    return out


def _reads(op: str, args: str) -> set:
    """Registers an instruction reads (a store reads all its operands; any
    other instruction all but its first, the destination)."""
    if op.startswith(_STORES):
        return _regs(args)
    return _regs(args.split(",", 1)[1]) if "," in args else set()


def kernels(asm: str):
    """(name, [(mnemonic, operands)], {label: index}) per kernel."""
    cur, ins, labels = None, [], {}
    for line in asm.splitlines():
        m = re.match(r"^(_Z\w+):", line)
        if m:
            cur, ins, labels = m.group(1), [], {}
            continue
        if cur is None:
            continue
        if line.startswith(".Lfunc_end"):
            yield cur, ins, labels
            cur = None
            continue
        text = line.split(";")[0].rstrip()
        if not text.strip():
            continue
        if not text.startswith(("\t", " ")) and text.endswith(":"):
            labels[text[:-1]] = len(ins)
            continue
        text = text.strip()
        if text.startswith("."):
            continue
        parts = text.split(None, 1)
        ins.append((parts[0], parts[1] if len(parts) > 1 else ""))


@dataclass
class Gap:
    kernel: str
    mfma: str
    reader: str
    wait_states: int
    via_branch: bool


def mfma_read_gaps(name, ins, labels, horizon: int = 32):
    """For each MFMA of a kernel, the fewest wait states before a
    non-MFMA instruction reads its destination, along straight-line paths and
    along paths through a branch (None where no read comes within horizon)."""
    gaps = []
    for i, (op, args) in enumerate(ins):
        if not op.startswith("v_mfma"):
            continue
        dst = _regs(args.split(",", 1)[0])
        best = {False: None, True: None}
        stack = [(i + 1, 0, False)]
        seen = {}
        while stack:
            j, w, br = stack.pop()
            if w >= horizon or j >= len(ins) or seen.get((j, br), horizon) <= w:
                continue
            seen[(j, br)] = w
            o, a = ins[j]
            if o.startswith("v_mfma"):
                if _regs(a.split(",", 1)[0]) & dst and not (_reads(o, a) & dst):
                    continue  # overwritten before any other read on this path
                stack.append((j + 1, w + 1, br))
                continue
            if not o.startswith("s_") and _reads(o, a) & dst:
                if best[br] is None or w < best[br][0]:
                    best[br] = (w, o)
                continue
            if o == "s_endpgm":
                continue
            cost = int(a.strip(), 0) + 1 if o == "s_nop" else 1
            if o == "s_branch":
                stack.append((labels[a.strip()], w + cost, True))
            elif o.startswith("s_cbranch"):
                stack.append((labels[a.strip()], w + cost, True))
                stack.append((j + 1, w + cost, br))
            else:
                stack.append((j + 1, w + cost, br))
        for br, hit in best.items():
            if hit is not None:
                gaps.append(Gap(name, op, hit[1], hit[0], br))
    return gaps
