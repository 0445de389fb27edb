"""Continuous-batching simulation of the split decode path on the GPU.

Protocol of the reference's GPU self-test (scripts/gpu_selftest.py:39-282),
at vicuna-7b head shapes: requests arrive (Poisson, `arrivals` per step),
prefill once (write-only here: prefill attention is not on the decode path),
then decode one token per step until their output budget is spent, and free
their blocks. Allocation is GPU-first from ids [1, G) (block 0 is vLLM's null
block), then host ids [G, G+C); freed HBM blocks are reused first (LIFO),
freed host blocks last (FIFO) (gpu_selftest.py:124-136, patches.py:41-48). A
request that needs a block when none is free is dropped (the stand-in for
preemption, gpu_selftest.py:149-154).

Every step runs twice on the same q/k/v:
  split       G HBM blocks + C pinned host blocks, through the planner and
              SplitDecodeImpl._forward_split (HIP kernels for both tiers);
  monolithic  one HBM pool of G + C blocks, the same cache writes, one paged
              decode over all of each row's blocks (fp32 output).
Both start from different random garbage, so any read of an unwritten slot
shows. A host copy of the monolithic pool (same garbage) receives the same
writes through the oracle's slot write. Checked per step: every decode row of
the split path against the monolithic output; every slot written this step
bit-exact in its tier, in the monolithic pool and in the host copy; every
`oracle_every` steps every decode row of both paths against the float64
oracle over the host copy. Reported besides:
the split path's wall time per step (planning, KV writes and attention, with
the prefill rows' attention stubbed as below), `split_path_ms`.
"""

from __future__ import annotations

import math
import random
import time
from types import SimpleNamespace

import numpy as np
import torch

import oracle
from vllm_fastdecoder_amd import backend, ops, plan, state
from vllm_fastdecoder_amd.pinned import pinned_empty


class _SimOps(backend.HipOps):
    """HIP decode partials; the P rows' call computes its one-token rows with
    the same paged decode kernel and leaves multi-token (prefill) rows zero,
    F rows (prefills) are not computed -- both unchecked prefill work."""

    @staticmethod
    def fa(q, k, v, cu_seqlens_q=None, max_seqlen_q=1, seqused_k=None, max_seqlen_k=None,
           softmax_scale=None, causal=False, block_table=None, return_softmax_lse=False, **kw):
        if not causal and max_seqlen_q == 1 and block_table is not None:
            return backend.HipOps.fa(q=q, k=k, v=v, cu_seqlens_q=cu_seqlens_q, max_seqlen_q=1,
                                     seqused_k=seqused_k, softmax_scale=softmax_scale,
                                     block_table=block_table,
                                     return_softmax_lse=return_softmax_lse)
        out = torch.zeros_like(q)
        if block_table is None:
            return out
        qlens = (cu_seqlens_q[1:] - cu_seqlens_q[:-1]).cpu()
        rows = (qlens == 1).nonzero().flatten()
        if rows.numel():
            rows_d = rows.to(q.device)
            tok = cu_seqlens_q[:-1].to(torch.int64)[rows_d]
            o, _ = ops.paged_decode(q.index_select(0, tok), k, v,
                                    block_table.index_select(0, rows_d).contiguous(),
                                    seqused_k.index_select(0, rows_d).contiguous(), softmax_scale)
            out.index_copy_(0, tok, o)
        return out


def run_simulation(steps: int = 300, seed: int = 4, device=None, G: int = 256, C: int = 2048,
                   H: int = 32, KVH: int = 32, D: int = 128, BS: int = 16,
                   dtype: torch.dtype = torch.float16, arrivals: float = 4.0,
                   prompt: tuple[int, int] = (64, 512), output: tuple[int, int] = (32, 512),
                   tol: float = 2e-3, oracle_every: int = 10, fused: bool = True,
                   planner: str = "host", cpu_fraction: float = 0.0) -> dict:
    dev = device or torch.device("cuda", 0)
    rng = random.Random(seed)
    nrng = np.random.default_rng(seed)
    torch.manual_seed(seed)
    scale = 1.0 / math.sqrt(D)
    name = "model.layers.0.self_attn.attn"
    layer = SimpleNamespace(layer_name=name, _k_scale=None, _v_scale=None)

    # split tiers (garbage-filled) and the unified pool (different garbage)
    phys = (torch.randn(G, BS, KVH, 2 * D, device=dev) * 10).to(dtype)
    kv_cache = phys.permute(0, 2, 1, 3)  # logical [B, KVH, BS, 2D]
    store = state.HostKVStore(G, C, BS, KVH, D, dtype)
    for t in ("k", "v"):
        buf = pinned_empty((C, KVH, BS, D), dtype)
        gen = torch.Generator(device=dev).manual_seed(seed + (1 if t == "k" else 2))
        for s0 in range(0, C, 512):
            s1 = min(C, s0 + 512)
            buf[s0:s1].copy_((torch.randn(s1 - s0, KVH, BS, D, generator=gen, device=dev) * 10)
                             .to(dtype).cpu())
        getattr(store, t)[name] = buf
    prev_store, prev_ops = state.STORE, backend.OPS
    state.STORE = store
    backend.OPS = _SimOps
    uphys = (torch.randn(G + C, BS, KVH, 2 * D, device=dev) * 10).to(dtype)
    ukc, uvc = uphys[..., :D], uphys[..., D:]
    # the oracle's copy of the monolithic pool: same garbage, same writes
    mirror = uphys.cpu()
    mk, mv = mirror[..., :D], mirror[..., D:]
    m_strides = (mirror.stride(0), mirror.stride(1), mirror.stride(2))
    impl = backend.SplitDecodeImpl(H, KVH, D, scale, fused_split=fused, cpu_fraction=cpu_fraction,
                                   hybrid_min_host_bytes=0,
                                   device_step_hybrid=cpu_fraction != 0.0)

    free_gpu = list(range(1, G))
    free_host = list(range(G, G + C))

    def alloc():
        if free_gpu:
            return free_gpu.pop(0)
        if free_host:
            return free_host.pop(0)
        return None

    def release(blocks):
        free_gpu[:0] = [b for b in blocks if b < G]
        free_host.extend(b for b in blocks if b >= G)

    running = []
    stats = {"failures": [], "split_steps": 0, "decode_rows": 0, "split_rows": 0,
             "host_tokens": 0, "max_err_vs_mono": 0.0, "max_err_vs_f64": 0.0, "dropped": 0,
             "device_planned_steps": 0, "rows_vs_f64": 0}
    plan_errors = torch.zeros(1, dtype=torch.int32, device=dev)
    step_ms = []
    try:
        for step in range(steps):
            rows = []
            for r in list(running):
                if r["L"] % BS == 0:
                    b = alloc()
                    if b is None:
                        running.remove(r)
                        release(r["blocks"])
                        stats["dropped"] += 1
                        continue
                    r["blocks"].append(b)
                rows.append((r, r["L"], 1))
            for _ in range(int(nrng.poisson(arrivals))):
                P = rng.randint(*prompt)
                need = (P + BS - 1) // BS
                if need > len(free_gpu) + len(free_host):
                    stats["dropped"] += 1
                    continue
                r = {"blocks": [alloc() for _ in range(need)], "L": 0,
                     "left": rng.randint(*output)}
                running.append(r)
                rows.append((r, 0, P))
            if not rows:
                continue
            rng.shuffle(rows)
            R = len(rows)
            qlens = [ql for _, _, ql in rows]
            seqs = [ctx + ql for _, ctx, ql in rows]
            T = sum(qlens)
            W = max(len(r["blocks"]) for r, _, _ in rows) + 2
            bt = torch.zeros(R, W, dtype=torch.int32)
            slots = []
            for i, (r, ctx, ql) in enumerate(rows):
                bl = r["blocks"]
                bt[i, : len(bl)] = torch.tensor(bl, dtype=torch.int32)
                bt[i, len(bl):] = torch.randint(0, G + C, (W - len(bl),), dtype=torch.int32)
                for p in range(ctx, ctx + ql):
                    slots.append(bl[p // BS] * BS + p % BS)
            qsl = torch.zeros(R + 1, dtype=torch.int32)
            qsl[1:] = torch.cumsum(torch.tensor(qlens), 0)
            seq = torch.tensor(seqs, dtype=torch.int32)
            slots = torch.tensor(slots, dtype=torch.int64)
            # q/k/v as strided views of one fused qkv tensor, plus padding rows
            Tp = T + rng.randint(0, 7)
            qkv = torch.randn(Tp, (H + 2 * KVH) * D, device=dev).to(dtype)
            q, k, v = qkv.split([H * D, KVH * D, KVH * D], dim=-1)
            q = (q * 2).view(Tp, H, D)
            k = k.view(Tp, KVH, D)
            v = v.view(Tp, KVH, D)
            bt_d, slots_d = bt.to(dev), slots.to(dev)

            # ---- split path (timed from planning to its last kernel)
            out_split = torch.full((Tp, H, D), float("nan"), dtype=dtype, device=dev)
            torch.cuda.synchronize(dev)
            t_split = time.perf_counter()
            ds = (backend.build_device_step(qsl, seq, bt_d, slots_d, R, store, dev)
                  if planner == "device" else None)
            dp = backend.build_split_plan(qsl, seq, bt_d, slots_d, R, store, dev) \
                if ds is None else None
            if ds is not None:
                stats["device_planned_steps"] += 1
                impl._forward_device(layer, q, k, v, kv_cache, ds, out_split)
                plan_errors += ds.errors
            elif dp is None:
                ops.reshape_and_cache(k, v, kv_cache.transpose(1, 2)[..., :D],
                                      kv_cache.transpose(1, 2)[..., D:], slots_d)
                dec = [i for i in range(R) if qlens[i] == 1]
                if dec:
                    tok = qsl[:-1][dec].to(torch.int64).to(dev)
                    o, _ = ops.paged_decode(q.index_select(0, tok), phys[..., :D], phys[..., D:],
                                            bt_d[dec].contiguous(), seq[dec].to(dev), scale)
                    out_split.index_copy_(0, tok, o)
            else:
                stats["split_steps"] += 1
                stats["split_rows"] += dp.host.n_s
                stats["host_tokens"] += int(dp.host.s_cpu_lens.sum())
                impl._forward_split(layer, q, k, v, kv_cache, dp, out_split)

            torch.cuda.synchronize(dev)
            step_ms.append((time.perf_counter() - t_split) * 1e3)

            # ---- monolithic path: same writes into one pool, fp32 decode
            ops.reshape_and_cache(k, v, ukc, uvc, slots_d)
            st_w, _ = oracle.cache_write(k[:T], v[:T], mk, mv, m_strides, G + C, BS, slots, True)
            if st_w != 0:
                stats["failures"].append(f"step {step}: slot past the pool")
            dec = [i for i in range(R) if qlens[i] == 1]
            stats["decode_rows"] += len(dec)
            if dec:
                tok = qsl[:-1][dec].to(torch.int64)
                mono = torch.empty(len(dec), H, D, dtype=torch.float32, device=dev)
                ops.paged_decode(q.index_select(0, tok.to(dev)), ukc, uvc, bt_d[dec].contiguous(),
                                 seq[dec].to(dev), scale, out=mono)
                got = out_split.index_select(0, tok.to(dev)).float()
                err = float((got - mono).abs().max())
                stats["max_err_vs_mono"] = max(stats["max_err_vs_mono"], err)
                if not err <= tol:
                    stats["failures"].append(f"step {step}: decode rows off by {err:.3g}")
                if oracle_every and step % oracle_every == 0:
                    # every decode row, both paths, against float64 attention
                    # over the oracle's own copy of the pool
                    o64, _, st = oracle.decode_attn_f64(
                        q.index_select(0, tok.to(dev)).cpu(), mk, mv, oracle.VLLM_DIMS,
                        bt[dec].contiguous(), seq[dec], scale)
                    e64 = float((got.double().cpu() - o64).abs().max())
                    em = float((mono.double().cpu() - o64).abs().max())
                    stats["max_err_vs_f64"] = max(stats["max_err_vs_f64"], e64, em)
                    stats["rows_vs_f64"] += len(dec)
                    if st != 0 or not e64 <= tol or not em <= 2e-3:
                        stats["failures"].append(
                            f"step {step}: vs f64: split {e64:.3g}, monolithic {em:.3g}")

            # ---- every slot written this step holds the oracle's KV in its
            #      tier and in the monolithic pool
            sb, so = slots // BS, slots % BS
            if not (torch.equal(ukc[sb.to(dev), so.to(dev)].cpu(), mk[sb, so]) and
                    torch.equal(uvc[sb.to(dev), so.to(dev)].cpu(), mv[sb, so])):
                stats["failures"].append(f"step {step}: monolithic KV write mismatch")
            g = sb < G
            if bool(g.any()):
                gi = g.nonzero().flatten()
                a, b_ = sb[gi], so[gi]
                pa = phys[a.to(dev), b_.to(dev)].cpu()
                if not (torch.equal(pa[..., :D], mk[a, b_]) and torch.equal(pa[..., D:], mv[a, b_])):
                    stats["failures"].append(f"step {step}: HBM-tier KV write mismatch")
            if bool((~g).any()):
                hi = (~g).nonzero().flatten()
                hk = store.k[name][sb[hi] - G, :, so[hi]]
                hv = store.v[name][sb[hi] - G, :, so[hi]]
                if not (torch.equal(hk, mk[sb[hi], so[hi]]) and torch.equal(hv, mv[sb[hi], so[hi]])):
                    stats["failures"].append(f"step {step}: host-tier KV write mismatch")

            for r, ctx, ql in rows:
                r["L"] = ctx + ql
                r["left"] -= 1
                if r["left"] <= 0 and r in running:
                    running.remove(r)
                    release(r["blocks"])
        torch.cuda.synchronize()
        if step_ms:  # wall time of the split path per step (planning, KV writes, attention)
            t = np.array(step_ms[10:] or step_ms)  # the first steps warm up
            stats["split_path_ms"] = {"median": round(float(np.median(t)), 3),
                                      "mean": round(float(t.mean()), 3),
                                      "p90": round(float(np.percentile(t, 90)), 3)}
        if int(plan_errors.item()):
            stats["failures"].append(f"device planner counted {int(plan_errors.item())} errors")
    finally:
        state.STORE = prev_store
        backend.OPS = prev_ops
    return stats
