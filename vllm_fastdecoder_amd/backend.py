"""Split decode path on MI355X: the GPU-op seam and the per-layer orchestration.

Mirrors the reference backend's hot path (fastdecode/backend.py) without
vLLM's base classes:

  * `HipOps` / `OPS` -- the seam of backend.py:42-64 (`fa`, `reshape_and_cache`,
    `merge`, `event`), routed to libfdattn. `fa` implements the paged decode
    form the split path uses (one query token per row, block table,
    return_softmax_lse); prefill forms raise NotImplementedError (FlashAttention
    prefill is not on this path). `split_decode` (no counterpart in the
    reference) is the fused form of the S rows' two partials and their merge. Tests swap
    OPS the way the reference's tests do (tests/test_plan_and_forward.py:106-113).
  * `build_split_plan` -- FastDecodeMetadataBuilder.build (backend.py:140-178):
    one device-to-host copy of the step's block table and slots, the host
    planner, then the device plan.
  * `SplitDecodeImpl._forward_split` -- FastDecodeImpl._forward_split
    (backend.py:257-357). The structure is the reference's. The host tier's
    KV rows are written into the pinned tier by the GPU (no staging copy);
    its partial is shared between the host cores (each row's trailing host
    blocks, as in the reference) and the GPU reading the rest zero-copy, the
    share balanced online (`cpu_fraction="auto"`, the default); a layer with
    little host-tier KV, or `cpu_fraction=0`, leaves the whole host tier to
    the GPU with no host wait.
  * `build_device_step` / `SplitDecodeImpl._forward_device` -- no
    counterpart in the reference: the same step planned on the GPU (fd_plan_tiers), with no
    device-to-host copy, for steps whose prefill rows (if any) are fresh.
"""

from __future__ import annotations

import logging
import threading
from dataclasses import dataclass, field

import torch

from . import config, ops, state
from .plan import DevicePlan, build_host_plan, longest_first, to_device

logger = logging.getLogger("fastdecode")


class HipOps:
    """GPU primitives of the split path (swapped for stand-ins in tests)."""

    @staticmethod
    def fa(q, k, v, cu_seqlens_q=None, max_seqlen_q=1, seqused_k=None, max_seqlen_k=None,
           softmax_scale=None, causal=False, block_table=None, softcap=0.0,
           return_softmax_lse=False, out=None, row_order=None, total_tokens=None, **_):
        """Paged decode partial in flash_attn_varlen_func's calling convention
        (backend.py:306-314): k/v are the [B, BS, KVH, D] cache views, one query
        token per row, seqused_k the per-row token counts (0 allowed),
        max_seqlen_k the longest of them (only the table columns it needs are
        read). Beyond the reference's call: row_order schedules rows (e.g. longest
        first); total_tokens, the sum of seqused_k known on the host, lets the
        launch plan size tasks for rows of uneven length."""
        if block_table is None or max_seqlen_q != 1 or seqused_k is None:
            raise NotImplementedError("HipOps.fa: only the paged decode form (one query "
                                      "token per row with a block table) is implemented")
        if softcap:
            raise NotImplementedError("HipOps.fa: logits soft-cap is not supported")
        o, lse = ops.paged_decode(q, k, v, block_table, seqused_k, softmax_scale, out=out,
                                  row_order=row_order, max_seqlen_k=max_seqlen_k,
                                  total_tokens=total_tokens)
        return (o, lse) if return_softmax_lse else o

    @staticmethod
    def split_decode(q, key_cache, value_cache, gpu_block_table, gpu_lens, host_k_cache,
                     host_v_cache, host_block_table, host_lens, softmax_scale, row_order=None):
        """Both tiers of every S row in one launch: the result of the GPU-tier
        partial, the host-tier partial and their merge (backend.py:293-356)."""
        return ops.split_decode(q, key_cache, value_cache, gpu_block_table, gpu_lens,
                                host_k_cache, host_v_cache, host_block_table, host_lens,
                                softmax_scale, row_order=row_order)

    @staticmethod
    def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, kv_cache_dtype="auto",
                          k_scale=None, v_scale=None):
        ops.reshape_and_cache(key, value, key_cache, value_cache, slot_mapping, kv_cache_dtype)

    @staticmethod
    def merge(out, o_a, lse_a, o_b, lse_b):
        ops.merge_attn_states(out, o_a, lse_a, o_b, lse_b)

    @staticmethod
    def event():
        ev = torch.cuda.Event()
        ev.record()
        return ev


OPS = HipOps


def is_decode_form(kw: dict) -> bool:
    """Whether an OPS.fa call is the split path's paged decode (backend.py:
    306-314: one query token per row over the paged cache, block table and
    per-row lengths, not causal, no soft-cap), the only form HipOps.fa runs.
    The P rows' causal prefill over the paged cache (:317-327) and the F
    rows' prefill over this step's q/k/v without a block table (:328-340)
    are other forms."""
    return (kw.get("max_seqlen_q") == 1 and kw.get("block_table") is not None
            and kw.get("seqused_k") is not None and not kw.get("causal", False)
            and not kw.get("softcap"))


def make_ops(prefill_fa):
    """The OPS seam for the reference plugin (backend.py:42-64): the paged
    decode form of fa, reshape_and_cache, merge and the fused split go to
    this library; every other form of fa (the P and F prefill calls) goes to
    `prefill_fa`, i.e. vLLM's flash_attn_varlen_func, unchanged."""

    def fa(**kw):
        if is_decode_form(kw):
            return HipOps.fa(**kw)
        return prefill_fa(**kw)

    return type("RoutedOps", (HipOps,), {"fa": staticmethod(fa),
                                         "prefill_fa": staticmethod(prefill_fa)})


def _write_hbm_tier(key, value, key_cache, value_cache, slots, kv_cache_dtype, layer,
                    write_gate=None):
    """The HBM-tier KV write through the OPS seam; with this library's op the
    write also honours a device write gate (nothing is written when it is
    non-zero), which a stand-in of vLLM's signature cannot take."""
    if OPS.reshape_and_cache is HipOps.reshape_and_cache:
        ops.reshape_and_cache(key, value, key_cache, value_cache, slots, kv_cache_dtype,
                              write_gate=write_gate)
    else:
        OPS.reshape_and_cache(key, value, key_cache, value_cache, slots, kv_cache_dtype,
                              getattr(layer, "_k_scale", None), getattr(layer, "_v_scale", None))


# The planner's capacity error (plan.py:133-137), raised by the host planner
# (plan.build_host_plan) and, for steps planned on the GPU, by
# raise_step_errors one step later.
CAPACITY_ERROR = ("FastDecode: block id beyond GPU+CPU capacity; engine and worker "
                  "disagree on FASTDECODE_CPU_BLOCKS / FASTDECODE_CPU_KV_GB")

_PENDING_ERRORS: list[tuple[torch.cuda.Event, torch.Tensor]] = []
_PENDING_LOCK = threading.Lock()


def raise_step_errors(wait: bool = False) -> None:
    """Raises the planner's RuntimeError for an earlier step planned on the GPU
    (build_device_step) whose tier planner counted a host block id or host
    slot past the host tier, or a length past the table. Such a step wrote no
    KV and its affected rows came out NaN. Each step's count comes back by an
    asynchronous copy into pinned memory; only copies that have landed are
    read (wait=True waits for the rest), so a caller at a step boundary,
    where the previous step's work is normally done, adds no wait. Both step
    builders call it first."""
    global _PENDING_ERRORS
    bad = 0
    with _PENDING_LOCK:
        keep = []
        for ev, count in _PENDING_ERRORS:
            if wait:
                ev.synchronize()
            if ev.query():
                bad += int(count[0])
            else:
                keep.append((ev, count))
        _PENDING_ERRORS = keep
    if bad:
        raise RuntimeError(f"{CAPACITY_ERROR} ({bad} host block id(s), host slot(s) or "
                           "length(s) past the table in a step planned on the GPU; that step "
                           "wrote no KV and its affected rows are NaN)")


class _StepStats:
    """Step statistics under FASTDECODE_STATS, as the reference's builder
    keeps them (backend.py:180-198): every 50 host-planned steps, the
    average requests per step that stayed all-HBM, were split decodes or
    fresh prefills with host slots, and the host-tier tokens read per layer."""

    def __init__(self) -> None:
        self.acc = [0, 0, 0, 0, 0]  # steps, P reqs, S reqs, F reqs, host tokens

    def add(self, hp, num_reqs: int) -> None:
        a = self.acc
        a[0] += 1
        if hp is None:
            a[1] += num_reqs
        else:
            a[1] += int(hp.p_req.numel())
            a[2] += hp.n_s
            a[3] += int(hp.f_cu.numel()) - 1
            a[4] += int(hp.s_cpu_lens.sum())
        if a[0] % 50 == 0:
            logger.warning("FastDecode: per-step averages over 50 steps: %.1f all-HBM "
                           "requests, %.1f split decodes, %.1f fresh prefills with host "
                           "slots; %.0f host-tier tokens read per layer", a[1] / 50, a[2] / 50,
                           a[3] / 50, a[4] / 50)
            self.acc = [a[0], 0, 0, 0, 0]


STATS = _StepStats()


def build_split_plan(query_start_loc_cpu: torch.Tensor, seq_lens_cpu: torch.Tensor,
                     block_table: torch.Tensor, slot_mapping: torch.Tensor, num_reqs: int,
                     store: state.HostKVStore | None, device) -> DevicePlan | None:
    """Per-step plan (backend.py:140-178): None when no host tier is set up or
    no request touches it (the step then runs plain paged attention)."""
    raise_step_errors()
    if store is None or num_reqs == 0:
        return None
    bs = store.block_size
    qsl = query_start_loc_cpu[: num_reqs + 1]
    seq = seq_lens_cpu[:num_reqs]
    max_blocks = int((int(seq.max()) + bs - 1) // bs)
    width = max(1, min(max_blocks, block_table.shape[1]))
    bt_dev = block_table[:num_reqs]
    n_tok = int(qsl[-1])
    bt = bt_dev[:, :width].cpu()  # the step's one device-to-host sync
    slots = slot_mapping[:n_tok].cpu()
    hp = build_host_plan(qsl, seq, bt, slots, store.num_gpu_blocks, store.num_cpu_blocks, bs)
    if config.stats_enabled():
        STATS.add(hp, num_reqs)
    if hp is None:
        return None
    return to_device(hp, bt_dev[:, :width], device)


@dataclass
class DeviceStep:
    """A step planned on the GPU: every row's per-tier tables, lengths and the
    split slot mapping (device tensors), plus what the host already knows
    from the step's CPU metadata: which tokens are decode rows and which
    belong to fresh prefills."""

    gpu_bt: torch.Tensor  # [R, W] int32
    cpu_bt: torch.Tensor  # [R, W] int32
    gpu_lens: torch.Tensor  # [R] int32
    cpu_lens: torch.Tensor  # [R] int32
    gpu_slots: torch.Tensor  # [T] int64
    host_slots: torch.Tensor  # [T] int64
    dec_rows: torch.Tensor  # [nD] int64: decode rows (one query token)
    dec_tok: torch.Tensor  # [nD] int64: their query tokens
    dec_order: torch.Tensor  # [nD] int32: longest first
    n_dec: int
    dec_tokens: int  # context tokens of the decode rows (both tiers): known on the host
    f_tok: torch.Tensor  # [nF_tok] int64: tokens of fresh prefills
    f_cu: torch.Tensor  # [nF + 1] int32
    f_max: int
    n_f_tok: int
    errors: torch.Tensor  # [1] int32: host ids / slots past the tier, lengths past the table
    # errors copied to pinned host memory, and the event after that copy
    errors_host: torch.Tensor | None = field(default=None, repr=False)
    errors_ready: torch.cuda.Event | None = field(default=None, repr=False)
    # the decode rows' host-tier view, fetched once per step for the hybrid
    # split (host_tables)
    _host: tuple | None = field(default=None, repr=False)

    def check_errors(self, wait: bool = True) -> None:
        """Raises the planner's RuntimeError if this step's tier planner found
        a host block id or host slot past the host tier (or a length past the
        table); wait=False returns quietly while the count is still on its way."""
        if self.errors_ready is None:
            return
        if wait:
            self.errors_ready.synchronize()
        if self.errors_ready.query() and int(self.errors_host[0]):
            raise RuntimeError(f"{CAPACITY_ERROR} ({int(self.errors_host[0])} host block id(s), "
                               "host slot(s) or length(s) past the table; this step wrote no KV "
                               "and its affected rows are NaN)")

    def host_tables(self) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        """(hbm_lens, host_bt, host_lens) of the decode rows on the host: one
        device-to-host copy per step (waits for the planning kernels), reused
        by every layer."""
        if self._host is None:
            rows = self.dec_rows
            packed = torch.cat([self.gpu_lens.index_select(0, rows)[:, None],
                                self.cpu_lens.index_select(0, rows)[:, None],
                                self.cpu_bt.index_select(0, rows)], dim=1).cpu()
            self._host = (packed[:, 0].contiguous(), packed[:, 2:].contiguous(),
                          packed[:, 1].contiguous())
        return self._host


def build_device_step(query_start_loc_cpu: torch.Tensor, seq_lens_cpu: torch.Tensor,
                      block_table: torch.Tensor, slot_mapping: torch.Tensor, num_reqs: int,
                      store: state.HostKVStore | None, device) -> DeviceStep | None:
    """Plans a step on the GPU (fd_plan_tiers): no device-to-host copy. None
    when no host tier is set up, or when a prefill row extends prior context
    (whether it touches the host tier is only known on the device; such
    steps take build_split_plan, where the reference's rule applies,
    plan.py:142-149). A host block id or host slot past the host tier is
    counted on the GPU: the step's KV writes are then skipped, and the
    planner's RuntimeError is raised by the next step's builder (or by
    DeviceStep.check_errors)."""
    raise_step_errors()
    if store is None or num_reqs == 0:
        return None
    qsl = query_start_loc_cpu[: num_reqs + 1].to(torch.int64)
    seq = seq_lens_cpu[:num_reqs].to(torch.int64)
    qlen = qsl[1:] - qsl[:-1]
    ctx = seq - qlen
    if bool(((qlen > 1) & (ctx > 0)).any()):
        return None
    def d(t: torch.Tensor) -> torch.Tensor:
        # host metadata to the device through pinned memory: no host wait
        return t.pin_memory().to(device, non_blocking=True)

    n_tok = int(qsl[-1])
    bs = store.block_size
    width = max(1, min(int((int(seq.max()) + bs - 1) // bs), block_table.shape[1]))
    errors = torch.zeros(1, dtype=torch.int32, device=device)
    gpu_bt, cpu_bt, gpu_lens, cpu_lens, gpu_slots, host_slots = ops.plan_tiers(
        block_table[:num_reqs, :width], d(seq.to(torch.int32)), slot_mapping[:n_tok],
        store.num_gpu_blocks, store.num_cpu_blocks, bs, error_count=errors)
    # the count travels back asynchronously; the next step's builder reads it
    errors_host = torch.empty(1, dtype=torch.int32, pin_memory=True)
    errors_host.copy_(errors, non_blocking=True)
    errors_ready = torch.cuda.Event()
    errors_ready.record(torch.cuda.current_stream(device))
    with _PENDING_LOCK:
        _PENDING_ERRORS.append((errors_ready, errors_host))
    dec = torch.nonzero(qlen == 1).flatten()
    fre = torch.nonzero(qlen > 1).flatten()
    f_q = qlen[fre]
    f_tok = torch.cat([torch.arange(int(qsl[r]), int(qsl[r + 1])) for r in fre.tolist()]) \
        if fre.numel() else torch.zeros(0, dtype=torch.int64)
    f_cu = torch.zeros(fre.numel() + 1, dtype=torch.int32)
    f_cu[1:] = torch.cumsum(f_q, 0).to(torch.int32)
    return DeviceStep(
        gpu_bt=gpu_bt, cpu_bt=cpu_bt, gpu_lens=gpu_lens, cpu_lens=cpu_lens,
        gpu_slots=gpu_slots, host_slots=host_slots,
        dec_rows=d(dec), dec_tok=d(qsl[dec]), dec_order=d(longest_first(seq[dec])),
        n_dec=int(dec.numel()), dec_tokens=int(seq[dec].sum()), f_tok=d(f_tok), f_cu=d(f_cu),
        f_max=int(f_q.max()) if f_q.numel() else 0, n_f_tok=int(f_tok.numel()), errors=errors,
        errors_host=errors_host, errors_ready=errors_ready,
    )


@dataclass
class SplitDecodeImpl:
    """The attention-layer state the split path needs (FastDecodeImpl's
    fields, backend.py:200-214)."""

    num_heads: int
    num_kv_heads: int
    head_size: int
    scale: float
    kv_cache_dtype: str = "auto"
    logits_soft_cap: float = 0.0
    kv_sharing_target_layer_name: str | None = None
    # S rows through one fused launch (OPS.split_decode) instead of two
    # partials and a merge; the unfused path is the reference's contract
    fused_split: bool = True
    # share of each S row's host-tier blocks reduced by the host cores while
    # the GPU reads the rest over the link (ops.hybrid_split_begin; fused path
    # only). 0 = the GPU reads the whole host tier; 1 = the reference's
    # division (the host cores compute the whole host-tier partial); "auto" =
    # balanced online from each step's finishing order (plan.ShareTuner).
    cpu_fraction: float | str = "auto"
    # below this many bytes of host-tier KV in a layer the GPU alone reads the
    # host tier: the host share's fixed cost (q to the host, one wait, the
    # merge) outweighs what it saves
    hybrid_min_host_bytes: int = 32 << 20
    # the hybrid split in steps planned on the GPU (_forward_device) too, for
    # steps whose decode rows could hold hybrid_min_host_bytes of host-tier KV
    # (judged from their lengths, known on the host): one device-to-host copy
    # of the decode rows' tables per step and the per-layer wait for q the
    # host share needs. False keeps every GPU-planned step free of host waits
    # (the whole host tier then goes over the link).
    device_step_hybrid: bool = True

    def __post_init__(self) -> None:
        self._tuner = None
        if self.cpu_fraction == "auto":
            from .plan import ShareTuner

            self._tuner = ShareTuner()
        elif not isinstance(self.cpu_fraction, (int, float)) or not 0 <= self.cpu_fraction <= 1:
            raise ValueError(f"cpu_fraction must be in [0, 1] or 'auto', got {self.cpu_fraction!r}")

    def _host_share(self) -> float:
        return self._tuner.fraction if self._tuner is not None else float(self.cpu_fraction)

    def _forward_split(self, layer, query, key, value, kv_cache, dp: DevicePlan, output):
        """query [T, H, D]; key/value [T, KVH, D] (possibly strided views);
        kv_cache the logical [B, KVH, BS, 2D] view of the HBM tier; output
        [T, H, D], written for the plan's S, P and F token rows."""
        hp = dp.host
        store = state.STORE
        assert store is not None, "no host KV tier (state.ensure_store)"
        k_host = store.k[layer.layer_name]
        v_host = store.v[layer.layer_name]
        fa = OPS.fa
        H, D = self.num_heads, self.head_size
        key_cache, value_cache = kv_cache.transpose(1, 2).split(D, dim=-1)

        # 1) KV writes: HBM slots by reshape_and_cache (host slots are -1), host
        #    slots straight into the pinned tier by the GPU (no staging copy)
        if self.kv_sharing_target_layer_name is None:
            OPS.reshape_and_cache(key, value, key_cache, value_cache, dp.gpu_slot_mapping,
                                  self.kv_cache_dtype, getattr(layer, "_k_scale", None),
                                  getattr(layer, "_v_scale", None))
            if hp.cpu_w_tok.numel():
                kw = key.index_select(0, dp.cpu_w_tok)
                vw = value.index_select(0, dp.cpu_w_tok)
                ops.store_kv(kw, vw, hp.cpu_w_slot, k_host, v_host)

        # 2) split decodes: HBM-tier and host-tier partials, both on the GPU
        #    (or both tiers in one fused launch). Rows without HBM tokens come
        #    back as (0, -inf) from the kernel, so every S row goes in as is.
        ns = hp.n_s
        fused = self.fused_split and getattr(OPS, "split_decode", None) is not None
        hybrid = None
        share = self._host_share()
        if share > 0 and ns:
            host_bytes = (int(hp.s_cpu_lens.sum()) * 2 * self.num_kv_heads * self.head_size *
                          query.element_size())
            if host_bytes < self.hybrid_min_host_bytes:
                share = 0.0
        if ns and fused and share > 0:
            # the GPU's share is enqueued now; the host cores run after the P
            # and F launches below, so those queue behind it on the GPU
            qs = query.index_select(0, dp.s_tok)
            hybrid = ops.hybrid_split_begin(qs, key_cache, value_cache, dp.s_gpu_bt_all,
                                            hp.s_gpu_lens, k_host, v_host, hp.s_cpu_bt,
                                            hp.s_cpu_lens, float(self.scale), share,
                                            hbm_lens_dev=dp.s_gpu_lens_all,
                                            host_block_table_dev=dp.s_cpu_bt)
        elif ns and fused:
            qs = query.index_select(0, dp.s_tok)
            merged, _ = OPS.split_decode(qs, key_cache, value_cache, dp.s_gpu_bt_all,
                                         dp.s_gpu_lens_all, k_host, v_host, dp.s_cpu_bt,
                                         dp.s_cpu_lens, float(self.scale), row_order=dp.s_order)
        elif ns:
            qs = query.index_select(0, dp.s_tok)
            if hp.s_max_gpu_len > 0:
                o_gpu, lse_gpu = fa(
                    q=qs, k=key_cache, v=value_cache,
                    cu_seqlens_q=torch.arange(ns + 1, dtype=torch.int32, device=qs.device),
                    max_seqlen_q=1, seqused_k=dp.s_gpu_lens_all, max_seqlen_k=hp.s_max_gpu_len,
                    softmax_scale=self.scale, causal=False, block_table=dp.s_gpu_bt_all,
                    softcap=self.logits_soft_cap, return_softmax_lse=True, num_splits=1,
                    row_order=dp.s_gpu_order, total_tokens=hp.s_gpu_tokens,
                )
            else:
                o_gpu = torch.zeros_like(qs)
                lse_gpu = torch.full((H, ns), float("-inf"), dtype=torch.float32, device=qs.device)
            o_cpu = torch.empty_like(qs)
            lse_cpu = torch.empty(H, ns, dtype=torch.float32, device=qs.device)
            ops.decode_attn(qs, k_host, v_host, dp.s_cpu_bt, dp.s_cpu_lens, float(self.scale),
                            o_cpu, lse_cpu, row_order=dp.s_cpu_order)

        try:
            self._prefill_rows(query, key, value, key_cache, value_cache, dp, output)
        except BaseException:
            if hybrid is not None:  # free the staging of the split begun above
                hybrid.cancel()
            raise

        # 4) merge the split decodes' partials into their output rows
        if hybrid is not None:
            merged, _ = hybrid.finish()
            if self._tuner is not None:
                self._tuner.update(hybrid.gpu_finished_first)
        if ns:
            if not fused:
                merged = torch.empty_like(qs)
                OPS.merge(merged, o_gpu, lse_gpu, o_cpu, lse_cpu)
            output.index_copy_(0, dp.s_tok, merged)
        return output

    def _prefill_rows(self, query, key, value, key_cache, value_cache, dp: DevicePlan, output):
        """Step 3 of _forward_split: attention that touches no host block, P
        (all-HBM requests) and F (fresh prefills over this step's q/k/v), by
        the prefill forms of OPS.fa."""
        hp = dp.host
        fa = OPS.fa
        if hp.n_p_tok:
            q_p = query.index_select(0, dp.p_tok)
            o_p = fa(
                q=q_p, k=key_cache, v=value_cache, cu_seqlens_q=dp.p_cu, max_seqlen_q=hp.p_max_q,
                seqused_k=dp.p_seqlens, max_seqlen_k=hp.p_max_k, softmax_scale=self.scale,
                causal=True, block_table=dp.p_bt, softcap=self.logits_soft_cap,
            )
            output.index_copy_(0, dp.p_tok, o_p)
        if hp.n_f_tok:
            q_f = query.index_select(0, dp.f_tok)
            k_f = key.index_select(0, dp.f_tok)
            v_f = value.index_select(0, dp.f_tok)
            o_f = fa(
                q=q_f, k=k_f, v=v_f, cu_seqlens_q=dp.f_cu, cu_seqlens_k=dp.f_cu,
                max_seqlen_q=hp.f_max, max_seqlen_k=hp.f_max, softmax_scale=self.scale,
                causal=True, softcap=self.logits_soft_cap,
            )
            output.index_copy_(0, dp.f_tok, o_f)

    def _forward_device(self, layer, query, key, value, kv_cache, ds: DeviceStep, output):
        """The step of _forward_split planned on the GPU (build_device_step):
        KV writes into both tiers from the split slot mapping, every decode row
        (all-HBM and split alike) through one fused two-tier launch, fresh
        prefills through the prefill form of OPS.fa. No device-to-host copy,
        unless device_step_hybrid gives the decode rows' host tier to the
        hybrid split (one copy of their tables per step)."""
        store = state.STORE
        assert store is not None, "no host KV tier (state.ensure_store)"
        k_host = store.k[layer.layer_name]
        v_host = store.v[layer.layer_name]
        D = self.head_size
        key_cache, value_cache = kv_cache.transpose(1, 2).split(D, dim=-1)

        # 1) KV writes: both tiers by slot, slots of the other tier are -1;
        #    nothing is written when the planner counted an error (every slot
        #    is checked before any write, cpu_attn.cpp:506-510)
        if self.kv_sharing_target_layer_name is None:
            _write_hbm_tier(key, value, key_cache, value_cache, ds.gpu_slots,
                            self.kv_cache_dtype, layer, write_gate=ds.errors)
            ops.reshape_and_cache(key, value, k_host.transpose(1, 2), v_host.transpose(1, 2),
                                  ds.host_slots, write_gate=ds.errors)

        # 2) decode rows: both tiers in one launch (a row without host tokens
        #    is plain paged attention over its HBM blocks), or, with
        #    device_step_hybrid, the hybrid split of that launch
        hybrid = None
        if ds.n_dec:
            q = query.index_select(0, ds.dec_tok)
            gbt = ds.gpu_bt.index_select(0, ds.dec_rows)
            gl = ds.gpu_lens.index_select(0, ds.dec_rows)
            cbt = ds.cpu_bt.index_select(0, ds.dec_rows)
            share = self._host_share() if self.device_step_hybrid else 0.0
            # the rows' whole context bounds their host-tier bytes: below the
            # threshold the tables are not even fetched (no host wait)
            bound = ds.dec_tokens * 2 * self.num_kv_heads * self.head_size * query.element_size()
            if share > 0 and bound >= self.hybrid_min_host_bytes:
                hl_h, cbt_h, cl_h = ds.host_tables()
                host_bytes = (int(cl_h.sum()) * 2 * self.num_kv_heads * self.head_size *
                              query.element_size())
                if host_bytes >= self.hybrid_min_host_bytes:
                    hybrid = ops.hybrid_split_begin(q, key_cache, value_cache, gbt, hl_h, k_host,
                                                    v_host, cbt_h, cl_h, float(self.scale), share,
                                                    hbm_lens_dev=gl, host_block_table_dev=cbt)
            if hybrid is None:
                out, _ = OPS.split_decode(q, key_cache, value_cache, gbt, gl, k_host, v_host, cbt,
                                          ds.cpu_lens.index_select(0, ds.dec_rows),
                                          float(self.scale), row_order=ds.dec_order)
                output.index_copy_(0, ds.dec_tok, out)

        # 3) fresh prefills attend only this step's q/k/v (backend.py:331-340)
        try:
            if ds.n_f_tok:
                q_f = query.index_select(0, ds.f_tok)
                k_f = key.index_select(0, ds.f_tok)
                v_f = value.index_select(0, ds.f_tok)
                o_f = OPS.fa(
                    q=q_f, k=k_f, v=v_f, cu_seqlens_q=ds.f_cu, cu_seqlens_k=ds.f_cu,
                    max_seqlen_q=ds.f_max, max_seqlen_k=ds.f_max, softmax_scale=self.scale,
                    causal=True, softcap=self.logits_soft_cap,
                )
                output.index_copy_(0, ds.f_tok, o_f)
        except BaseException:
            if hybrid is not None:  # free the staging of the split begun above
                hybrid.cancel()
            raise
        if hybrid is not None:  # the host cores' share, while the GPU runs the above
            out, _ = hybrid.finish()
            if self._tuner is not None:
                self._tuner.update(hybrid.gpu_finished_first)
            output.index_copy_(0, ds.dec_tok, out)
        return output
