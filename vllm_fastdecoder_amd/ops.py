"""Torch-facing wrappers of the HIP kernels, with the reference's signatures.

Reference surfaces this mirrors:
  * the CPU extension loaded by fastdecode/cpu_ops.py:21-46 and defined in
    fastdecode/csrc/cpu_attn.cpp:452-537 -- `decode_attn` and `store_kv`;
  * the GPU primitives behind backend.OPS (fastdecode/backend.py:42-64) --
    FlashAttention's paged decode partial, `reshape_and_cache_flash` and
    `merge_attn_states`.

Every function launches on the current HIP stream of the output's device and
returns without synchronising. Argument checks mirror the reference's
TORCH_CHECKs and raise RuntimeError before anything is written. Host-tier
caches must be pinned (see pinned.py); the kernels read them in place.
"""

from __future__ import annotations

import ctypes
import os
import threading

import numpy as np
import torch

from . import _lib
from .pinned import device_ptr, pinned_empty
from .plan import longest_first as _longest_first
from .plan import share_host_blocks as _share_host_blocks

_DT = {torch.float16: _lib.FD_F16, torch.bfloat16: _lib.FD_BF16, torch.float32: _lib.FD_F32}


def _dtype_code(t: torch.Tensor, what: str) -> int:
    try:
        return _DT[t.dtype]
    except KeyError:
        raise RuntimeError(f"{what}: unsupported dtype {t.dtype}") from None


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise RuntimeError(msg)


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def _stream_for(t: torch.Tensor) -> int:
    """Handle of the current stream on t's device (the raw query where torch
    has it: it skips building a Stream object on every call)."""
    if t.device.index is not None:
        return _current_stream(t.device.index)
    return torch.cuda.current_stream(t.device).cuda_stream


def _current_stream(idx: int) -> int:
    """Handle of the current stream on device idx."""
    if _RAW_STREAM is not None:
        return int(_RAW_STREAM(idx))
    return torch.cuda.current_stream(idx).cuda_stream


def _on_device(t: torch.Tensor, device: torch.device) -> torch.Tensor:
    """Small index tensors given on the host are copied to the device."""
    if t.is_cuda:
        return t
    return t.to(device, non_blocking=False)


def _table_on_device(bt: torch.Tensor, device: torch.device) -> tuple[torch.Tensor, int]:
    """A block table on the device and the pointer to pass for it. A table of
    no columns is passed as a one-id stand-in buffer (returned to keep it
    alive) with width 0: the library takes no NULL table, reads nothing of a
    zero-width one, and treats any row with tokens as a range error (NaN
    row)."""
    if bt.shape[1] == 0:
        hold = torch.zeros(1, dtype=torch.int32, device=device)
        return hold, hold.data_ptr()
    t = _on_device(bt, device)
    return t, t.data_ptr()


class _Workspace:
    """Grow-only device scratch for the split partials (the same grow-only
    policy as the reference's PinnedStaging.get, state.py:115-124), one
    buffer per (device, stream): launches on one stream run in order and
    share it, launches on different streams may overlap and get their own.
    A buffer is allocated while its stream is current, so the caching
    allocator reuses a replaced one only after that stream's earlier work.
    At most `max_streams` buffers are kept; the least recently used one is
    dropped beyond that (its memory returns to its stream's pool, which only
    that stream's later allocations reuse).

    A stream's buffer can be pinned (reserve_workspace, for HIP graph
    capture): a captured graph keeps the raw address of the buffer its
    launches were given, so a pinned stream's buffers are never dropped,
    neither by the eviction above nor when growth replaces one, until the
    reservation is released (release_workspace)."""

    def __init__(self, max_streams: int = 16) -> None:
        self._bufs: dict[tuple[int, int], torch.Tensor] = {}
        # pinned (device, stream) -> every buffer the stream has held since
        self._pinned: dict[tuple[int, int], list[torch.Tensor]] = {}
        self._lock = threading.Lock()
        self.max_streams = max_streams

    @staticmethod
    def _key(device: torch.device, stream: int | None) -> tuple[int, int]:
        idx = device.index if device.index is not None else torch.cuda.current_device()
        return idx, _current_stream(idx) if stream is None else int(stream)

    def get(self, device: torch.device, nbytes: int, stream: int | None = None,
            pin: bool = False) -> torch.Tensor | None:
        """The workspace of `stream` (a raw handle; default: the current
        stream on `device`, the one the caller's launch goes on), at least
        nbytes long. pin: keep this stream's buffers alive (see above)."""
        if nbytes == 0 and not pin:
            return None
        key = self._key(device, stream)
        with self._lock:
            buf = self._bufs.pop(key, None)  # re-inserted below: most recent last
            if buf is None or buf.numel() < nbytes:
                cap = max(nbytes, 2 * (buf.numel() if buf is not None else 0), 16)
                buf = torch.empty(cap, dtype=torch.uint8, device=torch.device("cuda", key[0]))
                if key in self._pinned:
                    self._pinned[key].append(buf)
            if pin and key not in self._pinned:
                self._pinned[key] = [buf]
            self._bufs[key] = buf
            while len(self._bufs) > self.max_streams:
                victim = next((k for k in self._bufs if k not in self._pinned), None)
                if victim is None:
                    break
                del self._bufs[victim]
            return buf

    def release(self, device: torch.device, stream: int) -> None:
        """Ends a pin: the stream's replaced buffers go, its current one stays
        (and may be evicted again)."""
        with self._lock:
            self._pinned.pop(self._key(device, stream), None)


WORKSPACE = _Workspace()


def reserve_workspace(stream: torch.cuda.Stream, nbytes: int) -> torch.Tensor:
    """Allocates the split workspace of `stream` now, at least nbytes long
    (workspace_bytes of the largest shape to come), and pins it. For HIP
    graph capture: torch.cuda.graph captures on its own stream, so a
    workspace reserved for that stream before capture keeps the captured
    launches from allocating (otherwise the first captured launch of a shape
    that splits rows allocates it from the graph's memory pool). The graph
    keeps the buffer's raw address, so while the reservation holds, the
    buffer is neither evicted nor freed when a later, larger call on the
    same stream grows the workspace. Returns the buffer; call
    release_workspace(stream) once every graph captured with it is gone."""
    with torch.cuda.stream(stream):
        return WORKSPACE.get(stream.device, nbytes, pin=True)


def release_workspace(stream: torch.cuda.Stream) -> None:
    """Ends reserve_workspace's pin on `stream`'s workspace."""
    WORKSPACE.release(stream.device, stream.cuda_stream)


_WS_SIZES: dict = {}


def decode_plan_info(n: int, H: int, KVH: int, D: int, BS: int, width: int, dtype: torch.dtype,
                     aligned: bool = True, host_tier: bool = False,
                     total_tokens: int | None = None) -> dict:
    """The kernel a decode launch of these sizes takes on the current device and
    how it is cut into tasks (fd_decode_plan_info): {"kernel": "valu" | "mm" |
    "mfma" | "f32" | "generic", "heads_per_task", "passes", "split_blocks",
    "max_splits", "wg_cap" (workgroups per CU the launch allows, 0 = the
    kernel's own occupancy), "capped" (wg_cap > 0), "wave_blocks" (tiles per
    working wave, 0 = every wave works)}. total_tokens: the rows' token total
    a paged_decode call is given (None: unknown). Honours FD_DECODE_KERNEL /
    FD_SPLIT_BLOCKS / FD_WG_CAP / FD_WAVE_BLOCKS."""
    plan = _lib.FdDecodePlan()
    _lib.check(_lib.load_lib().fd_decode_plan_info(n, H, KVH, D, BS, width, _DT[dtype],
                                                   int(aligned), int(host_tier),
                                                   int(total_tokens or 0),
                                                   ctypes.byref(plan)))
    return {"kernel": _lib.FD_KERNEL_NAMES[plan.kernel], "heads_per_task": plan.heads_per_task,
            "passes": plan.passes, "split_blocks": plan.split_blocks,
            "max_splits": plan.max_splits, "wg_cap": plan.wg_cap, "capped": plan.wg_cap > 0,
            "wave_blocks": plan.wave_blocks}


_GET_DEVICE = getattr(torch._C, "_cuda_getDevice", None)


def _current_device() -> int:
    """Index of the current device (-1 without one); the raw query where torch
    has it, as a decode call's workspace lookup runs on every launch."""
    if _GET_DEVICE is not None and torch.cuda.is_initialized():
        return int(_GET_DEVICE())
    return torch.cuda.current_device() if torch.cuda.is_available() else -1


def workspace_bytes(n: int, H: int, KVH: int, D: int, BS: int, width: int) -> int:
    """Workspace a decode call of this shape needs on the current device
    (remembered per shape, device and the planner overrides it depends on:
    FD_SPLIT_BLOCKS, and FD_DECODE_KERNEL, which can allow more splits; the
    device's CU count sets the split bounds)."""
    env = os.environ
    key = (n, H, KVH, D, BS, width, env.get("FD_SPLIT_BLOCKS"), env.get("FD_DECODE_KERNEL"),
           _current_device())
    size = _WS_SIZES.get(key)
    if size is None:
        c = ctypes.c_size_t()
        _lib.check(_lib.load_lib().fd_paged_decode_workspace_size(n, H, KVH, D, BS, width,
                                                                  ctypes.byref(c)))
        size = int(c.value)
        if len(_WS_SIZES) > 4096:
            _WS_SIZES.clear()
        _WS_SIZES[key] = size
    return size


def paged_decode_partial(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    kv_strides: tuple[int, int, int],
    num_blocks: int,
    block_size: int,
    num_kv_heads: int,
    block_table: torch.Tensor,
    lens: torch.Tensor,
    scale: float,
    out: torch.Tensor,
    lse: torch.Tensor,
    workspace: torch.Tensor | None = None,
    row_order: torch.Tensor | None = None,
    total_tokens: int | None = None,
    timeline: torch.Tensor | None = None,
) -> None:
    """Layout-generic entry: kv_strides = (block, head, token) in elements.
    row_order: optional int32 [n] permutation scheduling the rows (e.g.
    longest_first(lens)); results do not depend on it. total_tokens: the
    rows' token total when the caller knows it on the host
    (fd_paged_decode_partial_hint); it steers the task sizes only.
    timeline: measurement only, a zeroed int64 [workgroups, 8] GPU tensor
    that receives each workgroup's time stamps (fd_paged_decode_timeline;
    launches on the 16-bit VALU kernel only)."""
    _require(q.is_cuda and out.is_cuda and lse.is_cuda, "q, out and lse must be on the GPU")
    _require(q.dim() == 3 and out.shape == q.shape, "q and out must be [n, H, D] of one shape")
    n, H, D = q.shape
    _require(q.stride(2) == 1 and out.stride(2) == 1, "head_size must be the contiguous dim")
    _require(lse.dtype == torch.float32 and lse.dim() == 2 and tuple(lse.shape) == (H, n),
             "lse must be float32 [H, n]")
    _require(n == 0 or lse.stride(1) == 1, "lse rows must be contiguous")
    _require(block_table.dtype == torch.int32 and lens.dtype == torch.int32,
             "block_table and lens must be int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == n and lens.shape == (n,),
             "block_table must be [n, W] and lens [n]")
    kv_dt = _dtype_code(k_cache, "k_cache")
    _require(q.dtype == k_cache.dtype and v_cache.dtype == k_cache.dtype,
             "q, k_cache and v_cache must share a dtype")
    _require(out.dtype == q.dtype or out.dtype == torch.float32, "out must be q's dtype or float32")
    _require(k_cache.stride() == v_cache.stride() and k_cache.shape == v_cache.shape,
             "k_cache and v_cache must share shape and strides")
    if n == 0:
        return
    dev = q.device
    W = block_table.shape[1]
    bt, bt_ptr = _table_on_device(block_table, dev)
    ln = _on_device(lens, dev)
    _require(W == 0 or bt.stride(1) == 1, "block_table rows must be contiguous")
    ln = ln.contiguous()
    need = workspace_bytes(n, H, num_kv_heads, D, block_size, W)
    if workspace is None:
        workspace = WORKSPACE.get(dev, need)
    ws_ptr = workspace.data_ptr() if workspace is not None else None
    ws_len = workspace.numel() * workspace.element_size() if workspace is not None else 0
    order_ptr = None
    if row_order is not None:
        _require(row_order.dtype == torch.int32 and row_order.shape == (n,),
                 "row_order must be int32 [n]")
        row_order = _on_device(row_order, dev).contiguous()
        order_ptr = row_order.data_ptr()
    lib = _lib.load_lib()
    args = (
        q.data_ptr(), q.stride(0), q.stride(1),
        device_ptr(k_cache), device_ptr(v_cache),
        kv_strides[0], kv_strides[1], kv_strides[2],
        num_blocks,
        bt_ptr, bt.stride(0) if W else 0, W,
        ln.data_ptr(), order_ptr,
        n, H, num_kv_heads, D,
        block_size, float(scale), kv_dt,
        out.data_ptr(), out.stride(0), out.stride(1), _DT[out.dtype],
        lse.data_ptr(), lse.stride(0),
        ws_ptr, ws_len,
        _stream_for(q),
    )
    if timeline is not None:
        _require(total_tokens is None, "timeline: no token-total hint")
        _require(timeline.is_cuda and timeline.dtype == torch.int64 and timeline.dim() == 2
                 and timeline.shape[1] == 8 and timeline.is_contiguous(),
                 "timeline must be a contiguous int64 [workgroups, 8] GPU tensor")
        _lib.check(lib.fd_paged_decode_timeline(*args, timeline.data_ptr(), timeline.shape[0]))
    elif total_tokens is None:
        _lib.check(lib.fd_paged_decode_partial(*args))
    else:
        _lib.check(lib.fd_paged_decode_partial_hint(*args, int(total_tokens)))


def _tier(k_cache, v_cache, strides, num_blocks, block_table, lens, n, dev, what):
    """fd_kv_tier for one tier (plus the index tensors it points at, which the
    caller keeps alive until the launch is enqueued)."""
    _require(block_table.dtype == torch.int32 and lens.dtype == torch.int32,
             f"{what}: block_table and lens must be int32")
    _require(block_table.dim() == 2 and block_table.shape[0] == n and lens.shape == (n,),
             f"{what}: block_table must be [n, W] and lens [n]")
    _require(k_cache.stride() == v_cache.stride() and k_cache.shape == v_cache.shape,
             f"{what}: k and v caches must share shape and strides")
    _require(k_cache.stride(-1) == 1, f"{what}: caches must be contiguous in head_size")
    W = block_table.shape[1]
    bt, bt_ptr = _table_on_device(block_table, dev)
    _require(W <= 1 or bt.stride(1) == 1, f"{what}: block_table rows must be contiguous")
    ln = _on_device(lens, dev).contiguous()
    desc = _lib.FdKvTier(
        device_ptr(k_cache), device_ptr(v_cache), strides[0], strides[1], strides[2], num_blocks,
        bt_ptr, bt.stride(0) if W else 0, W, ln.data_ptr(),
    )
    return desc, (bt, ln)


def split_decode(
    q: torch.Tensor,
    hbm_key_cache: torch.Tensor,
    hbm_value_cache: torch.Tensor,
    hbm_block_table: torch.Tensor,
    hbm_lens: torch.Tensor,
    host_k_cache: torch.Tensor,
    host_v_cache: torch.Tensor,
    host_block_table: torch.Tensor,
    host_lens: torch.Tensor,
    softmax_scale: float,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    row_order: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Fused split decode: attention over each row's HBM-tier and host-tier
    blocks in one launch, i.e. the GPU-tier partial, the host-tier partial and
    their merge of fastdecode/backend.py:293-356 in one call (the result of
    paged_decode + decode_attn + merge_attn_states, up to fp32 summation
    order).

    hbm_key_cache / hbm_value_cache [B, BS, KVH, D]: vLLM's cache halves;
    host_k_cache / host_v_cache [C, KVH, BS, D]: the pinned host tier;
    *_block_table int32 [n, W] tier-relative ids in sequence order and
    *_lens int32 [n] tier token counts (the planner's s_gpu_bt / s_gpu_lens
    and s_cpu_bt / s_cpu_lens; 0 allowed in either). Returns out [n, H, D]
    (q's dtype unless `out` is given) and lse [H, n] float32.
    """
    _require(q.is_cuda and q.dim() == 3 and q.stride(2) == 1, "q must be [n, H, D] on the GPU")
    n, H, D = q.shape
    _require(hbm_key_cache.dim() == 4 and host_k_cache.dim() == 4, "caches must be 4-d")
    B, BS, KVH, Dk = hbm_key_cache.shape
    C, KVH2, BS2, Dh = host_k_cache.shape
    _require(Dk == D and Dh == D and KVH2 == KVH and BS2 == BS,
             "the tiers' head size, kv heads and block size must agree with q")
    _require(H % KVH == 0, "num_heads must be a multiple of num_kv_heads")
    kv_dt = _dtype_code(q, "q")
    for t in (hbm_key_cache, hbm_value_cache, host_k_cache, host_v_cache):
        _require(t.dtype == q.dtype, "q and the caches must share a dtype")
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty(H, n, dtype=torch.float32, device=q.device)
    _require(out.is_cuda and out.shape == q.shape and out.stride(2) == 1,
             "out must be [n, H, D] on the GPU")
    _require(out.dtype == q.dtype or out.dtype == torch.float32, "out must be q's dtype or float32")
    _require(lse.dtype == torch.float32 and tuple(lse.shape) == (H, n) and (n == 0 or lse.stride(1) == 1),
             "lse must be float32 [H, n] with contiguous rows")
    if n == 0:
        return out, lse
    dev = q.device
    hbm, keep_a = _tier(hbm_key_cache, hbm_value_cache,
                        (hbm_key_cache.stride(0), hbm_key_cache.stride(2), hbm_key_cache.stride(1)),
                        B, hbm_block_table, hbm_lens, n, dev, "hbm tier")
    host, keep_b = _tier(host_k_cache, host_v_cache,
                         (host_k_cache.stride(0), host_k_cache.stride(1), host_k_cache.stride(2)),
                         C, host_block_table, host_lens, n, dev, "host tier")
    need = workspace_bytes(n, H, KVH, D, BS, hbm.bt_width + host.bt_width)
    ws = WORKSPACE.get(dev, need)
    order_ptr = None
    if row_order is not None:
        _require(row_order.dtype == torch.int32 and row_order.shape == (n,),
                 "row_order must be int32 [n]")
        row_order = _on_device(row_order, dev).contiguous()
        order_ptr = row_order.data_ptr()
    lib = _lib.load_lib()
    _lib.check(
        lib.fd_split_decode(
            q.data_ptr(), q.stride(0), q.stride(1),
            ctypes.byref(hbm), ctypes.byref(host), order_ptr,
            n, H, KVH, D, BS, float(softmax_scale), kv_dt,
            out.data_ptr(), out.stride(0), out.stride(1), _DT[out.dtype],
            lse.data_ptr(), lse.stride(0),
            ws.data_ptr() if ws is not None else None, ws.numel() if ws is not None else 0,
            _stream_for(q),
        )
    )
    del keep_a, keep_b  # the launch is enqueued; later reuse is stream-ordered
    return out, lse


class _StagingSet:
    """One set of the hybrid split's pinned host buffers (see _HybridStaging):
    grow-only buffers by name, their views cached by shape and dtype (a step
    of the same shape takes the same tensors), and the set's events."""

    def __init__(self, dev_idx: int) -> None:
        self.dev_idx = dev_idx
        self._bufs: dict[str, torch.Tensor] = {}
        self._views: dict[str, tuple] = {}
        # events behind the last step's copies and reads of the buffers (a
        # subset of release_events, which are reused step after step)
        self.released: tuple = ()
        self.release_events: list[torch.cuda.Event] = []
        # timing event behind the copy of q to the host (re-recorded by each
        # step; recorded once here so that its HIP event exists)
        self.q_ready = torch.cuda.Event(enable_timing=True)
        with torch.cuda.device(dev_idx):
            self.q_ready.record()
        # timing event behind the GPU's launch of each step
        self.gpu_done = torch.cuda.Event(enable_timing=True)

    def view(self, name: str, shape: tuple, dtype: torch.dtype) -> torch.Tensor:
        hit = self._views.get(name)
        if hit is not None and hit[0] == shape and hit[1] == dtype:
            return hit[2]
        numel = 1
        for d in shape:
            numel *= int(d)
        used = numel * dtype.itemsize
        buf = self._bufs.get(name)
        if buf is None or buf.numel() < max(used, 1):
            cap = max(used, 1, 2 * (buf.numel() if buf is not None else 0))
            # the library's mapped allocation: device_ptr finds its GPU address
            # without asking the runtime (the merge reads the host partial there)
            buf = pinned_empty((cap,), torch.uint8)
            self._bufs[name] = buf
        v = buf[:used].view(dtype).view(tuple(shape))
        self._views[name] = (tuple(shape), dtype, v)
        return v


class _HybridStaging:
    """Grow-only pinned host buffers of the hybrid split (the grow-only policy
    of the reference's PinnedStaging, state.py:93-124): q on its way to the
    host cores, their fp32 partial on its way back, the division of the host
    blocks, and the host-planned index tensors on their way to the GPU.
    Reused every step, so a step allocates no pinned memory. Two sets per
    device, used in turn: a step's merge may still be reading its set while
    the next step fills the other one. One hybrid step may be in flight per
    device; a step waits (usually not at all) until the work of the step
    before last that read or wrote its set has completed."""

    def __init__(self) -> None:
        self._sets: dict[tuple[int, int], _StagingSet] = {}
        self._turn: dict[int, int] = {}
        self._pending: set[int] = set()
        self._lock = threading.Lock()

    def acquire(self, dev: torch.device) -> _StagingSet:
        idx = dev.index if dev.index is not None else torch.cuda.current_device()
        with self._lock:
            if idx in self._pending:
                raise RuntimeError("a hybrid split is already in flight on this device; "
                                   "finish() it before starting another")
            self._pending.add(idx)
            slot = self._turn.get(idx, 0)
            self._turn[idx] = slot ^ 1
            st = self._sets.get((idx, slot))
        try:
            if st is None:
                st = _StagingSet(idx)
                with self._lock:
                    self._sets[(idx, slot)] = st
            for ev in st.released:
                if not ev.query():
                    ev.synchronize()
        except BaseException:  # the device stays free for the next split
            with self._lock:
                self._pending.discard(idx)
            raise
        return st

    def release(self, st: _StagingSet, streams) -> None:
        """Frees the set once the work enqueued so far on every stream in
        `streams` (those whose copies read or write it) is done."""
        evs = []
        for k, s in enumerate(dict.fromkeys(streams)):  # distinct, in order
            while len(st.release_events) <= k:
                st.release_events.append(torch.cuda.Event())
            ev = st.release_events[k]
            ev.record(s)
            evs.append(ev)
        st.released = tuple(evs)
        with self._lock:
            self._pending.discard(st.dev_idx)

    def upload(self, st: _StagingSet, name: str, t: torch.Tensor,
               dev: torch.device) -> torch.Tensor:
        """A host tensor copied to the device through its pinned buffer (the
        host-side copy by numpy: single-threaded, leaving no spinning OpenMP
        team behind on the host cores)."""
        if t.is_cuda:
            return t
        v = st.view(name, tuple(t.shape), t.dtype)
        np.copyto(v.numpy(), t.numpy())
        return v.to(dev, non_blocking=True)


HYBRID_STAGING = _HybridStaging()


class HybridSplit:
    """A hybrid split decode in flight (hybrid_split_begin): the GPU's share
    is enqueued and the host cores' share is queued on the library's runner
    thread; finish() waits for the latter and enqueues the merge."""

    def __init__(self, out, lse, o_gpu=None, l_gpu=None, o_cpu=None, l_cpu=None,
                 host_call: HostDecodeCall | None = None, staging: _StagingSet | None = None,
                 stream=None, owned=()):
        self.out, self.lse = out, lse
        # those of out / lse that begin() allocated (on its stream)
        self._owned = owned
        # the staging set in use and the stream begin() enqueued its copies on
        self._staging, self._stream = staging, stream
        self._o_gpu, self._l_gpu = o_gpu, l_gpu
        self._o_cpu, self._l_cpu = o_cpu, l_cpu
        self._call = host_call
        self.cpu_seconds = 0.0  # time of the host cores' share (0 before finish)
        # whether the GPU's fused launch had completed when the host cores
        # finished (None before finish): the signal that balances the share
        self.gpu_finished_first: bool | None = None
        # the merge's arguments but the stream, checked while begin() runs
        # (the host cores' share keeps finish() off the critical path then)
        self._merge = (_merge_args(out, o_gpu, l_gpu, o_cpu, l_cpu, lse)
                       if o_gpu is not None else None)

    def _drop(self) -> None:
        # begin's uploads and the merge's reads of the host partial may sit
        # on different streams if the caller switched streams in between
        streams = (self._stream,)
        if _current_stream(self._staging.dev_idx) != self._stream.cuda_stream:
            streams += (torch.cuda.current_stream(self.out.device),)
        HYBRID_STAGING.release(self._staging, streams)
        self._o_gpu = self._l_gpu = self._o_cpu = self._l_cpu = self._call = None

    def cancel(self) -> None:
        """Abandons a split that will not be finished (the caller's step
        failed between begin and finish): waits for the host cores' share to
        stop using the staging, frees it for the next split and leaves out /
        lse unwritten. No-op after finish()."""
        if self._o_gpu is None:
            return
        try:
            self._call.wait()
        finally:
            self._drop()

    def finish(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Waits for the host cores' share and enqueues the merge, which
        reads that partial from the pinned staging."""
        if self._o_gpu is None:
            return self.out, self.lse
        try:
            self.cpu_seconds = self._call.wait()
            cur = _current_stream(self._staging.dev_idx)
            if cur != self._stream.cuda_stream:
                # the GPU partial (and out / lse when begin() allocated them)
                # came from begin's stream: keep the allocator from reusing
                # them before this stream's merge and later work are done
                for t in (self._o_gpu, self._l_gpu, *self._owned):
                    t.record_stream(torch.cuda.current_stream(self.out.device))
            # the host partial is read by the merge straight from the pinned staging
            _lib.check(_lib.load_lib().fd_merge_attn_states(*self._merge, cur))
            # the GPU finished first if its launch is complete now and took no
            # longer, from q's arrival on the host, than the host cores' share
            st = self._staging
            self.gpu_finished_first = bool(st.gpu_done.query()) and (
                st.q_ready.elapsed_time(st.gpu_done) <= self.cpu_seconds * 1e3)
        finally:
            if self._call is not None:
                self._call.wait()  # finish interrupted: let the share stop first
            self._drop()
        return self.out, self.lse


def _host_share_start(st: _StagingSet, stream: int, q: torch.Tensor, host_k_cache, host_v_cache,
                      host_block_table, host_lens, softmax_scale: float, cpu_fraction: float,
                      num_threads: int):
    """Starts the host cores' share of a hybrid step in one library call
    (fd_hybrid_share_start: the copy of q to the staging, its event, the
    division of the host blocks, the queued host call). Returns the call,
    the host partial (o, lse) and the GPU's host-tier lengths."""
    n, H, D = q.shape
    _require(host_k_cache.dim() == 4 and host_v_cache.shape == host_k_cache.shape
             and host_k_cache.stride() == host_v_cache.stride() and host_k_cache.stride(3) == 1,
             "host_k_cache/host_v_cache must be [C, KVH, BS, D], contiguous in D")
    C, KVH, BS, Dc = host_k_cache.shape
    _require(Dc == D and H % KVH == 0, "q must be [n, H, D] with the host cache's head size")
    kv_dt = _dtype_code(host_k_cache, "host_k_cache")
    _require(q.dtype == host_k_cache.dtype and host_v_cache.dtype == host_k_cache.dtype,
             "q and the host caches must share a dtype")
    _require(host_block_table.dim() == 2 and host_block_table.shape[0] == n
             and host_lens.shape == (n,), "host_block_table must be [n, W] and host_lens [n]")
    bt = host_block_table
    if bt.dtype != torch.int32 or bt.stride(-1) != 1:
        bt = bt.to(torch.int32).contiguous()
    hl = host_lens
    if hl.dtype != torch.int32 or not hl.is_contiguous():
        hl = hl.to(torch.int32).contiguous()
    W = bt.shape[1]
    qc = q if q.is_contiguous() else q.contiguous()
    q_host = st.view("q", (n, H, D), q.dtype)
    o_cpu = st.view("o", (n, H, D), torch.float32)
    l_cpu = st.view("lse", (H, n), torch.float32)
    gpu_lens = st.view("gpu_lens", (n,), torch.int32)
    cpu_lens = st.view("cpu_lens", (n,), torch.int32)
    cpu_bt = st.view("cpu_bt", (n, max(W, 1)), torch.int32)
    call_id = ctypes.c_int64()
    _lib.check(_lib.load_lib().fd_hybrid_share_start(
        stream, st.q_ready.cuda_event, qc.data_ptr(), q_host.data_ptr(),
        bt.data_ptr(), bt.stride(0) if n else W, W, hl.data_ptr(), float(cpu_fraction),
        gpu_lens.data_ptr(), cpu_bt.data_ptr(), cpu_bt.stride(0), cpu_lens.data_ptr(),
        host_k_cache.data_ptr(), host_v_cache.data_ptr(),
        host_k_cache.stride(0), host_k_cache.stride(1), host_k_cache.stride(2), C,
        n, H, KVH, D, BS, float(softmax_scale), kv_dt,
        o_cpu.data_ptr(), l_cpu.data_ptr(), int(num_threads), ctypes.byref(call_id)))
    keep = (qc, host_k_cache, host_v_cache, bt, hl)
    return HostDecodeCall(call_id.value or None, keep), o_cpu, l_cpu, gpu_lens


def hybrid_split_begin(
    q: torch.Tensor,
    hbm_key_cache: torch.Tensor,
    hbm_value_cache: torch.Tensor,
    hbm_block_table: torch.Tensor,
    hbm_lens: torch.Tensor,
    host_k_cache: torch.Tensor,
    host_v_cache: torch.Tensor,
    host_block_table: torch.Tensor,
    host_lens: torch.Tensor,
    softmax_scale: float,
    cpu_fraction: float,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    num_threads: int = 0,
    hbm_lens_dev: torch.Tensor | None = None,
    host_block_table_dev: torch.Tensor | None = None,
) -> HybridSplit:
    """First half of hybrid_split_decode: starts the copy of q to the host,
    divides the host tier and queues the host cores' share behind the copy on
    the library's runner thread (it starts as soon as q is on the host; all
    three in one library call), then enqueues the GPU's fused launch. Other
    GPU work can be enqueued before HybridSplit.finish(), which waits for the
    host cores and enqueues the merge. hbm_lens_dev / host_block_table_dev:
    device copies of hbm_lens / host_block_table the caller already holds
    (the GPU's share reads the host table unchanged, only with shorter
    lengths), saving their uploads."""
    _require(q.is_cuda and q.dim() == 3, "q must be [n, H, D] on the GPU")
    _require(host_block_table.device.type == "cpu" and host_lens.device.type == "cpu",
             "host_block_table and host_lens must be CPU tensors")
    _require(host_k_cache.device.type == "cpu" and host_v_cache.device.type == "cpu",
             "the host tier must be in host memory")
    n, H, D = q.shape
    dev = q.device
    owned = []
    if out is None:
        out = torch.empty_like(q)
        owned.append(out)
    if lse is None:
        lse = torch.empty(H, n, dtype=torch.float32, device=dev)
        owned.append(lse)
    if n == 0:
        _share_host_blocks(host_block_table, host_lens, host_k_cache.shape[2], cpu_fraction)
        return HybridSplit(out, lse)
    st = HYBRID_STAGING.acquire(dev)
    stream = None
    call = None
    try:
        # the host cores' share first: it is the step's longer half (the
        # stream's torch object, slower to get, only once it is queued)
        call, o_cpu, l_cpu, gpu_lens = _host_share_start(
            st, _current_stream(st.dev_idx), q, host_k_cache, host_v_cache, host_block_table,
            host_lens, softmax_scale, cpu_fraction, num_threads)
        stream = torch.cuda.current_stream(dev)

        def up(name, t):  # host index tensors: through pinned staging, asynchronous
            return HYBRID_STAGING.upload(st, name, t, dev)

        # rows by decreasing GPU work when the HBM lengths are known on the host
        order = None
        if not hbm_lens.is_cuda:
            work = hbm_lens.numpy().astype(np.int64) + gpu_lens.numpy()
            order = up("order", torch.from_numpy(
                np.argsort(-work, kind="stable").astype(np.int32)))
        o_gpu = torch.empty(n, H, D, dtype=torch.float32, device=dev)
        l_gpu = torch.empty(H, n, dtype=torch.float32, device=dev)
        hl = hbm_lens_dev if hbm_lens_dev is not None else up("hbm_lens", hbm_lens)
        hbt = (host_block_table_dev if host_block_table_dev is not None
               else up("host_bt", host_block_table))
        # the GPU's host-tier lengths are already in pinned staging
        split_decode(q, hbm_key_cache, hbm_value_cache, up("hbm_bt", hbm_block_table), hl,
                     host_k_cache, host_v_cache, hbt, gpu_lens.to(dev, non_blocking=True),
                     softmax_scale, out=o_gpu, lse=l_gpu, row_order=order)
        st.gpu_done.record(stream)
        h = HybridSplit(out, lse, o_gpu, l_gpu, o_cpu, l_cpu, call, staging=st, stream=stream,
                        owned=tuple(owned))
    except BaseException:
        try:
            if call is not None:
                call.wait()  # the share reads the staging: let it stop first
        finally:
            HYBRID_STAGING.release(st, (stream or torch.cuda.current_stream(dev),))
        raise
    return h


def hybrid_split_decode(
    q: torch.Tensor,
    hbm_key_cache: torch.Tensor,
    hbm_value_cache: torch.Tensor,
    hbm_block_table: torch.Tensor,
    hbm_lens: torch.Tensor,
    host_k_cache: torch.Tensor,
    host_v_cache: torch.Tensor,
    host_block_table: torch.Tensor,
    host_lens: torch.Tensor,
    softmax_scale: float,
    cpu_fraction: float,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    num_threads: int = 0,
) -> tuple[torch.Tensor, torch.Tensor]:
    """split_decode with the host tier shared between the GPU and the host
    cores: the reference's split step (fastdecode/backend.py:293-356: GPU
    partial, host-core partial of the host tier, merge) with part of the host
    tier moved back to the GPU.

    Each row's host blocks are divided by plan.share_host_blocks: the GPU's
    fused launch reads the HBM tier plus the leading host blocks over the
    link; meanwhile the host cores (fd_host_decode_partial) reduce the
    trailing ones from their own DRAM; the two fp32 partials are LSE-merged
    on the GPU. cpu_fraction 1 is the reference's division of work, 0 is
    split_decode. host_block_table / host_lens must be CPU tensors (the
    host-side planner's s_cpu_bt / s_cpu_lens); the other arguments are those
    of split_decode (tables and lengths on the host are uploaded
    asynchronously).

    Synchronises the host with the GPU once, for the copy of q to the host
    (which is ordered before the fused launch, so the wait does not include
    it), and blocks the caller while the host cores run. Host-tier KV written
    by earlier work on the stream is visible to the host cores.
    """
    return hybrid_split_begin(q, hbm_key_cache, hbm_value_cache, hbm_block_table, hbm_lens,
                              host_k_cache, host_v_cache, host_block_table, host_lens,
                              softmax_scale, cpu_fraction, out=out, lse=lse,
                              num_threads=num_threads).finish()


def plan_tiers(block_table: torch.Tensor, seq_lens: torch.Tensor, slot_mapping: torch.Tensor,
               num_gpu_blocks: int, num_cpu_blocks: int, block_size: int,
               error_count: torch.Tensor | None = None):
    """Device-side tier split of a step (fd_plan_tiers): the per-row, per-tier
    block compaction and token counts and the slot split of
    fastdecode/plan.py:82-100,150-152,165-170, computed on the GPU.

    block_table int32 [R, W] on the GPU; seq_lens int32 [R] (a host tensor is
    uploaded, never read back); slot_mapping int64 [T] on the GPU;
    error_count optional int32 [1] GPU counter of host ids past the host tier,
    host slots past it and lengths past the table. Returns (gpu_bt [R, W], cpu_bt [R, W],
    gpu_lens [R], cpu_lens [R], gpu_slots [T], host_slots [T])."""
    _require(block_table.is_cuda and block_table.dtype == torch.int32 and block_table.dim() == 2,
             "block_table must be int32 [R, W] on the GPU")
    R, W = block_table.shape
    dev = block_table.device
    _require(R == 0 or W <= 1 or block_table.stride(1) == 1, "block_table rows must be contiguous")
    _require(seq_lens.dtype == torch.int32 and seq_lens.shape == (R,), "seq_lens must be int32 [R]")
    _require(slot_mapping.dtype == torch.int64 and slot_mapping.dim() == 1,
             "slot_mapping must be int64 [T]")
    T = slot_mapping.shape[0]
    ln = _on_device(seq_lens, dev).contiguous()
    sm = _on_device(slot_mapping, dev).contiguous()
    gpu_bt = torch.empty(R, W, dtype=torch.int32, device=dev)
    cpu_bt = torch.empty(R, W, dtype=torch.int32, device=dev)
    gpu_lens = torch.empty(R, dtype=torch.int32, device=dev)
    cpu_lens = torch.empty(R, dtype=torch.int32, device=dev)
    gpu_slots = torch.empty(T, dtype=torch.int64, device=dev)
    host_slots = torch.empty(T, dtype=torch.int64, device=dev)
    err_ptr = None
    if error_count is not None:
        _require(error_count.is_cuda and error_count.dtype == torch.int32, "error_count: int32 GPU")
        err_ptr = error_count.data_ptr()
    _lib.check(
        _lib.load_lib().fd_plan_tiers(
            block_table.data_ptr(), block_table.stride(0) if R else W, W,
            ln.data_ptr(), R,
            int(num_gpu_blocks), int(num_cpu_blocks), int(block_size),
            gpu_bt.data_ptr(), cpu_bt.data_ptr(), W, W,
            gpu_lens.data_ptr(), cpu_lens.data_ptr(),
            sm.data_ptr(), T,
            gpu_slots.data_ptr(), host_slots.data_ptr(),
            err_ptr, _stream_for(block_table),
        )
    )
    return gpu_bt, cpu_bt, gpu_lens, cpu_lens, gpu_slots, host_slots


def longest_first(lens: torch.Tensor) -> torch.Tensor:
    """int32 permutation of the rows by decreasing length, computed on the
    host (the planner already holds the lengths there)."""
    return _longest_first(lens.cpu())


def decode_attn(q, k_cache, v_cache, block_table, lens, scale, out, lse, row_order=None) -> None:
    """Host-tier layout partial, signature of cpu_attn.cpp:456-489.

    q [n, H, D]; k_cache/v_cache [C, KVH, BS, D] (pinned host memory or HBM);
    block_table [n, W] int32 (tier-relative ids in sequence order); lens [n]
    int32; out [n, H, D] (q's dtype, or float32); lse [H, n] float32.
    row_order: optional scheduling permutation (no counterpart in the
    reference).
    """
    _require(k_cache.dim() == 4 and v_cache.shape == k_cache.shape,
             "k_cache/v_cache must be [C, KVH, BS, D]")
    C, KVH, BS, D = k_cache.shape
    _require(q.dim() == 3 and q.shape[2] == D, "head size mismatch")
    _require(q.shape[1] % KVH == 0, "num_heads must be a multiple of num_kv_heads")
    _require(k_cache.stride(3) == 1, "k_cache must be contiguous in head_size")
    paged_decode_partial(
        q, k_cache, v_cache, (k_cache.stride(0), k_cache.stride(1), k_cache.stride(2)),
        C, BS, KVH, block_table, lens, scale, out, lse, row_order=row_order,
    )


def _host_decode_args(q, k_cache, v_cache, block_table, lens, scale, out, lse,
                      num_threads: int):
    """fd_host_decode_partial's arguments for host_decode_attn /
    host_decode_start (None: no rows), after the checks both share."""
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache),
                    ("block_table", block_table), ("lens", lens), ("out", out), ("lse", lse)):
        _require(t.device.type == "cpu", f"{name} must be in host memory")
    _require(k_cache.dim() == 4 and v_cache.shape == k_cache.shape
             and k_cache.stride() == v_cache.stride(), "k_cache/v_cache must be [C, KVH, BS, D]")
    C, KVH, BS, D = k_cache.shape
    _require(q.dim() == 3 and q.shape[2] == D and out.shape == q.shape,
             "q and out must be [n, H, D] with the cache's head size")
    n, H = q.shape[0], q.shape[1]
    _require(H % KVH == 0, "num_heads must be a multiple of num_kv_heads")
    _require(k_cache.stride(3) == 1 and q.stride(2) == 1 and out.stride(2) == 1,
             "head_size must be the contiguous dim")
    kv_dt = _dtype_code(k_cache, "k_cache")
    _require(q.dtype == k_cache.dtype and v_cache.dtype == k_cache.dtype,
             "q, k_cache and v_cache must share a dtype")
    _require(out.dtype == q.dtype or out.dtype == torch.float32, "out must be q's dtype or float32")
    _require(lse.dtype == torch.float32 and tuple(lse.shape) == (H, n)
             and (n == 0 or lse.stride(1) == 1), "lse must be float32 [H, n]")
    _require(block_table.dtype == torch.int32 and lens.dtype == torch.int32
             and block_table.dim() == 2 and block_table.shape[0] == n and lens.shape == (n,),
             "block_table must be int32 [n, W] and lens int32 [n]")
    if n == 0:
        return None
    _require(block_table.stride(1) == 1, "block_table rows must be contiguous")
    _require(lens.is_contiguous(), "lens must be contiguous")
    return (q.data_ptr(), q.stride(0), q.stride(1),
            k_cache.data_ptr(), v_cache.data_ptr(),
            k_cache.stride(0), k_cache.stride(1), k_cache.stride(2),
            C,
            block_table.data_ptr(), block_table.stride(0), block_table.shape[1],
            lens.data_ptr(),
            n, H, KVH, D,
            BS, float(scale), kv_dt,
            out.data_ptr(), out.stride(0), out.stride(1), _DT[out.dtype],
            lse.data_ptr(), lse.stride(0),
            int(num_threads))


def host_decode_attn(q, k_cache, v_cache, block_table, lens, scale, out, lse,
                     num_threads: int = 0) -> None:
    """Host-tier partial computed by the host cores (fd_host_decode_partial):
    the signature and results of decode_attn above, i.e. of the reference's
    decode_attn (fastdecode/csrc/cpu_attn.cpp:456-489), with every tensor in
    host memory. Runs synchronously; num_threads 0 = one worker per CPU of
    the affinity mask (or FASTDECODE_CPU_THREADS)."""
    args = _host_decode_args(q, k_cache, v_cache, block_table, lens.contiguous(), scale, out,
                             lse, num_threads)
    if args is not None:
        _lib.check(_lib.load_lib().fd_host_decode_partial(*args))


class HostDecodeCall:
    """A host_decode_attn call queued on the library's runner thread
    (fd_host_decode_partial_start). It holds the call's tensors until
    wait(), which must be called once: it blocks until the call has run and
    returns the seconds the call itself took."""

    def __init__(self, call_id: int | None, keep: tuple) -> None:
        self._id, self._keep = call_id, keep

    def wait(self) -> float:
        if self._id is None:  # no rows, or already waited for
            self._keep = ()
            return 0.0
        secs = ctypes.c_double()
        call_id, self._id = self._id, None
        try:
            _lib.check(_lib.load_lib().fd_host_decode_wait(call_id, ctypes.byref(secs)))
        finally:
            self._keep = ()
        return secs.value


def host_decode_start(q, k_cache, v_cache, block_table, lens, scale, out, lse,
                      num_threads: int = 0, ready: torch.cuda.Event | None = None
                      ) -> HostDecodeCall:
    """host_decode_attn in the background: checks the arguments, queues the
    call on the library's runner thread (fd_host_decode_partial_start) and
    returns at once. The runner first waits for `ready` (e.g. an event
    recorded behind the copy of q to the host). out / lse are written by the
    time the returned call's wait() returns; until then no argument may be
    changed or freed."""
    lens = lens.contiguous()
    args = _host_decode_args(q, k_cache, v_cache, block_table, lens, scale, out, lse,
                             num_threads)
    if args is None:
        return HostDecodeCall(None, ())
    ev = None
    if ready is not None:
        ev = ready.cuda_event
        _require(ev != 0, "host_decode_start: the ready event was never recorded")
    call_id = ctypes.c_int64()
    _lib.check(_lib.load_lib().fd_host_decode_partial_start(ev, *args, ctypes.byref(call_id)))
    return HostDecodeCall(call_id.value, (q, k_cache, v_cache, block_table, lens, out, lse, ready))


def paged_decode(
    q: torch.Tensor,
    key_cache: torch.Tensor,
    value_cache: torch.Tensor,
    block_table: torch.Tensor,
    seqused_k: torch.Tensor,
    softmax_scale: float,
    out: torch.Tensor | None = None,
    lse: torch.Tensor | None = None,
    row_order: torch.Tensor | None = None,
    max_seqlen_k: int | None = None,
    total_tokens: int | None = None,
    timeline: torch.Tensor | None = None,
) -> tuple[torch.Tensor, torch.Tensor]:
    """HBM-tier partial in vLLM's paged layout: the decode call of
    flash_attn_varlen_func at fastdecode/backend.py:306-314 (one query token
    per row, block_table + seqused_k, return_softmax_lse=True).

    key_cache/value_cache [B, BS, KVH, D] (e.g. the K and V halves of the
    interleaved [B, BS, KVH, 2D] cache). Returns out [n, H, D] (q's dtype
    unless `out` is given) and lse [H, n] float32. Rows with seqused_k == 0
    give out = 0 and lse = -inf (no FA row filtering is needed).

    max_seqlen_k (flash_attn_varlen_func's argument: the longest row's token
    count, an int the host knows): when given, only the table's first
    ceil(max_seqlen_k / BS) columns are planned and read (a view with the
    table's row stride), so a table sized to the cache's capacity costs no
    more than one sized to the batch. A row longer than max_seqlen_k is then a
    range error: its out and lse are NaN.

    total_tokens (no counterpart in the reference: the sum of seqused_k,
    which a serving step's scheduler knows on the host): lets the launch plan tell rows of
    uneven length from equal ones, which want different task sizes. Results
    do not depend on it.

    timeline: measurement only (see paged_decode_partial).
    """
    _require(key_cache.dim() == 4 and value_cache.shape == key_cache.shape,
             "key_cache/value_cache must be [B, BS, KVH, D]")
    B, BS, KVH, D = key_cache.shape
    if max_seqlen_k is not None and block_table.dim() == 2:
        cols = max(1, -(-int(max_seqlen_k) // BS))
        if cols < block_table.shape[1]:
            block_table = block_table[:, :cols]
    n, H = q.shape[0], q.shape[1]
    if out is None:
        out = torch.empty_like(q)
    if lse is None:
        lse = torch.empty(H, n, dtype=torch.float32, device=q.device)
    _require(key_cache.stride(3) == 1, "key_cache must be contiguous in head_size")
    paged_decode_partial(
        q, key_cache, value_cache,
        (key_cache.stride(0), key_cache.stride(2), key_cache.stride(1)),
        B, BS, KVH, block_table, seqused_k, softmax_scale, out, lse, row_order=row_order,
        total_tokens=total_tokens, timeline=timeline,
    )
    return out, lse


def merge_attn_states(out, o_a, lse_a, o_b, lse_b, out_lse=None) -> None:
    """out = LSE-merge of two partials; vLLM merge_attn_states signature as
    used at fastdecode/backend.py:53-55 (rule of cpu_ops.py:93-113). o_b /
    lse_b may also be views of pinned host memory (the host cores' partial):
    the merge then reads them zero-copy over the link."""
    _lib.check(_lib.load_lib().fd_merge_attn_states(
        *_merge_args(out, o_a, lse_a, o_b, lse_b, out_lse), _stream_for(out)))


def _merge_args(out, o_a, lse_a, o_b, lse_b, out_lse) -> tuple:
    """fd_merge_attn_states' arguments but the stream, after the checks."""
    _require(out.dim() == 3 and o_a.shape == out.shape and o_b.shape == out.shape,
             "out, o_a, o_b must be [n, H, D] of one shape")
    n, H, D = out.shape
    for t, name in ((out, "out"), (o_a, "o_a")):
        _require(t.is_cuda and t.stride(2) == 1, f"{name} must be a GPU tensor contiguous in D")
    _require(o_b.stride(2) == 1, "o_b must be contiguous in D")
    _require(lse_a.is_cuda, "lse_a must be on the GPU")
    for t, name in ((lse_a, "lse_a"), (lse_b, "lse_b")):
        _require(t.dtype == torch.float32 and tuple(t.shape) == (H, n),
                 f"{name} must be float32 [H, n]")
        _require(n == 0 or t.stride(1) == 1, f"{name} rows must be contiguous")
    if out_lse is not None:
        _require(out_lse.dtype == torch.float32 and tuple(out_lse.shape) == (H, n) and
                 (n == 0 or out_lse.stride(1) == 1), "out_lse must be float32 [H, n]")
    return (out.data_ptr(), out.stride(0), out.stride(1), _dtype_code(out, "out"),
            o_a.data_ptr(), o_a.stride(0), o_a.stride(1), _dtype_code(o_a, "o_a"),
            lse_a.data_ptr(), lse_a.stride(0),
            device_ptr(o_b), o_b.stride(0), o_b.stride(1), _dtype_code(o_b, "o_b"),
            device_ptr(lse_b), lse_b.stride(0),
            out_lse.data_ptr() if out_lse is not None else None,
            out_lse.stride(0) if out_lse is not None else 0,
            n, H, D)


def _device_counter(t, what):
    if t is None:
        return None
    _require(t.is_cuda and t.dtype == torch.int32, f"{what}: int32 GPU tensor")
    return t.data_ptr()


def _cache_write(key, value, k_cache, v_cache, strides_btg, num_blocks, block_size,
                 slot_mapping, error_count, write_gate=None) -> None:
    _require(key.dim() == 3 and value.shape == key.shape, "key/value must be [T, KVH, D]")
    T, KVH, D = key.shape
    _require(key.stride(2) == 1 and value.stride(2) == 1, "key/value must be contiguous in D")
    _require(key.dtype == k_cache.dtype and value.dtype == key.dtype and v_cache.dtype == key.dtype,
             "key, value and caches must share a dtype")
    _require(slot_mapping.dtype == torch.int64 and slot_mapping.dim() == 1
             and slot_mapping.shape[0] >= T, "slot_mapping must be int64 [>= T]")
    if T == 0:
        return
    _require(key.is_cuda and value.is_cuda, "key/value must be on the GPU")
    slots = _on_device(slot_mapping, key.device).contiguous()
    err_ptr = _device_counter(error_count, "error_count")
    gate_ptr = _device_counter(write_gate, "write_gate")
    _require(err_ptr is None or err_ptr != gate_ptr,
             "error_count and write_gate must be different counters")
    _lib.check(
        _lib.load_lib().fd_reshape_and_cache(
            key.data_ptr(), key.stride(0), key.stride(1),
            value.data_ptr(), value.stride(0), value.stride(1),
            device_ptr(k_cache), device_ptr(v_cache),
            strides_btg[0], strides_btg[1], strides_btg[2],
            num_blocks,
            slots.data_ptr(), T,
            KVH, D, block_size,
            _dtype_code(key, "key"), err_ptr, gate_ptr,
            _stream_for(key),
        )
    )


def reshape_and_cache(key, value, key_cache, value_cache, slot_mapping,
                      kv_cache_dtype: str = "auto", k_scale=None, v_scale=None,
                      error_count: torch.Tensor | None = None,
                      write_gate: torch.Tensor | None = None) -> None:
    """vLLM reshape_and_cache_flash signature (fastdecode/backend.py:270-273):
    key_cache/value_cache [B, BS, KVH, D] views; slots < 0 are skipped.
    Only the unquantised cache ("auto"/fp16/bf16) is supported, as in the
    reference backend (fastdecode/backend.py:68,211-212).
    error_count: int32 [1] GPU counter of slots past the cache (never written).
    write_gate: int32 [1] GPU counter written by earlier work on the stream
    (e.g. plan_tiers' error count); nothing is written when it is non-zero."""
    _require(kv_cache_dtype in ("auto", "float16", "bfloat16", "fp16", "bf16"),
             f"quantized KV cache ({kv_cache_dtype}) is not supported")
    _require(key_cache.dim() == 4 and value_cache.shape == key_cache.shape
             and key_cache.stride() == value_cache.stride(), "caches must be [B, BS, KVH, D]")
    B, BS, KVH, D = key_cache.shape
    _require(key.shape[1] == KVH and key.shape[2] == D, "key shape does not match the cache")
    # the token count is the slot mapping's; key/value may carry padding rows
    T = slot_mapping.shape[0]
    _require(key.shape[0] >= T and value.shape[0] >= T, "fewer key/value rows than slots")
    _cache_write(key[:T], value[:T], key_cache, value_cache,
                 (key_cache.stride(0), key_cache.stride(1), key_cache.stride(2)),
                 B, BS, slot_mapping, error_count, write_gate)


def store_kv(k, v, slots, k_cache, v_cache) -> None:
    """Host-tier KV write, signature of cpu_attn.cpp:492-517.

    k, v [m, KVH, D]; slots [m] int64 (tier-relative); k_cache/v_cache
    [C, KVH, BS, D] pinned host memory (or HBM). Every slot is range-checked
    before anything is written; an out-of-range slot raises RuntimeError.
    """
    _require(k_cache.dim() == 4 and v_cache.shape == k_cache.shape
             and k_cache.stride() == v_cache.stride(), "caches must be [C, KVH, BS, D]")
    C, KVH, BS, D = k_cache.shape
    _require(slots.dtype == torch.int64, "slots must be int64")
    m = k.shape[0]
    if m == 0:
        return
    _require(k.dim() == 3 and k.shape[1] == KVH and k.shape[2] == D and v.shape == k.shape,
             "k/v must be [m, KVH, D] matching the cache")
    cap = C * BS
    if slots.is_cuda:
        bad = int(((slots[:m] < 0) | (slots[:m] >= cap)).sum())  # synchronises
        _require(bad == 0, f"host-tier slot out of range (capacity {cap})")
    else:
        host = slots[:m].contiguous()
        first = ctypes.c_int64(-1)
        _lib.check(_lib.load_lib().fd_check_slots(host.data_ptr(), m, cap, ctypes.byref(first)))
    dev = k.device if k.is_cuda else torch.device("cuda", torch.cuda.current_device())
    kk = _on_device(k, dev)
    vv = _on_device(v, dev)
    _cache_write(kk, vv, k_cache, v_cache,
                 (k_cache.stride(0), k_cache.stride(2), k_cache.stride(1)),
                 C, BS, slots[:m], None)


def stream_copy(dst: torch.Tensor, src: torch.Tensor) -> None:
    """Byte copy on the GPU with the attention kernels' 16-byte loads
    (measurement aid). Either side may be pinned host memory (read or written
    over the link); the copy runs on the current stream of the GPU side."""
    nbytes = src.numel() * src.element_size()
    _require(dst.numel() * dst.element_size() >= nbytes, "dst too small")
    gpu_side = dst if dst.is_cuda else src
    _require(gpu_side.is_cuda or torch.cuda.is_available(), "stream_copy needs a GPU")
    stream = _stream_for(gpu_side) if gpu_side.is_cuda else \
        torch.cuda.current_stream().cuda_stream
    _lib.check(_lib.load_lib().fd_stream_copy(device_ptr(dst), device_ptr(src), nbytes, stream))


def host_stream_read(t: torch.Tensor, num_threads: int = 0) -> int:
    """Reads every byte of the contiguous host tensor t (64-byte aligned, a
    multiple of 64 bytes long) on the host cores (fd_host_stream_read) and
    returns the XOR of its 64-bit words: the host cores' DRAM read rate, the
    bound of the host-core leg of the split step (measurement aid)."""
    _require(not t.is_cuda and t.is_contiguous(), "host_stream_read: contiguous host tensor")
    out = ctypes.c_uint64()
    _lib.check(_lib.load_lib().fd_host_stream_read(t.data_ptr(), t.numel() * t.element_size(),
                                                   int(num_threads), ctypes.byref(out)))
    return int(out.value)
