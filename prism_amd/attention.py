"""flash_attn_with_kvcache drop-in over the gfx950 HIP kernels, plus the individual ops.

Prism imports ``from flash_attn import flash_attn_with_kvcache`` (engine/executor.py:11,
engine/speculative_executor.py:13) and calls it as
``flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v, cache_seqlens=sl, block_table=bt,
causal=True)`` (engine/executor.py:119-120, :151-153, :260-261, :385-386;
engine/speculative_executor.py:150-153).  This module provides a function of the same name and
argument meaning:

* ``q`` [B, s_q, n_heads, head_dim] bf16; ``k_cache``/``v_cache`` [num_pages, page_size, n_kv,
  head_dim] bf16 (page stride free, inner dims contiguous) mutated in place by the append;
* ``k``/``v`` [B, s_q, n_kv, head_dim] (optional) appended at ``cache_seqlens`` (int32 [B], the
  length before the append) through ``block_table`` (int32 [B, max_blocks]);
* query j attends keys ``t <= L_b - s_q + j`` when ``causal`` (bottom-right aligned), scale
  ``softmax_scale`` (default 1/sqrt(head_dim)); query head h reads KV head h // (n_heads/n_kv);
* returns a new bf16 ``out`` [B, s_q, n_heads, head_dim]; errors raise ``RuntimeError``.

Calls are asynchronous on the caller's current stream, allocate only ``out`` (and a cached,
grow-only split-K workspace per device and stream), and can be captured in a HIP graph once an
eager call on the device has sized the workspace (on any stream: a capture stream without one of
its own shares the largest, as Prism's warm-up on its current stream then capture on a new stream
needs).
"""
from __future__ import annotations

import math
import threading

import torch

from . import _lib

_BF16 = torch.bfloat16
_ws_lock = threading.Lock()
_workspaces: dict[tuple[int, int], torch.Tensor] = {}
_captured: set[int] = set()         # data_ptr of every workspace handed to a call under graph capture
_retired: list[torch.Tensor] = []   # outgrown workspaces a captured graph may still use
_status: dict[int, torch.Tensor] = {}
_STATUS_NAMES = {1: "BAD_PAGE", 2: "BAD_POSITION", 4: "SHARED_PREFIX", 8: "PARTIAL_RANGE", 16: "MERGE_TIMEOUT"}
# The split-K workspace's leading counter region (kCounterBytes in prism_amd/csrc/pkv_attention.hip:
# 16384 int32 arrival counters), then the balanced kernel's partial rows: per workgroup two slots of
# at most 4 KV heads x R rows x (128 fp16 + one fp32 log-sum-exp) = 260 bytes per row.
_COUNTER_BYTES = 65536
_LEAN_ROW_BYTES = 260


def _stream_ptr(device: torch.device) -> int:
    return torch.cuda.current_stream(device).cuda_stream


def _require_gpu(t: torch.Tensor, name: str) -> None:
    if t.device.type != "cuda":
        raise RuntimeError(f"{name} must be a ROCm device tensor (got {t.device}); "
                           "prism_amd has no CPU path")


def status_tensor(device: torch.device) -> torch.Tensor:
    """Per-device int32 the kernels OR error bits into (PKV_STATUS_BAD_PAGE = 1)."""
    idx = device.index if device.index is not None else torch.cuda.current_device()
    t = _status.get(idx)
    if t is None:
        t = torch.zeros(1, dtype=torch.int32, device=device)
        _status[idx] = t
    return t


def _dev_index(device: torch.device) -> int:
    return device.index if device.index is not None else torch.cuda.current_device()


class PrismKVStatusError(RuntimeError):
    """A kernel flagged an error bit in the device status word (PKV_STATUS_*): an output or a
    page write of some earlier call was skipped or is not to be trusted.  Raised at a host point
    the caller already passes through (FlashAttnKVCache.build_block_table / update_seqlens,
    DecodeBatch.step), a step or two after the call that set it."""

    def __init__(self, bits: int, device: int):
        names = [n for b, n in _STATUS_NAMES.items() if bits & b] or [hex(bits)]
        super().__init__(f"prism_amd kernel status on cuda:{device}: {'|'.join(names)} ({bits}) "
                         "(see PKV_STATUS_* in include/prism_kv.h)")
        self.bits = bits
        self.device = device


class _StatusCopies:
    """Asynchronous reads of one device's status word: pkv_status_take moves the bits into a
    device slot (atomic exchange with 0), a non-blocking copy brings the slot to pinned host
    memory, and an event says when it has landed.  Nothing on the host waits."""

    SLOTS = 4

    def __init__(self, device: torch.device):
        self.dev_slots = torch.zeros(self.SLOTS, dtype=torch.int32, device=device)
        self.host = torch.zeros(self.SLOTS, dtype=torch.int32, pin_memory=True)
        self.free = list(range(self.SLOTS))
        self.pending: list[tuple[torch.cuda.Event, int]] = []
        self.bits = 0   # landed on the host and not reported yet

    def collect(self, wait: bool) -> None:
        keep = []
        for ev, slot in self.pending:
            if wait:
                ev.synchronize()
            if wait or ev.query():
                self.bits |= int(self.host[slot])
                self.free.append(slot)
            else:
                keep.append((ev, slot))
        self.pending = keep

    def take(self, device: torch.device, status: torch.Tensor) -> None:
        if not self.free:
            return
        slot = self.free.pop()
        stream = torch.cuda.current_stream(device)
        rc = _lib.load().pkv_status_take(status.data_ptr(), self.dev_slots[slot:].data_ptr(), stream.cuda_stream)
        _lib.check(rc, "pkv_status_take")
        self.host[slot:slot + 1].copy_(self.dev_slots[slot:slot + 1], non_blocking=True)
        ev = torch.cuda.Event()
        ev.record(stream)
        self.pending.append((ev, slot))


_monitors: dict[int, _StatusCopies] = {}
_checks_enabled = True
_reset_counters: set[int] = set()   # devices whose noalloc scratch counters need clearing


def set_status_checks(enabled: bool) -> None:
    """Turn the status polls at build_block_table / update_seqlens / DecodeBatch.step on (the
    default) or off."""
    global _checks_enabled
    _checks_enabled = bool(enabled)


def _recover(idx: int, bits: int) -> None:
    """After PKV_STATUS_MERGE_TIMEOUT the split-K arrival counters of this device's workspaces may
    no longer be zero: clear them (stream-ordered) and have the next noalloc call clear the
    library's static scratch (PKV_DECODE_RESET_COUNTERS)."""
    if not bits & _lib.PKV_STATUS_MERGE_TIMEOUT:
        return
    with _ws_lock:
        for (d, _), ws in _workspaces.items():
            if d == idx:
                ws[:_COUNTER_BYTES].zero_()
    _reset_counters.add(idx)


def poll_status(device: torch.device | str = "cuda", raise_on_error: bool = True) -> int:
    """Non-blocking status check for a host point the caller passes through every step: collect
    the reads that have landed, start a new one (pkv_status_take on the current stream), and,
    when some landed read holds error bits, raise PrismKVStatusError (or return the bits with
    raise_on_error=False).  A bit set by a call is seen one or two polls later.  Nothing happens
    under HIP graph capture or with set_status_checks(False)."""
    device = torch.device(device)
    if not _checks_enabled or device.type != "cuda" or torch.cuda.is_current_stream_capturing():
        return 0
    idx = _dev_index(device)
    mon = _monitors.get(idx)
    if mon is None:
        mon = _monitors[idx] = _StatusCopies(device)
    mon.collect(wait=False)
    mon.take(device, status_tensor(device))
    bits, mon.bits = mon.bits, 0
    if bits:
        _recover(idx, bits)
        if raise_on_error:
            raise PrismKVStatusError(bits, idx)
    return bits


def read_status(device: torch.device | str = "cuda", clear: bool = True) -> int:
    """Synchronously read (and by default clear) the device status word, together with any bits
    an earlier poll_status moved to the host and has not reported yet."""
    device = torch.device(device)
    t = status_tensor(device)
    idx = _dev_index(device)
    mon = _monitors.get(idx)
    pending = 0
    if mon is not None:
        mon.collect(wait=True)
        pending = mon.bits
        if clear:
            mon.bits = 0
    v = int(t.item()) | pending
    if clear:
        t.zero_()
        _recover(idx, v)
    return v


def _workspace(device: torch.device, nbytes: int, stream: int, allow_static: bool = False) -> torch.Tensor | None:
    """Split-K workspace per (device, stream), grow-only, allocated zero-filled: its counter
    region must start at zero, and every call leaves it zero again.

    Under HIP graph capture nothing may be allocated.  Prism warms up on its current stream and
    then captures on a new one (engine/executor.py:186-197, :288-303), so a capture stream with
    no workspace of its own takes the largest one an eager call on this device sized; the graph's
    replays and the eager calls then share it, which is safe because Prism issues both from one
    thread in order.  With allow_static, a capture that finds no sized workspace gets None: the
    decode call then runs pkv_decode_attn_noalloc, whose scratch is the library's static device
    array.  A workspace that grows is dropped (the caching allocator reuses its memory) unless a
    call under graph capture was handed it: a captured graph keeps its address, so such a
    workspace is retired instead, kept alive for the rest of the process."""
    if nbytes == 0:
        return None
    idx = _dev_index(device)
    key = (idx, stream)
    capturing = torch.cuda.is_current_stream_capturing()
    with _ws_lock:
        ws = _workspaces.get(key)
        if ws is not None and ws.numel() >= nbytes:
            if capturing:
                _captured.add(ws.data_ptr())
            return ws
        if capturing:
            sized = [t for (d, _), t in _workspaces.items() if d == idx and t.numel() >= nbytes]
            if not sized:
                if allow_static:
                    return None   # the caller takes pkv_decode_attn_noalloc (the library's own scratch)
                raise RuntimeError(
                    f"split-K workspace of {nbytes} bytes must be sized by an eager call on this device "
                    "before HIP graph capture")
            ws = max(sized, key=lambda t: t.numel())
            _captured.add(ws.data_ptr())
        else:
            ws = torch.zeros(max(nbytes, 1 << 20), dtype=torch.uint8, device=device)
        old = _workspaces.get(key)
        _workspaces[key] = ws
        if old is not None and old.data_ptr() in _captured and \
                all(t.data_ptr() != old.data_ptr() for t in _workspaces.values()):
            _retired.append(old)
        return ws


def _decode_flags(two_pass: bool | None, kernel: str, grid: int) -> int:
    flags = 0
    if two_pass is not None:
        flags |= _lib.PKV_DECODE_TWO_PASS if two_pass else _lib.PKV_DECODE_FUSED_MERGE
    if kernel == "heads":
        flags |= _lib.PKV_DECODE_HEADS
    elif kernel != "auto":
        raise ValueError(f"kernel must be 'auto' or 'heads', got {kernel!r}")
    if not 0 <= int(grid) <= 0xFFFF:
        raise ValueError(f"grid {grid} outside [0, 65535]")
    return flags | (int(grid) << 8)


def _rows(t: torch.Tensor, name: str, nheads: int, hd: int) -> tuple[int, int, int]:
    if t.dtype != _BF16:
        raise RuntimeError(f"{name} must be bfloat16, got {t.dtype}")
    if t.dim() != 4 or t.shape[2] != nheads or t.shape[3] != hd:
        raise RuntimeError(f"{name} has shape {tuple(t.shape)}, expected [B, s, {nheads}, {hd}]")
    if t.stride(3) != 1:
        raise RuntimeError(f"{name} must be contiguous in head_dim")
    return t.stride(0), t.stride(1), t.stride(2)


def _check_cache(k_cache: torch.Tensor, v_cache: torch.Tensor) -> tuple[int, int, int, int]:
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        _require_gpu(t, name)
        if t.dtype != _BF16:
            raise RuntimeError(f"{name} must be bfloat16, got {t.dtype}")
        if t.dim() != 4:
            raise RuntimeError(f"{name} must be [num_pages, page_size, n_kv, head_dim]")
    if k_cache.shape != v_cache.shape or k_cache.stride() != v_cache.stride():
        raise RuntimeError("k_cache and v_cache must have the same shape and strides")
    num_pages, page_size, n_kv, hd = k_cache.shape
    if k_cache.stride()[1:] != (n_kv * hd, hd, 1):
        raise RuntimeError("k_cache/v_cache must be contiguous within a page")
    return num_pages, page_size, n_kv, hd


def _check_table(block_table: torch.Tensor, cache_seqlens: torch.Tensor, batch: int, device) -> None:
    if block_table.dtype != torch.int32 or cache_seqlens.dtype != torch.int32:
        raise RuntimeError("block_table and cache_seqlens must be int32")
    if block_table.dim() != 2 or block_table.shape[0] != batch or block_table.stride(1) != 1:
        raise RuntimeError(f"block_table must be [B={batch}, max_blocks] with unit column stride")
    if cache_seqlens.dim() != 1 or cache_seqlens.shape[0] != batch or cache_seqlens.stride(0) != 1:
        raise RuntimeError(f"cache_seqlens must be a contiguous [B={batch}] tensor")
    if block_table.device != device or cache_seqlens.device != device:
        raise RuntimeError("block_table/cache_seqlens must live on the cache's device")


def append_kv(k_cache, v_cache, k, v, cache_seqlens, block_table, *, status=None) -> None:
    """Slot-mapped append only (the append half of flash_attn_with_kvcache)."""
    num_pages, page_size, n_kv, hd = _check_cache(k_cache, v_cache)
    batch, s_new = k.shape[0], k.shape[1]
    ks = _rows(k, "k", n_kv, hd)
    vs = _rows(v, "v", n_kv, hd)
    if tuple(v.shape) != tuple(k.shape):
        raise RuntimeError("k and v must have the same shape")
    _check_table(block_table, cache_seqlens, batch, k_cache.device)
    if batch == 0 or s_new == 0:
        return
    st = status if status is not None else status_tensor(k_cache.device)
    lib = _lib.load()
    rc = lib.pkv_append(
        k.data_ptr(), *ks, v.data_ptr(), *vs,
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
        block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(),
        batch, s_new, n_kv, hd, page_size, num_pages, block_table.shape[1],
        st.data_ptr(), _stream_ptr(k_cache.device))
    _lib.check(rc, "pkv_append")


# Cascade attention is taken by itself (shared_prefix_tokens=None) from this many shared keys and
# sequences on: at the Qwen2.5-7B verify shape (64 sequences, 5 query rows) the ordinary call is
# faster at a 1792-key shared prefix (58.1-58.2 vs 59.8-60.7 us per layer) and the cascade 1.9x
# faster at 7936; interpolated, the two cross near 2.2k shared keys.
AUTO_CASCADE_MIN_TOKENS = 2048
AUTO_CASCADE_MIN_BATCH = 4


def shared_prefix_of(block_table: torch.Tensor, cache_seqlens, *, s_q: int = 1, causal: bool = True,
                     appends: bool = True, page_size: int | None = None) -> int:
    """Keys every sequence of the batch shares, as FlashAttnKVCache.build_block_table recorded
    them for this block_table (identical leading pages that every sequence fills); 0 when the
    table did not come from there, when either tensor has been written since (torch's version
    counters), when cache_seqlens is not the tensor built with it, or under HIP graph capture
    (a captured launch would keep the prefix for every replay).

    Cascade attention gives every query row the whole prefix.  Without an append, a causal call
    with s_q > 1 lets query row 0 see only keys t <= min(cache_seqlens) - s_q, so the prefix is
    cut to the whole pages below that bound (page_size: the cache's)."""
    meta = getattr(block_table, "_pkv_shared_prefix", None)
    if not meta or not isinstance(cache_seqlens, torch.Tensor):
        return 0
    tokens, bt_version, sl_ptr, sl_version, sl_min = meta
    if tokens <= 0 or block_table._version != bt_version:
        return 0
    if cache_seqlens.data_ptr() != sl_ptr or cache_seqlens._version != sl_version:
        return 0
    if block_table.is_cuda and torch.cuda.is_current_stream_capturing():
        return 0
    if causal and not appends and s_q > 1:
        seen = sl_min - s_q + 1            # keys row 0 sees in the shortest sequence
        P = int(page_size) if page_size else 1
        tokens = min(tokens, max(seen, 0) // P * P)
    return int(tokens)


def flash_attn_with_kvcache(
    q: torch.Tensor,
    k_cache: torch.Tensor,
    v_cache: torch.Tensor,
    k: torch.Tensor | None = None,
    v: torch.Tensor | None = None,
    rotary_cos=None,
    rotary_sin=None,
    cache_seqlens: torch.Tensor | int | None = None,
    cache_batch_idx=None,
    cache_leftpad=None,
    block_table: torch.Tensor | None = None,
    softmax_scale: float | None = None,
    causal: bool = False,
    window_size=(-1, -1),
    softcap: float = 0.0,
    rotary_interleaved: bool = True,
    alibi_slopes=None,
    num_splits: int = 0,
    return_softmax_lse: bool = False,
    *,
    out: torch.Tensor | None = None,
    split_tokens: int = 0,
    two_pass: bool | None = None,
    kernel: str = "auto",
    grid: int = 0,
    shared_prefix_tokens: int | None = None,
    noalloc: bool = False,
    status: torch.Tensor | None = None,
) -> torch.Tensor:
    """Append k/v into the paged cache and attend (see module docstring for the contract).

    Arguments Prism never passes (rotary_*, cache_batch_idx, cache_leftpad, window_size,
    softcap, alibi_slopes, return_softmax_lse) must keep their defaults.  ``num_splits`` > 0
    fixes the number of KV splits per sequence; ``split_tokens`` > 0 (a multiple of 32) fixes
    the split length directly (both select the per-head kernel); ``two_pass`` True merges the
    split-K partials in a second launch, False inside the attention launch (by the last split to
    finish, or by merge workgroups of the balanced kernel), None lets the library choose (the
    per-head kernel merges in the launch; the balanced kernel does when its merge workgroups,
    batch * n_kv * ceil(s_q * n_heads / n_kv / 4), are no more than its CUs, and decode rows
    only).  ``kernel="heads"`` forces the per-head kernel where the balanced one would run;
    ``grid`` > 0 runs the balanced kernel on that many workgroups instead of one per CU.

    ``shared_prefix_tokens`` > 0 (a multiple of the page size) declares that every sequence of
    the batch lists the same pages for its first shared_prefix_tokens keys and holds at least
    that many keys before the append (branches of one prompt, e.g. a speculative verify batch):
    cascade attention then reads that prefix once for the whole batch (pkv_cascade_attn).
    A sequence that breaks the promise sets PKV_STATUS_SHARED_PREFIX in the status word.
    Shapes the cascade does not cover run the ordinary decode path.  None (the default) takes
    the prefix FlashAttnKVCache.build_block_table recorded for this block_table and
    cache_seqlens (shared_prefix_of), when it is at least AUTO_CASCADE_MIN_TOKENS keys over at
    least AUTO_CASCADE_MIN_BATCH sequences; 0 never takes the cascade.

    ``noalloc`` runs a decode / verify call on pkv_decode_attn_noalloc: its split-K scratch is the
    library's static 48 MiB device array instead of a workspace this module allocates (calls on
    one GPU then share that array and must be ordered).  A decode call under HIP graph capture
    with no workspace sized by an earlier eager call takes the same path.
    """
    if rotary_cos is not None or rotary_sin is not None or cache_batch_idx is not None \
            or cache_leftpad is not None or tuple(window_size) != (-1, -1) or softcap != 0.0 \
            or alibi_slopes is not None or return_softmax_lse:
        raise NotImplementedError("prism_amd.flash_attn_with_kvcache supports the arguments Prism uses: "
                                  "q, k_cache, v_cache, k, v, cache_seqlens, block_table, "
                                  "softmax_scale, causal, num_splits")
    _require_gpu(q, "q")
    num_pages, page_size, n_kv, hd = _check_cache(k_cache, v_cache)
    if q.dim() != 4:
        raise RuntimeError(f"q must be [B, s_q, n_heads, head_dim], got {tuple(q.shape)}")
    batch, s_q, n_heads, qhd = q.shape
    if qhd != hd:
        raise RuntimeError(f"q head_dim {qhd} != cache head_dim {hd}")
    if n_heads % n_kv:
        raise RuntimeError(f"n_heads {n_heads} must be a multiple of n_kv {n_kv}")
    qs = _rows(q, "q", n_heads, hd)
    device = k_cache.device
    if q.device != device:
        raise RuntimeError("q must be on the cache's device")

    if (k is None) != (v is None):
        raise RuntimeError("k and v must both be given or both be None")
    if k is not None:
        if k.shape[0] != batch or k.shape[1] != s_q or tuple(v.shape) != tuple(k.shape):
            raise RuntimeError("k/v must be [B, s_q, n_kv, head_dim] matching q")
        ks = _rows(k, "k", n_kv, hd)
        vs = _rows(v, "v", n_kv, hd)
        kp, vp = k.data_ptr(), v.data_ptr()
    else:
        ks = vs = (0, 0, 0)
        kp = vp = 0

    if cache_seqlens is None:
        raise RuntimeError("cache_seqlens is required")
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((batch,), cache_seqlens, dtype=torch.int32, device=device)
    if block_table is None:
        # a non-paged cache [B, seqlen, n_kv, hd] is one page per sequence
        if num_pages != batch:
            raise RuntimeError("without block_table, k_cache must be [B, seqlen_cache, n_kv, head_dim]")
        block_table = torch.arange(batch, dtype=torch.int32, device=device).view(batch, 1)
    _check_table(block_table, cache_seqlens, batch, device)
    if page_size < 16 or page_size & (page_size - 1):
        raise RuntimeError(f"page_size {page_size} must be a power of two >= 16")
    max_blocks = block_table.shape[1]
    scale = float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(hd)

    if out is None:
        out = torch.empty((batch, s_q, n_heads, hd), dtype=_BF16, device=device)
    os_ = _rows(out, "out", n_heads, hd)
    if batch == 0:
        return out
    st = status if status is not None else status_tensor(device)
    lib = _lib.load()
    stream = _stream_ptr(device)
    g = n_heads // n_kv
    if shared_prefix_tokens is None:
        auto = shared_prefix_of(block_table, cache_seqlens, s_q=s_q, causal=causal, appends=k is not None,
                                page_size=page_size)
        shared_prefix_tokens = auto if auto >= AUTO_CASCADE_MIN_TOKENS and batch >= AUTO_CASCADE_MIN_BATCH else 0
    if noalloc:
        shared_prefix_tokens = 0   # the cascade needs a workspace of this module's
    if s_q * g <= 64:
        if num_splits and num_splits > 0 and not split_tokens:
            per_split = -(-(max_blocks * page_size) // num_splits)
            split_tokens = max(32, -(-per_split // 32) * 32)
        if shared_prefix_tokens and not split_tokens and kernel == "auto" and not grid and two_pass is not False:
            nbytes = lib.pkv_cascade_workspace_bytes(batch, s_q, n_heads, n_kv, hd, page_size, max_blocks,
                                                     int(shared_prefix_tokens))
            ws = _workspace(device, nbytes, stream)
            rc = lib.pkv_cascade_attn(
                q.data_ptr(), *qs, kp, *ks, vp, *vs,
                k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
                block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(),
                out.data_ptr(), *os_,
                ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0,
                batch, s_q, n_heads, n_kv, hd, page_size, num_pages, max_blocks, int(shared_prefix_tokens),
                1 if causal else 0, scale, st.data_ptr(), stream)
            _lib.check(rc, "pkv_cascade_attn")
            return out
        nbytes = lib.pkv_decode_workspace_bytes(batch, s_q, n_heads, n_kv, hd, page_size, max_blocks,
                                                int(split_tokens))
        if grid:  # the balanced kernel's partials for `grid` workgroups (prism_kv.h's bound)
            nbytes = max(nbytes, _COUNTER_BYTES + 2 * int(grid) * 4 * s_q * g * _LEAN_ROW_BYTES)
        ws = None if noalloc else _workspace(device, nbytes, stream, allow_static=True)
        if noalloc or (ws is None and nbytes > 0):
            idx = _dev_index(device)
            flags = _decode_flags(two_pass, kernel, grid)
            reset = idx in _reset_counters and not torch.cuda.is_current_stream_capturing()
            if reset:   # after a merge timeout: clear the static scratch's counters first
                flags |= _lib.PKV_DECODE_RESET_COUNTERS
            rc = lib.pkv_decode_attn_noalloc(
                q.data_ptr(), *qs, kp, *ks, vp, *vs,
                k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
                block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(),
                out.data_ptr(), *os_,
                batch, s_q, n_heads, n_kv, hd, page_size, num_pages, max_blocks,
                1 if causal else 0, scale, int(split_tokens), flags,
                st.data_ptr(), stream)
            _lib.check(rc, "pkv_decode_attn_noalloc")
            if reset:
                _reset_counters.discard(idx)
            return out
        rc = lib.pkv_decode_attn(
            q.data_ptr(), *qs, kp, *ks, vp, *vs,
            k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
            block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(),
            out.data_ptr(), *os_,
            ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0,
            batch, s_q, n_heads, n_kv, hd, page_size, num_pages, max_blocks,
            1 if causal else 0, scale, int(split_tokens), _decode_flags(two_pass, kernel, grid),
            st.data_ptr(), stream)
        _lib.check(rc, "pkv_decode_attn")
    else:
        rc = lib.pkv_prefill_attn(
            q.data_ptr(), *qs, kp, *ks, vp, *vs,
            k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
            block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(),
            out.data_ptr(), *os_,
            batch, s_q, n_heads, n_kv, hd, page_size, num_pages, max_blocks,
            1 if causal else 0, scale, st.data_ptr(), stream)
        _lib.check(rc, "pkv_prefill_attn")
    return out


def decode_attention(q, k_cache, v_cache, k=None, v=None, *, cache_seqlens, block_table,
                     causal=True, softmax_scale=None, split_tokens=0, two_pass=None, kernel="auto", grid=0,
                     out=None, status=None):
    """Force the split-K decode kernel (s_q * n_heads / n_kv <= 64)."""
    n_kv = k_cache.shape[2]
    if q.shape[1] * (q.shape[2] // n_kv) > 64:
        raise RuntimeError("decode_attention needs s_q * n_heads / n_kv <= 64")
    return flash_attn_with_kvcache(q, k_cache, v_cache, k, v, cache_seqlens=cache_seqlens,
                                   block_table=block_table, causal=causal, softmax_scale=softmax_scale,
                                   split_tokens=split_tokens, two_pass=two_pass, kernel=kernel, grid=grid,
                                   shared_prefix_tokens=0, out=out, status=status)


def rope_decode_attention(qkv: torch.Tensor, k_cache: torch.Tensor, v_cache: torch.Tensor, cos: torch.Tensor,
                          sin: torch.Tensor, *, cache_seqlens: torch.Tensor, block_table: torch.Tensor, n_heads: int,
                          n_kv: int, causal: bool = True, softmax_scale: float | None = None,
                          two_pass: bool | None = None, grid: int = 0, out: torch.Tensor | None = None,
                          status: torch.Tensor | None = None) -> torch.Tensor:
    """The reference's decode attention from the fused QKV projection on, in one launch
    (pkv_decode_attn_rope): the QKV split of ``qkv`` [B, s_q, (n_heads + 2 n_kv) * hd] by strided
    views, q and k rotated at positions cache_seqlens[b] + j with rows of ``cos`` / ``sin``
    ([n_pos, hd], rope_tables), the rotated k and v appended at cache_seqlens[b] + j, and paged
    attention over the cache -- the same values as

        q, k, v = split(qkv); q = q * cos + rotate_half(q) * sin; k = k * cos + rotate_half(k) * sin
        flash_attn_with_kvcache(q, k_cache, v_cache, k=k, v=v, cache_seqlens=..., block_table=...)

    (engine/executor.py:141-153, :250-261; the appended rows bit-identical to rope_qk's).  Decode
    shapes only: the balanced kernel with s_q * n_heads / n_kv + 2 s_q <= 16 (every Qwen2.5
    model's decode step); other shapes raise -- call rope_qk, then flash_attn_with_kvcache."""
    _require_gpu(qkv, "qkv")
    num_pages, page_size, kv_heads, hd = _check_cache(k_cache, v_cache)
    if kv_heads != n_kv:
        raise RuntimeError(f"n_kv {n_kv} != the cache's {kv_heads} KV heads")
    if qkv.dtype != _BF16 or qkv.dim() != 3 or qkv.shape[2] != (n_heads + 2 * n_kv) * hd or qkv.stride(2) != 1:
        raise RuntimeError(f"qkv must be bfloat16 [B, s_q, {(n_heads + 2 * n_kv) * hd}], contiguous in its last dim")
    if qkv.device != k_cache.device:
        raise RuntimeError("qkv must be on the cache's device")
    for name, t in (("cos", cos), ("sin", sin)):
        if t.dtype != _BF16 or t.dim() != 2 or t.shape[1] != hd or not t.is_contiguous() or t.device != qkv.device:
            raise RuntimeError(f"{name} must be a contiguous bfloat16 [n_pos, {hd}] table on the qkv device")
    if cos.shape != sin.shape:
        raise RuntimeError("cos and sin tables differ in shape")
    batch, s_q = qkv.shape[0], qkv.shape[1]
    q = qkv[:, :, :n_heads * hd].unflatten(2, (n_heads, hd))
    k = qkv[:, :, n_heads * hd:(n_heads + n_kv) * hd].unflatten(2, (n_kv, hd))
    v = qkv[:, :, (n_heads + n_kv) * hd:].unflatten(2, (n_kv, hd))
    qs, ks, vs = _rows(q, "q", n_heads, hd), _rows(k, "k", n_kv, hd), _rows(v, "v", n_kv, hd)
    device = k_cache.device
    _check_table(block_table, cache_seqlens, batch, device)
    max_blocks = block_table.shape[1]
    scale = float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(hd)
    if out is None:
        out = torch.empty((batch, s_q, n_heads, hd), dtype=_BF16, device=device)
    os_ = _rows(out, "out", n_heads, hd)
    if batch == 0:
        return out
    st = status if status is not None else status_tensor(device)
    lib = _lib.load()
    stream = _stream_ptr(device)
    nbytes = lib.pkv_decode_workspace_bytes(batch, s_q, n_heads, n_kv, hd, page_size, max_blocks, 0)
    if grid:
        nbytes = max(nbytes, _COUNTER_BYTES + 2 * int(grid) * 4 * s_q * (n_heads // n_kv) * _LEAN_ROW_BYTES)
    ws = _workspace(device, nbytes, stream)
    rc = lib.pkv_decode_attn_rope(
        q.data_ptr(), *qs, k.data_ptr(), *ks, v.data_ptr(), *vs,
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
        block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(),
        cos.data_ptr(), sin.data_ptr(), cos.shape[0],
        out.data_ptr(), *os_,
        ws.data_ptr() if ws is not None else 0, ws.numel() if ws is not None else 0,
        batch, s_q, n_heads, n_kv, hd, page_size, num_pages, max_blocks,
        1 if causal else 0, scale, _decode_flags(two_pass, "auto", grid), st.data_ptr(), stream)
    _lib.check(rc, "pkv_decode_attn_rope")
    return out


def prefill_attention(q, k_cache, v_cache, k=None, v=None, *, cache_seqlens, block_table,
                      causal=True, softmax_scale=None, out=None, status=None):
    """Force the row-parallel prefill kernel (any s_q)."""
    _require_gpu(q, "q")
    num_pages, page_size, n_kv, hd = _check_cache(k_cache, v_cache)
    batch, s_q, n_heads, _ = q.shape
    qs = _rows(q, "q", n_heads, hd)
    if k is not None:
        ks, vs, kp, vp = _rows(k, "k", n_kv, hd), _rows(v, "v", n_kv, hd), k.data_ptr(), v.data_ptr()
    else:
        ks = vs = (0, 0, 0)
        kp = vp = 0
    _check_table(block_table, cache_seqlens, batch, k_cache.device)
    if out is None:
        out = torch.empty((batch, s_q, n_heads, hd), dtype=_BF16, device=q.device)
    os_ = _rows(out, "out", n_heads, hd)
    if batch == 0:
        return out
    st = status if status is not None else status_tensor(k_cache.device)
    scale = float(softmax_scale) if softmax_scale is not None else 1.0 / math.sqrt(hd)
    rc = _lib.load().pkv_prefill_attn(
        q.data_ptr(), *qs, kp, *ks, vp, *vs,
        k_cache.data_ptr(), v_cache.data_ptr(), k_cache.stride(0),
        block_table.data_ptr(), block_table.stride(0), cache_seqlens.data_ptr(),
        out.data_ptr(), *os_, batch, s_q, n_heads, n_kv, hd, page_size, num_pages,
        block_table.shape[1], 1 if causal else 0, scale, st.data_ptr(), _stream_ptr(q.device))
    _lib.check(rc, "pkv_prefill_attn")
    return out
