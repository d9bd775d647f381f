"""ctypes binding of libprism_kv.so (declared in include/prism_kv.h).

The library is the only compute path: if it is missing or fails to load, every device op in this
package raises.  There is no CPU or PyTorch fallback.
"""
from __future__ import annotations

import ctypes
import re
import threading
from ctypes import c_float, c_int32, c_int64, c_size_t, c_void_p, c_char_p, POINTER
from pathlib import Path

LIB_PATH = Path(__file__).resolve().parent / "libprism_kv.so"
HEADER_PATH = Path(__file__).resolve().parent.parent / "include" / "prism_kv.h"

PKV_OK = 0
PKV_EINVAL = -1
PKV_EHIP = -2
PKV_ENOSPC = -3
PKV_STATUS_BAD_PAGE = 1
PKV_STATUS_BAD_POSITION = 2
PKV_STATUS_SHARED_PREFIX = 4
PKV_STATUS_PARTIAL_RANGE = 8
PKV_STATUS_MERGE_TIMEOUT = 16
PKV_DECODE_TWO_PASS = 1
PKV_DECODE_FUSED_MERGE = 2
PKV_DECODE_HEADS = 4
PKV_DECODE_RESET_COUNTERS = 8
ABI_VERSION = 1

_I64 = c_int64
_I32 = c_int32
_P = c_void_p

# argument lists mirror include/prism_kv.h one for one
_SIGNATURES = {
    "pkv_abi_version": (c_int32, []),
    "pkv_last_error": (c_char_p, []),
    "pkv_append": (c_int32, [
        _P, _I64, _I64, _I64,            # k_new + strides
        _P, _I64, _I64, _I64,            # v_new + strides
        _P, _P, _I64,                    # k_cache, v_cache, page stride
        _P, _I64, _P,                    # block_table, bt_stride, cache_seqlens
        _I32, _I32, _I32, _I32,          # batch, s_new, n_kv, head_dim
        _I32, _I32, _I32,                # page_size, num_pages, max_blocks
        _P, _P,                          # status, stream
    ]),
    "pkv_decode_workspace_bytes": (c_size_t, [_I32] * 8),
    "pkv_decode_attn": (c_int32, [
        _P, _I64, _I64, _I64,            # q
        _P, _I64, _I64, _I64,            # k_new
        _P, _I64, _I64, _I64,            # v_new
        _P, _P, _I64,                    # caches
        _P, _I64, _P,                    # block table, seqlens
        _P, _I64, _I64, _I64,            # out
        _P, c_size_t,                    # workspace
        _I32, _I32, _I32, _I32, _I32,    # batch, s_q, n_heads, n_kv, head_dim
        _I32, _I32, _I32,                # page_size, num_pages, max_blocks
        _I32, c_float, _I32, _I32,       # causal, scale, split_tokens, flags
        _P, _P,                          # status, stream
    ]),
    "pkv_decode_attn_rope": (c_int32, [
        _P, _I64, _I64, _I64,            # q
        _P, _I64, _I64, _I64,            # k_new
        _P, _I64, _I64, _I64,            # v_new
        _P, _P, _I64,                    # caches
        _P, _I64, _P,                    # block table, seqlens
        _P, _P, _I32,                    # cos, sin tables, n_pos
        _P, _I64, _I64, _I64,            # out
        _P, c_size_t,                    # workspace
        _I32, _I32, _I32, _I32, _I32,    # batch, s_q, n_heads, n_kv, head_dim
        _I32, _I32, _I32,                # page_size, num_pages, max_blocks
        _I32, c_float, _I32,             # causal, scale, flags
        _P, _P,                          # status, stream
    ]),
    "pkv_decode_attn_noalloc": (c_int32, [
        _P, _I64, _I64, _I64,            # q
        _P, _I64, _I64, _I64,            # k_new
        _P, _I64, _I64, _I64,            # v_new
        _P, _P, _I64,                    # caches
        _P, _I64, _P,                    # block table, seqlens
        _P, _I64, _I64, _I64,            # out
        _I32, _I32, _I32, _I32, _I32,    # batch, s_q, n_heads, n_kv, head_dim
        _I32, _I32, _I32,                # page_size, num_pages, max_blocks
        _I32, c_float, _I32, _I32,       # causal, scale, split_tokens, flags
        _P, _P,                          # status, stream
    ]),
    "pkv_prefill_attn": (c_int32, [
        _P, _I64, _I64, _I64,
        _P, _I64, _I64, _I64,
        _P, _I64, _I64, _I64,
        _P, _P, _I64,
        _P, _I64, _P,
        _P, _I64, _I64, _I64,
        _I32, _I32, _I32, _I32, _I32,
        _I32, _I32, _I32,
        _I32, c_float,
        _P, _P,
    ]),
    "pkv_copy_pages": (c_int32, [
        _P, _P, _I32,                    # src_bases, dst_bases, n_tensors
        _P, _P, _P, _I32,                # src_ids, dst_ids, fill_slots, n_pages
        _I64, _I64, _I64, _I32,          # strides, slot_bytes, page_slots
        _I32, _I32,                      # src/dst num pages
        _P, _P,
    ]),
    "pkv_gather_pages": (c_int32, [
        _P, _P, _I32,
        _P, _I32, _I32,                  # src_ids, n_pages, dst_first
        _I64, _I64, _I64,                # strides, page_bytes
        _I32, _I32,
        _P, _P,
    ]),
    "pkv_rope_qk": (c_int32, [
        _P, _I64, _I64, _P,              # qkv + strides, positions
        _P, _P, _I32,                    # cos, sin, n_pos
        _P, _P, c_float,                 # q_norm_w, k_norm_w, eps
        _P, _I64, _I64, _I64,            # q_out
        _P, _I64, _I64, _I64,            # k_out
        _P, _P, _I64,                    # caches
        _P, _I64, _P,                    # block table, seqlens
        _I32, _I32, _I32, _I32, _I32,    # batch, s_new, n_heads, n_kv, head_dim
        _I32, _I32, _I32,                # page_size, num_pages, max_blocks
        _P, _P,                          # status, stream
    ]),
    "pkv_rms_norm": (c_int32, [
        _P, _I64, _P, _I64, _P, _I64,    # x, residual, h_out
        _P, _P, _I64,                    # weight, out
        _I64, _I32, c_float, _P,         # rows, hidden, eps, stream
    ]),
    "pkv_silu_mul": (c_int32, [_P, _I64, _P, _I64, _P, _I64, _I64, _I32, _P]),
    "pkv_table_update": (c_int32, [_P, _I32, _I32, _P, _I64, _P, _I32, _I32, _I32, _P, _P]),
    "pkv_status_take": (c_int32, [_P, _P, _P]),           # status, dst, stream
    "pkv_cascade_workspace_bytes": (c_size_t, [_I32] * 8),
    "pkv_cascade_attn": (c_int32, [_P, _I64, _I64, _I64, _P, _I64, _I64, _I64, _P, _I64, _I64, _I64,
                                   _P, _P, _I64, _P, _I64, _P, _P, _I64, _I64, _I64, _P, c_size_t,
                                   _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, _I32, c_float, _P, _P]),
}

_lock = threading.Lock()
_lib: ctypes.CDLL | None = None


class PrismKVError(RuntimeError):
    """A libprism_kv call returned an error code."""


def header_symbols() -> list[str]:
    """Function names declared in include/prism_kv.h (read from the header text)."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"^\s*(?:const\s+)?\w+\*?\s+\*?(pkv_\w+)\s*\(", text, re.M)))


def load() -> ctypes.CDLL:
    """Load libprism_kv.so once; raise if it is not built."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is not None:
            return _lib
        if not LIB_PATH.exists():
            raise PrismKVError(
                f"{LIB_PATH} is not built; run `python -m prism_amd.build` (hipcc, gfx950) first")
        lib = ctypes.CDLL(str(LIB_PATH))
        for name, (res, args) in _SIGNATURES.items():
            fn = getattr(lib, name)
            fn.restype = res
            fn.argtypes = args
        ver = lib.pkv_abi_version()
        if ver != ABI_VERSION:
            raise PrismKVError(f"libprism_kv ABI version {ver} != expected {ABI_VERSION}")
        _lib = lib
        return lib


def use(path: Path) -> ctypes.CDLL:
    """Load another build of the library (bench.py's timeline-stamp variant) in place of the one
    loaded so far: every later call of this package goes to it."""
    global _lib, LIB_PATH
    with _lock:
        _lib = None
        LIB_PATH = Path(path)
    return load()


def check(rc: int, what: str) -> None:
    if rc != PKV_OK:
        msg = load().pkv_last_error().decode(errors="replace")
        raise PrismKVError(f"{what} failed (code {rc}): {msg}")
