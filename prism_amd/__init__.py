"""prism_amd: MI355X-native paged KV-cache hot path of Prism (andre-fu/prism).

Drop-ins for Prism's engine/kv_cache.py (FlashAttnKVCache), engine/prefix_cache.py
(PrefixCache), the flash_attn.flash_attn_with_kvcache op it calls and the elementwise steps on
either side of it (QKV split + RoPE, RMSNorm, SiLU-mul; engine/executor.py,
engine/fused_kernels.py) and a device-resident block table for graph-captured decode batches
(DecodeBatch, replacing the per-step refill of engine/executor.py:320-356), backed by
hand-written gfx950 HIP kernels in libprism_kv.so (C ABI: include/prism_kv.h).  There is no
CPU path: device ops raise if the library is not built.
"""
from .attention import (PrismKVStatusError, append_kv, decode_attention, flash_attn_with_kvcache, poll_status,
                        prefill_attention, read_status, rope_decode_attention, set_status_checks, shared_prefix_of,
                        status_tensor)
from .decode_batch import DecodeBatch
from .epilogue import fused_rms_norm, fused_silu_mul, rms_norm, rope_qk, rope_tables, silu_mul
from .kv_cache import FlashAttnKVCache, KVCacheOutOfPages, copy_pages
from .prefix_cache import CachedPrefix, PrefixCache

__all__ = [
    "FlashAttnKVCache", "KVCacheOutOfPages", "PrefixCache", "CachedPrefix",
    "flash_attn_with_kvcache", "append_kv", "decode_attention", "prefill_attention",
    "copy_pages", "read_status", "poll_status", "set_status_checks", "PrismKVStatusError", "status_tensor",
    "shared_prefix_of", "rope_decode_attention",
    "rope_tables", "rope_qk", "rms_norm", "fused_rms_norm", "silu_mul", "fused_silu_mul",
    "DecodeBatch",
]
