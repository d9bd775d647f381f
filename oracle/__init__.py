"""ORACLE -- test infrastructure, not product code.

CPU restatement of the reference's paged KV-cache hot path, used only as the checker:
only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import it.  The
product package (prism_amd) never imports it and has no CPU fallback.

Modules
  paged_attention  flash_attn_with_kvcache semantics as Prism uses them: slot mapping, append,
                   fp64 brute-force paged attention, and the torch-CPU "reference path"
                   (index_select page gather + fp32 SDPA with GQA) timed as the CPU baseline.
  page_ops         page copy / copy-on-write / gather-compaction restatements (bit-exact).
  kv_state         the FlashAttnKVCache allocator and PrefixCache state machines, restated
                   from engine/kv_cache.py and engine/prefix_cache.py without tensors.
  epilogue         the elementwise steps around attention: rotary tables, QKV split + QK-norm +
                   RoPE, RMSNorm with the residual add, SiLU(gate) * up.

How each function is pinned (tests/test_oracle.py; the epilogue in tests/test_epilogue_oracle.py):
  slot_mapping / append_kv     docs/architecture.md:140-147 worked example, hand-computed slots,
                               a per-token brute-force loop, and the flash_attn docstring's layout.
  attention_fp64               torch SDPA (fp64, enable_gqa) on s_q == s_k where top-left and
                               bottom-right causal coincide; the flash_attn docstring's causal
                               mask example (seqlen_q=2, seqlen_k=5) and GQA head map example;
                               closed forms (one key -> out = v, identical keys -> mean(V),
                               a dominant logit selects its V row).
  flash_attn_cpu               agrees with attention_fp64 (two independent formulations).
  page_ops                     closed-form index arithmetic against per-element loops.
  kv_state                     golden traces recorded from the reference's own
                               engine/kv_cache.py / engine/prefix_cache.py (tests/golden/).
  epilogue.rope_bf16           an element-by-element restatement with explicit bf16 rounding
                               (bit-exact), the identity at position 0, the fp64 complex rotation
                               (rope_f64) and norm preservation; rope_tables against math.cos/sin.
  epilogue.rms_norm_f64        torch.nn.functional.rms_norm (fp64), constant rows (closed form),
                               scale invariance.
  epilogue.silu_mul_ref        torch.nn.functional.silu (fp64), silu(0) = 0 and the large-|g| limits.
"""
