/*
 * prism_kv.h -- C ABI of libprism_kv.so, the MI355X (gfx950) paged KV-cache hot path.
 *
 * The library replaces the GPU half of Prism's paged KV cache:
 *   - the third-party op flash_attn.flash_attn_with_kvcache(q, k_cache, v_cache, k=, v=,
 *     cache_seqlens=, block_table=, causal=True), which Prism calls at
 *     engine/executor.py:119-120, :151-153, :260-261, :385-386 and
 *     engine/speculative_executor.py:150-153 (append + paged attention in one call);
 *   - the per-page torch copy_ loop of FlashAttnKVCache.transfer_sequence
 *     (engine/kv_cache.py:189-207), generalised to copy-on-write and compaction;
 *   - the elementwise steps on either side of attention (QKV split + QK-norm + RoPE with the
 *     paged append, RMSNorm with the residual add, SiLU-mul: engine/executor.py,
 *     engine/fused_kernels.py);
 *   - the per-step refill of a graph-captured decode batch's block table and lengths
 *     (engine/kv_cache.py:147-151, engine/executor.py:345-353), as incremental updates.
 *
 * Conventions shared by every entry point:
 *   - All tensors are device pointers owned by the caller.  Nothing here allocates device
 *     memory or synchronises the host, so every call can be captured in a HIP graph.  The one
 *     piece of global mutable state is the static split-K scratch of pkv_decode_attn_noalloc
 *     (one array per GPU, shared by every noalloc call on it); every other entry point touches
 *     only the memory its arguments name.  Work is enqueued on `stream` (a hipStream_t; NULL =
 *     default).
 *   - K/V element type is bf16 (passed as raw 16-bit words).  A paged cache is laid out
 *     [num_pages, page_size, n_kv, head_dim] with the last three dims contiguous
 *     (engine/kv_cache.py:37-46); `*_page_stride` is the element distance between pages.
 *   - Strides are in elements (16-bit words) unless the name says _bytes.  The innermost
 *     (head_dim) dimension must be contiguous and every row 16-byte aligned.
 *   - block_table is int32 [batch, bt_stride] (only the first max_blocks columns are read;
 *     max_blocks * page_size, the keys a sequence may hold, is at most 2^27);
 *     cache_seqlens is int32 [batch] and holds each sequence's length BEFORE the append
 *     (engine/kv_cache.py:123-153).
 *   - `status` (nullable) is a device int32 the kernels OR error bits into instead of
 *     touching memory they must not: PKV_STATUS_BAD_PAGE when a block-table entry the call
 *     needs lies outside [0, num_pages).  The host reads it when it chooses to.
 *   - Return value: PKV_OK, or a negative PKV_E* code with a message in pkv_last_error()
 *     (thread-local).  Argument checks run on the host before anything is launched.
 */
#ifndef PRISM_KV_H
#define PRISM_KV_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PKV_ABI_VERSION 1

#define PKV_OK 0
#define PKV_EINVAL (-1)  /* bad shape, stride, alignment or size */
#define PKV_EHIP (-2)    /* a HIP runtime call or kernel launch failed */
#define PKV_ENOSPC (-3)  /* workspace smaller than pkv_decode_workspace_bytes() */

#define PKV_STATUS_BAD_PAGE 1
#define PKV_STATUS_BAD_POSITION 2  /* a rotary position outside the cos/sin table (clamped) */
#define PKV_STATUS_SHARED_PREFIX 4 /* pkv_cascade_attn: a sequence shorter than the shared prefix
                                      or not listing its pages, or (no append, causal) a query row
                                      that may not see the whole prefix */
#define PKV_STATUS_PARTIAL_RANGE 8 /* a balanced-kernel split-K partial (fp16 O / l) would exceed
                                      fp16's range: |V| >= 65520 somewhere; that output is inf.
                                      PKV_DECODE_HEADS keeps fp32 partials */
#define PKV_STATUS_MERGE_TIMEOUT 16 /* an in-launch merge (PKV_DECODE_FUSED_MERGE) waited past its
                                       bound for a sequence's split-K parts, or found its arrival
                                       counter left over from such a call; that output is stale.
                                       Never expected: it reports a broken arrival count.  The
                                       workspace's counter region (its first 64 KiB) is then no
                                       longer zero: clear it, or pass PKV_DECODE_RESET_COUNTERS
                                       once, before the next call that uses it */

/* pkv_decode_attn flags (0 = the library's choice of kernel and merge) */
#define PKV_DECODE_TWO_PASS 1    /* merge split-K partials in a second launch */
#define PKV_DECODE_FUSED_MERGE 2 /* merge split-K partials in the attention launch (per-head kernel:
                                    the last split to finish; balanced kernel with <= 16 query rows
                                    per KV head: merge workgroups appended to its grid) */
#define PKV_DECODE_HEADS 4       /* use the per-head kernel where the balanced one would run */
#define PKV_DECODE_RESET_COUNTERS 8 /* clear the workspace's (noalloc: the static scratch's) split-K
                                       arrival counters before the call: the recovery after
                                       PKV_STATUS_MERGE_TIMEOUT */
#define PKV_DECODE_GRID(n) ((int32_t)(n) << 8) /* balanced kernel on n (1..65535) workgroups, not one per CU */

/* ABI version of the loaded library (PKV_ABI_VERSION it was built with). */
int pkv_abi_version(void);

/* Message for the last failed call on this thread ("" if none). */
const char* pkv_last_error(void);

/*
 * Slot-mapped append (replaces the append half of flash_attn_with_kvcache(k=, v=)).
 * For b < batch, j < s_new:  slot = cache_seqlens[b] + j,
 *   k_cache[block_table[b, slot / page_size], slot % page_size] = k_new[b, j]   (same for v).
 * Bit-exact 16-byte copies.  k_new/v_new are [batch, s_new, n_kv, head_dim] with the given
 * batch/seq/head strides (Prism passes views into the fused QKV projection output).
 */
int pkv_append(const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
               const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh,
               void* k_cache, void* v_cache, int64_t cache_page_stride,
               const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens,
               int32_t batch, int32_t s_new, int32_t n_kv, int32_t head_dim,
               int32_t page_size, int32_t num_pages, int32_t max_blocks,
               int32_t* status, void* stream);

/*
 * Bytes of workspace pkv_decode_attn needs for these sizes (split-K partial outputs and
 * log-sum-exp terms).  split_tokens = 0 asks for the library's own choice, exactly as
 * pkv_decode_attn would make it with flags = 0 (a PKV_DECODE_GRID(n) above the device's CU count
 * needs 65536 + 2 n * 4 * R * 260 bytes, R = s_q * n_heads / n_kv).
 */
size_t pkv_decode_workspace_bytes(int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv,
                                  int32_t head_dim, int32_t page_size, int32_t max_blocks,
                                  int32_t split_tokens);

/*
 * Paged decode attention with GQA and split-K (flash_attn_with_kvcache with s_q small:
 * decode, s_q = 1, engine/executor.py:151-153, :260-261, :385-386; speculative verify,
 * s_q = k+1, engine/speculative_executor.py:150-153).  Needs s_q * (n_heads / n_kv) <= 64.
 *
 * If k_new/v_new are non-NULL they are appended at cache_seqlens[b] (as pkv_append) and the
 * keys are [0, cache_seqlens[b] + s_q); otherwise the keys are [0, cache_seqlens[b]).
 * Query j of sequence b (length L_b keys) attends to keys t <= L_b - s_q + j when causal
 * (bottom-right aligned), to all L_b keys otherwise.  Query head h reads KV head
 * h / (n_heads / n_kv).  Scores are scaled by softmax_scale (Prism uses the default
 * 1/sqrt(head_dim)); softmax and accumulation are fp32, out is bf16 [batch, s_q, n_heads,
 * head_dim] with the given strides.  A query row with no visible key gets zeros.
 * Two kernels serve the call.  Where head_dim = 128 (any n_kv) or head_dim = 64 with an even
 * n_kv (the Qwen2.5 decode and verify shapes, 0.5B to 72B, and their tensor-parallel shards),
 * batch <= 256, split_tokens = 0 and PKV_DECODE_HEADS is not set, a balanced kernel gives every
 * workgroup an equal share of all sequences' KV tiles (of every group of 4, 2 or 1 KV heads; a
 * tile is 32 tokens of 4 heads x 128, 64 of 2 x 128 or 4 x 64, 128 of 1 x 128 or 2 x 64, and
 * page_size must hold a whole tile); the sequences that straddle shares are merged by a second
 * launch (PKV_DECODE_TWO_PASS) or, for decode's <= 16 query rows per KV head, inside the launch
 * by merge workgroups that wait for a sequence's shares (PKV_DECODE_FUSED_MERGE).  With neither
 * flag the library merges inside the launch when those merge workgroups, batch * n_kv *
 * ceil(R / 4), are no more than the decode workgroups (one per CU), else in a second launch.
 * Otherwise a per-(sequence, KV head, split) kernel reduces split_tokens keys (a multiple of 32;
 * 0 = 512) per workgroup and merges the splits inside the launch (PKV_DECODE_TWO_PASS: in a
 * second launch).  Results agree up to rounding (fp32 order, fp16 split-K partials).
 * The balanced kernel keeps each split's normalised output in fp16, so it needs |V| < 65520
 * (bf16 V beyond that overflows the partial to inf and sets PKV_STATUS_PARTIAL_RANGE);
 * PKV_DECODE_HEADS keeps fp32 partials.
 * workspace must hold pkv_decode_workspace_bytes() bytes and be
 * zero-filled before its first use; every call leaves it in that state again (its first 64 KiB
 * hold the in-launch merges' arrival counters: per (sequence, KV head) for the per-head kernel,
 * so batch * n_kv <= 16384 when a sequence can span more than one split, and per (sequence, KV
 * head, group of 4 query rows) for the balanced kernel, which merges in a second launch when
 * more than 16384 would be needed).  Calls that share a workspace must be ordered (same
 * stream).  It may be NULL when pkv_decode_workspace_bytes() returns 0.
 */
int pkv_decode_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                    const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                    const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh,
                    void* k_cache, void* v_cache, int64_t cache_page_stride,
                    const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens,
                    void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                    void* workspace, size_t workspace_bytes,
                    int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                    int32_t page_size, int32_t num_pages, int32_t max_blocks,
                    int32_t causal, float softmax_scale, int32_t split_tokens, int32_t flags,
                    int32_t* status, void* stream);

/*
 * pkv_decode_attn without the workspace argument; it allocates nothing.  No counterpart in the
 * reference: it is for callers that cannot allocate or pass device memory for scratch (code
 * under HIP graph capture, tight serving loops, harnesses that forbid hipMalloc).  The split-K
 * counters and partials live in the library's own static device array of 48 MiB, one per GPU,
 * held until the process exits; a call that would need more (pkv_decode_workspace_bytes() >
 * 48 MiB, e.g. more than ~64 KiB of counters plus 2 * #CU * 4 * R * 260 bytes on the balanced
 * kernel) fails with PKV_ENOSPC before anything is launched.  Every call on a GPU shares that
 * GPU's array: calls that overlap on one GPU (unordered streams) race.  The first call on a
 * device looks the array up and clears its counters with a kernel on `stream`.  Same arguments
 * (minus workspace), results and errors as pkv_decode_attn, bit for bit.
 */
int pkv_decode_attn_noalloc(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                            const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                            const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh,
                            void* k_cache, void* v_cache, int64_t cache_page_stride,
                            const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens,
                            void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                            int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                            int32_t page_size, int32_t num_pages, int32_t max_blocks,
                            int32_t causal, float softmax_scale, int32_t split_tokens, int32_t flags,
                            int32_t* status, void* stream);

/*
 * pkv_decode_attn with the rotary embedding of the call's new tokens fused in: q and k_new arrive
 * unrotated (the QKV projection's output, e.g. strided views of one [B, s_q, (n_heads + 2 n_kv)
 * * head_dim] tensor) and token j of sequence b is rotated with row cache_seqlens[b] + j of
 * cos_tab / sin_tab ([n_pos, head_dim] bf16, the reference's cat([cos, cos]) tables) exactly as
 * the reference rotates q and k before its flash_attn call (engine/executor.py:149-153, :258-261:
 * out = x * cos + rotate_half(x) * sin, each bf16 op rounded), in the attention launch itself:
 * the appended cache rows are bit-identical to pkv_rope_qk's.  A position outside the table is
 * clamped and sets PKV_STATUS_BAD_POSITION.  Runs on the balanced decode kernel only (head_dim
 * 128, or 64 with an even n_kv; page_size a tile or more; batch <= 256) with s_q * n_heads / n_kv
 * + 2 s_q <= 16 (decode of every Qwen2.5 shape): other shapes fail with PKV_EINVAL.  Same
 * workspace (pkv_decode_workspace_bytes with split_tokens 0) and flags (PKV_DECODE_HEADS
 * excepted) as pkv_decode_attn.
 */
int pkv_decode_attn_rope(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                         const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                         const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh,
                         void* k_cache, void* v_cache, int64_t cache_page_stride,
                         const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens,
                         const void* cos_tab, const void* sin_tab, int32_t n_pos,
                         void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                         void* workspace, size_t workspace_bytes,
                         int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                         int32_t page_size, int32_t num_pages, int32_t max_blocks,
                         int32_t causal, float softmax_scale, int32_t flags,
                         int32_t* status, void* stream);

/*
 * Cascade (shared-prefix) attention: pkv_decode_attn for a batch whose sequences all list the
 * same pages for their first shared_tokens keys (branches of one prompt: the speculative verify
 * of engine/speculative_executor.py:113-164 over a cached prefix, engine/prefix_cache.py).
 * Same arguments and results as pkv_decode_attn (flags 0), plus shared_tokens: a multiple of
 * page_size, every sequence holding at least shared_tokens keys before the append.  The prefix
 * is read once for the whole batch (every query row against it, in key splits, on MFMA), the
 * rest of each sequence by the balanced decode kernel, and one launch merges both.  A sequence
 * shorter than the prefix or not listing sequence 0's prefix pages sets
 * PKV_STATUS_SHARED_PREFIX (its output is then meaningless; every access stays in the pool).
 * Shapes outside the balanced kernel's (see pkv_decode_attn) and shared_tokens = 0 run
 * pkv_decode_attn.  workspace: pkv_cascade_workspace_bytes() bytes, same rules as
 * pkv_decode_attn's.
 */
size_t pkv_cascade_workspace_bytes(int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv,
                                   int32_t head_dim, int32_t page_size, int32_t max_blocks,
                                   int32_t shared_tokens);

int pkv_cascade_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                     const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                     const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh,
                     void* k_cache, void* v_cache, int64_t cache_page_stride,
                     const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens,
                     void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                     void* workspace, size_t workspace_bytes,
                     int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                     int32_t page_size, int32_t num_pages, int32_t max_blocks, int32_t shared_tokens,
                     int32_t causal, float softmax_scale, int32_t* status, void* stream);

/*
 * Varlen chunked-prefill attention over paged KV (flash_attn_with_kvcache with s_q = chunk,
 * engine/executor.py:119-120), bf16 MFMA.  Same arguments and semantics as
 * pkv_decode_attn without the split-K workspace; any s_q >= 1.  When k_new/v_new are given
 * the chunk is appended first (pkv_append) and attention then reads it from the cache.
 */
int pkv_prefill_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                     const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                     const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh,
                     void* k_cache, void* v_cache, int64_t cache_page_stride,
                     const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens,
                     void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                     int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                     int32_t page_size, int32_t num_pages, int32_t max_blocks,
                     int32_t causal, float softmax_scale,
                     int32_t* status, void* stream);

/*
 * Batched page copy (generalises engine/kv_cache.py:189-207, the per-layer, per-page copy_
 * loop of transfer_sequence; also copy-on-write of a shared partially filled page and
 * live-page migration).  For every tensor i < n_tensors and pair p < n_pages:
 *   dst_bases[i] + dst_ids[p] * dst_page_stride_bytes  <-  the first fill_slots[p] slots
 *   (slot_bytes each) of  src_bases[i] + src_ids[p] * src_page_stride_bytes.
 * src_bases/dst_bases are DEVICE arrays of n_tensors addresses (e.g. the K then V base of
 * every layer); src_ids/dst_ids/fill_slots are DEVICE int32 arrays (fill_slots NULL = whole
 * page of page_slots slots).  Ids outside [0, src_num_pages) / [0, dst_num_pages) are
 * skipped and flagged in status.  Source and destination pages must not overlap.
 * Bit-exact 16-byte copies; slot_bytes and page strides must be multiples of 16.
 */
int pkv_copy_pages(const uint64_t* src_bases, const uint64_t* dst_bases, int32_t n_tensors,
                   const int32_t* src_ids, const int32_t* dst_ids, const int32_t* fill_slots,
                   int32_t n_pages, int64_t src_page_stride_bytes, int64_t dst_page_stride_bytes,
                   int64_t slot_bytes, int32_t page_slots,
                   int32_t src_num_pages, int32_t dst_num_pages,
                   int32_t* status, void* stream);

/*
 * Page gather / compaction into a fresh pool: pkv_copy_pages with dst_ids[p] = dst_first + p
 * and whole pages.  Used to pack every live page of a pool into pages [0, n) of another.
 */
int pkv_gather_pages(const uint64_t* src_bases, const uint64_t* dst_bases, int32_t n_tensors,
                     const int32_t* src_ids, int32_t n_pages, int32_t dst_first,
                     int64_t src_page_stride_bytes, int64_t dst_page_stride_bytes,
                     int64_t page_bytes, int32_t src_num_pages, int32_t dst_num_pages,
                     int32_t* status, void* stream);

/*
 * Pre-attention epilogue: QKV split, optional per-head RMSNorm (QK-norm) and rotary embedding,
 * replacing engine/executor.py:108-118 / :143-150 (q = qkv[..., :qs].view(.., nh, hd),
 * k, v likewise; fused_rms_norm(q, q_norm_w) and (k, k_norm_w) when the model has QK-norm;
 * q * cos + rotate_half(q) * sin and the same for k, with cos/sin rows from the
 * engine/executor.py:45-57 table).  For b < batch, j < s_new, token row
 * qkv + b * qkv_sb + j * qkv_ss = [q (n_heads * head_dim) | k (n_kv * head_dim) | v (n_kv * head_dim)]
 * at position positions[b] + j (row of cos_tab / sin_tab, bf16 [n_pos, head_dim]):
 *   q_out[b, j, h] = rope(norm(q_h)), k_out[b, j, h] = rope(norm(k_h)) (k_out may be NULL),
 * with the reference's bf16 rounding after each torch op, so the result is bit-exact against it
 * (to a bf16 unit where QK-norm is on).  q_norm_w / k_norm_w NULL = no QK-norm.
 * If k_cache/v_cache are non-NULL the rotated k and the unrotated v are also appended at
 * slot cache_seqlens[b] + j, as pkv_append (the flash_attn_with_kvcache(k=, v=) append half),
 * so the attention call that follows can pass k = v = NULL with cache_seqlens + s_new.
 * Positions outside [0, n_pos) are clamped and flag PKV_STATUS_BAD_POSITION.
 */
int pkv_rope_qk(const void* qkv, int64_t qkv_sb, int64_t qkv_ss, const int32_t* positions,
                const void* cos_tab, const void* sin_tab, int32_t n_pos,
                const void* q_norm_w, const void* k_norm_w, float eps,
                void* q_out, int64_t qo_sb, int64_t qo_ss, int64_t qo_sh,
                void* k_out, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh,
                void* k_cache, void* v_cache, int64_t cache_page_stride,
                const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens,
                int32_t batch, int32_t s_new, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                int32_t page_size, int32_t num_pages, int32_t max_blocks,
                int32_t* status, void* stream);

/*
 * RMSNorm over rows (engine/fused_kernels.py:31-65 fused_rms_norm; called at
 * engine/executor.py:106, :122, :131): out[r] = bf16(h * rsqrt(mean(h^2) + eps) * weight) in
 * fp32, h = x[r], or, when residual is non-NULL, h = bf16(x[r] + residual[r]) (the preceding
 * `hidden = residual + ...` of engine/executor.py:121, :127), also stored to h_out if non-NULL.
 * hidden a multiple of 8, at most 8192; rows 16-byte aligned.
 */
int pkv_rms_norm(const void* x, int64_t x_stride, const void* residual, int64_t r_stride,
                 void* h_out, int64_t h_stride, const void* weight, void* out, int64_t o_stride,
                 int64_t rows, int32_t hidden, float eps, void* stream);

/*
 * SiLU-gated MLP activation (engine/executor.py:127: F.silu(gu[..., :m]) * gu[..., m:], i.e.
 * gate = gu, up = gu + m; the Triton engine/fused_kernels.py:8-28 fused_silu_mul(gate, up)):
 * out[r, i] = bf16(bf16(silu(gate[r, i])) * up[r, i]) for i < m.  m a multiple of 8; rows
 * 16-byte aligned (row strides in elements).
 */
int pkv_silu_mul(const void* gate, int64_t g_stride, const void* up, int64_t u_stride,
                 void* out, int64_t o_stride, int64_t rows, int32_t m, void* stream);

/*
 * Incremental update of a device-resident decode block table and its cache_seqlens (replaces the
 * per-step refill of the reference's graph buffers: engine/kv_cache.py:147-151 writes every
 * block_table[i, j] and cache_seqlens[i] of the batch element by element, then
 * engine/executor.py:345-353 zeroes and copies the graph's static bt / sl).  packet (device
 * int32) holds n_len (row, length) pairs, then n_ent (row, column, page) triples:
 *   cache_seqlens[row] = length;   block_table[row * bt_stride + column] = page.
 * Entries outside rows x cols, negative lengths and pages outside [0, num_pages) are skipped and
 * flag PKV_STATUS_BAD_PAGE in *status.  One launch; asynchronous on `stream`.
 */
int pkv_table_update(const int32_t* packet, int32_t n_len, int32_t n_ent, int32_t* block_table,
                     int64_t bt_stride, int32_t* cache_seqlens, int32_t rows, int32_t cols,
                     int32_t num_pages, int32_t* status, void* stream);

/*
 * Asynchronous read of a status word: one atomic exchange on `stream` moves its bits to *dst (a
 * device int32) and leaves it 0, so bits that a kernel on another stream sets at the same time
 * are never lost between a read and a clear.  No counterpart in the reference (flash_attn has no
 * status word); it lets a host poll the word at the points it already passes through (a copy of
 * *dst to pinned memory and an event, no synchronisation) instead of after every call.
 */
int pkv_status_take(int32_t* status, int32_t* dst, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* PRISM_KV_H */
