// Slot-mapped K/V append into a paged cache: one 16-byte chunk per lane, so a wavefront moves
// 1 KiB of a token row with coalesced global_load_dwordx4 / global_store_dwordx4.
//
// Semantics follow the append half of flash_attn_with_kvcache as Prism drives it
// (engine/executor.py:119-120, :260-261; block-table format engine/kv_cache.py:123-153):
//   slot = cache_seqlens[b] + j;  page = block_table[b, slot / P];  row = slot % P.
#include "pkv_common.h"

namespace pkv {

struct AppendParams {
  const uint16_t* k_new;
  const uint16_t* v_new;
  int64_t kn_sb, kn_ss, kn_sh, vn_sb, vn_ss, vn_sh;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t page_stride;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* seqlens;
  int32_t* status;
  int64_t total_chunks;  // batch * s_new * n_kv * (head_dim / 8)
  int s_new, n_kv, head_dim, chunks_per_head, log2_page, num_pages, max_blocks;
};

__global__ __launch_bounds__(256) void append_kernel(const AppendParams p) {
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < p.total_chunks; i += stride) {
    const int c8 = int(i % p.chunks_per_head);
    int64_t r = i / p.chunks_per_head;
    const int hh = int(r % p.n_kv);
    r /= p.n_kv;
    const int j = int(r % p.s_new);
    const int b = int(r / p.s_new);

    const int slot = p.seqlens[b] + j;
    const int col = slot >> p.log2_page;
    if (slot < 0 || col >= p.max_blocks) {
      flag_status(p.status, PKV_STATUS_BAD_PAGE);
      continue;
    }
    const int pid = p.block_table[int64_t(b) * p.bt_stride + col];
    if (pid < 0 || pid >= p.num_pages) {
      flag_status(p.status, PKV_STATUS_BAD_PAGE);
      continue;
    }
    const int row = slot & ((1 << p.log2_page) - 1);
    const int64_t dst = int64_t(pid) * p.page_stride + (int64_t(row) * p.n_kv + hh) * p.head_dim + c8 * 8;
    const u32x4 kv = ld16(p.k_new + b * p.kn_sb + j * p.kn_ss + hh * p.kn_sh + c8 * 8);
    const u32x4 vv = ld16(p.v_new + b * p.vn_sb + j * p.vn_ss + hh * p.vn_sh + c8 * 8);
    st16(p.k_cache + dst, kv);
    st16(p.v_cache + dst, vv);
  }
}

// Host-side validation shared with the attention launchers.
int validate_paged(const char* fn, const void* k_cache, const void* v_cache, int64_t page_stride,
                   const int32_t* block_table, int64_t bt_stride, const int32_t* seqlens, int batch,
                   int n_kv, int head_dim, int page_size, int num_pages, int max_blocks) {
  if (!k_cache || !v_cache || !block_table || !seqlens)
    return fail(PKV_EINVAL, "%s: null cache, block_table or cache_seqlens pointer", fn);
  if (batch < 0 || n_kv <= 0 || num_pages <= 0 || max_blocks <= 0)
    return fail(PKV_EINVAL, "%s: bad sizes batch=%d n_kv=%d num_pages=%d max_blocks=%d", fn, batch,
                n_kv, num_pages, max_blocks);
  if (head_dim != 64 && head_dim != 128)
    return fail(PKV_EINVAL, "%s: head_dim %d unsupported (64 or 128)", fn, head_dim);
  if (!is_pow2(page_size) || page_size < 16)
    return fail(PKV_EINVAL, "%s: page_size %d must be a power of two >= 16", fn, page_size);
  // every kernel indexes a sequence's keys in 32 bits, and the balanced decode split counts tiles
  // with single-precision arithmetic: at most 2^27 keys per sequence
  if (int64_t(max_blocks) * page_size > (int64_t(1) << 27))
    return fail(PKV_EINVAL, "%s: max_blocks %d x page_size %d > 2^27 keys per sequence", fn, max_blocks, page_size);
  if (bt_stride < max_blocks)
    return fail(PKV_EINVAL, "%s: bt_stride %lld < max_blocks %d", fn, (long long)bt_stride, max_blocks);
  if (page_stride < int64_t(page_size) * n_kv * head_dim || (page_stride % 8) != 0)
    return fail(PKV_EINVAL, "%s: page stride %lld too small or not 16-byte aligned", fn,
                (long long)page_stride);
  if (!aligned16(k_cache) || !aligned16(v_cache))
    return fail(PKV_EINVAL, "%s: k_cache/v_cache not 16-byte aligned", fn);
  return PKV_OK;
}

int validate_rows(const char* fn, const char* name, const void* ptr, int64_t sb, int64_t ss, int64_t sh) {
  if (!aligned16(ptr)) return fail(PKV_EINVAL, "%s: %s not 16-byte aligned", fn, name);
  if ((sb % 8) || (ss % 8) || (sh % 8))
    return fail(PKV_EINVAL, "%s: %s strides (%lld,%lld,%lld) must be multiples of 8 elements", fn, name,
                (long long)sb, (long long)ss, (long long)sh);
  return PKV_OK;
}

int launch_append(const char* fn, const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                  const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh, void* k_cache,
                  void* v_cache, int64_t page_stride, const int32_t* block_table, int64_t bt_stride,
                  const int32_t* seqlens, int batch, int s_new, int n_kv, int head_dim, int page_size,
                  int num_pages, int max_blocks, int32_t* status, hipStream_t stream) {
  AppendParams p;
  p.k_new = static_cast<const uint16_t*>(k_new);
  p.v_new = static_cast<const uint16_t*>(v_new);
  p.kn_sb = kn_sb; p.kn_ss = kn_ss; p.kn_sh = kn_sh;
  p.vn_sb = vn_sb; p.vn_ss = vn_ss; p.vn_sh = vn_sh;
  p.k_cache = static_cast<uint16_t*>(k_cache);
  p.v_cache = static_cast<uint16_t*>(v_cache);
  p.page_stride = page_stride;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.seqlens = seqlens;
  p.status = status;
  p.s_new = s_new;
  p.n_kv = n_kv;
  p.head_dim = head_dim;
  p.chunks_per_head = head_dim / 8;
  p.log2_page = ilog2(page_size);
  p.num_pages = num_pages;
  p.max_blocks = max_blocks;
  p.total_chunks = int64_t(batch) * s_new * n_kv * p.chunks_per_head;
  if (p.total_chunks == 0) return PKV_OK;
  const int64_t want = (p.total_chunks + 255) / 256;
  const int blocks = int(want < 8192 ? want : 8192);
  append_kernel<<<blocks, 256, 0, stream>>>(p);
  return check_launch(fn);
}

}  // namespace pkv

extern "C" int pkv_append(const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                          const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh, void* k_cache,
                          void* v_cache, int64_t cache_page_stride, const int32_t* block_table,
                          int64_t bt_stride, const int32_t* cache_seqlens, int32_t batch, int32_t s_new,
                          int32_t n_kv, int32_t head_dim, int32_t page_size, int32_t num_pages,
                          int32_t max_blocks, int32_t* status, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_append";
  int rc = validate_paged(fn, k_cache, v_cache, cache_page_stride, block_table, bt_stride, cache_seqlens,
                          batch, n_kv, head_dim, page_size, num_pages, max_blocks);
  if (rc) return rc;
  if (s_new < 0) return fail(PKV_EINVAL, "%s: s_new %d < 0", fn, s_new);
  if (!k_new || !v_new) return fail(PKV_EINVAL, "%s: null k_new/v_new", fn);
  if ((rc = validate_rows(fn, "k_new", k_new, kn_sb, kn_ss, kn_sh))) return rc;
  if ((rc = validate_rows(fn, "v_new", v_new, vn_sb, vn_ss, vn_sh))) return rc;
  return launch_append(fn, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache, v_cache,
                       cache_page_stride, block_table, bt_stride, cache_seqlens, batch, s_new, n_kv,
                       head_dim, page_size, num_pages, max_blocks, status,
                       static_cast<hipStream_t>(stream));
}
