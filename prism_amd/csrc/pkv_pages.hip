// Batched page copy / gather for the paged KV pool: copy-on-write of shared pages, sequence
// transfer and live-page compaction into a fresh pool, all in one launch.
//
// Generalises FlashAttnKVCache.transfer_sequence (engine/kv_cache.py:174-209), which issues
// 2 * num_layers * num_pages separate copy_() calls of one page each.  Here one workgroup moves
// one (tensor, page pair): a contiguous byte range of fill_slots * slot_bytes, 16 bytes per lane
// per step, sixteen steps in flight per lane.
#include "pkv_common.h"

namespace pkv {

struct PageCopyParams {
  const uint64_t* src_bases;  // device [n_tensors]
  const uint64_t* dst_bases;  // device [n_tensors]
  const int32_t* src_ids;     // device [n_pages]
  const int32_t* dst_ids;     // device [n_pages] or nullptr (then dst = dst_first + p)
  const int32_t* fill_slots;  // device [n_pages] or nullptr (whole pages)
  int32_t* status;
  int64_t src_page_stride, dst_page_stride, slot_bytes;
  int n_pages, page_slots, src_num_pages, dst_num_pages, dst_first;
};

__global__ __launch_bounds__(256) void copy_pages_kernel(const PageCopyParams p) {
  // blockIdx.x = pair index, blockIdx.y = tensor index
  const int pr = blockIdx.x;
  const int ti = blockIdx.y;
  const int sid = p.src_ids[pr];
  const int did = p.dst_ids ? p.dst_ids[pr] : p.dst_first + pr;
  int fill = p.fill_slots ? p.fill_slots[pr] : p.page_slots;
  if (sid < 0 || sid >= p.src_num_pages || did < 0 || did >= p.dst_num_pages || fill < 0 ||
      fill > p.page_slots) {
    if (threadIdx.x == 0) flag_status(p.status, PKV_STATUS_BAD_PAGE);
    return;
  }
  const char* src = reinterpret_cast<const char*>(p.src_bases[ti]) + int64_t(sid) * p.src_page_stride;
  char* dst = reinterpret_cast<char*>(p.dst_bases[ti]) + int64_t(did) * p.dst_page_stride;
  const int64_t n16 = int64_t(fill) * p.slot_bytes / 16;
  // 16 x 16 bytes per lane in flight (64 KiB per workgroup), destination rows written
  // non-temporally: the copy is read by nobody in this launch, and streaming it past the caches
  // keeps the source rows there, which matters when one page is copied into many (copy-on-write
  // of a shared boundary page into 63 children: 144 against 224 us with 4 in flight and ordinary
  // stores; compaction of 246 whole pages x 56 tensors 1.33 against 1.39 ms).  Non-temporal
  // loads would evict that shared source (332 us).
  constexpr int U = 16;
  int64_t i = threadIdx.x;
  for (; i + int64_t(U - 1) * 256 < n16; i += U * 256) {
    u32x4 v[U];
#pragma unroll
    for (int u = 0; u < U; ++u) v[u] = ld16(src + (i + u * 256) * 16);
#pragma unroll
    for (int u = 0; u < U; ++u) __builtin_nontemporal_store(v[u], reinterpret_cast<u32x4*>(dst + (i + u * 256) * 16));
  }
  for (; i < n16; i += 256) st16(dst + i * 16, ld16(src + i * 16));
}

static int launch_copy(const char* fn, const PageCopyParams& p, int n_tensors, hipStream_t stream) {
  if (p.n_pages == 0 || n_tensors == 0) return PKV_OK;
  dim3 grid(p.n_pages, n_tensors);
  copy_pages_kernel<<<grid, 256, 0, stream>>>(p);
  return check_launch(fn);
}

static int validate_copy(const char* fn, const uint64_t* src_bases, const uint64_t* dst_bases, int n_tensors,
                         const int32_t* src_ids, int n_pages, int64_t src_stride, int64_t dst_stride, int64_t slot_bytes,
                         int page_slots, int src_num_pages, int dst_num_pages) {
  if (n_tensors < 0 || n_pages < 0) return fail(PKV_EINVAL, "%s: negative n_tensors/n_pages", fn);
  if (n_tensors == 0 || n_pages == 0) return PKV_OK;
  if (!src_bases || !dst_bases || !src_ids) return fail(PKV_EINVAL, "%s: null base or id array", fn);
  if (n_tensors > 65535) return fail(PKV_EINVAL, "%s: n_tensors %d exceeds the grid limit", fn, n_tensors);
  if (slot_bytes <= 0 || slot_bytes % 16 || src_stride % 16 || dst_stride % 16)
    return fail(PKV_EINVAL, "%s: slot_bytes / page strides must be positive multiples of 16", fn);
  if (page_slots <= 0 || int64_t(page_slots) * slot_bytes > src_stride || int64_t(page_slots) * slot_bytes > dst_stride)
    return fail(PKV_EINVAL, "%s: page of %d slots x %lld bytes exceeds a page stride", fn, page_slots,
                (long long)slot_bytes);
  if (src_num_pages <= 0 || dst_num_pages <= 0) return fail(PKV_EINVAL, "%s: empty pool", fn);
  return PKV_OK;
}

}  // namespace pkv

extern "C" int pkv_copy_pages(const uint64_t* src_bases, const uint64_t* dst_bases, int32_t n_tensors,
                              const int32_t* src_ids, const int32_t* dst_ids, const int32_t* fill_slots,
                              int32_t n_pages, int64_t src_page_stride_bytes, int64_t dst_page_stride_bytes,
                              int64_t slot_bytes, int32_t page_slots, int32_t src_num_pages, int32_t dst_num_pages,
                              int32_t* status, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_copy_pages";
  int rc = validate_copy(fn, src_bases, dst_bases, n_tensors, src_ids, n_pages, src_page_stride_bytes,
                         dst_page_stride_bytes, slot_bytes, page_slots, src_num_pages, dst_num_pages);
  if (rc) return rc;
  if (n_pages > 0 && n_tensors > 0 && !dst_ids) return fail(PKV_EINVAL, "%s: null dst_ids", fn);
  PageCopyParams p;
  p.src_bases = src_bases;
  p.dst_bases = dst_bases;
  p.src_ids = src_ids;
  p.dst_ids = dst_ids;
  p.fill_slots = fill_slots;
  p.status = status;
  p.src_page_stride = src_page_stride_bytes;
  p.dst_page_stride = dst_page_stride_bytes;
  p.slot_bytes = slot_bytes;
  p.n_pages = n_pages;
  p.page_slots = page_slots;
  p.src_num_pages = src_num_pages;
  p.dst_num_pages = dst_num_pages;
  p.dst_first = 0;
  return launch_copy(fn, p, n_tensors, static_cast<hipStream_t>(stream));
}

extern "C" int pkv_gather_pages(const uint64_t* src_bases, const uint64_t* dst_bases, int32_t n_tensors,
                                const int32_t* src_ids, int32_t n_pages, int32_t dst_first,
                                int64_t src_page_stride_bytes, int64_t dst_page_stride_bytes, int64_t page_bytes,
                                int32_t src_num_pages, int32_t dst_num_pages, int32_t* status, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_gather_pages";
  int rc = validate_copy(fn, src_bases, dst_bases, n_tensors, src_ids, n_pages, src_page_stride_bytes,
                         dst_page_stride_bytes, page_bytes, 1, src_num_pages, dst_num_pages);
  if (rc) return rc;
  if (dst_first < 0) return fail(PKV_EINVAL, "%s: dst_first %d < 0", fn, dst_first);
  PageCopyParams p;
  p.src_bases = src_bases;
  p.dst_bases = dst_bases;
  p.src_ids = src_ids;
  p.dst_ids = nullptr;
  p.fill_slots = nullptr;
  p.status = status;
  p.src_page_stride = src_page_stride_bytes;
  p.dst_page_stride = dst_page_stride_bytes;
  p.slot_bytes = page_bytes;
  p.n_pages = n_pages;
  p.page_slots = 1;
  p.src_num_pages = src_num_pages;
  p.dst_num_pages = dst_num_pages;
  p.dst_first = dst_first;
  return launch_copy(fn, p, n_tensors, static_cast<hipStream_t>(stream));
}
