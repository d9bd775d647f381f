// Device-resident block tables for a graph-captured decode batch.  One launch applies a step's
// update packet: the new length of every row whose length changed, then the (row, column, page)
// entries that differ from what the device table already holds (pages appended at a page
// boundary, pages replaced by copy-on-write, rows handed to another sequence or to padding).
//
// Replaces the reference's per-step refill of its static graph buffers, which rewrites the whole
// table element by element from the host (engine/kv_cache.py:147-151 build_block_table, then
// engine/executor.py:345-353 g["bt"][:] = 0; g["bt"][:B, :nb] = bt; g["sl"][:] = 0; ...).
#include "pkv_common.h"

namespace pkv {

struct TableUpdateParams {
  const int32_t* packet;  // [n_len][2] (row, length), then [n_ent][3] (row, column, page)
  int32_t* block_table;
  int64_t bt_stride;
  int32_t* seqlens;
  int32_t* status;
  int n_len, n_ent, rows, cols, num_pages;
};

__global__ __launch_bounds__(256) void table_update_kernel(const TableUpdateParams p) {
  const int i = int(blockIdx.x) * 256 + int(threadIdx.x);
  if (i < p.n_len) {
    const int row = p.packet[2 * i];
    const int len = p.packet[2 * i + 1];
    if (unsigned(row) < unsigned(p.rows) && len >= 0)
      p.seqlens[row] = len;
    else
      flag_status(p.status, PKV_STATUS_BAD_PAGE);
    return;
  }
  const int k = i - p.n_len;
  if (k >= p.n_ent) return;
  const int32_t* e = p.packet + 2 * int64_t(p.n_len) + 3 * int64_t(k);
  const int row = e[0], col = e[1], page = e[2];
  if (unsigned(row) < unsigned(p.rows) && unsigned(col) < unsigned(p.cols) && unsigned(page) < unsigned(p.num_pages))
    p.block_table[int64_t(row) * p.bt_stride + col] = page;
  else
    flag_status(p.status, PKV_STATUS_BAD_PAGE);
}

}  // namespace pkv

extern "C" int pkv_table_update(const int32_t* packet, int32_t n_len, int32_t n_ent, int32_t* block_table,
                                int64_t bt_stride, int32_t* seqlens, int32_t rows, int32_t cols, int32_t num_pages,
                                int32_t* status, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_table_update";
  if (n_len < 0 || n_ent < 0) return fail(PKV_EINVAL, "%s: negative entry counts", fn);
  if (int64_t(n_len) + n_ent > 0x7fffff00LL) return fail(PKV_EINVAL, "%s: too many entries", fn);
  if (n_len + n_ent == 0) return PKV_OK;
  if (!packet || !block_table || !seqlens) return fail(PKV_EINVAL, "%s: null argument", fn);
  if (rows <= 0 || cols <= 0 || bt_stride < cols) return fail(PKV_EINVAL, "%s: bad table shape", fn);
  if (num_pages <= 0) return fail(PKV_EINVAL, "%s: empty pool", fn);
  TableUpdateParams p;
  p.packet = packet;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.seqlens = seqlens;
  p.status = status;
  p.n_len = n_len;
  p.n_ent = n_ent;
  p.rows = rows;
  p.cols = cols;
  p.num_pages = num_pages;
  const int total = n_len + n_ent;
  table_update_kernel<<<(total + 255) / 256, 256, 0, static_cast<hipStream_t>(stream)>>>(p);
  return check_launch(fn);
}

namespace pkv {

// The status word's bits so far, moved to *dst and cleared in one atomic exchange, so a kernel on
// another stream that flags a bit meanwhile is never lost between a read and a clear.
__global__ void status_take_kernel(int32_t* status, int32_t* dst) { *dst = atomicExch(status, 0); }

}  // namespace pkv

extern "C" int pkv_status_take(int32_t* status, int32_t* dst, void* stream) {
  using namespace pkv;
  clear_error();
  if (!status || !dst) return fail(PKV_EINVAL, "pkv_status_take: null argument");
  status_take_kernel<<<1, 1, 0, static_cast<hipStream_t>(stream)>>>(status, dst);
  return check_launch("pkv_status_take");
}
