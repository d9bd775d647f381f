// Paged attention for gfx950 (MI355X): decode / speculative verify (split-K over the KV range)
// and varlen chunked prefill (query rows spread over waves), both over Prism's paged cache.
//
// Replaces flash_attn_with_kvcache as Prism calls it (engine/executor.py:119-120, :151-153,
// :260-261, :385-386; engine/speculative_executor.py:150-153): new K/V rows are appended at
// cache_seqlens[b], and query j of sequence b (L_b keys after the append) attends to keys
// t <= L_b - s_q + j (causal, bottom-right aligned) through the block table; query head hq
// reads KV head hq / g with g = n_heads / n_kv.
//
// Orientation.  All query rows that read one KV head (row = j * g + head-in-group) are the N
// side of v_mfma_f32_16x16x32_bf16, 16 rows per N tile; 32-token KV tiles are the M side:
//
//   S^T[tok, row] = K[tok, :] . Q[row, :]          A = K rows straight from memory (16 B/lane),
//                                                  B = Q^T held in registers for the whole call
//   O^T[d, row]  += V^T[d, tok] . P^T[tok, row]     A = V^T repacked in registers,
//                                                  B = P^T = the S^T accumulator, in place
//
// The S^T accumulator a lane holds (4 tokens x 1 row per MFMA) is exactly the P^T operand the
// PV MFMA wants, and all softmax statistics of a lane's row live in that lane, so the
// online-softmax rescale of O needs no cross-lane traffic; only the tile max is reduced across
// the four 16-lane groups.  V rows arrive head_dim-contiguous: each lane loads 8 tokens x
// head_dim/16 elements and transposes them with byte permutes into the token-major V^T operand,
// except where a kernel stages V tiles in LDS at head_dim 128: there LDS transpose reads
// (ds_read_b64_tr_b16) deliver the operand directly.
// Every K/V byte of a (sequence, KV head) is fetched once per query-row tile.
#include <math.h>

#include <mutex>
#include <type_traits>

#include "pkv_common.h"

namespace pkv {

struct AttnParams {
  const uint16_t* q;
  int64_t q_sb, q_ss, q_sh;
  const uint16_t* k_new;
  int64_t kn_sb, kn_ss, kn_sh;
  const uint16_t* v_new;
  int64_t vn_sb, vn_ss, vn_sh;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t page_stride;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* seqlens;
  uint16_t* out;
  int64_t o_sb, o_ss, o_sh;
  float* ws_o;   // [batch, n_kv, max_splits, R, head_dim] unnormalised split partials
  float* ws_ml;  // [batch, n_kv, max_splits, R, 2] (row max in log2 units, row sum of exp2)
  int32_t* ws_cnt;  // [batch, n_kv] split arrival counters, zero between calls
  int32_t* status;
  int batch, s_q, g, R, n_kv, log2_page, num_pages, max_blocks, split_tokens, max_splits;
  int causal, has_new, two_pass;
  int lean_grid;  // workgroups of a decode_lean_kernel launch (its combine needs the same split)
  // Cascade (shared-prefix) attention: the first k0 keys of every sequence are the same pages
  // (k0 a multiple of the page size).  cascade_splits > 0 turns it on: the prefix pass writes
  // cascade_splits partials per sequence (slots 2 G + b S + s), decode_lean_kernel covers keys
  // [k0, L) and writes every segment as a partial (whole sequences to slot 2 G + B S + b), and
  // the combine merges them all.  k0 = 0 and cascade_splits = 0 otherwise.
  int k0, cascade_splits;
  // balanced decode kernel: the KV heads go in n_groups head groups, the tiles of group g after
  // those of group g - 1; tok_elems = n_kv * head_dim, the elements of a token row; cnt_stride:
  // int32 words between the in-launch merge's arrival counters
  int n_groups, tok_elems, cnt_stride;
  // pkv_decode_attn_rope: q and k_new arrive unrotated; the balanced kernel applies the
  // reference's rotary embedding (rows positions[b] + j of rot_cos / rot_sin, [n_pos, head_dim])
  // to both.  Null otherwise.
  const uint16_t* rot_cos;
  const uint16_t* rot_sin;
  int n_pos;
  float scale_log2;  // softmax_scale * log2(e)
};

// Maxima of attention scores without IEEE-mode canonicalisation.  fmaxf on an MFMA result makes
// the compiler quieten each operand first (v_max_f32 x, x, x); scores here are finite or -inf,
// never NaN, so the raw v_max3_f32 / v_max_f32 give the same value in a third of the
// instructions.
__device__ __forceinline__ float max3_raw(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}
__device__ __forceinline__ float max_raw(float a, float b) {
  float r;
  asm("v_max_f32 %0, %1, %2" : "=v"(r) : "v"(a), "v"(b));
  return r;
}

// Reductions over the four lanes {l, l^16, l^32, l^48} that hold the same query row, with the
// gfx950 row-swap permutes: permlane16_swap(x, x) hands lane l the pair {x[l], x[l^16]} and
// permlane32_swap(x, x) the pair {x[l], x[l^32]} (no LDS round trip, unlike ds_bpermute).
__device__ __forceinline__ float max_over_quads(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = max_raw(__uint_as_float(a[0]), __uint_as_float(a[1]));
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return max_raw(__uint_as_float(b[0]), __uint_as_float(b[1]));
}

__device__ __forceinline__ float sum_over_quads(float v) {
  const auto a = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  v = __uint_as_float(a[0]) + __uint_as_float(a[1]);
  const auto b = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(b[0]) + __uint_as_float(b[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

// One lane's slice of a V row: head_dim/16 bf16 values as 32-bit words.
template <int HD>
struct VRow {
  uint32_t w[HD / 32];
};

template <int HD>
__device__ __forceinline__ void load_vrow(VRow<HD>& r, const uint16_t* ptr) {
  if constexpr (HD == 128) {
    const u32x4 v = ld16(ptr);
    r.w[0] = v[0]; r.w[1] = v[1]; r.w[2] = v[2]; r.w[3] = v[3];
  } else {
    const u32x2 v = ld8(ptr);
    r.w[0] = v[0]; r.w[1] = v[1];
  }
}

// Keys of sequence b: (cache length c, total L).  A length outside what the block table can
// address is flagged and clamped, so work and workspace indices stay bounded.
__device__ __forceinline__ void seq_lengths(const AttnParams& p, int b, int& c, int& L) {
  const int cap = p.max_blocks << p.log2_page;
  c = p.seqlens[b];
  L = c + (p.has_new ? p.s_q : 0);
  if (c < 0 || L > cap) {
    if (threadIdx.x == 0) flag_status(p.status, PKV_STATUS_BAD_PAGE);
    c = min(max(c, 0), cap);
    L = min(c + (p.has_new ? p.s_q : 0), cap);
  }
}

// Work item of a prefill workgroup, heaviest first.  Workgroups start in launch order, a few
// hundred at a time, and a (sequence, KV head, row block) item costs about as many KV tiles as
// its rows can see: more for a longer sequence and, causally, for a later row block.  The grid
// (row blocks, KV heads, sequences) is therefore walked sequence by sequence in descending cache
// length (ties by index), row blocks in descending order, KV heads innermost: longest-first list
// scheduling, which shortens the launch's tail when prefixes differ (14B chunks onto prefixes
// U{0..4096}: 242 -> 211 tile-times in a 512-slot model).  Batches above 64 keep launch order.
__device__ __forceinline__ void prefill_item(const AttnParams& p, int& b, int& h, int& xblk) {
  const int nx = int(gridDim.x), nkv = int(gridDim.y);
  const int i = int(blockIdx.x) + nx * (int(blockIdx.y) + nkv * int(blockIdx.z));
  const int per_seq = nx * nkv;
  const int rank = i / per_seq;
  const int r = i - rank * per_seq;
  xblk = nx - 1 - r / nkv;
  h = r - (r / nkv) * nkv;
  const int nb = int(gridDim.z);
  if (nb > 64) {
    b = rank;
    return;
  }
  const int lane = threadIdx.x & 63;
  const int cl = lane < nb ? p.seqlens[lane] : 0;
  int mine = 0;  // lane's place in descending length order
  for (int k = 0; k < nb; ++k) {
    const int ck = __shfl(cl, k, 64);
    mine += (ck > cl || (ck == cl && k < lane)) ? 1 : 0;
  }
  const uint64_t hit = __ballot(lane < nb && mine == rank);
  b = int(__builtin_ctzll(hit));
}

__device__ __forceinline__ int num_splits(const AttnParams& p, int L) {
  const int n = L > 0 ? (L + p.split_tokens - 1) / p.split_tokens : 1;
  return min(n, p.max_splits);
}

// Split count of a sequence from its raw cache length (same clamping as seq_lengths).
__device__ __forceinline__ int splits_of(const AttnParams& p, int c_raw) {
  const int cap = p.max_blocks << p.log2_page;
  const int c = min(max(c_raw, 0), cap);
  const int L = min(c + (p.has_new ? p.s_q : 0), cap);
  return num_splits(p, L);
}

// Map dense slot j (0-based over every (sequence, split) pair, sequence-major) to (b, split) with
// a 64-lane prefix scan over the sequences' split counts; false when j is past the last pair.
// Every lane of the wave gets the same answer.
__device__ __forceinline__ bool locate_item(const AttnParams& p, int batch, int j, int& b, int& split) {
  const int lane = threadIdx.x & 63;
  int base = 0;
  for (int b0 = 0; b0 < batch; b0 += 64) {
    const int bb = b0 + lane;
    const int nb = bb < batch ? splits_of(p, p.seqlens[bb]) : 0;
    int incl = nb;
#pragma unroll
    for (int off = 1; off < 64; off <<= 1) {
      const int t = __shfl_up(incl, off, 64);
      if (lane >= off) incl += t;
    }
    const int total = __shfl(incl, 63, 64);
    if (j < base + total) {
      const unsigned long long hit = __ballot(base + incl > j);
      const int first = __ffsll(static_cast<long long>(hit)) - 1;
      b = b0 + first;
      split = j - base - __shfl(incl - nb, first, 64);
      return true;
    }
    base += total;
  }
  return false;
}

// Per-(sequence, KV head) view used by the wave routine.
struct SeqView {
  int b, h, c, t_end;
  const int32_t* bt;
};

// Block-table window of one wave: lane l holds block_table[b, col0 + l] (or -1 past max_blocks),
// so the page of a tile is one v_readlane away instead of a memory round trip per tile.
struct BtWindow {
  int col0;
  int ids;
};

__device__ __forceinline__ void bt_window_load(const AttnParams& p, const SeqView& sv, int col0, BtWindow& w) {
  const int lane = threadIdx.x & 63;
  const int col = col0 + lane;
  w.col0 = col0;
  w.ids = col < p.max_blocks ? sv.bt[col] : -1;
}

// Page id of block-table column `col` (uniform); refills the window when col leaves it.
__device__ __forceinline__ int bt_page(const AttnParams& p, const SeqView& sv, int col, BtWindow& w) {
  if (col - w.col0 >= 64 || col < w.col0) bt_window_load(p, sv, col, w);
  return __builtin_amdgcn_readlane(w.ids, col - w.col0);
}

// The last visible key of a padding row (a row past the real query rows, computed and never
// stored).  Real rows keep their own limit, negative when they see no key (causal rows of a call
// whose keys are fewer than its queries), and only padding rows are left out of the wave's
// minimum limit, which decides whether a tile needs the mask at all.
constexpr int kNoQueryRow = INT_MIN;

__device__ __forceinline__ int min_real_limit(int acc, int lim) { return min(acc, lim == kNoQueryRow ? INT_MAX : lim); }

// Load the Q^T operand for the 16*NT rows starting at row0 and the last key each row may see.
template <int HD, int NT>
__device__ __forceinline__ void load_q(const AttnParams& p, const SeqView& sv, int L, int row0,
                                       bf16x8 (&qf)[NT][HD / 32], int (&lim)[NT]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rr = row0 + li + 16 * nt;
    if (rr < p.R) {
      const int j = rr / p.g;
      const int hq = rr - j * p.g;
      const uint16_t* base = p.q + sv.b * p.q_sb + j * p.q_ss + (sv.h * p.g + hq) * p.q_sh + 8 * lq;
#pragma unroll
      for (int kk = 0; kk < HD / 32; ++kk) qf[nt][kk] = __builtin_bit_cast(bf16x8, ld16(base + 32 * kk));
      const int last = p.causal ? (L - p.s_q + j) : (L - 1);
      lim[nt] = min(last, sv.t_end - 1);
    } else {
#pragma unroll
      for (int kk = 0; kk < HD / 32; ++kk) qf[nt][kk] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
      lim[nt] = kNoQueryRow;
    }
  }
}

// load_q for the cascade prefix pass: rows r < batch * R of the whole batch (sequence r / R,
// row r % R of it), every one seeing keys [0, last_key].
template <int HD, int NT>
__device__ __forceinline__ void load_q_batch_rows(const AttnParams& p, int h, int row0, int last_key,
                                                  bf16x8 (&qf)[NT][HD / 32], int (&lim)[NT]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int ra = row0 + li + 16 * nt;
    if (ra < p.batch * p.R) {
      const int b = ra / p.R;
      const int rr = ra - b * p.R;
      const int j = rr / p.g;
      const int hq = rr - j * p.g;
      const uint16_t* base = p.q + b * p.q_sb + j * p.q_ss + (h * p.g + hq) * p.q_sh + 8 * lq;
#pragma unroll
      for (int kk = 0; kk < HD / 32; ++kk) qf[nt][kk] = __builtin_bit_cast(bf16x8, ld16(base + 32 * kk));
      lim[nt] = last_key;
    } else {
#pragma unroll
      for (int kk = 0; kk < HD / 32; ++kk) qf[nt][kk] = __builtin_bit_cast(bf16x8, u32x4{0u, 0u, 0u, 0u});
      lim[nt] = kNoQueryRow;
    }
  }
}

// A pointer the whole wave agrees on, pinned to scalar registers.
template <typename T>
__device__ __forceinline__ T* uniform_ptr(T* ptr) {
  const uint64_t a = reinterpret_cast<uint64_t>(ptr);
  const uint32_t lo = __builtin_amdgcn_readfirstlane(uint32_t(a));
  const uint32_t hi = __builtin_amdgcn_readfirstlane(uint32_t(a >> 32));
  return reinterpret_cast<T*>((uint64_t(hi) << 32) | lo);
}

// Registers of one 32-token tile: the K rows of both QK MFMA groups and the V slices.
template <int HD>
struct KVTile {
  u32x4 kr[2][HD / 32];
  VRow<HD> vr[8];
};

// Per-lane constant byte offsets of the K and V slices a lane loads, relative to the tile's
// first row (token T0) of head h in its page: valid for every tile that lies in one page.
struct LaneOffsets {
  uint32_t k[2];  // K row of QK group a, + 64 * kk bytes per 32-element chunk
  uint32_t v;     // V row of token 8lq (token 8lq + e is e * row_bytes further)
};

template <int HD>
__device__ __forceinline__ LaneOffsets lane_offsets(const AttnParams& p) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
  const uint32_t row_elems = uint32_t(p.n_kv * HD);
  LaneOffsets o;
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const uint32_t tt = 8 * (li >> 2) + 4 * a + (li & 3);
    o.k[a] = (tt * row_elems + 8 * lq) * 2u;
  }
  o.v = ((8 * lq) * row_elems + (HD / 16) * li) * 2u;
  return o;
}

// Issue every load of the tile at token T0 (uniform) into tl.  Every row is read from the cache
// (rows appended by this call were written before the tile loop).  Addressing is a per-tile base
// plus constant per-lane offsets; rows of the half after token T0 + 16 use a second base, which
// differs from the first only for 16-row pages.  V rows past t_end (only in the last tile) are
// zeroed, since P = 0 times a stale NaN would still poison the PV product; K rows past t_end need
// nothing, their scores are masked.  A page id outside the pool is flagged and read as page 0.
template <int HD>
__device__ __forceinline__ void load_tile(const AttnParams& p, const SeqView& sv, int T0, BtWindow& btw,
                                          const LaneOffsets& lo, KVTile<HD>& tl) {
  constexpr int KK = HD / 32;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
  const int row_elems = p.n_kv * HD;
  const int pmask = (1 << p.log2_page) - 1;
  const int pidA = bt_page(p, sv, T0 >> p.log2_page, btw);
  const bool okA = unsigned(pidA) < unsigned(p.num_pages);
  if (!okA && T0 < sv.t_end) flag_status(p.status, PKV_STATUS_BAD_PAGE);
  const int64_t offA = int64_t(okA ? pidA : 0) * p.page_stride + int64_t(T0 & pmask) * row_elems + sv.h * HD;
  if (p.log2_page >= 5) {
    // scalar bases + 32-bit per-lane offsets: global_load ... voffset, saddr
    const char* kb = uniform_ptr(reinterpret_cast<const char*>(p.k_cache + offA));
    const char* vb = uniform_ptr(reinterpret_cast<const char*>(p.v_cache + offA));
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) tl.kr[a][kk] = ld16(kb + (lo.k[a] + 64 * kk));
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const char* vbe = uniform_ptr(vb + int64_t(e) * row_elems * 2);
      load_vrow<HD>(tl.vr[e], reinterpret_cast<const uint16_t*>(vbe + lo.v));
    }
  } else {
    // 16-row pages: the tile's second half lives on the next page
    const int pidB = bt_page(p, sv, (T0 + 16) >> p.log2_page, btw);
    const bool okB = unsigned(pidB) < unsigned(p.num_pages);
    if (!okB && T0 + 16 < sv.t_end) flag_status(p.status, PKV_STATUS_BAD_PAGE);
    const int64_t offB = int64_t(okB ? pidB : 0) * p.page_stride - 16 * int64_t(row_elems) + sv.h * HD;
    const char* kb = reinterpret_cast<const char*>(p.k_cache + (li >= 8 ? offB : offA));
    const char* vb = reinterpret_cast<const char*>(p.v_cache + (lq >= 2 ? offB : offA));
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int kk = 0; kk < KK; ++kk) tl.kr[a][kk] = ld16(kb + lo.k[a] + 64 * kk);
#pragma unroll
    for (int e = 0; e < 8; ++e)
      load_vrow<HD>(tl.vr[e], reinterpret_cast<const uint16_t*>(vb + uint32_t(e * row_elems * 2) + lo.v));
  }
  if (T0 + 32 > sv.t_end) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool keep = T0 + 8 * lq + e < sv.t_end;
#pragma unroll
      for (int w = 0; w < HD / 32; ++w) tl.vr[e].w[w] = keep ? tl.vr[e].w[w] : 0u;
    }
  }
}

// Rows rescale their output only when their running max grows by more than this (log2 units),
// so exp2 arguments stay <= kRescaleSlack and P <= 2^kRescaleSlack: the rescale of the MFMA
// accumulators becomes a rare, wave-uniform branch instead of work on every tile.
constexpr float kRescaleSlack = 8.0f;
#ifndef PKV_DECODE_DEPTH
#define PKV_DECODE_DEPTH 2
#endif
#ifndef PKV_PREFILL_DEPTH
#define PKV_PREFILL_DEPTH 1
#endif
// prefill's software pipeline, and the vector instructions between its interleaved MFMAs
#ifndef PKV_PREFILL_PIPE
#define PKV_PREFILL_PIPE 1
#endif
#ifndef PKV_PREFILL_PIPE_VALU
#define PKV_PREFILL_PIPE_VALU 2
#endif
constexpr int kDecodeDepth = PKV_DECODE_DEPTH;
constexpr int kPrefillDepth = PKV_PREFILL_DEPTH;

// Online-softmax update of one wave's 16*NT query rows with the tile at token T0.
// SPLIT_P feeds P to the PV MFMA as a bf16 hi + lo pair (two MFMAs) instead of one bf16
// rounding: decode has an order of magnitude of MFMA headroom, and short contexts then keep the
// output error down to the output's own bf16 rounding.
template <int HD, int NT, bool SPLIT_P, bool VT = false>
__device__ __forceinline__ void compute_tile(const AttnParams& p, const KVTile<HD>& tl, int T0,
                                             const bf16x8 (&qf)[NT][HD / 32], const int (&lim)[NT], int lim_min,
                                             float (&m_run)[NT], float (&l_run)[NT], f32x4 (&acc)[NT][HD / 16]) {
  constexpr int KK = HD / 32;
  constexpr int DPL = HD / 16;
  const int lane = threadIdx.x & 63;
  const int lq = lane >> 4;

  // V^T operands: PV MFMA n covers head-dim elements d = DPL*i + n (i = M row = lane li), or
  // with VT the operands rows_read_tile_vt read; element e of the operand is token T0 + 8lq + e.
  bf16x8 vt[DPL];
#pragma unroll
  for (int n = 0; n < DPL; ++n) {
    if constexpr (VT) {
      vt[n] = __builtin_bit_cast(bf16x8, u32x4{tl.vr[n].w[0], tl.vr[n].w[1], tl.vr[n].w[2], tl.vr[n].w[3]});
      continue;
    }
    const int w = n >> 1;
    const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
    u32x4 pk;
#pragma unroll
    for (int pp = 0; pp < 4; ++pp) pk[pp] = __builtin_amdgcn_perm(tl.vr[2 * pp + 1].w[w], tl.vr[2 * pp].w[w], sel);
    vt[n] = __builtin_bit_cast(bf16x8, pk);
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    f32x4 s[2];
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      s[a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < KK; ++kk)
        s[a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, tl.kr[a][kk]), qf[nt][kk], s[a],
                                                      0, 0, 0);
    }
    // s[a][r]: score of token T0 + 8lq + 4a + r against query row li + 16nt.  Only tiles that
    // reach past some real row's last visible key pay for the mask (a wave-uniform test).
    float x[8];
    if (T0 + 31 > lim_min) {
#pragma unroll
      for (int a = 0; a < 2; ++a) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int t = T0 + 8 * lq + 4 * a + r;
          x[4 * a + r] = (t <= lim[nt]) ? s[a][r] * p.scale_log2 : -INFINITY;
        }
      }
    } else {
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r) x[4 * a + r] = s[a][r] * p.scale_log2;
    }
    float mx = max3_raw(max3_raw(x[0], x[1], x[2]), max3_raw(x[3], x[4], x[5]), max_raw(x[6], x[7]));
    mx = max_over_quads(mx);
    const bool grow = mx > m_run[nt] + kRescaleSlack;
    if (__any(grow)) {
      const float m_new = grow ? mx : m_run[nt];
      // 0 on a row's first visible tile, 1 if unchanged; a row that has seen no key yet keeps
      // -inf while other rows grow (split-K parts of speculative verify that start past its last
      // visible key), and -inf - -inf would make its state NaN
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run[nt] - m_new);
      l_run[nt] *= alpha;
#pragma unroll
      for (int n = 0; n < DPL; ++n) acc[nt][n] *= alpha;
      m_run[nt] = m_new;
    }
    const float m_use = (m_run[nt] == -INFINITY) ? 0.f : m_run[nt];
    float psum = 0.f;
    u32x4 pk, pk_lo;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float p0 = fast_exp2(x[e] - m_use);
      const float p1 = fast_exp2(x[e + 1] - m_use);
      psum += p0 + p1;
      pk[e >> 1] = pack_bf16x2(p0, p1);
      if constexpr (SPLIT_P) {
        const float h0 = bf16_bits_to_f32(pk[e >> 1] & 0xffffu);
        const float h1 = bf16_bits_to_f32(pk[e >> 1] >> 16);
        pk_lo[e >> 1] = pack_bf16x2(p0 - h0, p1 - h1);
      }
    }
    l_run[nt] += psum;
    const bf16x8 pb = __builtin_bit_cast(bf16x8, pk);
#pragma unroll
    for (int n = 0; n < DPL; ++n) {
      acc[nt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[n], pb, acc[nt][n], 0, 0, 0);
      if constexpr (SPLIT_P)
        acc[nt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[n], __builtin_bit_cast(bf16x8, pk_lo), acc[nt][n],
                                                            0, 0, 0);
    }
  }
}

// Online-softmax attention of one wave's 16*NT query rows over the 32-token tiles starting at
// token T_first (uniform), T_step apart, below T_stop.  With DEPTH = 2, two register tiles
// alternate so the loads of tile i+1 are in flight while tile i is computed.  m_run is the
// row's softmax reference (within kRescaleSlack of its running max); l_run is a per-lane partial
// (sum over the lane's own tokens) to be reduced with sum_over_quads.
template <int HD, int NT, bool SPLIT_P, int DEPTH>
__device__ __forceinline__ void wave_attend(const AttnParams& p, const SeqView& sv, const bf16x8 (&qf)[NT][HD / 32],
                                            const int (&lim)[NT], int T_first, int T_stop, int T_step,
                                            float (&m_run)[NT], float (&l_run)[NT], f32x4 (&acc)[NT][HD / 16]) {
  int T0 = __builtin_amdgcn_readfirstlane(T_first);
  T_stop = __builtin_amdgcn_readfirstlane(T_stop);
  T_step = __builtin_amdgcn_readfirstlane(T_step);
  if (T0 >= T_stop) return;
  const LaneOffsets lo = lane_offsets<HD>(p);
  // smallest last-visible key over the wave's real rows (padding rows have lim = -1 and never
  // reach the output, so they are left out)
  int lim_min = 0x7fffffff;
  const int lane = threadIdx.x & 63;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) lim_min = min_real_limit(lim_min, lim[nt]);
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, off, 64));
  lim_min = __builtin_amdgcn_readfirstlane(lim_min);
  (void)lane;
  BtWindow btw;
  bt_window_load(p, sv, T0 >> p.log2_page, btw);
  if constexpr (DEPTH == 1) {
    for (; T0 < T_stop; T0 += T_step) {
      KVTile<HD> t0;
      load_tile<HD>(p, sv, T0, btw, lo, t0);
      compute_tile<HD, NT, SPLIT_P>(p, t0, T0, qf, lim, lim_min, m_run, l_run, acc);
    }
  } else {
    KVTile<HD> t0, t1;
    load_tile<HD>(p, sv, T0, btw, lo, t0);
    for (;;) {
      int T1 = T0 + T_step;
      if (T1 < T_stop) load_tile<HD>(p, sv, T1, btw, lo, t1);
      compute_tile<HD, NT, SPLIT_P>(p, t0, T0, qf, lim, lim_min, m_run, l_run, acc);
      if (T1 >= T_stop) break;
      T0 = T1 + T_step;
      if (T0 < T_stop) load_tile<HD>(p, sv, T0, btw, lo, t0);
      compute_tile<HD, NT, SPLIT_P>(p, t1, T1, qf, lim, lim_min, m_run, l_run, acc);
      if (T0 >= T_stop) break;
    }
  }
}

// Copy the rows of this call that land in tokens [a0, a1) of (b, h) into the cache.
template <int HD>
__device__ __forceinline__ void append_rows(const AttnParams& p, const SeqView& sv, int a0, int a1, int tid,
                                            int nthreads) {
  constexpr int CPR = HD / 8;
  const int n_items = (a1 - a0) * 2 * CPR;
  for (int idx = tid; idx < n_items; idx += nthreads) {
    const int row = idx / (2 * CPR);
    const int rem = idx - row * (2 * CPR);
    const bool is_v = rem >= CPR;
    const int c8 = is_v ? rem - CPR : rem;
    const int t = a0 + row;
    const int j = t - sv.c;
    const int col = t >> p.log2_page;
    const int pid = col < p.max_blocks ? sv.bt[col] : -1;
    if (pid < 0 || pid >= p.num_pages) {
      flag_status(p.status, PKV_STATUS_BAD_PAGE);
      continue;
    }
    const int64_t dst =
        int64_t(pid) * p.page_stride + int64_t(t & ((1 << p.log2_page) - 1)) * (p.n_kv * HD) + sv.h * HD + c8 * 8;
    const uint16_t* src = is_v ? p.v_new + sv.b * p.vn_sb + j * p.vn_ss + sv.h * p.vn_sh
                               : p.k_new + sv.b * p.kn_sb + j * p.kn_ss + sv.h * p.kn_sh;
    st16((is_v ? p.v_cache : p.k_cache) + dst, ld16(src + c8 * 8));
  }
}

__device__ __forceinline__ void store_out_row8(const AttnParams& p, int b, int h, int row, int d0, const float (&o)[8],
                                               float lsum) {
  const int j = row / p.g;
  const int hq = row - j * p.g;
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  u32x4 ov;
#pragma unroll
  for (int k = 0; k < 4; ++k) ov[k] = pack_bf16x2(o[2 * k] * inv, o[2 * k + 1] * inv);
  st16(p.out + b * p.o_sb + j * p.o_ss + (h * p.g + hq) * p.o_sh + d0, ov);
}

// Split partials cross workgroups that may run on different XCDs, whose L2s are not coherent
// with each other.  They are written and read with agent-scope relaxed atomics, which gfx950
// issues as plain global_store / global_load with the sc1 bit (coherent at device scope), so no
// L2-wide writeback or invalidate is needed anywhere in the protocol.
__device__ __forceinline__ void st_coherent(float* ptr, float v) {
  __hip_atomic_store(ptr, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float ld_coherent(const float* ptr) {
  return __hip_atomic_load(ptr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Log-sum-exp merge of the n_split partials of (b, h) into the bf16 output, by `nthreads` threads.
// Splits are merged kMergeChunk at a time with every load of a chunk issued before any is used,
// so the merge costs one memory round trip per chunk rather than one per split.
constexpr int kMergeChunk = 8;

template <int HD>
__device__ __forceinline__ void combine_splits(const AttnParams& p, int b, int h, int n_split, int tid, int nthreads) {
  constexpr int CPR = HD / 8;
  for (int idx = tid; idx < p.R * CPR; idx += nthreads) {
    const int row = idx / CPR;
    const int d0 = (idx - row * CPR) * 8;
    const int64_t base = int64_t(b * p.n_kv + h) * p.max_splits * p.R + row;
    float M = -INFINITY;
    float lsum = 0.f;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    for (int s0 = 0; s0 < n_split; s0 += kMergeChunk) {
      float m[kMergeChunk], l[kMergeChunk], x[kMergeChunk][8];
#pragma unroll
      for (int u = 0; u < kMergeChunk; ++u) {
        const int64_t slot = base + int64_t(min(s0 + u, n_split - 1)) * p.R;
        m[u] = ld_coherent(p.ws_ml + slot * 2);
        l[u] = ld_coherent(p.ws_ml + slot * 2 + 1);
#pragma unroll
        for (int k = 0; k < 8; ++k) x[u][k] = ld_coherent(p.ws_o + slot * HD + d0 + k);
      }
      float Mc = M;
#pragma unroll
      for (int u = 0; u < kMergeChunk; ++u)
        if (s0 + u < n_split) Mc = fmaxf(Mc, m[u]);
      const float M_use = (Mc == -INFINITY) ? 0.f : Mc;
      const float f_old = fast_exp2(M - M_use);
      lsum *= f_old;
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] *= f_old;
#pragma unroll
      for (int u = 0; u < kMergeChunk; ++u) {
        const float f = (s0 + u < n_split) ? fast_exp2(m[u] - M_use) : 0.f;
        lsum += f * l[u];
#pragma unroll
        for (int k = 0; k < 8; ++k) o[k] += f * x[u][k];
      }
      M = Mc;
    }
    store_out_row8(p, b, h, row, d0, o, lsum);
  }
}

// ---------------------------------------------------------------------------------------------
// Decode / verify: grid (split, KV head, sequence).  The W waves take interleaved 32-token tiles
// of the split and merge (m, l, O) through LDS.  A sequence whose keys fit one split writes the
// bf16 output directly.  Otherwise each split writes its partial to the workspace and bumps the
// (b, h) arrival counter; the last split to arrive merges all partials and writes the output, and
// resets the counter to zero for the next call.  One launch per call, no separate combine pass.
// ---------------------------------------------------------------------------------------------
#ifndef PKV_DECODE_W
#define PKV_DECODE_W 4
#endif
#ifndef PKV_DECODE_MIN_BLOCKS
#define PKV_DECODE_MIN_BLOCKS 1
#endif

template <int HD, int NT, int W>
__global__ __launch_bounds__(64 * W, PKV_DECODE_MIN_BLOCKS) void decode_kernel(const AttnParams p) {
  constexpr int DPL = HD / 16;
  constexpr int ROWS = 16 * NT;
  constexpr int CPR = HD / 8;

  __shared__ float sm_o[W][ROWS][HD + 4];
  __shared__ float sm_m[W][ROWS];
  __shared__ float sm_l[W][ROWS];
  __shared__ int sm_last;

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int lq = lane >> 4;
  // Dense work numbering: item = ((sequence, split) slot) * n_kv + head, so the real work fills
  // the front of the 1-D grid and consecutive items land on different XCDs.
  const int h = blockIdx.x % p.n_kv;
  int b, split;
  if (!locate_item(p, p.batch, blockIdx.x / p.n_kv, b, split)) return;

  int c, L;
  seq_lengths(p, b, c, L);
  const int t_begin = split * p.split_tokens;
  const int n_split_b = num_splits(p, L);
  SeqView sv;
  sv.b = b;
  sv.h = h;
  sv.c = c;
  sv.t_end = min(t_begin + p.split_tokens, L);
  sv.bt = p.block_table + int64_t(b) * p.bt_stride;

  // Append the new rows that fall in this split.  Only this workgroup reads them, after the
  // barrier: its waves share one CU and its L1, so the stores are visible to their loads.
  if (p.has_new) {
    append_rows<HD>(p, sv, max(max(c, t_begin), 0), sv.t_end, threadIdx.x, 64 * W);
    __syncthreads();
  }

  bf16x8 qf[NT][HD / 32];
  int lim[NT];
  load_q<HD, NT>(p, sv, L, 0, qf, lim);

  float m_run[NT], l_run[NT];
  f32x4 acc[NT][DPL];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.f;
#pragma unroll
    for (int n = 0; n < DPL; ++n) acc[nt][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // The last query row (j = s_q - 1) sees every key of the split, so the whole split is walked.
  wave_attend<HD, NT, true, kDecodeDepth>(p, sv, qf, lim, t_begin + 32 * wave, sv.t_end, 32 * W, m_run, l_run,
                                         acc);

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = li + 16 * nt;
    const float l_tot = sum_over_quads(l_run[nt]);
    if (lq == 0) {
      sm_m[wave][row] = m_run[nt];
      sm_l[wave][row] = l_tot;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int n = 0; n < DPL; ++n) sm_o[wave][row][DPL * (4 * lq + r) + n] = acc[nt][n][r];
  }
  __syncthreads();

  const int n_items = p.R * CPR;
  for (int idx = threadIdx.x; idx < n_items; idx += 64 * W) {
    const int row = idx / CPR;
    const int d0 = (idx - row * CPR) * 8;
    float M = -INFINITY;
#pragma unroll
    for (int w = 0; w < W; ++w) M = fmaxf(M, sm_m[w][row]);
    const float M_use = (M == -INFINITY) ? 0.f : M;
    float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
    float lsum = 0.f;
#pragma unroll
    for (int w = 0; w < W; ++w) {
      const float f = fast_exp2(sm_m[w][row] - M_use);
      lsum += f * sm_l[w][row];
#pragma unroll
      for (int k = 0; k < 8; ++k) o[k] += f * sm_o[w][row][d0 + k];
    }
    if (n_split_b == 1) {
      store_out_row8(p, b, h, row, d0, o, lsum);
    } else {
      const int64_t slot = (int64_t(b * p.n_kv + h) * p.max_splits + split) * p.R + row;
      float* dst = p.ws_o + slot * HD + d0;
#pragma unroll
      for (int k = 0; k < 8; ++k) st_coherent(dst + k, o[k]);
      if (d0 == 0) {
        st_coherent(p.ws_ml + slot * 2, M);
        st_coherent(p.ws_ml + slot * 2 + 1, lsum);
      }
    }
  }
  if (n_split_b == 1 || p.two_pass) return;

  // Count this split's arrival once all of its partial stores have completed; the last split
  // of (b, h) to arrive merges every partial and re-arms the counter for the next call.
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (threadIdx.x == 0) {
    const int prev = atomicAdd(p.ws_cnt + (b * p.n_kv + h), 1);
    sm_last = (prev == n_split_b - 1);
  }
  __syncthreads();
  if (!sm_last) return;
  combine_splits<HD>(p, b, h, n_split_b, threadIdx.x, 64 * W);
  if (threadIdx.x == 0) __hip_atomic_store(p.ws_cnt + (b * p.n_kv + h), 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Two-pass mode: the split-K merge as its own launch.  The kernel boundary orders the partial
// stores before these loads, so plain vector loads serve, and every split's loads of a thread are
// issued before any is used: one memory round trip per kMergeBatch splits.  Grid (n_kv, batch,
// groups of 16 query rows); thread t of the workgroup owns (row, 4 head-dim elements) =
// (16 blockIdx.z + t / (HD/4), t % (HD/4)).
constexpr int kMergeBatch = 32;

template <int HD>
__global__ __launch_bounds__(512) void combine_kernel(const AttnParams p) {
  constexpr int Q4 = HD / 4;
  __shared__ float sm_m_in[kMergeBatch][16], sm_l_in[kMergeBatch][16];
  __shared__ float sm_m[16], sm_l[16], sm_rescale[16];
  const int h = blockIdx.x;
  const int b = blockIdx.y;
  int c, L;
  seq_lengths(p, b, c, L);
  const int n_split = num_splits(p, L);
  if (n_split <= 1) return;
  const int rg = int(blockIdx.z) * 16;  // this workgroup's 16 query rows: rg .. rg + 15
  const int lr = threadIdx.x / Q4;
  const int row = rg + lr;
  const int d0 = (threadIdx.x - lr * Q4) * 4;
  // 512 threads cover 512 / Q4 rows: 16 at head_dim 128, 32 at head_dim 64, where the upper half
  // (rows of the next workgroup) only helps stage the (m, l) pairs
  const bool active = lr < 16 && row < p.R;
  const int64_t base = int64_t(b * p.n_kv + h) * p.max_splits * p.R;
  if (threadIdx.x < 16) {
    sm_m[threadIdx.x] = -INFINITY;
    sm_l[threadIdx.x] = 0.f;
  }
  f32x4 o = {0.f, 0.f, 0.f, 0.f};
  for (int s0 = 0; s0 < n_split; s0 += kMergeBatch) {
    const int ns = min(kMergeBatch, n_split - s0);
    f32x4 x[kMergeBatch];
#pragma unroll
    for (int u = 0; u < kMergeBatch; ++u)
      x[u] = (active && u < ns) ? *reinterpret_cast<const f32x4*>(p.ws_o + (base + int64_t(s0 + u) * p.R + row) * HD + d0)
                                : f32x4{0.f, 0.f, 0.f, 0.f};
    // (m, l) of every (split, row) of the batch into LDS, one pair per thread
    {
      const int u = threadIdx.x / 16, r = threadIdx.x % 16;
      const bool ok = u < ns && rg + r < p.R;
      const f32x2 ml = ok ? *reinterpret_cast<const f32x2*>(p.ws_ml + (base + int64_t(s0 + u) * p.R + rg + r) * 2)
                          : f32x2{-INFINITY, 0.f};
      sm_m_in[u][r] = ml[0];
      sm_l_in[u][r] = ml[1];
    }
    __syncthreads();
    if (threadIdx.x < 16) {
      const int r = threadIdx.x;
      float M = sm_m[r];
      for (int u = 0; u < ns; ++u) M = fmaxf(M, sm_m_in[u][r]);
      const float M_use = (M == -INFINITY) ? 0.f : M;
      const float rescale = fast_exp2(sm_m[r] - M_use);
      float lsum = sm_l[r] * rescale;
      for (int u = 0; u < ns; ++u) {
        const float w = fast_exp2(sm_m_in[u][r] - M_use);
        lsum += w * sm_l_in[u][r];
        sm_m_in[u][r] = w;  // now the batch weight
      }
      sm_m[r] = M;
      sm_l[r] = lsum;
      sm_rescale[r] = rescale;
    }
    __syncthreads();
    if (active) {
      o *= sm_rescale[lr];
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u)
        if (u < ns) o += sm_m_in[u][lr] * x[u];
    }
    __syncthreads();  // the batch's weights are consumed before the next batch overwrites them
  }
  if (active) {
    const float inv = sm_l[lr] > 0.f ? 1.f / sm_l[lr] : 0.f;
    const int j = row / p.g;
    const int hq = row - j * p.g;
    const u32x2 ov = {pack_bf16x2(o[0] * inv, o[1] * inv), pack_bf16x2(o[2] * inv, o[3] * inv)};
    *reinterpret_cast<u32x2*>(p.out + b * p.o_sb + j * p.o_ss + (h * p.g + hq) * p.o_sh + d0) = ov;
  }
}

// ---------------------------------------------------------------------------------------------
// Balanced row-streaming decode for the shape the 7B decode step runs at (head_dim 128, 4 KV
// heads, pages of >= 32 rows, <= 16 query rows per KV head, <= 256 sequences).
//
// Reading one KV head's 256-byte slice out of every 1 KiB token row (decode_kernel, one
// workgroup per head) opens each DRAM row four times, at different moments, from four
// workgroups; whole rows stream ~30% faster.  Here one workgroup handles all four heads of the
// tokens it owns (wave h = KV head h).
//
// Work split.  Every sequence is cut into 32-token tiles (a sequence without keys still counts
// one tile, which yields its zero output); the tiles of all sequences, in sequence order, form
// one list of T tiles, and persistent workgroup w of G owns the contiguous range
// [w * per, (w + 1) * per), per = ceil(T / G).  Every workgroup streams the same bytes to within
// one tile, whatever the context lengths.  (For decode rows of a few sequences, and wherever a
// head's keys are split over phase waves, the host picks a variant that cuts each sequence into
// ceil(t_b / per) ranges of its own when those fit the grid: aligned_range.)  The sequences a
// range touches are its segments; a
// segment holding a whole sequence writes the bf16 output directly, the others (at most the
// first and the last segment of a range) write an fp32 partial (m, l, O) to workspace slot
// 2w (first segment of the range) or 2w + 1 (last), merged by combine_lean_kernel.
//
// Streaming.  A 32-token tile of K and of V is one contiguous 32 KiB run of its page, copied
// into LDS with global_load_lds_dwordx4 (no VGPR staging, tracked by vmcnt) and double-buffered
// so tile j+1 streams in while tile j is consumed; wave h then reads head h's MFMA operands from
// LDS.  The 16-byte chunks of row r are XOR-swizzled by g(r) = (r & 3) | ((r >> 3) & 3) << 2, so
// every group of 8 or 16 consecutive lanes hits distinct bank groups both for the K-operand
// reads (16 rows, one chunk) and the V-operand reads (one row, 16 chunks).  A segment's Q
// operand and a tile's new rows are loaded along with the tile copies, two tiles ahead.
//
// Append.  The tile holding a sequence's new rows is copied from the cache like any other (its
// new rows are stale there); each wave then overwrites its head's slice of those rows in LDS
// from registers and stores the same bytes to the cache.  Only this workgroup touches those
// rows during the launch, so nothing orders the append before the attention reads.
// ---------------------------------------------------------------------------------------------
namespace rows {
// chunk swizzle of row r (bits 0-3 of the 16-byte chunk index; stays inside a wave's 256 B slice)
__device__ __forceinline__ int swz(int r) { return (r & 3) | (((r >> 3) & 3) << 2); }
// The 4 KV heads x head_dim 128 geometry: the cascade path's, and the per-slot bound of the
// split-K workspace (no geometry holds more than 4 x 128 elements per partial row block).
constexpr int HD = 128;
constexpr int NKV = 4;
constexpr int ROW_BYTES = 1024;           // one LDS row: four 256-byte wave slices
constexpr int TILE = 32;                  // LDS rows per tile = keys per MFMA subtile
constexpr int TILE_BYTES = TILE * ROW_BYTES;
constexpr int kMaxBatch = 256;            // sequences the in-register scan covers
constexpr int kChunks = kMaxBatch / 64;
// Cache policy of the K/V tile copies: non-temporal (the nt bit).  Every cache byte is read once
// per call, and streaming it past the caches' normal allocation measured ~12% faster for the
// 7B decode step's 115 MB (18.7 vs 21.1 us per launch for the bare copy loop).
constexpr int kStreamPolicy = 2;
// Verify (several query rows per head) reads its tiles with the default policy instead: the
// sequences of a verify batch usually share a cached prefix, whose pages then stay in the caches
// for the next sequence (config-5 verify: 78.3 vs 82.0 us per call).  The suffix pass of a cascade
// launch reads private pages only, and streams them non-temporally (config 5: 69.9 -> 65.5 us per
// cascade call).
constexpr int kVerifyPolicy = 0;
typedef __attribute__((address_space(3))) void lds_void;
}  // namespace rows

// Geometry of a balanced launch: HG KV heads of head_dim HD form a head group, whose slice of a
// token row (HG * HD * 2 bytes: 1 KiB, 512 B or 256 B) the four waves share.  Wave w takes the
// 256-byte slice w of every 1 KiB LDS row: head hg = w % HG of the group, phase ph = w / HG.  With
// P = 4 / HG phases the LDS row packs P token rows: a tile holds TOK = 32 P S tokens and wave
// (hg, ph) owns the consecutive keys [32 S ph, 32 S (ph + 1)) of it for head hg, as S 32-key MFMA
// subtiles (S = 2 at head_dim 64, whose head slice is 128 B).  The P phases of a head keep
// separate softmax states, merged through LDS when a segment ends.  Geom<128, 4> is the 7B shape
// (one token row of four heads per LDS row, no phases).
template <int HD_, int HG_>
struct Geom {
  static_assert(HD_ == 64 || HD_ == 128, "head_dim 64 or 128");
  static_assert(HG_ == 1 || HG_ == 2 || HG_ == 4, "1, 2 or 4 KV heads per group");
  static constexpr int HD = HD_;
  static constexpr int HG = HG_;
  static constexpr int S = 128 / HD;                 // 32-key subtiles per wave and tile
  static constexpr int P = 4 / HG;                   // phases (waves per head)
  static constexpr int TOK = rows::TILE * P * S;     // tokens per tile
  static constexpr int SCH = 16 / S;                 // 16-byte chunks of one head row (HD / 8)
  static constexpr int QROW = HD * 2;                // bytes of one Q row
  static constexpr int QCH = QROW / 16;
  static constexpr int Q_BYTES = 16 * HG * QROW;     // Q area: 16 rows per head of the group
  static constexpr int Q_COPIES = Q_BYTES / 4096;    // 1 KiB copies per wave that fill it
  static_assert(Q_COPIES >= 1, "the Q area must give every wave a copy");
};
using Geom7B = Geom<128, 4>;

// Workgroup barrier that only orders memory operations for the compiler: the hardware waits for
// nothing beyond the explicit s_waitcnt the caller issued (a __syncthreads fence would also
// drain the next tile's in-flight LDS copies, serialising the double buffer).
__device__ __forceinline__ void raw_barrier() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

__device__ __forceinline__ void rows_wait_vm(bool keep_one_tile) {
  // vmcnt <= 16 (the next tile's copies may stay in flight) or vmcnt == 0
  if (keep_one_tile)
    __builtin_amdgcn_s_waitcnt(0x4F70);  // vmcnt(16): [3:0] = 0, [15:14] = 1; expcnt/lgkmcnt: no wait
  else
    __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
}

// Inclusive prefix sum over the 64 lanes: shifts inside each 16-lane row, then the GFX9 row
// broadcasts carry the row totals on (lane 15 into row 1 and lane 47 into row 3, then lane 31
// into rows 2 and 3).  A lane whose source falls outside its row adds 0.
__device__ __forceinline__ int wave_incl_scan(int v) {
  v += __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false);  // row_shr:1
  v += __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false);  // row_shr:2
  v += __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false);  // row_shr:4
  v += __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false);  // row_shr:8
  v += __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false);  // row_bcast:15
  v += __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false);  // row_bcast:31
  return v;
}

template <int TOK>
__device__ __forceinline__ int tiles_of(int L) { return L > 0 ? (L + TOK - 1) / TOK : 1; }

// Tiles of TOK tokens of a sequence of L keys in a balanced launch: keys [k0, L) (k0
// tile-aligned), at least one (a sequence without keys there still yields its zero output or
// empty partial).
template <int TOK>
__device__ __forceinline__ int seq_tiles(const AttnParams& p, int L) {
  const int t = tiles_of<TOK>(L) - p.k0 / TOK;
  return t > 0 ? t : 1;
}

// Every sequence's clamped lengths and first tile, 64 sequences per register (lane l of register
// q holds sequence 64q + l), from one read of cache_seqlens per wave.  The clamp is seq_lengths'.
template <int NCH>
struct SeqTable {
  int c[NCH], L[NCH], first[NCH];
  int end[NCH];  // uniform: one past the last tile of chunk q
  int total;               // T, tiles over all sequences
};

template <int NCH, int TOK>
__device__ __forceinline__ void seq_table(const AttnParams& p, SeqTable<NCH>& st) {
  const int lane = threadIdx.x & 63;
  const int cap = p.max_blocks << p.log2_page;
  const int s_new = p.has_new ? p.s_q : 0;
  int raw[NCH];
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int b = 64 * q + lane;
    raw[q] = 0;
    if (64 * q < p.batch && b < p.batch) raw[q] = p.seqlens[b];
  }
  int base = 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int b = 64 * q + lane;
    int c = raw[q];
    int L = c + s_new;
    if (b < p.batch && (c < 0 || L > cap)) {
      if (threadIdx.x < 64) flag_status(p.status, PKV_STATUS_BAD_PAGE);
      c = min(max(c, 0), cap);
      L = min(c + s_new, cap);
    }
    const int n = b < p.batch ? seq_tiles<TOK>(p, L) : 0;
    const int incl = base + wave_incl_scan(n);
    st.c[q] = c;
    st.L[q] = L;
    st.first[q] = incl - n;
    base = __builtin_amdgcn_readlane(incl, 63);
    st.end[q] = base;
  }
  st.total = base;
}

// Sequence of tile x (per lane, x < total): its index, first tile and lengths.  A binary search
// over the chunk's first tiles (non-decreasing across lanes) with lane permutes.
template <int NCH>
__device__ __forceinline__ void locate_tile(const AttnParams& p, const SeqTable<NCH>& st, int x, int& b, int& first,
                                            int& c, int& L) {
  b = 0;
  first = 0;
  c = 0;
  L = 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    if (64 * q >= p.batch) break;
    int pos = 0;
#pragma unroll
    for (int step = 32; step >= 1; step >>= 1) {
      const int f = __shfl(st.first[q], min(pos + step, 63), 64);
      if (pos + step <= 63 && f <= x) pos += step;
    }
    const int fq = __shfl(st.first[q], pos, 64);
    const int cq = __shfl(st.c[q], pos, 64);
    const int Lq = __shfl(st.L[q], pos, 64);
    const int lo = q == 0 ? 0 : st.end[q - 1];
    if (x >= lo && x < st.end[q]) {
      b = 64 * q + pos;
      first = fq;
      c = cq;
      L = Lq;
    }
  }
}

// Descriptors of tiles x0 + lane (< e) of a workgroup's range: head group, sequence, first token,
// lengths and page.  Tile x of the launch is tile x - g T1 of head group g = x / T1 (T1 tiles per
// group).  A page id outside the pool is flagged (when the tile has keys) and kept as -1.
struct TileWin {
  int x0;
  int g, b, T0, c, L, pid;
};

struct TileDesc {
  int g, b, T0, c, L, pid;
};

template <int NCH, int TOK>
__device__ __forceinline__ void tile_window(const AttnParams& p, const SeqTable<NCH>& st, int x0, int e, int T1,
                                            TileWin& w) {
  const int lane = threadIdx.x & 63;
  const int xg = min(x0 + lane, e - 1);
  const int g = xg / T1;
  const int x = xg - g * T1;
  int b, first, c, L;
  locate_tile(p, st, x, b, first, c, L);
  b = min(b, p.batch - 1);
  const int T0 = (x - first) * TOK + p.k0;
  const int col = T0 >> p.log2_page;
  const int pid = unsigned(col) < unsigned(p.max_blocks) ? p.block_table[int64_t(b) * p.bt_stride + col] : -1;
  const bool ok = unsigned(pid) < unsigned(p.num_pages);
  if (!ok && T0 < L && x0 + lane < e && threadIdx.x < 64) flag_status(p.status, PKV_STATUS_BAD_PAGE);
  w.x0 = x0;
  w.g = g;
  w.b = b;
  w.T0 = T0;
  w.c = c;
  w.L = L;
  w.pid = ok ? pid : -1;
}

__device__ __forceinline__ TileDesc tile_desc(const TileWin& w, int x) {
  const int i = x - w.x0;
  TileDesc d;
  d.g = __builtin_amdgcn_readlane(w.g, i);
  d.b = __builtin_amdgcn_readlane(w.b, i);
  d.T0 = __builtin_amdgcn_readlane(w.T0, i);
  d.c = __builtin_amdgcn_readlane(w.c, i);
  d.L = __builtin_amdgcn_readlane(w.L, i);
  d.pid = __builtin_amdgcn_readlane(w.pid, i);
  return d;
}

template <int TOK>
__device__ __forceinline__ bool tile_has_new(const AttnParams& p, const TileDesc& d) {
  return p.has_new && d.T0 + TOK > d.c && d.T0 < d.L;
}

// Rotary position of a token, clamped into the table (outside it: flagged, PKV_STATUS_BAD_POSITION).
__device__ __forceinline__ int rope_position(const AttnParams& p, int pos) {
  if (pos < 0 || pos >= p.n_pos) {
    if ((threadIdx.x & 63) == 0) flag_status(p.status, PKV_STATUS_BAD_POSITION);
    pos = min(max(pos, 0), p.n_pos - 1);
  }
  return pos;
}

__device__ __forceinline__ float bf16r(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }
__device__ __forceinline__ void unpack_bf16x8(const u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = bf16_bits_to_f32(v[k] & 0xffffu);
    f[2 * k + 1] = bf16_bits_to_f32(v[k] >> 16);
  }
}
// The reference's rotary step on one 8-element chunk pair, x1 = elements d .. d+7 (first half of
// the head) and x2 = d + hd/2 .. (its rotate_half partner): out = x * cos + rotate_half(x) * sin
// with rotate_half(x) = (-x2, x1), every torch bf16 op rounded (engine/executor.py:149-150):
// o1 = bf16(bf16(x1 c1) + bf16(-x2 s1)), o2 = bf16(bf16(x2 c2) + bf16(x1 s2)).
__device__ __forceinline__ void rope_pair(u32x4& a, u32x4& b, const u32x4 c1v, const u32x4 s1v, const u32x4 c2v,
                                          const u32x4 s2v) {
  float x1[8], x2[8], c1[8], s1[8], c2[8], s2[8];
  unpack_bf16x8(a, x1);
  unpack_bf16x8(b, x2);
  unpack_bf16x8(c1v, c1);
  unpack_bf16x8(s1v, s1);
  unpack_bf16x8(c2v, c2);
  unpack_bf16x8(s2v, s2);
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    a[k] = pack_bf16x2(bf16r(bf16r(x1[2 * k] * c1[2 * k]) + bf16r(-x2[2 * k] * s1[2 * k])),
                       bf16r(bf16r(x1[2 * k + 1] * c1[2 * k + 1]) + bf16r(-x2[2 * k + 1] * s1[2 * k + 1])));
    b[k] = pack_bf16x2(bf16r(bf16r(x2[2 * k] * c2[2 * k]) + bf16r(x1[2 * k] * s2[2 * k])),
                       bf16r(bf16r(x2[2 * k + 1] * c2[2 * k + 1]) + bf16r(x1[2 * k + 1] * s2[2 * k + 1])));
  }
}
// rope_pair on one word (two elements) of x1 and of its partner x2.
__device__ __forceinline__ void rope_word(uint32_t& a, uint32_t& b, uint32_t c1, uint32_t s1, uint32_t c2,
                                          uint32_t s2) {
  u32x4 va = {a, 0u, 0u, 0u}, vb = {b, 0u, 0u, 0u};
  rope_pair(va, vb, u32x4{c1, 0u, 0u, 0u}, u32x4{s1, 0u, 0u, 0u}, u32x4{c2, 0u, 0u, 0u}, u32x4{s2, 0u, 0u, 0u});
  a = va[0];
  b = vb[0];
}

// Where lane l's 16 bytes of LDS row r of a tile come from: LDS chunk l holds chunk
// v = (l & 15) ^ swz(r) of wave slice w = l / 16 (head hg = w % HG, phase ph = w / HG): chunk
// v % SCH of head hg's row of token 32 (S ph + v / SCH) + r of the tile.
template <typename G>
struct LaneSrc {
  int tt;  // token within the tile
  int hg;  // head within the group
  int cc;  // 16-byte chunk within the head row
};

template <typename G>
__device__ __forceinline__ LaneSrc<G> lane_src(int r, int lane) {
  const int w = lane >> 4;
  const int v = (lane & 15) ^ rows::swz(r);
  LaneSrc<G> ls;
  ls.hg = w % G::HG;
  ls.tt = rows::TILE * ((w / G::HG) * G::S + v / G::SCH) + r;
  ls.cc = v % G::SCH;
  return ls;
}

// Per-lane byte offsets of a wave's row copies inside a tile's K (or V) run: copy i of wave w
// fills LDS row r = 4 i + w (lane_src gives the token, head and chunk; tok_elems * 2 bytes per
// token).  The same for every tile, so they are computed once per launch.
struct RowOffsets {
  uint32_t v[rows::TILE / 4];
};

template <typename G>
__device__ __forceinline__ RowOffsets row_offsets(const AttnParams& p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  RowOffsets ro;
#pragma unroll
  for (int i = 0; i < rows::TILE / 4; ++i) {
    const LaneSrc<G> ls = lane_src<G>(i * 4 + wave, lane);
    ro.v[i] = uint32_t(ls.tt * p.tok_elems * 2 + ls.hg * G::HD * 2 + ls.cc * 16);
  }
  return ro;
}

// The rotary kernel's offsets: row_offsets' plus, per Q copy i, the element offset inside q of
// the lane's chunk less the sequence and head-group terms (the query row and head a lane copies
// are the same for every segment start of the launch).  Precomputed so the rotary instantiation
// (more registers live than the plain one) does not redo the divisions by g at every segment.
struct RowOffsetsQ : RowOffsets {
  int64_t q[4];
};

template <typename G>
__device__ __forceinline__ RowOffsetsQ row_offsets_q(const AttnParams& p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  RowOffsetsQ ro;
  static_cast<RowOffsets&>(ro) = row_offsets<G>(p);
  static_assert(G::Q_COPIES <= 4, "Q copies per wave");
#pragma unroll
  for (int i = 0; i < G::Q_COPIES; ++i) {
    const int qi = wave * G::Q_COPIES + i;
    const int ar = qi * (1024 / G::QROW) + lane / G::QCH;
    const int hq_g = ar / 16;
    const int row = ar % 16;
    const int rr = min(row, p.R - 1);
    const int jq = rr / p.g;
    const int hq = rr - jq * p.g;
    const int gq = (lane % G::QCH) ^ (row % G::QCH);
    ro.q[i] = jq * p.q_ss + int64_t(hq_g * p.g + hq) * p.q_sh + gq * 8;
  }
  return ro;
}

// Copies of tile d into LDS buffer `buf`, 16 per wave: K then V rows, wave w filling LDS rows
// w, w + 4, ..., lane l writing LDS chunk l of a row (row_offsets' mapping).  A tile without new
// rows is two buffers (its K and its V run, TOK token rows each, base and range in scalar
// registers) read at the precomputed lane offsets: one M0 write and one buffer load per copy.
// In a tile holding one of this call's new tokens (t >= c), that token's chunks are sourced from
// k_new / v_new instead of the cache, so attention sees them without waiting for the append.
// When the tile starts a segment (with_q), Q_COPIES more copies per wave bring the Q operand rows
// of the group's heads into the buffer's Q area: row r (clamped to R - 1) of head hg at
// [hg][r], LDS chunk c holding global chunk c ^ (r % QCH).
template <typename G, int POLICY = rows::kStreamPolicy, bool ROPE = false, typename RO = RowOffsets>
__device__ __forceinline__ void rows_issue(const AttnParams& p, const TileDesc& d, bool with_q, char* buf,
                                           const RO& ro, int I0 = 0, int I1 = rows::TILE / 4) {
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(int(threadIdx.x >> 6));
  const int64_t off = int64_t(d.pid < 0 ? 0 : d.pid) * p.page_stride +
                      int64_t(d.T0 & ((1 << p.log2_page) - 1)) * p.tok_elems + d.g * (G::HG * G::HD);
  const int tok_bytes = p.tok_elems * 2;
  if (__builtin_expect(!tile_has_new<G::TOK>(p, d), 1)) {
    const int range = G::TOK * tok_bytes;
    const __amdgpu_buffer_rsrc_t rk = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(p.k_cache + off), 0, range, 0x00020000);
    const __amdgpu_buffer_rsrc_t rv = __builtin_amdgcn_make_buffer_rsrc(uniform_ptr(p.v_cache + off), 0, range, 0x00020000);
#pragma unroll
    for (int i = I0; i < I1; ++i) {
      char* dst = buf + (i * 4 + wave) * rows::ROW_BYTES;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rk, (rows::lds_void*)dst, 16, int(ro.v[i]), 0, 0, POLICY);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rv, (rows::lds_void*)(dst + rows::TILE_BYTES), 16, int(ro.v[i]), 0,
                                               0, POLICY);
    }
  } else if constexpr (ROPE && G::P == 1 && G::S == 1) {
    // Rotary kernel: every lane of copy i reads token T0 + r (lane_src's token is the row), so a
    // row is one of this call's new tokens or a cached one for the whole wave; each copy picks its
    // base (the cache run, or the new row of k_new / v_new) with a scalar select and its lane
    // offset with a vector one, instead of per-lane 64-bit source arithmetic for every copy.
    const char* kg = uniform_ptr(reinterpret_cast<const char*>(p.k_cache + off));
    const char* vg = uniform_ptr(reinterpret_cast<const char*>(p.v_cache + off));
    const int hgl = (lane >> 4) % G::HG;
    // new row t of the sequence sits at kn0 + t * kn_ss (elements)
    const uint16_t* kn0 = uniform_ptr(p.k_new + d.b * p.kn_sb + int64_t(d.g * G::HG) * p.kn_sh - d.c * p.kn_ss);
    const uint16_t* vn0 = uniform_ptr(p.v_new + d.b * p.vn_sb + int64_t(d.g * G::HG) * p.vn_sh - d.c * p.vn_ss);
    const int64_t lk = 2 * (hgl * p.kn_sh), lv = 2 * (hgl * p.vn_sh);  // bytes
#pragma unroll
    for (int i = I0; i < I1; ++i) {
      const int r = i * 4 + wave;
      const int t = d.T0 + r;
      const bool nw = t >= d.c && t < d.L;  // wave-uniform
      const int64_t cc16 = 16 * ((lane & 15) ^ rows::swz(r));
      const char* ks = nw ? reinterpret_cast<const char*>(kn0 + t * p.kn_ss) + lk + cc16 : kg + ro.v[i];
      const char* vs = nw ? reinterpret_cast<const char*>(vn0 + t * p.vn_ss) + lv + cc16 : vg + ro.v[i];
      __builtin_amdgcn_global_load_lds(ks, (rows::lds_void*)(buf + r * rows::ROW_BYTES), 16, 0, POLICY);
      __builtin_amdgcn_global_load_lds(vs, (rows::lds_void*)(buf + rows::TILE_BYTES + r * rows::ROW_BYTES), 16, 0,
                                       POLICY);
    }
  } else {
    const char* kg = uniform_ptr(reinterpret_cast<const char*>(p.k_cache + off));
    const char* vg = uniform_ptr(reinterpret_cast<const char*>(p.v_cache + off));
#pragma unroll
    for (int i = I0; i < I1; ++i) {
      const int r = i * 4 + wave;
      const LaneSrc<G> ls = lane_src<G>(r, lane);
      const int t = d.T0 + ls.tt;
      const char* ks = kg + ro.v[i];
      const char* vs = vg + ro.v[i];
      if (t >= d.c && t < d.L) {
        const int jn = t - d.c;
        const int hh = d.g * G::HG + ls.hg;
        ks = reinterpret_cast<const char*>(p.k_new + d.b * p.kn_sb + jn * p.kn_ss + hh * p.kn_sh + 8 * ls.cc);
        vs = reinterpret_cast<const char*>(p.v_new + d.b * p.vn_sb + jn * p.vn_ss + hh * p.vn_sh + 8 * ls.cc);
      }
      __builtin_amdgcn_global_load_lds(ks, (rows::lds_void*)(buf + r * rows::ROW_BYTES), 16, 0, POLICY);
      __builtin_amdgcn_global_load_lds(vs, (rows::lds_void*)(buf + rows::TILE_BYTES + r * rows::ROW_BYTES), 16, 0,
                                       POLICY);
    }
  }
  if (with_q) {
#pragma unroll
    for (int i = 0; i < G::Q_COPIES; ++i) {
      const int qi = wave * G::Q_COPIES + i;                      // 1 KiB piece of the Q area
      const int ar = qi * (1024 / G::QROW) + lane / G::QCH;       // area row: head hq_g, query row rr
      const int row = ar % 16;
      const int gq = (lane % G::QCH) ^ (row % G::QCH);
      const uint16_t* src;
      if constexpr (ROPE) {
        src = uniform_ptr(p.q + d.b * p.q_sb + int64_t(d.g * G::HG) * p.g * p.q_sh) + ro.q[i];
      } else {
        const int hq_g = ar / 16;
        const int rr = min(row, p.R - 1);
        const int jq = rr / p.g;
        const int hq = rr - jq * p.g;
        src = p.q + d.b * p.q_sb + jq * p.q_ss + ((d.g * G::HG + hq_g) * p.g + hq) * p.q_sh + gq * 8;
      }
      if (ROPE && row >= p.R && row < p.R + 2 * p.s_q) {
        // rotary: rows R + 2 j and R + 2 j + 1 of every head's area hold the cos and sin rows of
        // position c + j (token j of this call)
        const int jr = (row - p.R) >> 1;
        const int pos = rope_position(p, d.c + jr);
        src = ((row - p.R) & 1 ? p.rot_sin : p.rot_cos) + int64_t(pos) * G::HD + gq * 8;
      }
      __builtin_amdgcn_global_load_lds(src, (rows::lds_void*)(buf + 2 * rows::TILE_BYTES + qi * 1024), 16, 0, 0);
    }
  }
}

// LDS byte address of a pointer into a __shared__ array.
__device__ __forceinline__ uint32_t lds_addr(const void* p) {
  return uint32_t(reinterpret_cast<uintptr_t>((const rows::lds_void*)p));
}

// LDS transpose reads (ds_read_b64_tr_b16) issued from inline assembly, and their wait.  The
// compiler's builtin for this instruction makes it wait for every outstanding global-to-LDS copy
// first (vmcnt(0)), which would drain the copy pipeline of the next tiles on every tile; as
// assembly the read issues at once.  The compiler does not track these reads: the values must not
// be touched before lds_tr_wait, which waits for every outstanding LDS access and hands the
// registers on (its "+v" operands keep every use of them after the wait).
template <int OFF>
__device__ __forceinline__ u32x2 lds_read_tr16_issue(uint32_t addr) {
  u32x2 r;
  asm volatile("ds_read_b64_tr_b16 %0, %1 offset:%2" : "=v"(r) : "v"(addr), "i"(OFF));
  return r;
}

__device__ __forceinline__ void lds_tr_wait(u32x2 (&a)[8], u32x2 (&b)[8]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+v"(a[0]), "+v"(a[1]), "+v"(a[2]), "+v"(a[3]), "+v"(a[4]), "+v"(a[5]), "+v"(a[6]), "+v"(a[7]),
                 "+v"(b[0]), "+v"(b[1]), "+v"(b[2]), "+v"(b[3]), "+v"(b[4]), "+v"(b[5]), "+v"(b[6]), "+v"(b[7]));
}

// MFMA operands of subtile s of wave w's slice of the tile in LDS buffer `buf` (load_tile's
// register layout); T0s is the subtile's first token, V rows at or past t_end read as zero.
template <typename G>
__device__ __forceinline__ void rows_read_tile(const char* buf, int w, int s, int T0s, int t_end,
                                               KVTile<G::HD>& tl) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int r = 8 * (li >> 2) + 4 * a + (li & 3);
#pragma unroll
    for (int kk = 0; kk < G::HD / 32; ++kk) {
      const int chunk = w * 16 + ((s * G::SCH + 4 * kk + lq) ^ rows::swz(r));
      tl.kr[a][kk] = *reinterpret_cast<const u32x4*>(buf + r * rows::ROW_BYTES + chunk * 16);
    }
  }
  const char* vb = buf + rows::TILE_BYTES;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    const int r = 8 * lq + e;
    if constexpr (G::HD == 128) {
      const int chunk = w * 16 + (li ^ rows::swz(r));
      const u32x4 v = *reinterpret_cast<const u32x4*>(vb + r * rows::ROW_BYTES + chunk * 16);
#pragma unroll
      for (int k = 0; k < 4; ++k) tl.vr[e].w[k] = v[k];
    } else {
      const int chunk = w * 16 + ((s * G::SCH + (li >> 1)) ^ rows::swz(r));
      const u32x2 v = *reinterpret_cast<const u32x2*>(vb + r * rows::ROW_BYTES + chunk * 16 + (li & 1) * 8);
      tl.vr[e].w[0] = v[0];
      tl.vr[e].w[1] = v[1];
    }
  }
  // rows past the sequence: P = 0 must not meet a stale NaN (only a sequence's last subtile has
  // them, so the selects stay off the common path)
  if (__builtin_expect(T0s + rows::TILE > t_end, 0)) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool keep = T0s + 8 * lq + e < t_end;
#pragma unroll
      for (int k = 0; k < G::HD / 32; ++k) tl.vr[e].w[k] = keep ? tl.vr[e].w[k] : 0u;
    }
  }
}

// The same tile at head_dim 128 with the V^T operands read by LDS transpose reads
// (ds_read_b64_tr_b16) instead of gathered from V rows by byte permutes.  In each 16-lane group,
// lane 4 j + c names 4 consecutive elements of row j of a 4 x 16 block and receives column (its
// index in the group) of the block.  Naming elements 32 c + 4 n .. + 3 of token rows 8 lq + j
// (then 8 lq + 4 + j) hands lane (li, lq) operand n = head-dim element 32 (li >> 2) + 4 n +
// (li & 3) over keys 8 lq .. 8 lq + 7, so the PV product leaves element 32 lq + 4 n + r of the
// lane's row in acc[n][r] (o_elem reads it).  vto[m] is the lane's byte offset in wave slice w of
// a V tile for operands 2 m and 2 m + 1 (+ 8 B), the same for every tile; the second four rows
// lie 4 KiB further, under the same swizzle (swz ignores bit 2 of the row).
template <typename G>
__device__ __forceinline__ void rows_vt_offsets(int w, uint32_t (&vto)[4]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
  const int t = 8 * lq + (li >> 2);
  const int c = li & 3;
#pragma unroll
  for (int m = 0; m < 4; ++m) vto[m] = uint32_t(t * rows::ROW_BYTES + (w * 16 + ((4 * c + m) ^ rows::swz(t))) * 16);
}

template <typename G>
__device__ __forceinline__ void rows_read_tile_vt(const char* buf, int w, int T0s, int t_end, const uint32_t (&vto)[4],
                                                  KVTile<G::HD>& tl) {
  static_assert(G::HD == 128 && G::S == 1, "transpose reads cover one 128-wide head row per LDS row");
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
  constexpr int kHi = 4 * rows::ROW_BYTES;
  const uint32_t vb = lds_addr(buf + rows::TILE_BYTES);
  u32x2 lo[8], hi[8];
  asm volatile("" ::: "memory");  // after this wave's own LDS stores (appended rows)
#pragma unroll
  for (int m = 0; m < 4; ++m) {
    const uint32_t a = vb + vto[m];
    lo[2 * m] = lds_read_tr16_issue<0>(a);
    lo[2 * m + 1] = lds_read_tr16_issue<8>(a);
    hi[2 * m] = lds_read_tr16_issue<kHi>(a);
    hi[2 * m + 1] = lds_read_tr16_issue<kHi + 8>(a);
  }
#pragma unroll
  for (int a = 0; a < 2; ++a) {
    const int r = 8 * (li >> 2) + 4 * a + (li & 3);
#pragma unroll
    for (int kk = 0; kk < 4; ++kk) {
      const int chunk = w * 16 + ((4 * kk + lq) ^ rows::swz(r));
      tl.kr[a][kk] = *reinterpret_cast<const u32x4*>(buf + r * rows::ROW_BYTES + chunk * 16);
    }
  }
  lds_tr_wait(lo, hi);
#pragma unroll
  for (int n = 0; n < 8; ++n) {
    tl.vr[n].w[0] = lo[n][0];
    tl.vr[n].w[1] = lo[n][1];
    tl.vr[n].w[2] = hi[n][0];
    tl.vr[n].w[3] = hi[n][1];
  }
  // keys past the sequence: P = 0 must not meet a stale NaN (word k of an operand holds keys
  // 8 lq + 2 k and 2 k + 1); only a sequence's last subtile has them
  if (__builtin_expect(T0s + rows::TILE > t_end, 0)) {
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const int t = T0s + 8 * lq + 2 * k;
      const uint32_t keep = (t < t_end ? 0x0000FFFFu : 0u) | (t + 1 < t_end ? 0xFFFF0000u : 0u);
#pragma unroll
      for (int n = 0; n < 8; ++n) tl.vr[n].w[k] &= keep;
    }
  }
}

// Element 4 DPL lq + DPL r + n of the lane's output row from its accumulators: acc[n][r] with V^T
// gathered by permutes, acc[2 r + n / 4][n % 4] with V^T from transpose reads (rows_read_tile_vt).
template <bool VT, int DPL>
__device__ __forceinline__ float o_elem(const f32x4 (&a)[DPL], int n, int r) {
  if constexpr (VT)
    return a[2 * r + (n >> 2)][n & 3];
  else
    return a[n][r];
}

// Chunk ch of row `row` of group head hg's part of the buffer's Q area (stored at chunk
// ch ^ (row % QCH)).
template <typename G>
__device__ __forceinline__ u32x4 q_area_chunk(const char* buf, int hg, int row, int ch) {
  return *reinterpret_cast<const u32x4*>(buf + 2 * rows::TILE_BYTES + (hg * 16 + row) * G::QROW +
                                         ((ch ^ (row % G::QCH)) << 4));
}

// Q^T operand (load_q's layout) of group head hg's rows from the buffer's Q area; rows li >= R
// get 0.
template <typename G>
__device__ __forceinline__ void rows_read_q(const AttnParams& p, const char* buf, int hg,
                                            bf16x8 (&qf)[1][G::HD / 32]) {
  constexpr int KK = G::HD / 32;
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
#pragma unroll
  for (int kk = 0; kk < KK; ++kk) {
    const u32x4 v = q_area_chunk<G>(buf, hg, li, lq + 4 * kk);
    qf[0][kk] = __builtin_bit_cast(bf16x8, li < p.R ? v : u32x4{0u, 0u, 0u, 0u});
  }
}

// Rotary for the Q rows of a segment start in the buffer's Q area, in place: row r < R of head
// hg (token j = r / g) with the cos / sin rows of its position, R + 2 j and R + 2 j + 1 of the
// area.  The waves of head hg (one per phase) share its rows, lane (row, pair c) rotating chunk c
// and its rotate_half partner c + HD/16: one chunk pair per lane at R <= 8, where rotating in
// load_q's layout costs every lane HD/64 pairs for all 16 area rows (7B decode: 31.8 us per call
// that way, against 29.3 us without rotary).  With phases the other waves of the head then read
// what this one wrote, behind a barrier.
template <typename G>
__device__ __forceinline__ void rows_rope_q_area(const AttnParams& p, char* buf) {
  constexpr int PC = G::HD / 16;  // chunk pairs per head row
  constexpr int RPW = 64 / PC;    // rows per wave and pass
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hg = w % G::HG;
  const int ph = w / G::HG;
  const int pc = lane % PC;
  for (int r0 = ph * RPW; r0 < p.R; r0 += G::P * RPW) {
    const int row = r0 + lane / PC;
    if (row < p.R) {
      const int rc = p.R + 2 * (row / p.g);
      char* rb = buf + 2 * rows::TILE_BYTES + (hg * 16 + row) * G::QROW;
      u32x4* pa = reinterpret_cast<u32x4*>(rb + ((pc ^ (row % G::QCH)) << 4));
      u32x4* pb = reinterpret_cast<u32x4*>(rb + (((pc + PC) ^ (row % G::QCH)) << 4));
      u32x4 a = *pa, b = *pb;
      rope_pair(a, b, q_area_chunk<G>(buf, hg, rc, pc), q_area_chunk<G>(buf, hg, rc + 1, pc),
                q_area_chunk<G>(buf, hg, rc, pc + PC), q_area_chunk<G>(buf, hg, rc + 1, pc + PC));
      *pa = a;
      *pb = b;
    }
  }
  if constexpr (G::P > 1) {
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's rows are written
    raw_barrier();
  }
}

// Whether tile d's copies bring the buffer's Q area (Q in LDS): when the tile starts a segment,
// and with rotary tables when it holds new rows, whose rotation needs the cos / sin rows there.
template <typename G, bool ROPE>
__device__ __forceinline__ bool q_area_copy(const AttnParams& p, const TileDesc& d, bool q_in_lds) {
  return q_in_lds && (d.T0 == p.k0 || (ROPE && tile_has_new<G::TOK>(p, d)));
}

// Word wd (elements 2 wd, 2 wd + 1) of chunk ch of row `row` of group head hg's part of the
// buffer's Q area.
template <typename G>
__device__ __forceinline__ uint32_t q_area_word(const char* buf, int hg, int row, int ch, int wd) {
  return *reinterpret_cast<const uint32_t*>(buf + 2 * rows::TILE_BYTES + (hg * 16 + row) * G::QROW +
                                            ((ch ^ (row % G::QCH)) << 4) + 4 * wd);
}

// Rotary for this call's new K rows of tile d in LDS buffer `buf` (wave w's slice: head hg, its
// phase's tokens), before they are read or appended: lane (row t, word i of the first half)
// rotates that word and its rotate_half partner HD/4 words on with the cos / sin rows of the
// token's position from head hg's Q area -- a decode step's one new row spread over HD/4 lanes.
template <typename G>
__device__ __forceinline__ void rows_rope_new_k(const AttnParams& p, const TileDesc& d, char* buf) {
  constexpr int PC = G::HD / 16;  // rotary chunk pairs per head row
  constexpr int WPR = 4 * PC;     // word pairs per head row
  constexpr int RPP = 64 / WPR;   // token rows per pass
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hg = w % G::HG;
  const int ph = w / G::HG;
  const int pc = (lane % WPR) >> 2;
  const int wd = lane & 3;
#pragma unroll
  for (int s = 0; s < G::S; ++s) {
    const int T0s = d.T0 + rows::TILE * (ph * G::S + s);
    const int t_lo = max(T0s, d.c);
    const int t_hi = min(T0s + rows::TILE, d.L);
    for (int t0 = t_lo; t0 < t_hi; t0 += RPP) {
      const int t = t0 + lane / WPR;
      if (t < t_hi) {
        const int r = t - T0s;
        const int rc = p.R + 2 * (t - d.c);
        char* row = buf + r * rows::ROW_BYTES + w * 256;
        uint32_t* pa = reinterpret_cast<uint32_t*>(row + (((s * G::SCH + pc) ^ rows::swz(r)) << 4) + 4 * wd);
        uint32_t* pb = reinterpret_cast<uint32_t*>(row + (((s * G::SCH + pc + PC) ^ rows::swz(r)) << 4) + 4 * wd);
        uint32_t a = *pa, b = *pb;
        rope_word(a, b, q_area_word<G>(buf, hg, rc, pc, wd), q_area_word<G>(buf, hg, rc + 1, pc, wd),
                  q_area_word<G>(buf, hg, rc, pc + PC, wd), q_area_word<G>(buf, hg, rc + 1, pc + PC, wd));
        *pa = a;
        *pb = b;
      }
    }
  }
}

// Append: wave w stores its slice of the new rows of tile d (head hg, its phase's tokens),
// already in LDS buffer `buf`, to the cache (a page id outside the pool was flagged and is
// skipped).
template <typename G>
__device__ __forceinline__ void rows_append_from_lds(const AttnParams& p, const TileDesc& d, const char* buf) {
  if (d.pid < 0) return;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int hg = w % G::HG;
  const int ph = w / G::HG;
  constexpr int RPP = 64 / G::SCH;  // token rows per pass
  const int ch = lane % G::SCH;
#pragma unroll
  for (int s = 0; s < G::S; ++s) {
    const int T0s = d.T0 + rows::TILE * (ph * G::S + s);
    const int t_lo = max(T0s, d.c);
    const int t_hi = min(T0s + rows::TILE, d.L);
    for (int t0 = t_lo; t0 < t_hi; t0 += RPP) {
      const int t = t0 + lane / G::SCH;
      if (t < t_hi) {
        const int r = t - T0s;
        const int pos = (w * 16 + ((s * G::SCH + ch) ^ rows::swz(r))) * 16;
        const u32x4 kv = *reinterpret_cast<const u32x4*>(buf + r * rows::ROW_BYTES + pos);
        const u32x4 vv = *reinterpret_cast<const u32x4*>(buf + rows::TILE_BYTES + r * rows::ROW_BYTES + pos);
        const int64_t dst = int64_t(d.pid) * p.page_stride + int64_t(t & ((1 << p.log2_page) - 1)) * p.tok_elems +
                            (d.g * G::HG + hg) * G::HD + 8 * ch;
        st16(p.k_cache + dst, kv);
        st16(p.v_cache + dst, vv);
      }
    }
  }
}

// s_waitcnt vmcnt(n) for a wave-uniform n, rounded down to a multiple of 4 (a stricter wait) and
// capped at 60: the immediate must be a constant, so the count selects among the encodings
// (vmcnt bits [3:0] and [15:14]; expcnt and lgkmcnt fields left at "no wait").  (An exact wait,
// one encoding per count, measured 6.5 us slower per config-5 verify call and no faster on decode.)
__device__ __forceinline__ void wait_vmcnt_at_most(int n) {
#define PKV_VMCNT_CASE(k) \
  case k: __builtin_amdgcn_s_waitcnt(0x0F70 | ((4 * k) & 15) | (((4 * k) >> 4) << 14)); break;
  switch (min(max(n, 0), 60) >> 2) {
    PKV_VMCNT_CASE(1) PKV_VMCNT_CASE(2) PKV_VMCNT_CASE(3) PKV_VMCNT_CASE(4) PKV_VMCNT_CASE(5)
    PKV_VMCNT_CASE(6) PKV_VMCNT_CASE(7) PKV_VMCNT_CASE(8) PKV_VMCNT_CASE(9) PKV_VMCNT_CASE(10)
    PKV_VMCNT_CASE(11) PKV_VMCNT_CASE(12) PKV_VMCNT_CASE(13) PKV_VMCNT_CASE(14) PKV_VMCNT_CASE(15)
    default: __builtin_amdgcn_s_waitcnt(0x0F70); break;
  }
#undef PKV_VMCNT_CASE
}

// Q^T operand of head h's 16*NT rows of sequence d.b straight from q into registers (load_q's
// layout).  Used where NT > 1, whose Q does not fit the LDS buffers.  Padding rows (>= R) repeat
// row R - 1: they are computed and never stored, and registers kept exactly as loaded are waited
// for at their first use only (zeroing them would wait for the loads, and with them for every
// tile copy issued after them, where they are loaded).
template <int HD, int NT>
__device__ __forceinline__ void rows_load_q(const AttnParams& p, const TileDesc& d, int h,
                                            bf16x8 (&qf)[NT][HD / 32]) {
  const int lane = threadIdx.x & 63;
  const int li = lane & 15;
  const int lq = lane >> 4;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int rc = min(li + 16 * nt, p.R - 1);
    const int jq = rc / p.g;
    const int hq = rc - jq * p.g;
    const uint16_t* base = p.q + d.b * p.q_sb + jq * p.q_ss + (h * p.g + hq) * p.q_sh + 8 * lq;
#pragma unroll
    for (int kk = 0; kk < HD / 32; ++kk) qf[nt][kk] = __builtin_bit_cast(bf16x8, ld16(base + 32 * kk));
  }
}

template <int NT>
__device__ __forceinline__ void compute_tile_prefill(const AttnParams& p, const KVTile<128>& tl, int T0,
                                                     const bf16x8 (&qf)[NT][4], const int (&lim)[NT], int lim_min,
                                                     float (&m_run)[NT], float (&l_run)[NT], f32x4 (&acc)[NT][8]);
template <int NT>
__device__ __forceinline__ void compute_tile_prefill_vt(const AttnParams& p, const KVTile<128>& tl, int T0,
                                                        const bf16x8 (&qf)[NT][4], const int (&lim)[NT], int lim_min,
                                                        float (&m_run)[NT], float (&l_run)[NT],
                                                        f32x4 (&acc)[NT][8]);

// ---- split-K partials of decode_lean_kernel, merged inside the launch ----
// For the in-launch merge, partials are written and read with the sc1 cache policy:
// device-coherent accesses (what agent-scope atomics compile to on gfx950), so a workgroup on one
// XCD reads what another XCD wrote without any L2-wide writeback or invalidate.  Stores go
// through a buffer resource on the workspace (byte offsets from ws_o).
constexpr int kCoherent = 16;  // cache-policy bit sc1

__device__ __forceinline__ __amdgpu_buffer_rsrc_t ws_rsrc(const AttnParams& p) {
  return __builtin_amdgcn_make_buffer_rsrc(p.ws_o, 0, 0x7fffffff, 0x00020000);
}
// Stores of one (row, lane) share of an fp16 partial and its log-sum-exp with cache policy POL:
// device-coherent (kCoherent) when the merge runs inside the launch, plain for the two-pass merge.
// ov[r]: the lane's DPL head-dim elements of accumulator row r as fp16 pairs (DPL / 2 words).
template <int POL, int DPL>
__device__ __forceinline__ void ws_store_partial(__amdgpu_buffer_rsrc_t rs, uint32_t o_off,
                                                 const uint32_t (&ov)[4][DPL / 2], bool with_lse, uint32_t lse_off,
                                                 float lse) {
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    if constexpr (DPL == 8)
      __builtin_amdgcn_raw_buffer_store_b128(u32x4{ov[r][0], ov[r][1], ov[r][2], ov[r][3]}, rs,
                                             int(o_off + 16u * r), 0, POL);
    else
      __builtin_amdgcn_raw_buffer_store_b64(u32x2{ov[r][0], ov[r][1]}, rs, int(o_off + 8u * r), 0, POL);
  }
  if (with_lse) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, lse), rs, int(lse_off), 0, POL);
}

// Sequence-aligned split.  A range that holds the end of one sequence and the start of the next
// pays a second segment (its epilogue and partial, the next sequence's Q and limits) and ends
// ~2.4 us after a one-segment range at 7B decode, B = 8 (timeline stamps), so the merge waits for
// it.  When ceil(t_b / per) ranges per sequence (t_b tiles, per = ceil(T / G) as in the plain
// split), over every head group, fit the G workgroups, the launch uses those instead: sequence b's
// tiles in ranges of per tiles (the last shorter), ranges of head group g numbered after those of
// group g - 1, no range crossing a sequence.  Otherwise (7B decode at B = 32, 14B) the plain
// contiguous split stays.  RangeTable: lane l of register q holds the first aligned range of
// sequence 64q + l within its head group; rtotal is the aligned ranges of one head group.
template <int NCH>
struct RangeTable {
  int rfirst[NCH];
  int rtotal;
};

template <int NCH, int TOK>
__device__ __forceinline__ void range_table(const AttnParams& p, const SeqTable<NCH>& st, int per,
                                            RangeTable<NCH>& rt) {
  const int lane = threadIdx.x & 63;
  // ceil(t / per) from a float reciprocal: t < 2^22 tiles, so the estimate's floor is within one
  // of t / per from below, and two steps make it exact (shorter than an integer division on the
  // launch's critical path, before the first block-table read)
  const float inv = 1.f / float(per);
  int base = 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const int t = 64 * q + lane < p.batch ? seq_tiles<TOK>(p, st.L[q]) : 0;
    int r = int(float(t) * inv);
    r += r * per < t ? 1 : 0;
    r += r * per < t ? 1 : 0;
    const int incl = base + wave_incl_scan(r);
    rt.rfirst[q] = incl - r;
    base = __builtin_amdgcn_readlane(incl, 63);
  }
  rt.rtotal = base;
}

// Tiles [s, e) of workgroup w under the aligned split (s == e past its last range).  Every real
// sequence has at least one range, so the ranges' first indices rise strictly over the sequences
// and the sequence of range w is the last one whose first range is <= w.
template <int NCH, int TOK>
__device__ __forceinline__ void aligned_range(const AttnParams& p, const SeqTable<NCH>& st, const RangeTable<NCH>& rt,
                                              int T1, int per, int w, int& s, int& e) {
  const int lane = threadIdx.x & 63;
  const int g = w / rt.rtotal;
  const int wg = w - g * rt.rtotal;
  int first = 0, L = 0, r0 = 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    const uint64_t m = __ballot(64 * q + lane < p.batch && rt.rfirst[q] <= wg);
    if (m) {
      const int pos = 63 - __clzll(m);
      first = __builtin_amdgcn_readlane(st.first[q], pos);
      L = __builtin_amdgcn_readlane(st.L[q], pos);
      r0 = __builtin_amdgcn_readlane(rt.rfirst[q], pos);
    }
  }
  s = g * T1 + first + (wg - r0) * per;
  e = min(s + per, g * T1 + first + seq_tiles<TOK>(p, L));
  if (g >= p.n_groups) e = s;
}

// Parts of sequence b (head group g) in a balanced launch: np ranges from w0 on, and the
// workspace slot of part 0.  Plain split: the ranges its tiles fall in (per tiles each); range w0
// holds b in its first segment only when b starts at w0's first tile, and every later part is
// its range's first segment, slot 2w.  Aligned split: ceil(t_b / per) ranges of their own, each
// a first segment (slot 2w).
struct SeqParts {
  int np, w0, slot0;
};

template <int NCH, int TOK>
__device__ __forceinline__ SeqParts seq_parts(const AttnParams& p, const SeqTable<NCH>& st, const RangeTable<NCH>& rt,
                                              bool aligned, int b, int g, int T1, int per) {
  int first = 0, L = 0, r0 = 0;
#pragma unroll
  for (int q = 0; q < NCH; ++q) {
    if (q == (b >> 6)) {
      first = __builtin_amdgcn_readlane(st.first[q], b & 63);
      L = __builtin_amdgcn_readlane(st.L[q], b & 63);
      r0 = __builtin_amdgcn_readlane(rt.rfirst[q], b & 63);
    }
  }
  SeqParts sp;
  const int t = seq_tiles<TOK>(p, L);
  if (aligned) {
    sp.w0 = g * rt.rtotal + r0;
    sp.np = (t + per - 1) / per;
    sp.slot0 = 2 * sp.w0;
  } else {
    first += g * T1;  // the group's first tile
    sp.w0 = first / per;
    sp.np = (first + t - 1) / per - sp.w0 + 1;
    sp.slot0 = 2 * sp.w0 + (first != sp.w0 * per ? 1 : 0);
  }
  return sp;
}

// A split-K partial of (workspace slot, KV head h of the group): per query row, O / l as fp16
// (16 B per 8 head-dim elements; O / l is a convex combination of V rows, so fp16's range and
// 2^-11 rounding are ample next to the bf16 output) and its log-sum-exp lse = m + log2(l) in fp32
// (-inf when the row saw no key).  O of row r: byte (((slot * HG + h) * R + r) * head_dim) * 2
// from ws_o; lse: float ((slot * HG + h) * R + r) from ws_ml.
typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ uint32_t pack_f16x2(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2{lo, hi}, f16x2));  // RNE
}
// A finite value fp16 cannot hold: under round-to-nearest-even everything from 65520 up becomes
// inf (bf16 V rows beyond that magnitude; flagged as PKV_STATUS_PARTIAL_RANGE).
__device__ __forceinline__ bool f16_overflows(float lo, float hi) {
  return fmaxf(fabsf(lo), fabsf(hi)) >= 65520.f;
}
__device__ __forceinline__ void unpack_f16x8(const u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const _Float16 lo = __builtin_bit_cast(_Float16, uint16_t(v[k] & 0xffffu));
    const _Float16 hi = __builtin_bit_cast(_Float16, uint16_t(v[k] >> 16));
    f[2 * k] = float(lo);
    f[2 * k + 1] = float(hi);
  }
}

// Butterfly max / sum over all 64 lanes without LDS: DPP swaps inside each 16-lane row, then the
// row swaps of max_over_quads / sum_over_quads.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false)));   // lane ^ 1
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false)));   // lane ^ 2
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false)));  // half-row mirror
  v = fmaxf(v, __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xf, 0xf, false)));  // row mirror
  return max_over_quads(v);
}
__device__ __forceinline__ float wave_sum(float v) {
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xf, 0xf, false));
  v += __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xf, 0xf, false));
  return sum_over_quads(v);
}

// Log-sum-exp merge of query rows rr[0 .. NR) of (sequence b, KV head hk; rr[q] < 0: none) over
// n_parts split-K partials (part u of row r at workspace row row_of(u, r)) into the bf16 output,
// by one wave.  The merge is latency-bound, so everything one round trip can fetch is fetched at
// once, for up to BIG parts:
// lane u loads part u's log-sum-exp, and lane (g, c) = (lane / CPR, lane % CPR) loads the 16 bytes
// of head-dim chunk c (elements 8c .. 8c + 7; CPR = head_dim / 8 chunks per row) of parts g,
// g + PG, g + 2 PG, ... of the row (PG = 64 / CPR part groups; 16 or 8 loads in flight per lane:
// one round trip for 64 parts, where 4-byte loads needed one per 8).  Weights reach the lanes by
// ds_bpermute, the part groups are summed with lane swaps, and lanes of group 0 store the row.
// No LDS, no barrier; loops stay rolled where the code would otherwise grow (every launch starts
// from a cold instruction cache).  COH: device-coherent loads (partials written during this
// launch, by workgroups on any XCD).
// BIG: parts per round trip beyond the first 8 (64: up to 16 loads in flight per lane; the
// combine launch takes 32, for a register count at which several of its workgroups share a CU:
// config-5 verify's combine 9.9 -> 7.9 us, its cascade merge 13.5 -> 9.2 us; 128 for a single
// sequence's parts, lane u then loading the log-sum-exps of parts u and u + 64).
template <typename G, bool COH, int NR, int BIG, typename RowOf>
__device__ __forceinline__ void merge_rows(const AttnParams& p, int hk, int b, const int (&rr)[NR], int n_parts,
                                           RowOf row_of) {
  constexpr int HD = G::HD;
  constexpr int CPR = HD / 8;   // 16-byte chunks per part row
  constexpr int PG = 64 / CPR;  // part groups
  const int lane = threadIdx.x & 63;
  const int pg = lane / CPR;
  const int dc = lane % CPR;
  const __amdgpu_buffer_rsrc_t rs = ws_rsrc(p);
  const uint32_t lse0 = uint32_t(p.ws_ml - p.ws_o) * 4u;
  const char* o16 = reinterpret_cast<const char*>(p.ws_o);  // fp16 rows of HD * 2 bytes
  float M_run[NR], S_run[NR];
  float acc[NR][8];
#pragma unroll
  for (int q = 0; q < NR; ++q) {
    M_run[q] = -INFINITY;
    S_run[q] = 0.f;
#pragma unroll
    for (int e = 0; e < 8; ++e) acc[q][e] = 0.f;
  }
  // parts u0 .. u0 + nb - 1 (nb <= PG KP) of every row: every load at once, then the weights and
  // the sums (rows with rr[q] < 0 are skipped)
  auto batch = [&](auto kp, int u0, int nb) {
    constexpr int KP = decltype(kp)::value;
    constexpr int NL = (KP * PG + 63) / 64;  // log-sum-exps per lane: part u at lane u % 64, slot u / 64
    float lse[NR][NL];
    u32x4 x[NR][KP];
#pragma unroll
    for (int q = 0; q < NR; ++q) {
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        lse[q][l] = -INFINITY;
        if (rr[q] >= 0 && lane + 64 * l < nb) {
          const int64_t row = row_of(u0 + lane + 64 * l, rr[q]);
          if constexpr (COH)
            lse[q][l] = __builtin_bit_cast(
                float, __builtin_amdgcn_raw_buffer_load_b32(rs, int(lse0 + uint32_t(row) * 4u), 0, kCoherent));
          else
            lse[q][l] = p.ws_ml[row];
        }
      }
#pragma unroll
      for (int k = 0; k < KP; ++k) {
        const int part = PG * k + pg;
        x[q][k] = u32x4{0u, 0u, 0u, 0u};
        if (rr[q] >= 0 && part < nb) {
          const int64_t row = row_of(u0 + part, rr[q]);
          if constexpr (COH)
            x[q][k] = __builtin_amdgcn_raw_buffer_load_b128(rs, int(uint32_t(row) * (HD * 2) + dc * 16), 0, kCoherent);
          else
            x[q][k] = ld16(o16 + row * (HD * 2) + dc * 16);
        }
      }
    }
#pragma unroll
    for (int q = 0; q < NR; ++q) {
      float lmax = lse[q][0];
#pragma unroll
      for (int l = 1; l < NL; ++l) lmax = fmaxf(lmax, lse[q][l]);
      const float M_new = fmaxf(M_run[q], wave_max(lmax));
      const float M_use = (M_new == -INFINITY) ? 0.f : M_new;
      float w[NL], wsum = 0.f;
#pragma unroll
      for (int l = 0; l < NL; ++l) {
        w[l] = fast_exp2(lse[q][l] - M_use);  // 0 for parts past the batch
        wsum += w[l];
      }
      const float resc = fast_exp2(M_run[q] - M_use);
      S_run[q] = S_run[q] * resc + wave_sum(wsum);
      M_run[q] = M_new;
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[q][e] *= resc;
#pragma unroll
      for (int k = 0; k < KP; ++k) {
        // part PG k + pg: slot (PG k) / 64 for every pg (PG divides 64)
        const float wk = __shfl(w[(PG * k) / 64], (PG * k + pg) & 63, 64);
        float f[8];
        unpack_f16x8(x[q][k], f);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[q][e] += wk * f[e];
      }
    }
  };
  if (n_parts <= 8) {
    batch(std::integral_constant<int, 8 / PG>(), 0, n_parts);
  } else {
#pragma unroll 1
    for (int u0 = 0; u0 < n_parts; u0 += BIG)
      batch(std::integral_constant<int, BIG / PG>(), u0, min(BIG, n_parts - u0));
  }
#pragma unroll
  for (int q = 0; q < NR; ++q) {
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      if constexpr (PG == 8) acc[q][e] += __shfl_xor(acc[q][e], 8, 64);
      acc[q][e] = sum_over_quads(acc[q][e]);
    }
    if (pg == 0 && rr[q] >= 0) {
      const float inv = S_run[q] > 0.f ? 1.f / S_run[q] : 0.f;
      const int j = rr[q] / p.g;
      const int hq = rr[q] - j * p.g;
      u32x4 ov;
#pragma unroll
      for (int k = 0; k < 4; ++k) ov[k] = pack_bf16x2(acc[q][2 * k] * inv, acc[q][2 * k + 1] * inv);
      st16(p.out + b * p.o_sb + j * p.o_ss + (hk * p.g + hq) * p.o_sh + 8 * dc, ov);
    }
  }
}

// The in-launch merge (decode rows, R <= 16).  Workgroups lean_grid, lean_grid + 1, ... of a
// balanced launch merge the partials of (sequence b, KV head hk, query rows 4 rq .. 4 rq + 3),
// one wave per row (two rows per wave, with half the workgroups, measured no faster): they wait
// for the arrival counter of (sequence, head, row group) to reach the part count, then merge with
// merge_rows.  Every XCD dispatches its workgroups in order, so these start only on CUs that
// decode workgroups of lower index (which never wait) have left or never needed: a merge
// workgroup waits only for workgroups that are already running.  The wait is bounded
// (kMergeSpinLimit polls; beyond it the wave flags PKV_STATUS_MERGE_TIMEOUT and leaves), so
// every wave exits.
// Each row group has a counter of its own, which only its merge workgroup reads: a decode wave
// adds 1 to the counter of every row group of each (sequence, head) it wrote a part of, and the
// merge workgroup re-arms its counter with an atomic store of 0 (no read-modify-write, nothing
// waits for it) as soon as the count is complete
// (every part has arrived, so nothing adds to it again in this launch).  No atomic round trip
// follows the merge: with one shared counter whose readers counted themselves out, the last
// reader's fetch-and-add (and its re-arming store) sat between the merge and the end of the launch.
// A merge that times out marks its counter with kMergePoison (parts still arriving add below it);
// a later call's merge workgroup that finds the mark, or a count above the part count, flags
// PKV_STATUS_MERGE_TIMEOUT and merges nothing until the counters are cleared.
#ifndef PKV_MERGE_SPIN_LIMIT
#define PKV_MERGE_SPIN_LIMIT (1 << 20)
#endif
constexpr int kMergeSpinLimit = PKV_MERGE_SPIN_LIMIT;
constexpr int kMergePoison = 1 << 30;

#ifdef PKV_TILE_STAMPS
// Timeline instrumentation of decode_lean_kernel (decode rows), compiled only into the stamps
// variant of the library (libprism_kv_stamps.so, built with -DPKV_TILE_STAMPS): s_memrealtime
// readings (a 100 MHz clock) of every decode workgroup's start, each tile's landing (after the
// wait and barrier at the top of its iteration; kept in lanes of one register, so no memory
// operation enters the tile loop), the end of its range and its arrival, and of every merge
// workgroup's start, count complete and merge done.  Decode workgroup w: words w * 32 + [0 start,
// 1 range end, 2 arrival counted, 3 tiles, 4 mask of segment-end iterations, 8 + j tile j
// landed (j < 24)]; merge workgroup m: words kStampMerge0 + 4 m + [0 start, 1 count complete,
// 2 merge stored, 3 parts].  Read by pkv_tile_stamps, cleared by pkv_tile_stamps_clear.
constexpr int kStampWgs = 1024, kStampWgWords = 32, kStampMerges = 4096;
constexpr int kStampMerge0 = kStampWgs * kStampWgWords;
constexpr int kStampWords = kStampMerge0 + 4 * kStampMerges;
__device__ uint64_t g_tile_stamps[kStampWords];
__device__ __forceinline__ void stamp_now(int i) {
  if (i < kStampWords) g_tile_stamps[i] = __builtin_amdgcn_s_memrealtime();
}
__device__ __forceinline__ void stamp_value(int i, uint64_t v) {
  if (i < kStampWords) g_tile_stamps[i] = v;
}
#endif

// Arrival counter of (segment gb = g * batch + b, head h of the group, row group rq).
template <typename G>
__device__ __forceinline__ int* merge_counter(const AttnParams& p, int gb, int h, int rq, int n_rq) {
  return p.ws_cnt + ((gb * G::HG + h) * n_rq + rq) * p.cnt_stride;
}

template <typename G, int NCH, int MBIG>
__device__ __forceinline__ void merge_workgroup(const AttnParams& p, const SeqTable<NCH>& st,
                                                const RangeTable<NCH>& rt, bool aligned, int T1, int per,
                                                int* ready_s) {
  const int m = int(blockIdx.x) - p.lean_grid;
  const int n_rq = (p.R + 3) / 4;
  const int hk = m % p.n_kv;
  const int rq = (m / p.n_kv) % n_rq;
  const int b = m / (p.n_kv * n_rq);
  if (b >= p.batch) return;
  const int g = hk / G::HG;
  const int h = hk - g * G::HG;
  const SeqParts sp = seq_parts<NCH, G::TOK>(p, st, rt, aligned, b, g, T1, per);
  if (sp.np <= 1) return;  // the sequence lies in one range: its output is written already
  int* cnt = merge_counter<G>(p, g * p.batch + b, h, rq, n_rq);
#ifdef PKV_TILE_STAMPS
  if (threadIdx.x == 0) stamp_now(kStampMerge0 + 4 * m);
#endif
  // one poller per workgroup (every poll is a device-coherent load of a line that the arrivals
  // update; more pollers only queue behind each other and the arrivals), the others wait at the
  // barrier (ready_s: a word of the launch's LDS, which merge workgroups use for nothing else)
  if (threadIdx.x == 0) {
    int seen = 0;
    for (int i = 0; i < kMergeSpinLimit; ++i) {
      seen = __hip_atomic_load(cnt, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if (seen >= sp.np) break;
      __builtin_amdgcn_s_sleep(4);
    }
    // 1: every part is in; 2: a count an earlier call left (poisoned by its timeout, or above the
    // part count); 0: timed out
    const int state = seen == sp.np ? 1 : (seen > sp.np ? 2 : 0);
    *ready_s = state;
#ifdef PKV_TILE_STAMPS
    stamp_now(kStampMerge0 + 4 * m + 1);
#endif
    if (state == 1)
      __hip_atomic_store(cnt, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    else
      flag_status(p.status, PKV_STATUS_MERGE_TIMEOUT);
    if (state == 0) __hip_atomic_fetch_or(cnt, kMergePoison, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  __syncthreads();
  const int r0 = 4 * rq + int(threadIdx.x >> 6);
  const int rr[1] = {r0 < p.R ? r0 : -1};
  if (*ready_s == 1 && rr[0] >= 0)
    merge_rows<G, true, 1, MBIG>(p, hk, b, rr, sp.np, [&](int part, int r) -> int64_t {
      const int slot = part == 0 ? sp.slot0 : 2 * (sp.w0 + part);
      return (int64_t(slot) * G::HG + h) * p.R + r;
    });
#ifdef PKV_TILE_STAMPS
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the merged rows are stored
  __syncthreads();
  if (threadIdx.x == 0) {
    stamp_now(kStampMerge0 + 4 * m + 2);
    stamp_value(kStampMerge0 + 4 * m + 3, uint64_t(sp.np));
  }
#endif
}

// Phase merge at the end of a segment (geometries with P > 1): the waves of phases 1 .. P-1
// publish their softmax state (m, the lane's partial l, O) for their head in the K/V area of
// the tile buffer `buf` just consumed (its next copies are issued only after this), and the
// phase-0 wave of each head folds them into its own; as many states per round as the 64 KiB
// area holds, lane-major so every access is conflict-free.  Every wave of the workgroup calls it.
template <typename G, int NT>
__device__ __forceinline__ void phase_merge(char* buf, float (&m_run)[NT], float (&l_run)[NT],
                                            f32x4 (&acc)[NT][G::HD / 16]) {
  constexpr int DPL = G::HD / 16;
  constexpr int FPL = NT * (4 * DPL + 2);  // floats of one lane's state
  constexpr int SLOTS = (2 * rows::TILE_BYTES / 4) / (FPL * 64);
  static_assert(SLOTS >= 1, "a wave state must fit the tile buffer");
  constexpr int WRITERS = (G::P - 1) * G::HG;
  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  const int k = w - G::HG;  // writer index of phases >= 1 (wave w = hg + HG ph)
  float* area = reinterpret_cast<float*>(buf);
#pragma unroll 1
  for (int k0 = 0; k0 < WRITERS; k0 += SLOTS) {
    if (k >= k0 && k < k0 + SLOTS) {
      float* a = area + (k - k0) * FPL * 64 + lane;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        float* an = a + nt * (4 * DPL + 2) * 64;
        an[0] = m_run[nt];
        an[64] = l_run[nt];
#pragma unroll
        for (int n = 0; n < DPL; ++n)
#pragma unroll
          for (int r = 0; r < 4; ++r) an[(2 + 4 * n + r) * 64] = acc[nt][n][r];
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    raw_barrier();
    if (w < G::HG) {
#pragma unroll 1
      for (int kw = w + ((k0 + G::HG - 1 - w) / G::HG) * G::HG; kw < min(WRITERS, k0 + SLOTS); kw += G::HG) {
        // writer kw: head kw % HG = w
        const float* a = area + (kw - k0) * FPL * 64 + lane;
#pragma unroll
        for (int nt = 0; nt < NT; ++nt) {
          const float* an = a + nt * (4 * DPL + 2) * 64;
          const float mo = an[0];
          const float lo = an[64];
          const float M = fmaxf(m_run[nt], mo);
          const float Mu = M == -INFINITY ? 0.f : M;
          const float fs = fast_exp2(m_run[nt] - Mu);  // 0 for a state that saw no key
          const float fo = fast_exp2(mo - Mu);
          l_run[nt] = l_run[nt] * fs + lo * fo;
#pragma unroll
          for (int n = 0; n < DPL; ++n)
#pragma unroll
            for (int r = 0; r < 4; ++r) acc[nt][n][r] = acc[nt][n][r] * fs + an[(2 + 4 * n + r) * 64] * fo;
          m_run[nt] = M;
        }
      }
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);
    raw_barrier();
  }
}

// MBIG: split-K parts the in-launch merge fetches per round trip (64; 128 in the instantiation for a
// single sequence, whose parts number one per workgroup: a 2048-key call has 65, a 32767-key
// call 256, and each further round trip is ~1 us on the launch's critical path).
template <int NT, int NCH, bool CASCADE_SUFFIX, typename G, bool ROPE = false, bool ALIGN = false, int MBIG = 64>
__global__ __launch_bounds__(256, 1) void decode_lean_kernel(const AttnParams p) {
  static_assert(!ALIGN || (NT == 1 && !CASCADE_SUFFIX), "the aligned split is for decode rows");
  static_assert(MBIG == 64 || (NT == 1 && !CASCADE_SUFFIX && !ALIGN), "wide merges are for one decode sequence");
  constexpr int HD = G::HD;
  constexpr int DPL = HD / 16;
  constexpr int KK = HD / 32;
  constexpr int TOK = G::TOK;
  constexpr bool kQInLds = NT == 1;
  constexpr bool kRope = ROPE && kQInLds;  // rotary of q and the new K rows (rot_cos / rot_sin)
  constexpr int kQCopies = kQInLds ? G::Q_COPIES : 0;
  constexpr int BUF = 2 * rows::TILE_BYTES + (kQInLds ? G::Q_BYTES : 0);  // K tile | V tile | Q
  constexpr int kPolicy = NT == 1 || CASCADE_SUFFIX ? rows::kStreamPolicy : rows::kVerifyPolicy;
  // V^T operands by LDS transpose reads at head_dim 128 (config-5 verify 58.1-58.2 against
  // 60.2-60.3 us per call with byte permutes, 7B decode at B = 8 16.3 against 16.4-16.5)
  constexpr bool kVTr = HD == 128;
  __shared__ __attribute__((aligned(16))) char lds[2 * BUF];

  const int lane = threadIdx.x & 63;
  const int w = threadIdx.x >> 6;
  // The wave's slice of every LDS row.  Spelled w & 3 (w < 4 anyway), this build of the verify
  // kernel keeps 145 scalar spill reloads in its tile loop, against 305 with w: config-5 verify
  // 57.7 against 62.3 us per call, config-3 decode 28.3 against 28.5-29.0.
  const int hw = w & 3;
  const int hg = hw % G::HG;  // KV head within the group
  const int ph = hw / G::HG;  // phase: keys [32 S ph, 32 S (ph + 1)) of every tile
  const bool leader = ph == 0;
  const int li = lane & 15;
  const int lq = lane >> 4;
#ifdef PKV_TILE_STAMPS
  if (threadIdx.x == 0 && int(blockIdx.x) < min(p.lean_grid, kStampWgs)) stamp_now(int(blockIdx.x) * kStampWgWords);
  uint64_t st_tiles = 0, st_mask = 0;  // lane 8 + j: tile j's landing; bit j: iteration j ends a segment
#endif

  SeqTable<NCH> st;
  seq_table<NCH, TOK>(p, st);
  const int T1 = st.total;  // tiles of one head group
  const int total = T1 * p.n_groups;
  const int per = (total + p.lean_grid - 1) / p.lean_grid;
  // an instantiation of its own (the host's choice): its prologue code costs the launches that
  // keep the plain split 0.3-0.4 us
  RangeTable<NCH> rt;
  bool aligned = false;
  if constexpr (ALIGN) {
    range_table<NCH, TOK>(p, st, per, rt);
    aligned = rt.rtotal * p.n_groups <= p.lean_grid;
  }
  if (int(blockIdx.x) >= p.lean_grid) {
    if constexpr (NT == 1) merge_workgroup<G, NCH, MBIG>(p, st, rt, aligned, T1, per, reinterpret_cast<int*>(lds));
    return;
  }
  int s, e;
  if (aligned) {
    aligned_range<NCH, TOK>(p, st, rt, T1, per, int(blockIdx.x), s, e);
  } else {
    s = min(int(blockIdx.x) * per, total);
    e = min(s + per, total);
  }
  if (s >= e) return;
  const int n = e - s;

  // Verify rows (Q in registers) load the first segment's Q ahead of the block-table read, whose
  // wait covers it.  Loaded at the segment start, behind the first two tiles' copies, its wait
  // (vmcnt retires in order) held tile 0's compute until tile 1 had landed as well (config-5
  // verify: tile 1 landed 4.1 us after tile 0, against 1.9 us between later tiles).
  bf16x8 qf[NT][KK];
  if constexpr (!kQInLds) {
    TileDesc d0;  // the range's first tile as tile_window finds it: head group and sequence
    d0.g = s / T1;
    int first0, c0, L0;
    locate_tile(p, st, s - d0.g * T1, d0.b, first0, c0, L0);
    d0.b = __builtin_amdgcn_readfirstlane(min(d0.b, p.batch - 1));
    d0.g = __builtin_amdgcn_readfirstlane(d0.g);
    rows_load_q<HD, NT>(p, d0, d0.g * G::HG + hg, qf);
  }
  TileWin win;
  tile_window<NCH, TOK>(p, st, s, e, T1, win);
  TileDesc dA = tile_desc(win, s);
  TileDesc dB = dA;
  const auto ro = [&] {
    if constexpr (kRope)
      return row_offsets_q<G>(p);
    else
      return row_offsets<G>(p);
  }();
  rows_issue<G, kPolicy, kRope>(p, dA, kQInLds, lds, ro);
  if (n > 1) {
    dB = tile_desc(win, s + 1);
    rows_issue<G, kPolicy, kRope>(p, dB, q_area_copy<G, kRope>(p, dB, kQInLds), lds + BUF, ro);
  }

  uint32_t vto[4];
  if constexpr (kVTr) rows_vt_offsets<G>(hw, vto);
  int lim[NT];
  int lim_min = 0x7fffffff;
  float m_run[NT], l_run[NT];
  f32x4 acc[NT][DPL];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    lim[nt] = kNoQueryRow;
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.f;
#pragma unroll
    for (int k = 0; k < DPL; ++k) acc[nt][k] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  int seg_j0 = 0;  // range index of the current segment's first tile
  int seg_T0 = 0;  // its first token
  int stores_prev = 0, stores_prev2 = 0;  // epilogue stores of iterations j-1 and j-2 (lower bounds)
  int pub_first = -1, pub_last = -1;  // segments (g * batch + b) of the partials in slots 2w, 2w + 1
  // The rare branches of the tile loop (segment start, new rows, segment end, a window refresh)
  // carry expect hints, so the block layout keeps one tile's common path in straight-line code:
  // each workgroup runs only a few dozen tiles, and an instruction-cache miss behind the saturated
  // HBM stream costs about a microsecond (config-5 verify 60.7 us per call with the hints; 62-68 us
  // when an unrelated edit let the new-row copies fall inline ahead of the common path).
  for (int j = 0; j < n; ++j) {
    const TileDesc d = dA;
    char* buf = lds + (j & 1) * BUF;
    // This wave's copies of tile j have landed once at most the operations issued after them are
    // outstanding (vmcnt retires in order): the epilogue stores of iteration j-2 (issued after
    // group j), group j+1 (16 row copies, + the Q copies when Q goes through LDS and tile j+1
    // starts a segment) and the epilogue stores of iteration j-1.  Store counts are lower bounds
    // (the append's stores are left out): the wait is never looser than it must be, and no
    // longer stalls on the next tile after a segment ends.
    if (j + 1 >= n)
      __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
    else
      wait_vmcnt_at_most(16 + (q_area_copy<G, kRope>(p, dB, kQInLds) ? kQCopies : 0) + stores_prev + stores_prev2);
    raw_barrier();  // ... and every other wave's
#ifdef PKV_TILE_STAMPS
    if (j < 24) st_tiles = lane == 8 + j ? __builtin_amdgcn_s_memrealtime() : st_tiles;
#endif
    if (__builtin_expect(j == 0 || d.T0 == p.k0, 0)) {
      // a segment starts: its Q operand, row limits and a fresh softmax state
      if constexpr (kQInLds) {
        if constexpr (kRope) rows_rope_q_area<G>(p, buf);
        rows_read_q<G>(p, buf, hg, qf);
      } else if (j > 0) {
        // a later segment's Q: waited for here, so no wait for loads in flight reaches the
        // products on the loop's common path
        rows_load_q<HD, NT>(p, d, d.g * G::HG + hg, qf);
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
      }
      seg_j0 = j;
      seg_T0 = d.T0;
      lim_min = 0x7fffffff;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int rr = li + 16 * nt;
        lim[nt] = kNoQueryRow;
        if (rr < p.R) {
          const int jr = rr / p.g;
          const int last = p.causal ? (d.L - p.s_q + jr) : (d.L - 1);
          lim[nt] = min(last, d.L - 1);
        }
        lim_min = min_real_limit(lim_min, lim[nt]);
        m_run[nt] = -INFINITY;
        l_run[nt] = 0.f;
#pragma unroll
        for (int k = 0; k < DPL; ++k) acc[nt][k] = f32x4{0.f, 0.f, 0.f, 0.f};
      }
#pragma unroll
      for (int off = 1; off < 16; off <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, off, 64));
      lim_min = __builtin_amdgcn_readfirstlane(lim_min);
    }
    if (__builtin_expect(tile_has_new<TOK>(p, d), 0)) {
      if constexpr (kRope) rows_rope_new_k<G>(p, d, buf);
      rows_append_from_lds<G>(p, d, buf);
    }
    KVTile<HD> tl[G::S];
    if constexpr (kVTr) {
      rows_read_tile_vt<G>(buf, hw, d.T0 + rows::TILE * ph, d.L, vto, tl[0]);
    } else {
#pragma unroll
      for (int sub = 0; sub < G::S; ++sub)
        rows_read_tile<G>(buf, hw, sub, d.T0 + rows::TILE * (ph * G::S + sub), d.L, tl[sub]);
    }
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's LDS reads are done
    raw_barrier();                       // nobody reads this buffer any more
    const bool seg_end = !(j + 1 < n && d.T0 + TOK < d.L);
#ifdef PKV_TILE_STAMPS
    if (seg_end && j < 64) st_mask |= 1ull << j;
#endif
    // With phases, a segment end merges the phase states in this buffer first, and tile j + 2's
    // copies wait until that is done.
    const bool defer = G::P > 1 && seg_end;
    // Verify rows issue tile j + 2's copies in two halves, one before and one after tile j's
    // compute: the wave's copy issue stalls while earlier copies drain, and the split lets that
    // stall overlap the longer compute (config-5 verify 60.3 against 66.7 us per call with every
    // copy first).  Decode rows' compute is short: every row copy goes out first, the Q rows
    // after the compute (7B decode at B = 8 16.9 against 17.3 us, at B = 32 29.2 against
    // 29.3-29.4).
    constexpr int kIssueFirst = NT == 1 ? rows::TILE / 4 : rows::TILE / 8;
    TileDesc d2 = dB;
    const bool next2 = j + 2 < n;
    if (next2) {
      const int x2 = s + j + 2;
      if (__builtin_expect(x2 - win.x0 >= 64, 0)) tile_window<NCH, TOK>(p, st, x2, e, T1, win);
      d2 = tile_desc(win, x2);
      if (!defer) rows_issue<G, kPolicy, kRope>(p, d2, false, buf, ro, 0, kIssueFirst);
    }
    dA = dB;
    dB = d2;
#pragma unroll
    for (int sub = 0; sub < G::S; ++sub) {
      const int T0s = d.T0 + rows::TILE * (ph * G::S + sub);
      if (T0s < d.L) {
        // verify: the prefill kernel's ILP-ordered tile update (all QK products, then the softmax
        // of every N tile, then every PV product)
        if constexpr (NT > 1 && kVTr)
          compute_tile_prefill_vt<NT>(p, tl[sub], T0s, qf, lim, lim_min, m_run, l_run, acc);
        else if constexpr (NT > 1 && HD == 128)
          compute_tile_prefill<NT>(p, tl[sub], T0s, qf, lim, lim_min, m_run, l_run, acc);
        else
          compute_tile<HD, NT, true, kVTr>(p, tl[sub], T0s, qf, lim, lim_min, m_run, l_run, acc);
      }
    }
    if (next2 && !defer)  // the rest, and the Q rows when tile j + 2 starts a segment
      rows_issue<G, kPolicy, kRope>(p, d2, q_area_copy<G, kRope>(p, d2, kQInLds), buf, ro, kIssueFirst, rows::TILE / 4);

    stores_prev2 = stores_prev;
    stores_prev = 0;
    if (__builtin_expect(!seg_end, 1)) continue;  // the segment goes on
    if constexpr (G::P > 1) {
      phase_merge<G, NT>(buf, m_run, l_run, acc);
      if (next2) rows_issue<G, kPolicy, kRope>(p, d2, q_area_copy<G, kRope>(p, d2, kQInLds), buf, ro);
      if (!leader) continue;  // the phase-0 wave of each head holds the merged state
    }
    // ---- segment epilogue: wave (hg, phase 0) owns head hg's rows li + 16 nt < R (per N tile 4
    // stores, or 4 + 1 for a partial; every N tile has a real row) ----
    // a segment holding the sequence's keys [k0, L) complete: its final output, or in a cascade
    // launch its suffix partial (one slot per sequence: a range may hold several)
    const bool complete = seg_T0 == p.k0 && d.T0 + TOK >= d.L;
    const bool whole = complete && !p.cascade_splits;
    stores_prev = (whole ? 4 : 5) * NT;
    float lsum[NT];
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) lsum[nt] = sum_over_quads(l_run[nt]);
    if (whole) {
      // the whole sequence: final output
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int rr = li + 16 * nt;
        if (rr < p.R) {
          const int jr = rr / p.g;
          const int hq = rr - jr * p.g;
          const float inv = lsum[nt] > 0.f ? 1.f / lsum[nt] : 0.f;
          uint16_t* dst =
              p.out + d.b * p.o_sb + jr * p.o_ss + ((d.g * G::HG + hg) * p.g + hq) * p.o_sh + 4 * DPL * lq;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            if constexpr (DPL == 8) {
              u32x4 ov;
#pragma unroll
              for (int k = 0; k < 4; ++k)
                ov[k] = pack_bf16x2(o_elem<kVTr, DPL>(acc[nt], 2 * k, r) * inv,
                                    o_elem<kVTr, DPL>(acc[nt], 2 * k + 1, r) * inv);
              st16(dst + DPL * r, ov);
            } else {
              u32x2 ov;
#pragma unroll
              for (int k = 0; k < 2; ++k) ov[k] = pack_bf16x2(acc[nt][2 * k][r] * inv, acc[nt][2 * k + 1][r] * inv);
              *reinterpret_cast<u32x2*>(dst + DPL * r) = ov;
            }
          }
        }
      }
    } else {
      // part of a sequence shared with a neighbouring range: unnormalised partial (device-
      // coherent stores), merged at the end of the launch by the last range to finish its part,
      // or by the combine launch (two-pass)
      const int slot = complete ? 2 * p.lean_grid + p.batch * p.cascade_splits + d.b
                                : 2 * int(blockIdx.x) + (seg_j0 == 0 ? 0 : 1);
      // the merge below names a segment by g * batch + b
      if (complete)
        ;
      else if (seg_j0 == 0)
        pub_first = d.g * p.batch + d.b;
      else
        pub_last = d.g * p.batch + d.b;
      const uint32_t lse0 = uint32_t(p.ws_ml - p.ws_o) * 4u;
      const __amdgpu_buffer_rsrc_t rs = ws_rsrc(p);
      bool ovf = false;
#pragma unroll
      for (int nt = 0; nt < NT; ++nt) {
        const int rr = li + 16 * nt;
        if (rr < p.R) {
          const uint32_t row = uint32_t((slot * G::HG + hg) * p.R + rr);
          const float inv = lsum[nt] > 0.f ? 1.f / lsum[nt] : 0.f;
          uint32_t ov[4][DPL / 2];
#pragma unroll
          for (int r = 0; r < 4; ++r)
#pragma unroll
            for (int k = 0; k < DPL / 2; ++k) {
              const float lo = o_elem<kVTr, DPL>(acc[nt], 2 * k, r) * inv;
              const float hi = o_elem<kVTr, DPL>(acc[nt], 2 * k + 1, r) * inv;
              ovf |= f16_overflows(lo, hi);
              ov[r][k] = pack_f16x2(lo, hi);
            }
          const float lse = lsum[nt] > 0.f ? m_run[nt] + __builtin_amdgcn_logf(lsum[nt]) : -INFINITY;
          const uint32_t o_off = (row * HD + 4 * DPL * lq) * 2u;
          if (p.two_pass)
            ws_store_partial<0, DPL>(rs, o_off, ov, lq == 0, lse0 + row * 4u, lse);
          else
            ws_store_partial<kCoherent, DPL>(rs, o_off, ov, lq == 0, lse0 + row * 4u, lse);
        }
      }
      if (__any(ovf) && lane == 0) flag_status(p.status, PKV_STATUS_PARTIAL_RANGE);
    }
  }
#ifdef PKV_TILE_STAMPS
  const int st_base = int(blockIdx.x) * kStampWgWords;
  if (int(blockIdx.x) < kStampWgs) {
    if (threadIdx.x == 0) {
      stamp_now(st_base + 1);
      stamp_value(st_base + 3, uint64_t(n));
      stamp_value(st_base + 4, st_mask);
    }
    if (w == 0 && lane >= 8 && lane < 8 + min(n, 24)) stamp_value(st_base + lane, st_tiles);
  }
#endif
  // verify rows (NT > 1: more than 16 rows per KV head) always merge in a second launch
  if (NT > 1 || p.two_pass || (pub_first < 0 && pub_last < 0)) return;
  // In-launch merge: once this wave's partial stores have completed (device-coherent), count
  // its arrival at each (sequence, head) it wrote a part of, on the counter of every row group
  // (lanes [0, n_rq): the first segment's, [4, 4 + n_rq): the last's); a merge workgroup of this
  // launch waits for its count to reach the part count.
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0): the partial stores are device-visible
  {
    const int n_rq = (p.R + 3) / 4;
    const int rq = lane & 3;
    const int pub = lane < 4 ? pub_first : pub_last;
    if (lane < 8 && rq < n_rq && pub >= 0)
      __hip_atomic_fetch_add(merge_counter<G>(p, pub, hg, rq, n_rq), 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
#ifdef PKV_TILE_STAMPS
  if (threadIdx.x == 0 && int(blockIdx.x) < kStampWgs) stamp_now(st_base + 2);
#endif
}

// Two-pass merge (PKV_DECODE_TWO_PASS) of the partials a decode_lean_kernel launch of `grid`
// workgroups left in the workspace.  Workgroup (KV head, sequence, group of 8 query rows), one
// wave per query row (merge_rows; 8-wave workgroups pack three to a CU at its register count,
// where 16-wave ones ran one at a time); only sequences whose tiles span more than one range have
// partials, and in a cascade launch every sequence has the prefix pass's parts as well.
template <typename G>
__global__ __launch_bounds__(512) void combine_lean_kernel(const AttnParams p, int grid, int align) {
  const int hk = blockIdx.x;  // KV head; its group's tiles follow those of the groups before it
  const int g = hk / G::HG;
  const int h = hk - g * G::HG;  // head within the group (the partials hold HG per slot)
  const int b = blockIdx.y;
  const int r = int(blockIdx.z) * 8 + int(threadIdx.x >> 6);  // query row of this wave
  const int lane = threadIdx.x & 63;
  if (r >= p.R) return;

  // first tile and key count of sequence b and the tiles of all sequences: the prefix sum of
  // seq_table (same clamp), one 64-sequence chunk at a time
  const int cap = p.max_blocks << p.log2_page;
  const int s_new = p.has_new ? p.s_q : 0;
  auto tiles_of_lane = [&](int bb, int& Lb) {
    int c = bb < p.batch ? p.seqlens[bb] : 0;
    Lb = c + s_new;
    if (c < 0 || Lb > cap) {
      c = min(max(c, 0), cap);
      Lb = min(c + s_new, cap);
    }
    return bb < p.batch ? seq_tiles<G::TOK>(p, Lb) : 0;
  };
  int first = 0, L = 0, total = 0;
#pragma unroll 1
  for (int q0 = 0; q0 < p.batch; q0 += 64) {
    int Lb;
    const int n = tiles_of_lane(q0 + lane, Lb);
    const int incl = total + wave_incl_scan(n);
    if (b >= q0 && b < q0 + 64) {
      first = __builtin_amdgcn_readlane(incl - n, b - q0);
      L = __builtin_amdgcn_readlane(Lb, b - q0);
    }
    total = __builtin_amdgcn_readlane(incl, 63);
  }
  const int per = (total * p.n_groups + grid - 1) / grid;
  // the split the decode launch chose (range_table, aligned_range): a second pass over the lengths
  // for the aligned split's range counts
  int r0 = 0, rtotal = 0;
#pragma unroll 1
  for (int q0 = 0; q0 < (align ? p.batch : 0); q0 += 64) {
    int Lb;
    const int r = (tiles_of_lane(q0 + lane, Lb) + per - 1) / per;
    const int incl = rtotal + wave_incl_scan(r);
    if (b >= q0 && b < q0 + 64) r0 = __builtin_amdgcn_readlane(incl - r, b - q0);
    rtotal = __builtin_amdgcn_readlane(incl, 63);
  }
  const int t_b = seq_tiles<G::TOK>(p, L);
  int w0, np, slot0;
  if (align && rtotal * p.n_groups <= grid) {
    w0 = g * rtotal + r0;
    np = (t_b + per - 1) / per;
    slot0 = 2 * w0;
  } else {
    first += g * total;
    w0 = first / per;
    np = (first + t_b - 1) / per - w0 + 1;
    // the first range holds b in its first segment only if b starts exactly at the range start
    slot0 = 2 * w0 + (first != w0 * per ? 1 : 0);
  }
  // cascade: the prefix pass's S parts first, then the sequence's suffix partial(s)
  const int S = p.cascade_splits;
  if (np <= 1 && S == 0) return;
  const int n_parts = S + (np <= 1 ? 1 : np);
  const int rr[1] = {r};
  merge_rows<G, false, 1, 32>(p, hk, b, rr, n_parts, [&](int part, int r) -> int64_t {
    int slot;
    if (part < S) {
      slot = 2 * grid + b * S + part;
    } else {
      const int v = part - S;
      slot = np <= 1 ? 2 * grid + p.batch * S + b : (v == 0 ? slot0 : 2 * (w0 + v));
    }
    return (int64_t(slot) * G::HG + h) * p.R + r;
  });
}

// ---------------------------------------------------------------------------------------------
// Prefill: grid (row tile, KV head, sequence).  Each wave owns 16*NT consecutive query rows and
// walks every KV tile its rows can see (causal: up to the wave's last visible key); the W waves
// of a workgroup read the same tiles at about the same time, so the second and later reads hit
// the CU's L1.  No split-K: each wave normalises and writes its own rows.  The new rows were
// appended to the cache by a preceding append launch, so every key is read from the cache.
// ---------------------------------------------------------------------------------------------
template <int HD, int NT, int W>
__global__ __launch_bounds__(64 * W) void prefill_kernel(const AttnParams p) {
  constexpr int DPL = HD / 16;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int lq = lane >> 4;
  int b, h, xblk;
  prefill_item(p, b, h, xblk);

  int c, L;
  seq_lengths(p, b, c, L);
  SeqView sv;
  sv.b = b;
  sv.h = h;
  sv.c = c;
  sv.t_end = L;
  sv.bt = p.block_table + int64_t(b) * p.bt_stride;

  const int row0 = (xblk * W + wave) * 16 * NT;
  if (row0 >= p.R) return;

  bf16x8 qf[NT][HD / 32];
  int lim[NT];
  load_q<HD, NT>(p, sv, L, row0, qf, lim);
  // rows increase with j, so the wave's last row bounds every row's visible range
  const int last_row = min(row0 + 16 * NT, p.R) - 1;
  const int t_stop = p.causal ? min(L, L - p.s_q + last_row / p.g + 1) : L;

  float m_run[NT], l_run[NT];
  f32x4 acc[NT][DPL];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = 0.f;
#pragma unroll
    for (int n = 0; n < DPL; ++n) acc[nt][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  wave_attend<HD, NT, false, kPrefillDepth>(p, sv, qf, lim, 0, t_stop, 32, m_run, l_run, acc);

  // acc[nt][n][r] = O[row li + 16nt][d = DPL*(4lq + r) + n]: the lane owns 4*DPL consecutive
  // head-dim elements of its row, starting at 4*DPL*lq.
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + li + 16 * nt;
    const float lsum = sum_over_quads(l_run[nt]);
    if (row >= p.R) continue;
    const int j = row / p.g;
    const int hq = row - j * p.g;
    const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
    uint16_t* dst = p.out + b * p.o_sb + j * p.o_ss + (h * p.g + hq) * p.o_sh + 4 * DPL * lq;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      if constexpr (DPL == 8) {
        u32x4 ov;
#pragma unroll
        for (int k = 0; k < 4; ++k) ov[k] = pack_bf16x2(acc[nt][2 * k][r] * inv, acc[nt][2 * k + 1][r] * inv);
        st16(dst + DPL * r, ov);
      } else {
        u32x2 ov;
#pragma unroll
        for (int k = 0; k < 2; ++k) ov[k] = pack_bf16x2(acc[nt][2 * k][r] * inv, acc[nt][2 * k + 1][r] * inv);
        *reinterpret_cast<u32x2*>(dst + DPL * r) = ov;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Chunked prefill with LDS-staged KV tiles (head_dim 128, pages of >= 32 rows): grid (row block,
// KV head, sequence).  The W waves of a workgroup own 16*NT consecutive query rows each (row =
// j * g + head-in-group, so a block spans a few query positions of every head of the group) and
// share each 32-token K / V tile of their KV head: the workgroup copies a tile into LDS once
// (16 buffer loads of 1 KiB straight into LDS, 16 / W per wave) into one of NBUF stage buffers,
// and every wave reads its MFMA operands from there (16-byte chunks XOR-swizzled per row: K rows
// by swz as in the decode kernel, V rows by swz_v for the transpose reads).
// The block walks keys up to its last row's last visible key; rows that see fewer keys are masked
// inside the tiles that cross their limit.  No split-K: every wave writes its own rows.
// ---------------------------------------------------------------------------------------------
namespace pf {
constexpr int HD = 128;
constexpr int ROW = HD * 2;            // one KV head's slice of a token row: 256 B
constexpr int TILE = 32;
constexpr int KV_BYTES = TILE * ROW;   // 8 KiB of K (or V) per tile
constexpr int BUF = 2 * KV_BYTES;      // K | V
// 16-byte chunk swizzle of V row r (LDS chunk c holds global chunk c ^ swz_v(r)).  A transpose
// read of V^T operand n touches, in each half wave, token rows 8 q + 4 h + j (j < 4, q one of two
// adjacent values) at global chunks 2 n and 2 n + 1: bits 1..3 of the swizzle take 8 distinct
// values over those rows, so the 8 chunk pairs fall in 8 different bank ranges.
__device__ __forceinline__ int swz_v(int r) { return ((r & 3) << 1) | (((r >> 3) & 1) << 3); }
}  // namespace pf

template <int OPS, int NBUF>
__device__ __forceinline__ void pf_wait(int ahead) {
  // at most `ahead` later tiles' copies (OPS per tile for this wave) may stay in flight
  static_assert(OPS * (NBUF - 1) <= 15, "vmcnt immediate");
  switch (ahead) {
    case 0: __builtin_amdgcn_s_waitcnt(0x0F70); break;
    case 1: __builtin_amdgcn_s_waitcnt(0x0F70 | OPS); break;
    case 2: __builtin_amdgcn_s_waitcnt(0x0F70 | (NBUF > 2 ? 2 * OPS : OPS)); break;
    default: __builtin_amdgcn_s_waitcnt(0x0F70 | (OPS * (NBUF - 1))); break;
  }
}

// Online-softmax update of a wave's 16*NT prefill rows with one 32-token tile, arranged for
// instruction-level parallelism across the N tiles: every S^T product first (NT x 2 independent
// MFMA chains), then the softmax of all tiles with one wave-uniform rescale test, then every PV
// product.  The row max is taken on raw scores (the scale is positive) and the scale is folded
// into the exponent's FMA.  P is rounded to bf16 once (prefill has no MFMA headroom to spare).
// The update itself, on ready operands: kr the tile's K rows (QK^T A operands), vt[n] the V^T
// A operands (lane (i, q): 8 keys 8 q .. 8 q + 7 of one head-dim element per operand; which
// element lane i holds in operand n is the caller's layout, and the accumulator row of that lane
// follows it).
// l_run is either a per-lane partial row sum (float: this lane's keys, summed over the four lanes
// of a row at the end) or the whole row sum kept by the matrix cores (f32x4: P times a ones
// operand, every element the row's sum, of the same bf16 P the PV product uses), which takes the
// 16 additions per tile off the vector ALU for NT extra products.
// S^T products of a tile: NT x 2 independent chains of 4 MFMAs over the head dimension.
template <int NT>
__device__ __forceinline__ void pf_qk(const u32x4 (&kr)[2][4], const bf16x8 (&qf)[NT][4], f32x4 (&s)[NT][2]) {
#pragma unroll
  for (int nt = 0; nt < NT; ++nt)
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      s[nt][a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kk = 0; kk < 4; ++kk)
        s[nt][a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kr[a][kk]), qf[nt][kk],
                                                           s[nt][a], 0, 0, 0);
    }
}

// The rest of the update from the scores s: mask, rescale, P, row sums and PV.  With NEXT, the
// next tile's S^T products (K operands kn, into sn) go out interleaved with this tile's
// exponentials, one MFMA between every few vector instructions: a wave issues in order and its
// next MFMA waits for the matrix pipe, so products placed back to back would hold the softmax
// behind them, while interleaved the two pipes work at once.
// PRIO: the PV products issue at raised wave priority.  With two waves per SIMD (prefill), the
// wave holding its PV products then wins the issue slots over the other wave's exponentials
// whenever the matrix pipe can take a product, so the two waves drift into opposite phases
// instead of queueing for the same pipe (prefill-4096 142.7 -> 132.8 us; verify, at one wave per
// SIMD, 57.7 -> 58.0, so it stays off there).
template <int NT, bool NEXT, bool PRIO = false, typename LT, typename VOps>
__device__ __forceinline__ void pf_softmax_pv(const AttnParams& p, f32x4 (&s)[NT][2], const u32x4 (&kn)[2][4],
                                              f32x4 (&sn)[NT][2], VOps&& v_ops, int T0, const bf16x8 (&qf)[NT][4],
                                              const int (&lim)[NT], int lim_min, float (&m_run)[NT],
                                              LT (&l_run)[NT], f32x4 (&acc)[NT][8]) {
  constexpr bool kLByMfma = std::is_same<LT, f32x4>::value;
  constexpr int DPL = 8;
  const int lane = threadIdx.x & 63;
  const int lq = lane >> 4;
  if (T0 + 31 > lim_min) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int a = 0; a < 2; ++a)
#pragma unroll
        for (int r = 0; r < 4; ++r)
          if (T0 + 8 * lq + 4 * a + r > lim[nt]) s[nt][a][r] = -INFINITY;
  }
  // The rescale test runs on each lane's own 8 scores: scaling by the positive scale_log2 keeps
  // the order, so some lane of a row passes it exactly when the row's maximum does.  Only then is
  // the row maximum taken across the row's four lanes.
  float lmax[NT];
  bool grow_any = false;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    lmax[nt] = max3_raw(max3_raw(s[nt][0][0], s[nt][0][1], s[nt][0][2]),
                        max3_raw(s[nt][0][3], s[nt][1][0], s[nt][1][1]), max_raw(s[nt][1][2], s[nt][1][3]));
    grow_any |= lmax[nt] * p.scale_log2 > m_run[nt] + kRescaleSlack;
  }
  if (__any(grow_any)) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const float mx = max_over_quads(lmax[nt]) * p.scale_log2;
      const float m_new = mx > m_run[nt] + kRescaleSlack ? mx : m_run[nt];
      const float alpha = m_new == -INFINITY ? 1.f : fast_exp2(m_run[nt] - m_new);  // see compute_tile
      l_run[nt] *= alpha;
#pragma unroll
      for (int n = 0; n < DPL; ++n) acc[nt][n] *= alpha;
      m_run[nt] = m_new;
    }
  }
  bf16x8 pb[NT];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const float neg_m = (m_run[nt] == -INFINITY) ? 0.f : -m_run[nt];
    float psum = 0.f;
    u32x4 pk;
#pragma unroll
    for (int e = 0; e < 8; e += 2) {
      const float p0 = fast_exp2(fmaf(s[nt][e >> 2][e & 3], p.scale_log2, neg_m));
      const float p1 = fast_exp2(fmaf(s[nt][e >> 2][(e & 3) + 1], p.scale_log2, neg_m));
      if constexpr (!kLByMfma) psum += p0 + p1;
      pk[e >> 1] = pack_bf16x2(p0, p1);
    }
    if constexpr (!kLByMfma) l_run[nt] += psum;
    pb[nt] = __builtin_bit_cast(bf16x8, pk);
  }
  if constexpr (NEXT) {
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
#pragma unroll
      for (int a = 0; a < 2; ++a) sn[nt][a] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int kk = 0; kk < 4; ++kk)
#pragma unroll
      for (int nt = 0; nt < NT; ++nt)
#pragma unroll
        for (int a = 0; a < 2; ++a)
          sn[nt][a] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, kn[a][kk]), qf[nt][kk],
                                                              sn[nt][a], 0, 0, 0);
#pragma unroll
    for (int i = 0; i < 8 * NT; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, PKV_PREFILL_PIPE_VALU, 0);  // then vector ALU work
    }
  }
  if constexpr (kLByMfma) {
    const u32x4 one2 = {0x3F803F80u, 0x3F803F80u, 0x3F803F80u, 0x3F803F80u};  // bf16 1.0 pairs
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      l_run[nt] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, one2), pb[nt], l_run[nt], 0, 0, 0);
  }
  bf16x8 vt[DPL];
  v_ops(vt);
  if constexpr (PRIO) __builtin_amdgcn_s_setprio(1);
#pragma unroll
  for (int n = 0; n < DPL; ++n)
#pragma unroll
    for (int nt = 0; nt < NT; ++nt)
      acc[nt][n] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(vt[n], pb[nt], acc[nt][n], 0, 0, 0);
  if constexpr (PRIO) __builtin_amdgcn_s_setprio(0);
}

template <int NT, typename LT, typename VIssue, typename VOps>
__device__ __forceinline__ void compute_tile_prefill_ops(const AttnParams& p, const u32x4 (&kr)[2][4],
                                                         VIssue&& v_issue, VOps&& v_ops, int T0,
                                                         const bf16x8 (&qf)[NT][4],
                                                         const int (&lim)[NT], int lim_min, float (&m_run)[NT],
                                                         LT (&l_run)[NT], f32x4 (&acc)[NT][8]) {
  f32x4 s[NT][2];
  pf_qk<NT>(kr, qf, s);
  v_issue();
  f32x4 sn_unused[NT][2];
  pf_softmax_pv<NT, false>(p, s, kr, sn_unused, v_ops, T0, qf, lim, lim_min, m_run, l_run, acc);
}

// The same update on a tile read row-wise (KVTile): V^T operand n of lane (i, q) is head-dim
// element 8 i + n, gathered from the V rows by byte permutes.
template <int NT>
__device__ __forceinline__ void compute_tile_prefill(const AttnParams& p, const KVTile<128>& tl, int T0,
                                                     const bf16x8 (&qf)[NT][4], const int (&lim)[NT], int lim_min,
                                                     float (&m_run)[NT], float (&l_run)[NT], f32x4 (&acc)[NT][8]) {
  auto v_ops = [&](bf16x8 (&vt)[8]) {
#pragma unroll
    for (int n = 0; n < 8; ++n) {
      const int w = n >> 1;
      const uint32_t sel = (n & 1) ? 0x07060302u : 0x05040100u;
      u32x4 pk;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) pk[pp] = __builtin_amdgcn_perm(tl.vr[2 * pp + 1].w[w], tl.vr[2 * pp].w[w], sel);
      vt[n] = __builtin_bit_cast(bf16x8, pk);
    }
  };
  compute_tile_prefill_ops<NT>(p, tl.kr, [] {}, v_ops, T0, qf, lim, lim_min, m_run, l_run, acc);
}

// The same update on a tile whose V^T operands came from transpose reads (rows_read_tile_vt).
template <int NT>
__device__ __forceinline__ void compute_tile_prefill_vt(const AttnParams& p, const KVTile<128>& tl, int T0,
                                                        const bf16x8 (&qf)[NT][4], const int (&lim)[NT], int lim_min,
                                                        float (&m_run)[NT], float (&l_run)[NT],
                                                        f32x4 (&acc)[NT][8]) {
  auto v_ops = [&](bf16x8 (&vt)[8]) {
#pragma unroll
    for (int n = 0; n < 8; ++n)
      vt[n] = __builtin_bit_cast(bf16x8, u32x4{tl.vr[n].w[0], tl.vr[n].w[1], tl.vr[n].w[2], tl.vr[n].w[3]});
  };
  compute_tile_prefill_ops<NT>(p, tl.kr, [] {}, v_ops, T0, qf, lim, lim_min, m_run, l_run, acc);
}

// Input check of a cascade launch, by one wave: sequences b0..b1 must list sequence 0's first
// k0 / P pages (the prefix pass reads only those), and every query row must see all k0 prefix
// keys, which the prefix pass gives it: at least k0 keys before an append; without an append,
// causal row 0 of s_q sees keys [0, c - s_q], so c >= k0 + s_q - 1.  A violation flags
// PKV_STATUS_SHARED_PREFIX; the output of such a sequence is then meaningless, but every access
// stays inside the pool.
__device__ __forceinline__ void cascade_check_sharing(const AttnParams& p, int b0, int b1) {
  if (threadIdx.x >= 64) return;
  const int lane = threadIdx.x & 63;
  const int np = p.k0 >> p.log2_page;
  const int need = p.k0 + (p.has_new || !p.causal ? 0 : p.s_q - 1);
  bool bad = false;
  for (int b = b0; b <= b1 && b < p.batch; ++b) {
    bad |= p.seqlens[b] < need;
    for (int c0 = 0; c0 < np; c0 += 64) {
      const int c = c0 + lane;
      if (c < np) bad |= p.block_table[int64_t(b) * p.bt_stride + c] != p.block_table[c];
    }
  }
  if (__any(bad) && lane == 0) flag_status(p.status, PKV_STATUS_SHARED_PREFIX);
}

// CASCADE: the shared-prefix pass of a cascade launch.  Grid (row blocks of the whole batch's
// query rows, KV heads, key splits); block-table row 0 holds the shared pages; split z covers
// tiles [z chunk, (z + 1) chunk) of the k0 shared keys, which every row sees whole; the result is
// a partial (fp16 O / l and fp32 log-sum-exp) in workspace slot 2 G + b S + z of each row.
template <int NT, int W, int NBUF, int SUB, bool CASCADE = false>
__global__ __launch_bounds__(64 * W) void prefill_lds_kernel(const AttnParams p) {
  constexpr int HD = pf::HD;
  constexpr int DPL = HD / 16;
  constexpr int OPS = 16 / W * SUB;  // copies per wave per stage (SUB tiles of 32 tokens)
  static_assert(16 % W == 0, "waves must split the 16 copies of a tile");
  __shared__ __attribute__((aligned(16))) char lds[NBUF * SUB * pf::BUF];

  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int li = lane & 15;
  const int lq = lane >> 4;
  int b, h, xblk;
  int c, L;
  const int R_all = CASCADE ? p.batch * p.R : p.R;  // query rows of the launch's row space
  int t_first = 0;                                  // first tile of this workgroup's key range
  int n_tiles;
  if constexpr (CASCADE) {
    xblk = blockIdx.x;
    h = blockIdx.y;
    b = 0;
    c = 0;
    L = p.k0;
    const int n_shared = p.k0 / pf::TILE;
    const int chunk = (n_shared + int(gridDim.z) - 1) / int(gridDim.z);
    t_first = int(blockIdx.z) * chunk;
    n_tiles = min(chunk, n_shared - t_first);
  } else {
    prefill_item(p, b, h, xblk);
    seq_lengths(p, b, c, L);
  }
  SeqView sv;
  sv.b = b;
  sv.h = h;
  sv.c = c;
  sv.t_end = L;
  sv.bt = p.block_table + int64_t(b) * p.bt_stride;

  const int blk_row0 = xblk * W * 16 * NT;
  if (blk_row0 >= R_all) return;
  const int row0 = blk_row0 + wave * 16 * NT;
  // the block's last row sees the most keys (rows increase with j)
  const int blk_last = min(blk_row0 + W * 16 * NT, R_all) - 1;
  if constexpr (CASCADE) {
    if (blockIdx.z == 0 && h == 0) cascade_check_sharing(p, blk_row0 / p.R, blk_last / p.R);
    if (n_tiles <= 0) n_tiles = 0;
  } else {
    const int t_stop = p.causal ? min(L, L - p.s_q + blk_last / p.g + 1) : L;
    n_tiles = t_stop > 0 ? (t_stop + pf::TILE - 1) / pf::TILE : 0;
  }
  const int n_stages = (n_tiles + SUB - 1) / SUB;

  bf16x8 qf[NT][HD / 32];
  int lim[NT];
  if constexpr (CASCADE)
    load_q_batch_rows<HD, NT>(p, h, row0, p.k0 - 1, qf, lim);
  else
    load_q<HD, NT>(p, sv, L, row0, qf, lim);
  // Q is in registers before any tile copy goes out: the tile loop's waits then never have to
  // account for it (the copy pipeline's own waits are the explicit pf_wait ones)
  __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0)
  int lim_min = 0x7fffffff;
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) lim_min = min_real_limit(lim_min, lim[nt]);
#pragma unroll
  for (int off = 1; off < 16; off <<= 1) lim_min = min(lim_min, __shfl_xor(lim_min, off, 64));
  lim_min = __builtin_amdgcn_readfirstlane(lim_min);

  BtWindow btw;
  bt_window_load(p, sv, (t_first * pf::TILE) >> p.log2_page, btw);
  const int row_elems = p.n_kv * HD;
  // Stage st holds tiles SUB*st .. SUB*st + SUB-1 (the last stage repeats its last real tile so
  // every stage issues the same number of copies).  Copy instruction i of a tile: K (i < 8) or V
  // rows 4 (i % 8) .. +3, lane l -> row + l / 16, LDS chunk l % 16 <- global chunk (l % 16) ^ swizzle
  // (swz for K rows, swz_v for V rows).
  // The copies are buffer loads: a tile's K and V rows of this head are one buffer each (base and
  // range in scalar registers), and each lane's byte offset inside it is the same for every tile.
  uint32_t voff[16 / W];
#pragma unroll
  for (int k = 0; k < 16 / W; ++k) {
    const int i = wave + k * W;
    const int r = 4 * (i & 7) + (lane >> 4);
    voff[k] = uint32_t(r * row_elems + ((lane & 15) ^ (i < 8 ? rows::swz(r) : pf::swz_v(r))) * 8) * 2u;
  }
  const int tile_bytes = pf::TILE * row_elems * 2;
  auto issue = [&](int st) {
    char* stage = lds + (st % NBUF) * SUB * pf::BUF;
#pragma unroll
    for (int u = 0; u < SUB; ++u) {
      const int T0 = (t_first + min(st * SUB + u, n_tiles - 1)) * pf::TILE;
      const int pid = bt_page(p, sv, T0 >> p.log2_page, btw);
      const bool ok = unsigned(pid) < unsigned(p.num_pages);
      if (!ok && T0 < L && lane == 0) flag_status(p.status, PKV_STATUS_BAD_PAGE);
      const int64_t off = int64_t(ok ? pid : 0) * p.page_stride +
                          int64_t(T0 & ((1 << p.log2_page) - 1)) * row_elems + h * HD;
      char* buf = stage + u * pf::BUF;
#pragma unroll
      for (int k = 0; k < 16 / W; ++k) {
        const int i = wave + k * W;
        const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc(
            uniform_ptr((i < 8 ? p.k_cache : p.v_cache) + off), 0, tile_bytes, 0x00020000);
        __builtin_amdgcn_raw_ptr_buffer_load_lds(rs,
                                                 (rows::lds_void*)(buf + (i >= 8 ? pf::KV_BYTES : 0) + (i & 7) * 1024),
                                                 16, int(voff[k]), 0, 0, 0);
      }
    }
  };
  // NBUF == 2: stage st + 2 is issued into st's buffer once every wave has read it (a second
  // barrier per tile).  NBUF >= 3: stage st + NBUF - 1 is issued into the buffer of stage st - 1
  // right after the tile's first barrier, which every wave passes only after it has consumed
  // stage st - 1: one barrier per tile, and NBUF - 1 stages in flight during the compute.
  constexpr bool kOneBarrier = NBUF >= 3;
  for (int st = 0; st < (kOneBarrier ? NBUF - 1 : NBUF) && st < n_stages; ++st) issue(st);
  // V^T operands come from LDS transpose reads (ds_read_b64_tr_b16): in each 16-lane group, lane
  // 4 j + c names 4 consecutive elements of row j of a 4 x 16 block of 16-bit values and receives
  // column (its index in the group) of that block.  Operand n of lane (li, lq) is head-dim element
  // 16 n + li over keys 8 lq .. 8 lq + 7: two reads, of token rows 8 lq + j and 8 lq + 4 + j (the
  // same swizzle, 4 rows further), each lane naming elements 16 n + 4 c .. + 3.  vtr[n] is that
  // lane's byte offset inside a tile's V rows, the same for every tile.
  uint32_t vtr[8];
  {
    const int t = 8 * lq + (li >> 2);
    const int c = li & 3;
#pragma unroll
    for (int n = 0; n < 8; ++n)
      vtr[n] = uint32_t(t * pf::ROW + (((2 * n + (c >> 1)) ^ pf::swz_v(t)) << 4) + 8 * (c & 1));
  }

  float m_run[NT];
  f32x4 l_run[NT];  // row sums kept by the matrix cores (every element the row's sum)
  f32x4 acc[NT][DPL];
#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    m_run[nt] = -INFINITY;
    l_run[nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int n = 0; n < DPL; ++n) acc[nt][n] = f32x4{0.f, 0.f, 0.f, 0.f};
  }
  // Software pipeline (one tile per stage, NBUF >= 3): tile t's softmax and PV products run with
  // tile t + 1's S^T products interleaved, so every iteration first waits for stage t + 1.  After
  // that wait's barrier no wave reads stage t - 1 any more (its K went into the products of
  // iteration t - 2, its V into those of t - 1), so stage t + NBUF - 1 is issued into its buffer.
  constexpr bool kPipe = kOneBarrier && SUB == 1 && PKV_PREFILL_PIPE;
  if constexpr (kPipe) {
    auto read_k = [&](int t, u32x4 (&kr)[2][4]) {
      const char* buf = lds + (t % NBUF) * pf::BUF;
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const int r = 8 * (li >> 2) + 4 * a + (li & 3);
#pragma unroll
        for (int kk = 0; kk < 4; ++kk)
          kr[a][kk] = *reinterpret_cast<const u32x4*>(buf + r * pf::ROW + (((4 * kk + lq) ^ rows::swz(r)) << 4));
      }
    };
    f32x4 s[NT][2];
    pf_wait<OPS, NBUF>(min(NBUF - 2, n_stages - 1));
    raw_barrier();
    if (row0 < R_all && n_tiles > 0) {
      u32x4 kr[2][4];
      read_k(0, kr);
      pf_qk<NT>(kr, qf, s);
    }
    // tile t's update, with tile t + 1's products when NEXT
    auto step = [&](int t, auto next) {
      constexpr bool NEXT = decltype(next)::value;
      if (row0 >= R_all) return;
      const int T0 = (t_first + t) * pf::TILE;
      const uint32_t vrows = lds_addr(lds + (t % NBUF) * pf::BUF + pf::KV_BYTES);
      u32x2 vlo[8], vhi[8];
      // the V^T reads go out before the next tile's K reads, so the compiler's own wait for
      // those (it does not count these) also covers them
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int n = 0; n < 8; ++n) {
        vlo[n] = lds_read_tr16_issue<0>(vrows + vtr[n]);
        vhi[n] = lds_read_tr16_issue<4 * pf::ROW>(vrows + vtr[n]);
      }
      __builtin_amdgcn_sched_barrier(0);
      auto v_ops = [&](bf16x8 (&vt)[8]) {
        lds_tr_wait(vlo, vhi);
        u32x4 vw[8];
#pragma unroll
        for (int n = 0; n < 8; ++n) vw[n] = u32x4{vlo[n][0], vlo[n][1], vhi[n][0], vhi[n][1]};
        if (T0 + pf::TILE > L) {
          // keys past the sequence: P = 0 must not meet a stale NaN (word w holds keys 2 w, 2 w + 1)
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const int k = T0 + 8 * lq + 2 * w;
            const uint32_t keep = (k < L ? 0x0000FFFFu : 0u) | (k + 1 < L ? 0xFFFF0000u : 0u);
#pragma unroll
            for (int n = 0; n < 8; ++n) vw[n][w] &= keep;
          }
        }
#pragma unroll
        for (int n = 0; n < 8; ++n) vt[n] = __builtin_bit_cast(bf16x8, vw[n]);
      };
      u32x4 kn[2][4];
      f32x4 sn[NT][2];
      if constexpr (NEXT) read_k(t + 1, kn);
      pf_softmax_pv<NT, NEXT, true>(p, s, kn, sn, v_ops, T0, qf, lim, lim_min, m_run, l_run, acc);
      if constexpr (NEXT) {
#pragma unroll
        for (int nt = 0; nt < NT; ++nt)
#pragma unroll
          for (int a = 0; a < 2; ++a) s[nt][a] = sn[nt][a];
      }
    };
    for (int t = 0; t + 1 < n_tiles; ++t) {
      pf_wait<OPS, NBUF>(min(NBUF - 3, n_stages - 2 - t));
      raw_barrier();
      if (t + NBUF - 1 < n_stages) issue(t + NBUF - 1);
      step(t, std::true_type{});
    }
    if (n_tiles > 0) step(n_tiles - 1, std::false_type{});
  } else {
    for (int st = 0; st < n_stages; ++st) {
      if constexpr (kOneBarrier) {
        pf_wait<OPS, NBUF>(min(NBUF - 2, n_stages - 1 - st));
        raw_barrier();
        if (st + NBUF - 1 < n_stages) issue(st + NBUF - 1);
      } else {
        pf_wait<OPS, NBUF>(min(NBUF - 1, n_stages - 1 - st));
        raw_barrier();
      }
  #pragma unroll
      for (int u = 0; u < SUB; ++u) {
        const int t = st * SUB + u;
        if (t >= n_tiles) break;
        const int T0 = (t_first + t) * pf::TILE;
        const char* buf = lds + ((st % NBUF) * SUB + u) * pf::BUF;
        u32x4 kr[2][4];
  #pragma unroll
        for (int a = 0; a < 2; ++a) {
          const int r = 8 * (li >> 2) + 4 * a + (li & 3);
  #pragma unroll
          for (int kk = 0; kk < 4; ++kk)
            kr[a][kk] = *reinterpret_cast<const u32x4*>(buf + r * pf::ROW + (((4 * kk + lq) ^ rows::swz(r)) << 4));
        }
        // the V^T reads go out once the QK products are issued (so the compiler's waits for the K
        // reads, which do not count these, stay exact) and are waited for just before the PV
        // products (lds_tr_wait): their latency hides behind the QK products and the softmax
        const uint32_t vrows = lds_addr(buf + pf::KV_BYTES);
        u32x2 vlo[8], vhi[8];
        auto v_issue = [&] {
          __builtin_amdgcn_sched_barrier(0);
  #pragma unroll
          for (int n = 0; n < 8; ++n) {
            vlo[n] = lds_read_tr16_issue<0>(vrows + vtr[n]);
            vhi[n] = lds_read_tr16_issue<4 * pf::ROW>(vrows + vtr[n]);
          }
        };
        auto v_ops = [&](bf16x8 (&vt)[8]) {
          lds_tr_wait(vlo, vhi);
          u32x4 vw[8];
  #pragma unroll
          for (int n = 0; n < 8; ++n) vw[n] = u32x4{vlo[n][0], vlo[n][1], vhi[n][0], vhi[n][1]};
          if (T0 + pf::TILE > L) {
            // keys past the sequence: P = 0 must not meet a stale NaN (word w holds keys 2 w, 2 w + 1)
  #pragma unroll
            for (int w = 0; w < 4; ++w) {
              const int k = T0 + 8 * lq + 2 * w;
              const uint32_t keep = (k < L ? 0x0000FFFFu : 0u) | (k + 1 < L ? 0xFFFF0000u : 0u);
  #pragma unroll
              for (int n = 0; n < 8; ++n) vw[n][w] &= keep;
            }
          }
  #pragma unroll
          for (int n = 0; n < 8; ++n) vt[n] = __builtin_bit_cast(bf16x8, vw[n]);
        };
        if (row0 < R_all) compute_tile_prefill_ops<NT>(p, kr, v_issue, v_ops, T0, qf, lim, lim_min, m_run, l_run, acc);
      }
      if constexpr (!kOneBarrier) {
        __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the stage are done
        raw_barrier();                       // the stage's buffer is free
        if (st + NBUF < n_stages) issue(st + NBUF);
      }
    }
  }
  if (row0 >= R_all) return;
  if constexpr (CASCADE) {
    // the split's partial of every row: fp16 O / l and the log-sum-exp, as the balanced kernel
    // writes its partials
    const uint32_t lse0 = uint32_t(p.ws_ml - p.ws_o) * 4u;
    const __amdgpu_buffer_rsrc_t rs = ws_rsrc(p);
    bool ovf = false;
#pragma unroll
    for (int nt = 0; nt < NT; ++nt) {
      const int ra = row0 + li + 16 * nt;
      const float lsum = l_run[nt][0];
      if (ra < R_all) {
        const int br = ra / p.R;
        const int rr = ra - br * p.R;
        const int slot = 2 * p.lean_grid + br * p.cascade_splits + int(blockIdx.z);
        const uint32_t row = uint32_t((slot * rows::NKV + h) * p.R + rr);
        const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
        // accumulator n of lane (li, lq) holds head-dim elements 16 n + 4 lq .. + 3
#pragma unroll
        for (int n = 0; n < DPL; ++n) {
          const f32x4 o = acc[nt][n] * inv;
          ovf = ovf || f16_overflows(o[0], o[1]) || f16_overflows(o[2], o[3]);
          const u32x2 ov = {pack_f16x2(o[0], o[1]), pack_f16x2(o[2], o[3])};
          __builtin_amdgcn_raw_buffer_store_b64(ov, rs, int((row * HD + 16 * n + 4 * lq) * 2u), 0, 0);
        }
        const float lse = lsum > 0.f ? m_run[nt] + __builtin_amdgcn_logf(lsum) : -INFINITY;
        if (lq == 0) __builtin_amdgcn_raw_buffer_store_b32(__builtin_bit_cast(uint32_t, lse), rs, int(lse0 + row * 4u), 0, 0);
      }
    }
    if (__any(ovf) && lane == 0) flag_status(p.status, PKV_STATUS_PARTIAL_RANGE);
    return;
  }

#pragma unroll
  for (int nt = 0; nt < NT; ++nt) {
    const int row = row0 + li + 16 * nt;
    const float lsum = l_run[nt][0];
    if (row < p.R) {
      const int j = row / p.g;
      const int hq = row - j * p.g;
      const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
      uint16_t* dst = p.out + b * p.o_sb + j * p.o_ss + (h * p.g + hq) * p.o_sh + 4 * lq;
#pragma unroll
      for (int n = 0; n < DPL; ++n) {
        const u32x2 ov = {pack_bf16x2(acc[nt][n][0] * inv, acc[nt][n][1] * inv),
                          pack_bf16x2(acc[nt][n][2] * inv, acc[nt][n][3] * inv)};
        *reinterpret_cast<u32x2*>(dst + 16 * n) = ov;
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// Host side
// ---------------------------------------------------------------------------------------------
// Default KV range per workgroup of decode_kernel (decode_lean_kernel splits by range instead).
constexpr int kHeadSplitDefault = 512;

static int device_cu_count() {
  static int counts[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (counts[dev] == 0) {
    int n = 0;
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
    counts[dev] = n;
  }
  return counts[dev];
}

static int64_t max_splits_for(int split_tokens, int page_size, int max_blocks) {
  const int64_t cap = int64_t(max_blocks) * page_size;
  const int64_t n = (cap + split_tokens - 1) / split_tokens;
  return n > 0 ? n : 1;
}

static size_t ws_floats_o(int batch, int R, int n_kv, int head_dim, int64_t max_splits) {
  return size_t(batch) * n_kv * size_t(max_splits) * R * head_dim;
}

// Workspace layout: a fixed counter region of kMaxCounters int32 (so that no call's partials
// ever land where another call's counters live) | partial O | (m, l) pairs.
constexpr int kMaxCounters = 16384;
constexpr size_t kCounterBytes = size_t(kMaxCounters) * 4;

static size_t ws_bytes(int batch, int R, int n_kv, int head_dim, int64_t max_splits) {
  const size_t rows = size_t(batch) * n_kv * size_t(max_splits) * R;
  return kCounterBytes + (ws_floats_o(batch, R, n_kv, head_dim, max_splits) + rows * 2) * sizeof(float);
}

// Geometry of the balanced kernel for (head_dim, n_kv): the largest head group of 4, 2 or 1 KV
// heads that divides n_kv (head_dim 128), or of 4 or 2 (head_dim 64); kGeomNone where there is
// none.  Its tile holds tokens_per_tile tokens, which must lie in one page.
enum LeanGeom { kGeomNone, kGeom128x4, kGeom128x2, kGeom128x1, kGeom64x4, kGeom64x2 };
static LeanGeom lean_geom(int head_dim, int n_kv) {
  if (head_dim == 128) return n_kv % 4 == 0 ? kGeom128x4 : n_kv % 2 == 0 ? kGeom128x2 : kGeom128x1;
  if (head_dim == 64) return n_kv % 4 == 0 ? kGeom64x4 : n_kv % 2 == 0 ? kGeom64x2 : kGeomNone;
  return kGeomNone;
}
static int lean_tokens_per_tile(LeanGeom g) {
  switch (g) {
    case kGeom128x4: return Geom<128, 4>::TOK;
    case kGeom128x2: return Geom<128, 2>::TOK;
    case kGeom128x1: return Geom<128, 1>::TOK;
    case kGeom64x4: return Geom<64, 4>::TOK;
    case kGeom64x2: return Geom<64, 2>::TOK;
    default: return 1 << 30;
  }
}

// decode_lean_kernel covers head_dim 128 with any n_kv and head_dim 64 with an even n_kv (pages
// holding whole tiles, <= kLeanMaxRows query rows per KV head, <= 256 sequences) and runs there
// unless the caller fixes split_tokens or asks for decode_kernel (PKV_DECODE_HEADS).
#ifndef PKV_LEAN_MAX_ROWS
#define PKV_LEAN_MAX_ROWS 64
#endif
constexpr int kLeanMaxRows = PKV_LEAN_MAX_ROWS;
static bool use_lean_kernel(int batch, int head_dim, int n_kv, int R, int page_size, int split_tokens,
                            int32_t flags) {
  const LeanGeom g = lean_geom(head_dim, n_kv);
  return g != kGeomNone && R <= kLeanMaxRows && page_size >= lean_tokens_per_tile(g) &&
         batch <= rows::kMaxBatch && int64_t(batch) * n_kv <= kMaxCounters && split_tokens <= 0 &&
         !(flags & PKV_DECODE_HEADS);
}

// Workgroups of a decode_lean_kernel launch: PKV_DECODE_GRID(n) of the flags, else one per CU.
static int lean_grid(int32_t flags) {
  const int g = int((uint32_t(flags) >> 8) & 0xffffu);
  return g > 0 ? g : device_cu_count();
}

// decode_lean_kernel for R query rows per KV head (NT = R / 16 MFMA row tiles, rounded up) and
// a batch of up to 64 or up to 256 sequences (the sequence table's register chunks: a kernel for
// small batches carries a quarter of the scan and search code, which every launch fetches cold).
// The launch's workgroups: `grid` that decode, then (in-launch merge) one per (sequence, KV head,
// group of 4 query rows) that merge.
template <int NT, bool CS, typename G>
static void launch_lean_nt(const AttnParams& p, int batch, int grid, bool align, hipStream_t s) {
  const int wgs = grid + (p.two_pass ? 0 : batch * p.n_kv * ((p.R + 3) / 4));
  if constexpr (NT == 1 && !CS) {
    if (p.rot_cos) {  // a separate kernel: the rotary code costs the plain decode a few tenths of a us
      if (align)
        batch <= 64 ? decode_lean_kernel<NT, 1, CS, G, true, true><<<wgs, 256, 0, s>>>(p)
                    : decode_lean_kernel<NT, rows::kChunks, CS, G, true, true><<<wgs, 256, 0, s>>>(p);
      else
        batch <= 64 ? decode_lean_kernel<NT, 1, CS, G, true><<<wgs, 256, 0, s>>>(p)
                    : decode_lean_kernel<NT, rows::kChunks, CS, G, true><<<wgs, 256, 0, s>>>(p);
      return;
    }
    if (align) {
      batch <= 64 ? decode_lean_kernel<NT, 1, CS, G, false, true><<<wgs, 256, 0, s>>>(p)
                  : decode_lean_kernel<NT, rows::kChunks, CS, G, false, true><<<wgs, 256, 0, s>>>(p);
      return;
    }
    // not for 1 or 2 KV heads of head_dim 128 per group, whose wide-merge instantiation compiles
    // to a tile loop with 5-7x the scalar spills
    if constexpr (!(G::HD == 128 && G::HG < 4)) {
      if (batch == 1 && !p.two_pass) {
        decode_lean_kernel<NT, 1, CS, G, false, false, 128><<<wgs, 256, 0, s>>>(p);
        return;
      }
    }
  }
  if (batch <= 64)
    decode_lean_kernel<NT, 1, CS, G><<<wgs, 256, 0, s>>>(p);
  else
    decode_lean_kernel<NT, rows::kChunks, CS, G><<<wgs, 256, 0, s>>>(p);
}
// The launch (and the two-pass merge's) for geometry G; the suffix pass of a cascade launch
// (cascade_splits > 0) exists for the 7B geometry only.
template <typename G>
static void launch_lean_g(const AttnParams& p, int R, int batch, int grid, bool align, hipStream_t s) {
  const bool cs = p.cascade_splits > 0;
  if constexpr (std::is_same<G, Geom7B>::value) {
    switch ((R + 15) / 16) {
      case 1: launch_lean_nt<1, false, G>(p, batch, grid, align, s); break;
      case 2: cs ? launch_lean_nt<2, true, G>(p, batch, grid, align, s) : launch_lean_nt<2, false, G>(p, batch, grid, align, s); break;
      case 3: cs ? launch_lean_nt<3, true, G>(p, batch, grid, align, s) : launch_lean_nt<3, false, G>(p, batch, grid, align, s); break;
      default: cs ? launch_lean_nt<4, true, G>(p, batch, grid, align, s) : launch_lean_nt<4, false, G>(p, batch, grid, align, s); break;
    }
  } else {
    (void)cs;
    switch ((R + 15) / 16) {
      case 1: launch_lean_nt<1, false, G>(p, batch, grid, align, s); break;
      case 2: launch_lean_nt<2, false, G>(p, batch, grid, align, s); break;
      case 3: launch_lean_nt<3, false, G>(p, batch, grid, align, s); break;
      default: launch_lean_nt<4, false, G>(p, batch, grid, align, s); break;
    }
  }
  if (p.two_pass)
    combine_lean_kernel<G><<<dim3(p.n_kv, batch, (R + 7) / 8), 64 * (R < 8 ? R : 8), 0, s>>>(p, grid, align ? 1 : 0);
}
static void launch_lean(const AttnParams& p, int head_dim, int R, int batch, int grid, bool align, hipStream_t s) {
  switch (lean_geom(head_dim, p.n_kv)) {
    case kGeom128x4: launch_lean_g<Geom<128, 4>>(p, R, batch, grid, align, s); break;
    case kGeom128x2: launch_lean_g<Geom<128, 2>>(p, R, batch, grid, align, s); break;
    case kGeom128x1: launch_lean_g<Geom<128, 1>>(p, R, batch, grid, align, s); break;
    case kGeom64x4: launch_lean_g<Geom<64, 4>>(p, R, batch, grid, align, s); break;
    case kGeom64x2: launch_lean_g<Geom<64, 2>>(p, R, batch, grid, align, s); break;
    default: break;
  }
}

static int lean_heads_per_group(int head_dim, int n_kv) {
  switch (lean_geom(head_dim, n_kv)) {
    case kGeom128x4: case kGeom64x4: return 4;
    case kGeom128x2: case kGeom64x2: return 2;
    default: return 1;
  }
}

// Same counter region | partial O / l [2 grid, HG, R, head_dim] fp16 | log-sum-exp
// [2 grid, HG, R] fp32, sized for the widest geometry (4 heads of head_dim 128 per slot).
constexpr size_t kLeanRowBytes = rows::HD * 2 + sizeof(float);
static size_t ws_bytes_lean(int grid, int R) {
  return kCounterBytes + size_t(2) * grid * rows::NKV * R * kLeanRowBytes;
}
// First log-sum-exp float after `slots` fp16 partial blocks of n_kv x R rows.
static float* lean_lse_base(float* ws_o, size_t slots, int R) {
  return ws_o + slots * rows::NKV * R * rows::HD / 2;
}

static int validate_attn(const char* fn, const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, const void* k_new,
                         int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new, int64_t vn_sb, int64_t vn_ss,
                         int64_t vn_sh, void* k_cache, void* v_cache, int64_t page_stride, const int32_t* block_table,
                         int64_t bt_stride, const int32_t* seqlens, const void* out, int64_t o_sb, int64_t o_ss,
                         int64_t o_sh, int batch, int s_q, int n_heads, int n_kv, int head_dim, int page_size,
                         int num_pages, int max_blocks, float softmax_scale) {
  int rc = validate_paged(fn, k_cache, v_cache, page_stride, block_table, bt_stride, seqlens, batch, n_kv, head_dim,
                          page_size, num_pages, max_blocks);
  if (rc) return rc;
  if (!q || !out) return fail(PKV_EINVAL, "%s: null q/out", fn);
  if (s_q <= 0) return fail(PKV_EINVAL, "%s: s_q %d must be >= 1", fn, s_q);
  if (n_heads <= 0 || n_heads % n_kv)
    return fail(PKV_EINVAL, "%s: n_heads %d not a multiple of n_kv %d", fn, n_heads, n_kv);
  if ((k_new == nullptr) != (v_new == nullptr))
    return fail(PKV_EINVAL, "%s: k_new and v_new must both be given or both be null", fn);
  if ((rc = validate_rows(fn, "q", q, q_sb, q_ss, q_sh))) return rc;
  if ((rc = validate_rows(fn, "out", out, o_sb, o_ss, o_sh))) return rc;
  if (k_new) {
    if ((rc = validate_rows(fn, "k_new", k_new, kn_sb, kn_ss, kn_sh))) return rc;
    if ((rc = validate_rows(fn, "v_new", v_new, vn_sb, vn_ss, vn_sh))) return rc;
  }
  if (!(softmax_scale > 0.f) || !isfinite(softmax_scale)) return fail(PKV_EINVAL, "%s: bad softmax_scale", fn);
  if (batch > 65535 || n_kv > 65535) return fail(PKV_EINVAL, "%s: batch/n_kv exceed the grid limit", fn);
  return PKV_OK;
}

static void fill_params(AttnParams& p, const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, const void* k_new,
                        int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new, int64_t vn_sb, int64_t vn_ss,
                        int64_t vn_sh, void* k_cache, void* v_cache, int64_t page_stride, const int32_t* block_table,
                        int64_t bt_stride, const int32_t* seqlens, void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                        int s_q, int n_heads, int n_kv, int page_size, int num_pages, int max_blocks, int causal,
                        float softmax_scale, int32_t* status) {
  p.q = static_cast<const uint16_t*>(q);
  p.q_sb = q_sb; p.q_ss = q_ss; p.q_sh = q_sh;
  p.k_new = static_cast<const uint16_t*>(k_new);
  p.kn_sb = kn_sb; p.kn_ss = kn_ss; p.kn_sh = kn_sh;
  p.v_new = static_cast<const uint16_t*>(v_new);
  p.vn_sb = vn_sb; p.vn_ss = vn_ss; p.vn_sh = vn_sh;
  p.k_cache = static_cast<uint16_t*>(k_cache);
  p.v_cache = static_cast<uint16_t*>(v_cache);
  p.page_stride = page_stride;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.seqlens = seqlens;
  p.out = static_cast<uint16_t*>(out);
  p.o_sb = o_sb; p.o_ss = o_ss; p.o_sh = o_sh;
  p.ws_o = nullptr;
  p.ws_ml = nullptr;
  p.ws_cnt = nullptr;
  p.status = status;
  p.batch = 0;
  p.s_q = s_q;
  p.g = n_heads / n_kv;
  p.R = s_q * p.g;
  p.n_kv = n_kv;
  p.log2_page = ilog2(page_size);
  p.num_pages = num_pages;
  p.max_blocks = max_blocks;
  p.split_tokens = 1 << 30;
  p.max_splits = 1;
  p.causal = causal ? 1 : 0;
  p.has_new = k_new ? 1 : 0;
  p.two_pass = 0;
  p.lean_grid = 0;
  p.k0 = 0;
  p.cascade_splits = 0;
  p.n_groups = 1;
  p.tok_elems = 0;  // set by the balanced-kernel launches
  p.cnt_stride = 1;
  p.rot_cos = nullptr;
  p.rot_sin = nullptr;
  p.n_pos = 0;
  p.scale_log2 = softmax_scale * 1.4426950408889634f;
}

template <int HD, int NT, int W>
static void launch_decode_t(const AttnParams& p, int batch, hipStream_t stream) {
  // upper bound of the dense item count; items past the real total exit at once
  const int64_t items = int64_t(batch) * p.n_kv * p.max_splits;
  decode_kernel<HD, NT, W><<<dim3(unsigned(items)), 64 * W, 0, stream>>>(p);
  if (p.two_pass && p.max_splits > 1)
    combine_kernel<HD><<<dim3(p.n_kv, batch, (p.R + 15) / 16), 512, 0, stream>>>(p);
}

template <int HD>
static void launch_decode_hd(const AttnParams& p, int batch, hipStream_t stream) {
  switch ((p.R + 15) / 16) {
    case 1: launch_decode_t<HD, 1, PKV_DECODE_W>(p, batch, stream); break;
    case 2: launch_decode_t<HD, 2, 4>(p, batch, stream); break;
    case 3: launch_decode_t<HD, 3, 2>(p, batch, stream); break;
    default: launch_decode_t<HD, 4, 2>(p, batch, stream); break;
  }
}

constexpr int kPrefillNT = 2;
constexpr int kPrefillW = 4;

#ifndef PKV_PREFILL_LDS_NT
#define PKV_PREFILL_LDS_NT 2
#endif
#ifndef PKV_PREFILL_LDS_W
#define PKV_PREFILL_LDS_W 4
#endif
#ifndef PKV_PREFILL_LDS_NBUF
#define PKV_PREFILL_LDS_NBUF 4  // 64 KiB of LDS per workgroup, one barrier per tile
#endif

#ifndef PKV_PREFILL_LDS_SUB
#define PKV_PREFILL_LDS_SUB 1
#endif

static void launch_prefill_lds(const AttnParams& p, int batch, hipStream_t stream) {
  constexpr int NT = PKV_PREFILL_LDS_NT, W = PKV_PREFILL_LDS_W;
  constexpr int rows_per_wg = 16 * NT * W;
  dim3 grid((p.R + rows_per_wg - 1) / rows_per_wg, p.n_kv, batch);
  prefill_lds_kernel<NT, W, PKV_PREFILL_LDS_NBUF, PKV_PREFILL_LDS_SUB><<<grid, 64 * W, 0, stream>>>(p);
}

template <int HD>
static void launch_prefill_hd(const AttnParams& p, int batch, hipStream_t stream) {
  constexpr int rows_per_wg = 16 * kPrefillNT * kPrefillW;
  dim3 grid((p.R + rows_per_wg - 1) / rows_per_wg, p.n_kv, batch);
  prefill_kernel<HD, kPrefillNT, kPrefillW><<<grid, 64 * kPrefillW, 0, stream>>>(p);
}

}  // namespace pkv

extern "C" size_t pkv_decode_workspace_bytes(int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv,
                                             int32_t head_dim, int32_t page_size, int32_t max_blocks,
                                             int32_t split_tokens) {
  using namespace pkv;
  if (batch <= 0 || s_q <= 0 || n_kv <= 0 || n_heads <= 0 || max_blocks <= 0 || page_size <= 0 || head_dim <= 0)
    return 0;
  const int R = s_q * (n_heads / n_kv);
  // enough for either decode kernel the call may run
  const int st = split_tokens > 0 ? split_tokens : kHeadSplitDefault;
  const int64_t ms = max_splits_for(st, page_size, max_blocks);
  size_t need = ms > 1 ? ws_bytes(batch, R, n_kv, head_dim, ms) : 0;
  if (use_lean_kernel(batch, head_dim, n_kv, R, page_size, split_tokens, 0)) {
    const size_t lean = ws_bytes_lean(lean_grid(0), R);
    need = lean > need ? lean : need;
  }
  return need;
}

namespace pkv {

// ---------------------------------------------------------------------------------------------
// Static split-K scratch for pkv_decode_attn_noalloc, the allocation-free variant of
// pkv_decode_attn: the arrival counters and partials live in this file-scope device array (each
// GPU the library runs on holds its own copy, kScratchBytes, until the process exits).  Host code
// never passes the array's name to a kernel or a copy: in host code it is a stand-in, not a
// device address.  Its device address comes from hipGetSymbolAddress, once per device, with that
// device current, and is kept per device.  Every call on a GPU shares that GPU's array, so calls
// that overlap on one GPU (different streams, no ordering between them) race.
// ---------------------------------------------------------------------------------------------
constexpr size_t kScratchBytes = size_t(48) << 20;
static __device__ __align__(256) char scratch[kScratchBytes];
constexpr int kMaxDevices = 64;
static std::mutex g_scratch_mu;
static void* g_scratch[kMaxDevices];

__global__ __launch_bounds__(256) void zero_words_kernel(uint32_t* p, int n) {
  for (int i = int(blockIdx.x) * 256 + int(threadIdx.x); i < n; i += int(gridDim.x) * 256) p[i] = 0u;
}

// Device address of the current device's scratch.  The first call on a device looks it up and
// clears the counter region (a kernel on `stream`, not a memset, so that a first call under HIP
// graph capture records an ordinary kernel node); every decode call leaves the counters at zero
// again, and the partial regions are written before they are read within each call.
static int scratch_for_current_device(const char* fn, hipStream_t stream, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PKV_EHIP, "%s: hipGetDevice failed: %s", fn, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices) return fail(PKV_EINVAL, "%s: device %d beyond %d", fn, dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(PKV_EHIP, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", fn, dev,
                  hipGetErrorString(e));
    zero_words_kernel<<<int(kCounterBytes / 4 / 256), 256, 0, stream>>>(static_cast<uint32_t*>(ptr),
                                                                         int(kCounterBytes / 4));
    const int rc = check_launch(fn);
    if (rc) return rc;
    g_scratch[dev] = ptr;
  }
  *out = g_scratch[dev];
  return PKV_OK;
}

// The body of pkv_decode_attn and pkv_decode_attn_noalloc.  With use_scratch the split-K
// workspace is the static scratch (sizes beyond it are rejected before anything is launched);
// otherwise the caller's.
static int decode_attn(const char* fn, bool use_scratch, const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh,
                       const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new,
                       int64_t vn_sb, int64_t vn_ss, int64_t vn_sh, void* k_cache, void* v_cache,
                       int64_t cache_page_stride, const int32_t* block_table, int64_t bt_stride,
                       const int32_t* cache_seqlens, void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                       void* workspace, size_t workspace_bytes, int32_t batch, int32_t s_q, int32_t n_heads,
                       int32_t n_kv, int32_t head_dim, int32_t page_size, int32_t num_pages, int32_t max_blocks,
                       int32_t causal, float softmax_scale, int32_t split_tokens, int32_t flags, int32_t* status,
                       void* stream, const void* rot_cos = nullptr, const void* rot_sin = nullptr,
                       int32_t n_pos = 0) {
  int rc = validate_attn(fn, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache,
                         v_cache, cache_page_stride, block_table, bt_stride, cache_seqlens, out, o_sb, o_ss, o_sh,
                         batch, s_q, n_heads, n_kv, head_dim, page_size, num_pages, max_blocks, softmax_scale);
  if (rc) return rc;
  const int R = s_q * (n_heads / n_kv);
  if (R > 64) return fail(PKV_EINVAL, "%s: s_q * n_heads / n_kv = %d > 64; use pkv_prefill_attn", fn, R);
  const int32_t merge = flags & (PKV_DECODE_TWO_PASS | PKV_DECODE_FUSED_MERGE);
  if ((flags & ~(PKV_DECODE_TWO_PASS | PKV_DECODE_FUSED_MERGE | PKV_DECODE_HEADS | PKV_DECODE_RESET_COUNTERS |
                 PKV_DECODE_GRID(0xffff))) ||
      merge == (PKV_DECODE_TWO_PASS | PKV_DECODE_FUSED_MERGE))
    return fail(PKV_EINVAL, "%s: bad flags 0x%x", fn, unsigned(flags));
  if (split_tokens < 0 || split_tokens % 32)
    return fail(PKV_EINVAL, "%s: split_tokens %d must be 0 or a positive multiple of 32", fn, split_tokens);
  const bool lean = use_lean_kernel(batch, head_dim, n_kv, R, page_size, split_tokens, flags);
  if (rot_cos || rot_sin) {
    // rotary is applied by the balanced kernel as it stages Q and the new rows: its cos / sin rows
    // share the Q area of 16 rows per KV head with the R query rows (2 rows per new token)
    if (!rot_cos || !rot_sin || n_pos <= 0 || !aligned16(rot_cos) || !aligned16(rot_sin))
      return fail(PKV_EINVAL, "%s: cos / sin tables must be 16-byte aligned [n_pos >= 1, head_dim]", fn);
    if (!k_new) return fail(PKV_EINVAL, "%s: rotary needs the new k / v rows", fn);
    if (!lean || R + 2 * s_q > 16)
      return fail(PKV_EINVAL, "%s: rotary is fused into the balanced decode kernel only (head_dim 128, or 64 with "
                  "an even n_kv; page_size a tile or more; batch <= 256; s_q * n_heads / n_kv + 2 s_q <= 16 = %d; "
                  "no split_tokens or PKV_DECODE_HEADS): rotate with pkv_rope_qk and call pkv_decode_attn",
                  fn, R + 2 * s_q);
  }
  const int st = split_tokens > 0 ? split_tokens : kHeadSplitDefault;
  const int64_t ms = max_splits_for(st, page_size, max_blocks);
  if (ms > 65535) return fail(PKV_EINVAL, "%s: %lld splits exceed the grid limit", fn, (long long)ms);
  if (int64_t(batch) * n_kv * ms > (int64_t(1) << 30))
    return fail(PKV_EINVAL, "%s: %lld work items exceed the grid limit", fn, (long long)(int64_t(batch) * n_kv * ms));
  if (!lean && ms > 1 && int64_t(batch) * n_kv > kMaxCounters)
    return fail(PKV_EINVAL, "%s: batch * n_kv = %lld exceeds %d split-K counters; pass split_tokens >= "
                "max_blocks * page_size", fn, (long long)batch * n_kv, kMaxCounters);
  if (batch == 0) return PKV_OK;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const int grid = lean ? lean_grid(flags) : 0;
  const size_t need = lean ? ws_bytes_lean(grid, R) : (ms > 1 ? ws_bytes(batch, R, n_kv, head_dim, ms) : 0);
  if (lean && need - kCounterBytes >= (size_t(1) << 31))
    return fail(PKV_EINVAL, "%s: %d workgroups need a %zu-byte workspace (partials must stay under 2 GiB)",
                fn, grid, need);
  if (use_scratch && need > 0) {
    if (need > kScratchBytes)
      return fail(PKV_ENOSPC, "%s: this call needs %zu bytes of split-K scratch, more than the library's "
                  "%zu-byte static scratch; call pkv_decode_attn with a workspace", fn, need, kScratchBytes);
    if ((rc = scratch_for_current_device(fn, s, &workspace))) return rc;
    workspace_bytes = kScratchBytes;
  }
  if (need > 0) {
    if (!workspace || workspace_bytes < need)
      return fail(PKV_ENOSPC, "%s: workspace %zu bytes < %zu needed", fn, workspace_bytes, need);
    if (!aligned16(workspace)) return fail(PKV_EINVAL, "%s: workspace not 16-byte aligned", fn);
    if (flags & PKV_DECODE_RESET_COUNTERS) {
      zero_words_kernel<<<int(kCounterBytes / 4 / 256), 256, 0, s>>>(static_cast<uint32_t*>(workspace),
                                                                       int(kCounterBytes / 4));
      if ((rc = check_launch(fn))) return rc;
    }
  }
  if (!use_scratch) {
    // look the noalloc scratch up at the first eager decode call on the device, so that a later
    // pkv_decode_attn_noalloc made under HIP graph capture finds it ready
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(s, &cs) == hipSuccess && cs == hipStreamCaptureStatusNone) {
      void* unused = nullptr;
      if (scratch_for_current_device(fn, s, &unused) != PKV_OK) clear_error();  // the noalloc call reports it
    }
  }

  AttnParams p;
  fill_params(p, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache, v_cache,
              cache_page_stride, block_table, bt_stride, cache_seqlens, out, o_sb, o_ss, o_sh, s_q, n_heads, n_kv,
              page_size, num_pages, max_blocks, causal, softmax_scale, status);
  p.batch = batch;
  p.rot_cos = static_cast<const uint16_t*>(rot_cos);
  p.rot_sin = static_cast<const uint16_t*>(rot_sin);
  p.n_pos = n_pos;
  if (lean) {
    p.ws_cnt = static_cast<int32_t*>(workspace);
    p.ws_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    p.ws_ml = lean_lse_base(p.ws_o, size_t(2) * grid, R);
    // balanced row-streaming kernel; partials merged by a second launch, or inside the launch by
    // merge workgroups appended to the grid (decode rows only: verify's row count would need too
    // many merge workgroups, so it always merges in a second launch).  Without a merge flag the
    // call merges in the launch when its merge workgroups (one per sequence, KV head and 4 query
    // rows) are at most one per CU, one round of the CUs as the decode workgroups leave them: each
    // then starts as soon as a decode workgroup has left its CU and merges without the second
    // launch's dispatch.  Measured per call, in the launch against
    // a second launch (interleaved on one box): 7B at B = 32 28.4-28.9 against 28.9 us, with a
    // 32767-key and a 12000-key sequence in that batch 41.8-42.1 against 45.0-45.2, one 32767-key
    // sequence 25.9 against 32.0, B = 8 16.2 against 17.0, the 0.5B and 7B TP-4 shapes of the
    // B = 32 batch 15.6-15.7 against 16.0 and 18.1 against 19.2.  The 14B shape's 512 merge
    // workgroups take two rounds of the CUs: 44.7-44.9 us with the second launch, 46.9-47.7 in it.
    bool fused = merge == PKV_DECODE_FUSED_MERGE;
    if (merge == 0) fused = int64_t(batch) * n_kv * ((R + 3) / 4) <= grid;
    p.two_pass = fused && R <= 16 ? 0 : 1;
    // the counters 128 bytes apart where the counter region has room
    p.cnt_stride = 1;
    // one arrival counter per (sequence, KV head, group of 4 query rows) for the in-launch merge
    const int64_t n_cnt = int64_t(batch) * n_kv * ((R + 3) / 4);
    if (!p.two_pass && n_cnt > kMaxCounters) p.two_pass = 1;
    while (p.cnt_stride < 32 && n_cnt * p.cnt_stride * 2 <= kMaxCounters) p.cnt_stride *= 2;
    p.lean_grid = grid;
    p.n_groups = n_kv / lean_heads_per_group(head_dim, n_kv);
    // The sequence-aligned split (aligned_range; used where its ranges fit the grid) for decode
    // rows of several sequences where a range crossing a sequence costs most: geometries with
    // phase waves (fewer than 4 KV heads per group: a segment end merges the phases through LDS)
    // and batches of up to 8 (ranges of a few tiles).  Interleaved on one box, per call: 7B at
    // B = 8 14.9 against 16.1 us, 0.5B at B = 32 14.0 against 15.2-15.4, 7B TP-4 15.0 against
    // 17.6; its prologue made 7B at B = 1, 16 and 32 0.3-0.4 us slower.  Not for 4 KV heads of
    // head_dim 64, whose aligned instantiation compiles to a tile loop with 3x the scalar spills.
    const int geom = lean_geom(head_dim, n_kv);
    const bool align = R <= 16 && batch >= 2 && geom != kGeom64x4 &&
                       (lean_heads_per_group(head_dim, n_kv) < 4 || batch <= 8);
    p.tok_elems = n_kv * head_dim;
    // every balanced launch writes split-K partials and counters: never launch one without them
    if (!p.ws_cnt || !p.ws_o || !p.ws_ml) return fail(PKV_EINVAL, "%s: balanced launch without a workspace", fn);
    launch_lean(p, head_dim, R, batch, grid, align, s);
    return check_launch(fn);
  }

  p.split_tokens = st;
  p.max_splits = int(ms);
  p.two_pass = merge == PKV_DECODE_TWO_PASS ? 1 : 0;
  if (ms > 1) {
    p.ws_cnt = static_cast<int32_t*>(workspace);
    p.ws_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
    p.ws_ml = p.ws_o + ws_floats_o(batch, R, n_kv, head_dim, ms);
  }
  if (head_dim == 128)
    launch_decode_hd<128>(p, batch, s);
  else
    launch_decode_hd<64>(p, batch, s);
  return check_launch(fn);
}

}  // namespace pkv

extern "C" int pkv_decode_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, const void* k_new,
                               int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new, int64_t vn_sb,
                               int64_t vn_ss, int64_t vn_sh, void* k_cache, void* v_cache, int64_t cache_page_stride,
                               const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens, void* out,
                               int64_t o_sb, int64_t o_ss, int64_t o_sh, void* workspace, size_t workspace_bytes,
                               int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                               int32_t page_size, int32_t num_pages, int32_t max_blocks, int32_t causal,
                               float softmax_scale, int32_t split_tokens, int32_t flags, int32_t* status,
                               void* stream) {
  pkv::clear_error();
  return pkv::decode_attn("pkv_decode_attn", false, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb,
                          vn_ss, vn_sh, k_cache, v_cache, cache_page_stride, block_table, bt_stride, cache_seqlens,
                          out, o_sb, o_ss, o_sh, workspace, workspace_bytes, batch, s_q, n_heads, n_kv, head_dim,
                          page_size, num_pages, max_blocks, causal, softmax_scale, split_tokens, flags, status,
                          stream);
}

extern "C" int pkv_decode_attn_rope(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, const void* k_new,
                                    int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new, int64_t vn_sb,
                                    int64_t vn_ss, int64_t vn_sh, void* k_cache, void* v_cache,
                                    int64_t cache_page_stride, const int32_t* block_table, int64_t bt_stride,
                                    const int32_t* cache_seqlens, const void* cos_tab, const void* sin_tab,
                                    int32_t n_pos, void* out, int64_t o_sb, int64_t o_ss, int64_t o_sh,
                                    void* workspace, size_t workspace_bytes, int32_t batch, int32_t s_q,
                                    int32_t n_heads, int32_t n_kv, int32_t head_dim, int32_t page_size,
                                    int32_t num_pages, int32_t max_blocks, int32_t causal, float softmax_scale,
                                    int32_t flags, int32_t* status, void* stream) {
  pkv::clear_error();
  return pkv::decode_attn("pkv_decode_attn_rope", false, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new,
                          vn_sb, vn_ss, vn_sh, k_cache, v_cache, cache_page_stride, block_table, bt_stride,
                          cache_seqlens, out, o_sb, o_ss, o_sh, workspace, workspace_bytes, batch, s_q, n_heads,
                          n_kv, head_dim, page_size, num_pages, max_blocks, causal, softmax_scale, 0, flags, status,
                          stream, cos_tab, sin_tab, n_pos);
}

extern "C" int pkv_decode_attn_noalloc(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, const void* k_new,
                                       int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new, int64_t vn_sb,
                                       int64_t vn_ss, int64_t vn_sh, void* k_cache, void* v_cache,
                                       int64_t cache_page_stride, const int32_t* block_table, int64_t bt_stride,
                                       const int32_t* cache_seqlens, void* out, int64_t o_sb, int64_t o_ss,
                                       int64_t o_sh, int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv,
                                       int32_t head_dim, int32_t page_size, int32_t num_pages, int32_t max_blocks,
                                       int32_t causal, float softmax_scale, int32_t split_tokens, int32_t flags,
                                       int32_t* status, void* stream) {
  pkv::clear_error();
  return pkv::decode_attn("pkv_decode_attn_noalloc", true, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new,
                          vn_sb, vn_ss, vn_sh, k_cache, v_cache, cache_page_stride, block_table, bt_stride,
                          cache_seqlens, out, o_sb, o_ss, o_sh, nullptr, 0, batch, s_q, n_heads, n_kv, head_dim,
                          page_size, num_pages, max_blocks, causal, softmax_scale, split_tokens, flags, status,
                          stream);
}

// ---------------------------------------------------------------------------------------------
// Cascade (shared-prefix) attention: the balanced decode shapes with a prefix of shared_tokens
// keys that every sequence of the batch holds in the same pages (speculative verify of branches
// of one prompt, engine/speculative_executor.py:113-164).  The prefix is read once for the whole
// batch instead of once per sequence.
// ---------------------------------------------------------------------------------------------
namespace pkv {

static bool cascade_eligible(int batch, int head_dim, int n_kv, int R, int page_size, int max_blocks,
                             int shared_tokens) {
  return n_kv == rows::NKV && head_dim == rows::HD && use_lean_kernel(batch, head_dim, n_kv, R, page_size, 0, 0) &&
         shared_tokens > 0 &&
         shared_tokens % page_size == 0 && int64_t(shared_tokens) <= int64_t(max_blocks) * page_size;
}

// Key splits of the prefix pass: as many as keep (row blocks of 128 rows x KV heads x splits)
// within one round of two workgroups per CU, at least two 32-token tiles per split.
static int cascade_splits_for(int batch, int R, int shared_tokens) {
  const int n_shared = shared_tokens / rows::TILE;
  const int blocks = ((batch * R + 127) / 128) * rows::NKV;
  const int want = 2 * device_cu_count() / blocks;
  const int cap = n_shared / 2 > 0 ? n_shared / 2 : 1;
  return want < 1 ? 1 : (want > cap ? cap : want);
}

// Counter region | partial O [2 G + B (S + 1) slots, n_kv, R, head_dim] | log-sum-exps, slots
// 0 .. 2G-1 for the balanced ranges, 2G + b S + s for the prefix splits, 2G + B S + b for a
// sequence whose suffix one range holds whole.
static size_t ws_bytes_cascade(int grid, int R, int batch, int S) {
  const size_t slots = size_t(2) * grid + size_t(batch) * (S + 1);
  return kCounterBytes + slots * rows::NKV * R * kLeanRowBytes;
}

}  // namespace pkv

extern "C" size_t pkv_cascade_workspace_bytes(int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv,
                                              int32_t head_dim, int32_t page_size, int32_t max_blocks,
                                              int32_t shared_tokens) {
  using namespace pkv;
  if (batch <= 0 || s_q <= 0 || n_kv <= 0 || n_heads <= 0 || max_blocks <= 0 || page_size <= 0 || head_dim <= 0)
    return 0;
  const int R = s_q * (n_heads / n_kv);
  if (!cascade_eligible(batch, head_dim, n_kv, R, page_size, max_blocks, shared_tokens))
    return pkv_decode_workspace_bytes(batch, s_q, n_heads, n_kv, head_dim, page_size, max_blocks, 0);
  return ws_bytes_cascade(lean_grid(0), R, batch, cascade_splits_for(batch, R, shared_tokens));
}

extern "C" int pkv_cascade_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, const void* k_new,
                                int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new, int64_t vn_sb,
                                int64_t vn_ss, int64_t vn_sh, void* k_cache, void* v_cache, int64_t cache_page_stride,
                                const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens, void* out,
                                int64_t o_sb, int64_t o_ss, int64_t o_sh, void* workspace, size_t workspace_bytes,
                                int32_t batch, int32_t s_q, int32_t n_heads, int32_t n_kv, int32_t head_dim,
                                int32_t page_size, int32_t num_pages, int32_t max_blocks, int32_t shared_tokens,
                                int32_t causal, float softmax_scale, int32_t* status, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_cascade_attn";
  int rc = validate_attn(fn, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache,
                         v_cache, cache_page_stride, block_table, bt_stride, cache_seqlens, out, o_sb, o_ss, o_sh,
                         batch, s_q, n_heads, n_kv, head_dim, page_size, num_pages, max_blocks, softmax_scale);
  if (rc) return rc;
  if (shared_tokens < 0) return fail(PKV_EINVAL, "%s: shared_tokens %d < 0", fn, shared_tokens);
  const int R = s_q * (n_heads / n_kv);
  if (R > 64) return fail(PKV_EINVAL, "%s: s_q * n_heads / n_kv = %d > 64; use pkv_prefill_attn", fn, R);
  if (!cascade_eligible(batch, head_dim, n_kv, R, page_size, max_blocks, shared_tokens))
    return pkv_decode_attn(q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache,
                           v_cache, cache_page_stride, block_table, bt_stride, cache_seqlens, out, o_sb, o_ss, o_sh,
                           workspace, workspace_bytes, batch, s_q, n_heads, n_kv, head_dim, page_size, num_pages,
                           max_blocks, causal, softmax_scale, 0, 0, status, stream);
  if (batch == 0) return PKV_OK;
  const int grid = lean_grid(0);
  const int S = cascade_splits_for(batch, R, shared_tokens);
  const size_t need = ws_bytes_cascade(grid, R, batch, S);
  if (need - kCounterBytes >= (size_t(1) << 31))
    return fail(PKV_EINVAL, "%s: a %zu-byte workspace (partials must stay under 2 GiB)", fn, need);
  if (!workspace || workspace_bytes < need)
    return fail(PKV_ENOSPC, "%s: workspace %zu bytes < %zu needed", fn, workspace_bytes, need);
  if (!aligned16(workspace)) return fail(PKV_EINVAL, "%s: workspace not 16-byte aligned", fn);

  AttnParams p;
  fill_params(p, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache, v_cache,
              cache_page_stride, block_table, bt_stride, cache_seqlens, out, o_sb, o_ss, o_sh, s_q, n_heads, n_kv,
              page_size, num_pages, max_blocks, causal, softmax_scale, status);
  p.batch = batch;
  const size_t slots = size_t(2) * grid + size_t(batch) * (S + 1);
  p.ws_cnt = static_cast<int32_t*>(workspace);
  p.ws_o = reinterpret_cast<float*>(static_cast<char*>(workspace) + kCounterBytes);
  p.ws_ml = lean_lse_base(p.ws_o, slots, R);
  p.two_pass = 1;
  p.lean_grid = grid;
  p.tok_elems = n_kv * head_dim;
  p.k0 = shared_tokens;
  p.cascade_splits = S;
  if (!p.ws_cnt || !p.ws_o || !p.ws_ml) return fail(PKV_EINVAL, "%s: cascade launch without a workspace", fn);
  hipStream_t s = static_cast<hipStream_t>(stream);
  constexpr int NT = PKV_PREFILL_LDS_NT, W = PKV_PREFILL_LDS_W;
  const dim3 pgrid((batch * R + 16 * NT * W - 1) / (16 * NT * W), rows::NKV, S);
  prefill_lds_kernel<NT, W, PKV_PREFILL_LDS_NBUF, PKV_PREFILL_LDS_SUB, true><<<pgrid, 64 * W, 0, s>>>(p);
  launch_lean_g<Geom7B>(p, R, batch, grid, false, s);  // suffix pass + the merge of every part (two_pass)
  return check_launch(fn);
}

extern "C" int pkv_prefill_attn(const void* q, int64_t q_sb, int64_t q_ss, int64_t q_sh, const void* k_new,
                                int64_t kn_sb, int64_t kn_ss, int64_t kn_sh, const void* v_new, int64_t vn_sb,
                                int64_t vn_ss, int64_t vn_sh, void* k_cache, void* v_cache, int64_t cache_page_stride,
                                const int32_t* block_table, int64_t bt_stride, const int32_t* cache_seqlens, void* out,
                                int64_t o_sb, int64_t o_ss, int64_t o_sh, int32_t batch, int32_t s_q, int32_t n_heads,
                                int32_t n_kv, int32_t head_dim, int32_t page_size, int32_t num_pages,
                                int32_t max_blocks, int32_t causal, float softmax_scale, int32_t* status,
                                void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_prefill_attn";
  int rc = validate_attn(fn, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache,
                         v_cache, cache_page_stride, block_table, bt_stride, cache_seqlens, out, o_sb, o_ss, o_sh,
                         batch, s_q, n_heads, n_kv, head_dim, page_size, num_pages, max_blocks, softmax_scale);
  if (rc) return rc;
  const int64_t R = int64_t(s_q) * (n_heads / n_kv);
  if (R > (int64_t(1) << 30)) return fail(PKV_EINVAL, "%s: too many query rows", fn);
  if (batch == 0) return PKV_OK;
  AttnParams p;
  fill_params(p, q, q_sb, q_ss, q_sh, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache, v_cache,
              cache_page_stride, block_table, bt_stride, cache_seqlens, out, o_sb, o_ss, o_sh, s_q, n_heads, n_kv,
              page_size, num_pages, max_blocks, causal, softmax_scale, status);
  hipStream_t s = static_cast<hipStream_t>(stream);
  if (k_new) {
    rc = launch_append(fn, k_new, kn_sb, kn_ss, kn_sh, v_new, vn_sb, vn_ss, vn_sh, k_cache, v_cache,
                       cache_page_stride, block_table, bt_stride, cache_seqlens, batch, s_q, n_kv, head_dim,
                       page_size, num_pages, max_blocks, status, s);
    if (rc) return rc;
  }
  if (head_dim == 128 && page_size >= pf::TILE)
    launch_prefill_lds(p, batch, s);
  else if (head_dim == 128)
    launch_prefill_hd<128>(p, batch, s);
  else
    launch_prefill_hd<64>(p, batch, s);
  return check_launch(fn);
}

#ifdef PKV_TILE_STAMPS
// Stamps variant only (libprism_kv_stamps.so; bench.py --workload tile-stamps): copy the current
// device's stamp words (kStampWords uint64) to host memory `dst` on `stream`, or zero them.  No
// counterpart in the reference: timeline instrumentation of decode_lean_kernel.
extern "C" int pkv_tile_stamps(void* dst, size_t bytes, void* stream) {
  void* ptr = nullptr;
  if (bytes < sizeof(uint64_t) * pkv::kStampWords) return PKV_EINVAL;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(pkv::g_tile_stamps)) != hipSuccess) return PKV_EHIP;
  return hipMemcpyAsync(dst, ptr, sizeof(uint64_t) * pkv::kStampWords, hipMemcpyDeviceToHost,
                        static_cast<hipStream_t>(stream)) == hipSuccess ? PKV_OK : PKV_EHIP;
}
extern "C" int pkv_tile_stamps_clear(void* stream) {
  void* ptr = nullptr;
  if (hipGetSymbolAddress(&ptr, HIP_SYMBOL(pkv::g_tile_stamps)) != hipSuccess) return PKV_EHIP;
  return hipMemsetAsync(ptr, 0, sizeof(uint64_t) * pkv::kStampWords, static_cast<hipStream_t>(stream)) == hipSuccess
             ? PKV_OK
             : PKV_EHIP;
}
extern "C" int pkv_tile_stamp_words(void) { return pkv::kStampWords; }
#endif
