// The per-layer elementwise steps on either side of paged attention in Prism's decoder loop, for
// gfx950: the QKV split with optional per-head RMSNorm (QK-norm) and rotary embedding, fused with
// the paged K/V append; RMSNorm (optionally fused with the residual add before it); SiLU(gate) *
// up.  All are HBM-bound streams: 16-byte loads and stores per lane, fp32 arithmetic, and the
// bf16 rounding points of the reference's torch expressions, so results match it bit for bit
// where the reference's own arithmetic is exact in fp32 (RoPE) and to a bf16 unit otherwise.
//
// Reference: engine/executor.py:45-57 (cos/sin tables), :108-118 and :143-150 (QKV split,
// QK-norm, q * cos + rotate_half(q) * sin), :122-127 (residual adds, RMSNorm, silu(gate) * up);
// engine/fused_kernels.py:8-65 (the Triton RMSNorm and SiLU-mul).
#include <math.h>

#include "pkv_common.h"

namespace pkv {

__device__ __forceinline__ float bf16r(float x) { return bf16_bits_to_f32(f32_to_bf16_bits(x)); }

__device__ __forceinline__ void unpack8(const u32x4 v, float (&f)[8]) {
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    f[2 * k] = bf16_bits_to_f32(v[k] & 0xffffu);
    f[2 * k + 1] = bf16_bits_to_f32(v[k] >> 16);
  }
}

__device__ __forceinline__ u32x4 pack8(const float (&f)[8]) {
  u32x4 v;
#pragma unroll
  for (int k = 0; k < 4; ++k) v[k] = pack_bf16x2(f[2 * k], f[2 * k + 1]);
  return v;
}

// ---------------------------------------------------------------------------------------------
// QKV split + QK-norm + RoPE (+ append).  One workgroup per token.  Work item i of a token:
//   i < (n_heads + n_kv) * hd/16: rotary pair chunk c of head hh (a Q head, then a K head):
//     elements 8c .. 8c+7 and their rotate_half partners hd/2 + 8c .. +7;
//   then (append only) n_kv * hd/8 V chunks copied to the cache.
// The hd/16 pair chunks of a head are consecutive lanes (aligned groups of 8 or 4), which reduce
// the head's sum of squares for QK-norm with lane shuffles.
// ---------------------------------------------------------------------------------------------
struct RopeParams {
  const uint16_t* qkv;
  int64_t qkv_sb, qkv_ss;
  const int32_t* positions;
  const uint16_t* cos_tab;
  const uint16_t* sin_tab;
  int n_pos;
  const uint16_t* q_norm_w;
  const uint16_t* k_norm_w;
  float eps;
  uint16_t* q_out;
  int64_t qo_sb, qo_ss, qo_sh;
  uint16_t* k_out;
  int64_t ko_sb, ko_ss, ko_sh;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t page_stride;
  const int32_t* block_table;
  int64_t bt_stride;
  const int32_t* seqlens;
  int32_t* status;
  int s_new, n_heads, n_kv, head_dim, log2_page, num_pages, max_blocks;
};

// Cache row of token j of sequence b (slot cache_seqlens[b] + j), or -1 (flagged) if unmapped.
__device__ __forceinline__ int64_t cache_row(const RopeParams& p, int b, int j) {
  const int slot = p.seqlens[b] + j;
  const int col = slot >> p.log2_page;
  if (slot < 0 || col >= p.max_blocks) return -1;
  const int pid = p.block_table[int64_t(b) * p.bt_stride + col];
  if (pid < 0 || pid >= p.num_pages) return -1;
  return int64_t(pid) * p.page_stride + int64_t(slot & ((1 << p.log2_page) - 1)) * p.n_kv * p.head_dim;
}

__device__ __forceinline__ void stnt16(void* ptr, u32x4 v) {
  __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(ptr));
}

template <int HD>
__global__ __launch_bounds__(256) void rope_qk_kernel(const RopeParams p) {
  constexpr int PC = HD / 16;  // pair chunks per head
  const int tok = blockIdx.x;
  const int b = tok / p.s_new;
  const int j = tok - b * p.s_new;
  const uint16_t* row = p.qkv + b * p.qkv_sb + j * p.qkv_ss;
  int pos = p.positions[b] + j;
  if (pos < 0 || pos >= p.n_pos) {
    if (threadIdx.x == 0) flag_status(p.status, PKV_STATUS_BAD_POSITION);
    pos = min(max(pos, 0), p.n_pos - 1);
  }
  const bool append = p.k_cache != nullptr;
  int64_t crow = -1;
  if (append) {
    crow = cache_row(p, b, j);
    if (crow < 0 && threadIdx.x == 0) flag_status(p.status, PKV_STATUS_BAD_PAGE);
  }
  const int n_rot = (p.n_heads + p.n_kv) * PC;
  const int n_items = n_rot + (append ? p.n_kv * (HD / 8) : 0);
  for (int i = threadIdx.x; i < n_items; i += blockDim.x) {
    if (i >= n_rot) {
      // V chunk: copied unchanged
      const int v = i - n_rot;
      const int hh = v / (HD / 8);
      const int c8 = v - hh * (HD / 8);
      const u32x4 x = ld16(row + (p.n_heads + p.n_kv + hh) * HD + 8 * c8);
      if (crow >= 0) stnt16(p.v_cache + crow + hh * HD + 8 * c8, x);
      continue;
    }
    const int hh = i / PC;  // Q heads 0 .. n_heads-1, then K heads
    const int c = i - hh * PC;
    const bool is_k = hh >= p.n_heads;
    float x1[8], x2[8];
    unpack8(ld16(row + hh * HD + 8 * c), x1);
    unpack8(ld16(row + hh * HD + HD / 2 + 8 * c), x2);
    const uint16_t* nw = is_k ? p.k_norm_w : p.q_norm_w;
    if (nw) {
      // per-head RMSNorm over head_dim (fp32), rounded to bf16 as the reference's norm output
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += x1[e] * x1[e] + x2[e] * x2[e];
#pragma unroll
      for (int off = 1; off < PC; off <<= 1) ss += __shfl_xor(ss, off, 64);
      const float r = rsqrtf(ss * (1.f / HD) + p.eps);
      float w1[8], w2[8];
      unpack8(ld16(nw + 8 * c), w1);
      unpack8(ld16(nw + HD / 2 + 8 * c), w2);
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        x1[e] = bf16r(x1[e] * r * w1[e]);
        x2[e] = bf16r(x2[e] * r * w2[e]);
      }
    }
    float c1[8], s1[8], c2[8], s2[8];
    const uint16_t* ct = p.cos_tab + int64_t(pos) * HD;
    const uint16_t* st = p.sin_tab + int64_t(pos) * HD;
    unpack8(ld16(ct + 8 * c), c1);
    unpack8(ld16(st + 8 * c), s1);
    unpack8(ld16(ct + HD / 2 + 8 * c), c2);
    unpack8(ld16(st + HD / 2 + 8 * c), s2);
    // out = x * cos + rotate_half(x) * sin with rotate_half(x) = (-x2, x1), each torch bf16 op
    // rounded: bf16(bf16(x * cos) + bf16(rot * sin))
    float o1[8], o2[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      o1[e] = bf16r(bf16r(x1[e] * c1[e]) + bf16r(-x2[e] * s1[e]));
      o2[e] = bf16r(bf16r(x2[e] * c2[e]) + bf16r(x1[e] * s2[e]));
    }
    const u32x4 v1 = pack8(o1), v2 = pack8(o2);
    if (!is_k) {
      uint16_t* dst = p.q_out + b * p.qo_sb + j * p.qo_ss + hh * p.qo_sh;
      stnt16(dst + 8 * c, v1);
      stnt16(dst + HD / 2 + 8 * c, v2);
    } else {
      const int kh = hh - p.n_heads;
      if (p.k_out) {
        uint16_t* dst = p.k_out + b * p.ko_sb + j * p.ko_ss + kh * p.ko_sh;
        stnt16(dst + 8 * c, v1);
        stnt16(dst + HD / 2 + 8 * c, v2);
      }
      if (crow >= 0) {
        stnt16(p.k_cache + crow + kh * HD + 8 * c, v1);
        stnt16(p.k_cache + crow + kh * HD + HD / 2 + 8 * c, v2);
      }
    }
  }
}

// ---------------------------------------------------------------------------------------------
// RMSNorm over rows of `hidden` bf16 values: out = bf16(h * rsqrt(mean(h^2) + eps) * w), with
// h = x, or h = bf16(x + residual) stored to h_out when a residual is given (the reference's
// `hidden = residual + ...` followed by fused_rms_norm).  One 256-thread workgroup per row.
// ---------------------------------------------------------------------------------------------
struct NormParams {
  const uint16_t* x;
  int64_t x_stride;
  const uint16_t* residual;
  int64_t r_stride;
  uint16_t* h_out;
  int64_t h_stride;
  const uint16_t* w;
  uint16_t* out;
  int64_t o_stride;
  int hidden;
  float eps;
};

constexpr int kNormMaxChunks = 4;  // 16-byte chunks per thread: hidden <= 256 * 8 * 4 = 8192

__global__ __launch_bounds__(256) void rms_norm_kernel(const NormParams p) {
  __shared__ float part[4];
  const int r = blockIdx.x;
  const int nch = p.hidden / 8;
  const uint16_t* x = p.x + r * p.x_stride;
  // the weight chunks go out with the row's loads: they are independent of the sum of squares
  u32x4 wv[kNormMaxChunks];
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int c = threadIdx.x + 256 * k;
    if (c < nch) wv[k] = ld16(p.w + 8 * c);
  }
  u32x4 hv[kNormMaxChunks];
  float ss = 0.f;
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int c = threadIdx.x + 256 * k;
    hv[k] = u32x4{0u, 0u, 0u, 0u};
    if (c < nch) {
      u32x4 v = ld16(x + 8 * c);
      if (p.residual) {
        float a[8], bb[8];
        unpack8(v, a);
        unpack8(ld16(p.residual + r * p.r_stride + 8 * c), bb);
#pragma unroll
        for (int e = 0; e < 8; ++e) a[e] = a[e] + bb[e];
        v = pack8(a);
        if (p.h_out) __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p.h_out + r * p.h_stride + 8 * c));
      }
      hv[k] = v;
      float f[8];
      unpack8(v, f);
#pragma unroll
      for (int e = 0; e < 8; ++e) ss += f[e] * f[e];
    }
  }
#pragma unroll
  for (int off = 32; off >= 1; off >>= 1) ss += __shfl_xor(ss, off, 64);
  if ((threadIdx.x & 63) == 0) part[threadIdx.x >> 6] = ss;
  __syncthreads();
  ss = part[0] + part[1] + part[2] + part[3];
  const float rs = rsqrtf(ss / float(p.hidden) + p.eps);
#pragma unroll
  for (int k = 0; k < kNormMaxChunks; ++k) {
    const int c = threadIdx.x + 256 * k;
    if (c < nch) {
      float f[8], w[8];
      unpack8(hv[k], f);
      unpack8(wv[k], w);
#pragma unroll
      for (int e = 0; e < 8; ++e) f[e] = f[e] * rs * w[e];
      __builtin_nontemporal_store(pack8(f), reinterpret_cast<u32x4*>(p.out + r * p.o_stride + 8 * c));
    }
  }
}

// ---------------------------------------------------------------------------------------------
// SiLU(gate) * up over rows of m values: out = bf16(bf16(silu(g)) * u), the two roundings of the
// reference's F.silu(gu[..., :m]) * gu[..., m:] on bf16 tensors.  Grid-stride over 16-byte chunks.
// ---------------------------------------------------------------------------------------------
struct SiluParams {
  const uint16_t* gate;
  int64_t g_stride;
  const uint16_t* up;
  int64_t u_stride;
  uint16_t* out;
  int64_t o_stride;
  int64_t rows;
  int m;
};

__global__ __launch_bounds__(256) void silu_mul_kernel(const SiluParams p) {
  const int cpr = p.m / 8;
  const int64_t total = p.rows * cpr;
  const int64_t stride = int64_t(gridDim.x) * blockDim.x;
  for (int64_t i = int64_t(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += stride) {
    const int64_t r = i / cpr;
    const int c = int(i - r * cpr);
    float gf[8], uf[8], o[8];
    unpack8(ld16(p.gate + r * p.g_stride + 8 * c), gf);
    unpack8(ld16(p.up + r * p.u_stride + 8 * c), uf);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float s = bf16r(gf[e] / (1.f + __expf(-gf[e])));
      o[e] = s * uf[e];
    }
    __builtin_nontemporal_store(pack8(o), reinterpret_cast<u32x4*>(p.out + r * p.o_stride + 8 * c));
  }
}

}  // namespace pkv

extern "C" int pkv_rope_qk(const void* qkv, int64_t qkv_sb, int64_t qkv_ss, const int32_t* positions,
                           const void* cos_tab, const void* sin_tab, int32_t n_pos, const void* q_norm_w,
                           const void* k_norm_w, float eps, void* q_out, int64_t qo_sb, int64_t qo_ss,
                           int64_t qo_sh, void* k_out, int64_t ko_sb, int64_t ko_ss, int64_t ko_sh, void* k_cache,
                           void* v_cache, int64_t cache_page_stride, const int32_t* block_table, int64_t bt_stride,
                           const int32_t* cache_seqlens, int32_t batch, int32_t s_new, int32_t n_heads,
                           int32_t n_kv, int32_t head_dim, int32_t page_size, int32_t num_pages,
                           int32_t max_blocks, int32_t* status, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_rope_qk";
  int rc;
  if (!qkv || !positions || !cos_tab || !sin_tab || !q_out) return fail(PKV_EINVAL, "%s: null argument", fn);
  if (batch < 0 || s_new < 0 || n_heads <= 0 || n_kv <= 0 || n_pos <= 0)
    return fail(PKV_EINVAL, "%s: bad sizes batch=%d s_new=%d n_heads=%d n_kv=%d n_pos=%d", fn, batch, s_new,
                n_heads, n_kv, n_pos);
  if (head_dim != 64 && head_dim != 128) return fail(PKV_EINVAL, "%s: head_dim %d unsupported (64 or 128)", fn, head_dim);
  if (!aligned16(qkv) || (qkv_sb % 8) || (qkv_ss % 8))
    return fail(PKV_EINVAL, "%s: qkv rows must be 16-byte aligned", fn);
  if (!aligned16(cos_tab) || !aligned16(sin_tab)) return fail(PKV_EINVAL, "%s: cos/sin tables not 16-byte aligned", fn);
  if ((q_norm_w && !aligned16(q_norm_w)) || (k_norm_w && !aligned16(k_norm_w)))
    return fail(PKV_EINVAL, "%s: norm weights not 16-byte aligned", fn);
  if (!(eps >= 0.f)) return fail(PKV_EINVAL, "%s: eps must be >= 0", fn);
  if ((rc = validate_rows(fn, "q_out", q_out, qo_sb, qo_ss, qo_sh))) return rc;
  if (k_out && (rc = validate_rows(fn, "k_out", k_out, ko_sb, ko_ss, ko_sh))) return rc;
  if ((k_cache == nullptr) != (v_cache == nullptr))
    return fail(PKV_EINVAL, "%s: k_cache and v_cache must both be given or both be null", fn);
  if (k_cache && (rc = validate_paged(fn, k_cache, v_cache, cache_page_stride, block_table, bt_stride,
                                      cache_seqlens, batch, n_kv, head_dim, page_size, num_pages, max_blocks)))
    return rc;
  if (int64_t(batch) * s_new > 0x7fffffff) return fail(PKV_EINVAL, "%s: too many tokens", fn);
  if (int64_t(batch) * s_new == 0) return PKV_OK;
  RopeParams p;
  p.qkv = static_cast<const uint16_t*>(qkv);
  p.qkv_sb = qkv_sb;
  p.qkv_ss = qkv_ss;
  p.positions = positions;
  p.cos_tab = static_cast<const uint16_t*>(cos_tab);
  p.sin_tab = static_cast<const uint16_t*>(sin_tab);
  p.n_pos = n_pos;
  p.q_norm_w = static_cast<const uint16_t*>(q_norm_w);
  p.k_norm_w = static_cast<const uint16_t*>(k_norm_w);
  p.eps = eps;
  p.q_out = static_cast<uint16_t*>(q_out);
  p.qo_sb = qo_sb; p.qo_ss = qo_ss; p.qo_sh = qo_sh;
  p.k_out = static_cast<uint16_t*>(k_out);
  p.ko_sb = ko_sb; p.ko_ss = ko_ss; p.ko_sh = ko_sh;
  p.k_cache = static_cast<uint16_t*>(k_cache);
  p.v_cache = static_cast<uint16_t*>(v_cache);
  p.page_stride = cache_page_stride;
  p.block_table = block_table;
  p.bt_stride = bt_stride;
  p.seqlens = cache_seqlens;
  p.status = status;
  p.s_new = s_new;
  p.n_heads = n_heads;
  p.n_kv = n_kv;
  p.head_dim = head_dim;
  p.log2_page = k_cache ? ilog2(page_size) : 0;
  p.num_pages = num_pages;
  p.max_blocks = max_blocks;
  hipStream_t s = static_cast<hipStream_t>(stream);
  const unsigned grid = unsigned(int64_t(batch) * s_new);
  if (head_dim == 128)
    rope_qk_kernel<128><<<grid, 256, 0, s>>>(p);
  else
    rope_qk_kernel<64><<<grid, 256, 0, s>>>(p);
  return check_launch(fn);
}

extern "C" int pkv_rms_norm(const void* x, int64_t x_stride, const void* residual, int64_t r_stride, void* h_out,
                            int64_t h_stride, const void* weight, void* out, int64_t o_stride, int64_t rows,
                            int32_t hidden, float eps, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_rms_norm";
  if (!x || !weight || !out) return fail(PKV_EINVAL, "%s: null argument", fn);
  if (rows < 0 || rows > 0x7fffffff) return fail(PKV_EINVAL, "%s: bad row count %lld", fn, (long long)rows);
  if (hidden <= 0 || hidden % 8 || hidden > 256 * 8 * kNormMaxChunks)
    return fail(PKV_EINVAL, "%s: hidden %d must be a multiple of 8 up to %d", fn, hidden, 256 * 8 * kNormMaxChunks);
  if (!(eps >= 0.f)) return fail(PKV_EINVAL, "%s: eps must be >= 0", fn);
  const bool ok = aligned16(x) && aligned16(weight) && aligned16(out) && !(x_stride % 8) && !(o_stride % 8) &&
                  (!residual || (aligned16(residual) && !(r_stride % 8))) &&
                  (!h_out || (aligned16(h_out) && !(h_stride % 8)));
  if (!ok) return fail(PKV_EINVAL, "%s: rows must be 16-byte aligned", fn);
  if (h_out && !residual) return fail(PKV_EINVAL, "%s: h_out needs a residual", fn);
  if (rows == 0) return PKV_OK;
  NormParams p;
  p.x = static_cast<const uint16_t*>(x);
  p.x_stride = x_stride;
  p.residual = static_cast<const uint16_t*>(residual);
  p.r_stride = r_stride;
  p.h_out = static_cast<uint16_t*>(h_out);
  p.h_stride = h_stride;
  p.w = static_cast<const uint16_t*>(weight);
  p.out = static_cast<uint16_t*>(out);
  p.o_stride = o_stride;
  p.hidden = hidden;
  p.eps = eps;
  rms_norm_kernel<<<unsigned(rows), 256, 0, static_cast<hipStream_t>(stream)>>>(p);
  return check_launch(fn);
}

extern "C" int pkv_silu_mul(const void* gate, int64_t g_stride, const void* up, int64_t u_stride, void* out,
                            int64_t o_stride, int64_t rows, int32_t m, void* stream) {
  using namespace pkv;
  clear_error();
  const char* fn = "pkv_silu_mul";
  if (!gate || !up || !out) return fail(PKV_EINVAL, "%s: null argument", fn);
  if (rows < 0 || m <= 0 || m % 8) return fail(PKV_EINVAL, "%s: bad sizes rows=%lld m=%d", fn, (long long)rows, m);
  if (!aligned16(gate) || !aligned16(up) || !aligned16(out) || (g_stride % 8) || (u_stride % 8) || (o_stride % 8))
    return fail(PKV_EINVAL, "%s: rows must be 16-byte aligned", fn);
  const int64_t total = rows * (m / 8);
  if (total == 0) return PKV_OK;
  SiluParams p;
  p.gate = static_cast<const uint16_t*>(gate);
  p.g_stride = g_stride;
  p.up = static_cast<const uint16_t*>(up);
  p.u_stride = u_stride;
  p.out = static_cast<uint16_t*>(out);
  p.o_stride = o_stride;
  p.rows = rows;
  p.m = m;
  const int64_t want = (total + 255) / 256;
  const int blocks = int(want < 16384 ? want : 16384);
  silu_mul_kernel<<<blocks, 256, 0, static_cast<hipStream_t>(stream)>>>(p);
  return check_launch(fn);
}
