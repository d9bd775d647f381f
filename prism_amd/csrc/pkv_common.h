// Shared definitions for the gfx950 paged KV-cache kernels and their host launchers.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/prism_kv.h"

namespace pkv {

// ---------------------------------------------------------------------------------------------
// Host side: error reporting (thread-local message, negative return codes).
// ---------------------------------------------------------------------------------------------
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();
// Returns PKV_OK, or PKV_EHIP with the launch error recorded, after a kernel launch.
int check_launch(const char* what);

// Host validation / launch helpers shared between translation units (pkv_append.hip).
int validate_paged(const char* fn, const void* k_cache, const void* v_cache, int64_t page_stride,
                   const int32_t* block_table, int64_t bt_stride, const int32_t* seqlens, int batch,
                   int n_kv, int head_dim, int page_size, int num_pages, int max_blocks);
int validate_rows(const char* fn, const char* name, const void* ptr, int64_t sb, int64_t ss, int64_t sh);
int launch_append(const char* fn, const void* k_new, int64_t kn_sb, int64_t kn_ss, int64_t kn_sh,
                  const void* v_new, int64_t vn_sb, int64_t vn_ss, int64_t vn_sh, void* k_cache,
                  void* v_cache, int64_t page_stride, const int32_t* block_table, int64_t bt_stride,
                  const int32_t* seqlens, int batch, int s_new, int n_kv, int head_dim, int page_size,
                  int num_pages, int max_blocks, int32_t* status, hipStream_t stream);

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }
inline bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }
inline int ilog2(int64_t x) {
  int r = 0;
  while ((int64_t(1) << r) < x) ++r;
  return r;
}

// ---------------------------------------------------------------------------------------------
// Device side: vector types and bf16 helpers.
// ---------------------------------------------------------------------------------------------
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

__device__ __forceinline__ float bf16_bits_to_f32(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even (the rounding torch uses for .to(torch.bfloat16)).
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  __bf16 h = static_cast<__bf16>(f);
  return static_cast<uint32_t>(__builtin_bit_cast(uint16_t, h));
}

typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));

// Two fp32 -> one packed bf16 pair (RNE), a single v_cvt_pk_bf16_f32 on gfx950.
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
  const bf16x2 v = __builtin_convertvector(f32x2{lo, hi}, bf16x2);
  return __builtin_bit_cast(uint32_t, v);
}

// 16-byte global load / store of a row chunk.
__device__ __forceinline__ u32x4 ld16(const void* p) { return *reinterpret_cast<const u32x4*>(p); }
__device__ __forceinline__ void st16(void* p, u32x4 v) { *reinterpret_cast<u32x4*>(p) = v; }
__device__ __forceinline__ u32x2 ld8(const void* p) { return *reinterpret_cast<const u32x2*>(p); }

__device__ __forceinline__ void flag_status(int32_t* status, int32_t bit) {
  if (status) atomicOr(status, bit);
}

}  // namespace pkv
