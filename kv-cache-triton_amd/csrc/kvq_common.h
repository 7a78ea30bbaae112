// Shared definitions for the gfx950 INT4 KV kernels: dtype codes, scalar
// load/store with round-to-nearest-even narrowing, and the thread-local error
// slot behind kvq_last_error().
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "../../include/kvint4.h"

namespace kvq {

// bf16 <-> fp32. Widening is exact (bf16 is the top half of an fp32 word).
// Narrowing rounds to nearest, ties to even, like torch's Tensor.to(bfloat16);
// NaN stays a quiet NaN.
__device__ __forceinline__ float bf16_bits_to_f32(uint32_t h) {
  return __builtin_bit_cast(float, h << 16);
}
__device__ __forceinline__ uint32_t f32_to_bf16_bits(float f) {
  uint32_t u = __builtin_bit_cast(uint32_t, f);
  if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
  u += 0x7fffu + ((u >> 16) & 1u);
  return u >> 16;
}
__device__ __forceinline__ float f16_bits_to_f32(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}
__device__ __forceinline__ uint32_t f32_to_f16_bits(float f) {
  return __builtin_bit_cast(uint16_t, (_Float16)f);
}

// The group scale absmax / 7 as the IEEE (correctly rounded) fp32 quotient,
// or 1 for an all-zero group (the reference's rule,
// kernels/llama3/quantize.py:137-141), without a division: q = am * RN(1/7)
// corrected once with an fma, q1 = q + (am - 7 q) * RN(1/7). q1 equals the
// quotient bit for bit for every non-negative finite am (checked exhaustively
// by oracle/kvq_ref.c kvq_ref_check_div7, a CPU test). An infinite absmax
// keeps q (infinity, like the division); NaN yields 1, as the comparison
// with zero does in the reference.
__device__ __forceinline__ float group_scale(float am) {
  constexpr float kInv7 = 1.0f / 7.0f;
  const float q = am * kInv7;
  const float q1 = __builtin_fmaf(__builtin_fmaf(-q, 7.0f, am), kInv7, q);
  const float s = q1 == q1 ? q1 : q;
  return am > 0.0f ? s : 1.0f;
}

// rint(x / s) where x / s is the IEEE (correctly rounded) fp32 quotient, for
// |x| <= 7 s (x an element of the group whose absmax / 7 is s, s a moderate
// normal number): with inv = v_rcp_f32(s), within 1 ulp of 1 / s (relative
// 2^-23; the instruction's documented accuracy), t = RN(x * inv) differs from
// x / s by a relative 2^-23 + 2^-24 and from the rounded quotient by at most
// 7 (2^-23 + 2^-24 + 2^-24) = 7 * 2^-22 ~ 2^-19.2 on |x / s| <= 7, so rint(t)
// is rint of the quotient unless t lies within that distance of a
// half-integer. Such elements (and groups whose scale is not in [2^-100,
// 2^100]) take the division itself. The threshold used, 2^-17, leaves a
// margin of 4.6x (3x for an inverse off by 2 ulp). oracle/kvq_ref.c
// kvqref_check_rint_margin samples scales and elements (random, and a few
// ulps from every tie) with inverses up to 8 ulps off and finds no element
// rounded differently outside the margin; with 2^-20 at 1 ulp it does.
__device__ __forceinline__ float group_inverse(float s) { return __builtin_amdgcn_rcpf(s); }
__device__ __forceinline__ bool near_half(float t, float r) { return fabsf(t - r) > 0.5f - 0x1p-17f; }
__device__ __forceinline__ float rint_quotient(float x, float s, float inv, bool fast) {
  const float t = x * inv;
  const float r = __builtin_rintf(t);
  if (fast && !near_half(t, r)) return r;
  return __builtin_rintf(x / s);
}

// Load element i of a tensor of dtype `dt` as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dt) {
  if (dt == KVQ_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  if (dt == KVQ_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  return ((const float*)p)[i];
}

// load_as_f32 of N elements, with one dtype branch around all N loads so
// that they are in flight together.
template <int N>
__device__ __forceinline__ void load_n_as_f32(const void* p, const int64_t* i, int dt, float* out) {
  if (dt == KVQ_F32) {
#pragma unroll
    for (int k = 0; k < N; ++k) out[k] = ((const float*)p)[i[k]];
    return;
  }
  uint32_t raw[N];
#pragma unroll
  for (int k = 0; k < N; ++k) raw[k] = ((const uint16_t*)p)[i[k]];
#pragma unroll
  for (int k = 0; k < N; ++k) out[k] = dt == KVQ_BF16 ? bf16_bits_to_f32(raw[k]) : f16_bits_to_f32(raw[k]);
}

// Store fp32 `v` into element i of a tensor of dtype `dt` (RNE narrowing).
__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dt, float v) {
  if (dt == KVQ_BF16) ((uint16_t*)p)[i] = (uint16_t)f32_to_bf16_bits(v);
  else if (dt == KVQ_F16) ((uint16_t*)p)[i] = (uint16_t)f32_to_f16_bits(v);
  else ((float*)p)[i] = v;
}

// Paged cache rows. A pool holds num_blocks blocks of 2^page_shift rows per
// head; sequence b's token t lives in pool row
//   table[b * tab_stride + (t >> page_shift)] << page_shift | (t & (page_size - 1)).
// paged == 0 means the contiguous [B, H, S] layout. A table entry that is
// negative or >= n_blocks, or a page index >= n_pages, has no row (-1); the
// table is read only where n_pages > 0 (a table with no columns may be null).
struct PageMap {
  int paged;
  const int32_t* table;
  int64_t tab_stride;  // int32 entries between sequences' table rows
  int64_t n_pages;     // entries of a table row in use
  int64_t n_blocks;    // blocks in the pool
  int page_shift;
};

__device__ __forceinline__ int64_t page_row(const PageMap& m, int64_t b, int64_t t) {
  const int64_t p = t >> m.page_shift;
  if (t < 0 || p >= m.n_pages) return -1;
  const int64_t blk = m.table[b * m.tab_stride + p];
  if (blk < 0 || blk >= m.n_blocks) return -1;
  return (blk << m.page_shift) | (t & ((int64_t(1) << m.page_shift) - 1));
}

// page_row of N positions (sequence b[k], token t[k]) at once, with every
// table read in flight together: each read is taken from an in-range entry
// (column 0 for a position off the table) and the result selected after, so
// no read waits inside a per-position branch. Contiguous layout: t itself.
template <int N>
__device__ __forceinline__ void page_rows(const PageMap& m, const uint32_t* b, const int64_t* t,
                                          int64_t* out) {
  if (!m.paged) {
#pragma unroll
    for (int k = 0; k < N; ++k) out[k] = t[k];
    return;
  }
  int64_t blk[N];
  if (m.n_pages > 0) {
#pragma unroll
    for (int k = 0; k < N; ++k) {
      const int64_t p = t[k] >> m.page_shift;
      const bool on = t[k] >= 0 && p < m.n_pages;
      blk[k] = m.table[(int64_t)b[k] * m.tab_stride + (on ? p : 0)];
    }
  } else {
#pragma unroll
    for (int k = 0; k < N; ++k) blk[k] = -1;
  }
#pragma unroll
  for (int k = 0; k < N; ++k) {
    const int64_t p = t[k] >> m.page_shift;
    const bool ok = t[k] >= 0 && p < m.n_pages && blk[k] >= 0 && blk[k] < m.n_blocks;
    out[k] = ok ? (blk[k] << m.page_shift) | (t[k] & ((int64_t(1) << m.page_shift) - 1)) : -1;
  }
}

// Division by a divisor 1 <= d < 2^32 fixed at launch, for dividends
// n < 2^32, without a divide instruction: q = (mulhi(n, m) + n) >> s with
// s = ceil(log2 d) and m = floor(2^32 (2^s - d) / d) + 1 < 2^32, i.e.
// q = floor(n (2^32 + m) / 2^(32 + s)) (Granlund and Montgomery, "Division by
// invariant integers using multiplication", PLDI 1994, section 4; the sum is
// formed in 64 bits, so it cannot overflow). A runtime divide compiles to ~25
// dependent scalar and vector instructions (reciprocal, conversions,
// corrections); this is four scalar ones.
struct FastDiv {
  uint32_t d, m, s;
};

inline FastDiv make_fastdiv(uint32_t d) {
  uint32_t s = 0;
  while ((uint64_t(1) << s) < d) ++s;
  const uint64_t m = ((uint64_t(1) << 32) * ((uint64_t(1) << s) - d)) / d + 1;
  return FastDiv{d, (uint32_t)m, s};
}

__device__ __forceinline__ uint32_t fdiv(uint32_t n, const FastDiv& f) {
  return (uint32_t)(((uint64_t)__umulhi(n, f.m) + n) >> f.s);
}

inline int dtype_size(int dt) { return dt == KVQ_F32 ? 4 : 2; }
inline bool dtype_ok(int dt) { return dt == KVQ_BF16 || dt == KVQ_F16 || dt == KVQ_F32; }

// Thread-local error message (host side).
void set_error(const char* fmt, ...);
void clear_error();

}  // namespace kvq

#define KVQ_CHECK_ARG(cond, ...)          \
  do {                                    \
    if (!(cond)) {                        \
      ::kvq::set_error(__VA_ARGS__);      \
      return KVQ_EINVAL;                  \
    }                                     \
  } while (0)

#define KVQ_CHECK_LAUNCH(what)                                                   \
  do {                                                                           \
    hipError_t e_ = hipGetLastError();                                           \
    if (e_ != hipSuccess) {                                                      \
      ::kvq::set_error("%s: kernel launch failed: %s", what, hipGetErrorString(e_)); \
      return KVQ_EHIP;                                                           \
    }                                                                            \
  } while (0)
