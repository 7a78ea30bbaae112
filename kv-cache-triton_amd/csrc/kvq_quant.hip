// INT4 group quantize/pack (written in place into a cache slot) and dequantize.
//
// Semantics follow the reference's CPU path exactly:
//   quantize:   kernels/llama3/quantize.py:126-148 (_quantize_int4_torch)
//               kernels/gpt2/quantize.py:111-133 (same codes, fp16 scales)
//   dequantize: kernels/llama3/quantize.py:210-234, kernels/gpt2/quantize.py:217-235
// i.e. scale = max|x_g| / 7 in fp32 (1 for an all-zero group), code =
// round_half_even(x / scale) (IEEE fp32 division) clamped to [-8, 7] plus 8,
// element 2i -> low nibble of byte i, element 2i+1 -> high nibble, zero padding
// of the last group when G does not divide D, and for odd G one zero nibble
// closing each group. Dequant = (nibble - 8) * fp32(scale), narrowed once.
//
// One thread owns one (row, group): the group's absmax is a private loop, so
// no cross-lane reduction is needed, and consecutive threads own consecutive
// groups of the same row, which keeps the global accesses of a wave dense.

#include <algorithm>
#include <limits>

#include "kvq_common.h"

namespace kvq {

struct QuantArgs {
  const void* x;
  int64_t xs_b, xs_h, xs_s, xs_d;   // element strides of x
  int64_t H, S, D, G, ngroups, bpg; // bpg = bytes per group = ceil(G/2)
  int64_t rows;                     // B*H*S
  uint8_t* packed;
  int64_t ps_b, ps_h, ps_s;         // byte strides of packed
  void* scales;
  int64_t ss_b, ss_h, ss_s;         // element strides of scales
  const int32_t* write_pos;
  int64_t write_pos0;
  int64_t cap;  // contiguous layout: destination rows per (b, h); rows at or past it are dropped
  int x_dtype, scale_dtype;
  PageMap pm;  // pm.paged: packed/scales are pools (ps_b = ss_b = 0)
  // row -> (b, h, s) and thread -> (row, chunk) without runtime divides
  // (vector path; rows * D / 8 < 2^32)
  FastDiv div_s, div_h, div_cpr;
};

// Destination row of (b, position), or -1 where it does not exist: the
// position itself in the contiguous layout (if inside [0, cap)), its pool row
// in the paged one.
__device__ __forceinline__ int64_t dest_row(const QuantArgs& a, int64_t b, int64_t pos) {
  return a.pm.paged ? page_row(a.pm, b, pos) : (pos >= 0 && pos < a.cap ? pos : -1);
}

template <int XDT>
__device__ __forceinline__ float ld_x(const void* p, int64_t i) {
  if constexpr (XDT == KVQ_BF16) return bf16_bits_to_f32(((const uint16_t*)p)[i]);
  else if constexpr (XDT == KVQ_F16) return f16_bits_to_f32(((const uint16_t*)p)[i]);
  else return ((const float*)p)[i];
}

template <int XDT>
__global__ __launch_bounds__(256) void quantize_kernel(const QuantArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.rows * a.ngroups) return;
  const int64_t row = idx / a.ngroups;
  const int64_t g = idx - row * a.ngroups;
  const int64_t s = row % a.S;
  const int64_t bh = row / a.S;
  const int64_t h = bh % a.H;
  const int64_t b = bh / a.H;

  const int64_t xbase = b * a.xs_b + h * a.xs_h + s * a.xs_s;
  const int64_t c0 = g * a.G;
  const int64_t c1 = (c0 + a.G < a.D) ? c0 + a.G : a.D;  // real columns [c0, c1)

  float amax = 0.0f;
  for (int64_t c = c0; c < c1; ++c) amax = fmaxf(amax, fabsf(ld_x<XDT>(a.x, xbase + c * a.xs_d)));
  const float scale = group_scale(amax);  // amax / 7, correctly rounded

  const int64_t pos = dest_row(a, b, (a.write_pos ? (int64_t)a.write_pos[b] : a.write_pos0) + s);
  if (pos < 0) return;  // no destination row: past the capacity, or no block holds it
  uint8_t* prow = a.packed + b * a.ps_b + h * a.ps_h + pos * a.ps_s + g * a.bpg;

  for (int64_t j = 0; j < a.bpg; ++j) {
    uint32_t nib[2];
#pragma unroll
    for (int e = 0; e < 2; ++e) {
      const int64_t k = 2 * j + e;  // element index inside the group
      if (k >= a.G) {               // odd G: the closing pad nibble is 0
        nib[e] = 0u;
        continue;
      }
      const int64_t c = c0 + k;
      const float v = c < c1 ? ld_x<XDT>(a.x, xbase + c * a.xs_d) : 0.0f;
      float qf = __builtin_rintf(v / scale);  // round half to even
      qf = fminf(fmaxf(qf, -8.0f), 7.0f);
      nib[e] = (uint32_t)((int)qf + 8);
    }
    prow[j] = (uint8_t)(nib[0] | (nib[1] << 4));
  }
  const int64_t sidx = b * a.ss_b + h * a.ss_h + pos * a.ss_s + g;
  store_from_f32(a.scales, sidx, a.scale_dtype, scale);
}

// ---------------------------------------------------------------------------
// Vector path: one thread per 8-element chunk of a row (one 16-byte load for
// 16-bit inputs, two for fp32), G/8 consecutive lanes per group. The group's
// absmax is all-reduced across those lanes with DPP (quad xor 1, quad xor 2,
// half-row mirror, row mirror), every lane divides its own 8 elements by the
// group scale and packs them into one 4-byte store; the group's first lane
// stores the scale. Taken when G is 8..128 (power of two), G divides D, x rows
// have unit inner stride and 16-byte aligned starts, and packed rows are
// 4-byte aligned; everything else takes quantize_kernel.

// The vector kernels stream every byte once, so their bulk accesses carry
// the nontemporal hint (the `nt` bit): the quantizer's input loads and code
// stores, and the dequantizer's output stores. Measured on prompt appends of
// [1, 8, 16384, 128] and [8, 8, 32768, 128] bf16: quantize 14.0 -> 12.7 and
// 135 -> 131 us a launch, dequantize 12.3 -> 9.7 and 122 -> 117 us. (The
// dequantizer's code loads gained nothing from it; the decode kernels' cache
// loads lost with it at large batch, and keep the default policy.)
typedef uint32_t nt_u32x4 __attribute__((ext_vector_type(4)));

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL,
                                                               0xF, 0xF, false));
}


// Each thread takes chunk ch of RPT rows (row slot r0 and r0 + k * rq); for
// every k the G/8 lanes of a group hold adjacent chunks of one row. All of
// its loads are issued before any store, in this order: the x chunks of the
// RPT rows, their write positions, then (paged) the page-table entries, which
// need the positions. Placing each row only after the previous row's loads
// had arrived cost a memory round trip per row (2.6 us of a 4.8 us launch
// for one token of 8 heads). Index arithmetic is 32-bit (the host takes this
// path only when rows * D / 8 < 2^32).
// Rows per thread of the vector quantize / dequantize kernels: four for
// large launches (more loads in flight per lane), one for launches of at
// most kSmallChunks 8-element chunks. A small launch (a decode token's K or
// V) runs one or a few waves whose time is their instruction latency: for
// one token of 8 heads, four rows per lane took 4.5 us and one row 2.2 us.
constexpr int kQuantRows = 4;
constexpr int64_t kSmallChunks = 256 * 1024;

template <int XDT, int LPG, int RPT>  // LPG = lanes per group = G / 8
__global__ __launch_bounds__(256) void quantize_vec_kernel(const QuantArgs a) {
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t cpr = (uint32_t)a.D >> 3;  // chunks per row
  const uint32_t rows = (uint32_t)a.rows;
  const uint32_t rq = (rows + RPT - 1) / RPT;
  const bool slot = idx < rq * cpr;
  const uint32_t r0 = slot ? fdiv(idx, a.div_cpr) : 0u;
  const uint32_t ch = slot ? idx - r0 * cpr : 0u;
  const uint32_t S = (uint32_t)a.S, H = (uint32_t)a.H;

  constexpr int NW = XDT == KVQ_F32 ? 2 : 1;  // 16-byte loads per chunk
  bool live[RPT];
  uint32_t bb[RPT], hh[RPT], ss[RPT];
  uint4 raw[RPT][NW];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const uint32_t row = r0 + (uint32_t)k * rq;
    live[k] = slot && row < rows;
    const uint32_t rw = live[k] ? row : 0u;
    const uint32_t bh = fdiv(rw, a.div_s);
    ss[k] = rw - bh * S;
    bb[k] = fdiv(bh, a.div_h);
    hh[k] = bh - bb[k] * H;
    const int64_t xoff = (int64_t)bb[k] * a.xs_b + (int64_t)hh[k] * a.xs_h + (int64_t)ss[k] * a.xs_s + 8 * ch;
#pragma unroll
    for (int n = 0; n < NW; ++n)
      raw[k][n] = __builtin_bit_cast(
          uint4, __builtin_nontemporal_load((const nt_u32x4*)((const uint8_t*)a.x + (xoff + 4 * n) * (NW * 2))));
  }
  int64_t pos[RPT];
  if (a.write_pos) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) pos[k] = (int64_t)a.write_pos[bb[k]] + ss[k];
  } else {
#pragma unroll
    for (int k = 0; k < RPT; ++k) pos[k] = a.write_pos0 + ss[k];
  }
  int64_t dst[RPT];  // destination row; < 0: none (past the capacity, or no block holds it)
  page_rows<RPT>(a.pm, bb, pos, dst);
  if (!a.pm.paged) {
#pragma unroll
    for (int k = 0; k < RPT; ++k) dst[k] = dst[k] < a.cap ? dst[k] : -1;
  }
  float x[RPT][8];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    if constexpr (XDT == KVQ_F32) {
#pragma unroll
      for (int n = 0; n < 2; ++n) {
        x[k][4 * n + 0] = __builtin_bit_cast(float, raw[k][n].x);
        x[k][4 * n + 1] = __builtin_bit_cast(float, raw[k][n].y);
        x[k][4 * n + 2] = __builtin_bit_cast(float, raw[k][n].z);
        x[k][4 * n + 3] = __builtin_bit_cast(float, raw[k][n].w);
      }
    } else {
      const uint32_t wd[4] = {raw[k][0].x, raw[k][0].y, raw[k][0].z, raw[k][0].w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (XDT == KVQ_BF16) {
          x[k][2 * j] = bf16_bits_to_f32(wd[j] & 0xffffu);
          x[k][2 * j + 1] = bf16_bits_to_f32(wd[j] >> 16);
        } else {
          x[k][2 * j] = f16_bits_to_f32(wd[j] & 0xffffu);
          x[k][2 * j + 1] = f16_bits_to_f32(wd[j] >> 16);
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) amax = fmaxf(amax, fabsf(x[k][e]));
    // Every lane of the wave takes part in the DPP steps (dead lanes carry 0).
    if constexpr (LPG >= 2) amax = fmaxf(amax, dpp_f<0xB1>(amax));   // quad_perm [1,0,3,2]
    if constexpr (LPG >= 4) amax = fmaxf(amax, dpp_f<0x4E>(amax));   // quad_perm [2,3,0,1]
    if constexpr (LPG >= 8) amax = fmaxf(amax, dpp_f<0x141>(amax));  // row_half_mirror
    if constexpr (LPG >= 16) amax = fmaxf(amax, dpp_f<0x140>(amax)); // row_mirror
    if (!live[k]) continue;
    const float scale = group_scale(amax);  // amax / 7, correctly rounded
    const float inv = group_inverse(scale);
    // Codes + 8 without a divide: t = x * inv + 8 in one fma, rounded to an
    // integer (ties to even) by adding 2^23, so that the sum's low byte is
    // the code + 8, in [1, 15] for |x| <= 7 s (no clamp). That is rint of
    // the correctly rounded quotient unless t lies within 2^-17 of a
    // half-integer (the residual t - rint(t) is exact; the bound is that of
    // rint_quotient plus the fma's rounding); such elements, and every
    // element of a group whose scale is outside [2^-100, 2^100], take the
    // division. One test per row (the residuals' maximum, which propagates
    // NaN, so a NaN element divides too and gets the division path's code)
    // keeps the common case free of per-element branches; inside it each
    // element divides on its own, since with 16-bit inputs exact ties are
    // common and dividing the whole row cost more than it saved.
    // oracle/kvq_ref.c kvqref_check_rint_margin_fma8 pins the margin.
    const bool fast = scale >= 0x1p-100f && scale <= 0x1p100f;
    uint32_t cb[8];
    float rmax = 0.0f;
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float t = __builtin_fmaf(x[k][e], inv, 8.0f);
      const float u = t + 0x1p23f;
      rmax = __builtin_elementwise_maximum(rmax, fabsf(t - (u - 0x1p23f)));
      cb[e] = __builtin_bit_cast(uint32_t, u);
    }
    if (!(rmax <= 0.5f - 0x1p-17f && fast)) {
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float t = __builtin_fmaf(x[k][e], inv, 8.0f);
        const float u = t + 0x1p23f;
        if (!(fast && fabsf(t - (u - 0x1p23f)) <= 0.5f - 0x1p-17f)) {
          const float qf = fminf(fmaxf(__builtin_rintf(x[k][e] / scale), -8.0f), 7.0f);  // round half to even
          cb[e] = (uint32_t)((int)qf + 8);
        }
      }
    }
    // byte 0 of cb[e] is element e's code + 8: even elements to the low
    // nibbles, odd ones to the high nibbles (v_perm_b32 byte gathers)
    const uint32_t lo = __builtin_amdgcn_perm(__builtin_amdgcn_perm(cb[6], cb[4], 0x0c0c0400u),
                                              __builtin_amdgcn_perm(cb[2], cb[0], 0x0c0c0400u), 0x05040100u);
    const uint32_t hi = __builtin_amdgcn_perm(__builtin_amdgcn_perm(cb[7], cb[5], 0x0c0c0400u),
                                              __builtin_amdgcn_perm(cb[3], cb[1], 0x0c0c0400u), 0x05040100u);
    const uint32_t word = lo | (hi << 4);
    const int64_t b = bb[k], h = hh[k], pos = dst[k];
    if (pos < 0) continue;  // no destination row
    // chunk ch covers bytes [4 ch, 4 ch + 4) of the packed row (G even, no padding)
    __builtin_nontemporal_store(word, (uint32_t*)(a.packed + b * a.ps_b + h * a.ps_h + pos * a.ps_s + 4 * ch));
    if (ch % LPG == 0) {
      const int64_t g = ch / LPG;
      store_from_f32(a.scales, b * a.ss_b + h * a.ss_h + pos * a.ss_s + g, a.scale_dtype, scale);
    }
  }
}

struct DequantArgs {
  const uint8_t* packed;
  int64_t ps_b, ps_h, ps_s;
  const void* scales;
  int64_t ss_b, ss_h, ss_s;
  int64_t H, S, G, ngroups, bpg, d_out, rows;
  void* out;
  int64_t os_b, os_h, os_s, os_d;
  int scale_dtype, out_dtype;
  PageMap pm;  // pm.paged: packed/scales are pools (ps_b = ss_b = 0)
  FastDiv div_s, div_h, div_cpr;  // as in QuantArgs (vector path)
};

__global__ __launch_bounds__(256) void dequantize_kernel(const DequantArgs a) {
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= a.rows * a.ngroups) return;
  const int64_t row = idx / a.ngroups;
  const int64_t g = idx - row * a.ngroups;
  const int64_t s = row % a.S;
  const int64_t bh = row / a.S;
  const int64_t h = bh % a.H;
  const int64_t b = bh / a.H;

  const int64_t obase = b * a.os_b + h * a.os_h + s * a.os_s;
  const int64_t r = a.pm.paged ? page_row(a.pm, b, s) : s;
  if (r < 0) {  // paged: no block holds this position -> zeros
    for (int64_t c = g * a.G; c < (g + 1) * a.G && c < a.d_out; ++c)
      store_from_f32(a.out, obase + c * a.os_d, a.out_dtype, 0.0f);
    return;
  }
  const uint8_t* prow = a.packed + b * a.ps_b + h * a.ps_h + r * a.ps_s + g * a.bpg;
  const float scale = load_as_f32(a.scales, b * a.ss_b + h * a.ss_h + r * a.ss_s + g, a.scale_dtype);
  for (int64_t k = 0; k < a.G; ++k) {
    const int64_t c = g * a.G + k;
    if (c >= a.d_out) break;
    const uint32_t byte = prow[k >> 1];
    const uint32_t nib = (k & 1) ? (byte >> 4) : (byte & 15u);
    const float v = (float)((int)nib - 8) * scale;
    store_from_f32(a.out, obase + c * a.os_d, a.out_dtype, v);
  }
}

// Vector path: one thread per 8 consecutive elements of a row (one 4-byte
// code word and its group's scale in, one 16-byte store of 16-bit outputs or
// two of fp32 out). Taken when G is a multiple of 8 dividing d_out (=
// groups * G), packed rows are 4-byte aligned and output rows have unit
// inner stride and 16-byte aligned starts.
template <int ODT, int RPT>
__global__ __launch_bounds__(256) void dequantize_vec_kernel(const DequantArgs a) {
  const uint32_t idx = blockIdx.x * blockDim.x + threadIdx.x;
  const uint32_t cpr = (uint32_t)a.d_out >> 3;  // chunks per row
  const uint32_t rows = (uint32_t)a.rows;
  const uint32_t rq = (rows + RPT - 1) / RPT;
  if (idx >= rq * cpr) return;
  const uint32_t r0 = fdiv(idx, a.div_cpr);
  const uint32_t ch = idx - r0 * cpr;
  const uint32_t S = (uint32_t)a.S, H = (uint32_t)a.H;
  uint32_t w[RPT];
  float sc[RPT];
  int64_t obase[RPT], pos[RPT], r[RPT];
  uint32_t bb[RPT], hh[RPT];
  bool live[RPT];
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    const uint32_t row = r0 + (uint32_t)k * rq;
    live[k] = row < rows;
    const uint32_t rw = live[k] ? row : 0u;
    const uint32_t bh = fdiv(rw, a.div_s), s = rw - bh * S;
    bb[k] = fdiv(bh, a.div_h);
    hh[k] = bh - bb[k] * H;
    pos[k] = s;
    obase[k] = (int64_t)bb[k] * a.os_b + (int64_t)hh[k] * a.os_h + (int64_t)s * a.os_s + 8 * ch;
  }
  // All table reads in flight together, then all code and scale reads. An
  // absent position reads pool row 0 (present whenever the pool has a block)
  // and has its result replaced by zeros.
  page_rows<RPT>(a.pm, bb, pos, r);
  if (!a.pm.paged || a.pm.n_blocks > 0) {
    int64_t si[RPT];
#pragma unroll
    for (int k = 0; k < RPT; ++k) {
      const int64_t b = bb[k], h = hh[k], rr = r[k] < 0 ? 0 : r[k];
      w[k] = *(const uint32_t*)(a.packed + b * a.ps_b + h * a.ps_h + rr * a.ps_s + 4 * ch);
      si[k] = b * a.ss_b + h * a.ss_h + rr * a.ss_s + (8 * ch) / a.G;
    }
    load_n_as_f32<RPT>(a.scales, si, a.scale_dtype, sc);
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    if (r[k] < 0) {  // paged: no block holds this position -> zeros
      w[k] = 0x88888888u;
      sc[k] = 0.0f;
    }
  }
#pragma unroll
  for (int k = 0; k < RPT; ++k) {
    if (!live[k]) continue;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = (float)((int)((w[k] >> (4 * e)) & 15u) - 8) * sc[k];
    const int64_t o = obase[k];
    if constexpr (ODT == KVQ_F32) {
      *(float4*)((float*)a.out + o) = make_float4(v[0], v[1], v[2], v[3]);
      *(float4*)((float*)a.out + o + 4) = make_float4(v[4], v[5], v[6], v[7]);
    } else {
      // finite values: the hardware conversions round to nearest even, as
      // f32_to_bf16_bits / f32_to_f16_bits do
      uint32_t p[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        if constexpr (ODT == KVQ_BF16) {
          typedef __bf16 bf16x2_v __attribute__((ext_vector_type(2)));
          const bf16x2_v h = {(__bf16)v[2 * j], (__bf16)v[2 * j + 1]};
          p[j] = __builtin_bit_cast(uint32_t, h);
        } else {
          typedef _Float16 f16x2_v __attribute__((ext_vector_type(2)));
          const f16x2_v h = {(_Float16)v[2 * j], (_Float16)v[2 * j + 1]};
          p[j] = __builtin_bit_cast(uint32_t, h);
        }
      }
      __builtin_nontemporal_store(nt_u32x4{p[0], p[1], p[2], p[3]}, (nt_u32x4*)((uint16_t*)a.out + o));
    }
  }
}

}  // namespace kvq

using namespace kvq;

namespace {

template <int XDT, int RPT>
void launch_qvec(int lpg, dim3 grid, hipStream_t st, const QuantArgs& a) {
  switch (lpg) {
    case 1: hipLaunchKernelGGL((quantize_vec_kernel<XDT, 1, RPT>), grid, dim3(256), 0, st, a); break;
    case 2: hipLaunchKernelGGL((quantize_vec_kernel<XDT, 2, RPT>), grid, dim3(256), 0, st, a); break;
    case 4: hipLaunchKernelGGL((quantize_vec_kernel<XDT, 4, RPT>), grid, dim3(256), 0, st, a); break;
    case 8: hipLaunchKernelGGL((quantize_vec_kernel<XDT, 8, RPT>), grid, dim3(256), 0, st, a); break;
    default: hipLaunchKernelGGL((quantize_vec_kernel<XDT, 16, RPT>), grid, dim3(256), 0, st, a); break;
  }
}

template <int ODT, int RPT>
void launch_dqvec(dim3 grid, hipStream_t st, const DequantArgs& a) {
  hipLaunchKernelGGL((dequantize_vec_kernel<ODT, RPT>), grid, dim3(256), 0, st, a);
}

// Checks a paged-pool description shared by the paged entry points and
// fills `pm`. Pools are [H, num_blocks << page_shift, ...]; the entry point's
// stride arrays give (head, row) strides and the batch stride is 0.
int page_map(const char* who, const int32_t* block_table, int64_t table_stride, int64_t table_cols,
             int64_t num_blocks, int64_t page_size, int64_t B, PageMap* pm) {
  KVQ_CHECK_ARG(page_size >= 1 && (page_size & (page_size - 1)) == 0 && page_size <= (1 << 20),
                "%s: page_size must be a power of two in [1, 2^20] (got %lld)", who, (long long)page_size);
  KVQ_CHECK_ARG(num_blocks >= 0 && table_cols >= 0 && table_stride >= table_cols,
                "%s: bad block table geometry (num_blocks %lld, cols %lld, stride %lld)", who,
                (long long)num_blocks, (long long)table_cols, (long long)table_stride);
  KVQ_CHECK_ARG(block_table != nullptr || B == 0 || table_cols == 0, "%s: null block table", who);
  KVQ_CHECK_ARG(num_blocks <= (int64_t(1) << 31) / page_size, "%s: pool too large", who);
  int shift = 0;
  while ((int64_t(1) << shift) < page_size) ++shift;
  pm->paged = 1;
  pm->table = block_table;
  pm->tab_stride = table_stride;
  pm->n_pages = table_cols;
  pm->n_blocks = num_blocks;
  pm->page_shift = shift;
  return KVQ_OK;
}

int quantize_impl(const char* who, const void* x, int x_dtype, const int64_t* x_strides,
                  int64_t B, int64_t H, int64_t S, int64_t D, int64_t group_size,
                  void* packed, const int64_t* packed_strides,
                  void* scales, int scale_dtype, const int64_t* scale_strides,
                  const int32_t* write_pos, int64_t write_pos0, int64_t capacity,
                  const PageMap& pm, void* stream) {
  KVQ_CHECK_ARG(group_size > 0, "kvq_quantize: group_size must be > 0");
  KVQ_CHECK_ARG(dtype_ok(x_dtype), "kvq_quantize: x dtype must be bf16/fp16/fp32");
  KVQ_CHECK_ARG(dtype_ok(scale_dtype), "kvq_quantize: scale dtype must be bf16/fp16/fp32");
  KVQ_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && D >= 0, "kvq_quantize: negative extent");
  KVQ_CHECK_ARG(x_strides && packed_strides && scale_strides, "kvq_quantize: null stride array");
  KVQ_CHECK_ARG(write_pos0 >= 0, "kvq_quantize: write_pos0 must be >= 0");
  KVQ_CHECK_ARG(capacity >= 0, "kvq_quantize: capacity must be >= 0");
  KVQ_CHECK_ARG(write_pos != nullptr || B * H * S == 0 || write_pos0 + S <= capacity,
                "kvq_quantize: rows %lld..%lld outside the destination's %lld rows", (long long)write_pos0,
                (long long)(write_pos0 + S - 1), (long long)capacity);
  const int64_t rows = B * H * S;
  const int64_t ngroups = (D + group_size - 1) / group_size;
  if (rows == 0 || ngroups == 0) return KVQ_OK;
  KVQ_CHECK_ARG(x && packed && scales, "kvq_quantize: null data pointer");
  KVQ_CHECK_ARG(rows * std::max<int64_t>(ngroups, (D + 7) / 8) / 256 < 0x7fffffffll,
                "kvq_quantize: input too large for one launch");

  QuantArgs a;
  a.x = x;
  a.xs_b = x_strides[0]; a.xs_h = x_strides[1]; a.xs_s = x_strides[2]; a.xs_d = x_strides[3];
  a.H = H; a.S = S; a.D = D; a.G = group_size; a.ngroups = ngroups; a.bpg = (group_size + 1) / 2;
  a.rows = rows;
  a.packed = (uint8_t*)packed;
  a.ps_b = packed_strides[0]; a.ps_h = packed_strides[1]; a.ps_s = packed_strides[2];
  a.scales = scales;
  a.ss_b = scale_strides[0]; a.ss_h = scale_strides[1]; a.ss_s = scale_strides[2];
  a.write_pos = write_pos; a.write_pos0 = write_pos0;
  a.cap = capacity;
  a.x_dtype = x_dtype; a.scale_dtype = scale_dtype;
  a.pm = pm;
  a.div_s = make_fastdiv((uint32_t)S);
  a.div_h = make_fastdiv((uint32_t)H);
  a.div_cpr = make_fastdiv((uint32_t)std::max<int64_t>(1, D / 8));

  hipStream_t st = (hipStream_t)stream;
  const int lpg = (int)(group_size / 8);
  const int64_t esz = dtype_size(x_dtype);
  const bool vec = group_size % 8 == 0 && group_size <= 128 && (lpg & (lpg - 1)) == 0 &&
                   D % group_size == 0 && a.xs_d == 1 &&
                   (uintptr_t)x % 16 == 0 && (a.xs_b * esz) % 16 == 0 && (a.xs_h * esz) % 16 == 0 &&
                   (a.xs_s * esz) % 16 == 0 &&
                   (uintptr_t)packed % 4 == 0 && a.ps_b % 4 == 0 && a.ps_h % 4 == 0 && a.ps_s % 4 == 0 &&
                   rows * (D / 8) < (1ll << 32) - 256 * kQuantRows;
  if (vec) {
    const bool small = rows * (D / 8) <= kSmallChunks;
    const int rpt = small ? 1 : kQuantRows;
    const int64_t total = (rows + rpt - 1) / rpt * (D / 8);
    const dim3 grid((unsigned)((total + 255) / 256));
    switch (x_dtype) {
      case KVQ_BF16: small ? launch_qvec<KVQ_BF16, 1>(lpg, grid, st, a) : launch_qvec<KVQ_BF16, kQuantRows>(lpg, grid, st, a); break;
      case KVQ_F16: small ? launch_qvec<KVQ_F16, 1>(lpg, grid, st, a) : launch_qvec<KVQ_F16, kQuantRows>(lpg, grid, st, a); break;
      default: small ? launch_qvec<KVQ_F32, 1>(lpg, grid, st, a) : launch_qvec<KVQ_F32, kQuantRows>(lpg, grid, st, a); break;
    }
    KVQ_CHECK_LAUNCH(who);
    return KVQ_OK;
  }

  const int64_t total = rows * ngroups;
  const dim3 block(256);
  const dim3 grid((unsigned)((total + 255) / 256));
  switch (x_dtype) {
    case KVQ_BF16: hipLaunchKernelGGL(quantize_kernel<KVQ_BF16>, grid, block, 0, st, a); break;
    case KVQ_F16: hipLaunchKernelGGL(quantize_kernel<KVQ_F16>, grid, block, 0, st, a); break;
    default: hipLaunchKernelGGL(quantize_kernel<KVQ_F32>, grid, block, 0, st, a); break;
  }
  KVQ_CHECK_LAUNCH(who);
  return KVQ_OK;
}

int dequantize_impl(const void* packed, const int64_t* packed_strides,
                    const void* scales, int scale_dtype, const int64_t* scale_strides,
                    int64_t B, int64_t H, int64_t S, int64_t group_size, int64_t num_groups,
                    void* out, int out_dtype, const int64_t* out_strides, int64_t d_out,
                    const PageMap& pm, void* stream) {
  KVQ_CHECK_ARG(group_size > 0, "kvq_dequantize: group_size must be > 0");
  KVQ_CHECK_ARG(dtype_ok(scale_dtype), "kvq_dequantize: scale dtype must be bf16/fp16/fp32");
  KVQ_CHECK_ARG(dtype_ok(out_dtype), "kvq_dequantize: out dtype must be bf16/fp16/fp32");
  KVQ_CHECK_ARG(B >= 0 && H >= 0 && S >= 0 && num_groups >= 0 && d_out >= 0,
                "kvq_dequantize: negative extent");
  KVQ_CHECK_ARG(d_out <= num_groups * group_size, "kvq_dequantize: d_out exceeds num_groups*group_size");
  KVQ_CHECK_ARG(packed_strides && scale_strides && out_strides, "kvq_dequantize: null stride array");
  const int64_t rows = B * H * S;
  if (rows == 0 || num_groups == 0 || d_out == 0) return KVQ_OK;
  KVQ_CHECK_ARG(packed && scales && out, "kvq_dequantize: null data pointer");

  DequantArgs a;
  a.packed = (const uint8_t*)packed;
  a.ps_b = packed_strides[0]; a.ps_h = packed_strides[1]; a.ps_s = packed_strides[2];
  a.scales = scales;
  a.ss_b = scale_strides[0]; a.ss_h = scale_strides[1]; a.ss_s = scale_strides[2];
  a.H = H; a.S = S; a.G = group_size; a.ngroups = num_groups; a.bpg = (group_size + 1) / 2;
  a.d_out = d_out; a.rows = rows;
  a.out = out;
  a.os_b = out_strides[0]; a.os_h = out_strides[1]; a.os_s = out_strides[2]; a.os_d = out_strides[3];
  a.scale_dtype = scale_dtype; a.out_dtype = out_dtype;
  a.pm = pm;
  a.div_s = make_fastdiv((uint32_t)S);
  a.div_h = make_fastdiv((uint32_t)H);
  a.div_cpr = make_fastdiv((uint32_t)std::max<int64_t>(1, d_out / 8));

  const int64_t oes = dtype_size(out_dtype);
  const bool vec = group_size % 8 == 0 && d_out == num_groups * group_size && a.os_d == 1 &&
                   (uintptr_t)out % 16 == 0 && (a.os_b * oes) % 16 == 0 && (a.os_h * oes) % 16 == 0 &&
                   (a.os_s * oes) % 16 == 0 && (uintptr_t)packed % 4 == 0 && a.ps_b % 4 == 0 &&
                   a.ps_h % 4 == 0 && a.ps_s % 4 == 0 && rows * (d_out / 8) < (1ll << 32) - 256 * kQuantRows;
  hipStream_t st = (hipStream_t)stream;
  if (vec) {
    const bool small = rows * (d_out / 8) <= kSmallChunks;
    const int rpt = small ? 1 : kQuantRows;
    const int64_t total = (rows + rpt - 1) / rpt * (d_out / 8);
    const dim3 grid((unsigned)((total + 255) / 256));
    switch (out_dtype) {
      case KVQ_BF16: small ? launch_dqvec<KVQ_BF16, 1>(grid, st, a) : launch_dqvec<KVQ_BF16, kQuantRows>(grid, st, a); break;
      case KVQ_F16: small ? launch_dqvec<KVQ_F16, 1>(grid, st, a) : launch_dqvec<KVQ_F16, kQuantRows>(grid, st, a); break;
      default: small ? launch_dqvec<KVQ_F32, 1>(grid, st, a) : launch_dqvec<KVQ_F32, kQuantRows>(grid, st, a); break;
    }
    KVQ_CHECK_LAUNCH("kvq_dequantize");
    return KVQ_OK;
  }
  const int64_t total = rows * num_groups;
  hipLaunchKernelGGL(dequantize_kernel, dim3((unsigned)((total + 255) / 256)), dim3(256), 0, st, a);
  KVQ_CHECK_LAUNCH("kvq_dequantize");
  return KVQ_OK;
}

}  // namespace

extern "C" int kvq_quantize(const void* x, int x_dtype, const int64_t* x_strides,
                            int64_t B, int64_t H, int64_t S, int64_t D, int64_t group_size,
                            void* packed, const int64_t* packed_strides,
                            void* scales, int scale_dtype, const int64_t* scale_strides,
                            const int32_t* write_pos, int64_t write_pos0, int64_t capacity,
                            void* stream) {
  clear_error();
  const PageMap pm{0, nullptr, 0, 0, 0, 0};
  return quantize_impl("kvq_quantize", x, x_dtype, x_strides, B, H, S, D, group_size, packed,
                       packed_strides, scales, scale_dtype, scale_strides, write_pos, write_pos0, capacity,
                       pm, stream);
}

extern "C" int kvq_quantize_paged(const void* x, int x_dtype, const int64_t* x_strides,
                                  int64_t B, int64_t H, int64_t S, int64_t D, int64_t group_size,
                                  void* packed_pool, const int64_t* pool_strides,
                                  void* scale_pool, int scale_dtype, const int64_t* scale_pool_strides,
                                  const int32_t* block_table, int64_t table_stride, int64_t table_cols,
                                  int64_t num_blocks, int64_t page_size,
                                  const int32_t* write_pos, int64_t write_pos0,
                                  void* stream) {
  clear_error();
  KVQ_CHECK_ARG(pool_strides && scale_pool_strides, "kvq_quantize_paged: null stride array");
  PageMap pm;
  const int rc = page_map("kvq_quantize_paged", block_table, table_stride, table_cols, num_blocks,
                          page_size, B, &pm);
  if (rc != KVQ_OK) return rc;
  const int64_t ps[3] = {0, pool_strides[0], pool_strides[1]};
  const int64_t ss[3] = {0, scale_pool_strides[0], scale_pool_strides[1]};
  return quantize_impl("kvq_quantize_paged", x, x_dtype, x_strides, B, H, S, D, group_size,
                       packed_pool, ps, scale_pool, scale_dtype, ss, write_pos, write_pos0,
                       std::numeric_limits<int64_t>::max(), pm, stream);
}

extern "C" int kvq_dequantize(const void* packed, const int64_t* packed_strides,
                              const void* scales, int scale_dtype, const int64_t* scale_strides,
                              int64_t B, int64_t H, int64_t S, int64_t group_size, int64_t num_groups,
                              void* out, int out_dtype, const int64_t* out_strides, int64_t d_out,
                              void* stream) {
  clear_error();
  const PageMap pm{0, nullptr, 0, 0, 0, 0};
  return dequantize_impl(packed, packed_strides, scales, scale_dtype, scale_strides, B, H, S,
                         group_size, num_groups, out, out_dtype, out_strides, d_out, pm, stream);
}

extern "C" int kvq_dequantize_paged(const void* packed_pool, const int64_t* pool_strides,
                                    const void* scale_pool, int scale_dtype,
                                    const int64_t* scale_pool_strides,
                                    const int32_t* block_table, int64_t table_stride,
                                    int64_t table_cols, int64_t num_blocks, int64_t page_size,
                                    int64_t B, int64_t H, int64_t S, int64_t group_size,
                                    int64_t num_groups, void* out, int out_dtype,
                                    const int64_t* out_strides, int64_t d_out, void* stream) {
  clear_error();
  KVQ_CHECK_ARG(pool_strides && scale_pool_strides, "kvq_dequantize_paged: null stride array");
  PageMap pm;
  const int rc = page_map("kvq_dequantize_paged", block_table, table_stride, table_cols, num_blocks,
                          page_size, B, &pm);
  if (rc != KVQ_OK) return rc;
  const int64_t ps[3] = {0, pool_strides[0], pool_strides[1]};
  const int64_t ss[3] = {0, scale_pool_strides[0], scale_pool_strides[1]};
  return dequantize_impl(packed_pool, ps, scale_pool, scale_dtype, ss, B, H, S, group_size,
                         num_groups, out, out_dtype, out_strides, d_out, pm, stream);
}
