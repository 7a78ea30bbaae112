// Attention of long query blocks over the INT4 cache on the matrix cores
// (gfx950): prompt prefill and prompt chunks after cached tokens.
//
// Reference: kernels/llama3/attention_quant.py:24-152 (_attention_fwd_quant_gqa_
// _kernel) computes the same thing per (batch, query head, 16-query block):
// dequantize 64-key tiles of K and V, scores q.k * d^-1/2, bottom-right causal
// mask (:91-97, :123), online softmax, o += p.v. Here one workgroup takes 64
// query rows of one KV head (GQA group x positions, so each K/V tile is read
// once for the whole group), dequantizes each 64-key tile into LDS once for
// its four waves, and runs both products on v_mfma_f32_16x16x32 bf16/f16.
//
// Layout of one wave's work (16 query rows, lane l: lq = l % 16, lg = l / 16;
// MFMA 16x16x32: A[i][k] at lane (i, k / 8), register k % 8; B[k][n] at lane
// (n, k / 8); C[i][n] at lane (n, i / 4), register i % 4):
//   S^T = K Q^T   four 16-key blocks per 64-key tile, 32 dims per MFMA:
//                 A = K rows from LDS, B = the wave's Q (registers, loaded
//                 once). Block kb's row i is key 32 (kb / 2) + 8 (i / 4) +
//                 4 (kb % 2) + i % 4, so lane (lq, lg) ends up holding the
//                 scores of query row lq for keys 32 h + 8 lg .. + 7 in blocks
//                 2 h and 2 h + 1;
//   O^T += V^T P^T  A = V^T rows from LDS (V is stored transposed), B = P^T
//                 over 32 keys, which is exactly what the lane holds, so the
//                 softmax weights never leave the lane; lane (lq, lg)
//                 accumulates dims 4 lg .. 4 lg + 3 of each 16-dim block of
//                 query row lq.
// Every per-row scalar (running max, sum, rescale) thus lives on the lanes of
// that row: lq, lq + 16, lq + 32, lq + 48, combined with two xor shuffles.
//
// K and V are dequantized exactly as kvq_dequantize does ((n - 8) * scale in
// fp32, rounded to the query dtype), i.e. the numerics of dequantize + SDPA.

#include <algorithm>

#include "kvq_common.h"

namespace kvq {
namespace {

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

constexpr int kWaveRows = 16;  // query rows per wave and row block
constexpr int kKeys = 64;    // keys per tile
constexpr float kNegP = -1.0e30f;
// Running-max slack (log2 units): a row's reference max moves, and its state
// is rescaled, only when a tile's max exceeds it by more than this, so
// weights 2^(s - m) stay below 2^8, which the fp16/bf16 weights and fp32 sums
// hold with their full precision.
constexpr float kLazyMaxP = 8.0f;

struct PrefillArgs {
  const uint16_t* q;
  int64_t qs_b, qs_h, qs_s;  // element strides (dims contiguous)
  const uint8_t* kp;
  int64_t kps_b, kps_h, kps_s;  // byte strides
  const uint16_t* ks;
  int64_t kss_b, kss_h, kss_s;  // element strides
  const uint8_t* vp;
  int64_t vps_b, vps_h, vps_s;
  const uint16_t* vs;
  int64_t vss_b, vss_h, vss_s;
  uint16_t* out;
  int64_t os_b, os_h, os_s;
  int Hkv, ratio, Sq, Sk, G, row_blocks, causal;
  float scale_log2;  // sm_scale * log2(e): scores in base 2
  // paged cache: K/V are pools [Hkv, n_blocks << page_shift, .] (batch
  // strides 0); sequence b's token t is pool row bt[b * bt_stride +
  // (t >> page_shift)] << page_shift | (t & (page size - 1)); entries outside
  // [0, n_blocks), or pages >= bt_cols, have no rows. Pages hold a multiple of
  // 64 rows, so a 64-key tile lies in one page.
  const int32_t* bt;
  int64_t bt_stride;
  int bt_cols, n_blocks, page_shift;
  // split over keys (n_split > 1): workgroup split sp of a row block takes an
  // equal share of its 64-key tiles and writes fp32 partials — unnormalised
  // O rows [D] and (running max, sum) — for prefill_merge_kernel
  int n_split;
  float* ws_o;   // [unit][split][rows][D]
  float* ws_ml;  // [unit][split][rows][2]
};

__device__ __forceinline__ __amdgpu_buffer_rsrc_t prefill_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes, 0x00020000);
}

template <bool F16>
__device__ __forceinline__ f32x4_t mfma32(uint4 a, uint4 b, f32x4_t c) {
  if constexpr (F16)
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8_t, a), __builtin_bit_cast(f16x8_t, b),
                                                  c, 0, 0, 0);
  else
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8_t, a), __builtin_bit_cast(bf16x8_t, b),
                                                   c, 0, 0, 0);
}

// two values rounded to the MFMA input type, packed low | high << 16
template <bool F16>
__device__ __forceinline__ uint32_t pack2(float lo, float hi) {
  if constexpr (F16) {
    const f16x2_t h = {(_Float16)lo, (_Float16)hi};
    return __builtin_bit_cast(uint32_t, h);
  } else {
    const bf16x2_t h = {(__bf16)lo, (__bf16)hi};
    return __builtin_bit_cast(uint32_t, h);
  }
}

template <bool S_F16>
__device__ __forceinline__ float scale_f32(uint32_t bits) {
  return S_F16 ? f16_bits_to_f32(bits & 0xffffu) : bf16_bits_to_f32(bits & 0xffffu);
}

// The tile's share of one thread dequantized as (n - 8) sc directly (the
// rare tiles with a scale beyond 2^125, where -8 sc would overflow): K code
// dwords k (D / 32 of them used), V code words v (one per key), raw scales.
template <int D, bool F16, bool S_F16, int KP, int VP, int KB, int VD>
__device__ __attribute__((noinline)) void store_tile_direct(uint16_t* k_dst, uint16_t* v_dst, uint4 k,
                                                            uint32_t ksc, uint4 v, uint4 vsc) {
  const uint32_t kw[4] = {k.x, k.y, k.z, k.w};
  const float ksf = scale_f32<S_F16>(ksc);
#pragma unroll
  for (int w = 0; w < KB / 4; ++w) {
    uint32_t pk[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const uint32_t byte = (kw[w] >> (8 * j)) & 0xffu;
      pk[j] = pack2<F16>((float)((int)(byte & 15u) - 8) * ksf, (float)((int)(byte >> 4) - 8) * ksf);
    }
    *(uint4*)(k_dst + 8 * w) = make_uint4(pk[0], pk[1], pk[2], pk[3]);
  }
  const uint32_t vw[4] = {v.x, v.y, v.z, v.w}, vs[4] = {vsc.x, vsc.y, vsc.z, vsc.w};
  float vf[4][VD];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const float sc = scale_f32<S_F16>(vs[i]);
#pragma unroll
    for (int d = 0; d < VD; ++d) vf[i][d] = (float)((int)((vw[i] >> (4 * d)) & 15u) - 8) * sc;
  }
#pragma unroll
  for (int d = 0; d < VD; ++d)
    *(uint2*)(v_dst + d * VP) = make_uint2(pack2<F16>(vf[0][d], vf[1][d]), pack2<F16>(vf[2][d], vf[3][d]));
}

// RB = 16-row blocks per wave (1 or 2): with two, every K and V fragment read
// from LDS feeds two MFMAs, halving LDS traffic and dequantize work per row.
// Two row blocks per wave must stay within 256 registers (two waves per
// SIMD): one more register halves the occupancy. NW = waves per workgroup
// (4, or 8 for D = 128 with two row blocks): the workgroup's threads share
// the dequantize of each K/V tile, so eight waves (one workgroup per CU
// instead of two of four) halve its VALU per wave.
template <int D, bool F16, bool S_F16, int RB, bool PAGED, int NW>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(RB == 2 ? 2 : 1)))
void prefill_attn_kernel(const PrefillArgs a) {
  constexpr int NT = 64 * NW;
  constexpr int ROWS = kWaveRows * NW * RB;  // query rows per workgroup
  constexpr int KP = D + 8;      // K tile row pitch in LDS (elements)
  constexpr int VP = kKeys + 8;  // V^T tile row pitch
  constexpr int NK = D / 32;     // 32-dim steps of S^T
  constexpr int NB = D / 16;     // 16-dim blocks of O^T
  // two tile buffers: tile i is read from buffer i % 2 while tile i + 1 is
  // dequantized into the other one
  __shared__ __align__(16) uint16_t k_lds[2][kKeys * KP];
  __shared__ __align__(16) uint16_t v_lds[2][D * VP];

  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int lq = lane & 15, lg = lane >> 4;
  // workgroup -> (KV head fastest, so that one head's row blocks share an
  // XCD and its L2; row blocks with the most keys first; batch)
  int wg = blockIdx.x;
  const int kvh = wg % a.Hkv;
  wg /= a.Hkv;
  const int sp = wg % a.n_split;
  wg /= a.n_split;
  const int blk = a.row_blocks - 1 - wg % a.row_blocks;
  const int b = wg / a.row_blocks;

  // this lane's query rows (one per row block) and the keys each may attend:
  // [0, lim)
  int s[RB], head[RB], lim[RB];
  bool row_ok[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const int R = blk * ROWS + wave * 16 * RB + 16 * r + lq;
    s[r] = R / a.ratio;
    head[r] = kvh * a.ratio + R % a.ratio;
    row_ok[r] = s[r] < a.Sq;
    int l = row_ok[r] ? (a.causal ? a.Sk - a.Sq + s[r] + 1 : a.Sk) : 0;
    lim[r] = l < 0 ? 0 : (l > a.Sk ? a.Sk : l);
  }
  // keys every row of the wave may attend: [0, lim_wave) (lim grows with the
  // row, so this is the first row's; a wave with no row in the sequence
  // masks nothing, its rows are never stored). Tiles inside it take the
  // softmax without key masks.
  int lim_wave;
  {
    const int R0 = blk * ROWS + __builtin_amdgcn_readfirstlane(wave) * 16 * RB;
    const int s0 = R0 / a.ratio;
    int l = a.causal ? a.Sk - a.Sq + s0 + 1 : a.Sk;
    l = l < 0 ? 0 : (l > a.Sk ? a.Sk : l);
    lim_wave = s0 < a.Sq ? l : 0x7fffffff;
  }
  // keys any row of the workgroup attends
  const int r_last = min((blk + 1) * ROWS, a.Sq * a.ratio) - 1;
  int kend = a.causal ? a.Sk - a.Sq + r_last / a.ratio + 1 : a.Sk;
  kend = kend < 0 ? 0 : (kend > a.Sk ? a.Sk : kend);
  // this split's tiles of the row block's key range
  const int tiles_all = (kend + kKeys - 1) / kKeys;
  const int tps = (tiles_all + a.n_split - 1) / a.n_split;
  const int tile_lo = sp * tps;
  const int tile_hi = min(tiles_all, tile_lo + tps);

  // the wave's queries as the B operand of S^T: lane (lq, lg) holds dims
  // 32 kk + 8 lg .. + 7 of row lq (rows past Sq are zero). Scores reach the
  // softmax as fma(s, c, -m) with c = |sm_scale| log2(e) > 0, so that the
  // row max can be taken over the unscaled scores; a negative sm_scale
  // negates the queries instead (a sign flip, exact).
  // (c is kept above 0 so that the -inf scores of masked keys give 0, never
  // NaN; sm_scale = 0 then weighs every key 2^(~1e-30 s) = 1, as it should)
  const float c = fmaxf(fabsf(a.scale_log2), 1.0e-30f);
  const uint32_t qneg = a.scale_log2 < 0.0f ? 0x80008000u : 0u;
  uint4 qf[RB][NK];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    const uint16_t* qr =
        a.q + (int64_t)b * a.qs_b + (int64_t)head[r] * a.qs_h + (int64_t)(row_ok[r] ? s[r] : 0) * a.qs_s;
#pragma unroll
    for (int kk = 0; kk < NK; ++kk) {
      const uint16_t* p = qr + 32 * kk + 8 * lg;
      uint32_t x[4];
#pragma unroll
      for (int w = 0; w < 4; ++w)
        x[w] = row_ok[r] ? ((uint32_t)p[2 * w] | ((uint32_t)p[2 * w + 1] << 16)) ^ qneg : 0u;
      qf[r][kk] = make_uint4(x[0], x[1], x[2], x[3]);
    }
  }

  // cache slices of this (batch, KV head) as bounds-checked buffers: rows at
  // or past Sk read as zero
  const uint32_t kps = (uint32_t)a.kps_s, vps = (uint32_t)a.vps_s;
  const uint32_t kss2 = 2u * (uint32_t)a.kss_s, vss2 = 2u * (uint32_t)a.vss_s;
  const uint32_t Sk = (uint32_t)a.Sk;
  const uint8_t* kp_bh = a.kp + b * a.kps_b + kvh * a.kps_h;
  const uint8_t* ks_bh = (const uint8_t*)(a.ks + b * a.kss_b + kvh * a.kss_h);
  const uint8_t* vp_bh = a.vp + b * a.vps_b + kvh * a.vps_h;
  const uint8_t* vs_bh = (const uint8_t*)(a.vs + b * a.vss_b + kvh * a.vss_h);
  const __amdgpu_buffer_rsrc_t rk = prefill_rsrc(kp_bh, Sk * kps);
  const __amdgpu_buffer_rsrc_t rks = prefill_rsrc(ks_bh, Sk * kss2);
  const __amdgpu_buffer_rsrc_t rv = prefill_rsrc(vp_bh, Sk * vps);
  const __amdgpu_buffer_rsrc_t rvs = prefill_rsrc(vs_bh, Sk * vss2);
  const int32_t* bt_b = PAGED ? a.bt + (int64_t)b * a.bt_stride : nullptr;

  // tile loaders. K: thread (key tid / KQ, part tid % KQ) takes D / KQ dims
  // (KB = D / (2 KQ) code bytes, within one scale group). V: thread (keys
  // 4 (tid % 16) .. + 3, dims (tid / 16) VD .. + VD) so that it writes V^T
  // rows of four consecutive keys.
  constexpr int KQ = NT / 64;          // threads per key row
  constexpr int KB = D / (2 * KQ);     // K code bytes per thread
  constexpr int VD = D / (NT / 16);    // V dims per thread
  static_assert(KB == 16 || KB == 8 || KB == 4, "K loader width");
  static_assert(VD == 8 || VD == 4, "V loader width");
  const int k_key = tid / KQ, k_q = tid % KQ;
  const int v_kq = tid & 15, v_dq = tid >> 4;
  const uint32_t k_grp = (uint32_t)((k_q * (2 * KB)) / a.G);
  const uint32_t v_grp = (uint32_t)((v_dq * VD) / a.G);
  uint32_t kraw[KB / 4];
  uint32_t ksc;
  uint32_t vraw[4];
  uint32_t vsc[4];
  auto load_tile = [&](uint32_t t0) {
    // contiguous: the slice's buffers at row t0. Paged: buffers over the
    // tile's own rows (its page's pool rows from the first one), holding the
    // keys before Sk, or none if no block holds the page.
    __amdgpu_buffer_rsrc_t tk = rk, tks = rks, tv = rv, tvs = rvs;
    uint32_t r0 = t0;
    if constexpr (PAGED) {
      const uint32_t pg = t0 >> a.page_shift;
      const int32_t blk = __builtin_amdgcn_readfirstlane(pg < (uint32_t)a.bt_cols ? bt_b[pg] : -1);
      const bool ok = blk >= 0 && blk < a.n_blocks && t0 < Sk;
      const uint32_t rb = __builtin_amdgcn_readfirstlane(
          ok ? ((uint32_t)blk << a.page_shift) | (t0 & ((1u << a.page_shift) - 1u)) : 0u);
      const uint32_t lim = __builtin_amdgcn_readfirstlane(ok ? min((uint32_t)kKeys, Sk - t0) : 0u);
      tk = prefill_rsrc(kp_bh + (size_t)rb * kps, lim * kps);
      tks = prefill_rsrc(ks_bh + (size_t)rb * kss2, lim * kss2);
      tv = prefill_rsrc(vp_bh + (size_t)rb * vps, lim * vps);
      tvs = prefill_rsrc(vs_bh + (size_t)rb * vss2, lim * vss2);
      r0 = 0;
    }
    const uint32_t kr = r0 + (uint32_t)k_key;
    if constexpr (KB == 16) {
      const u32x4_t w = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(tk, kr * kps + 16u * k_q, 0, 0));
      kraw[0] = w.x; kraw[1] = w.y; kraw[2] = w.z; kraw[3] = w.w;
    } else if constexpr (KB == 8) {
      const uint2 w = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(tk, kr * kps + 8u * k_q, 0, 0));
      kraw[0] = w.x; kraw[1] = w.y;
    } else {
      kraw[0] = __builtin_amdgcn_raw_buffer_load_b32(tk, kr * kps + 4u * k_q, 0, 0);
    }
    ksc = __builtin_amdgcn_raw_buffer_load_b16(tks, kr * kss2 + 2u * k_grp, 0, 0);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t vr = r0 + 4u * (uint32_t)v_kq + (uint32_t)i;
      if constexpr (VD == 8)
        vraw[i] = __builtin_amdgcn_raw_buffer_load_b32(tv, vr * vps + 4u * v_dq, 0, 0);
      else
        vraw[i] = __builtin_amdgcn_raw_buffer_load_b16(tv, vr * vps + 2u * v_dq, 0, 0);
      vsc[i] = __builtin_amdgcn_raw_buffer_load_b16(tvs, vr * vss2 + 2u * v_grp, 0, 0);
    }
  };
  // Dequantize: (n - 8) sc rounded once to fp32, then to the operand type.
  // With -8 sc exact (|sc| <= 2^125) that product is fma(n, sc, -8 sc), n
  // taken straight from a byte of nibbles (v_cvt_f32_ubyte): two
  // instructions an element. A wave holding a scale beyond 2^125 (or not
  // finite) writes the tile again with the direct product, in a function of
  // its own (inlined, a second copy of the tile code in the loop doubles the
  // registers the compiler holds across it).
  auto store_tile = [&](int buf) {
    uint16_t* k_dst = k_lds[buf] + k_key * KP + k_q * (2 * KB);
    uint16_t* v_dst = v_lds[buf] + (v_dq * VD) * VP + 4 * v_kq;
    const float ksf = scale_f32<S_F16>(ksc);
    bool wide = !(fabsf(ksf) <= 0x1p125f);
    // the nibble mask through an empty asm: with the constant visible the
    // compiler folds mask and byte select into a 4-bit extract, and then
    // converts byte 0 of that (two instructions, not one v_cvt_f32_ubyteN)
    uint32_t m4 = 0x0f0f0f0fu;
    asm volatile("" : "+s"(m4));
    {  // K row k_key, dims k_q * D / 4 .. + D / 4 (element 2j of a byte's pair in the low nibble)
      const float s8 = -8.0f * ksf;
      uint32_t pk[KB];
#pragma unroll
      for (int w = 0; w < KB / 4; ++w) {
        const uint32_t lo = kraw[w] & m4, hi = (kraw[w] >> 4) & m4;
#pragma unroll
        for (int j = 0; j < 4; ++j)
          pk[4 * w + j] = pack2<F16>(__builtin_fmaf((float)((lo >> (8 * j)) & 0xffu), ksf, s8),
                                     __builtin_fmaf((float)((hi >> (8 * j)) & 0xffu), ksf, s8));
      }
#pragma unroll
      for (int w = 0; w < KB / 4; ++w)
        *(uint4*)(k_dst + 8 * w) = make_uint4(pk[4 * w], pk[4 * w + 1], pk[4 * w + 2], pk[4 * w + 3]);
    }
    {  // V^T rows v_dq * VD + d, keys 4 v_kq .. + 3
      float vf[4][VD];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const float sc = scale_f32<S_F16>(vsc[i]);
        wide = wide || !(fabsf(sc) <= 0x1p125f);
        const float s8 = -8.0f * sc;
        const uint32_t lo = vraw[i] & m4, hi = (vraw[i] >> 4) & m4;
#pragma unroll
        for (int d = 0; d < VD; ++d)
          vf[i][d] = __builtin_fmaf((float)((((d & 1) ? hi : lo) >> (8 * (d >> 1))) & 0xffu), sc, s8);
      }
#pragma unroll
      for (int d = 0; d < VD; ++d)
        *(uint2*)(v_dst + d * VP) = make_uint2(pack2<F16>(vf[0][d], vf[1][d]), pack2<F16>(vf[2][d], vf[3][d]));
    }
    if (__builtin_amdgcn_ballot_w64(wide) != 0)
      store_tile_direct<D, F16, S_F16, KP, VP, KB, VD>(k_dst, v_dst,
                                                       make_uint4(kraw[0], kraw[KB / 4 > 1 ? 1 : 0],
                                                                  kraw[KB / 4 > 2 ? 2 : 0], kraw[KB / 4 > 2 ? 3 : 0]),
                                               ksc, make_uint4(vraw[0], vraw[1], vraw[2], vraw[3]),
                                               make_uint4(vsc[0], vsc[1], vsc[2], vsc[3]));
  };

  f32x4_t o[RB][NB];
  float m_run[RB], l_run[RB];
#pragma unroll
  for (int r = 0; r < RB; ++r) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) o[r][nb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    m_run[r] = kNegP;
    l_run[r] = 0.0f;
  }

  // Tile i's codes are loaded into registers during tile i - 2, dequantized
  // into buffer i % 2 during tile i - 1 (after that tile's S^T products are
  // issued, so the dequantize overlaps them) and read during tile i. One
  // barrier per tile: at its end every wave has read buffer i % 2 (written
  // again during tile i + 1) and written buffer (i + 1) % 2 (read during
  // tile i + 1).
  if (tile_lo < tile_hi) {
    load_tile((uint32_t)(tile_lo * kKeys));
    store_tile(0);
    if (tile_lo + 1 < tile_hi) load_tile((uint32_t)((tile_lo + 1) * kKeys));
  }
  __syncthreads();
  for (int tile = tile_lo; tile < tile_hi; ++tile) {
    const int t0 = tile * kKeys;
    const int cur = (tile - tile_lo) & 1;
    const uint16_t* kt = k_lds[cur];
    const uint16_t* vt = v_lds[cur];

    // ---- S^T = K Q^T, 4 blocks of 16 keys (block kb, row i: key
    //      32 (kb / 2) + 8 (i / 4) + 4 (kb % 2) + i % 4) ----
    f32x4_t st[RB][4];
#pragma unroll
    for (int kb = 0; kb < 4; ++kb) {
      const int krow = 32 * (kb >> 1) + 8 * (lq >> 2) + 4 * (kb & 1) + (lq & 3);
#pragma unroll
      for (int r = 0; r < RB; ++r) st[r][kb] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int kk = 0; kk < NK; ++kk) {
        const uint4 ka = *(const uint4*)(kt + krow * KP + 32 * kk + 8 * lg);
#pragma unroll
        for (int r = 0; r < RB; ++r) st[r][kb] = mfma32<F16>(ka, qf[r][kk], st[r][kb]);
      }
    }
    // the next tile into the other buffer while the products run
    if (tile + 1 < tile_hi) {
      store_tile(cur ^ 1);
      if (tile + 2 < tile_hi) load_tile((uint32_t)(t0 + 2 * kKeys));
    }
    // ---- online softmax (base 2) per query row; register j of block kb is
    //      key t = t0 + 32 (kb / 2) + 8 lg + 4 (kb % 2) + j. Only tiles where
    //      some row of the wave may not attend every key (the causal
    //      diagonal, the sequence's last partial tile) set the scores of the
    //      keys outside a row's range to -inf (weight exactly 0); the rest
    //      skip the per-key compares and selects. ----
    if (t0 + kKeys > lim_wave) {
#pragma unroll
      for (int r = 0; r < RB; ++r)
#pragma unroll
        for (int kb = 0; kb < 4; ++kb)
#pragma unroll
          for (int j = 0; j < 4; ++j)
            if (t0 + 32 * (kb >> 1) + 8 * lg + 4 * (kb & 1) + j >= lim[r]) st[r][kb][j] = -__builtin_inff();
    }
    uint2 pf[RB][4];
    float mt[RB];
    bool grow = false;
#pragma unroll
    for (int r = 0; r < RB; ++r) {
      float mx = st[r][0][0];
#pragma unroll
      for (int kb = 0; kb < 4; ++kb)
#pragma unroll
        for (int j = 0; j < 4; ++j) mx = fmaxf(mx, st[r][kb][j]);
      mx = fmaxf(mx, __shfl_xor(mx, 16));
      mx = fmaxf(mx, __shfl_xor(mx, 32));
      mt[r] = mx * c;  // -inf if no key of the tile is in the row's range
      grow = grow || mt[r] > m_run[r] + kLazyMaxP;
    }
    // lazy running max: the state is rescaled only in tiles where some row
    // of the wave outgrows its reference by more than kLazyMaxP (wave-uniform)
    if (__builtin_amdgcn_ballot_w64(grow) != 0) {
#pragma unroll
      for (int r = 0; r < RB; ++r) {
        const float m_new = fmaxf(m_run[r], mt[r]);
        const float alpha = __builtin_amdgcn_exp2f(m_run[r] - m_new);
        m_run[r] = m_new;
        l_run[r] *= alpha;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) o[r][nb] *= alpha;
      }
    }
#pragma unroll
    for (int r = 0; r < RB; ++r) {
#pragma unroll
      for (int kb = 0; kb < 4; ++kb) {
        float p[4];
#pragma unroll
        for (int j = 0; j < 4; ++j) {
          p[j] = __builtin_amdgcn_exp2f(__builtin_fmaf(st[r][kb][j], c, -m_run[r]));
          l_run[r] += p[j];
        }
        pf[r][kb] = make_uint2(pack2<F16>(p[0], p[1]), pack2<F16>(p[2], p[3]));
      }
    }
    // ---- O^T += V^T P^T, 32 keys per MFMA: keys 32 h + 8 lg .. + 7 ----
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint4 va = *(const uint4*)(vt + (16 * nb + lq) * VP + 32 * h + 8 * lg);
#pragma unroll
        for (int r = 0; r < RB; ++r) {
          const uint4 pb = make_uint4(pf[r][2 * h].x, pf[r][2 * h].y, pf[r][2 * h + 1].x, pf[r][2 * h + 1].y);
          o[r][nb] = mfma32<F16>(va, pb, o[r][nb]);
        }
      }
    __syncthreads();
  }

  // ---- normalise and store: lane (lq, lg) holds dims 16 nb + 4 lg .. + 3 ----
#pragma unroll
  for (int r = 0; r < RB; ++r) {
    float l_tot = l_run[r] + __shfl_xor(l_run[r], 16);
    l_tot += __shfl_xor(l_tot, 32);
    if (a.n_split > 1) {  // partial of this split, merged by prefill_merge_kernel
      const int rr = wave * kWaveRows * RB + 16 * r + lq;
      const int64_t slot = ((((int64_t)b * a.row_blocks + blk) * a.Hkv + kvh) * a.n_split + sp) * ROWS + rr;
      float* po = a.ws_o + slot * D;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        *(float4*)(po + 16 * nb + 4 * lg) = make_float4(o[r][nb][0], o[r][nb][1], o[r][nb][2], o[r][nb][3]);
      if (lg == 0) *(float2*)(a.ws_ml + 2 * slot) = make_float2(m_run[r], l_tot);
      continue;
    }
    const float inv = l_tot > 0.0f ? 1.0f / l_tot : 0.0f;
    if (row_ok[r]) {
      uint16_t* orow = a.out + (int64_t)b * a.os_b + (int64_t)head[r] * a.os_h + (int64_t)s[r] * a.os_s;
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const uint32_t w0 = pack2<F16>(o[r][nb][0] * inv, o[r][nb][1] * inv);
        const uint32_t w1 = pack2<F16>(o[r][nb][2] * inv, o[r][nb][3] * inv);
        uint16_t* p = orow + 16 * nb + 4 * lg;
        p[0] = (uint16_t)w0; p[1] = (uint16_t)(w0 >> 16);
        p[2] = (uint16_t)w1; p[3] = (uint16_t)(w1 >> 16);
      }
    }
  }
}

// Combines the n_split partials of one query row (log-sum-exp in base 2):
// one workgroup of D threads per (unit, row), thread d owns output dim d.
template <int D, bool F16>
__global__ __launch_bounds__(D) void prefill_merge_kernel(const PrefillArgs a, int rows) {
  const int64_t g = blockIdx.x;
  const int rr = (int)(g % rows);
  const int64_t unit = g / rows;  // (b * row_blocks + blk) * Hkv + kvh
  const int kvh = (int)(unit % a.Hkv);
  const int64_t t = unit / a.Hkv;
  const int blk = (int)(t % a.row_blocks);
  const int b = (int)(t / a.row_blocks);
  const int R = blk * rows + rr;
  const int s = R / a.ratio;
  if (s >= a.Sq) return;
  const int head = kvh * a.ratio + R % a.ratio;
  const int d = threadIdx.x;
  const int64_t slot0 = unit * a.n_split * rows + rr;  // split sp: slot0 + sp * rows
  float M = kNegP;
  for (int sp = 0; sp < a.n_split; ++sp) M = fmaxf(M, a.ws_ml[2 * (slot0 + (int64_t)sp * rows)]);
  float L = 0.0f, acc = 0.0f;
  for (int sp = 0; sp < a.n_split; ++sp) {
    const int64_t slot = slot0 + (int64_t)sp * rows;
    const float2 ml = *(const float2*)(a.ws_ml + 2 * slot);
    const float w = __builtin_amdgcn_exp2f(ml.x - M);
    L += ml.y * w;
    acc += a.ws_o[slot * D + d] * w;
  }
  const float v = L > 0.0f ? acc / L : 0.0f;
  uint16_t* orow = a.out + (int64_t)b * a.os_b + (int64_t)head * a.os_h + (int64_t)s * a.os_s;
  orow[d] = F16 ? (uint16_t)f32_to_f16_bits(v) : (uint16_t)f32_to_bf16_bits(v);
}

template <int D, bool F16, int RB, int NW>
void launch_prefill(const PrefillArgs& a, bool s_f16, dim3 grid, hipStream_t st) {
  const dim3 block(64 * NW);
  if (a.bt) {
    if (s_f16) hipLaunchKernelGGL((prefill_attn_kernel<D, F16, true, RB, true, NW>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((prefill_attn_kernel<D, F16, false, RB, true, NW>), grid, block, 0, st, a);
  } else {
    if (s_f16) hipLaunchKernelGGL((prefill_attn_kernel<D, F16, true, RB, false, NW>), grid, block, 0, st, a);
    else hipLaunchKernelGGL((prefill_attn_kernel<D, F16, false, RB, false, NW>), grid, block, 0, st, a);
  }
}

template <int D, bool F16>
void launch_prefill_rb(const PrefillArgs& a, bool s_f16, int rb, int nw, dim3 grid, hipStream_t st) {
  if constexpr (D == 128) {
    if (nw == 8) launch_prefill<D, F16, 2, 8>(a, s_f16, grid, st);
    else if (rb == 2) launch_prefill<D, F16, 2, 4>(a, s_f16, grid, st);
    else launch_prefill<D, F16, 1, 4>(a, s_f16, grid, st);
  } else {
    if (rb == 2) launch_prefill<D, F16, 2, 4>(a, s_f16, grid, st);
    else launch_prefill<D, F16, 1, 4>(a, s_f16, grid, st);
  }
  if (a.n_split > 1) {
    const int rows = kWaveRows * nw * rb;
    const int64_t n = (int64_t)grid.x / a.n_split * rows;
    hipLaunchKernelGGL((prefill_merge_kernel<D, F16>), dim3((unsigned)n), dim3(D), 0, st, a, rows);
  }
}

// Launch plan: waves per workgroup (nw), rows per workgroup (nw waves of rb
// 16-row blocks), row blocks, and the split over keys. Two row blocks per
// wave once that still gives a workgroup of four waves per CU of a 256-CU
// device. D = 128 with two row blocks takes eight waves per workgroup (one
// workgroup of 256 rows per CU) once that still gives a workgroup per CU.
// Below 512 workgroups of four waves (two per CU), splits of at least 512
// keys bring the launch to ~512.
struct PrefillPlan {
  int rb, nw, n_split;
  int64_t row_blocks;
};

PrefillPlan prefill_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t Sk, int64_t D) {
  const int64_t ratio = Hq / Hkv;
  const int64_t rows = Sq * ratio;
  PrefillPlan p;
  p.rb = B * Hkv * ((rows + 8 * kWaveRows - 1) / (8 * kWaveRows)) >= 256 ? 2 : 1;
  p.nw = (D == 128 && p.rb == 2 && B * Hkv * ((rows + 16 * kWaveRows - 1) / (16 * kWaveRows)) >= 256) ? 8 : 4;
  const int64_t wg_rows = kWaveRows * p.nw * p.rb;
  p.row_blocks = (rows + wg_rows - 1) / wg_rows;
  const int64_t n_wg = B * Hkv * p.row_blocks;
  int64_t ns = 1;
  if (p.nw == 4 && n_wg > 0 && n_wg < 512) {
    ns = (512 + n_wg - 1) / n_wg;
    ns = std::min<int64_t>(ns, std::max<int64_t>(1, Sk / 512));
    ns = std::min<int64_t>(ns, 64);
  }
  p.n_split = (int)ns;
  return p;
}

int64_t prefill_ws_bytes(const PrefillPlan& p, int64_t B, int64_t Hkv, int64_t D) {
  if (p.n_split <= 1) return 0;
  return B * Hkv * p.row_blocks * p.n_split * (kWaveRows * p.nw * p.rb) * (D + 2) * 4;
}

}  // namespace
}  // namespace kvq

using namespace kvq;

namespace {

struct PrefillPaged {
  const int32_t* bt;
  int64_t bt_stride, bt_cols, n_blocks, page_size;
};

// Shared by the contiguous and paged entry points. Strides are [3] (batch,
// head, row); the paged entry point passes batch strides of 0.
int prefill_impl(const void* q, int q_dtype, const int64_t* q_strides, const void* k_packed,
                 const int64_t* kp_strides, const void* k_scales, const int64_t* ks_strides,
                 const void* v_packed, const int64_t* vp_strides, const void* v_scales,
                 const int64_t* vs_strides, int scale_dtype, void* out, const int64_t* out_strides, int64_t B,
                 int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D, int64_t group_size, int64_t Sk,
                 int is_causal, float sm_scale, void* workspace, int64_t workspace_bytes, void* stream,
                 const PrefillPaged* pg) {
  KVQ_CHECK_ARG(q_strides && out_strides, "kvq_prefill_attn: null stride array");
  KVQ_CHECK_ARG(B >= 0 && Hq >= 1 && Hkv >= 1 && Sq >= 0 && Sk >= 0 && Hq % Hkv == 0,
                "kvq_prefill_attn: bad shape (B=%lld Hq=%lld Hkv=%lld Sq=%lld Sk=%lld)", (long long)B,
                (long long)Hq, (long long)Hkv, (long long)Sq, (long long)Sk);
  if (!((q_dtype == KVQ_BF16 || q_dtype == KVQ_F16) && (scale_dtype == KVQ_BF16 || scale_dtype == KVQ_F16))) {
    set_error("kvq_prefill_attn: bf16/fp16 queries and scales only");
    return KVQ_EUNSUP;
  }
  const int64_t ratio = Hq / Hkv;
  if (!(D == 64 || D == 128) || !(group_size == 32 || group_size == 64 || group_size == 128) ||
      D % group_size != 0 || 64 % ratio != 0) {
    set_error("kvq_prefill_attn: unsupported shape (D=%lld G=%lld Hq/Hkv=%lld)", (long long)D,
              (long long)group_size, (long long)ratio);
    return KVQ_EUNSUP;
  }
  if (q_strides[3] != 1 || out_strides[3] != 1) {
    set_error("kvq_prefill_attn: q and out rows must be contiguous");
    return KVQ_EUNSUP;
  }
  KVQ_CHECK_ARG(kp_strides[2] >= D / 2 && vp_strides[2] >= D / 2 && ks_strides[2] >= D / group_size &&
                    vs_strides[2] >= D / group_size,
                "kvq_prefill_attn: cache rows narrower than D / 2 code bytes or D / G scales");
  // rows addressed through one buffer: a (batch, head) slice, or a head's pool
  const int64_t rows_addr = pg ? pg->n_blocks * pg->page_size : Sk;
  if (rows_addr * kp_strides[2] >= (1ll << 31) || rows_addr * vp_strides[2] >= (1ll << 31) ||
      rows_addr * ks_strides[2] * 2 >= (1ll << 31) || rows_addr * vs_strides[2] * 2 >= (1ll << 31)) {
    set_error("kvq_prefill_attn: a (batch, head) slice of the cache (or a head's pool) exceeds 2 GiB");
    return KVQ_EUNSUP;
  }
  int page_shift = 0;
  if (pg) {
    KVQ_CHECK_ARG(pg->page_size >= 64 && (pg->page_size & (pg->page_size - 1)) == 0 && pg->page_size <= (1 << 20),
                  "kvq_prefill_attn_paged: page_size must be a power of two >= 64 (got %lld)",
                  (long long)pg->page_size);
    KVQ_CHECK_ARG(pg->n_blocks >= 0 && pg->n_blocks < (1ll << 31) && pg->bt_cols >= 0 && pg->bt_cols < (1ll << 31) &&
                      pg->bt_stride >= pg->bt_cols && Sk <= pg->bt_cols * pg->page_size,
                  "kvq_prefill_attn_paged: bad block table geometry or Sk past the table");
    KVQ_CHECK_ARG(pg->bt != nullptr || pg->bt_cols == 0 || B == 0, "kvq_prefill_attn_paged: null block table");
    while ((int64_t(1) << page_shift) < pg->page_size) ++page_shift;
  }
  if (B == 0 || Sq == 0) return KVQ_OK;
  KVQ_CHECK_ARG(q && out && (Sk == 0 || (k_packed && k_scales && v_packed && v_scales)),
                "kvq_prefill_attn: null data pointer");
  PrefillPlan plan = prefill_plan(B, Hq, Hkv, Sq, Sk, D);
  // the split over keys needs the workspace; without one the launch is unsplit
  const int64_t need = prefill_ws_bytes(plan, B, Hkv, D);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) plan.n_split = 1;
  const int rb = plan.rb;
  const int64_t row_blocks = plan.row_blocks;
  const int64_t n_wg = B * Hkv * row_blocks * plan.n_split;
  KVQ_CHECK_ARG(n_wg < (1ll << 31) && Sq < (1ll << 30) && Sk < (1ll << 30), "kvq_prefill_attn: too large");

  PrefillArgs a;
  a.q = (const uint16_t*)q;
  a.qs_b = q_strides[0]; a.qs_h = q_strides[1]; a.qs_s = q_strides[2];
  a.kp = (const uint8_t*)k_packed;
  a.kps_b = kp_strides[0]; a.kps_h = kp_strides[1]; a.kps_s = kp_strides[2];
  a.ks = (const uint16_t*)k_scales;
  a.kss_b = ks_strides[0]; a.kss_h = ks_strides[1]; a.kss_s = ks_strides[2];
  a.vp = (const uint8_t*)v_packed;
  a.vps_b = vp_strides[0]; a.vps_h = vp_strides[1]; a.vps_s = vp_strides[2];
  a.vs = (const uint16_t*)v_scales;
  a.vss_b = vs_strides[0]; a.vss_h = vs_strides[1]; a.vss_s = vs_strides[2];
  a.out = (uint16_t*)out;
  a.os_b = out_strides[0]; a.os_h = out_strides[1]; a.os_s = out_strides[2];
  a.Hkv = (int)Hkv; a.ratio = (int)ratio; a.Sq = (int)Sq; a.Sk = (int)Sk; a.G = (int)group_size;
  a.row_blocks = (int)row_blocks; a.causal = is_causal ? 1 : 0;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  // a paged call with no table columns maps no key: it runs as an empty cache
  a.bt = (pg && pg->bt_cols > 0) ? pg->bt : nullptr;
  a.bt_stride = pg ? pg->bt_stride : 0;
  a.bt_cols = pg ? (int)pg->bt_cols : 0;
  a.n_blocks = pg ? (int)pg->n_blocks : 0;
  a.page_shift = page_shift;
  if (pg && pg->bt_cols == 0) a.Sk = 0;
  a.n_split = plan.n_split;
  a.ws_o = plan.n_split > 1 ? (float*)workspace : nullptr;
  a.ws_ml = plan.n_split > 1 ? (float*)workspace + B * Hkv * row_blocks * plan.n_split * (kWaveRows * plan.nw * rb) * D
                              : nullptr;

  const dim3 grid((unsigned)n_wg);
  hipStream_t st = (hipStream_t)stream;
  const bool f16 = q_dtype == KVQ_F16, s_f16 = scale_dtype == KVQ_F16;
  if (D == 128) {
    if (f16) launch_prefill_rb<128, true>(a, s_f16, rb, plan.nw, grid, st);
    else launch_prefill_rb<128, false>(a, s_f16, rb, plan.nw, grid, st);
  } else {
    if (f16) launch_prefill_rb<64, true>(a, s_f16, rb, plan.nw, grid, st);
    else launch_prefill_rb<64, false>(a, s_f16, rb, plan.nw, grid, st);
  }
  KVQ_CHECK_LAUNCH("kvq_prefill_attn");
  return KVQ_OK;
}

}  // namespace

extern "C" int kvq_prefill_attn(const void* q, int q_dtype, const int64_t* q_strides,
                                const void* k_packed, const int64_t* kp_strides,
                                const void* k_scales, const int64_t* ks_strides,
                                const void* v_packed, const int64_t* vp_strides,
                                const void* v_scales, const int64_t* vs_strides,
                                int scale_dtype,
                                void* out, const int64_t* out_strides,
                                int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                                int64_t group_size, int64_t Sk, int is_causal, float sm_scale,
                                void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  KVQ_CHECK_ARG(kp_strides && ks_strides && vp_strides && vs_strides, "kvq_prefill_attn: null stride array");
  return prefill_impl(q, q_dtype, q_strides, k_packed, kp_strides, k_scales, ks_strides, v_packed, vp_strides,
                      v_scales, vs_strides, scale_dtype, out, out_strides, B, Hq, Hkv, Sq, D, group_size, Sk,
                      is_causal, sm_scale, workspace, workspace_bytes, stream, nullptr);
}

extern "C" int64_t kvq_prefill_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                                                    int64_t Sk) {
  clear_error();
  if (B < 0 || Hq < 1 || Hkv < 1 || Sq < 0 || Sk < 0 || Hq % Hkv != 0 || !(D == 64 || D == 128)) {
    set_error("kvq_prefill_attn_workspace_bytes: bad shape");
    return KVQ_EINVAL;
  }
  if (B == 0 || Sq == 0) return 0;
  return prefill_ws_bytes(prefill_plan(B, Hq, Hkv, Sq, Sk, D), B, Hkv, D);
}

extern "C" int kvq_prefill_attn_paged(const void* q, int q_dtype, const int64_t* q_strides,
                                      const void* k_pool, const int64_t* kp_strides,
                                      const void* k_scale_pool, const int64_t* ks_strides,
                                      const void* v_pool, const int64_t* vp_strides,
                                      const void* v_scale_pool, const int64_t* vs_strides,
                                      int scale_dtype,
                                      const int32_t* block_table, int64_t table_stride,
                                      int64_t table_cols, int64_t num_blocks, int64_t page_size,
                                      void* out, const int64_t* out_strides,
                                      int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                                      int64_t group_size, int64_t Sk, int is_causal, float sm_scale,
                                      void* workspace, int64_t workspace_bytes, void* stream) {
  clear_error();
  KVQ_CHECK_ARG(kp_strides && ks_strides && vp_strides && vs_strides, "kvq_prefill_attn_paged: null stride array");
  const int64_t kp3[3] = {0, kp_strides[0], kp_strides[1]}, ks3[3] = {0, ks_strides[0], ks_strides[1]};
  const int64_t vp3[3] = {0, vp_strides[0], vp_strides[1]}, vs3[3] = {0, vs_strides[0], vs_strides[1]};
  const PrefillPaged pg{block_table, table_stride, table_cols, num_blocks, page_size};
  return prefill_impl(q, q_dtype, q_strides, k_pool, kp3, k_scale_pool, ks3, v_pool, vp3, v_scale_pool, vs3,
                      scale_dtype, out, out_strides, B, Hq, Hkv, Sq, D, group_size, Sk, is_causal, sm_scale,
                      workspace, workspace_bytes, stream, &pg);
}
