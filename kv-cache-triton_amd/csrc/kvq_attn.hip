// Fused INT4-KV GQA decode attention for gfx950 (CDNA4, wave64).
//
// Replaces the reference's fused kernels
//   kernels/llama3/attention_quant.py:24-152 (_attention_fwd_quant_gqa_kernel)
//   kernels/gpt2/attention_quant.py:12-137   (_attention_fwd_quant_kernel, MHA)
// for short query blocks. The reference runs one program per *query* head and
// walks the sequence serially (kv = h // ratio, :71; tile loop :104), so K/V
// are re-read once per GQA group member and only B*Hq programs exist. Here one
// workgroup owns one (batch, kv head, query-row chunk) and one slice of the
// sequence (split-K): every query head of the GQA group (times the Sq query
// positions) is a "row" processed against the same K/V bytes, so each cache
// byte crosses HBM once, and B*Hkv*n_split workgroups fill the CUs. Partial
// (max, sum, o) triples are merged across the 4 waves of a workgroup in LDS and
// then across splits by the last workgroup of the unit (device-scope counter),
// which writes the output.
//
// Two kernels share that frame:
//
// decode_attn_mfma_kernel (bf16 / fp16 queries, 16-bit scales) puts both
//   products on the matrix cores with v_mfma_f32_4x4x4_{bf16,f16}: 16
//   independent 4x4 blocks per instruction.
//   * QK: lane l owns token l of a 64-token tile. A = 4 query rows (lane l%4
//     holds row l%4), B = 4 dims of the lane's token, D = that token's scores
//     for the 4 rows. One accumulator per 32-dim chunk, so the per-(token,
//     group) key scale is applied once per chunk afterwards.
//   * PV: lane (token subset ts, dim block j) holds codes of 4 tokens x 1 dim
//     per instruction (B) and reads A = softmax weights w = p * v_scale of 4
//     rows x the same 4 tokens from LDS. All 4 lanes of a block share one
//     32-dim chunk, so the per-chunk value scale rides in A.
//   The VALU only converts nibbles to bf16/fp16 and runs the softmax.
// decode_attn_valu_kernel (fp32 queries or fp32 scales) keeps exact fp32
//   arithmetic (v_fmac) for the 1e-4 bar of fp32 inputs; MHA-sized row counts.
//
// Nibble -> number: a magic-number OR makes an exact float of 128 + n (bf16,
// 0x4300 | n) or 1024 + n (fp16, 0x6400 | n).
//   bf16: scores accumulate q*(128+n) on top of an initial -136*sum(q) per
//         chunk; values accumulate w*(128+n) and subtract 136*sum(w) at the
//         end, sum(w) coming from one extra MFMA on the same rounded weights.
//   fp16: (1024+n) - 1032 = n - 8 exactly (v_pk_add_f16), no correction.
// Softmax runs in base 2 with sm_scale*log2(e) folded into the key scale.
#include <algorithm>
#include <type_traits>

#include "kvq_common.h"

namespace kvq {

struct AttnArgs {
  const void* q;
  int64_t qs_b, qs_h, qs_s, qs_d;
  const uint8_t* kp;
  int64_t kps_b, kps_h, kps_s;
  const void* ks;
  int64_t kss_b, kss_h, kss_s;
  const uint8_t* vp;
  int64_t vps_b, vps_h, vps_s;
  const void* vs;
  int64_t vss_b, vss_h, vss_s;
  void* out;
  int64_t os_b, os_h, os_s, os_d;
  const int32_t* seq_lens;
  int Hkv, Sq, G, Sk, ratio, rows_total, row_chunks, n_units;
  int n_split, split_len, causal, scale_dtype, xcd_remap, q_vec;
  float scale_log2;
  float* ws_ml;  // [n_units][n_split][ROWS][2]  (max, sum)
  float* ws_o;   // [n_units][n_split][ROWS][D]
};

constexpr float kNeg = -1.0e30f;
constexpr int kMaxSplit = 64;  // split-K fan-out cap (bounds the merge's LDS)
constexpr uint32_t kNibPairs = 0x000F000Fu;
constexpr uint32_t kBf16Magic = 0x43004300u;  // bf16(128), bf16(128)
constexpr uint32_t kF16Magic = 0x64006400u;   // fp16(1024), fp16(1024)
constexpr uint32_t kBf16OnePair = 0x3F803F80u;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c,
                                false);
}

// One v_mfma_f32_4x4x4 on operands given as two packed dwords each:
// A = {a0, a1} (4 x 16-bit), B = {b0, b1}.
template <bool F16>
__device__ __forceinline__ f32x4_t mfma4(uint32_t a0, uint32_t a1, uint32_t b0, uint32_t b1,
                                         f32x4_t c) {
  const uint2 av = make_uint2(a0, a1), bv = make_uint2(b0, b1);
  if constexpr (F16) {
    return __builtin_amdgcn_mfma_f32_4x4x4f16(__builtin_bit_cast(f16x4_t, av),
                                              __builtin_bit_cast(f16x4_t, bv), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_4x4x4bf16_1k(__builtin_bit_cast(s16x4_t, av),
                                                  __builtin_bit_cast(s16x4_t, bv), c, 0, 0, 0);
  }
}

template <int CTRL, int ROW_MASK = 0xF>
__device__ __forceinline__ float dpp(float v, float old) {
  return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(__builtin_bit_cast(int, old),
                                                               __builtin_bit_cast(int, v), CTRL,
                                                               ROW_MASK, 0xF, false));
}

// Full-wave reductions; the result is read from lane 63 and is wave-uniform.
__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp<0x111>(v, kNeg));  // row_shr:1
  v = fmaxf(v, dpp<0x112>(v, kNeg));  // row_shr:2
  v = fmaxf(v, dpp<0x114>(v, kNeg));  // row_shr:4
  v = fmaxf(v, dpp<0x118>(v, kNeg));  // row_shr:8
  v = fmaxf(v, dpp<0x142, 0xA>(v, kNeg));  // row_bcast:15
  v = fmaxf(v, dpp<0x143, 0xC>(v, kNeg));  // row_bcast:31
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}
__device__ __forceinline__ float wave_sum(float v) {
  v += dpp<0x111>(v, 0.0f);
  v += dpp<0x112>(v, 0.0f);
  v += dpp<0x114>(v, 0.0f);
  v += dpp<0x118>(v, 0.0f);
  v += dpp<0x142, 0xA>(v, 0.0f);
  v += dpp<0x143, 0xC>(v, 0.0f);
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), 63));
}

// 16-bit scale -> fp32 without a branch (both decodings, then a select).
__device__ __forceinline__ float scale16_to_f32(uint32_t h, bool is_f16) {
  const float fb = bf16_bits_to_f32(h);
  const float fh = f16_bits_to_f32(h);
  return is_f16 ? fh : fb;
}

// Scale at element offset `off` of a per-(batch, head) base pointer (any dtype).
__device__ __forceinline__ float load_scale(const char* base, uint32_t off, int dt) {
  if (dt == KVQ_F32) return ((const float*)base)[off];
  return scale16_to_f32(((const uint16_t*)base)[off], dt == KVQ_F16);
}

// Workgroup -> (unit, split). With XCD remapping all splits of one unit run on
// the same XCD (workgroups are dealt to the 8 XCDs round-robin), so the split
// merge reads partials written through the same L2.
__device__ __forceinline__ void unit_and_split(const AttnArgs& a, int& unit, int& split) {
  const int j = blockIdx.x;
  if (a.xcd_remap) {
    const int xcd = j & 7, local = j >> 3;
    unit = xcd + 8 * (local / a.n_split);
    split = local % a.n_split;
  } else {
    unit = j / a.n_split;
    split = j % a.n_split;
  }
}

__device__ __forceinline__ int64_t out_index(const AttnArgs& a, int b, int kvh, int rho, int d) {
  const int head = kvh * a.ratio + rho / a.Sq, qi = rho % a.Sq;
  return (int64_t)b * a.os_b + (int64_t)head * a.os_h + (int64_t)qi * a.os_s + (int64_t)d * a.os_d;
}

struct MergeLds {
  float l[8];
  float m[8];
  float wf[8][8];  // per-wave rescale factors 2^(m_wave - M)
};

// Merge the partials of the NW waves — NW * PPW partial slots in o_lds, slot p
// belonging to wave p / PPW, with (max, sum) per wave in ml_lds; the caller
// has already passed a barrier — and store either the output (single split) or
// this split's partial (max, sum, o) for decode_attn_merge_kernel.
template <int ROWS, int D, int OUT_DT, int NW, int PPW>
__device__ __forceinline__ void finish_block(const AttnArgs& a, int unit, int split, int rc,
                                             int kvh, int b, const float (*o_lds)[ROWS][D],
                                             const float (*ml_lds)[ROWS][2], MergeLds& mg) {
  constexpr int NP = NW * PPW;
  const int tid = threadIdx.x;
  const bool single = a.n_split == 1;
  if (tid < ROWS) {
    float M = kNeg;
#pragma unroll
    for (int w = 0; w < NW; ++w) M = fmaxf(M, ml_lds[w][tid][0]);
    float Ls = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __builtin_amdgcn_exp2f(ml_lds[w][tid][0] - M);
      mg.wf[w][tid] = f;
      Ls += ml_lds[w][tid][1] * f;
    }
    mg.l[tid] = Ls;
    mg.m[tid] = M;
  }
  __syncthreads();
  for (int idx = tid; idx < ROWS * D; idx += 64 * NW) {
    const int r = idx / D, d = idx % D;
    float Os = 0.0f;
#pragma unroll
    for (int p = 0; p < NP; ++p) Os = fmaf(o_lds[p][r][d], mg.wf[p / PPW][r], Os);
    const float Ls = mg.l[r];
    const int rho = rc * ROWS + r;
    if (single) {
      if (rho < a.rows_total)
        store_from_f32(a.out, out_index(a, b, kvh, rho, d), OUT_DT, Ls > 0.0f ? Os / Ls : 0.0f);
    } else {
      const int64_t slot = ((int64_t)unit * a.n_split + split) * ROWS + r;
      a.ws_o[slot * D + d] = Os;
      if (d == 0) {
        a.ws_ml[slot * 2 + 0] = mg.m[r];
        a.ws_ml[slot * 2 + 1] = Ls;
      }
    }
  }
}

// Split-K merge, launched after the attention kernel on the same stream (the
// kernel boundary orders the partials' stores before these loads). One thread
// per (unit, row, dim): out = sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s,
// M = max_s m_s, over the n_split partials, BATCH of them per round of loads.
// A row no split saw a key for (all l_s = 0) yields zeros.
template <int OUT_DT>
__global__ __launch_bounds__(128) void decode_attn_merge_kernel(const AttnArgs a, int rows, int D) {
  constexpr int BATCH = 32;
  const int64_t gid = (int64_t)blockIdx.x * 128 + threadIdx.x;
  if (gid >= (int64_t)a.n_units * rows * D) return;
  const int d = (int)(gid % D);
  const int64_t ur = gid / D;
  const int r = (int)(ur % rows);
  const int unit = (int)(ur / rows);
  const int rc = unit % a.row_chunks;
  const int bh = unit / a.row_chunks;
  const int kvh = bh % a.Hkv, b = bh / a.Hkv;
  const int rho = rc * rows + r;
  if (rho >= a.rows_total) return;
  const int64_t slot0 = (int64_t)unit * a.n_split * rows + r;  // + split * rows
  const float2* ml2 = (const float2*)a.ws_ml + slot0;
  const float* ob = a.ws_o + slot0 * D + d;
  const int64_t o_step = (int64_t)rows * D;
  float M = kNeg, Ls = 0.0f, acc = 0.0f;
  for (int sp0 = 0; sp0 < a.n_split; sp0 += BATCH) {
    float2 ml[BATCH];
    float ov[BATCH];
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const int64_t sp = min(sp0 + j, a.n_split - 1);
      ml[j] = ml2[sp * rows];
      ov[j] = ob[sp * o_step];
    }
    float Mb = M;
#pragma unroll
    for (int j = 0; j < BATCH; ++j)
      if (sp0 + j < a.n_split) Mb = fmaxf(Mb, ml[j].x);
    const float f = __builtin_amdgcn_exp2f(M - Mb);
    Ls *= f;
    acc *= f;
    M = Mb;
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      if (sp0 + j < a.n_split) {
        const float w = __builtin_amdgcn_exp2f(ml[j].x - M);
        Ls = fmaf(ml[j].y, w, Ls);
        acc = fmaf(ov[j], w, acc);
      }
    }
  }
  store_from_f32(a.out, out_index(a, b, kvh, rho, d), OUT_DT, Ls > 0.0f ? acc / Ls : 0.0f);
}

// ===========================================================================
// MFMA kernel: bf16 / fp16 queries, 16-bit scales, D in {64, 128},
// RS row sets of 4 rows (ROWS = 4 * RS), tiles of 64 tokens per wave.
//
// Nibbles become MFMA operands with one v_perm_b32 per output dword: with
// lo = w & 0x0F0F0F0F (bytes = elements 0,2,4,6 of a code dword) and
// hi = (w >> 4) & 0x0F0F0F0F (elements 1,3,5,7), perm(MAGIC, lo, sel) builds
// {0x43 | lo.byte_i, 0x43 | lo.byte_j} pairs = bf16(128 + n) (fp16: 0x64 ->
// 1024 + n). Key dword k therefore feeds the MFMA k-order (0,2,1,3) and
// (4,6,5,7); the staged query rows are permuted the same way.

// Buffer descriptor over `bytes` bytes at p (raw, 32-bit data format): loads
// at offsets >= bytes return zero and touch no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           0x00020000);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

template <int D, int RS, int QM, bool ROWMASK, int NW>
__global__ __launch_bounds__(64 * NW) void decode_attn_mfma_kernel(const AttnArgs a) {
  constexpr bool F16 = QM == KVQ_F16;
  constexpr int LPT = D / 32;     // 32-dim chunks per token
  constexpr int VLPT = D / 8;     // V lanes per token row (one dword each)
  constexpr int VTS = 64 / VLPT;  // V token subsets
  constexpr int SUB = 4 * VTS;    // tokens per V sub-tile
  constexpr int NSUB = 64 / SUB;  // V sub-tiles per 64-token tile
  constexpr int CH = NW == 8 ? 1 : 2;  // tiles per wave per chunk (all their loads in flight)
  constexpr int ROWS = 4 * RS;
  constexpr int QT = ROWS * D / 8;  // threads staging the query rows, 8 elements each
  constexpr uint32_t MAGIC = F16 ? 0x64646464u : 0x43434343u;
  constexpr uint32_t NEG_BIAS = F16 ? 0xE408E408u : 0xC308C308u;  // {-1032, -1032} / {-136, -136}
  constexpr uint32_t SEL_02 = 0x04010400u;  // {MAGIC | byte0, MAGIC | byte1}
  constexpr uint32_t SEL_46 = 0x04030402u;  // {MAGIC | byte2, MAGIC | byte3}
  static_assert(QT <= 64 * NW, "query staging");

  __shared__ __attribute__((aligned(16))) uint32_t q_lds[ROWS][D / 2];
  // softmax weights, per wave: [tile][rowset][row][chunk][subtile][tsub][4 tokens]
  __shared__ __attribute__((aligned(16))) uint16_t w_lds[NW][CH][RS][4][LPT][NSUB][VTS][4];
  // partial outputs, one slot per (wave, token subset)
  __shared__ __attribute__((aligned(16))) float o_lds[NW * VTS][ROWS][D];
  __shared__ float ml_lds[NW][ROWS][2];
  __shared__ MergeLds mg;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int unit, split;
  unit_and_split(a, unit, split);
  const int rc = unit % a.row_chunks;
  const int bh = unit / a.row_chunks;
  const int kvh = bh % a.Hkv;
  const int b = bh / a.Hkv;

  int L = a.Sk;
  if (a.seq_lens) {
    const int sl = a.seq_lens[b];
    L = sl < 0 ? 0 : (sl < a.Sk ? sl : a.Sk);
  }
  const int t_begin = split * a.split_len;
  const int t_end = min(t_begin + a.split_len, L);
  const int ntiles = t_end > t_begin ? (t_end - t_begin + 63) / 64 : 0;

  // ---- query staging loads go out first: thread (q_r, q_k) of every wave
  //      reads elements [8 q_k, 8 q_k + 8) of row q_r with 16-bit loads (no
  //      branch, so the compiler can wait for them alone later); rows past
  //      the last one read row 0 and are zeroed ----
  const int q_r = (tid % QT) / (D / 8), q_k = tid % (D / 8);
  const int q_rho = rc * ROWS + q_r;
  const bool q_ok = q_rho < a.rows_total;
  uint32_t qe[8];
  {
    const int rho = q_ok ? q_rho : 0;
    const int head = kvh * a.ratio + rho / a.Sq, qi = rho % a.Sq;
    const uint16_t* q16 = (const uint16_t*)a.q +
                          ((int64_t)b * a.qs_b + (int64_t)head * a.qs_h + (int64_t)qi * a.qs_s +
                           (int64_t)(8 * q_k) * a.qs_d);
#pragma unroll
    for (int j = 0; j < 8; ++j) qe[j] = q16[(int64_t)j * a.qs_d];
  }
  __builtin_amdgcn_sched_barrier(0);  // keep the query loads ahead of the cache loads

  // ---- cache slices as bounds-checked buffers (rows >= L read as zero) ----
  const uint8_t* kp_bh = a.kp + (int64_t)b * a.kps_b + (int64_t)kvh * a.kps_h;
  const uint8_t* vp_bh = a.vp + (int64_t)b * a.vps_b + (int64_t)kvh * a.vps_h;
  const uint16_t* ks_bh = (const uint16_t*)a.ks + ((int64_t)b * a.kss_b + (int64_t)kvh * a.kss_h);
  const uint16_t* vs_bh = (const uint16_t*)a.vs + ((int64_t)b * a.vss_b + (int64_t)kvh * a.vss_h);
  const uint32_t kps = (uint32_t)a.kps_s, vps = (uint32_t)a.vps_s;
  const uint32_t kss2 = 2u * (uint32_t)a.kss_s, vss2 = 2u * (uint32_t)a.vss_s;
  const uint32_t Lu = (uint32_t)L;
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kp_bh, Lu * kps);
  const __amdgpu_buffer_rsrc_t rks = buffer_rsrc(ks_bh, Lu * kss2);
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(vp_bh, Lu * vps);
  const __amdgpu_buffer_rsrc_t rvs = buffer_rsrc(vs_bh, Lu * vss2);
  const bool s_f16 = a.scale_dtype == KVQ_F16;
  uint32_t goff[LPT];  // byte offset of each 32-dim chunk's scale in a row
#pragma unroll
  for (int c = 0; c < LPT; ++c) goff[c] = 2u * (uint32_t)((c * 32) / a.G);

  // V lane layout and the LDS slot this lane's token fills
  const int vts = lane / VLPT;
  const int vj = lane % VLPT;
  const int v_row = vj & 3;   // A-operand row of this lane's block
  const int v_chunk = vj >> 2;
  const int w_sub = lane / SUB;             // sub-tile of token `lane`
  const int w_ts = (lane % SUB) % VTS;      // its token subset
  const int w_k = (lane % SUB) / VTS;       // its position in the subset

  // Chunk registers (CH tiles of 64 tokens). Tile i of a chunk is computed
  // start to finish before tile i + 1, and each of its parts is refilled for
  // the next chunk as soon as it is consumed, so loads overlap the math.
  u32x4_t kc4[CH][LPT];
  uint32_t skr[CH][LPT], svr[CH][LPT];
  uint32_t vcode[CH][NSUB][4];
  // Loads are never behind a branch (the compiler's wait counting stays exact
  // across them); a load that is not needed gets an offset past every buffer
  // (kOob) and returns zero without touching memory.
  constexpr uint32_t kOob = 0x80000000u;
  auto load_k = [&](int i, int base, bool live) {
    const uint32_t t = (uint32_t)(t_begin + (base + NW * i) * 64 + lane);
    const uint32_t ko = live ? t * kps : kOob, so = live ? t * kss2 : kOob;
#pragma unroll
    for (int c = 0; c < LPT; ++c) {
      kc4[i][c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(rk, ko + 16u * c, 0, 0));
      skr[i][c] = __builtin_amdgcn_raw_buffer_load_b16(rks, so + goff[c], 0, 0);
    }
  };
  auto load_vs = [&](int i, int base, bool live) {
    const uint32_t so = live ? (uint32_t)(t_begin + (base + NW * i) * 64 + lane) * vss2 : kOob;
#pragma unroll
    for (int c = 0; c < LPT; ++c) svr[i][c] = __builtin_amdgcn_raw_buffer_load_b16(rvs, so + goff[c], 0, 0);
  };
  auto load_v = [&](int i, int base, bool live) {
    const uint32_t vo = live ? (uint32_t)(t_begin + (base + NW * i) * 64 + vts) * vps + 4u * vj : kOob;
#pragma unroll
    for (int s = 0; s < NSUB; ++s) {
#pragma unroll
      for (int k = 0; k < 4; ++k)
        vcode[i][s][k] = __builtin_amdgcn_raw_buffer_load_b32(rv, vo + (uint32_t)(s * SUB + VTS * k) * vps, 0, 0);
    }
  };
  auto load_tile = [&](int i, int base, bool live) {
    load_k(i, base, live);
    load_vs(i, base, live);
    load_v(i, base, live);
  };
  // With one row set the first chunk's loads go out before the query is
  // processed; two row sets have no registers to spare for that and load each
  // chunk at the top of the loop.
  constexpr bool PIPE = RS == 1;
  if constexpr (PIPE) {
#pragma unroll
    for (int i = 0; i < CH; ++i) load_tile(i, wave, wave + NW * i < ntiles);
  }

  // ---- query rows -> LDS, permuted to the key operand order ----
  if (tid < QT) {
    const uint32_t keep = q_ok ? 0xffffu : 0u;
    const u32x4_t qp = {(qe[0] & keep) | ((qe[2] & keep) << 16), (qe[1] & keep) | ((qe[3] & keep) << 16),
                        (qe[4] & keep) | ((qe[6] & keep) << 16), (qe[5] & keep) | ((qe[7] & keep) << 16)};
    *(u32x4_t*)&q_lds[q_r][4 * q_k] = qp;  // (e0,e2) (e1,e3) (e4,e6) (e5,e7)
  }
  __syncthreads();

  // ---- this lane's query row (row lane % 4 of each row set) and the
  //      accumulator init -bias * sum(q) per 32-dim chunk, on the MFMA ----
  const int my_row = lane & 3;
  f32x4_t qinit[RS][LPT];
  int lim[RS][4];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rho = rc * ROWS + rs * 4 + i;
      int lm = a.causal ? L - a.Sq + (rho % a.Sq) + 1 : L;
      lm = lm < 0 ? 0 : lm;
      lim[rs][i] = rho < a.rows_total ? lm : 0;
    }
#pragma unroll
    for (int c = 0; c < LPT; ++c) {
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        const u32x4_t qv = *(const u32x4_t*)&q_lds[rs * 4 + my_row][16 * c + 4 * k4];
        acc = mfma4<F16>(qv.x, qv.y, NEG_BIAS, NEG_BIAS, acc);
        acc = mfma4<F16>(qv.z, qv.w, NEG_BIAS, NEG_BIAS, acc);
      }
      qinit[rs][c] = acc;
    }
  }

  // ---- running softmax state ----
  float m_run[RS][4], l_acc[RS][4];
  f32x4_t o_acc[RS][8], w_acc[RS];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      m_run[rs][i] = kNeg;
      l_acc[rs][i] = 0.0f;
    }
#pragma unroll
    for (int m = 0; m < 8; ++m) o_acc[rs][m] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
    w_acc[rs] = f32x4_t{0.0f, 0.0f, 0.0f, 0.0f};
  }

  for (int base = wave; base < ntiles; base += NW * CH) {
    if constexpr (!PIPE) {
#pragma unroll
      for (int i = 0; i < CH; ++i) load_tile(i, base, base + NW * i < ntiles);
    }
    const bool more = PIPE && base + NW * CH < ntiles;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      // ---- QK on the matrix cores: scores of token `lane` for every row ----
      float sc[RS][4];
      {
        f32x4_t acc[RS][LPT];
#pragma unroll
        for (int rs = 0; rs < RS; ++rs)
#pragma unroll
          for (int c = 0; c < LPT; ++c) acc[rs][c] = qinit[rs][c];
#pragma unroll
        for (int c = 0; c < LPT; ++c) {
#pragma unroll
          for (int k4 = 0; k4 < 4; ++k4) {
            const uint32_t w = kc4[i][c][k4];
            const int kd = 4 * c + k4;  // code dword index in the row
            const uint32_t lo = w & 0x0F0F0F0Fu, hi = (w >> 4) & 0x0F0F0F0Fu;
            const uint32_t b02 = __builtin_amdgcn_perm(MAGIC, lo, SEL_02);  // (e0, e2)
            const uint32_t b13 = __builtin_amdgcn_perm(MAGIC, hi, SEL_02);  // (e1, e3)
            const uint32_t b46 = __builtin_amdgcn_perm(MAGIC, lo, SEL_46);  // (e4, e6)
            const uint32_t b57 = __builtin_amdgcn_perm(MAGIC, hi, SEL_46);  // (e5, e7)
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) {
              const u32x4_t qv = *(const u32x4_t*)&q_lds[rs * 4 + my_row][4 * kd];
              acc[rs][c] = mfma4<F16>(qv.x, qv.y, b02, b13, acc[rs][c]);
              acc[rs][c] = mfma4<F16>(qv.z, qv.w, b46, b57, acc[rs][c]);
            }
          }
        }
        const int t = t_begin + (base + NW * i) * 64 + lane;
        const bool tok_ok = (base + NW * i < ntiles) && (t < t_end);
        float skl[LPT];
#pragma unroll
        for (int c = 0; c < LPT; ++c) skl[c] = scale16_to_f32(skr[i][c], s_f16) * a.scale_log2;
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float s = 0.0f;
#pragma unroll
            for (int c = 0; c < LPT; ++c) s = fmaf(acc[rs][c][r], skl[c], s);
            bool ok = tok_ok;
            if constexpr (ROWMASK) ok = ok && (t < lim[rs][r]);
            sc[rs][r] = ok ? s : kNeg;
          }
        }
      }
      load_k(i, base + NW * CH, more && base + NW * (CH + i) < ntiles);

      // ---- tile max and rescale of the running state ----
      bool grow = false;
      float m_new[RS][4];
#pragma unroll
      for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          m_new[rs][r] = fmaxf(m_run[rs][r], wave_max(sc[rs][r]));
          grow = grow || (m_new[rs][r] > m_run[rs][r]);
        }
      }
      if (grow) {
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
          f32x4_t al;
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            al[r] = __builtin_amdgcn_exp2f(m_run[rs][r] - m_new[rs][r]);
            l_acc[rs][r] *= al[r];
            m_run[rs][r] = m_new[rs][r];
          }
#pragma unroll
          for (int m = 0; m < 8; ++m) o_acc[rs][m] *= al;
          w_acc[rs] *= al;
        }
      }

      // ---- p and w = p * v_scale (bf16) -> LDS ----
      {
        float svl[LPT];
#pragma unroll
        for (int c = 0; c < LPT; ++c) svl[c] = scale16_to_f32(svr[i][c], s_f16);
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float s = sc[rs][r];
            const float p = s > kNeg ? __builtin_amdgcn_exp2f(s - m_run[rs][r]) : 0.0f;
            l_acc[rs][r] += p;
#pragma unroll
            for (int c = 0; c < LPT; ++c)
              w_lds[wave][i][rs][r][c][w_sub][w_ts][w_k] = __builtin_bit_cast(uint16_t, (__bf16)(p * svl[c]));
          }
        }
      }
      load_vs(i, base + NW * CH, more && base + NW * (CH + i) < ntiles);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // ---- PV on the matrix cores ----
      // u = bytes {t0.b, t1.b, t0.b', t1.b'} of two tokens' code dwords; its low
      // and high nibbles then give (token0, token1) pairs of one dim per perm.
#pragma unroll
      for (int s = 0; s < NSUB; ++s) {
        uint32_t bp[2][8];  // [token pair][dim within the lane's 8]
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
          const uint32_t v0 = vcode[i][s][2 * tp], v1 = vcode[i][s][2 * tp + 1];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {  // dims 0-3, dims 4-7
            const uint32_t u = __builtin_amdgcn_perm(v1, v0, hh ? 0x07030602u : 0x05010400u);
            const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
            bp[tp][4 * hh + 0] = __builtin_amdgcn_perm(0x43434343u, lo, SEL_02);
            bp[tp][4 * hh + 1] = __builtin_amdgcn_perm(0x43434343u, hi, SEL_02);
            bp[tp][4 * hh + 2] = __builtin_amdgcn_perm(0x43434343u, lo, SEL_46);
            bp[tp][4 * hh + 3] = __builtin_amdgcn_perm(0x43434343u, hi, SEL_46);
          }
        }
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
          const uint2 wa = *(const uint2*)&w_lds[wave][i][rs][v_row][v_chunk][s][vts][0];
#pragma unroll
          for (int m = 0; m < 8; ++m)
            o_acc[rs][m] = mfma4<false>(wa.x, wa.y, bp[0][m], bp[1][m], o_acc[rs][m]);
          w_acc[rs] = mfma4<false>(wa.x, wa.y, kBf16OnePair, kBf16OnePair, w_acc[rs]);
        }
      }
      load_v(i, base + NW * CH, more && base + NW * (CH + i) < ntiles);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
    }
  }

  // ---- wave partial -> LDS: one slot per token subset, o[row][8*vj + m] ----
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float* dst = &o_lds[wave * VTS + vts][rs * 4 + r][8 * vj];
      float v[8];
#pragma unroll
      for (int m = 0; m < 8; ++m) v[m] = fmaf(-136.0f, w_acc[rs][r], o_acc[rs][m][r]);
      *(float4*)dst = make_float4(v[0], v[1], v[2], v[3]);
      *(float4*)(dst + 4) = make_float4(v[4], v[5], v[6], v[7]);
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const float lsum = wave_sum(l_acc[rs][r]);
      if (lane == 0) {
        ml_lds[wave][rs * 4 + r][0] = m_run[rs][r];
        ml_lds[wave][rs * 4 + r][1] = lsum;
      }
    }
  }
  __syncthreads();
  finish_block<ROWS, D, QM, NW, VTS>(a, unit, split, rc, kvh, b, o_lds, ml_lds, mg);
}

// ===========================================================================
// VALU kernel: fp32 queries (exact fp32 arithmetic) or fp32 scales.
// Lane = token * (D/32) + chunk for QK (quad-reduced with DPP); V lanes own 8
// output dims and four tokens per tile.

template <int D, int ROWS, int QM, bool ROWMASK>
__global__ __launch_bounds__(256) void decode_attn_valu_kernel(const AttnArgs a) {
  constexpr int LPT = D / 32;
  constexpr int TPT = 64 / LPT;
  constexpr int VLPT = D / 8;
  constexpr int VTS = 64 / VLPT;
  constexpr int CH = 8;
  constexpr bool DOT2 = QM != KVQ_F32;
  static_assert(TPT == 4 * VTS, "tile shape");
  using WT = typename std::conditional<DOT2, uint16_t, float>::type;

  __shared__ __attribute__((aligned(16))) WT w_lds[4][CH][ROWS][LPT][TPT];
  __shared__ float o_lds[4][ROWS][D];
  __shared__ float ml_lds[4][ROWS][2];
  __shared__ MergeLds mg;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  int unit, split;
  unit_and_split(a, unit, split);
  const int rc = unit % a.row_chunks;
  const int bh = unit / a.row_chunks;
  const int kvh = bh % a.Hkv;
  const int b = bh / a.Hkv;

  int L = a.Sk;
  if (a.seq_lens) {
    const int sl = a.seq_lens[b];
    L = sl < 0 ? 0 : (sl < a.Sk ? sl : a.Sk);
  }
  const int t_begin = split * a.split_len;
  const int t_end = min(t_begin + a.split_len, L);
  const int ntiles = t_end > t_begin ? (t_end - t_begin + TPT - 1) / TPT : 0;

  const int kt = lane / LPT;
  const int kc = lane % LPT;
  const int vts = lane / VLPT;
  const int vj = lane % VLPT;
  const int vc = vj >> 2;
  const uint32_t gK = (uint32_t)((kc * 32) / a.G);

  int lim[ROWS];
  uint32_t qp[DOT2 ? ROWS : 1][16];
  float qf[DOT2 ? 1 : ROWS][32];
  float qinit[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int rho = rc * ROWS + r;
    const bool row_ok = rho < a.rows_total;
    const int rho_c = row_ok ? rho : 0;
    const int head = kvh * a.ratio + rho_c / a.Sq;
    const int qi = rho_c % a.Sq;
    int lm = a.causal ? L - a.Sq + qi + 1 : L;
    lm = lm < 0 ? 0 : lm;
    lim[r] = row_ok ? lm : 0;
    const int64_t qbase = (int64_t)b * a.qs_b + (int64_t)head * a.qs_h + (int64_t)qi * a.qs_s;
    float qsum = 0.0f;
    if constexpr (DOT2) {
      const uint16_t* q16 = (const uint16_t*)a.q;
      const uint32_t keep = row_ok ? 0xffffu : 0u;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int e0 = kc * 32 + 8 * k + m;
          const uint32_t lo = q16[qbase + (int64_t)e0 * a.qs_d] & keep;
          const uint32_t hi = q16[qbase + (int64_t)(e0 + 4) * a.qs_d] & keep;
          qp[r][4 * k + m] = lo | (hi << 16);
          if constexpr (QM == KVQ_BF16) qsum += bf16_bits_to_f32(lo) + bf16_bits_to_f32(hi);
        }
      }
      qinit[r] = QM == KVQ_BF16 ? -136.0f * qsum : 0.0f;
    } else {
      const float* q32 = (const float*)a.q;
      const float keep = row_ok ? 1.0f : 0.0f;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const float v = q32[qbase + (int64_t)(kc * 32 + e) * a.qs_d] * keep;
        qf[r][e] = v;
        qsum += v;
      }
      qinit[r] = -8.0f * qsum;
    }
  }

  float m_run[ROWS], l_acc[ROWS], wsum[ROWS], o_acc[ROWS][8];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    m_run[r] = kNeg;
    l_acc[r] = 0.0f;
    wsum[r] = 0.0f;
#pragma unroll
    for (int m = 0; m < 8; ++m) o_acc[r][m] = 0.0f;
  }

  const uint8_t* kp_bh = a.kp + (int64_t)b * a.kps_b + (int64_t)kvh * a.kps_h;
  const uint8_t* vp_bh = a.vp + (int64_t)b * a.vps_b + (int64_t)kvh * a.vps_h;
  const int s_esize = a.scale_dtype == KVQ_F32 ? 4 : 2;
  const char* ks_bh = (const char*)a.ks + ((int64_t)b * a.kss_b + (int64_t)kvh * a.kss_h) * s_esize;
  const char* vs_bh = (const char*)a.vs + ((int64_t)b * a.vss_b + (int64_t)kvh * a.vss_h) * s_esize;
  const uint32_t kps = (uint32_t)a.kps_s, vps = (uint32_t)a.vps_s;
  const uint32_t kss = (uint32_t)a.kss_s, vss = (uint32_t)a.vss_s;
  const int last_tok = L > 0 ? L - 1 : 0;

  for (int base = wave; base < ntiles; base += 4 * CH) {
    uint4 kcode[CH];
    uint32_t vcode[CH][4];
    float sk[CH], sv[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int t0 = t_begin + (base + 4 * i) * TPT;
      const uint32_t tk = (uint32_t)min(t0 + kt, last_tok);
      kcode[i] = *(const uint4*)(kp_bh + (tk * kps + 16u * kc));
      sk[i] = load_scale(ks_bh, tk * kss + gK, a.scale_dtype);
      sv[i] = load_scale(vs_bh, tk * vss + gK, a.scale_dtype);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t tv = (uint32_t)min(t0 + vts + VTS * k, last_tok);
        vcode[i][k] = *(const uint32_t*)(vp_bh + (tv * vps + 4u * vj));
      }
    }

    float s[CH][ROWS];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int t = t_begin + (base + 4 * i) * TPT + kt;
      const bool tv_ok = (base + 4 * i < ntiles) && (t < t_end);
      float acc[ROWS];
#pragma unroll
      for (int r = 0; r < ROWS; ++r) acc[r] = qinit[r];
      const uint32_t wk[4] = {kcode[i].x, kcode[i].y, kcode[i].z, kcode[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t w = wk[k];
        if constexpr (QM == KVQ_BF16) {
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const uint32_t pm = ((w >> (4 * m)) & kNibPairs) | kBf16Magic;
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = dot2_bf16(qp[r][4 * k + m], pm, acc[r]);
          }
        } else if constexpr (QM == KVQ_F16) {
          const f16x2_t bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const f16x2_t h =
                __builtin_bit_cast(f16x2_t, ((w >> (4 * m)) & kNibPairs) | kF16Magic) + bias;
            const uint32_t pm = __builtin_bit_cast(uint32_t, h);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = dot2_f16(qp[r][4 * k + m], pm, acc[r]);
          }
        } else {
#pragma unroll
          for (int e = 0; e < 8; ++e) {
            const float n = (float)((w >> (4 * e)) & 15u);
#pragma unroll
            for (int r = 0; r < ROWS; ++r) acc[r] = fmaf(qf[r][8 * k + e], n, acc[r]);
          }
        }
      }
      const float skl = sk[i] * a.scale_log2;
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        float part = acc[r] * skl;
        if constexpr (LPT >= 2) part += dpp<0xB1>(part, 0.0f);  // quad_perm [1,0,3,2]
        if constexpr (LPT >= 4) part += dpp<0x4E>(part, 0.0f);  // quad_perm [2,3,0,1]
        bool ok = tv_ok;
        if constexpr (ROWMASK) ok = ok && (t < lim[r]);
        s[i][r] = ok ? part : kNeg;
      }
    }

    float m_new[ROWS];
    bool grow = false;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float mx = s[0][r];
#pragma unroll
      for (int i = 1; i < CH; ++i) mx = fmaxf(mx, s[i][r]);
      m_new[r] = fmaxf(m_run[r], wave_max(mx));
      grow = grow || (m_new[r] > m_run[r]);
    }
    if (grow) {
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        const float alpha = __builtin_amdgcn_exp2f(m_run[r] - m_new[r]);
        l_acc[r] *= alpha;
        wsum[r] *= alpha;
#pragma unroll
        for (int m = 0; m < 8; ++m) o_acc[r][m] *= alpha;
        m_run[r] = m_new[r];
      }
    }

    const int pos = (kt % VTS) * 4 + kt / VTS;
#pragma unroll
    for (int i = 0; i < CH; ++i) {
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        const float p = s[i][r] > kNeg ? __builtin_amdgcn_exp2f(s[i][r] - m_run[r]) : 0.0f;
        l_acc[r] += p;
        const float w = p * sv[i];
        if constexpr (DOT2) w_lds[wave][i][r][kc][pos] = (uint16_t)f32_to_bf16_bits(w);
        else w_lds[wave][i][r][kc][pos] = w;
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if constexpr (DOT2) {
        uint32_t cp01[8], cp23[8];
        const uint32_t plo01 = __builtin_amdgcn_perm(vcode[i][1], vcode[i][0], 0x05040100u);
        const uint32_t phi01 = __builtin_amdgcn_perm(vcode[i][1], vcode[i][0], 0x07060302u);
        const uint32_t plo23 = __builtin_amdgcn_perm(vcode[i][3], vcode[i][2], 0x05040100u);
        const uint32_t phi23 = __builtin_amdgcn_perm(vcode[i][3], vcode[i][2], 0x07060302u);
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          cp01[m] = ((plo01 >> (4 * m)) & kNibPairs) | kBf16Magic;
          cp01[m + 4] = ((phi01 >> (4 * m)) & kNibPairs) | kBf16Magic;
          cp23[m] = ((plo23 >> (4 * m)) & kNibPairs) | kBf16Magic;
          cp23[m + 4] = ((phi23 >> (4 * m)) & kNibPairs) | kBf16Magic;
        }
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
          const uint2 wp = *(const uint2*)&w_lds[wave][i][r][vc][vts * 4];
#pragma unroll
          for (int m = 0; m < 8; ++m) {
            o_acc[r][m] = dot2_bf16(wp.x, cp01[m], o_acc[r][m]);
            o_acc[r][m] = dot2_bf16(wp.y, cp23[m], o_acc[r][m]);
          }
          wsum[r] = dot2_bf16(wp.x, kBf16OnePair, wsum[r]);
          wsum[r] = dot2_bf16(wp.y, kBf16OnePair, wsum[r]);
        }
      } else {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) {
          const float4 wv = *(const float4*)&w_lds[wave][i][r][vc][vts * 4];
          const float wk4[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
          for (int k = 0; k < 4; ++k) {
#pragma unroll
            for (int m = 0; m < 8; ++m) {
              const float v = (float)((vcode[i][k] >> (4 * m)) & 15u) - 8.0f;
              o_acc[r][m] = fmaf(wk4[k], v, o_acc[r][m]);
            }
          }
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
  }

#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      float v = o_acc[r][m];
      if constexpr (DOT2) v = fmaf(-136.0f, wsum[r], v);
#pragma unroll
      for (int step = VLPT; step < 64; step *= 2) v += __shfl_xor(v, step, 64);
      if (vts == 0) o_lds[wave][r][8 * vj + m] = v;
    }
    const float lsum = wave_sum(kc == 0 ? l_acc[r] : 0.0f);
    if (lane == 0) {
      ml_lds[wave][r][0] = m_run[r];
      ml_lds[wave][r][1] = lsum;
    }
  }
  __syncthreads();
  finish_block<ROWS, D, QM, 4, 1>(a, unit, split, rc, kvh, b, o_lds, ml_lds, mg);
}

// ---------------------------------------------------------------------------
// Host side: planning and dispatch.

struct Plan {
  bool mfma;
  int rows, row_chunks, n_units, n_split, split_len;
};

// The MFMA kernel serves bf16/fp16 queries with 16-bit scales; everything else
// (fp32 queries, fp32 scales) runs on the VALU kernel.
static bool use_mfma(int q_dtype, int scale_dtype) {
  return q_dtype != KVQ_F32 && scale_dtype != KVQ_F32;
}

static int make_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D, int64_t s_max,
                     int q_dtype, int scale_dtype, int64_t n_split_req, int64_t num_cus, Plan* p) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Sq < 1 || s_max < 0 || Hq % Hkv != 0) return KVQ_EINVAL;
  if (!(D == 64 || D == 128)) return KVQ_EUNSUP;
  const int64_t rows_total = (Hq / Hkv) * Sq;
  p->mfma = use_mfma(q_dtype, scale_dtype);
  int tpt;  // tokens per wave tile
  if (p->mfma) {
    p->rows = rows_total <= 4 ? 4 : 8;
    tpt = 64;
  } else {
    const int cap = q_dtype == KVQ_F32 ? 2 : 8;
    int r = 1;
    while (r < rows_total && r < cap) r *= 2;
    p->rows = r;
    tpt = (int)(64 / (D / 32));
  }
  p->row_chunks = (int)((rows_total + p->rows - 1) / p->rows);
  const int64_t units = B * Hkv * p->row_chunks;
  if (units > (1ll << 30)) return KVQ_EUNSUP;
  p->n_units = (int)units;
  const int64_t max_split = std::max<int64_t>(1, (s_max + 4 * tpt - 1) / (4 * tpt));
  int64_t ns = n_split_req;
  if (ns <= 0) {
    const int64_t cus = std::max<int64_t>(1, num_cus);
    ns = (cus + units - 1) / units;
  }
  ns = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(ns, max_split), kMaxSplit));
  int64_t split_len = (s_max + ns - 1) / ns;
  split_len = std::max<int64_t>(tpt, ((split_len + tpt - 1) / tpt) * tpt);
  ns = std::max<int64_t>(1, (s_max + split_len - 1) / split_len);
  if (units * ns > 0x7fffffffll || units * p->rows * D / 128 >= 0x7fffffffll) return KVQ_EUNSUP;
  p->n_split = (int)ns;
  p->split_len = (int)std::min<int64_t>(split_len, 0x7fffffffll);
  return KVQ_OK;
}

// Workspace: per (unit, split, row) the partial (max, sum) pair, then the
// partial output row; the (max, sum) block is padded to 256 bytes.
static int64_t ws_ml_bytes(const Plan& p) {
  const int64_t slots = (int64_t)p.n_units * p.n_split * p.rows;
  return (slots * 2 * 4 + 255) / 256 * 256;
}

static int64_t workspace_bytes_for(const Plan& p, int64_t D) {
  if (p.n_split <= 1) return 0;
  return ws_ml_bytes(p) + (int64_t)p.n_units * p.n_split * p.rows * D * 4;
}

// Waves per workgroup of the MFMA kernel: one row set runs 8 waves of one tile
// each (two waves per SIMD hide each other's latency); two row sets need more
// registers than that allows and run 4 waves of two tiles.
template <int RS>
constexpr int mfma_waves() { return RS == 1 ? 8 : 4; }

template <int D, int RS, int QM>
static void launch_mfma_rs(const AttnArgs& a, bool rowmask, dim3 grid, hipStream_t st) {
  constexpr int NW = mfma_waves<RS>();
  if (rowmask) hipLaunchKernelGGL((decode_attn_mfma_kernel<D, RS, QM, true, NW>), grid, dim3(64 * NW), 0, st, a);
  else hipLaunchKernelGGL((decode_attn_mfma_kernel<D, RS, QM, false, NW>), grid, dim3(64 * NW), 0, st, a);
}

template <int D, int QM>
static void launch_mfma(const AttnArgs& a, int rows, bool rowmask, dim3 grid, hipStream_t st) {
  if (rows <= 4) launch_mfma_rs<D, 1, QM>(a, rowmask, grid, st);
  else launch_mfma_rs<D, 2, QM>(a, rowmask, grid, st);
}

template <int D, int ROWS, int QM>
static void launch_valu_rows(const AttnArgs& a, bool rowmask, dim3 grid, hipStream_t st) {
  if (rowmask) hipLaunchKernelGGL((decode_attn_valu_kernel<D, ROWS, QM, true>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((decode_attn_valu_kernel<D, ROWS, QM, false>), grid, dim3(256), 0, st, a);
}

template <int D, int QM>
static void launch_valu_qm(const AttnArgs& a, int rows, bool rowmask, dim3 grid, hipStream_t st) {
  switch (rows) {
    case 1: launch_valu_rows<D, 1, QM>(a, rowmask, grid, st); break;
    case 2: launch_valu_rows<D, 2, QM>(a, rowmask, grid, st); break;
    case 4:
      if constexpr (QM != KVQ_F32) launch_valu_rows<D, 4, QM>(a, rowmask, grid, st);
      break;
    default:
      if constexpr (QM != KVQ_F32) launch_valu_rows<D, 8, QM>(a, rowmask, grid, st);
      break;
  }
}

template <int D>
static void launch_d(const AttnArgs& a, const Plan& p, int q_dtype, bool rowmask, dim3 grid,
                     hipStream_t st) {
  if (p.mfma) {
    if (q_dtype == KVQ_BF16) launch_mfma<D, KVQ_BF16>(a, p.rows, rowmask, grid, st);
    else launch_mfma<D, KVQ_F16>(a, p.rows, rowmask, grid, st);
    return;
  }
  switch (q_dtype) {
    case KVQ_BF16: launch_valu_qm<D, KVQ_BF16>(a, p.rows, rowmask, grid, st); break;
    case KVQ_F16: launch_valu_qm<D, KVQ_F16>(a, p.rows, rowmask, grid, st); break;
    default: launch_valu_qm<D, KVQ_F32>(a, p.rows, rowmask, grid, st); break;
  }
}

}  // namespace kvq

using namespace kvq;

extern "C" int64_t kvq_decode_attn_num_splits(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                              int64_t D, int64_t s_max, int q_dtype,
                                              int scale_dtype, int64_t num_cus) {
  clear_error();
  if (!dtype_ok(q_dtype) || !dtype_ok(scale_dtype)) {
    set_error("kvq_decode_attn_num_splits: q and scale dtypes must be bf16/fp16/fp32");
    return KVQ_EINVAL;
  }
  Plan p;
  const int rc = make_plan(B, Hq, Hkv, Sq, D, s_max, q_dtype, scale_dtype, 0, num_cus, &p);
  if (rc != KVQ_OK) {
    set_error("kvq_decode_attn_num_splits: unsupported or invalid shape (B=%lld Hq=%lld Hkv=%lld "
              "Sq=%lld D=%lld)", (long long)B, (long long)Hq, (long long)Hkv, (long long)Sq,
              (long long)D);
    return rc;
  }
  return p.n_split;
}

extern "C" int64_t kvq_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                                   int64_t D, int q_dtype, int scale_dtype,
                                                   int64_t n_split) {
  clear_error();
  if (!dtype_ok(q_dtype) || !dtype_ok(scale_dtype) || n_split < 1) {
    set_error("kvq_decode_attn_workspace_bytes: bad dtype or n_split");
    return KVQ_EINVAL;
  }
  // s_max only bounds n_split in planning; pass one that keeps n_split.
  Plan p;
  const int rc =
      make_plan(B, Hq, Hkv, Sq, D, n_split * 4 * 64, q_dtype, scale_dtype, n_split, 1, &p);
  if (rc != KVQ_OK) {
    set_error("kvq_decode_attn_workspace_bytes: unsupported or invalid shape");
    return rc;
  }
  return workspace_bytes_for(p, D);
}

extern "C" int kvq_decode_attn(const void* q, int q_dtype, const int64_t* q_strides,
                               const void* k_packed, const int64_t* kp_strides,
                               const void* k_scales, const int64_t* ks_strides,
                               const void* v_packed, const int64_t* vp_strides,
                               const void* v_scales, const int64_t* vs_strides,
                               int scale_dtype,
                               void* out, const int64_t* out_strides,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                               int64_t group_size, int64_t Sk,
                               const int32_t* seq_lens, int is_causal, float sm_scale,
                               int64_t n_split, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  clear_error();
  KVQ_CHECK_ARG(dtype_ok(q_dtype), "kvq_decode_attn: q dtype must be bf16/fp16/fp32");
  KVQ_CHECK_ARG(dtype_ok(scale_dtype), "kvq_decode_attn: scale dtype must be bf16/fp16/fp32");
  KVQ_CHECK_ARG(q_strides && kp_strides && ks_strides && vp_strides && vs_strides && out_strides,
                "kvq_decode_attn: null stride array");
  KVQ_CHECK_ARG(B >= 0 && Hq >= 1 && Hkv >= 1 && Sq >= 0 && Sk >= 0,
                "kvq_decode_attn: bad extents");
  KVQ_CHECK_ARG(Hq % Hkv == 0, "kvq_decode_attn: Hq must be a multiple of Hkv");
  KVQ_CHECK_ARG(group_size > 0, "kvq_decode_attn: group_size must be > 0");
  KVQ_CHECK_ARG(n_split >= 1, "kvq_decode_attn: n_split must be >= 1");
  if (!(D == 64 || D == 128) || group_size % 32 != 0) {
    set_error("kvq_decode_attn: fused kernel needs D in {64,128} and group_size %% 32 == 0 "
              "(got D=%lld, group_size=%lld)", (long long)D, (long long)group_size);
    return KVQ_EUNSUP;
  }
  if (B == 0 || Sq == 0) return KVQ_OK;
  KVQ_CHECK_ARG(q && out, "kvq_decode_attn: null q/out");
  KVQ_CHECK_ARG(Sk == 0 || (k_packed && k_scales && v_packed && v_scales),
                "kvq_decode_attn: null K/V pointer");
  // Vector loads: 16-byte key chunks and 4-byte value dwords.
  const bool k_al = ((uintptr_t)k_packed % 16 == 0) && kp_strides[0] % 16 == 0 &&
                    kp_strides[1] % 16 == 0 && kp_strides[2] % 16 == 0;
  const bool v_al = ((uintptr_t)v_packed % 4 == 0) && vp_strides[0] % 4 == 0 &&
                    vp_strides[1] % 4 == 0 && vp_strides[2] % 4 == 0;
  if (!k_al || !v_al) {
    set_error("kvq_decode_attn: packed K rows must be 16-byte aligned and V rows 4-byte aligned");
    return KVQ_EUNSUP;
  }
  // Token offsets inside one (batch, head) slice are 32-bit.
  if (Sk > 0 && (Sk * kp_strides[2] >= (1ll << 31) || Sk * vp_strides[2] >= (1ll << 31) ||
                 Sk * ks_strides[2] * 4 >= (1ll << 31) || Sk * vs_strides[2] * 4 >= (1ll << 31))) {
    set_error("kvq_decode_attn: a (batch, head) slice of the cache exceeds 2 GiB");
    return KVQ_EUNSUP;
  }
  KVQ_CHECK_ARG(Sk <= 0x7fffffffll && Sq <= 0x7fffffffll, "kvq_decode_attn: sequence too long");

  Plan p;
  const int rc = make_plan(B, Hq, Hkv, Sq, D, Sk, q_dtype, scale_dtype, n_split, 1, &p);
  if (rc != KVQ_OK) {
    set_error("kvq_decode_attn: unsupported shape");
    return rc;
  }
  const int64_t need = workspace_bytes_for(p, D);
  if (need > 0 && (workspace == nullptr || workspace_bytes < need)) {
    set_error("kvq_decode_attn: workspace too small (%lld < %lld bytes)",
              (long long)workspace_bytes, (long long)need);
    return KVQ_ESPACE;
  }

  AttnArgs a;
  a.q = q;
  a.qs_b = q_strides[0]; a.qs_h = q_strides[1]; a.qs_s = q_strides[2]; a.qs_d = q_strides[3];
  a.kp = (const uint8_t*)k_packed;
  a.kps_b = kp_strides[0]; a.kps_h = kp_strides[1]; a.kps_s = kp_strides[2];
  a.ks = k_scales;
  a.kss_b = ks_strides[0]; a.kss_h = ks_strides[1]; a.kss_s = ks_strides[2];
  a.vp = (const uint8_t*)v_packed;
  a.vps_b = vp_strides[0]; a.vps_h = vp_strides[1]; a.vps_s = vp_strides[2];
  a.vs = v_scales;
  a.vss_b = vs_strides[0]; a.vss_h = vs_strides[1]; a.vss_s = vs_strides[2];
  a.out = out;
  a.os_b = out_strides[0]; a.os_h = out_strides[1]; a.os_s = out_strides[2]; a.os_d = out_strides[3];
  a.seq_lens = seq_lens;
  a.Hkv = (int)Hkv; a.Sq = (int)Sq; a.G = (int)group_size; a.Sk = (int)Sk;
  a.ratio = (int)(Hq / Hkv);
  a.rows_total = (int)((Hq / Hkv) * Sq);
  a.row_chunks = p.row_chunks;
  a.n_units = p.n_units;
  a.n_split = p.n_split;
  a.split_len = p.split_len;
  a.causal = is_causal ? 1 : 0;
  a.scale_dtype = scale_dtype;
  a.xcd_remap = (p.n_split > 1 && p.n_units % 8 == 0) ? 1 : 0;
  // 16-byte q loads need unit element stride and 16-byte aligned rows.
  a.q_vec = (q_dtype != KVQ_F32 && q_strides[3] == 1 && (uintptr_t)q % 16 == 0 &&
             q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0 && q_strides[2] % 8 == 0) ? 1 : 0;
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.ws_ml = nullptr; a.ws_o = nullptr;
  if (need > 0) {
    char* w = (char*)workspace;
    a.ws_ml = (float*)w;
    a.ws_o = (float*)(w + ws_ml_bytes(p));
  }
  const bool rowmask = is_causal && Sq > 1;
  const dim3 grid((unsigned)((int64_t)p.n_units * p.n_split));
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) launch_d<128>(a, p, q_dtype, rowmask, grid, st);
  else launch_d<64>(a, p, q_dtype, rowmask, grid, st);
  KVQ_CHECK_LAUNCH("kvq_decode_attn");
  if (p.n_split > 1) {
    const int64_t threads = (int64_t)p.n_units * p.rows * D;
    const dim3 mgrid((unsigned)((threads + 127) / 128));
    switch (q_dtype) {
      case KVQ_BF16:
        hipLaunchKernelGGL(decode_attn_merge_kernel<KVQ_BF16>, mgrid, dim3(128), 0, st, a, p.rows, (int)D);
        break;
      case KVQ_F16:
        hipLaunchKernelGGL(decode_attn_merge_kernel<KVQ_F16>, mgrid, dim3(128), 0, st, a, p.rows, (int)D);
        break;
      default:
        hipLaunchKernelGGL(decode_attn_merge_kernel<KVQ_F32>, mgrid, dim3(128), 0, st, a, p.rows, (int)D);
        break;
    }
    KVQ_CHECK_LAUNCH("kvq_decode_attn (split merge)");
  }
  return KVQ_OK;
}
