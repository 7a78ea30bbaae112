// Fused INT4-KV GQA decode attention for gfx950 (CDNA4, wave64).
//
// Replaces the reference's fused kernels
//   kernels/llama3/attention_quant.py:24-152 (_attention_fwd_quant_gqa_kernel)
//   kernels/gpt2/attention_quant.py:12-137   (_attention_fwd_quant_kernel, MHA)
// for short query blocks. The reference runs one program per *query* head and
// walks the whole sequence serially (kv = h // ratio, :71; tile loop :104), so
// K/V are re-read once per GQA group member and only B*Hq programs exist.
// Here one workgroup owns one (batch, kv head, query-row chunk) and one slice
// of the sequence (split-K): every query head of the GQA group (times the Sq
// query positions) is a "row" processed against the same K/V bytes, so each
// byte of the cache crosses HBM once, and B*Hkv*n_split workgroups fill the
// 256 CUs. Partial (max, sum, o) triples are merged first across the 4 waves
// of a workgroup (LDS) and then across splits by the last workgroup to finish
// (device-scope counter), which writes the output.
//
// Lane layout (D = head dim, chunks of 32 elements = 16 packed bytes):
//   K phase: lane = token * (D/32) + chunk. One 16-byte load per lane brings
//            one 32-element chunk of one token's key codes; a quad (D=128) of
//            lanes covers one token and a wave covers 64/(D/32) tokens (a
//            "tile"). Partial dot products are summed over the quad with DPP.
//   V phase: lane = token_subset * (D/8) + j. Lane j owns output dims
//            [8j, 8j+8) and reads one dword of value codes per token, for four
//            tokens of the tile; tokens are paired so that one v_dot2 adds two
//            tokens' contributions to one output dim.
// Softmax weights w = p * v_scale travel from K lanes to V lanes through a
// per-wave LDS slab (no workgroup barrier needed inside the token loop).
//
// Arithmetic. Codes n in 0..15 become exact bf16/fp16 numbers with a
// magic-number OR: bf16(128 + n) = 0x4300 | n, fp16(1024 + n) = 0x6400 | n.
//   bf16 q : score chunk = sum q*(128+n) - 136*sum(q) with v_dot2_f32_bf16
//            (the -136*sum(q) is the accumulator's initial value);
//   fp16 q : (1024+n) - 1032 = n - 8 exactly via v_pk_add_f16, v_dot2_f32_f16;
//   fp32 q : exact fp32 FMAs (used for fp32 inputs, where the bar is 1e-4).
// The value side for bf16/fp16 q uses bf16 weights with bf16(128+n) codes and
// subtracts 136*sum(w) (accumulated from the same rounded weights) at the end.
// Group scales are applied once per (token, chunk): s = sum_g sk_g*dot_g.
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
  int n_split, split_len, causal, scale_dtype, xcd_remap;
  float scale_log2;
  float* ws_ml;      // [n_units][n_split][ROWS][2]  (max, sum)
  float* ws_o;       // [n_units][n_split][ROWS][D]
  unsigned* ws_cnt;  // [n_units]
};

constexpr float kNeg = -1.0e30f;
constexpr uint32_t kNibPairs = 0x000F000Fu;
constexpr uint32_t kBf16Magic = 0x43004300u;  // bf16(128), bf16(128)
constexpr uint32_t kF16Magic = 0x64006400u;   // fp16(1024), fp16(1024)
constexpr uint32_t kBf16OnePair = 0x3F803F80u;

typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ float dot2_bf16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, a),
                                         __builtin_bit_cast(bf16x2_t, b), c, false);
}
__device__ __forceinline__ float dot2_f16(uint32_t a, uint32_t b, float c) {
  return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, a), __builtin_bit_cast(f16x2_t, b), c,
                                false);
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

__device__ __forceinline__ float load_scale(const void* p, int64_t i, int dt) {
  return load_as_f32(p, i, dt);
}

template <int D, int ROWS, int QM, bool ROWMASK>
__global__ __launch_bounds__(256) void decode_attn_kernel(const AttnArgs a) {
  constexpr int LPT = D / 32;    // K lanes per token
  constexpr int TPT = 64 / LPT;  // tokens per tile
  constexpr int VLPT = D / 8;    // V lanes per token
  constexpr int VTS = 64 / VLPT; // V token subsets; TPT == 4 * VTS
  constexpr int CH = ROWS >= 8 ? 4 : 8;  // tiles per chunk per wave
  constexpr bool DOT2 = QM != KVQ_F32;
  static_assert(TPT == 4 * VTS, "tile shape");
  using WT = typename std::conditional<DOT2, uint16_t, float>::type;

  __shared__ __attribute__((aligned(16))) WT w_lds[4][CH][ROWS][LPT][TPT];
  __shared__ float o_lds[4][ROWS][D];
  __shared__ float ml_lds[4][ROWS][2];
  __shared__ int last_flag;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;

  // Workgroup -> (unit, split). With XCD remapping, all splits of one unit run
  // on the same XCD (workgroups are dealt to the 8 XCDs round-robin), so the
  // split merge reads partials that the same L2 slice produced.
  int unit, split;
  {
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

  // ---- query rows of this chunk -> registers ----
  const int kt = lane / LPT;
  const int kc = lane % LPT;
  const int vts = lane / VLPT;
  const int vj = lane % VLPT;
  const int vc = vj >> 2;
  const int gK = (kc * 32) / a.G;

  int lim[ROWS];
  uint32_t qp[DOT2 ? ROWS : 1][16];
  float qf[DOT2 ? 1 : ROWS][32];
  float qinit[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int rho = rc * ROWS + r;
    const bool row_ok = rho < a.rows_total;
    const int hl = row_ok ? rho / a.Sq : 0;
    const int qi = row_ok ? rho % a.Sq : 0;
    const int head = kvh * a.ratio + hl;
    int lm = a.causal ? L - a.Sq + qi + 1 : L;
    lm = lm < 0 ? 0 : lm;
    lim[r] = row_ok ? lm : 0;
    const int64_t qbase = (int64_t)b * a.qs_b + (int64_t)head * a.qs_h + (int64_t)qi * a.qs_s;
    float qsum = 0.0f;
    if constexpr (DOT2) {
      const uint16_t* q16 = (const uint16_t*)a.q;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
#pragma unroll
        for (int m = 0; m < 4; ++m) {
          const int e0 = kc * 32 + 8 * k + m;
          uint32_t lo = 0, hi = 0;
          if (row_ok) {
            lo = q16[qbase + (int64_t)e0 * a.qs_d];
            hi = q16[qbase + (int64_t)(e0 + 4) * a.qs_d];
          }
          qp[r][4 * k + m] = lo | (hi << 16);
          if constexpr (QM == KVQ_BF16) qsum += bf16_bits_to_f32(lo) + bf16_bits_to_f32(hi);
        }
      }
      qinit[r] = QM == KVQ_BF16 ? -136.0f * qsum : 0.0f;
    } else {
      const float* q32 = (const float*)a.q;
#pragma unroll
      for (int e = 0; e < 32; ++e) {
        const float v = row_ok ? q32[qbase + (int64_t)(kc * 32 + e) * a.qs_d] : 0.0f;
        qf[r][e] = v;
        qsum += v;
      }
      qinit[r] = -8.0f * qsum;
    }
  }

  // ---- per-wave running softmax state ----
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
  const int64_t ks_bh = (int64_t)b * a.kss_b + (int64_t)kvh * a.kss_h;
  const int64_t vs_bh = (int64_t)b * a.vss_b + (int64_t)kvh * a.vss_h;
  const int last_tok = L > 0 ? L - 1 : 0;

  for (int base = wave; base < ntiles; base += 4 * CH) {
    // ---- issue every load of the chunk first ----
    uint4 kcode[CH];
    uint32_t vcode[CH][4];
    float sk[CH], sv[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int tile = base + 4 * i;
      const int t0 = t_begin + tile * TPT;
      if (tile < ntiles) {
        const int tk = min(t0 + kt, last_tok);
        kcode[i] = *(const uint4*)(kp_bh + (int64_t)tk * a.kps_s + 16 * kc);
        sk[i] = load_scale(a.ks, ks_bh + (int64_t)tk * a.kss_s + gK, a.scale_dtype);
        sv[i] = load_scale(a.vs, vs_bh + (int64_t)tk * a.vss_s + gK, a.scale_dtype);
#pragma unroll
        for (int k = 0; k < 4; ++k) {
          const int tv = min(t0 + vts + VTS * k, last_tok);
          vcode[i][k] = *(const uint32_t*)(vp_bh + (int64_t)tv * a.vps_s + 4 * vj);
        }
      } else {
        kcode[i] = make_uint4(0, 0, 0, 0);
        sk[i] = 0.0f;
        sv[i] = 0.0f;
#pragma unroll
        for (int k = 0; k < 4; ++k) vcode[i][k] = 0u;
      }
    }

    // ---- K phase: scores of every row for CH tiles ----
    float s[CH][ROWS];
    bool tv_ok[CH];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      const int tile = base + 4 * i;
      const int t = t_begin + tile * TPT + kt;
      tv_ok[i] = (tile < ntiles) && (t < t_end);
      float acc[ROWS];
#pragma unroll
      for (int r = 0; r < ROWS; ++r) acc[r] = qinit[r];
      const uint32_t wk[4] = {kcode[i].x, kcode[i].y, kcode[i].z, kcode[i].w};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t w = wk[k];
        if constexpr (QM == KVQ_BF16) {
          const uint32_t p0 = (w & kNibPairs) | kBf16Magic;
          const uint32_t p1 = ((w >> 4) & kNibPairs) | kBf16Magic;
          const uint32_t p2 = ((w >> 8) & kNibPairs) | kBf16Magic;
          const uint32_t p3 = ((w >> 12) & kNibPairs) | kBf16Magic;
#pragma unroll
          for (int r = 0; r < ROWS; ++r) {
            acc[r] = dot2_bf16(qp[r][4 * k + 0], p0, acc[r]);
            acc[r] = dot2_bf16(qp[r][4 * k + 1], p1, acc[r]);
            acc[r] = dot2_bf16(qp[r][4 * k + 2], p2, acc[r]);
            acc[r] = dot2_bf16(qp[r][4 * k + 3], p3, acc[r]);
          }
        } else if constexpr (QM == KVQ_F16) {
          const f16x2_t bias = {(_Float16)-1032.0f, (_Float16)-1032.0f};
          uint32_t p[4];
#pragma unroll
          for (int m = 0; m < 4; ++m) {
            const f16x2_t h =
                __builtin_bit_cast(f16x2_t, ((w >> (4 * m)) & kNibPairs) | kF16Magic) + bias;
            p[m] = __builtin_bit_cast(uint32_t, h);
          }
#pragma unroll
          for (int r = 0; r < ROWS; ++r) {
#pragma unroll
            for (int m = 0; m < 4; ++m) acc[r] = dot2_f16(qp[r][4 * k + m], p[m], acc[r]);
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
        bool ok = tv_ok[i];
        if constexpr (ROWMASK) ok = ok && (t < lim[r]);
        s[i][r] = ok ? part : kNeg;
      }
    }

    // ---- chunk max, rescale of the running state ----
    float m_new[ROWS];
    bool grow = false;
#pragma unroll
    for (int r = 0; r < ROWS; ++r) {
      float mx = s[0][r];
#pragma unroll
      for (int i = 1; i < CH; ++i) mx = fmaxf(mx, s[i][r]);
      mx = wave_max(mx);
      m_new[r] = fmaxf(m_run[r], mx);
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

    // ---- probabilities -> weights w = p * v_scale -> LDS ----
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

    // ---- V phase ----
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if (base + 4 * i >= ntiles) break;
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

  // ---- wave partial -> LDS ----
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
#pragma unroll
    for (int m = 0; m < 8; ++m) {
      float v = o_acc[r][m];
      if constexpr (DOT2) v = fmaf(-136.0f, wsum[r], v);
#pragma unroll
      for (int step = VLPT; step < 64; step *= 2) v += __shfl_xor(v, step, 64);
      o_acc[r][m] = v;
    }
    const float lsum = wave_sum(kc == 0 ? l_acc[r] : 0.0f);
    if (lane == 0) {
      ml_lds[wave][r][0] = m_run[r];
      ml_lds[wave][r][1] = lsum;
    }
    if (vts == 0) {
#pragma unroll
      for (int m = 0; m < 8; ++m) o_lds[wave][r][8 * vj + m] = o_acc[r][m];
    }
  }
  __syncthreads();

  // ---- merge the 4 waves; either write the output or this split's partial ----
  const bool single = a.n_split == 1;
  for (int idx = tid; idx < ROWS * D; idx += 256) {
    const int r = idx / D, d = idx % D;
    float M = kNeg;
#pragma unroll
    for (int w = 0; w < 4; ++w) M = fmaxf(M, ml_lds[w][r][0]);
    float Ls = 0.0f, Os = 0.0f;
#pragma unroll
    for (int w = 0; w < 4; ++w) {
      const float f = __builtin_amdgcn_exp2f(ml_lds[w][r][0] - M);
      Ls += ml_lds[w][r][1] * f;
      Os += o_lds[w][r][d] * f;
    }
    if (single) {
      const int rho = rc * ROWS + r;
      if (rho < a.rows_total) {
        const int head = kvh * a.ratio + rho / a.Sq, qi = rho % a.Sq;
        const int64_t oi = (int64_t)b * a.os_b + (int64_t)head * a.os_h + (int64_t)qi * a.os_s +
                           (int64_t)d * a.os_d;
        store_from_f32(a.out, oi, QM, Ls > 0.0f ? Os / Ls : 0.0f);
      }
    } else {
      const int64_t slot = ((int64_t)unit * a.n_split + split) * ROWS + r;
      a.ws_o[slot * D + d] = Os;
      if (d == 0) {
        a.ws_ml[slot * 2 + 0] = M;
        a.ws_ml[slot * 2 + 1] = Ls;
      }
    }
  }
  if (single) return;

  // ---- split merge by the last workgroup of this unit ----
  __threadfence();
  __syncthreads();
  if (tid == 0) {
    const unsigned prev = __hip_atomic_fetch_add(&a.ws_cnt[unit], 1u, __ATOMIC_ACQ_REL,
                                                 __HIP_MEMORY_SCOPE_AGENT);
    last_flag = prev == (unsigned)(a.n_split - 1);
  }
  __syncthreads();
  if (!last_flag) return;
  __threadfence();

  for (int idx = tid; idx < ROWS * D; idx += 256) {
    const int r = idx / D, d = idx % D;
    const int rho = rc * ROWS + r;
    if (rho >= a.rows_total) continue;
    const int64_t slot0 = (int64_t)unit * a.n_split * ROWS + r;
    float M = kNeg;
    for (int sp = 0; sp < a.n_split; ++sp) M = fmaxf(M, a.ws_ml[(slot0 + (int64_t)sp * ROWS) * 2]);
    float Ls = 0.0f, Os = 0.0f;
    for (int sp = 0; sp < a.n_split; ++sp) {
      const int64_t slot = slot0 + (int64_t)sp * ROWS;
      const float f = __builtin_amdgcn_exp2f(a.ws_ml[slot * 2] - M);
      Ls += a.ws_ml[slot * 2 + 1] * f;
      Os += a.ws_o[slot * D + d] * f;
    }
    const int head = kvh * a.ratio + rho / a.Sq, qi = rho % a.Sq;
    const int64_t oi = (int64_t)b * a.os_b + (int64_t)head * a.os_h + (int64_t)qi * a.os_s +
                       (int64_t)d * a.os_d;
    store_from_f32(a.out, oi, QM, Ls > 0.0f ? Os / Ls : 0.0f);
  }
  if (tid == 0) a.ws_cnt[unit] = 0u;
}

// ---------------------------------------------------------------------------
// Host side: planning and dispatch.

static int rows_per_chunk(int rows_total, int q_dtype) {
  const int cap = q_dtype == KVQ_F32 ? 2 : 8;
  int r = 1;
  while (r < rows_total && r < cap) r *= 2;
  return r;
}

static int tokens_per_tile(int64_t D) { return (int)(64 / (D / 32)); }

struct Plan {
  int rows, row_chunks, n_units, n_split, split_len;
};

static int make_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D, int64_t s_max,
                     int q_dtype, int64_t n_split_req, int64_t num_cus, Plan* p) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Sq < 1 || s_max < 0 || Hq % Hkv != 0) return KVQ_EINVAL;
  if (!(D == 64 || D == 128)) return KVQ_EUNSUP;
  const int64_t rows_total = (Hq / Hkv) * Sq;
  p->rows = rows_per_chunk((int)rows_total, q_dtype);
  p->row_chunks = (int)((rows_total + p->rows - 1) / p->rows);
  const int64_t units = B * Hkv * p->row_chunks;
  if (units > (1ll << 30)) return KVQ_EUNSUP;
  p->n_units = (int)units;
  const int tpt = tokens_per_tile(D);
  const int64_t max_split = std::max<int64_t>(1, (s_max + 4 * tpt - 1) / (4 * tpt));
  int64_t ns = n_split_req;
  if (ns <= 0) {
    const int64_t cus = std::max<int64_t>(1, num_cus);
    ns = (cus + units - 1) / units;
  }
  ns = std::max<int64_t>(1, std::min<int64_t>(ns, max_split));
  int64_t split_len = (s_max + ns - 1) / ns;
  split_len = std::max<int64_t>(tpt, ((split_len + tpt - 1) / tpt) * tpt);
  ns = std::max<int64_t>(1, (s_max + split_len - 1) / split_len);
  if (units * ns > 0x7fffffffll) return KVQ_EUNSUP;
  p->n_split = (int)ns;
  p->split_len = (int)std::min<int64_t>(split_len, 0x7fffffffll);
  return KVQ_OK;
}

static int64_t workspace_bytes_for(const Plan& p, int64_t D) {
  if (p.n_split <= 1) return 0;
  const int64_t slots = (int64_t)p.n_units * p.n_split * p.rows;
  const int64_t cnt = ((int64_t)p.n_units * 4 + 255) / 256 * 256;
  const int64_t ml = (slots * 2 * 4 + 255) / 256 * 256;
  const int64_t o = slots * D * 4;
  return cnt + ml + o;
}

template <int D, int ROWS, int QM>
static void launch_rows(const AttnArgs& a, bool rowmask, dim3 grid, hipStream_t st) {
  if (rowmask) hipLaunchKernelGGL((decode_attn_kernel<D, ROWS, QM, true>), grid, dim3(256), 0, st, a);
  else hipLaunchKernelGGL((decode_attn_kernel<D, ROWS, QM, false>), grid, dim3(256), 0, st, a);
}

template <int D, int QM>
static void launch_qm(const AttnArgs& a, int rows, bool rowmask, dim3 grid, hipStream_t st) {
  switch (rows) {
    case 1: launch_rows<D, 1, QM>(a, rowmask, grid, st); break;
    case 2: launch_rows<D, 2, QM>(a, rowmask, grid, st); break;
    case 4:
      if constexpr (QM != KVQ_F32) launch_rows<D, 4, QM>(a, rowmask, grid, st);
      break;
    default:
      if constexpr (QM != KVQ_F32) launch_rows<D, 8, QM>(a, rowmask, grid, st);
      break;
  }
}

template <int D>
static void launch_d(const AttnArgs& a, int q_dtype, int rows, bool rowmask, dim3 grid,
                     hipStream_t st) {
  switch (q_dtype) {
    case KVQ_BF16: launch_qm<D, KVQ_BF16>(a, rows, rowmask, grid, st); break;
    case KVQ_F16: launch_qm<D, KVQ_F16>(a, rows, rowmask, grid, st); break;
    default: launch_qm<D, KVQ_F32>(a, rows, rowmask, grid, st); break;
  }
}

}  // namespace kvq

using namespace kvq;

extern "C" int64_t kvq_decode_attn_num_splits(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                              int64_t D, int64_t s_max, int q_dtype,
                                              int64_t num_cus) {
  clear_error();
  if (!dtype_ok(q_dtype)) {
    set_error("kvq_decode_attn_num_splits: q dtype must be bf16/fp16/fp32");
    return KVQ_EINVAL;
  }
  Plan p;
  const int rc = make_plan(B, Hq, Hkv, Sq, D, s_max, q_dtype, 0, num_cus, &p);
  if (rc != KVQ_OK) {
    set_error("kvq_decode_attn_num_splits: unsupported or invalid shape (B=%lld Hq=%lld Hkv=%lld "
              "Sq=%lld D=%lld)", (long long)B, (long long)Hq, (long long)Hkv, (long long)Sq,
              (long long)D);
    return rc;
  }
  return p.n_split;
}

extern "C" int64_t kvq_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                                   int64_t D, int q_dtype, int64_t n_split) {
  clear_error();
  if (!dtype_ok(q_dtype) || n_split < 1) {
    set_error("kvq_decode_attn_workspace_bytes: bad q dtype or n_split");
    return KVQ_EINVAL;
  }
  // s_max only bounds n_split in planning; pass a value that keeps n_split.
  Plan p;
  const int rc = make_plan(B, Hq, Hkv, Sq, D, n_split * 4 * tokens_per_tile(D), q_dtype, n_split,
                           1, &p);
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
  Plan p;
  const int rc = make_plan(B, Hq, Hkv, Sq, D, Sk, q_dtype, n_split, 1, &p);
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
  KVQ_CHECK_ARG(Sk <= 0x7fffffffll && Sq <= 0x7fffffffll, "kvq_decode_attn: sequence too long");

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
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.ws_cnt = nullptr; a.ws_ml = nullptr; a.ws_o = nullptr;
  if (need > 0) {
    char* w = (char*)workspace;
    const int64_t slots = (int64_t)p.n_units * p.n_split * p.rows;
    const int64_t cnt = ((int64_t)p.n_units * 4 + 255) / 256 * 256;
    const int64_t ml = (slots * 2 * 4 + 255) / 256 * 256;
    a.ws_cnt = (unsigned*)w;
    a.ws_ml = (float*)(w + cnt);
    a.ws_o = (float*)(w + cnt + ml);
  }
  const bool rowmask = is_causal && Sq > 1;
  const dim3 grid((unsigned)((int64_t)p.n_units * p.n_split));
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) launch_d<128>(a, q_dtype, p.rows, rowmask, grid, st);
  else launch_d<64>(a, q_dtype, p.rows, rowmask, grid, st);
  KVQ_CHECK_LAUNCH("kvq_decode_attn");
  return KVQ_OK;
}
