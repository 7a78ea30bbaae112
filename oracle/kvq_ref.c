/*
 * kvq_ref.c — C restatement of the reference's CPU path for the INT4 KV hot
 * path. TEST INFRASTRUCTURE ONLY: used by tests/ as a second, independent
 * checker (cross-validated against oracle/kvq_oracle.py) and timed by
 * bench.py's cpu_baseline leg. The product library never links it.
 *
 *   kvqref_quantize    kernels/llama3/quantize.py:126-148 (_quantize_int4_torch)
 *   kvqref_dequantize  kernels/llama3/quantize.py:210-234 (_dequantize_int4_torch)
 *   kvqref_decode_attn dequantize + softmax(q k^T * scale) v, the reference's
 *                      attention oracle (tests/llama3/test_attention_quant_gqa.py:
 *                      21-40: dequantize, repeat_interleave over the GQA group,
 *                      SDPA) with the kernel's bottom-right causal alignment
 *                      (kernels/llama3/attention_quant.py:91-97,123).
 *
 * Values are passed as float32 (a bf16/fp16 tensor as the float32 array of its
 * values); scale_dtype / out_dtype select round-to-nearest-even narrowing:
 * 0 = bf16, 1 = fp16, 2 = fp32. Attention runs in fp32 with a split over the
 * key axis (partial max / sum / output per split, merged exactly as a
 * log-sum-exp), parallelised with OpenMP over (batch, kv head, split).
 */
#include <immintrin.h> /* F16C: _cvtss_sh / _cvtsh_ss (part of x86-64-v3) */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>
#ifdef _OPENMP
#include <omp.h>
#endif

static float round_bf16(float f) {
  uint32_t u;
  memcpy(&u, &f, 4);
  if ((u & 0x7fffffffu) > 0x7f800000u) {
    u = 0x7fc00000u;
  } else {
    u = (uint32_t)(((uint64_t)u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u);
  }
  memcpy(&f, &u, 4);
  return f;
}

static float round_f16(float f) { return _cvtsh_ss(_cvtss_sh(f, _MM_FROUND_TO_NEAREST_INT)); }

static float round_to(float f, int dt) {
  if (dt == 0) return round_bf16(f);
  if (dt == 1) return round_f16(f);
  return f;
}

int kvqref_num_threads(void) {
#ifdef _OPENMP
  return omp_get_max_threads();
#else
  return 1;
#endif
}

void kvqref_quantize(const float* x, int64_t rows, int64_t d, int64_t G, int scale_dtype,
                     uint8_t* packed, float* scales) {
  const int64_t ng = (d + G - 1) / G;
  const int64_t bpg = (G + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    const float* xr = x + r * d;
    uint8_t* pr = packed + r * ng * bpg;
    for (int64_t g = 0; g < ng; ++g) {
      float amax = 0.0f;
      for (int64_t k = 0; k < G; ++k) {
        const int64_t c = g * G + k;
        const float v = c < d ? fabsf(xr[c]) : 0.0f;
        if (v > amax) amax = v;
      }
      const float scale = amax > 0.0f ? amax / 7.0f : 1.0f;
      for (int64_t j = 0; j < bpg; ++j) {
        unsigned nib[2];
        for (int e = 0; e < 2; ++e) {
          const int64_t k = 2 * j + e;
          if (k >= G) {
            nib[e] = 0;
            continue;
          }
          const int64_t c = g * G + k;
          const float v = c < d ? xr[c] : 0.0f;
          float q = nearbyintf(v / scale); /* default FE_TONEAREST: half to even */
          if (q < -8.0f) q = -8.0f;
          if (q > 7.0f) q = 7.0f;
          nib[e] = (unsigned)((int)q + 8);
        }
        pr[g * bpg + j] = (uint8_t)(nib[0] | (nib[1] << 4));
      }
      scales[r * ng + g] = round_to(scale, scale_dtype);
    }
  }
}

void kvqref_dequantize(const uint8_t* packed, const float* scales, int64_t rows, int64_t ng,
                       int64_t G, int64_t d_out, int out_dtype, float* out) {
  const int64_t bpg = (G + 1) / 2;
#pragma omp parallel for schedule(static)
  for (int64_t r = 0; r < rows; ++r) {
    for (int64_t c = 0; c < d_out; ++c) {
      const int64_t g = c / G, k = c % G;
      const uint8_t byte = packed[r * ng * bpg + g * bpg + k / 2];
      const int nib = (k & 1) ? (byte >> 4) : (byte & 15);
      out[r * d_out + c] = round_to((float)(nib - 8) * scales[r * ng + g], out_dtype);
    }
  }
}

/* Dequantize one packed row of D elements (group size G) into dst. */
static void deq_row(const uint8_t* p, const float* s, int64_t D, int64_t G, float* dst) {
  const int64_t bpg = (G + 1) / 2;
  for (int64_t c = 0; c < D; ++c) {
    const int64_t g = c / G, k = c % G;
    const uint8_t byte = p[g * bpg + k / 2];
    const int nib = (k & 1) ? (byte >> 4) : (byte & 15);
    dst[c] = (float)(nib - 8) * s[g];
  }
}

int kvqref_decode_attn(const float* q, const uint8_t* kp, const float* ks, const uint8_t* vp,
                       const float* vs, int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                       int64_t Sk, int64_t D, int64_t G, const int32_t* seq_lens, int causal,
                       float scale, float* out, int nthreads) {
  if (B <= 0 || Hq <= 0 || Hkv <= 0 || Sq <= 0 || D <= 0 || G <= 0 || Hq % Hkv) return -1;
  const int64_t ratio = Hq / Hkv, rows = ratio * Sq;
  const int64_t ng = (D + G - 1) / G, W = ng * ((G + 1) / 2);
#ifdef _OPENMP
  if (nthreads <= 0) nthreads = omp_get_max_threads();
#else
  nthreads = 1;
#endif
  int64_t n_split = (2 * (int64_t)nthreads + B * Hkv - 1) / (B * Hkv);
  if (n_split < 1) n_split = 1;
  int64_t split_len = (Sk + n_split - 1) / n_split;
  if (split_len < 64) split_len = 64;
  n_split = Sk > 0 ? (Sk + split_len - 1) / split_len : 1;
  const int64_t tasks = B * Hkv * n_split;
  /* partials: [tasks][rows] (m, l) and [tasks][rows][D] o */
  float* pm = (float*)malloc(sizeof(float) * tasks * rows);
  float* pl = (float*)malloc(sizeof(float) * tasks * rows);
  float* po = (float*)malloc(sizeof(float) * tasks * rows * D);
  if (!pm || !pl || !po) {
    free(pm); free(pl); free(po);
    return -2;
  }
#pragma omp parallel for schedule(dynamic) num_threads(nthreads)
  for (int64_t t = 0; t < tasks; ++t) {
    const int64_t sp = t % n_split, bh = t / n_split, h = bh % Hkv, b = bh / Hkv;
    int64_t L = Sk;
    if (seq_lens) L = seq_lens[b] < 0 ? 0 : (seq_lens[b] < Sk ? seq_lens[b] : Sk);
    const int64_t j0 = sp * split_len, j1 = (j0 + split_len < L) ? j0 + split_len : L;
    const int64_t n = j1 > j0 ? j1 - j0 : 0;
    float* kbuf = (float*)malloc(sizeof(float) * (n > 0 ? n : 1) * D);
    float* vbuf = (float*)malloc(sizeof(float) * (n > 0 ? n : 1) * D);
    float* sc = (float*)malloc(sizeof(float) * (n > 0 ? n : 1));
    for (int64_t j = 0; j < n; ++j) {
      const int64_t row = (b * Hkv + h) * Sk + j0 + j;
      deq_row(kp + row * W, ks + row * ng, D, G, kbuf + j * D);
      deq_row(vp + row * W, vs + row * ng, D, G, vbuf + j * D);
    }
    for (int64_t rr = 0; rr < rows; ++rr) {
      const int64_t hq = h * ratio + rr / Sq, qi = rr % Sq;
      const float* qv = q + ((b * Hq + hq) * Sq + qi) * D;
      const int64_t lim = causal ? (L - Sq + qi + 1) : L; /* keys j < lim */
      float m = -INFINITY, l = 0.0f;
      float* o = po + (t * rows + rr) * D;
      for (int64_t c = 0; c < D; ++c) o[c] = 0.0f;
      for (int64_t j = 0; j < n; ++j) {
        if (j0 + j >= lim) { sc[j] = -INFINITY; continue; }
        float acc = 0.0f;
        const float* kr = kbuf + j * D;
        for (int64_t c = 0; c < D; ++c) acc += qv[c] * kr[c];
        sc[j] = acc * scale;
        if (sc[j] > m) m = sc[j];
      }
      if (m != -INFINITY) {
        for (int64_t j = 0; j < n; ++j) {
          if (sc[j] == -INFINITY) continue;
          const float p = expf(sc[j] - m);
          l += p;
          const float* vr = vbuf + j * D;
          for (int64_t c = 0; c < D; ++c) o[c] += p * vr[c];
        }
      }
      pm[t * rows + rr] = m;
      pl[t * rows + rr] = l;
    }
    free(kbuf); free(vbuf); free(sc);
  }
  /* merge the splits */
#pragma omp parallel for schedule(static) num_threads(nthreads)
  for (int64_t u = 0; u < B * Hkv * rows; ++u) {
    const int64_t rr = u % rows, bh = u / rows, h = bh % Hkv, b = bh / Hkv;
    const int64_t hq = h * ratio + rr / Sq, qi = rr % Sq;
    float M = -INFINITY;
    for (int64_t sp = 0; sp < n_split; ++sp) {
      const float m = pm[(bh * n_split + sp) * rows + rr];
      if (m > M) M = m;
    }
    float* dst = out + ((b * Hq + hq) * Sq + qi) * D;
    for (int64_t c = 0; c < D; ++c) dst[c] = 0.0f;
    if (M == -INFINITY) continue;
    float Ls = 0.0f;
    for (int64_t sp = 0; sp < n_split; ++sp) {
      const int64_t t = bh * n_split + sp;
      const float m = pm[t * rows + rr];
      if (m == -INFINITY) continue;
      const float f = expf(m - M);
      Ls += pl[t * rows + rr] * f;
      const float* o = po + (t * rows + rr) * D;
      for (int64_t c = 0; c < D; ++c) dst[c] += o[c] * f;
    }
    for (int64_t c = 0; c < D; ++c) dst[c] /= Ls;
  }
  free(pm); free(pl); free(po);
  return 0;
}

/*
 * Exhaustive check of the division-free group scale the HIP kernels use
 * (kv-cache-triton_amd/csrc/kvq_common.h group_scale): for every
 * non-negative finite fp32 value am with bit pattern in [lo, hi), the
 * product q = am * RN(1/7) corrected once with a fused multiply-add,
 * q + (am - 7 q) * RN(1/7), must equal the IEEE quotient am / 7 that the
 * reference's torch path computes (kernels/llama3/quantize.py:137-141).
 * Returns the number of bit patterns for which it does not ([0, 0x7f800000)
 * covers zero, the subnormals and every normal value).
 */
int64_t kvqref_check_div7(uint32_t lo, uint32_t hi) {
  const float inv7 = 1.0f / 7.0f;
  int64_t bad = 0;
  if (hi > 0x7f800000u) hi = 0x7f800000u;
#pragma omp parallel for schedule(static) reduction(+ : bad)
  for (int64_t u = lo; u < (int64_t)hi; ++u) {
    const uint32_t w = (uint32_t)u;
    float am;
    memcpy(&am, &w, 4);
    const float q = am * inv7;
    const float q1 = fmaf(fmaf(-q, 7.0f, am), inv7, q);
    const float e = am / 7.0f;
    if (memcmp(&q1, &e, 4) != 0) ++bad;
  }
  return bad;
}

/* Pins the divide-free rounding of the quantize kernels (rint_quotient in
 * kv-cache-triton_amd/csrc/kvq_common.h): with inv within `ulps` ulp of
 * 1 / s (the device takes v_rcp_f32, 1 ulp), t = RN(x * inv) and r = rint(t),
 * every element whose t is not within 2^-thr of a half-integer must give
 * r == rint(RN(x / s)), the quotient the reference rounds
 * (kernels/llama3/quantize.py:142-144). Samples n scales s (normal, in
 * [2^-100, 2^100], as the kernels' fast path requires) and per scale random
 * elements |x| <= 7 s plus elements a few ulps from every tie (k + 1/2) s;
 * each against every inverse from RN(1/s) - ulps to RN(1/s) + ulps ulp.
 * Returns the number of elements the fast path would round differently (0
 * for the kernels' threshold, 17; a threshold far too tight shows misses). */
static uint64_t kvqref_rng(uint64_t* s) {
  *s ^= *s << 13;
  *s ^= *s >> 7;
  *s ^= *s << 17;
  return *s;
}

int64_t kvqref_check_rint_margin(uint64_t seed, int64_t n, int ulps, int thr) {
  int64_t bad = 0;
  const float margin = 0.5f - ldexpf(1.0f, -thr);
#pragma omp parallel for schedule(static) reduction(+ : bad)
  for (int64_t i = 0; i < n; ++i) {
    uint64_t st = seed * 0x9E3779B97F4A7C15ull + (uint64_t)i * 0xD1B54A32D192ED03ull + 1;
    for (int w = 0; w < 4; ++w) kvqref_rng(&st);
    const int e = (int)(kvqref_rng(&st) % 200) - 100;
    const float s = ldexpf(1.0f + (float)(kvqref_rng(&st) % 8388608u) / 8388608.0f, e);
    const float inv0 = 1.0f / s;
    float xs[64];
    int nx = 0;
    for (int j = 0; j < 16; ++j) {  /* random elements in [-7 s, 7 s] */
      const float u = (float)((double)(kvqref_rng(&st) % 14000001u) / 1000000.0 - 7.0);
      xs[nx++] = u * s;
    }
    for (int k = -8; k <= 6 && nx < 62; k += 2) { /* near the ties (k + 1/2) s */
      const float tie = ((float)k + 0.5f + (float)(kvqref_rng(&st) % 2)) * s;
      const int d = (int)(kvqref_rng(&st) % 7) - 3;
      float x = tie;
      for (int m = 0; m < (d < 0 ? -d : d); ++m) x = nextafterf(x, d < 0 ? -INFINITY : INFINITY);
      xs[nx++] = x;
      xs[nx++] = -x;
    }
    for (int q = -ulps; q <= ulps; ++q) {
      float inv = inv0;
      for (int m = 0; m < (q < 0 ? -q : q); ++m) inv = nextafterf(inv, q < 0 ? 0.0f : INFINITY);
      for (int j = 0; j < nx; ++j) {
        const float x = xs[j];
        if (fabsf(x) > 7.0f * s) continue;
        const float t = x * inv;
        const float r = rintf(t);
        if (fabsf(t - r) > margin) continue; /* the kernels divide */
        if (r != rintf(x / s)) ++bad;
      }
    }
  }
  return bad;
}

/* Pins the packed form of the same rounding in the vector quantize kernel
 * (quantize_vec_kernel, kv-cache-triton_amd/csrc/kvq_quant.hip): t =
 * RN(x * inv + 8) in one fma, u = RN(t + 2^23) (t rounded to an integer,
 * ties to even), c = u - 2^23 and r = t - c (both exact). An element with
 * |r| <= 1/2 - 2^-thr must have c - 8 == rint(RN(x / s)) and c in [1, 15]
 * (so no clamp is needed); the kernel divides for the others. Samples as
 * kvqref_check_rint_margin, plus per scale the group extremes x = +-am for an
 * absmax am with s = RN(am / 7), the scale the kernels compute. Returns the
 * number of elements the fast path would get wrong. */
int64_t kvqref_check_rint_margin_fma8(uint64_t seed, int64_t n, int ulps, int thr) {
  int64_t bad = 0;
  const float margin = 0.5f - ldexpf(1.0f, -thr);
  const float magic = 8388608.0f; /* 2^23 */
#pragma omp parallel for schedule(static) reduction(+ : bad)
  for (int64_t i = 0; i < n; ++i) {
    uint64_t st = seed * 0x9E3779B97F4A7C15ull + (uint64_t)i * 0xD1B54A32D192ED03ull + 7;
    for (int w = 0; w < 4; ++w) kvqref_rng(&st);
    const int e = (int)(kvqref_rng(&st) % 200) - 100;
    const float am = ldexpf(1.0f + (float)(kvqref_rng(&st) % 8388608u) / 8388608.0f, e);
    const float s = am / 7.0f;
    const float inv0 = 1.0f / s;
    float xs[66];
    int nx = 0;
    xs[nx++] = am;
    xs[nx++] = -am;
    for (int j = 0; j < 16; ++j) { /* random elements in [-am, am] */
      const float u = (float)((double)(kvqref_rng(&st) % 14000001u) / 1000000.0 - 7.0);
      const float x = u * s;
      xs[nx++] = fabsf(x) <= am ? x : (x < 0 ? -am : am);
    }
    for (int k = -8; k <= 6 && nx < 64; k += 2) { /* near the ties (k + 1/2) s */
      const float tie = ((float)k + 0.5f + (float)(kvqref_rng(&st) % 2)) * s;
      const int d = (int)(kvqref_rng(&st) % 7) - 3;
      float x = tie;
      for (int m = 0; m < (d < 0 ? -d : d); ++m) x = nextafterf(x, d < 0 ? -INFINITY : INFINITY);
      xs[nx++] = x;
      xs[nx++] = -x;
    }
    for (int q = -ulps; q <= ulps; ++q) {
      float inv = inv0;
      for (int m = 0; m < (q < 0 ? -q : q); ++m) inv = nextafterf(inv, q < 0 ? 0.0f : INFINITY);
      for (int j = 0; j < nx; ++j) {
        const float x = xs[j];
        if (fabsf(x) > am) continue;
        const float t = fmaf(x, inv, 8.0f);
        const float u = t + magic;
        const float c = u - magic;
        const float r = t - c;
        if (fabsf(r) > margin) continue; /* the kernel divides */
        float ref = rintf(x / s);
        ref = fminf(fmaxf(ref, -8.0f), 7.0f);
        if (c - 8.0f != ref || c < 1.0f || c > 15.0f) ++bad;
      }
    }
  }
  return bad;
}
