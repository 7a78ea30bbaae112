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
// byte crosses HBM once, and B*Hkv*n_split workgroups fill the CUs. Splits are
// balanced to the token (split s of a sequence of L keys covers
// [s*L/n_split, (s+1)*L/n_split)), so ragged batches stay balanced too. Partial
// (max, sum, o) triples are merged across the waves of a workgroup in LDS and
// then across splits by the last workgroup of the unit to finish (all splits of
// a unit run on one XCD, so the partials go through that XCD's L2; arrivals
// are counted by a device-scope atomic), which writes the output and re-arms
// the counter. In a decode step
// the same launch also quantizes the new token's K/V into the cache row after
// the last one, and the unit's last split attends it from registers.
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
//     32-dim chunk, so the per-chunk value scale rides in A: bf16 weights,
//     or for fp16 models fp16 weights, with the power of two of the 4
//     tokens' largest scale carried by the code operand (PV16 below).
//   The VALU only converts nibbles to bf16/fp16 and runs the softmax.
// decode_attn_valu_kernel (fp32 queries or fp32 scales) keeps exact fp32
//   arithmetic (v_fmac) for the 1e-4 bar of fp32 inputs; MHA-sized row counts.
//
// Nibble -> number: a magic-number OR makes an exact float of 128 + n (bf16,
// 0x4300 | n) or 1024 + n (fp16, 0x6400 | n).
//   bf16: scores accumulate q*(128+n) on top of an initial -136*sum(q) per
//         chunk; values accumulate w*(128+n) and subtract 136*sum(w) at the
//         end, sum(w) coming from one extra MFMA on the same rounded weights.
//   fp16: scores take the same form with 1024 + n and -1032; values (PV16)
//         accumulate w*2^(E-25)(1024+n) and subtract the same product with
//         n = 8, one extra MFMA.
// Softmax runs in base 2 with sm_scale*log2(e) folded into the key scale.
#include <algorithm>
#include <cmath>
#include <cstring>
#include <mutex>
#include <type_traits>

#include "kvq_common.h"

namespace kvq {

// Phase stamps (instrumented builds only: -DKVQ_PHASE_STAMPS, the measurement
// library behind bench.py --stream-probe; the product library compiles these
// to nothing). Lane 0 of each wave writes the 100 MHz s_memrealtime clock at
// fixed points of the decode step into a.stamps[(workgroup * 16 + wave) *
// kPhaseSlots + point] (a kernel argument, so the pointer sits in scalar
// registers and a stamp is one clock read and one store); KVQ_STAMP_AFTER
// first waits for the value x (a load result), so the stamp marks its arrival.
constexpr int kPhaseSlots = 16;
#if defined(KVQ_PHASE_STAMPS)
#define KVQ_STAMP(point) ::kvq::phase_stamp(a.stamps, point)
#define KVQ_STAMP_AFTER(point, x)          \
  do {                                     \
    asm volatile("" ::"v"(x));             \
    ::kvq::phase_stamp(a.stamps, point);   \
  } while (0)
#else
#define KVQ_STAMP(point) \
  do {                   \
  } while (0)
#define KVQ_STAMP_AFTER(point, x) \
  do {                            \
  } while (0)
#endif
// Stamp points: 0 entry, 1 first tiles' loads issued, 2 first tile's keys
// arrived, 3 its values arrived, 4 tile loop done, 5 workgroup fold done,
// 6 partial stores acknowledged, 7 arrival counted (thread 0), 8 merge start,
// 9 merge inputs arrived, 10 merged output computed, 11 exit. Slot 12 holds
// the wave's XCC id (written with the entry stamp), not a time.
constexpr int kXccSlot = 12;

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
  int n_split, causal, scale_dtype, q_vec, out_vec;
  int grid_y;  // the launch's gridDim.y (read from here: the dispatch's own copy
               // would be one more scalar load round trip in the prologue)
  float scale_log2;
  // launch constants computed on the host, so that the prologue (which every
  // wave runs before it can issue a load) has no divide: unit = (b * Hkv + kvh)
  // * row_chunks + rc, query row rho = (head - kvh * ratio) * Sq + qi
  FastDiv div_rc, div_hkv, div_sq, div_g, div_ns;
  int ng;             // scales per token row, ceil(D / G)
  uint32_t gsh_pack;  // byte c: bit offset of 32-dim chunk c's scale in a token's scale row
  // decode step (append != 0): the new token's K/V rows [B, Hkv, 1, D] (q's
  // dtype, unit inner stride), quantized and written at each sequence's old
  // length (seq_lens[b], or pos0 for all) and attended along with the cache
  int append, pos0;
  const void* knew;
  const void* vnew;
  int64_t kns_b, kns_h, vns_b, vns_h;
  // paged cache (kernels instantiated with PAGED): kp/ks/vp/vs are pools
  // [Hkv, n_blocks << page_shift, ...] (batch strides 0, row strides k*s_s),
  // sequence b's token t is pool row bt[b * bt_stride + (t >> page_shift)]
  // << page_shift | (t & (page size - 1)); entries outside [0, n_blocks), or
  // pages >= bt_cols, have no rows. pool_rows = n_blocks << page_shift.
  const int32_t* bt;
  int64_t bt_stride;
  int bt_cols, n_blocks, page_shift;
  uint32_t pool_rows;
  uint32_t* ws_cnt;  // [kCntUnits] arrival counters, kCntStride words apart
                     // (zero between calls)
  float* ws_ml;      // [n_units][n_split][ROWS][2]  (max, sum)
  float* ws_o;       // [n_units][n_split][ROWS][D]
#if defined(KVQ_PHASE_STAMPS)
  unsigned long long* stamps;  // phase stamps, or null
#endif
};

#if defined(KVQ_PHASE_STAMPS)
__device__ __forceinline__ void phase_stamp(unsigned long long* p, int point) {
  // compiler fences: no memory operation moves across the clock read
  asm volatile("" ::: "memory");
  const unsigned long long t = __builtin_amdgcn_s_memrealtime();
  asm volatile("" ::: "memory");
  if (p != nullptr && (threadIdx.x & 63) == 0) {
    const size_t wg = blockIdx.x + (size_t)gridDim.x * (blockIdx.y + (size_t)gridDim.y * blockIdx.z);
    unsigned long long* slot = p + (wg * 16 + (threadIdx.x >> 6)) * kPhaseSlots;
    slot[point] = t;
    // at entry, also the XCD the wave runs on: HW_REG_XCC_ID (hwreg 20),
    // bits [3:0]
    if (point == 0) slot[kXccSlot] = __builtin_amdgcn_s_getreg(20 | (0 << 6) | ((4 - 1) << 11));
  }
}
#endif

constexpr float kNeg = -1.0e30f;
constexpr int kMaxSplit = 64;  // split-K fan-out cap (keeps split * L and merge offsets in 32 bits)
constexpr float kLazyMax = 8.0f;  // running-max slack of the MFMA kernel (log2 units)
constexpr int kCntStride = 16;  // uint32 words between counters (64 bytes)
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

// Lane swaps of gfx950: permlane32 exchanges lanes 32-63 of `x` with lanes
// 0-31 of `y`; permlane16 exchanges the odd 16-lane rows of `x` with the even
// rows of `y`. The two results are read out of the builtin's two-element
// vector by value (a bit cast applied directly to an element of it reads
// element 0 with this toolchain).
__device__ __forceinline__ void permlane32_swap(float& x, float& y) {
  const auto r = __builtin_amdgcn_permlane32_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, y), false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  x = __builtin_bit_cast(float, r0);
  y = __builtin_bit_cast(float, r1);
}
__device__ __forceinline__ void permlane16_swap(float& x, float& y) {
  const auto r = __builtin_amdgcn_permlane16_swap(__builtin_bit_cast(uint32_t, x),
                                                  __builtin_bit_cast(uint32_t, y), false, false);
  const uint32_t r0 = r[0], r1 = r[1];
  x = __builtin_bit_cast(float, r0);
  y = __builtin_bit_cast(float, r1);
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

// Workgroup -> (unit, split). The grid is (8 * n_split, Y, Z) with Y Z >=
// ceil(n_units / 8): split = x / 8, unit = x % 8 + 8 (y + Y z); workgroups of
// units past the last exit at once. The hardware deals the workgroups of a
// launch to the 8 XCDs round-robin in launch order (linear index
// x + X (y + Y z), from an XCD that varies per launch), and X = 8 n_split is a
// multiple of 8, so all splits of a unit share x % 8 and run on one XCD, whose
// L2 then carries the unit's partials.
__device__ __forceinline__ bool unit_and_split(const AttnArgs& a, int& unit, int& split) {
  split = (int)(blockIdx.x >> 3);
  unit = (int)((blockIdx.x & 7u) + 8u * (blockIdx.y + (uint32_t)a.grid_y * blockIdx.z));
  return unit < a.n_units;
}

// (b, kvh, rc) of a unit.
__device__ __forceinline__ void unit_coords(const AttnArgs& a, int unit, int& b, int& kvh, int& rc) {
  const uint32_t bh = fdiv((uint32_t)unit, a.div_rc);
  rc = unit - (int)bh * a.row_chunks;
  b = (int)fdiv(bh, a.div_hkv);
  kvh = (int)bh - b * a.Hkv;
}

__device__ __forceinline__ int64_t out_index(const AttnArgs& a, int b, int kvh, int rho, int d) {
  const int hq = (int)fdiv((uint32_t)rho, a.div_sq), qi = rho - hq * a.Sq;
  const int head = kvh * a.ratio + hq;
  return (int64_t)b * a.os_b + (int64_t)head * a.os_h + (int64_t)qi * a.os_s + (int64_t)d * a.os_d;
}

// Four consecutive output elements (dims d .. d + 3 of one row) from element
// index i: one 8-byte (16-bit types) or 16-byte (fp32) store when the host
// found the output's dims contiguous and every row aligned for it (out_vec),
// else four element stores.
__device__ __forceinline__ void store4_from_f32(const AttnArgs& a, int64_t i, int dt, float x, float y, float z,
                                                float w) {
  if (a.out_vec) {
    if (dt == KVQ_F32) {
      *(float4*)((float*)a.out + i) = make_float4(x, y, z, w);
    } else {
      const bool h = dt == KVQ_F16;
      const uint32_t e0 = h ? f32_to_f16_bits(x) : f32_to_bf16_bits(x), e1 = h ? f32_to_f16_bits(y) : f32_to_bf16_bits(y);
      const uint32_t e2 = h ? f32_to_f16_bits(z) : f32_to_bf16_bits(z), e3 = h ? f32_to_f16_bits(w) : f32_to_bf16_bits(w);
      *(uint2*)((uint16_t*)a.out + i) = make_uint2(e0 | (e1 << 16), e2 | (e3 << 16));
    }
    return;
  }
  store_from_f32(a.out, i, dt, x);
  store_from_f32(a.out, i + a.os_d, dt, y);
  store_from_f32(a.out, i + 2 * a.os_d, dt, z);
  store_from_f32(a.out, i + 3 * a.os_d, dt, w);
}

__device__ __forceinline__ int div_splits(const AttnArgs& a, uint32_t n) { return (int)fdiv(n, a.div_ns); }

// Element b of a device int32 array that no kernel of this launch writes,
// read through the scalar cache (a constant-address-space load with a
// wave-uniform address is a scalar load, counted apart from the vector
// loads, so waiting for it does not wait for the query and cache loads).
__device__ __forceinline__ int load_const_i32(const int32_t* p, int i) {
  return ((const __attribute__((address_space(4))) int32_t*)p)[i];
}

// The kernel arguments the prologue of the decode kernels reads, fetched
// before their first use. Without this the compiler issues the scalar loads of
// the argument block in several batches, one per branch of the prologue, and
// each batch is a round trip before the next one can start.
__device__ __forceinline__ void fetch_prologue_args(const AttnArgs& a) {
  asm volatile("" ::"s"(a.n_units), "s"(a.grid_y), "s"(a.div_rc.m), "s"(a.div_rc.s), "s"(a.row_chunks), "s"(a.div_hkv.m),
               "s"(a.div_hkv.s), "s"(a.Hkv), "s"(a.append), "s"(a.pos0), "s"(a.Sk), "s"(a.seq_lens),
               "s"(a.rows_total), "s"(a.div_sq.m), "s"(a.div_sq.s), "s"(a.Sq), "s"(a.ratio));
  asm volatile("" ::"s"(a.q), "s"(a.qs_b), "s"(a.qs_h), "s"(a.qs_s), "s"(a.qs_d), "s"(a.q_vec), "s"(a.n_split),
               "s"(a.div_ns.m), "s"(a.div_ns.s), "s"(a.kp), "s"(a.kps_b), "s"(a.kps_h), "s"(a.kps_s));
  asm volatile("" ::"s"(a.vp), "s"(a.vps_b), "s"(a.vps_h), "s"(a.vps_s), "s"(a.ks), "s"(a.kss_b), "s"(a.kss_h),
               "s"(a.kss_s), "s"(a.vs), "s"(a.vss_b), "s"(a.vss_h), "s"(a.vss_s));
}

// Token range [t0, t1) of split `split` over a sequence of L keys
// (split s covers [s L / n_split, (s + 1) L / n_split)). The host keeps
// Sk * kMaxSplit below 2^32.
__device__ __forceinline__ void split_range(const AttnArgs& a, int L, int split, int& t0, int& t1) {
  t0 = div_splits(a, (uint32_t)split * (uint32_t)L);
  t1 = div_splits(a, (uint32_t)(split + 1) * (uint32_t)L);
}

// The same with split boundaries rounded down to multiples of 64 keys, so
// that every 64-key tile of a split lies inside one page of a paged cache
// (pages are multiples of 64 rows).
__device__ __forceinline__ void split_range64(const AttnArgs& a, int L, int split, int& t0, int& t1) {
  const int ns = a.n_split;
  t0 = split == 0 ? 0 : (div_splits(a, (uint32_t)split * (uint32_t)L) & ~63);
  t1 = split + 1 == ns ? L : (div_splits(a, (uint32_t)(split + 1) * (uint32_t)L) & ~63);
}

// Block-table entry of page pg of a sequence (bt_b = its table row), -1 past
// the row's last column. pg must be wave-uniform: the entry is read through
// the scalar cache (no kernel of the launch writes the table), so waiting for
// it does not wait for vector loads issued before it (the query rows).
__device__ __forceinline__ int32_t table_entry(const AttnArgs& a, const int32_t* bt_b, uint32_t pg) {
  return pg < (uint32_t)a.bt_cols ? load_const_i32(bt_b, (int)pg) : -1;
}

// Pool row offset of token t of a paged sequence (bt_b = its block table
// row), relative to t: row = t + delta. ok is false when no block holds t.
// t must be wave-uniform.
__device__ __forceinline__ void page_delta(const AttnArgs& a, const int32_t* bt_b, uint32_t t,
                                           uint32_t& delta, bool& ok) {
  const uint32_t pg = t >> a.page_shift;
  const int32_t blk = table_entry(a, bt_b, pg);
  ok = blk >= 0 && blk < a.n_blocks;
  delta = ((uint32_t)blk - pg) << a.page_shift;
}

// Buffer descriptor over `bytes` bytes at p (raw, 32-bit data format): loads
// at offsets >= bytes return zero and touch no memory.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* p, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(p), (short)0, (int)bytes,
                                           0x00020000);
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

constexpr int kMaxRows = 8;  // query rows per workgroup (both kernels)

struct MergeLds {
  float2 ml[kMaxSplit * kMaxRows];  // the unit's (max, sum) pair of every (split, row)
  int last;                         // this workgroup merges the unit's splits
};

// Partials cross between workgroups of one unit, which all run on one XCD
// (unit_and_split), so they travel through that XCD's L2: plain stores, and
// loads with the sc0 policy (they miss the reading CU's L1, which may hold
// lines of the workspace from an earlier launch, and hit the L2). Device-scope
// stores (written through the L2) and loads measured 0.4 us slower per launch,
// and a device-scope fence would write back and invalidate the whole L2.
constexpr int kSc0 = 1;  // cache-policy bits of a buffer load: SC0 (miss L1)
// The cache tiles' value-code and scale loads carry the nontemporal hint (NT):
// each of those instructions reads whole 128-byte lines (a value load four
// consecutive 64-byte code rows of a tile, a scale load 64 consecutive scale
// rows), streamed once. The key loads keep the default policy: a key row is
// read by four 16-byte loads, each touching 64 rows' lines in part, and with
// the hint there the north star lost 0.2 us and C4 8 us per launch. Measured
// per launch with the hint on values and scales only: north star 9.86 -> 9.55
// us, C2 7.40 -> 7.30, C5 10.10 -> 10.01, C4 unchanged (62.8-64.0 against
// 63.2-63.4); outputs bit-identical.
constexpr int kNt = 2;  // cache-policy bits of a buffer load: NT

// Bits -> float through a by-value parameter. (This toolchain's
// __builtin_bit_cast applied directly to a vector element such as v.y reads
// element 0 whatever the element named.)
__device__ __forceinline__ float u32_as_f32(uint32_t u) { return __builtin_bit_cast(float, u); }

// max without NaN canonicalisation (v_maximum3_f32 on gfx950); the operands
// here are scores, never NaN.
__device__ __forceinline__ float fmax_nc(float a, float b) { return __builtin_elementwise_maximum(a, b); }

// Reduction over the P lanes l, l + 64 / P, l + 2 * 64 / P, ... of a wave
// (P in {1, 2, 4, 8, 16}): every one of them ends with their maximum (MAX) or
// sum. Lane index bits are combined from the top: xor 32 and xor 16 through
// ds_bpermute (__shfl_xor), xor 8 and xor 4 by rotating 16-lane rows by 8 and
// then by 4 (a full reduction over a row's residue class modulo 4).
template <int P, bool MAX>
__device__ __forceinline__ float group_reduce(float v) {
  static_assert(P == 1 || P == 2 || P == 4 || P == 8 || P == 16, "group size");
  auto op = [](float x, float y) { return MAX ? fmax_nc(x, y) : x + y; };
  if constexpr (P >= 2) v = op(v, __shfl_xor(v, 32));
  if constexpr (P >= 4) v = op(v, __shfl_xor(v, 16));
  if constexpr (P >= 8) v = op(v, dpp<0x128>(v, v));  // row_ror:8
  if constexpr (P >= 16) v = op(v, dpp<0x124>(v, v)); // row_ror:4
  return v;
}

// Cross-split merge, run by the last workgroup of a unit to finish: out =
// sum_s 2^(m_s - M) o_s / sum_s 2^(m_s - M) l_s with M = max_s m_s. The
// unit's partials are Q = ROWS * D / 4 pieces of 16 bytes (4 dims of one row)
// per split; P = threads / Q threads share a piece. Lane l of wave w takes
// piece w * 64 / P + l % (64 / P) and, of the splits, those congruent to
// l / (64 / P) modulo P: the P threads of a piece are lanes 64 / P apart in
// one wave, and the 64 / P consecutive lanes of one group read consecutive
// pieces of one split (coalesced). It issues its 16-byte partial loads for a
// batch of 8 splits at once and folds them with a running max. The unit's
// (max, sum) pairs (one per split and row, shared by the threads of a row)
// are read once, before the pieces, into LDS; the barrier that publishes them
// passes while the pieces are still in flight. The P partial folds of a piece
// are then combined across lanes (group_reduce: no LDS round trip and no
// barrier after the last load), and the lanes of group 0 store the 4
// outputs of their pieces. A row no split saw a key for (all l_s = 0) yields
// zeros.
template <int ROWS, int D, int OUT_DT, int NW>
__device__ __forceinline__ void merge_splits(const AttnArgs& a, int unit, int rc, int kvh, int b,
                                             MergeLds& mg) {
  constexpr int NT = 64 * NW;
  constexpr int Q = ROWS * D / 4;  // 16-byte pieces per split
  static_assert(Q <= NT && NT % Q == 0, "merge mapping");
  constexpr int P = NT / Q;         // threads per piece
  static_assert(64 % P == 0, "a piece's threads lie in one wave");
  constexpr int BATCH = 8;
  constexpr int MLPT = (kMaxSplit * kMaxRows + NT - 1) / NT;  // (max, sum) loads per thread
  constexpr int PW = 64 / P;       // pieces per wave
  const int tid = threadIdx.x;
  const int ns = a.n_split;
  const int lane = tid & 63;
  const int piece = (tid >> 6) * PW + lane % PW, grp = lane / PW;
  const int r = piece / (D / 4), d4 = piece % (D / 4);
  const int64_t slot0 = (int64_t)unit * ns * ROWS;  // + split * ROWS + row
  const __amdgpu_buffer_rsrc_t ro =
      buffer_rsrc(a.ws_o + slot0 * D, (uint32_t)((int64_t)ns * ROWS * D * 4));
  const __amdgpu_buffer_rsrc_t rm = buffer_rsrc(a.ws_ml + slot0 * 2, (uint32_t)(ns * ROWS * 8));
  const int nml = ns * ROWS;
  uint2 mlv[MLPT];
#pragma unroll
  for (int k = 0; k < MLPT; ++k)  // index past nml: zeros, not stored below
    mlv[k] = __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(rm, (uint32_t)(tid + k * NT) * 8u, 0, kSc0));
  // the pairs' loads go out before the pieces' (the compiler would otherwise
  // place them after): loads complete in issue order, so the LDS store below
  // then waits for the pairs alone
  asm volatile("" ::: "memory");
  const int nj = (ns - grp + P - 1) / P;  // splits grp, grp + P, ... < ns
  const int nj_max = (ns + P - 1) / P;    // the same for grp 0: every lane runs the loop alike
  u32x4_t ov[BATCH];
  auto issue = [&](int j0) {
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const uint32_t sp = (uint32_t)(grp + P * (j0 + j));  // past ns: zeros, masked below
      ov[j] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(
                                              ro, (sp * Q + piece) * 16u, 0, kSc0));
    }
  };
  issue(0);
#pragma unroll
  for (int k = 0; k < MLPT; ++k) {
    const int i = tid + k * NT;
    if (i < nml) mg.ml[i] = make_float2(u32_as_f32(mlv[k].x), u32_as_f32(mlv[k].y));
  }
  __syncthreads();
  float Mr = kNeg, Lr = 0.0f;
  float4 Or = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
  for (int j0 = 0; j0 < nj_max; j0 += BATCH) {
    if (j0 > 0) issue(j0);
    if (j0 == 0) KVQ_STAMP_AFTER(9, ov[BATCH - 1].x);
    // Straight-line fold (no branch per split, so every load above is in
    // flight before the first wait): splits past the last read as zero
    // (o = 0) and take max kNeg and sum 0, so they add nothing.
    float mj[BATCH], lj[BATCH];
    float mb = Mr;
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const bool ok = j0 + j < nj;
      const float2 ml = mg.ml[ok ? (grp + P * (j0 + j)) * ROWS + r : 0];
      mj[j] = ok ? ml.x : kNeg;
      lj[j] = ok ? ml.y : 0.0f;
      mb = fmax_nc(mb, mj[j]);
    }
    const float al = __builtin_amdgcn_exp2f(Mr - mb);
    Lr *= al;
    Or.x *= al; Or.y *= al; Or.z *= al; Or.w *= al;
#pragma unroll
    for (int j = 0; j < BATCH; ++j) {
      const float f = __builtin_amdgcn_exp2f(mj[j] - mb);
      Lr = fmaf(lj[j], f, Lr);
      Or.x = fmaf(u32_as_f32(ov[j].x), f, Or.x);
      Or.y = fmaf(u32_as_f32(ov[j].y), f, Or.y);
      Or.z = fmaf(u32_as_f32(ov[j].z), f, Or.z);
      Or.w = fmaf(u32_as_f32(ov[j].w), f, Or.w);
    }
    Mr = mb;
  }
  if constexpr (P > 1) {
    const float M = group_reduce<P, true>(Mr);
    const float f = __builtin_amdgcn_exp2f(Mr - M);
    Lr = group_reduce<P, false>(Lr * f);
    Or.x = group_reduce<P, false>(Or.x * f);
    Or.y = group_reduce<P, false>(Or.y * f);
    Or.z = group_reduce<P, false>(Or.z * f);
    Or.w = group_reduce<P, false>(Or.w * f);
  }
  KVQ_STAMP_AFTER(10, Lr);
  const int rho = rc * ROWS + r;
  if (grp == 0 && rho < a.rows_total) {
    const float inv = Lr > 0.0f ? 1.0f / Lr : 0.0f;
    store4_from_f32(a, out_index(a, b, kvh, rho, 4 * d4), OUT_DT, Or.x * inv, Or.y * inv, Or.z * inv, Or.w * inv);
  }
}

// Workgroup epilogue. Each of the NW waves has left its partial (max, sum)
// per row in ml_lds[w][r] and its partial output rows in o_lds[w][r][:], both
// relative to its own max, and the caller has passed a barrier. Thread (r, d)
// folds the NW partials of its element (every thread reads the row's NW
// (max, sum) pairs itself, so no serial step or extra barrier is needed) and
// either stores the output (single split) or publishes this split's partial
// (max, sum, o). With several splits every wave then waits until its partial
// stores are complete (acknowledged by the L2 all splits of the unit share),
// and after a barrier one thread records the arrival with a device-scope
// atomic add on the unit's counter. The workgroup that completes the count
// arrived last: it merges all partials and re-arms the counter for the next
// call. Ordering: every partial store of a split is complete before its
// arrival is counted (s_waitcnt vmcnt(0) in each wave, then the barrier),
// the merger's loads are issued only after its own atomic returned the final
// count, and they miss its L1 and read the L2 the stores completed in. (One
// counter per unit: a two-level count measured 0.3 us slower.)
//
// nt (may be null): one more partial, a single key, folded in with the
// waves' ones: its score per row at nt[r] (max = score, sum = 1; kNeg for a
// row it is masked from) and its values at nt[ROWS + d], the same for every
// row. The MFMA kernel's decode step passes the new token this way.
template <int ROWS, int D, int OUT_DT, int NW>
__device__ __forceinline__ void finish_block(const AttnArgs& a, int unit, int split, int rc,
                                             int kvh, int b, const float (*o_lds)[ROWS][D],
                                             const float (*ml_lds)[ROWS][2], MergeLds& mg,
                                             const float* nt = nullptr) {
  constexpr int NT = 64 * NW;
  const int tid = threadIdx.x;
  const bool single = a.n_split == 1;
  for (int idx = tid; idx < ROWS * D; idx += NT) {
    const int r = idx / D, d = idx % D;
    float mw[NW], lw[NW];
    float M = kNeg;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float2 ml = *(const float2*)&ml_lds[w][r][0];
      mw[w] = ml.x;
      lw[w] = ml.y;
      M = fmax_nc(M, ml.x);
    }
    const float sn = nt != nullptr ? nt[r] : kNeg;
    M = fmax_nc(M, sn);
    float Ls = 0.0f, Os = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float f = __builtin_amdgcn_exp2f(mw[w] - M);
      Ls = fmaf(lw[w], f, Ls);
      Os = fmaf(o_lds[w][r][d], f, Os);
    }
    if (nt != nullptr) {  // workgroup-uniform
      const float f = sn > kNeg ? __builtin_amdgcn_exp2f(sn - M) : 0.0f;
      Ls += f;
      Os = fmaf(nt[ROWS + d], f, Os);
    }
    const int rho = rc * ROWS + r;
    if (single) {
      if (rho < a.rows_total)
        store_from_f32(a.out, out_index(a, b, kvh, rho, d), OUT_DT, Ls > 0.0f ? Os / Ls : 0.0f);
    } else {
      const int64_t slot = ((int64_t)unit * a.n_split + split) * ROWS + r;
      a.ws_o[slot * D + d] = Os;
      if (d == 0) *(float2*)&a.ws_ml[slot * 2] = make_float2(M, Ls);
    }
  }
  if (single) return;
  KVQ_STAMP(5);
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wave's partial stores are complete
  KVQ_STAMP(6);
  __syncthreads();
  uint32_t* cnt = a.ws_cnt + (int64_t)unit * kCntStride;
  if (tid == 0)
    mg.last = __hip_atomic_fetch_add(cnt, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
              (uint32_t)(a.n_split - 1);
    KVQ_STAMP(7);
  __syncthreads();
  if (!mg.last) return;
  KVQ_STAMP(8);
  merge_splits<ROWS, D, OUT_DT, NW>(a, unit, rc, kvh, b, mg);
  if (tid == 0) __hip_atomic_store(cnt, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
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
// (4,6,5,7); the query rows, read from a wave-private LDS copy, are laid out
// the same way.

// Row max / row sum over a wave for the four values x[0..3] a lane holds for
// one row set (one per query row). Two swap steps (lanes 32 apart, then rows
// of 16 lanes) leave 16-lane row g holding row g's partial over four lanes;
// four DPP rotations inside the 16-lane rows finish it in every lane, and
// lane 16 g is read out. 14 VALU operations for the four rows.
__device__ __forceinline__ float row16_max(float m) {
  asm("s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:2 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_max_f32_dpp %0, %0, %0 row_ror:1 row_mask:0xf bank_mask:0xf"
      : "+v"(m));
  return m;
}
__device__ __forceinline__ float row16_sum(float m) {
  asm("s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_ror:8 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_ror:4 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_ror:2 row_mask:0xf bank_mask:0xf\n\t"
      "s_nop 1\n\t"
      "v_add_f32_dpp %0, %0, %0 row_ror:1 row_mask:0xf bank_mask:0xf"
      : "+v"(m));
  return m;
}
__device__ __forceinline__ float readlane_f(float v, int lane) {
  return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
template <bool SUM>
__device__ __forceinline__ void wave_reduce4(const float x[4], float out[4]) {
  float a0 = x[0], a2 = x[2], a1 = x[1], a3 = x[3];
  permlane32_swap(a0, a2);  // lanes < 32: row 0 (own, lane + 32); lanes >= 32: row 2
  permlane32_swap(a1, a3);  // lanes < 32: row 1; lanes >= 32: row 3
  float u = SUM ? a0 + a2 : fmax_nc(a0, a2);
  float v = SUM ? a1 + a3 : fmax_nc(a1, a3);
  permlane16_swap(u, v);    // 16-lane row g now holds two partials of row g
  float w = SUM ? u + v : fmax_nc(u, v);
  w = SUM ? row16_sum(w) : row16_max(w);
#pragma unroll
  for (int r = 0; r < 4; ++r) out[r] = readlane_f(w, 16 * r);
}

// fp32 values of the key or value scales of this lane's token for each
// 32-dim chunk, times `mul`. raw = the token's scale row (2, 4 or 8 bytes);
// with one scale per chunk (G = 32) chunk c is 16-bit word c, otherwise the
// word at bit offset gsh[c].
template <int LPT, bool S_F16>
__device__ __forceinline__ void chunk_scales(uint2 raw, bool g32, const uint32_t (&gsh)[LPT],
                                             float mul, float (&out)[LPT]) {
  if (g32) {
#pragma unroll
    for (int c = 0; c < LPT; ++c) {
      const uint32_t dw = c < 2 ? raw.x : raw.y;
      float f;
      if constexpr (S_F16) f = f16_bits_to_f32((c & 1) ? (dw >> 16) : (dw & 0xffffu));
      else f = __builtin_bit_cast(float, (c & 1) ? (dw & 0xffff0000u) : (dw << 16));
      out[c] = f * mul;
    }
  } else {
    const uint64_t w64 = ((uint64_t)raw.y << 32) | raw.x;
#pragma unroll
    for (int c = 0; c < LPT; ++c)
      out[c] = scale16_to_f32((uint32_t)(w64 >> gsh[c]) & 0xffffu, S_F16) * mul;
  }
}

// D = 64 with one row set fits 128 VGPRs: four waves per SIMD, so two
// 8-wave workgroups share a CU (a batch of many short sequences then runs
// in one round of workgroups instead of two). Two row sets are held to 256
// registers: two waves per SIMD, one 8-wave workgroup per CU.
template <int D, int RS>
constexpr int mfma_waves_per_simd() { return D == 64 && RS == 1 ? 4 : (RS == 2 ? 2 : 1); }

template <int D, int RS, int QM, int SM, bool ROWMASK, int NW, int CH, bool PAGED>
__global__ __launch_bounds__(64 * NW) __attribute__((amdgpu_waves_per_eu(mfma_waves_per_simd<D, RS>())))
void decode_attn_mfma_kernel(const AttnArgs a) {
  constexpr bool F16 = QM == KVQ_F16;
  constexpr bool S_F16 = SM == KVQ_F16;
  constexpr int LPT = D / 32;       // 32-dim chunks (16 code bytes) per token
  constexpr int KD = D / 8;         // code dwords per token row
  constexpr int VLPT = D / 8;       // PV lanes per token row (one code dword each)
  constexpr int VTS = 64 / VLPT;    // PV token subsets
  constexpr int SUB = 4 * VTS;      // tokens per PV sub-tile
  constexpr int NSUB = 64 / SUB;    // PV sub-tiles per 64-token tile
  constexpr int ROWS = 4 * RS;
  constexpr uint32_t MAGIC = F16 ? 0x64646464u : 0x43434343u;
  constexpr uint32_t NEG_BIAS = F16 ? 0xE408E408u : 0xC308C308u;  // {-1032, -1032} / {-136, -136}
  constexpr uint32_t SEL_02 = 0x04010400u;  // {MAGIC | byte0, MAGIC | byte1}
  constexpr uint32_t SEL_46 = 0x04030402u;  // {MAGIC | byte2, MAGIC | byte3}
  // PV in fp16 for fp16 models (fp16 queries and scales). A bf16 weight
  // p * v_scale keeps 8 significant bits, below what an fp16 output holds;
  // an fp16 weight keeps 11, but p * v_scale overflows fp16 for large scales.
  // So the scales' power of two moves into the code operand instead, per
  // group of four tokens that share a matrix block (token subset ts of a
  // subtile): with E = clamp(e + 10, 11, 30), e the fp16 exponent field of
  // the group's largest |v_scale| (over its tokens and chunks), the operand
  // fp16 {E, code n} is 2^(E - 25) (1024 + n), and a weight is p * v_scale *
  // 2^(25 - E): below 2p for the largest scale (a scale under 64), at most
  // p * 2047 otherwise. The running-max slack drops to 5 (p <= 32) so that
  // this stays within fp16's 65504. Weights of much smaller scales reach
  // fp16's subnormal range only where they are negligible against the
  // group's largest. The bias term is the same product with every code at 8
  // (operand 2^(E - 25) 1032); o and the bias accumulate p * v_scale * (1024
  // + n) and p * v_scale * 1032 whatever E a group took. The group's E << 2
  // goes through LDS to the PV lanes of its subset, one byte per subtile.
  constexpr bool PV16 = F16 && S_F16;
  constexpr float LAZY = PV16 ? 5.0f : kLazyMax;
  constexpr float PV_BIAS = PV16 ? -1.0f : -136.0f;

  // Per wave: the softmax weights of the tile, [rowset][subtile] blocks of
  // 4 * LPT * VTS * 4 bf16 in which (row, chunk) pair rc = 4 * chunk + row,
  // token subset ts and position k sit at ((rc ^ subtile) * VTS + ts) * 4 + k:
  // a PV read (one subtile, every (rc, ts)) covers one contiguous block and a
  // token-lane write (one rc, every token) spreads its subtiles over distinct
  // banks. Once the sequence loop is done the same bytes hold the per-wave
  // partial outputs.
  constexpr int W_BYTES = NW * RS * 4 * LPT * NSUB * VTS * 4 * 2;
  constexpr int O_BYTES = NW * ROWS * D * 4;
  constexpr int S_BYTES = W_BYTES > O_BYTES ? W_BYTES : O_BYTES;
  // query rows padded by 16 bytes so the four rows a QK read touches sit in
  // different LDS banks
  constexpr int QROW = D / 2 + 4;
  __shared__ __attribute__((aligned(16))) uint32_t q_lds[NW][ROWS][QROW];
  __shared__ __attribute__((aligned(16))) char smem[S_BYTES];
  __shared__ __attribute__((aligned(16))) float ml_lds[NW][ROWS][2];
  __shared__ MergeLds mg;
  // With two row sets, each wave's accumulator init per (row set, chunk),
  // the same in every lane and unchanged by the tile loop, is kept in LDS
  // rather than registers, so that the kernel fits two waves per SIMD. One
  // row set has registers to spare and keeps it in registers.
  constexpr bool KEEP_IN_LDS = RS > 1;
  __shared__ __attribute__((aligned(16))) float qb_lds[KEEP_IN_LDS ? NW : 1][RS][LPT][4];
  // the decode step's new token: its score per row, then its dequantized
  // values (two elements per lane of the V wave)
  __shared__ __attribute__((aligned(16))) float nt_lds[RS * 4 + 128];
  auto w_lds = reinterpret_cast<uint16_t(*)[RS][NSUB][4 * LPT * VTS * 4]>(smem);
  static_assert(NSUB <= 4, "one exponent byte per subtile in a dword");
  __shared__ __attribute__((aligned(4))) uint8_t hb_lds[PV16 ? NW : 1][VTS][4];
  auto o_lds = reinterpret_cast<float(*)[ROWS][D]>(smem);

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  KVQ_STAMP(0);
  // The paged one-row-set kernel at D = 128 skips the early fetch: with the
  // block-table state on top, holding all those arguments made it spill 15
  // scalar registers to VGPR lanes (and reload them over 100 times); without
  // the fetch it spills 2, and the paged north star went 10.95 -> 10.64 us.
  // The other paged kernels lost without it (C5 paged 10.40 -> 10.63 us).
  if constexpr (!(PAGED && D == 128 && RS == 1)) fetch_prologue_args(a);
  // One field of each of the argument block's last two 64-byte lines in the
  // first batch as well, so that both lines are in the scalar cache before
  // anything else reads them: the block table (paged kernels) before the first
  // tile, and the workspace pointers, whose load the compiler places among
  // the query's LDS reads (a scalar load in flight turns those reads' waits
  // into waits for it too).
  asm volatile("" ::"s"(a.bt_cols), "s"(a.ws_o));
  int unit, split;
  if (!unit_and_split(a, unit, split)) return;
  // The two waves of a SIMD (w and w + 4) run the same scalar prologue, and a
  // SIMD issues one scalar instruction per turn: raising the first one's
  // priority until its first tiles' loads are issued lets it reach them in
  // about half the time instead of both arriving late together (north star
  // 9.50 -> 9.45 us, C4 62.1 -> 61.6 us; outputs bit-identical). In the
  // split that appends the new token, the one-row-set kernel at D = 128 gives
  // the priority to the two appending waves (NW - 2, NW - 1) instead of their
  // partners: their extra work (the new token's quantize, store and score)
  // sets the end of that split, which the merge waits for (north star
  // 9.33 -> 9.26 us, C2 7.27 -> 7.29 us; with four waves per SIMD, C5 lost
  // 0.28 us that way).
  {
    const bool app = D == 128 && RS == 1 && a.append && split == a.n_split - 1 && (wave % (NW / 2)) >= NW / 2 - 2;
    if ((wave < NW / 2) != app) __builtin_amdgcn_s_setprio(1);
  }
  int b, kvh, rc;
  unit_coords(a, unit, b, kvh, rc);
  // the sequence's length is read first (its latency then overlaps the query
  // loads, which do not depend on it)
  int L = a.append ? a.pos0 : a.Sk;
  if (a.seq_lens) L = load_const_i32(a.seq_lens, b);

  // ---- query rows first (wave-private copy: QT pieces of 8 elements, lane
  //      handles pieces lane, lane + 64, ...; rows past the last one read row
  //      0 and are zeroed), then the first tiles' cache rows, so the query is
  //      waited for without waiting for the cache ----
  constexpr int QT = ROWS * D / 8;
  constexpr int QPL = (QT + 63) / 64;  // query pieces per lane
  uint4 qraw[QPL];
#pragma unroll
  for (int j = 0; j < QPL; ++j) {
    const int g = lane + 64 * j;
    const int q_r = (g / (D / 8)) % ROWS, q_k = g % (D / 8);
    const int rho = rc * ROWS + q_r;
    const int rho_c = rho < a.rows_total ? rho : 0;
    const int hq = (int)fdiv((uint32_t)rho_c, a.div_sq), qi = rho_c - hq * a.Sq;
    const int head = kvh * a.ratio + hq;
    const int64_t qoff = (int64_t)b * a.qs_b + (int64_t)head * a.qs_h + (int64_t)qi * a.qs_s +
                         (int64_t)(8 * q_k) * a.qs_d;
    const uint16_t* q16 = (const uint16_t*)a.q + qoff;
    if (a.q_vec) {
      qraw[j] = *(const uint4*)q16;
    } else {
      uint32_t e[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) e[k] = q16[(int64_t)k * a.qs_d];
      qraw[j] = make_uint4(e[0] | (e[1] << 16), e[2] | (e[3] << 16), e[4] | (e[5] << 16), e[6] | (e[7] << 16));
    }
  }

  const bool len_ok = L >= 0;  // a negative length: no keys, and no row written
  L = L < 0 ? 0 : L;
  // decode step: the new token goes to row L (if it fits the cache) and is
  // attended by the unit's last split from registers
  bool has_new = a.append && len_ok && L < a.Sk && split == a.n_split - 1;
  L = L < a.Sk ? L : a.Sk;
  // The new token's rows (lane l: elements 2l, 2l+1): the K row for the
  // split's last wave, which quantizes, stores and scores it, the V row for
  // the wave before it, which quantizes and stores it and leaves its
  // dequantized values in LDS (two waves share the work that one wave of
  // the split has on top of its tile). Loaded before the cache tiles where
  // registers allow: loads complete in issue order, so loaded after them a
  // row is waited for only once the whole tile has arrived, and the
  // new-token work starts late instead of overlapping the tile's transfer.
  // The kernel that runs four waves per SIMD has no register to spare over
  // that stretch (holding the row there spills) and loads it after the
  // tile. (A paged cache may still find no block for the row; it is then
  // loaded and left unused.)
  constexpr bool EARLY_NEW = mfma_waves_per_simd<D, RS>() < 4;
  uint32_t new_x2 = 0u;
  auto load_new_row = [&]() {
    if (has_new && wave >= NW - 2 && lane < D / 2) {
      const bool is_k = wave == NW - 1;  // wave-uniform
      const uint16_t* xrow = is_k ? (const uint16_t*)a.knew + (int64_t)b * a.kns_b + (int64_t)kvh * a.kns_h
                                  : (const uint16_t*)a.vnew + (int64_t)b * a.vns_b + (int64_t)kvh * a.vns_h;
      new_x2 = *((const uint32_t*)xrow + lane);
    }
  };
  if constexpr (EARLY_NEW) load_new_row();
  int t_begin, t_end;
  if constexpr (PAGED) split_range64(a, L, split, t_begin, t_end);
  else split_range(a, L, split, t_begin, t_end);
  const int32_t* bt_b = PAGED ? a.bt + (int64_t)b * a.bt_stride : nullptr;
  // paged: the block of this wave's first tile, read here so that the table
  // read's latency overlaps the rest of the prologue (read where the tile's
  // loads need it, it was a round trip of its own right before them: north
  // star paged 11.13 -> 11.00 us, C5 paged 10.55 -> 10.35 us)
  int32_t blk_first = -1;
  if constexpr (PAGED) blk_first = table_entry(a, bt_b, ((uint32_t)t_begin + 64u * (uint32_t)wave) >> a.page_shift);
  // decode step: the cache row the new token goes to (paged: its pool row; a
  // position no block holds is neither written nor attended)
  int64_t new_row = L;
  if constexpr (PAGED) {
    if (has_new) {
      uint32_t dl;
      bool ok;
      page_delta(a, bt_b, (uint32_t)L, dl, ok);
      has_new = ok;
      new_row = (int64_t)(uint32_t)((uint32_t)L + dl);
    }
  }
  // Tiles of 64 keys, dealt to the waves round-robin. A split of whole passes
  // (NW tiles each) plus at most NW keys does not open another pass for those
  // few keys (it would cost one wave a whole tile): wave w folds tail key w
  // into its partial at the end with a short VALU dot product.
  int ntiles = t_end > t_begin ? (t_end - t_begin + 63) / 64 : 0;
  int n_tail = 0;
  {
    const int full = (t_end - t_begin) / 64, rem = (t_end - t_begin) % 64;
    if (rem > 0 && rem <= NW && full > 0 && full % NW == 0) {
      ntiles = full;
      n_tail = rem;
    }
  }

  // ---- cache slices as bounds-checked buffers (contiguous: rows >= t_end
  //      read as zero; paged: the KV head's pool, rows addressed through the
  //      block table, tokens >= t_end given an out-of-range offset) ----
  // (b, kvh) slice offsets: head strides are below 2^32 (host), so the head
  // term is one 32 x 32 -> 64-bit product; b and kvh are non-negative
  auto slice_off = [&](int64_t sb, int64_t sh) -> uint64_t {
    return (uint64_t)(uint32_t)b * (uint64_t)sb + (uint64_t)(uint32_t)kvh * (uint32_t)sh;
  };
  const uint8_t* kp_bh = a.kp + slice_off(a.kps_b, a.kps_h);
  const uint8_t* vp_bh = a.vp + slice_off(a.vps_b, a.vps_h);
  const uint16_t* ks_bh = (const uint16_t*)a.ks + slice_off(a.kss_b, a.kss_h);
  const uint16_t* vs_bh = (const uint16_t*)a.vs + slice_off(a.vss_b, a.vss_h);
  const uint32_t kps = (uint32_t)a.kps_s, vps = (uint32_t)a.vps_s;
  const uint32_t kss2 = 2u * (uint32_t)a.kss_s, vss2 = 2u * (uint32_t)a.vss_s;
  const uint32_t Le = PAGED ? a.pool_rows : (uint32_t)t_end;
  const __amdgpu_buffer_rsrc_t rk = buffer_rsrc(kp_bh, Le * kps);
  const __amdgpu_buffer_rsrc_t rks = buffer_rsrc(ks_bh, Le * kss2);
  const __amdgpu_buffer_rsrc_t rv = buffer_rsrc(vp_bh, Le * vps);
  const __amdgpu_buffer_rsrc_t rvs = buffer_rsrc(vs_bh, Le * vss2);
  // Paged tiles: a 64-key tile starting at t0 (a multiple of 64) lies in one
  // page, so its keys are pool rows rb + j for j < lim (lim = the keys it has
  // before t_end, 0 if no block holds the page). Its loads go through buffers
  // that start at row rb and hold lim rows: key j >= lim falls outside them
  // and reads zero, with no per-load offset select.
  // The block of each of this wave's tiles (tiles wave, wave + NW, ... of
  // the split; lane k holds tile k's), read from the table once here so that
  // a refill's loads wait for no table read. The first CH tiles (loaded at
  // once, before this read could return) and tiles past the 64th read the
  // table directly (the first one early, as blk_first).
  int32_t wave_blk = -1;
  if constexpr (PAGED) {
    const int tk = wave + NW * lane;
    if (tk < ntiles) {
      const uint32_t pg = ((uint32_t)t_begin + 64u * (uint32_t)tk) >> a.page_shift;
      wave_blk = pg < (uint32_t)a.bt_cols ? bt_b[pg] : -1;
    }
  }
  auto tile_rows = [&](uint32_t t0, uint32_t& rb, uint32_t& lim) {
    rb = t0;
    lim = 64;
    if constexpr (PAGED) {
      const uint32_t pg = t0 >> a.page_shift;
      const uint32_t k = (((t0 - (uint32_t)t_begin) >> 6) - (uint32_t)wave) / (uint32_t)NW;  // wave-uniform
      int32_t blk;
      if (k == 0u) blk = blk_first;  // the first tile: read early, above
      else if (k >= (uint32_t)CH && k < 64u) blk = __builtin_amdgcn_readlane(wave_blk, (int)k);
      else blk = table_entry(a, bt_b, pg);
      const bool ok = blk >= 0 && blk < a.n_blocks && t0 < (uint32_t)t_end;
      // wave-uniform; readfirstlane keeps the tile's buffers in scalar registers
      rb = __builtin_amdgcn_readfirstlane(ok ? t0 + (((uint32_t)blk - pg) << a.page_shift) : 0u);
      lim = __builtin_amdgcn_readfirstlane(ok ? min(64u, (uint32_t)t_end - t0) : 0u);
    }
  };
  const int ng = a.ng;  // scales per token row: 1, 2 or 4 (wave-uniform)
  const bool g32 = a.G == 32;
  uint32_t gsh[LPT];  // bit offset of each 32-dim chunk's scale in the loaded scale row
#pragma unroll
  for (int c = 0; c < LPT; ++c) gsh[c] = (a.gsh_pack >> (8 * c)) & 0xffu;

  // PV lane layout and the LDS slot this lane's token fills
  const int vts = lane / VLPT;
  const int vj = lane % VLPT;
  const int v_rc = vj;                      // A-operand (row, chunk) of this lane's block:
                                            // row vj & 3, chunk vj >> 2, i.e. rc = vj
  const int w_sub = lane / SUB;             // sub-tile of token `lane`
  const int w_ts = (lane % SUB) % VTS;      // its token subset
  const int w_k = (lane % SUB) / VTS;       // its position in the subset

  // Register slots for CH tiles of 64 tokens. Tile i of a chunk is computed
  // start to finish before tile i + 1, and each of its parts is refilled for
  // the next chunk as soon as it is consumed, so loads overlap the math.
  // Per tile and lane: the lane's token's K row (LPT x 16 bytes), its K and V
  // scale rows (one 2/4/8-byte load each) and, in the PV layout, code dword
  // vj of the 4 * NSUB tokens (s * SUB + VTS * k + vts) it multiplies.
  u32x4_t kc4[CH][LPT];
  uint2 skr[CH], svr[CH];
  uint32_t vq[CH][NSUB][4];
  auto load_scales = [&](__amdgpu_buffer_rsrc_t r, uint32_t off) -> uint2 {
    if (ng >= 4) return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(r, off, 0, kNt));
    if (ng == 2) return make_uint2(__builtin_amdgcn_raw_buffer_load_b32(r, off, 0, kNt), 0u);
    return make_uint2(__builtin_amdgcn_raw_buffer_load_b16(r, off, 0, kNt), 0u);
  };
  auto tile_t0 = [&](int i, int base) { return (uint32_t)(t_begin + (base + NW * i) * 64); };
  auto load_k = [&](int i, int base) {
    uint32_t rb, lim;
    tile_rows(tile_t0(i, base), rb, lim);
    __amdgpu_buffer_rsrc_t tk = rk, tks = rks;
    uint32_t r0 = rb;
    if constexpr (PAGED) {
      tk = buffer_rsrc(kp_bh + (size_t)rb * kps, lim * kps);
      tks = buffer_rsrc((const uint8_t*)ks_bh + (size_t)rb * kss2, lim * kss2);
      r0 = 0;
    }
    const uint32_t r = r0 + lane;
#pragma unroll
    for (int c = 0; c < LPT; ++c)
      kc4[i][c] = __builtin_bit_cast(u32x4_t, __builtin_amdgcn_raw_buffer_load_b128(tk, r * kps + 16u * c, 0, 0));
    skr[i] = load_scales(tks, r * kss2);
  };
  auto load_v = [&](int i, int base) {
    uint32_t rb, lim;
    tile_rows(tile_t0(i, base), rb, lim);
    __amdgpu_buffer_rsrc_t tv = rv, tvs = rvs;
    uint32_t r0 = rb;
    if constexpr (PAGED) {
      tv = buffer_rsrc(vp_bh + (size_t)rb * vps, lim * vps);
      tvs = buffer_rsrc((const uint8_t*)vs_bh + (size_t)rb * vss2, lim * vss2);
      r0 = 0;
    }
    svr[i] = load_scales(tvs, (r0 + lane) * vss2);
    // token s * SUB + VTS * k + vts, dword vj: the lane's part of the offset
    // once per tile, plus a wave-uniform row offset per load (one add each,
    // not a 32 x 32-bit multiply-add; the whole offset stays in the vector
    // operand, so the buffer's range check sees it)
    const uint32_t vbase = (r0 + (uint32_t)vts) * vps + 4u * (uint32_t)vj;
#pragma unroll
    for (int s = 0; s < NSUB; ++s)
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t du = __builtin_amdgcn_readfirstlane((uint32_t)(s * SUB + VTS * k) * vps);
        vq[i][s][k] = __builtin_amdgcn_raw_buffer_load_b32(tv, vbase + du, 0, kNt);
      }
  };

  // ---- the first tiles' cache rows. Tile 0's loads are unconditional (a
  //      wave without a tile reads past the split's end: zeros, no memory
  //      traffic). ----
  int lim[RS][4];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int rr = rc * ROWS + rs * 4 + i;
      const int qi = rr - (int)fdiv((uint32_t)rr, a.div_sq) * a.Sq;
      int lm = a.causal ? L - a.Sq + qi + 1 : L;
      lm = lm < 0 ? 0 : lm;
      lim[rs][i] = rr < a.rows_total ? lm : 0;
    }
  }
  load_k(0, wave);
  load_v(0, wave);
#pragma unroll
  for (int i = 1; i < CH; ++i) {
    if (wave + NW * i < ntiles) {
      load_k(i, wave);
      load_v(i, wave);
    }
  }
  __builtin_amdgcn_s_setprio(0);
  KVQ_STAMP(1);
  // tail key of this wave (if any): lane l holds code byte l of its K and V
  // rows (dims 2l, 2l+1) and the scales of their group
  const int tail_t = t_begin + 64 * ntiles + wave;
  uint32_t tail_kb = 0u, tail_vb = 0u, tail_ks = 0u, tail_vs = 0u;
  if (wave < n_tail) {
    uint32_t tt = (uint32_t)tail_t;
    const uint32_t col = (uint32_t)(lane % (D / 2));
    if constexpr (PAGED) {
      uint32_t dl;
      bool ok;
      page_delta(a, bt_b, tt, dl, ok);
      tt = ok ? tt + dl : Le;  // no block: the pool's end, reads zero
    }
    const uint32_t sg = 2u * fdiv(2u * (uint32_t)(lane % (D / 2)), a.div_g);
    tail_kb = __builtin_amdgcn_raw_buffer_load_b8(rk, tt * kps + col, 0, 0);
    tail_vb = __builtin_amdgcn_raw_buffer_load_b8(rv, tt * vps + col, 0, 0);
    tail_ks = __builtin_amdgcn_raw_buffer_load_b16(rks, tt * kss2 + sg, 0, 0);
    tail_vs = __builtin_amdgcn_raw_buffer_load_b16(rvs, tt * vss2 + sg, 0, 0);
  }
  if constexpr (!EARLY_NEW) load_new_row();
  // decode step: the split's last wave takes the new token's K row, the
  // wave before it the V row
  const bool new_k_here = has_new && wave == NW - 1;
  const bool new_v_here = has_new && wave == NW - 2;
  // query rows -> this wave's LDS copy, permuted to the key operand order:
  // (e0,e2) (e1,e3) (e4,e6) (e5,e7) of every 8 elements
#pragma unroll
  for (int j = 0; j < QPL; ++j) {
    const int g = lane + 64 * j;
    if (g < QT) {
      const int q_r = g / (D / 8), q_k = g % (D / 8);
      const uint32_t keep = rc * ROWS + q_r < a.rows_total ? 0xffffffffu : 0u;
      const uint4 raw = qraw[j];
      const uint32_t x = raw.x & keep, y = raw.y & keep, z = raw.z & keep, w = raw.w & keep;
      *(u32x4_t*)&q_lds[wave][q_r][4 * q_k] =
          u32x4_t{__builtin_amdgcn_perm(y, x, 0x05040100u), __builtin_amdgcn_perm(y, x, 0x07060302u),
                  __builtin_amdgcn_perm(w, z, 0x05040100u), __builtin_amdgcn_perm(w, z, 0x07060302u)};
    }
  }
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const int my_row = lane & 3;
  // The one-row-set kernel for D = 128 has registers to spare (two waves per
  // SIMD, 256 VGPRs each): it keeps this lane's query operands (its row's 16
  // dwords of 4 packed elements) in registers across the tile loop instead
  // of reading them from LDS before each matrix instruction, where the
  // compiler waits for each read alone.
  constexpr bool Q_IN_REGS = RS == 1 && D == 128;
  u32x4_t qreg[Q_IN_REGS ? 4 * LPT : 1];
  if constexpr (Q_IN_REGS) {
#pragma unroll
    for (int kd = 0; kd < 4 * LPT; ++kd) qreg[kd] = *(const u32x4_t*)&q_lds[wave][my_row][4 * kd];
  }
  auto q_operand = [&](int rs, int kd) -> u32x4_t {
    if constexpr (Q_IN_REGS) return qreg[kd];
    else return *(const u32x4_t*)&q_lds[wave][rs * 4 + my_row][4 * kd];
  };
  // accumulator init -bias * sum(q) per 32-dim chunk, on the MFMA (every
  // lane gets the same four row values; with two row sets lane 0 keeps them
  // in LDS)
  f32x4_t qinit[RS][LPT];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
    for (int c = 0; c < LPT; ++c) {
      f32x4_t acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
      for (int k4 = 0; k4 < 4; ++k4) {
        const u32x4_t q4 = q_operand(rs, 4 * c + k4);
        acc = mfma4<F16>(q4.x, q4.y, NEG_BIAS, NEG_BIAS, acc);
        acc = mfma4<F16>(q4.z, q4.w, NEG_BIAS, NEG_BIAS, acc);
      }
      if constexpr (KEEP_IN_LDS) {
        if (lane == 0) *(f32x4_t*)&qb_lds[wave][rs][c][0] = acc;
      } else {
        qinit[rs][c] = acc;
      }
    }
  }
  if constexpr (KEEP_IN_LDS) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  }

  // ---- single keys outside the tile loop (a split's tail keys, a decode
  //      step's new token): lane l owns dims 2l, 2l+1 (k0, k1, v0, v1:
  //      dequantized fp32). key_scores gives s_r = q_r . k summed over the
  //      wave (log2 units, masked rows kNeg); fold_in then makes the wave's
  //      partial in LDS absorb the key: M = max(m, s), o = o 2^(m - M) +
  //      v 2^(s - M), l = l 2^(m - M) + 2^(s - M). ----
  const int lc = lane % (D / 2);
  const bool col_ok = lane < D / 2;
  auto key_scores = [&](float k0, float k1, int key, float (&st)[RS][4]) {
    // query elements 2l, 2l+1 from the permuted copy: element pairs of each 8
    // sit as (e0,e2) (e1,e3) (e4,e6) (e5,e7)
    const int kd = lc / 4, jj = lc % 4;
    const int dwa = 4 * kd + 2 * (jj >> 1);
    const bool hi = (jj & 1) != 0;
    k0 = col_ok ? k0 : 0.0f;
    k1 = col_ok ? k1 : 0.0f;
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const uint32_t qa = q_lds[wave][rs * 4 + r][dwa], qb = q_lds[wave][rs * 4 + r][dwa + 1];
        const uint32_t ha = hi ? (qa >> 16) : (qa & 0xffffu), hb = hi ? (qb >> 16) : (qb & 0xffffu);
        const float q0 = F16 ? f16_bits_to_f32(ha) : bf16_bits_to_f32(ha);
        const float q1 = F16 ? f16_bits_to_f32(hb) : bf16_bits_to_f32(hb);
        st[rs][r] = fmaf(q0, k0, q1 * k1);
      }
      float tot[4];
      wave_reduce4<true>(st[rs], tot);
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        bool ok = true;
        if constexpr (ROWMASK) ok = key < lim[rs][r];
        st[rs][r] = ok ? tot[r] * a.scale_log2 : kNeg;
      }
    }
  };
  auto fold_in = [&](const float (&st)[RS][4], float v0, float v1) {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int row = rs * 4 + r;
        const float m_old = ml_lds[wave][row][0], l_old = ml_lds[wave][row][1];
        const float sv = st[rs][r];
        const float M = fmax_nc(m_old, sv);
        const float fa = __builtin_amdgcn_exp2f(m_old - M);
        const float fb = sv > kNeg ? __builtin_amdgcn_exp2f(sv - M) : 0.0f;
        if (col_ok) {
          const float2 o2 = *(const float2*)&o_lds[wave][row][2 * lc];
          *(float2*)&o_lds[wave][row][2 * lc] = make_float2(fmaf(o2.x, fa, v0 * fb), fmaf(o2.y, fa, v1 * fb));
        }
        if (lane == 0) {
          ml_lds[wave][row][0] = M;
          ml_lds[wave][row][1] = fmaf(l_old, fa, fb);
        }
      }
    }
  };
  // decode step: quantize the new K or V row exactly as the quantize kernel
  // does (group absmax / 7 in fp32, IEEE division, round half to even, clamp,
  // +8; scale narrowed once for storage) and store it at row L, while the
  // tiles are in flight. The K wave scores the dequantized key (stored
  // scale) now and leaves the scores in LDS, the V wave the dequantized
  // values; the workgroup fold takes them in as one more partial. Lane l
  // owns code byte l of the packed row (packed width = groups x G/2 bytes
  // <= 64).
  if (new_k_here || new_v_here) {  // wave-uniform
    const bool is_k = new_k_here;
    const int G = a.G;
    const int W = ((D + G - 1) / G) * (G / 2);
    const bool byte_ok = lane < W;
    const float x0 = col_ok ? (F16 ? f16_bits_to_f32(new_x2 & 0xffffu) : bf16_bits_to_f32(new_x2 & 0xffffu)) : 0.0f;
    const float x1 = col_ok ? (F16 ? f16_bits_to_f32(new_x2 >> 16) : bf16_bits_to_f32(new_x2 >> 16)) : 0.0f;
    // group absmax: G / 2 consecutive lanes (16, 32 or 64)
    float am = row16_max(fmax_nc(fabsf(x0), fabsf(x1)));
    if (G >= 64) {  // rows of 16 lanes pairwise: (0, 1), (2, 3)
      float u = am, v = am;
      permlane16_swap(u, v);
      am = fmax_nc(u, v);
    }
    if (G >= 128) {  // halves of 32 lanes
      float u = am, v = am;
      permlane32_swap(u, v);
      am = fmax_nc(u, v);
    }
    const float scale = group_scale(am);  // am / 7, correctly rounded
    const float inv = group_inverse(scale);
    const bool fast = scale >= 0x1p-100f && scale <= 0x1p100f;
    float c0 = rint_quotient(x0, scale, inv, fast), c1 = rint_quotient(x1, scale, inv, fast);
    c0 = fminf(fmaxf(c0, -8.0f), 7.0f);
    c1 = fminf(fmaxf(c1, -8.0f), 7.0f);
    const uint32_t byte = (uint32_t)((int)c0 + 8) | ((uint32_t)((int)c1 + 8) << 4);
    const uint32_t sbits = S_F16 ? f32_to_f16_bits(scale) : f32_to_bf16_bits(scale);
    uint8_t* prow = const_cast<uint8_t*>(is_k ? kp_bh : vp_bh) + new_row * (is_k ? kps : vps);
    uint16_t* srow = const_cast<uint16_t*>(is_k ? ks_bh : vs_bh) + new_row * (is_k ? a.kss_s : a.vss_s);
    if (byte_ok) prow[lane] = (uint8_t)byte;
    if (byte_ok && ((2 * lane) & (G - 1)) == 0) srow[(2 * lane) / G] = (uint16_t)sbits;  // G: 32, 64 or 128
    const float sq = scale16_to_f32(sbits, S_F16);
    const float d0 = c0 * sq, d1 = c1 * sq;
    if (is_k) {
      float new_st[RS][4];
      key_scores(d0, d1, L, new_st);
      if (lane == 0) {
#pragma unroll
        for (int rs = 0; rs < RS; ++rs)
#pragma unroll
          for (int r = 0; r < 4; ++r) nt_lds[rs * 4 + r] = new_st[rs][r];
      }
    } else {
      *(float2*)&nt_lds[RS * 4 + 2 * lane] = make_float2(d0, d1);
    }
  }

  // ---- running softmax state (base 2; scores carry sm_scale * log2 e) ----
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

  bool fresh = true;  // no tile folded into the running state yet (wave-uniform)
  for (int base = wave; base < ntiles; base += NW * CH) {
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if (base + NW * i >= ntiles) break;  // wave-uniform: this wave has no tile i
      const bool refill = base + NW * (CH + i) < ntiles;
      const int t0 = t_begin + (base + NW * i) * 64;
      const bool masked = ROWMASK || t0 + 64 > t_end;  // wave-uniform
      // ---- QK on the matrix cores: scores of token `lane` for every row ----
      float sc[RS][4];
      if (i == 0 && base == wave) KVQ_STAMP_AFTER(2, kc4[i][LPT - 1][3]);
      {
        f32x4_t acc[RS][LPT];
#pragma unroll
        for (int rs = 0; rs < RS; ++rs)
#pragma unroll
          for (int c = 0; c < LPT; ++c) {
            if constexpr (KEEP_IN_LDS) acc[rs][c] = *(const f32x4_t*)&qb_lds[wave][rs][c][0];
            else acc[rs][c] = qinit[rs][c];
          }
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
              const u32x4_t q4 = q_operand(rs, kd);
              acc[rs][c] = mfma4<F16>(q4.x, q4.y, b02, b13, acc[rs][c]);
              acc[rs][c] = mfma4<F16>(q4.z, q4.w, b46, b57, acc[rs][c]);
            }
          }
        }
        float skl[LPT];
        chunk_scales<LPT, S_F16>(skr[i], g32, gsh, a.scale_log2, skl);
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            float s = acc[rs][0][r] * skl[0];
#pragma unroll
            for (int c = 1; c < LPT; ++c) s = fmaf(acc[rs][c][r], skl[c], s);
            sc[rs][r] = s;
          }
        }
        if (masked) {
          const int t = t0 + lane;
#pragma unroll
          for (int rs = 0; rs < RS; ++rs)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              bool ok = t < t_end;
              if constexpr (ROWMASK) ok = ok && (t < lim[rs][r]);
              sc[rs][r] = ok ? sc[rs][r] : (ROWMASK ? kNeg : -__builtin_inff());
            }
        }
      }
      if (refill) load_k(i, base + NW * CH);

      // PV16: the tile's V scales per chunk of this lane's token and its
      // group's exponent (the scale rows arrive right after the keys)
      float svl[LPT];
      if constexpr (PV16) {
        chunk_scales<LPT, S_F16>(svr[i], g32, gsh, 1.0f, svl);
        float smax = fabsf(svl[0]);
#pragma unroll
        for (int c = 1; c < LPT; ++c) smax = fmaxf(smax, fabsf(svl[c]));
        // over the group: the lanes VTS apart in the token's SUB-lane subtile
        if constexpr (VTS == 4) {  // D = 128: lanes ts + 4k of a 16-lane row
          smax = fmaxf(smax, dpp<0x124>(smax, 0.0f));  // row_ror:4
          smax = fmaxf(smax, dpp<0x128>(smax, 0.0f));  // row_ror:8
        } else {  // D = 64: lanes ts + 8k of two 16-lane rows
          smax = fmaxf(smax, dpp<0x128>(smax, 0.0f));  // row_ror:8
          float other = smax;
          permlane16_swap(smax, other);
          smax = fmaxf(smax, other);
        }
        // fp32 exponent field e32 = e + 112 for a normal fp16 scale
        const int e32 = (int)((__builtin_bit_cast(uint32_t, smax) >> 23) & 0xffu);
        const int E = min(max(e32 - 102, 11), 30);
#pragma unroll
        for (int c = 0; c < LPT; ++c) svl[c] = __builtin_amdgcn_ldexpf(svl[c], 25 - E);
        hb_lds[wave][w_ts][w_sub] = (uint8_t)(E << 2);
      }

      // ---- tile max, rescale of the running state (not for a wave's
      //      first tile: its accumulators are still zero). The running max
      //      is a reference, not the exact maximum: it moves (and the state
      //      is rescaled) only when a row's tile max exceeds it by more than
      //      kLazyMax, so after the first tiles almost no tile pays for the
      //      rescale; p = 2^(s - m) then stays below 2^kLazyMax, which fp32
      //      sums and the bf16 weights hold with their full precision. ----
      {
        float mt[RS][4];
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) wave_reduce4<false>(sc[rs], mt[rs]);
        if (fresh) {
#pragma unroll
          for (int rs = 0; rs < RS; ++rs)
#pragma unroll
            for (int r = 0; r < 4; ++r) m_run[rs][r] = mt[rs][r];
        } else {
          bool grow = false;
#pragma unroll
          for (int rs = 0; rs < RS; ++rs)
#pragma unroll
            for (int r = 0; r < 4; ++r) grow = grow || (mt[rs][r] > m_run[rs][r] + LAZY);
          if (grow) {
#pragma unroll
            for (int rs = 0; rs < RS; ++rs) {
              f32x4_t al;
#pragma unroll
              for (int r = 0; r < 4; ++r) {
                const float mn = fmax_nc(m_run[rs][r], mt[rs][r]);
                al[r] = __builtin_amdgcn_exp2f(m_run[rs][r] - mn);
                l_acc[rs][r] *= al[r];
                m_run[rs][r] = mn;
              }
#pragma unroll
              for (int m = 0; m < 8; ++m) o_acc[rs][m] *= al;
              w_acc[rs] *= al;
            }
          }
        }
        fresh = false;
      }

      // ---- p and w = p * v_scale (bf16; PV16: fp16, the tile's largest
      //      scale's power of two moved into the code operand) -> LDS ----
      {
        if constexpr (!PV16) chunk_scales<LPT, S_F16>(svr[i], g32, gsh, 1.0f, svl);
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const float s = sc[rs][r];
            // Masked keys: without row masks they score -inf, and a wave's
            // first tile holds a key of the split, so every row's running max
            // is finite and the weight 2^(-inf - m) is 0 with no select. With
            // row masks a row may have no key yet (max kNeg): they score kNeg
            // and their weight is set to 0.
            float p = __builtin_amdgcn_exp2f(s - m_run[rs][r]);
            if constexpr (ROWMASK) p = s > kNeg ? p : 0.0f;
            l_acc[rs][r] += p;
#pragma unroll
            for (int c = 0; c < LPT; c += 2) {
              uint32_t pk;
              if constexpr (PV16) {
                const f16x2_t pk2 = {(_Float16)(p * svl[c]), (_Float16)(p * svl[c + 1])};
                pk = __builtin_bit_cast(uint32_t, pk2);
              } else {
                const bf16x2_t pk2 = {(__bf16)(p * svl[c]), (__bf16)(p * svl[c + 1])};
                pk = __builtin_bit_cast(uint32_t, pk2);
              }
              w_lds[wave][rs][w_sub][(((4 * c + r) ^ w_sub) * VTS + w_ts) * 4 + w_k] = (uint16_t)pk;
              w_lds[wave][rs][w_sub][(((4 * c + 4 + r) ^ w_sub) * VTS + w_ts) * 4 + w_k] = (uint16_t)(pk >> 16);
            }
          }
        }
      }
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");

      // ---- PV on the matrix cores ----
      if (i == 0 && base == wave) KVQ_STAMP_AFTER(3, vq[i][NSUB - 1][3]);
      // u = bytes {t0.b, t1.b, t0.b', t1.b'} of two tokens' code dwords; its low
      // and high nibbles then give (token0, token1) pairs of one dim per perm.
      // PV16: the exponent bytes of this lane's subset, one per subtile
      const uint32_t hbd = PV16 ? *(const uint32_t*)&hb_lds[wave][vts][0] : 0u;
#pragma unroll
      for (int s = 0; s < NSUB; ++s) {
        // the operands' high bytes: bf16 128 + n, or (PV16) {E | n} with
        // byte s of hbd
        const uint32_t hb = PV16 ? hbd : 0x43434343u;
        const uint32_t s02 = PV16 ? ((0x04u + s) << 24) | (0x01u << 16) | ((0x04u + s) << 8) : SEL_02;
        const uint32_t s46 = PV16 ? ((0x04u + s) << 24) | (0x03u << 16) | ((0x04u + s) << 8) | 0x02u : SEL_46;
        uint32_t bp[2][8];  // [token pair][dim within the lane's 8]
#pragma unroll
        for (int tp = 0; tp < 2; ++tp) {
          const uint32_t v0 = vq[i][s][2 * tp], v1 = vq[i][s][2 * tp + 1];
#pragma unroll
          for (int hh = 0; hh < 2; ++hh) {  // dims 0-3, dims 4-7
            const uint32_t u = __builtin_amdgcn_perm(v1, v0, hh ? 0x07030602u : 0x05010400u);
            const uint32_t lo = u & 0x0F0F0F0Fu, hi = (u >> 4) & 0x0F0F0F0Fu;
            bp[tp][4 * hh + 0] = __builtin_amdgcn_perm(hb, lo, s02);
            bp[tp][4 * hh + 1] = __builtin_amdgcn_perm(hb, hi, s02);
            bp[tp][4 * hh + 2] = __builtin_amdgcn_perm(hb, lo, s46);
            bp[tp][4 * hh + 3] = __builtin_amdgcn_perm(hb, hi, s46);
          }
        }
#pragma unroll
        for (int rs = 0; rs < RS; ++rs) {
          const uint2 wa = *(const uint2*)&w_lds[wave][rs][s][((v_rc ^ s) * VTS + vts) * 4];
#pragma unroll
          for (int m = 0; m < 8; ++m)
            o_acc[rs][m] = mfma4<PV16>(wa.x, wa.y, bp[0][m], bp[1][m], o_acc[rs][m]);
          // the bias sum: weights times 1 (bf16, taken 136 times later), or
          // (PV16) times the code operand of n = 8
          const uint32_t bias_pair = PV16 ? __builtin_amdgcn_perm(hb, 0x08080808u, s02) : kBf16OnePair;
          w_acc[rs] = mfma4<PV16>(wa.x, wa.y, bias_pair, bias_pair, w_acc[rs]);
        }
      }
      if (refill) load_v(i, base + NW * CH);
      __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
      __builtin_amdgcn_wave_barrier();
      __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
    }
  }

  // ---- wave partial: the N = 32 * RS values of a lane (row rho = idx / 8,
  //      dim 8 vj + idx % 8, idx = 8 * rho + m) summed over the VTS token
  //      subsets (lanes VLPT apart) by swap-and-halve steps: each step pairs
  //      value i with value i + n/2 across lanes 32 (permlane32 swap), 16
  //      (permlane16 swap) or 8 (row rotate, D = 64) apart, and each lane keeps
  //      the half its side of the pair owns. Afterwards the lane of subset g
  //      holds values [g * N / VTS, (g + 1) * N / VTS). Then -> LDS (over the
  //      weight bytes, so every wave must be done with those). ----
  KVQ_STAMP(4);
  constexpr int NV = 32 * RS;
  float val[NV];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs)
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int m = 0; m < 8; ++m)
        val[(rs * 4 + r) * 8 + m] = fmaf(PV_BIAS, w_acc[rs][r], o_acc[rs][m][r]);
#pragma unroll
  for (int i = 0; i < NV / 2; ++i) {
    float x = val[i], y = val[i + NV / 2];
    permlane32_swap(x, y);
    val[i] = x + y;
  }
#pragma unroll
  for (int i = 0; i < NV / 4; ++i) {
    float x = val[i], y = val[i + NV / 4];
    permlane16_swap(x, y);
    val[i] = x + y;
  }
  if constexpr (VTS == 8) {
    const bool hi8 = (lane & 8) != 0;
#pragma unroll
    for (int i = 0; i < NV / 8; ++i) {
      const float send = hi8 ? val[i] : val[i + NV / 8];
      const float keep = hi8 ? val[i + NV / 8] : val[i];
      val[i] = keep + dpp<0x128>(send, 0.0f);  // row_ror:8 = the lane 8 apart
    }
  }
  constexpr int NK = NV / VTS;  // values a lane keeps
  float lsum[RS][4];
#pragma unroll
  for (int rs = 0; rs < RS; ++rs) wave_reduce4<true>(l_acc[rs], lsum[rs]);
  // o_lds[wave] occupies exactly the bytes of w_lds[wave] (RS * 16 * D of
  // them in both layouts), so only this wave's own weight reads must be done
  // before they are overwritten: a wave-level ordering point, no workgroup
  // barrier.
  static_assert(sizeof(float) * ROWS * D == 2 * RS * 4 * LPT * NSUB * VTS * 4, "o_lds[w] aliases w_lds[w] exactly");
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
#pragma unroll
  for (int i = 0; i < NK; i += 4) {
    const int idx = NK * vts + i;  // first of 4 consecutive values (same row)
    *(float4*)&o_lds[wave][idx / 8][8 * vj + idx % 8] = make_float4(val[i], val[i + 1], val[i + 2], val[i + 3]);
  }
  if (lane == 0) {
#pragma unroll
    for (int rs = 0; rs < RS; ++rs) {
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        ml_lds[wave][rs * 4 + r][0] = m_run[rs][r];
        ml_lds[wave][rs * 4 + r][1] = lsum[rs][r];
      }
    }
  }
  // ---- extra keys folded into this wave's partial (already in LDS): the
  //      split's tail key of this wave and, in a decode step, the new token
  //      (scored before the tile loop). ----
  // The tail key's raw loads are touched only here: an empty asm that
  // redefines them keeps the compiler from converting them right after the
  // loads, which (loads completing in issue order) would wait for the whole
  // tile before the loop.
  asm volatile("" : "+v"(tail_kb), "+v"(tail_vb), "+v"(tail_ks), "+v"(tail_vs)::"memory");
  if (wave < n_tail) {
    const float ksf = scale16_to_f32(tail_ks, S_F16), vsf = scale16_to_f32(tail_vs, S_F16);
    float st[RS][4];
    key_scores(((float)(int)(tail_kb & 15u) - 8.0f) * ksf, ((float)(int)((tail_kb >> 4) & 15u) - 8.0f) * ksf,
               tail_t, st);
    fold_in(st, ((float)(int)(tail_vb & 15u) - 8.0f) * vsf, ((float)(int)((tail_vb >> 4) & 15u) - 8.0f) * vsf);
  }
  __syncthreads();
  // the new token (scores and values in LDS, written by the K and V waves
  // before their tile loops) joins the waves' partials in the workgroup fold
  finish_block<ROWS, D, QM, NW>(a, unit, split, rc, kvh, b, o_lds, ml_lds, mg, has_new ? nt_lds : nullptr);
  KVQ_STAMP(11);
}

// ===========================================================================
// VALU kernel: fp32 queries (exact fp32 arithmetic) or fp32 scales.
// Lane = token * (D/32) + chunk for QK (quad-reduced with DPP); V lanes own 8
// output dims and four tokens per tile.

template <int D, int ROWS, int QM, bool ROWMASK, bool PAGED>
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
  __shared__ __attribute__((aligned(16))) float ml_lds[4][ROWS][2];
  __shared__ MergeLds mg;
  // the decode step's new token: its score per row, then its dequantized
  // values (two elements per lane of the V wave)
  __shared__ __attribute__((aligned(16))) float nt_lds[ROWS + 128];

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform (scalar)
  int unit, split;
  if (!unit_and_split(a, unit, split)) return;
  int b, kvh, rc;
  unit_coords(a, unit, b, kvh, rc);

  int L = !ROWMASK && a.append ? a.pos0 : a.Sk;
  if (a.seq_lens) L = a.seq_lens[b];
  const bool len_ok = L >= 0;  // a negative length: no keys, and no row written
  L = L < 0 ? 0 : L;
  // decode step: the new token goes to row L (if it fits the cache) and is
  // attended by the unit's last split: wave 3 quantizes, stores and scores
  // its K row, wave 2 quantizes and stores its V row (lane l: elements 2l,
  // 2l+1, loaded here, ahead of the tiles). A decode step has one query
  // position, so it never takes the row-masked instances.
  bool has_new = !ROWMASK && a.append && len_ok && L < a.Sk && split == a.n_split - 1;
  L = L < a.Sk ? L : a.Sk;
  float nx0 = 0.0f, nx1 = 0.0f;
  if (has_new && wave >= 2 && lane < D / 2) {
    const bool is_k = wave == 3;  // wave-uniform
    const int64_t off = (int64_t)b * (is_k ? a.kns_b : a.vns_b) + (int64_t)kvh * (is_k ? a.kns_h : a.vns_h) +
                        2 * lane;
    if constexpr (QM == KVQ_F32) {
      const float2 x = *(const float2*)((const float*)(is_k ? a.knew : a.vnew) + off);
      nx0 = x.x;
      nx1 = x.y;
    } else {
      const uint32_t x = *(const uint32_t*)((const uint16_t*)(is_k ? a.knew : a.vnew) + off);
      nx0 = QM == KVQ_F16 ? f16_bits_to_f32(x & 0xffffu) : bf16_bits_to_f32(x & 0xffffu);
      nx1 = QM == KVQ_F16 ? f16_bits_to_f32(x >> 16) : bf16_bits_to_f32(x >> 16);
    }
  }
  // Paged caches: split boundaries at multiples of 64 keys, so that a tile
  // of TPT (<= 64, dividing 64) keys lies inside one page and one table
  // entry gives its pool rows; a pool with no block has nothing to read.
  int t_begin, t_end;
  if constexpr (PAGED) split_range64(a, L, split, t_begin, t_end);
  else split_range(a, L, split, t_begin, t_end);
  int ntiles = t_end > t_begin ? (t_end - t_begin + TPT - 1) / TPT : 0;
  const int32_t* bt_b = PAGED ? a.bt + (int64_t)b * a.bt_stride : nullptr;
  int64_t new_row = L;  // the new token's cache row (paged: its pool row)
  if constexpr (PAGED) {
    if (a.n_blocks == 0) ntiles = 0;
    if (has_new) {
      uint32_t dl;
      bool ok;
      page_delta(a, bt_b, (uint32_t)L, dl, ok);
      has_new = ok;
      new_row = (int64_t)(uint32_t)((uint32_t)L + dl);
    }
  }

  const int kt = lane / LPT;
  const int kc = lane % LPT;
  const int vts = lane / VLPT;
  const int vj = lane % VLPT;
  const int vc = vj >> 2;
  const uint32_t gK = fdiv((uint32_t)(kc * 32), a.div_g);

  int lim[ROWS];
  uint32_t qp[DOT2 ? ROWS : 1][16];
  float qf[DOT2 ? 1 : ROWS][32];
  float qinit[ROWS];
#pragma unroll
  for (int r = 0; r < ROWS; ++r) {
    const int rho = rc * ROWS + r;
    const bool row_ok = rho < a.rows_total;
    const int rho_c = row_ok ? rho : 0;
    const int hq = (int)fdiv((uint32_t)rho_c, a.div_sq);
    const int head = kvh * a.ratio + hq;
    const int qi = rho_c - hq * a.Sq;
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

  // decode step: quantize the new K or V row exactly as the quantize kernel
  // does (group absmax / 7 in fp32, round half to even, clamp, +8; the scale
  // stored in the cache's scale dtype) and store it at row L. The K wave then
  // scores the key dequantized with the stored scale against the query rows
  // (exact fp32), the V wave leaves the dequantized values in LDS; the
  // workgroup fold takes them in as one more partial.
  if (has_new && wave >= 2) {  // wave-uniform
    const bool is_k = wave == 3;
    const int G = a.G;
    const int W = ((D + G - 1) / G) * (G / 2);
    const bool col_ok = lane < D / 2;
    const bool byte_ok = lane < W;
    const float x0 = col_ok ? nx0 : 0.0f, x1 = col_ok ? nx1 : 0.0f;
    float am = row16_max(fmax_nc(fabsf(x0), fabsf(x1)));  // group absmax: G / 2 lanes
    if (G >= 64) {
      float u = am, v = am;
      permlane16_swap(u, v);
      am = fmax_nc(u, v);
    }
    if (G >= 128) {
      float u = am, v = am;
      permlane32_swap(u, v);
      am = fmax_nc(u, v);
    }
    const float scale = group_scale(am);  // am / 7, correctly rounded
    const float inv = group_inverse(scale);
    const bool fast = scale >= 0x1p-100f && scale <= 0x1p100f;
    float c0 = rint_quotient(x0, scale, inv, fast), c1 = rint_quotient(x1, scale, inv, fast);
    c0 = fminf(fmaxf(c0, -8.0f), 7.0f);
    c1 = fminf(fmaxf(c1, -8.0f), 7.0f);
    const uint32_t byte = (uint32_t)((int)c0 + 8) | ((uint32_t)((int)c1 + 8) << 4);
    uint8_t* prow = const_cast<uint8_t*>(is_k ? kp_bh : vp_bh) + new_row * (is_k ? kps : vps);
    char* srow = const_cast<char*>(is_k ? ks_bh : vs_bh) + new_row * (is_k ? kss : vss) * s_esize;
    if (byte_ok) prow[lane] = (uint8_t)byte;
    float sq = scale;
    const bool scale_lane = byte_ok && (2 * lane) % G == 0;
    if (a.scale_dtype == KVQ_F32) {
      if (scale_lane) ((float*)srow)[(2 * lane) / G] = scale;
    } else {
      const bool h = a.scale_dtype == KVQ_F16;
      const uint32_t sbits = h ? f32_to_f16_bits(scale) : f32_to_bf16_bits(scale);
      if (scale_lane) ((uint16_t*)srow)[(2 * lane) / G] = (uint16_t)sbits;
      sq = scale16_to_f32(sbits, h);
    }
    const float d0 = c0 * sq, d1 = c1 * sq;
    if (is_k) {
#pragma unroll
      for (int r = 0; r < ROWS; ++r) {
        const int rho = rc * ROWS + r;
        const bool row_ok = rho < a.rows_total;
        const int rho_c = row_ok ? rho : 0;
        const int hq = (int)fdiv((uint32_t)rho_c, a.div_sq);
        const int head = kvh * a.ratio + hq;
        const int qi = rho_c - hq * a.Sq;
        const int64_t qbase = (int64_t)b * a.qs_b + (int64_t)head * a.qs_h + (int64_t)qi * a.qs_s;
        float part = 0.0f;
        if (col_ok) {
          const float q0 = load_as_f32(a.q, qbase + (int64_t)(2 * lane) * a.qs_d, QM);
          const float q1 = load_as_f32(a.q, qbase + (int64_t)(2 * lane + 1) * a.qs_d, QM);
          part = fmaf(q0, d0, q1 * d1);
        }
        const float sc = wave_sum(part) * a.scale_log2;
        if (lane == 0) nt_lds[r] = row_ok ? sc : kNeg;
      }
    } else {
      *(float2*)&nt_lds[ROWS + 2 * lane] = make_float2(d0, d1);
    }
  }

  for (int base = wave; base < ntiles; base += 4 * CH) {
    // tiles of this chunk the wave has (wave-uniform): a split's last chunk
    // may hold fewer than CH, and the rest are neither loaded nor computed
    const int nv = min(CH, (ntiles - base + 3) / 4);
    uint4 kcode[CH];
    uint32_t vcode[CH][4];
    float sk[CH], sv[CH];
    bool blk_ok[CH];  // paged: a block holds the tile's page (else its rows read pool row 0, masked)
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if (i >= nv) break;
      const int t0 = t_begin + (base + 4 * i) * TPT;
      // token -> cache row: the token itself, or (paged) its pool row; the
      // clamp to the last token stays inside the tile, hence inside its page
      uint32_t dl = 0u;
      blk_ok[i] = true;
      if constexpr (PAGED) page_delta(a, bt_b, (uint32_t)t0, dl, blk_ok[i]);
      auto row = [&](int t) -> uint32_t {
        const uint32_t tc = (uint32_t)min(t, last_tok);
        return blk_ok[i] ? tc + dl : 0u;
      };
      const uint32_t tk = row(t0 + kt);
      kcode[i] = *(const uint4*)(kp_bh + (tk * kps + 16u * kc));
      sk[i] = load_scale(ks_bh, tk * kss + gK, a.scale_dtype);
      sv[i] = load_scale(vs_bh, tk * vss + gK, a.scale_dtype);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const uint32_t tv = row(t0 + vts + VTS * k);
        vcode[i][k] = *(const uint32_t*)(vp_bh + (tv * vps + 4u * vj));
      }
    }

    float s[CH][ROWS];
#pragma unroll
    for (int i = 0; i < CH; ++i) {
      if (i >= nv) {
#pragma unroll
        for (int r = 0; r < ROWS; ++r) s[i][r] = kNeg;
        continue;
      }
      const int t = t_begin + (base + 4 * i) * TPT + kt;
      const bool tv_ok = (base + 4 * i < ntiles) && (t < t_end) && blk_ok[i];
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
      if (i >= nv) break;
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
      if (i >= nv) break;
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
  // the new token (scores and values in LDS, written by waves 3 and 2 before
  // their tile loops) joins the waves' partials in the workgroup fold
  finish_block<ROWS, D, QM, 4>(a, unit, split, rc, kvh, b, o_lds, ml_lds, mg, has_new ? nt_lds : nullptr);
}

// ---------------------------------------------------------------------------
// Host side: planning and dispatch.

struct Plan {
  bool mfma;
  int rows, row_chunks, n_units, n_split;
};

// The MFMA kernel serves bf16/fp16 queries with 16-bit scales; everything else
// (fp32 queries, fp32 scales) runs on the VALU kernel.
static bool use_mfma(int q_dtype, int scale_dtype) {
  return q_dtype != KVQ_F32 && scale_dtype != KVQ_F32;
}

// Fewest keys a split is given (when the sequence is long enough to split):
// the shortest split worth its share of the cross-split merge (measured):
// two 64-token tiles for the matrix-core kernel; the same 128 keys for the
// exact-fp32 VALU kernel (GPT-2-small shape, 1K keys, 12 heads: one split
// per head 11.8 us, 2 splits 10.6, 4 splits 9.1, 8 splits 8.3, 16 splits 8.4).
static int64_t min_split_tokens(bool mfma, int64_t D) {
  (void)mfma;
  (void)D;
  return 128;
}

// Split-K plan: enough splits that B * Hkv * row_chunks * n_split workgroups
// cover the CUs once (one resident workgroup per CU), no split shorter than
// min_split_tokens of the longest sequence, at most kMaxSplit.
static int make_plan(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D, int64_t s_max,
                     int q_dtype, int scale_dtype, int64_t n_split_req, int64_t num_cus, Plan* p) {
  if (B < 1 || Hq < 1 || Hkv < 1 || Sq < 1 || s_max < 0 || Hq % Hkv != 0) return KVQ_EINVAL;
  if (!(D == 64 || D == 128)) return KVQ_EUNSUP;
  const int64_t rows_total = (Hq / Hkv) * Sq;
  p->mfma = use_mfma(q_dtype, scale_dtype);
  if (p->mfma) {
    p->rows = rows_total <= 4 ? 4 : 8;
  } else {
    const int cap = q_dtype == KVQ_F32 ? 2 : 8;
    int r = 1;
    while (r < rows_total && r < cap) r *= 2;
    p->rows = r;
  }
  p->row_chunks = (int)((rows_total + p->rows - 1) / p->rows);
  const int64_t units = B * Hkv * p->row_chunks;
  if (units > (1ll << 30)) return KVQ_EUNSUP;
  p->n_units = (int)units;
  const int64_t mst = min_split_tokens(p->mfma, D);
  const int64_t max_split = std::max<int64_t>(1, s_max / mst);
  int64_t ns = n_split_req;
  if (ns <= 0) {
    const int64_t cus = std::max<int64_t>(1, num_cus);
    ns = (cus + units - 1) / units;
  }
  ns = std::max<int64_t>(1, std::min<int64_t>(std::min<int64_t>(ns, max_split), kMaxSplit));
  if (units * ns > 0x7fffffffll || units * p->rows * D / 128 >= 0x7fffffffll) return KVQ_EUNSUP;
  if (ns > 1 && units > 1024) return KVQ_EUNSUP;  // split plans keep their counters in a fixed block
  p->n_split = (int)ns;
  return KVQ_OK;
}

// Workspace: a fixed block of per-unit arrival counters (64 bytes apart; the
// same bytes for every plan, so a workspace reused by calls with different
// plans never reads another plan's partials as counters), per (unit, split,
// row) the partial (max, sum) pair (padded to 256 bytes), then the partial
// output rows.
constexpr int64_t kCntUnits = 1024;  // units a split plan may have
static int64_t ws_cnt_bytes(const Plan&) { return kCntUnits * kCntStride * 4; }
static int64_t ws_ml_bytes(const Plan& p) {
  const int64_t slots = (int64_t)p.n_units * p.n_split * p.rows;
  return (slots * 2 * 4 + 255) / 256 * 256;
}

static int64_t workspace_bytes_for(const Plan& p, int64_t D) {
  if (p.n_split <= 1) return 0;
  return ws_cnt_bytes(p) + ws_ml_bytes(p) + (int64_t)p.n_units * p.n_split * p.rows * D * 4;
}

// Waves per workgroup of the MFMA kernel: 8 (two per SIMD hide each other's
// latency), with one tile's loads in flight per wave (the SIMD partner covers
// the latency; a second slot measured 5-12 % slower from 4K to 128K keys with
// one row set). Two row sets fit two waves per SIMD too (212-223 VGPRs, no
// AGPRs) once the MFMA accumulators stay in VGPRs and the loop-invariant
// values live in LDS; before that they ran 4 waves with two tiles in flight.
template <int RS>
constexpr int mfma_waves() { return 8; }
template <int RS>
constexpr int mfma_tiles_in_flight() { return 1; }

template <int D, int RS, int QM, int SM, bool PAGED>
static void launch_mfma_rs(const AttnArgs& a, bool rowmask, dim3 grid, hipStream_t st) {
  constexpr int NW = mfma_waves<RS>();
  constexpr int CH = mfma_tiles_in_flight<RS>();
  if (rowmask) hipLaunchKernelGGL((decode_attn_mfma_kernel<D, RS, QM, SM, true, NW, CH, PAGED>), grid, dim3(64 * NW), 0, st, a);
  else hipLaunchKernelGGL((decode_attn_mfma_kernel<D, RS, QM, SM, false, NW, CH, PAGED>), grid, dim3(64 * NW), 0, st, a);
}

template <int D, int QM, bool PAGED>
static void launch_mfma_pg(const AttnArgs& a, int rows, bool rowmask, dim3 grid, hipStream_t st) {
  if (a.scale_dtype == KVQ_F16) {
    if (rows <= 4) launch_mfma_rs<D, 1, QM, KVQ_F16, PAGED>(a, rowmask, grid, st);
    else launch_mfma_rs<D, 2, QM, KVQ_F16, PAGED>(a, rowmask, grid, st);
  } else {
    if (rows <= 4) launch_mfma_rs<D, 1, QM, KVQ_BF16, PAGED>(a, rowmask, grid, st);
    else launch_mfma_rs<D, 2, QM, KVQ_BF16, PAGED>(a, rowmask, grid, st);
  }
}

template <int D, int QM>
static void launch_mfma(const AttnArgs& a, int rows, bool rowmask, dim3 grid, hipStream_t st) {
  if (a.bt) launch_mfma_pg<D, QM, true>(a, rows, rowmask, grid, st);
  else launch_mfma_pg<D, QM, false>(a, rows, rowmask, grid, st);
}

template <int D, int ROWS, int QM>
static void launch_valu_rows(const AttnArgs& a, bool rowmask, dim3 grid, hipStream_t st) {
  if (a.bt) {
    if (rowmask) hipLaunchKernelGGL((decode_attn_valu_kernel<D, ROWS, QM, true, true>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((decode_attn_valu_kernel<D, ROWS, QM, false, true>), grid, dim3(256), 0, st, a);
  } else {
    if (rowmask) hipLaunchKernelGGL((decode_attn_valu_kernel<D, ROWS, QM, true, false>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((decode_attn_valu_kernel<D, ROWS, QM, false, false>), grid, dim3(256), 0, st, a);
  }
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

#if defined(KVQ_PHASE_STAMPS)
// Instrumented builds only: the device buffer the decode launches that follow
// write their phase stamps to (null: none), [workgroups * 16 * kPhaseSlots]
// uint64.
static unsigned long long* g_phase_stamps = nullptr;
extern "C" int kvq_probe_set_phase_stamps(void* buf) {
  g_phase_stamps = (unsigned long long*)buf;
  return 0;
}
#endif

using namespace kvq;

extern "C" int64_t kvq_decode_attn_num_splits(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                              int64_t D, int64_t s_max, int q_dtype,
                                              int scale_dtype, int64_t num_cus) {
  clear_error();
  if (!dtype_ok(q_dtype) || !dtype_ok(scale_dtype)) {
    set_error("kvq_decode_attn_num_splits: q and scale dtypes must be bf16/fp16/fp32");
    return KVQ_EINVAL;
  }
  if ((B == 0 || Sq == 0) && B >= 0 && Sq >= 0) return 1;  // nothing to launch
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
  if ((B == 0 || Sq == 0) && B >= 0 && Sq >= 0) return 0;  // nothing to launch
  // s_max only bounds n_split in planning; pass one long enough that every
  // split reaches min_split_tokens, so the plan keeps n_split.
  Plan p;
  const int rc = make_plan(B, Hq, Hkv, Sq, D, n_split * min_split_tokens(use_mfma(q_dtype, scale_dtype), D),
                           q_dtype, scale_dtype, n_split, 1, &p);
  if (rc != KVQ_OK) {
    set_error("kvq_decode_attn_workspace_bytes: unsupported or invalid shape");
    return rc;
  }
  return workspace_bytes_for(p, D);
}

// Decode-step extras: the new token's K/V rows and where they go.
struct StepArgs {
  const void* knew;
  const int64_t* kn_strides;
  const void* vnew;
  const int64_t* vn_strides;
  int64_t pos0;
};

// Paged-cache extras: the block table and the pools' geometry. The stride
// arrays passed along with them are (0, head, row): pools have no batch axis.
struct PagedArgs {
  const int32_t* bt;
  int64_t bt_stride, bt_cols, n_blocks, page_size;
};

// The cross-split merge relies on how gfx950 (MI355X) deals workgroups to its
// XCDs: round-robin over the XCDs in launch order, 8 per device in SPX mode
// (fewer in the partition modes, still a divisor of 8), so the splits of a unit
// (equal x % 8, unit_and_split) share one XCD and its L2. The library is built
// for gfx950 only; the device's architecture is still checked, once per device,
// before a split plan runs, so a launch on another part is refused instead of
// merging partials across L2s it does not keep coherent.
static std::mutex g_arch_mu;
static int8_t g_arch_ok[64] = {};  // 0 not checked, 1 gfx950, -1 another part

static int split_merge_device_ok() {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    set_error("kvq_decode_attn: hipGetDevice: %s", hipGetErrorString(e));
    return KVQ_EHIP;
  }
  if (dev < 0 || dev >= 64) {
    set_error("kvq_decode_attn: device %d beyond the 64 devices the split check tracks", dev);
    return KVQ_EUNSUP;
  }
  std::lock_guard<std::mutex> lock(g_arch_mu);
  if (g_arch_ok[dev] == 0) {
    hipDeviceProp_t prop;
    e = hipGetDeviceProperties(&prop, dev);
    if (e != hipSuccess) {
      set_error("kvq_decode_attn: hipGetDeviceProperties(%d): %s", dev, hipGetErrorString(e));
      return KVQ_EHIP;
    }
    g_arch_ok[dev] = std::strncmp(prop.gcnArchName, "gfx950", 6) == 0 &&
                             (prop.gcnArchName[6] == '\0' || prop.gcnArchName[6] == ':')
                         ? 1 : -1;
  }
  if (g_arch_ok[dev] < 0) {
    set_error("kvq_decode_attn: split plans need a gfx950 device (MI355X); device %d is another part "
              "(use n_split = 1)", dev);
    return KVQ_EUNSUP;
  }
  return KVQ_OK;
}

static int decode_attn_impl(const void* q, int q_dtype, const int64_t* q_strides,
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
                               void* stream, const StepArgs* step, const PagedArgs* pg) {
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
  // Vector loads: 16-byte key chunks; 16-byte value pieces (matrix-core
  // kernel) or 4-byte value dwords (VALU kernel); the matrix-core kernel loads
  // a token's whole scale row (2, 4 or 8 bytes) at once.
  const bool mfma = use_mfma(q_dtype, scale_dtype);
  const int64_t v_align = mfma ? 16 : 4;
  const bool k_al = ((uintptr_t)k_packed % 16 == 0) && kp_strides[0] % 16 == 0 &&
                    kp_strides[1] % 16 == 0 && kp_strides[2] % 16 == 0;
  const bool v_al = ((uintptr_t)v_packed % v_align == 0) && vp_strides[0] % v_align == 0 &&
                    vp_strides[1] % v_align == 0 && vp_strides[2] % v_align == 0;
  if (!k_al || !v_al) {
    set_error("kvq_decode_attn: packed K rows must be 16-byte aligned and V rows %lld-byte aligned",
              (long long)v_align);
    return KVQ_EUNSUP;
  }
  if (mfma) {
    const int64_t ng = (D + group_size - 1) / group_size;
    const int64_t sz = ng >= 4 ? 8 : (ng == 2 ? 4 : 2);
    bool s_al = true;
    for (const int64_t* st : {ks_strides, vs_strides})
      for (int i = 0; i < 3; ++i) s_al = s_al && (st[i] * 2) % sz == 0;
    s_al = s_al && (uintptr_t)k_scales % sz == 0 && (uintptr_t)v_scales % sz == 0;
    if (!s_al) {
      set_error("kvq_decode_attn: scale rows must be %lld-byte aligned", (long long)sz);
      return KVQ_EUNSUP;
    }
  }
  // Cache strides are non-negative and head strides below 2^32 (the kernels
  // form the head term of a slice offset as a 32 x 32 -> 64-bit product).
  for (const int64_t* st : {kp_strides, ks_strides, vp_strides, vs_strides}) {
    if (st[0] < 0 || st[1] < 0 || st[1] >= (1ll << 32)) {
      set_error("kvq_decode_attn: cache strides must be non-negative and head strides below 2^32");
      return KVQ_EUNSUP;
    }
  }
  // Token offsets inside one (batch, head) slice, or one head's pool, are 32-bit.
  const int64_t rows_addr = pg ? pg->n_blocks * pg->page_size : Sk;
  if (rows_addr > 0 && (rows_addr * kp_strides[2] >= (1ll << 31) || rows_addr * vp_strides[2] >= (1ll << 31) ||
                        rows_addr * ks_strides[2] * 4 >= (1ll << 31) || rows_addr * vs_strides[2] * 4 >= (1ll << 31))) {
    set_error("kvq_decode_attn: a (batch, head) slice of the cache (or a head's pool) exceeds 2 GiB");
    return KVQ_EUNSUP;
  }
  if (pg) {
    KVQ_CHECK_ARG(pg->page_size >= 64 && (pg->page_size & (pg->page_size - 1)) == 0 && pg->page_size <= (1 << 20),
                  "kvq_decode_attn_paged: page_size must be a power of two >= 64 (got %lld)",
                  (long long)pg->page_size);
    KVQ_CHECK_ARG(pg->n_blocks >= 0 && pg->n_blocks < (1ll << 31) && pg->bt_cols >= 0 &&
                      pg->bt_cols < (1ll << 31) && pg->bt_stride >= pg->bt_cols,
                  "kvq_decode_attn_paged: bad block table geometry");
    KVQ_CHECK_ARG(pg->bt != nullptr || pg->bt_cols == 0, "kvq_decode_attn_paged: null block table");
  }
  KVQ_CHECK_ARG(Sk * kMaxSplit < (1ll << 32) && Sq <= 0x7fffffffll, "kvq_decode_attn: sequence too long");

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
  if (p.n_split > 1) {
    const int drc = split_merge_device_ok();
    if (drc != KVQ_OK) return drc;
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
  a.causal = is_causal ? 1 : 0;
  a.scale_dtype = scale_dtype;
  a.div_rc = make_fastdiv((uint32_t)p.row_chunks);
  a.div_hkv = make_fastdiv((uint32_t)Hkv);
  a.div_sq = make_fastdiv((uint32_t)Sq);
  a.div_g = make_fastdiv((uint32_t)group_size);
  a.div_ns = make_fastdiv((uint32_t)p.n_split);
  a.ng = (int)((D + group_size - 1) / group_size);
  a.gsh_pack = 0;
  for (int c = 0; c < (int)(D / 32); ++c) a.gsh_pack |= (uint32_t)(16 * ((c * 32) / group_size)) << (8 * c);
  // 16-byte q loads need unit element stride and 16-byte aligned rows.
  a.q_vec = (q_dtype != KVQ_F32 && q_strides[3] == 1 && (uintptr_t)q % 16 == 0 &&
             q_strides[0] % 8 == 0 && q_strides[1] % 8 == 0 && q_strides[2] % 8 == 0) ? 1 : 0;
  {
    // 4-element output stores: unit dim stride, every row start a multiple of
    // 4 elements, a base aligned to 4 elements (D is a multiple of 4)
    const int64_t esz = q_dtype == KVQ_F32 ? 4 : 2;
    a.out_vec = (out_strides[3] == 1 && out_strides[0] % 4 == 0 && out_strides[1] % 4 == 0 &&
                 out_strides[2] % 4 == 0 && (uintptr_t)out % (4 * esz) == 0) ? 1 : 0;
  }
  a.scale_log2 = sm_scale * 1.4426950408889634f;
  a.append = step ? 1 : 0;
  a.pos0 = step ? (int)step->pos0 : 0;
  a.knew = step ? step->knew : nullptr;
  a.vnew = step ? step->vnew : nullptr;
  a.kns_b = step ? step->kn_strides[0] : 0; a.kns_h = step ? step->kn_strides[1] : 0;
  a.vns_b = step ? step->vn_strides[0] : 0; a.vns_h = step ? step->vn_strides[1] : 0;
  a.bt = pg ? pg->bt : nullptr;
  a.bt_stride = pg ? pg->bt_stride : 0;
  a.bt_cols = pg ? (int)pg->bt_cols : 0;
  a.n_blocks = pg ? (int)pg->n_blocks : 0;
  a.page_shift = 0;
  if (pg)
    while ((int64_t(1) << a.page_shift) < pg->page_size) ++a.page_shift;
  a.pool_rows = pg ? (uint32_t)(pg->n_blocks * pg->page_size) : 0u;
  a.ws_cnt = nullptr; a.ws_ml = nullptr; a.ws_o = nullptr;
#if defined(KVQ_PHASE_STAMPS)
  a.stamps = g_phase_stamps;
#endif
  if (need > 0) {
    char* w = (char*)workspace;
    a.ws_cnt = (uint32_t*)w;
    a.ws_ml = (float*)(w + ws_cnt_bytes(p));
    a.ws_o = (float*)(w + ws_cnt_bytes(p) + ws_ml_bytes(p));
  }
  const bool rowmask = is_causal && Sq > 1;
  // grid (8 * n_split, Y, Z), Y Z >= ceil(n_units / 8): every split of a unit
  // on one XCD (unit_and_split)
  const int64_t groups = (p.n_units + 7) / 8;
  const int64_t gy = std::min<int64_t>(groups, 32768), gz = (groups + gy - 1) / gy;
  const dim3 grid((unsigned)(8 * p.n_split), (unsigned)gy, (unsigned)gz);
  a.grid_y = (int)gy;
  hipStream_t st = (hipStream_t)stream;
  if (D == 128) launch_d<128>(a, p, q_dtype, rowmask, grid, st);
  else launch_d<64>(a, p, q_dtype, rowmask, grid, st);
  KVQ_CHECK_LAUNCH("kvq_decode_attn");
  return KVQ_OK;
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
  return decode_attn_impl(q, q_dtype, q_strides, k_packed, kp_strides, k_scales, ks_strides, v_packed,
                          vp_strides, v_scales, vs_strides, scale_dtype, out, out_strides, B, Hq, Hkv, Sq,
                          D, group_size, Sk, seq_lens, is_causal, sm_scale, n_split, workspace,
                          workspace_bytes, stream, nullptr, nullptr);
}

static int decode_step_impl(const void* q, int q_dtype, const int64_t* q_strides,
                            const void* k_new, const int64_t* kn_strides,
                            const void* v_new, const int64_t* vn_strides,
                            void* k_packed, const int64_t* kp_strides,
                            void* k_scales, const int64_t* ks_strides,
                            void* v_packed, const int64_t* vp_strides,
                            void* v_scales, const int64_t* vs_strides,
                            int scale_dtype,
                            void* out, const int64_t* out_strides,
                            int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                            int64_t group_size, int64_t capacity,
                            const int32_t* positions, int64_t pos0, float sm_scale,
                            int64_t n_split, void* workspace, int64_t workspace_bytes,
                            void* stream, const PagedArgs* pg) {
  KVQ_CHECK_ARG(dtype_ok(q_dtype) && dtype_ok(scale_dtype), "kvq_decode_step: bad dtype");
  KVQ_CHECK_ARG(kn_strides && vn_strides && q_strides, "kvq_decode_step: null stride array");
  if (!(group_size == 32 || group_size == 64 || group_size == 128)) {
    set_error("kvq_decode_step: needs group_size in {32, 64, 128} (got %lld)", (long long)group_size);
    return KVQ_EUNSUP;
  }
  KVQ_CHECK_ARG(capacity >= 1, "kvq_decode_step: capacity must be >= 1");
  KVQ_CHECK_ARG(positions != nullptr || (pos0 >= 0 && pos0 < capacity),
                "kvq_decode_step: write position %lld outside the cache capacity %lld", (long long)pos0,
                (long long)capacity);
  if (B == 0) return KVQ_OK;
  KVQ_CHECK_ARG(k_new && v_new, "kvq_decode_step: null new K/V");
  // a lane loads two consecutive elements of a new row: 4 bytes (16-bit
  // rows) or 8 bytes (fp32 rows)
  const int64_t pair = q_dtype == KVQ_F32 ? 8 : 4;
  const bool kn_ok = kn_strides[3] == 1 && (uintptr_t)k_new % pair == 0 && kn_strides[0] % 2 == 0 &&
                     kn_strides[1] % 2 == 0;
  const bool vn_ok = vn_strides[3] == 1 && (uintptr_t)v_new % pair == 0 && vn_strides[0] % 2 == 0 &&
                     vn_strides[1] % 2 == 0;
  if (!kn_ok || !vn_ok) {
    set_error("kvq_decode_step: new K/V rows need unit inner stride and %lld-byte aligned element pairs",
              (long long)pair);
    return KVQ_EUNSUP;
  }
  const StepArgs step{k_new, kn_strides, v_new, vn_strides, pos0};
  return decode_attn_impl(q, q_dtype, q_strides, k_packed, kp_strides, k_scales, ks_strides, v_packed,
                          vp_strides, v_scales, vs_strides, scale_dtype, out, out_strides, B, Hq, Hkv, 1,
                          D, group_size, capacity, positions, 0, sm_scale, n_split, workspace,
                          workspace_bytes, stream, &step, pg);
}

extern "C" int kvq_decode_step(const void* q, int q_dtype, const int64_t* q_strides,
                               const void* k_new, const int64_t* kn_strides,
                               const void* v_new, const int64_t* vn_strides,
                               void* k_packed, const int64_t* kp_strides,
                               void* k_scales, const int64_t* ks_strides,
                               void* v_packed, const int64_t* vp_strides,
                               void* v_scales, const int64_t* vs_strides,
                               int scale_dtype,
                               void* out, const int64_t* out_strides,
                               int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                               int64_t group_size, int64_t capacity,
                               const int32_t* positions, int64_t pos0, float sm_scale,
                               int64_t n_split, void* workspace, int64_t workspace_bytes,
                               void* stream) {
  clear_error();
  return decode_step_impl(q, q_dtype, q_strides, k_new, kn_strides, v_new, vn_strides, k_packed,
                          kp_strides, k_scales, ks_strides, v_packed, vp_strides, v_scales, vs_strides,
                          scale_dtype, out, out_strides, B, Hq, Hkv, D, group_size, capacity, positions,
                          pos0, sm_scale, n_split, workspace, workspace_bytes, stream, nullptr);
}

namespace {
// (head, row) pool strides -> the (batch, head, row) arrays of the contiguous
// code path, with batch stride 0.
struct Strides3 {
  int64_t v[3];
  Strides3(const int64_t* hr) : v{0, hr ? hr[0] : 0, hr ? hr[1] : 0} {}
};
}  // namespace

extern "C" int kvq_decode_attn_paged(const void* q, int q_dtype, const int64_t* q_strides,
                                     const void* k_pool, const int64_t* kp_strides,
                                     const void* k_scale_pool, const int64_t* ks_strides,
                                     const void* v_pool, const int64_t* vp_strides,
                                     const void* v_scale_pool, const int64_t* vs_strides,
                                     int scale_dtype,
                                     const int32_t* block_table, int64_t table_stride,
                                     int64_t table_cols, int64_t num_blocks, int64_t page_size,
                                     void* out, const int64_t* out_strides,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                                     int64_t group_size, const int32_t* seq_lens, int64_t seq_len,
                                     int is_causal, float sm_scale,
                                     int64_t n_split, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  clear_error();
  KVQ_CHECK_ARG(kp_strides && ks_strides && vp_strides && vs_strides, "kvq_decode_attn_paged: null stride array");
  KVQ_CHECK_ARG(page_size >= 1 && table_cols >= 0 && table_cols <= (1ll << 31) / page_size,
                "kvq_decode_attn_paged: bad page size or table width");
  const int64_t cap = table_cols * page_size;
  KVQ_CHECK_ARG(seq_lens != nullptr || (seq_len >= 0 && seq_len <= cap),
                "kvq_decode_attn_paged: seq_len %lld outside [0, %lld]", (long long)seq_len, (long long)cap);
  const PagedArgs pg{block_table, table_stride, table_cols, num_blocks, page_size};
  const Strides3 kp(kp_strides), ks(ks_strides), vp(vp_strides), vs(vs_strides);
  return decode_attn_impl(q, q_dtype, q_strides, k_pool, kp.v, k_scale_pool, ks.v, v_pool, vp.v,
                          v_scale_pool, vs.v, scale_dtype, out, out_strides, B, Hq, Hkv, Sq, D, group_size,
                          seq_lens ? cap : seq_len, seq_lens, is_causal, sm_scale, n_split, workspace,
                          workspace_bytes, stream, nullptr, &pg);
}

extern "C" int kvq_decode_step_paged(const void* q, int q_dtype, const int64_t* q_strides,
                                     const void* k_new, const int64_t* kn_strides,
                                     const void* v_new, const int64_t* vn_strides,
                                     void* k_pool, const int64_t* kp_strides,
                                     void* k_scale_pool, const int64_t* ks_strides,
                                     void* v_pool, const int64_t* vp_strides,
                                     void* v_scale_pool, const int64_t* vs_strides,
                                     int scale_dtype,
                                     const int32_t* block_table, int64_t table_stride,
                                     int64_t table_cols, int64_t num_blocks, int64_t page_size,
                                     void* out, const int64_t* out_strides,
                                     int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t group_size,
                                     const int32_t* positions, int64_t pos0, float sm_scale,
                                     int64_t n_split, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  clear_error();
  KVQ_CHECK_ARG(kp_strides && ks_strides && vp_strides && vs_strides, "kvq_decode_step_paged: null stride array");
  KVQ_CHECK_ARG(page_size >= 1 && table_cols >= 1 && table_cols <= (1ll << 31) / page_size,
                "kvq_decode_step_paged: bad page size or table width");
  const PagedArgs pg{block_table, table_stride, table_cols, num_blocks, page_size};
  const Strides3 kp(kp_strides), ks(ks_strides), vp(vp_strides), vs(vs_strides);
  return decode_step_impl(q, q_dtype, q_strides, k_new, kn_strides, v_new, vn_strides, k_pool, kp.v,
                          k_scale_pool, ks.v, v_pool, vp.v, v_scale_pool, vs.v, scale_dtype, out,
                          out_strides, B, Hq, Hkv, D, group_size, table_cols * page_size, positions, pos0,
                          sm_scale, n_split, workspace, workspace_bytes, stream, &pg);
}

// ---------------------------------------------------------------------------
// Allocation-free decode step: the split workspace is a file-scope device
// array, not a caller buffer, for callers that cannot allocate (code under
// HIP graph capture, serving loops, harnesses that forbid hipMalloc).

namespace {
constexpr int64_t kScratchBytes = 4ll << 20;  // the largest split workspace a call may need
constexpr int kScratchDevices = 64;
}  // namespace

// One copy per GPU the library runs on, held until the process ends. It is
// zero at load, and every completed call leaves its counter block at zero
// again (the merging workgroup re-arms each counter it used), so no call
// clears it; the partials need no initialisation.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

static std::mutex g_scratch_mu;
static void* g_scratch_ptr[kScratchDevices] = {};

// The device address of `scratch` on the current device, looked up once per
// device with that device current. (The array's name in host code is a
// host-side handle, not a device address.)
static int scratch_on_current_device(void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) {
    kvq::set_error("kvq_decode_step_noalloc: hipGetDevice: %s", hipGetErrorString(e));
    return KVQ_EHIP;
  }
  if (dev < 0 || dev >= kScratchDevices) {
    kvq::set_error("kvq_decode_step_noalloc: device %d beyond the %d devices with a scratch slot", dev,
                   kScratchDevices);
    return KVQ_EUNSUP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_ptr[dev] == nullptr) {
    void* p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || p == nullptr) {
      kvq::set_error("kvq_decode_step_noalloc: hipGetSymbolAddress(scratch) on device %d: %s", dev,
                     hipGetErrorString(e));
      return KVQ_EHIP;
    }
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return KVQ_OK;
}

extern "C" int kvq_decode_step_noalloc(const void* q, int q_dtype, const int64_t* q_strides,
                                       const void* k_new, const int64_t* kn_strides,
                                       const void* v_new, const int64_t* vn_strides,
                                       void* k_packed, const int64_t* kp_strides,
                                       void* k_scales, const int64_t* ks_strides,
                                       void* v_packed, const int64_t* vp_strides,
                                       void* v_scales, const int64_t* vs_strides,
                                       int scale_dtype,
                                       void* out, const int64_t* out_strides,
                                       int64_t B, int64_t Hq, int64_t Hkv, int64_t D,
                                       int64_t group_size, int64_t capacity,
                                       const int32_t* positions, int64_t pos0, float sm_scale,
                                       int64_t n_split, void* stream) {
  kvq::clear_error();
  const int64_t need = kvq_decode_attn_workspace_bytes(B, Hq, Hkv, 1, D, q_dtype, scale_dtype, n_split);
  if (need < 0) return (int)need;  // the planner set the message
  if (need > kScratchBytes) {
    kvq::set_error("kvq_decode_step_noalloc: the split plan needs %lld workspace bytes, more than the "
                   "%lld-byte static scratch (use kvq_decode_step with a workspace, or fewer splits)",
                   (long long)need, (long long)kScratchBytes);
    return KVQ_ESPACE;
  }
  void* ws = nullptr;
  if (need > 0) {
    const int rc = scratch_on_current_device(&ws);
    if (rc != KVQ_OK) return rc;
  }
  return decode_step_impl(q, q_dtype, q_strides, k_new, kn_strides, v_new, vn_strides, k_packed,
                          kp_strides, k_scales, ks_strides, v_packed, vp_strides, v_scales, vs_strides,
                          scale_dtype, out, out_strides, B, Hq, Hkv, D, group_size, capacity, positions, pos0,
                          sm_scale, n_split, ws, need > 0 ? kScratchBytes : 0, stream, nullptr);
}
