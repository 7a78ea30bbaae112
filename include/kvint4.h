/*
 * kvint4.h — C ABI of libkvint4.so, the gfx950 (MI355X) INT4 KV-cache decode path.
 *
 * Conventions shared by every entry point:
 *   - Plain pointers and sizes only. All data pointers are device pointers
 *     (HBM); the caller owns every allocation. No entry point allocates device
 *     memory, synchronizes the stream, or touches the host except to read its
 *     scalar arguments.
 *   - Kernels are enqueued on `stream` (a hipStream_t passed as void*; NULL =
 *     the null stream). Work is asynchronous with respect to the host.
 *   - Return value: KVQ_OK (0) on success, a negative KVQ_E* code otherwise.
 *     kvq_last_error() returns a thread-local, human-readable message for the
 *     last failing call on the calling thread.
 *   - dtype codes: KVQ_BF16, KVQ_F16, KVQ_F32.
 *   - Strides are in elements of the tensor's own type, except for the packed
 *     uint8 tensors whose strides are in bytes (same thing for uint8). The last
 *     (innermost) dimension of packed codes and of scales must be contiguous.
 *
 * Storage format (identical to the reference's, bit for bit):
 *   packed[..., j] : uint8, per group of `G` elements a run of ceil(G/2) bytes;
 *                    element 2i of the group goes to the low nibble of byte i,
 *                    element 2i+1 to the high nibble; code = round_half_even(
 *                    x / scale) clamped to [-8, 7], plus 8. For odd G the last
 *                    high nibble of each group is 0.
 *   scales[..., g] : scale = max|x_g| / 7 (or 1 for an all-zero group), computed
 *                    in fp32 and rounded to nearest-even into the scale dtype.
 */
#ifndef KVINT4_H
#define KVINT4_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum kvq_dtype { KVQ_BF16 = 0, KVQ_F16 = 1, KVQ_F32 = 2 };

enum kvq_status {
  KVQ_OK = 0,
  KVQ_EINVAL = -1,   /* bad argument: shape, dtype, stride, group size, null pointer */
  KVQ_ESPACE = -2,   /* workspace too small */
  KVQ_EHIP = -3,     /* HIP runtime error (launch failure, no device) */
  KVQ_EUNSUP = -4    /* shape valid but not handled by the fused kernel */
};

/* Library version: major*10000 + minor*100 + patch. kvq_version() returns
 * the version the library was built as; a binding declares the argument lists
 * of one major version and must refuse a library of another. 2.0.0 added the
 * capacity argument of kvq_quantize (1.x had none). */
#define KVQ_VERSION 20000
int kvq_version(void);

/* Thread-local message describing the last error on this thread ("" if none). */
const char* kvq_last_error(void);

/*
 * kvq_quantize — INT4 group quantize + pack, written in place.
 *
 * Replaces the quantizer of the reference:
 *   kernels/llama3/quantize.py:189-207 quantize_int4 (and the CPU semantics it
 *   must match, _quantize_int4_torch :126-148; scales in the input dtype), and
 *   kernels/gpt2/quantize.py:174-187 (same codes, scales always fp16), plus the
 *   append half of models/llama3/kv_cache.py:76-102 (which concatenates the new
 *   rows onto the cache; here they are written straight into a preallocated one).
 *
 * x:        [B, H, S, D] of x_dtype, element strides x_strides[4] (b, h, s, d).
 * packed:   destination codes, row stride layout [B, H, *, ceil(D/G)*ceil(G/2)],
 *           byte strides packed_strides[3] (b, h, s); last dim contiguous.
 * scales:   destination scales [B, H, *, ceil(D/G)] of scale_dtype, element
 *           strides scale_strides[3] (b, h, s); last dim contiguous.
 * Row (b, h, s) of x is written to destination row (b, h, pos_b + s) where
 * pos_b = write_pos[b] when write_pos (device int32 [B]) is not NULL, else
 * write_pos0. capacity = the destination's rows per (b, h): with write_pos
 * NULL, write_pos0 + S > capacity is rejected (KVQ_EINVAL) before any launch;
 * with device positions, rows that land at or past capacity (or below 0) are
 * dropped, as the decode step drops a token past the capacity.
 */
int kvq_quantize(const void* x, int x_dtype, const int64_t* x_strides,
                 int64_t B, int64_t H, int64_t S, int64_t D, int64_t group_size,
                 void* packed, const int64_t* packed_strides,
                 void* scales, int scale_dtype, const int64_t* scale_strides,
                 const int32_t* write_pos, int64_t write_pos0, int64_t capacity,
                 void* stream);

/*
 * kvq_dequantize — unpack + scale back to floating point.
 *
 * Replaces kernels/llama3/quantize.py:274-308 dequantize_int4 (CPU semantics
 * :210-234: value = (nibble - 8) * float(scale), rounded once into out_dtype,
 * truncated to d_out columns) and kernels/gpt2/quantize.py:190-214 (fp16 out).
 *
 * packed/scales: [B, H, S, ...] as written by kvq_quantize (strides as there).
 * num_groups:    scales' last dimension; the packed row must hold
 *                num_groups*ceil(G/2) bytes.
 * out:           [B, H, S, d_out] of out_dtype, element strides out_strides[4];
 *                d_out <= num_groups*G.
 */
int kvq_dequantize(const void* packed, const int64_t* packed_strides,
                   const void* scales, int scale_dtype, const int64_t* scale_strides,
                   int64_t B, int64_t H, int64_t S, int64_t group_size, int64_t num_groups,
                   void* out, int out_dtype, const int64_t* out_strides, int64_t d_out,
                   void* stream);

/*
 * Split-K planning for kvq_decode_attn. Pure host arithmetic (no device call):
 * returns the number of sequence splits the fused kernel will use for this
 * shape on a device with `num_cus` compute units (>= 1), or a negative status.
 * `s_max` is the longest sequence (tokens) that will be attended. bf16/fp16
 * queries with 16-bit scales run on the matrix-core kernel, other dtype pairs
 * on the exact-fp32 VALU kernel; the plan depends on which. An empty batch
 * (B == 0 or Sq == 0) plans 1 split and needs no workspace.
 */
int64_t kvq_decode_attn_num_splits(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                   int64_t D, int64_t s_max, int q_dtype, int scale_dtype,
                                   int64_t num_cus);

/*
 * Workspace (device bytes) kvq_decode_attn needs for `n_split` splits: a fixed
 * 320 KiB block of per-(batch, KV head) arrival counters, then the splits'
 * partial results. The workspace must be zero-filled once before its first
 * use; the kernel leaves its counters at zero again on exit, so it can be
 * reused by later calls on the same stream, with any plan. Calls that overlap
 * in time must not share a workspace.
 */
int64_t kvq_decode_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq,
                                        int64_t D, int q_dtype, int scale_dtype,
                                        int64_t n_split);

/*
 * kvq_decode_attn — fused INT4 GQA attention for short query blocks (decode).
 *
 * Replaces kernels/llama3/attention_quant.py:159-286 attention_forward_quant_gqa
 * (kernel :24-152) and kernels/gpt2/attention_quant.py:140-248
 * attention_forward_quant (the MHA case, Hq == Hkv) for the shapes the fused
 * kernel handles (D in {32, 64, 128}, group_size a multiple of 32 dividing
 * into D's 32-element chunks); KVQ_EUNSUP otherwise.
 *
 * q:    [B, Hq, Sq, D] of q_dtype, element strides q_strides[4].
 * k_packed/v_packed: [B, Hkv, Sk, num_groups*G/2] uint8, byte strides [3].
 * k_scales/v_scales: [B, Hkv, Sk, num_groups] of scale_dtype, strides [3].
 * out:  [B, Hq, Sq, D] of q_dtype, element strides out_strides[4].
 * Query head h reads KV head h / (Hq / Hkv). Keys of sequence b are the first
 * L_b = min(seq_lens[b], Sk) rows (seq_lens: device int32 [B], or NULL for
 * L_b = Sk). With is_causal, query row i may attend key j iff
 * j <= L_b - Sq + i (bottom-right alignment, as the reference kernel). A row
 * with no admissible key yields zeros. Scores are scaled by sm_scale.
 * n_split must come from kvq_decode_attn_num_splits (or be >= 1); workspace must
 * hold kvq_decode_attn_workspace_bytes(...) bytes (may be NULL when that is 0).
 */
int kvq_decode_attn(const void* q, int q_dtype, const int64_t* q_strides,
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
                    void* stream);

/*
 * kvq_decode_step — one decode token of one layer in one launch: quantize the
 * new K and V rows and append them to the INT4 cache in place, then attend
 * over the cache including them.
 *
 * Replaces, for Sq = 1, the pair the reference runs per layer and token:
 * models/llama3/kv_cache.py:76-105 QuantizedKVCache.append (quantize_int4,
 * kernels/llama3/quantize.py:189-207, then torch.cat) followed by
 * kernels/llama3/attention_quant.py:159-286 attention_forward_quant_gqa
 * (llama3_quant.py:62-88); codes and scales written are bit-identical to
 * kvq_quantize's and the attention matches kvq_decode_attn over the appended
 * cache.
 *
 * q:      [B, Hq, 1, D] (bf16, fp16 or fp32), element strides q_strides[4].
 * k_new, v_new: [B, Hkv, 1, D] in q's dtype, element strides [4] with unit
 *         inner stride, even batch/head strides and rows aligned to two
 *         elements (4 bytes for bf16/fp16, 8 for fp32).
 * k_packed/v_packed [B, Hkv, capacity, G*groups/2] uint8 and k_scales/
 * v_scales [B, Hkv, capacity, groups] (scale_dtype bf16, fp16 or fp32),
 * byte / element strides [3]: the cache buffers. bf16/fp16 queries with
 * 16-bit scales run on the matrix cores, the rest on the fp32 VALU kernel. Sequence b's old length is positions[b]
 * (device int32 [B]) or pos0 for every sequence; its new row is written at
 * that index and it attends old length + 1 keys. A sequence whose old length
 * is not below `capacity` is left unchanged and attends its first `capacity`
 * keys; one whose old length is negative is left unchanged and yields zeros
 * (pos0 is checked on the host).
 * group_size in {32, 64, 128}; D in {64, 128}. n_split / workspace as for
 * kvq_decode_attn (plan with s_max = the longest attended length).
 */
int kvq_decode_step(const void* q, int q_dtype, const int64_t* q_strides,
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
                    void* stream);

/*
 * kvq_decode_step_noalloc — kvq_decode_step with no workspace argument: the
 * split partials and counters go to a 4 MiB array of device memory that the
 * library holds per GPU (a static device array, looked up once per device),
 * so the call allocates nothing. No counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid hipMalloc).
 *
 * Arguments, results and errors as kvq_decode_step without workspace /
 * workspace_bytes. A plan whose workspace (kvq_decode_attn_workspace_bytes)
 * exceeds 4 MiB is refused with KVQ_ESPACE before any device call. Every call
 * on one GPU shares that GPU's array: calls that overlap in time on one GPU
 * race (serialize them, e.g. one stream); consecutive calls need nothing in
 * between (each leaves the array ready for the next).
 */
int kvq_decode_step_noalloc(const void* q, int q_dtype, const int64_t* q_strides,
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
                            int64_t n_split, void* stream);

/*
 * kvq_prefill_attn — attention of a long query block (prompt prefill, or a
 * prompt chunk after cached tokens) over an INT4 cache, on the matrix cores.
 * Replaces the reference's fused GQA kernel at Sq > 1
 * (kernels/llama3/attention_quant.py:159-286, launched by
 * models/llama3/llama3_quant.py:74-88 for prompts) and, in this build, the
 * dequantize + dense SDPA route for long blocks.
 *
 * Arguments and layouts as kvq_decode_attn, with one sequence length Sk for
 * the whole batch (no seq_lens). With is_causal, query row i may
 * attend key j iff j <= Sk - Sq + i; a row with no admissible key yields
 * zeros. K and V are dequantized to q's dtype ((n - 8) * scale, rounded to
 * nearest even) and the products accumulate in fp32.
 * Supported: bf16/fp16 q with bf16/fp16 scales, D in {64, 128}, group_size in
 * {32, 64, 128} dividing D, Hq / Hkv dividing 64, q and out rows contiguous;
 * KVQ_EUNSUP otherwise. B == 0 or Sq == 0 launches nothing.
 * workspace: device scratch of kvq_prefill_attn_workspace_bytes(...) bytes
 * (no initialisation needed). When the launch would be too small to fill
 * the device, the key range is split and the splits' partials are merged in
 * a second launch through it; NULL (or too small) runs unsplit. Calls that
 * overlap in time must not share a workspace.
 */
int64_t kvq_prefill_attn_workspace_bytes(int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                                         int64_t Sk);
int kvq_prefill_attn(const void* q, int q_dtype, const int64_t* q_strides,
                     const void* k_packed, const int64_t* kp_strides,
                     const void* k_scales, const int64_t* ks_strides,
                     const void* v_packed, const int64_t* vp_strides,
                     const void* v_scales, const int64_t* vs_strides,
                     int scale_dtype,
                     void* out, const int64_t* out_strides,
                     int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                     int64_t group_size, int64_t Sk, int is_causal, float sm_scale,
                     void* workspace, int64_t workspace_bytes, void* stream);

/*
 * Paged caches.
 *
 * The reference keeps one contiguous tensor per layer and grows it with
 * torch.cat (models/llama3/kv_cache.py:76-105); it has no paged layout. These
 * entry points are the paged counterparts of the ones above (same arguments
 * and semantics) for a cache whose rows live in a block pool:
 *
 *   pools:  codes [H, num_blocks * page_size, W] uint8 and scales
 *           [H, num_blocks * page_size, num_groups] of scale_dtype; the stride
 *           arrays are [2]: (head, row), bytes for codes, elements for scales.
 *   block_table: device int32 [B, table_stride]; token t of sequence b is pool
 *           row block_table[b * table_stride + t / page_size] * page_size +
 *           t % page_size, for t < table_cols * page_size. page_size is a power
 *           of two. An entry < 0 or >= num_blocks marks a page with no block:
 *           writes to it are dropped and its rows are absent (dequantize writes
 *           zeros; attention never reads past a sequence's length, and its
 *           length must not reach such a page).
 *
 * The attention entry points (kvq_decode_attn_paged, kvq_decode_step_paged)
 * need page_size >= 64 (bf16/fp16 queries with 16-bit scales run on the
 * matrix cores, fp32 queries or scales on the exact-fp32 kernel); a head's
 * pool must stay below 2 GiB. Planning and workspace: kvq_decode_attn_num_splits
 * (s_max = the longest attended length) and kvq_decode_attn_workspace_bytes,
 * as for the contiguous cache.
 */
int kvq_quantize_paged(const void* x, int x_dtype, const int64_t* x_strides,
                       int64_t B, int64_t H, int64_t S, int64_t D, int64_t group_size,
                       void* packed_pool, const int64_t* pool_strides,
                       void* scale_pool, int scale_dtype, const int64_t* scale_pool_strides,
                       const int32_t* block_table, int64_t table_stride, int64_t table_cols,
                       int64_t num_blocks, int64_t page_size,
                       const int32_t* write_pos, int64_t write_pos0,
                       void* stream);

int kvq_dequantize_paged(const void* packed_pool, const int64_t* pool_strides,
                         const void* scale_pool, int scale_dtype, const int64_t* scale_pool_strides,
                         const int32_t* block_table, int64_t table_stride, int64_t table_cols,
                         int64_t num_blocks, int64_t page_size,
                         int64_t B, int64_t H, int64_t S, int64_t group_size, int64_t num_groups,
                         void* out, int out_dtype, const int64_t* out_strides, int64_t d_out,
                         void* stream);

/* Keys of sequence b: its first seq_lens[b] tokens (seq_lens: device int32
 * [B]), or seq_len for every sequence when seq_lens is NULL. */
int kvq_decode_attn_paged(const void* q, int q_dtype, const int64_t* q_strides,
                          const void* k_pool, const int64_t* kp_strides,
                          const void* k_scale_pool, const int64_t* ks_strides,
                          const void* v_pool, const int64_t* vp_strides,
                          const void* v_scale_pool, const int64_t* vs_strides,
                          int scale_dtype,
                          const int32_t* block_table, int64_t table_stride, int64_t table_cols,
                          int64_t num_blocks, int64_t page_size,
                          void* out, const int64_t* out_strides,
                          int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                          int64_t group_size, const int32_t* seq_lens, int64_t seq_len,
                          int is_causal, float sm_scale,
                          int64_t n_split, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* Capacity = table_cols * page_size; a position whose page has no block is
 * neither written nor attended. */
int kvq_decode_step_paged(const void* q, int q_dtype, const int64_t* q_strides,
                          const void* k_new, const int64_t* kn_strides,
                          const void* v_new, const int64_t* vn_strides,
                          void* k_pool, const int64_t* kp_strides,
                          void* k_scale_pool, const int64_t* ks_strides,
                          void* v_pool, const int64_t* vp_strides,
                          void* v_scale_pool, const int64_t* vs_strides,
                          int scale_dtype,
                          const int32_t* block_table, int64_t table_stride, int64_t table_cols,
                          int64_t num_blocks, int64_t page_size,
                          void* out, const int64_t* out_strides,
                          int64_t B, int64_t Hq, int64_t Hkv, int64_t D, int64_t group_size,
                          const int32_t* positions, int64_t pos0, float sm_scale,
                          int64_t n_split, void* workspace, int64_t workspace_bytes,
                          void* stream);

/* kvq_prefill_attn over a paged cache: every sequence attends its first Sk
 * tokens (Sk <= table_cols * page_size); page_size >= 64. A key whose page has
 * no block reads as zero codes and scales (score 0, value 0). */
int kvq_prefill_attn_paged(const void* q, int q_dtype, const int64_t* q_strides,
                           const void* k_pool, const int64_t* kp_strides,
                           const void* k_scale_pool, const int64_t* ks_strides,
                           const void* v_pool, const int64_t* vp_strides,
                           const void* v_scale_pool, const int64_t* vs_strides,
                           int scale_dtype,
                           const int32_t* block_table, int64_t table_stride, int64_t table_cols,
                           int64_t num_blocks, int64_t page_size,
                           void* out, const int64_t* out_strides,
                           int64_t B, int64_t Hq, int64_t Hkv, int64_t Sq, int64_t D,
                           int64_t group_size, int64_t Sk, int is_causal, float sm_scale,
                           void* workspace, int64_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* KVINT4_H */
