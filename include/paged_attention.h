/*
 * C ABI of the gfx950 paged-attention library (libpaged_attention.so).
 *
 * It replaces the device work behind simpissa/vllm-jax's attention seam
 * (vllm/model/qwen3.py:172-218): the KV-cache scatter, the Pallas prefill
 * kernel and the Pallas decode kernel.  Conventions:
 *
 *   - every pointer argument except `stream` is a device pointer;
 *   - bf16 tensors are passed as uint16_t bit patterns;
 *   - strides are in elements; the innermost (head_dim) stride is always 1;
 *   - a KV pool is addressed as (page, slot-in-page, kv-head, dim) with
 *     caller-given strides, so both the engine's native layout
 *     kv_cache[i] = [num_pages, page_size, Hkv, d] (model_runner.py:190-199)
 *     and the reference kernels' k_pages = [Hkv, num_pages, page_size, d]
 *     (prefill_paged_attention.py:186, decode_paged_attention.py:323-324)
 *     are accepted without a copy;
 *   - `stream` is a hipStream_t (NULL = the default stream); calls are
 *     asynchronous and stream-ordered, allocate nothing and never
 *     synchronise the host;
 *   - return value 0 = success, negative = error; pa_last_error() describes
 *     the last error of the calling thread.
 *
 * Device-side metadata is never trusted to be in range: negative block-table
 * entries read page 0 (as qwen3.py:179-180,198-199 sanitise them), entries
 * past the pool are clamped into it, and slots outside [0, pages*page_size)
 * are skipped by the KV store.
 *
 * Supported shapes: num_heads % num_kv_heads == 0, and
 *   - head_dim 128 in every entry (the tuned kernels); pa_prefill, pa_decode,
 *     pa_decode_noalloc, pa_mixed and the quantized-page entries
 *     (pa_kv_store_fp8, pa_decode_fp8 / _quant, pa_prefill_fp8 / _quant)
 *     also take any multiple of 16 from 16 to 256 (generic kernels, same
 *     arithmetic, lower throughput);
 *   - q heads per kv head: any number for decode, up to 256 for prefill and
 *     pa_mixed (up to 128 for prefill at head sizes from 144 on).
 */
#ifndef VLLM_JAX_AMD_PAGED_ATTENTION_H_
#define VLLM_JAX_AMD_PAGED_ATTENTION_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define PA_OK 0
#define PA_ERR_INVALID_ARGUMENT (-1)
#define PA_ERR_UNSUPPORTED (-2)
#define PA_ERR_WORKSPACE (-3)
#define PA_ERR_LAUNCH (-4)

/* Message for the last non-zero return code on this thread ("" if none). */
const char* pa_last_error(void);

/* ABI version; bumped on any signature change. */
int pa_abi_version(void);

/*
 * KV store: k_cache[slot[t]] = k[t], v_cache[slot[t]] = v[t] for every token
 * t whose slot lies in [0, num_pages*page_size); other tokens are skipped.
 * Slot s addresses page s / page_size, in-page slot s % page_size.
 * Replaces _update_kv_cache (vllm/model/qwen3.py:105-111), in place.
 * k: [num_tokens, Hkv, d] with strides (k_tok_stride, k_head_stride, 1);
 * v likewise.  Slots must be unique (the reference leaves the winner of a
 * duplicate unspecified).
 */
int pa_kv_store(const uint16_t* k, int64_t k_tok_stride, int64_t k_head_stride,
                const uint16_t* v, int64_t v_tok_stride, int64_t v_head_stride,
                const int32_t* slot_mapping, int32_t num_tokens,
                int32_t num_kv_heads, int32_t head_dim,
                uint16_t* k_cache, uint16_t* v_cache,
                int32_t num_pages, int32_t page_size,
                int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                void* stream);

/*
 * Block-table gather (test/debug entry): out[b, j] = cache[bt[b, j / page_size],
 * j % page_size] for j < lengths[b], zero for j >= lengths[b].
 * out: contiguous [batch, pages_per_seq * page_size, Hkv, d].
 * This is the address arithmetic of prefill_paged_attention.py:79-82 and
 * decode_paged_attention.py:69-71 (dense form: qwen3.py:114-134).
 */
int pa_gather_kv(const uint16_t* cache, int32_t num_pages, int32_t page_size,
                 int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                 const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                 const int32_t* lengths, int32_t batch,
                 int32_t num_kv_heads, int32_t head_dim, uint16_t* out, void* stream);

/*
 * Decode workspace in bytes for a launch of `batch` sequences whose block
 * tables are `pages_per_seq` wide: f32 split partials and their max/sum,
 * then a work list of (sequence, chunk) pairs.  From 2048 workgroups on,
 * pa_decode orders the pairs by length and deals them over the XCDs (one
 * extra launch); the output does not depend on the order.  The workspace is
 * 256-byte aligned.
 */
size_t pa_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t head_dim,
                                int32_t pages_per_seq, int32_t page_size);

/*
 * Split-K paged GQA decode: for each sequence b and q head h,
 *   out[b, h] = softmax_j(scale * q[b, h] . k_j) v_j,  j < lengths[b],
 * with k_j / v_j of kv head h / (num_heads / num_kv_heads) read through
 * block_tables[b].  lengths[b] == 0 gives a zero row.  soft_cap > 0 applies
 * soft_cap * tanh(logit / soft_cap).  Any number of q heads per kv head: a
 * work item takes them 16 at a time (32 at a time over bf16 pages above 16
 * per kv head, and at head sizes other than 128; the reference pads the
 * group to its block_h, decode_paged_attention.py:188-197), so each block
 * of q heads reads its kv head's K/V once.
 * Replaces decode_paged_attention (decode_paged_attention.py:300-397); that
 * entry expects q pre-scaled (qwen3.py:207), i.e. scale = 1.
 * q: [batch, H, d] strides (q_batch_stride, q_head_stride, 1);
 * out: [batch, H, d] strides (out_batch_stride, out_head_stride, 1).
 */
int pa_decode(const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
              const uint16_t* k_cache, const uint16_t* v_cache,
              int32_t num_pages, int32_t page_size,
              int64_t page_stride, int64_t slot_stride, int64_t head_stride,
              const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
              const int32_t* lengths, int32_t batch,
              int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
              float scale, float soft_cap,
              uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride,
              void* workspace, size_t workspace_bytes, void* stream);

/*
 * pa_decode without a caller workspace and without any allocation: the
 * split partials and the work list live in a static device array of
 * pa_decode_noalloc_max_workspace() bytes (64 MiB) that every GPU the library
 * runs on holds until the process ends.  Arguments, results and errors are
 * those of pa_decode; a launch whose pa_decode_workspace_size exceeds the
 * array returns PA_ERR_WORKSPACE before touching the device.  The array's
 * device address is looked up once per device, on the first call with that
 * device current (the stream must belong to the current device); a caller
 * that captures the call in a HIP graph makes one call on the device before
 * the capture, after which a call records only kernel launches.  Calls
 * that overlap on one GPU share the array and race: serialise them (one
 * stream, or events).  No counterpart in the reference: it exists for callers
 * that cannot allocate device memory (code under HIP graph capture, serving
 * loops that forbid hipMalloc).
 */
int pa_decode_noalloc(const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
                      const uint16_t* k_cache, const uint16_t* v_cache,
                      int32_t num_pages, int32_t page_size,
                      int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                      const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                      const int32_t* lengths, int32_t batch,
                      int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                      float scale, float soft_cap,
                      uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride, void* stream);

/* Bytes of pa_decode_noalloc's static scratch (the largest workspace it can serve). */
size_t pa_decode_noalloc_max_workspace(void);

/*
 * Ragged causal GQA paged prefill.  Sequence b owns q rows
 * [cu_seqlens_q[b], cu_seqlens_q[b+1]) and kv indices [0, Lk_b) with
 * Lk_b = cu_seqlens_k[b+1] - cu_seqlens_k[b] (cu_seqlens_k == NULL: Lk_b is
 * the q length, the reference's rule).  kv index j has position
 * j + input_positions[cu_seqlens_q[b]] - (Lk_b - Lq_b) and is visible to row
 * i iff that position <= input_positions[i].  Rows outside every sequence
 * are written as zeros.  max_seqlen_q bounds every q length (the reference's
 * static max_seqlen_bucket may be passed).
 * Replaces prefill_paged_attention (prefill_paged_attention.py:407-453),
 * which scales q by 1/sqrt(d) itself (prefill_paged_attention.py:60).
 * q/out: [num_tokens, H, d] with (tok, head) strides.
 * workspace (256-byte aligned, pa_prefill_workspace_size bytes, or NULL)
 * holds a work list that orders the (q tile, sequence, kv head) items by
 * their kv length, longest first; it changes no result.  Without it (or for
 * batch > 2048) items run from the last q tile down.
 */
int pa_prefill(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
               const uint16_t* k_cache, const uint16_t* v_cache,
               int32_t num_pages, int32_t page_size,
               int64_t page_stride, int64_t slot_stride, int64_t head_stride,
               const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
               const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
               const int32_t* input_positions,
               int32_t batch, int32_t num_tokens, int32_t max_seqlen_q,
               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
               float scale, float soft_cap,
               uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride,
               void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes of pa_prefill's work list (0 for bad sizes); no
 * counterpart in the reference, whose grid order is fixed. */
size_t pa_prefill_workspace_size(int32_t batch, int32_t max_seqlen_q, int32_t num_heads,
                                 int32_t num_kv_heads);

/*
 * The layer step between the q/k/v projections and attention, fused:
 *   q_out[t, h]        = rope(rmsnorm(q[t, h]) * q_norm_weight, pos[t])
 *   k_cache[slot[t], h] = rope(rmsnorm(k[t, h]) * k_norm_weight, pos[t])
 *   v_cache[slot[t], h] = v[t, h]
 * rmsnorm(x) = x * rsqrt(mean(x^2) + eps); rope rotates interleaved pairs
 * (x[2i], x[2i+1]) by pos * inv_freq[i], inv_freq = 1 / theta^(2i/d), with
 * positions divided by rope_scaling_factor (1 = no scaling), all evaluated
 * with bf16 operands as the reference does.  Tokens whose slot lies outside
 * [0, num_pages*page_size) store nothing (q_out is still written).
 * Replaces q_norm/k_norm + apply_rope (vllm/model/qwen3.py:286-296,
 * 59-78) and the K/V scatter of _update_kv_cache (qwen3.py:105-111).
 * q/k/v/q_out: [num_tokens, heads, d] with (tok, head) strides; the norm
 * weights are [d].  q_out may alias q (same strides).
 */
int pa_qk_norm_rope_store(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                          const uint16_t* k, int64_t k_tok_stride, int64_t k_head_stride,
                          const uint16_t* v, int64_t v_tok_stride, int64_t v_head_stride,
                          const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
                          float eps, float rope_theta, float rope_scaling_factor,
                          const int32_t* positions, const int32_t* slot_mapping,
                          int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                          uint16_t* q_out, int64_t q_out_tok_stride, int64_t q_out_head_stride,
                          uint16_t* k_cache, uint16_t* v_cache,
                          int32_t num_pages, int32_t page_size,
                          int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                          void* stream);

/*
 * Quantising KV store for float8 pages: for every token t with a slot in the
 * pool and every kv head h, the row x = k[t, h] (bf16, d = 128) is stored as
 * e4m3fn codes e4m3(x / s) (round to nearest even) with scale s, the
 * smallest power of two with amax / s <= 448 and s >= 2^-126 (amax = max |x|;
 * an all-zero row stores scale 1), and likewise v.  Readers take any
 * scales; power-of-two ones widen exactly in one conversion.  Code pools: (page, slot, head) byte strides as in pa_kv_store; scale
 * pools: float (page, slot, head) strides, e.g. the [Hkv, NB, BS] layout of
 * k_scales_pages (decode_paged_attention.py:206-217).  The reference reads
 * quantised pages but has no writer; this quantiser is the library's own.
 */
int pa_kv_store_fp8(const uint16_t* k, int64_t k_tok_stride, int64_t k_head_stride,
                    const uint16_t* v, int64_t v_tok_stride, int64_t v_head_stride,
                    const int32_t* slot_mapping, int32_t num_tokens,
                    int32_t num_kv_heads, int32_t head_dim,
                    uint8_t* k_cache, uint8_t* v_cache, float* k_scales, float* v_scales,
                    int32_t num_pages, int32_t page_size,
                    int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                    int64_t scale_page_stride, int64_t scale_slot_stride, int64_t scale_head_stride,
                    void* stream);

/*
 * Code types of 1-byte quantized pages (pa_decode_quant, pa_prefill_quant).
 * The reference casts quantized pages of any dtype to q's dtype before the
 * dot (decode_paged_attention.py:72-75, prefill_paged_attention.py:84-85):
 * e4m3fn codes are their float8 values, int8 / uint8 codes the integers
 * -128..127 / 0..255; all are exact in bf16.
 */
#define PA_CODE_E4M3 0
#define PA_CODE_INT8 1
#define PA_CODE_UINT8 2

/*
 * pa_decode over float8 e4m3fn pages with per-token scales: the logit of
 * token j is (q . bf16(k_j)) * k_scales[j] * scale, and P is multiplied by
 * v_scales[j] before PV (decode_paged_attention.py:72-81,108-115, the
 * k_scales_pages / v_scales_pages path of :300-397).  Code strides are in
 * bytes; scales are addressed page * scale_page_stride + head *
 * scale_head_stride + slot (slot stride 1; both strides multiples of 4).
 * page_size must be a multiple of 16.  Same workspace as pa_decode.
 */
int pa_decode_fp8(const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
                  const uint8_t* k_cache, const uint8_t* v_cache,
                  const float* k_scales, const float* v_scales,
                  int32_t num_pages, int32_t page_size,
                  int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                  int64_t scale_page_stride, int64_t scale_head_stride,
                  const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                  const int32_t* lengths, int32_t batch,
                  int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                  float scale, float soft_cap,
                  uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride,
                  void* workspace, size_t workspace_bytes, void* stream);

/*
 * pa_decode_fp8 for any code type (PA_CODE_*; pa_decode_fp8 is code_type
 * PA_CODE_E4M3): k_j is the code's value, exact in bf16, and the logit and P
 * scaling are the same.  Replaces the k_scales_pages / v_scales_pages path of
 * decode_paged_attention (decode_paged_attention.py:72-81,108-115) for int8
 * and uint8 pages as well.  An unknown code_type returns
 * PA_ERR_INVALID_ARGUMENT before the device is touched.
 */
int pa_decode_quant(int32_t code_type, const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
                    const uint8_t* k_cache, const uint8_t* v_cache,
                    const float* k_scales, const float* v_scales,
                    int32_t num_pages, int32_t page_size,
                    int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                    int64_t scale_page_stride, int64_t scale_head_stride,
                    const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                    const int32_t* lengths, int32_t batch,
                    int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                    float scale, float soft_cap,
                    uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride,
                    void* workspace, size_t workspace_bytes, void* stream);

/* Workspace bytes pa_prefill_fp8 / pa_prefill_quant need: room for two bf16 pages per
 * block-table entry (K and V), two int32 per entry and a count, then
 * pa_prefill's work list. */
size_t pa_prefill_fp8_workspace_size(int32_t batch, int32_t pages_per_seq, int32_t page_size,
                                     int32_t num_kv_heads, int32_t head_dim, int32_t max_seqlen_q,
                                     int32_t num_heads);

/*
 * pa_prefill over float8 e4m3fn pages with per-token scales
 * (prefill_paged_attention.py:169-170,255-266, in-kernel :84-92,120-123).
 * Every distinct physical page the sequences use is first widened once into
 * the workspace as bf16 (code * token scale, one rounding), so pages shared
 * between sequences (cached prefixes) are widened once; the bf16 prefill then
 * runs on those pages through a remapped table.  The reference scales the logits and P instead of K and V; the two
 * differ by that one bf16 rounding.  Strides and scales as in pa_decode_fp8;
 * the workspace (256-byte aligned) is caller-owned.
 */
int pa_prefill_fp8(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                   const uint8_t* k_cache, const uint8_t* v_cache,
                   const float* k_scales, const float* v_scales,
                   int32_t num_pages, int32_t page_size,
                   int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                   int64_t scale_page_stride, int64_t scale_head_stride,
                   const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                   const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                   const int32_t* input_positions,
                   int32_t batch, int32_t num_tokens, int32_t max_seqlen_q,
                   int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                   float scale, float soft_cap,
                   uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride,
                   void* workspace, size_t workspace_bytes, void* stream);

/*
 * pa_prefill_fp8 for any code type (PA_CODE_*; pa_prefill_fp8 is code_type
 * PA_CODE_E4M3): pages are widened to bf16(code value * token scale) and the
 * bf16 prefill runs on them.  Replaces the k_scales_pages / v_scales_pages
 * path of prefill_paged_attention (prefill_paged_attention.py:84-92,118-123)
 * for int8 and uint8 pages as well.  An unknown code_type returns
 * PA_ERR_INVALID_ARGUMENT before the device is touched.
 */
int pa_prefill_quant(int32_t code_type, const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                     const uint8_t* k_cache, const uint8_t* v_cache,
                     const float* k_scales, const float* v_scales,
                     int32_t num_pages, int32_t page_size,
                     int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                     int64_t scale_page_stride, int64_t scale_head_stride,
                     const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                     const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                     const int32_t* input_positions,
                     int32_t batch, int32_t num_tokens, int32_t max_seqlen_q,
                     int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                     float scale, float soft_cap,
                     uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride,
                     void* workspace, size_t workspace_bytes, void* stream);

/*
 * Workspace bytes pa_mixed needs (0 for bad sizes): decode partials when a
 * decode sequence can span more than one 4096-token chunk, then a work list
 * of (decode chunk | prefill q tile) pairs.  From 2048 workgroups on,
 * pa_mixed orders the pairs by their measured cost and deals them over the
 * XCDs (one extra launch); the output does not depend on the order.
 */
size_t pa_mixed_workspace_size(int32_t batch, int32_t num_decodes, int32_t max_seqlen_q,
                               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                               int32_t pages_per_seq, int32_t page_size);

/*
 * One launch for a scheduler step that mixes decode and prefill sequences,
 * unpadded.  Sequence b owns q rows [cu_seqlens_q[b], cu_seqlens_q[b+1]) and
 * kv indices [0, kv_lens[b]) through block_tables[b].
 *   - b < num_decodes (decode): its single q row attends to every kv index,
 *     scale decode_scale (the reference pre-scales q, qwen3.py:207: pass 1
 *     for such q); kv_lens[b] == 0 gives a zero row; a decode sequence
 *     without a q row writes nothing.
 *   - b >= num_decodes (prefill): as pa_prefill with Lk_b = kv_lens[b],
 *     scale prefill_scale, rows at offset >= max_seqlen_q left zero.
 * Rows outside every sequence, and rows past the first of a decode
 * sequence, are written as zeros.
 * Replaces the reference step's two jitted calls, decode then prefill, each
 * padded to a power-of-two bucket (vllm/src/model_runner.py:310-333, padding
 * 243-255, 286-292), at the attention seam (vllm/model/qwen3.py:172-218).
 * q/out: [num_tokens, H, d] with (tok, head) strides.
 */
int pa_mixed(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
             const uint16_t* k_cache, const uint16_t* v_cache,
             int32_t num_pages, int32_t page_size,
             int64_t page_stride, int64_t slot_stride, int64_t head_stride,
             const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
             const int32_t* cu_seqlens_q, const int32_t* kv_lens, const int32_t* input_positions,
             int32_t batch, int32_t num_decodes, int32_t num_tokens, int32_t max_seqlen_q,
             int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
             float prefill_scale, float decode_scale, float soft_cap,
             uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride,
             void* workspace, size_t workspace_bytes, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_JAX_AMD_PAGED_ATTENTION_H_ */
