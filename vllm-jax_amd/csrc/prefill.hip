// Ragged causal GQA paged prefill for gfx950: the kernel entry and its host
// launcher.  The work item (one q tile of one sequence and kv head) is
// prefill_body in prefill_impl.h.
#include "prefill_impl.h"

namespace pa {

template <bool kSoftCap, bool kAligned>
__global__ void __launch_bounds__(kThreads, 1)
prefill_kernel(PrefillParams p) {
  prefill_body<kSoftCap, kAligned>(p, blockIdx.x);
}

// Zero every output row the prefill kernel does not write: rows outside all
// sequences (before cu_q[0], from cu_q[batch] on) and rows at offset >=
// max_seqlen_q inside their sequence (the reference drops those too: its
// scatter only covers the first max_seqlen_bucket rows, prefill...:384-388).
// One wave per token row.
__global__ void __launch_bounds__(256)
prefill_zero_rows_kernel(const int32_t* __restrict__ cu_q, int32_t batch, int32_t num_tokens,
                         int32_t max_seqlen_q, int32_t num_heads, uint16_t* __restrict__ out,
                         int64_t o_ts, int64_t o_hs) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= num_tokens) return;
  bool covered = false;
  if (t >= cu_q[0] && t < cu_q[batch]) {
    // last b with cu_q[b] <= t
    int lo = 0, hi = batch;  // invariant: cu_q[lo] <= t < cu_q[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cu_q[mid] <= t) lo = mid;
      else hi = mid;
    }
    covered = t - cu_q[lo] < max_seqlen_q;
  }
  if (covered) return;
  const int chunks_per_head = kPHeadDim / 8;
  for (int c = lane; c < num_heads * chunks_per_head; c += 64) {
    const int hh = c / chunks_per_head;
    const int e = (c - hh * chunks_per_head) * 8;
    st16(out + t * o_ts + hh * o_hs + e, u32x4{0, 0, 0, 0});
  }
}

}  // namespace pa

using namespace pa;

extern "C" int pa_prefill(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
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
                          void* stream) {
  if (batch < 0 || num_tokens < 0 || max_seqlen_q < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_pages <= 0 || page_size <= 0 || pages_per_seq < 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_prefill: bad sizes (batch=%d, num_tokens=%d, max_seqlen_q=%d, num_heads=%d, "
                "num_kv_heads=%d, num_pages=%d, page_size=%d, pages_per_seq=%d)",
                batch, num_tokens, max_seqlen_q, num_heads, num_kv_heads, num_pages, page_size,
                pages_per_seq);
  if (num_heads % num_kv_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_prefill: Number of Q heads must be divisible by number of KV heads. Got %d and %d.",
                num_heads, num_kv_heads);
  if (head_dim != kPHeadDim)
    return fail(PA_ERR_UNSUPPORTED, "pa_prefill: head_dim %d not supported (only %d)", head_dim, kPHeadDim);
  const int group = num_heads / num_kv_heads;
  if (group > kRows)
    return fail(PA_ERR_UNSUPPORTED, "pa_prefill: %d q heads per kv head not supported (max %d)", group, kRows);
  if (num_tokens == 0) return PA_OK;
  if (!q || !out || !cu_seqlens_q || !input_positions || (batch > 0 && (!k_cache || !v_cache || !block_tables)))
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_prefill: null pointer");
  const uintptr_t align_bits = (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out;
  if ((align_bits & 15u) || (q_tok_stride | q_head_stride | page_stride | slot_stride | head_stride |
                             out_tok_stride | out_head_stride) % 8)
    return fail(PA_ERR_UNSUPPORTED, "pa_prefill: operands must be 16-byte aligned with strides multiple of 8");
  hipStream_t s = (hipStream_t)stream;

  {
    prefill_zero_rows_kernel<<<dim3((unsigned)((num_tokens + 3) / 4)), dim3(256), 0, s>>>(
        cu_seqlens_q, batch, num_tokens, max_seqlen_q, num_heads, out, out_tok_stride, out_head_stride);
    int rc = launch_status("pa_prefill(zero rows)");
    if (rc) return rc;
  }
  if (batch == 0 || max_seqlen_q == 0) return PA_OK;

  PrefillParams prm;
  prm.q = q;
  prm.q_ts = q_tok_stride;
  prm.q_hs = q_head_stride;
  prm.k_cache = k_cache;
  prm.v_cache = v_cache;
  prm.num_pages = num_pages;
  prm.page_size = page_size;
  prm.page_stride = page_stride;
  prm.slot_stride = slot_stride;
  prm.head_stride = head_stride;
  prm.block_tables = block_tables;
  prm.bt_stride = bt_stride;
  prm.pages_per_seq = pages_per_seq;
  prm.cu_q = cu_seqlens_q;
  prm.cu_k = cu_seqlens_k;
  prm.kv_lens = nullptr;
  prm.positions = input_positions;
  prm.batch = batch;
  prm.num_tokens = num_tokens;
  prm.num_heads = num_heads;
  prm.num_kv_heads = num_kv_heads;
  prm.group = group;
  prm.tile_tokens = kRows / group;
  prm.n_qtiles = (max_seqlen_q + prm.tile_tokens - 1) / prm.tile_tokens;
  prm.max_seqlen_q = max_seqlen_q;
  prm.soft_cap = soft_cap > 0.f ? soft_cap : 0.f;
  prm.logit_scale = prm.soft_cap > 0.f ? scale : scale * kLog2e;
  prm.out = out;
  prm.o_ts = out_tok_stride;
  prm.o_hs = out_head_stride;
  const int64_t blocks = (int64_t)prm.n_qtiles * batch * num_kv_heads;
  if (blocks > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "pa_prefill: grid of %lld workgroups too large", (long long)blocks);
  const bool aligned = page_size % kTileN == 0;
  if (prm.soft_cap > 0.f) {
    if (aligned) prefill_kernel<true, true><<<dim3((unsigned)blocks), dim3(kThreads), 0, s>>>(prm);
    else prefill_kernel<true, false><<<dim3((unsigned)blocks), dim3(kThreads), 0, s>>>(prm);
  } else {
    if (aligned) prefill_kernel<false, true><<<dim3((unsigned)blocks), dim3(kThreads), 0, s>>>(prm);
    else prefill_kernel<false, false><<<dim3((unsigned)blocks), dim3(kThreads), 0, s>>>(prm);
  }
  return launch_status("pa_prefill");
}
