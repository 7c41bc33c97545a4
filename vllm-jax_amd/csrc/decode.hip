// Split-K paged GQA decode for gfx950.
//
// Work item = (sequence b, kv head, chunk of kDecodeChunk = 1024 context tokens),
// one wavefront per item, four independent items per 256-thread workgroup.
// Each wave streams its chunk 32 tokens at a time straight from HBM into
// registers (no LDS):
//
//   S^T[t][q] = K[t][:] . Q[q][:]          two v_mfma_f32_16x16x32_bf16 tiles
//                                           (16 tokens x 16 q columns, K = d)
//   online softmax per q column (lane-local after two permlane swaps)
//   O^T[d][q] += V^T[d][t] . P^T[t][q]      eight 16x16x32 MFMAs (d = 128)
//
// Keeping the q heads of one kv head in the N dimension makes the softmax row
// of a lane equal to its accumulator column, so rescaling O needs no lane
// exchange.  V is loaded as 16-byte row pieces (each 16-lane group reads one
// whole 256-byte token row per instruction) and transposed in registers with
// v_perm_b32 into the MFMA A layout.  The M (d) dimension of the PV MFMA is
// permuted so that M-tile j row m holds d = 8m + j: a lane then owns the 8
// contiguous d values of its 16-byte load.
//
// Partials (unnormalised o, running max in log2 units, running sum) go to a
// caller-owned f32 workspace; decode_merge_kernel combines the chunks of a
// sequence with the log-sum-exp rule of decode_paged_attention.py:274-282.
#include "pa_common.h"
#include "pa_errors.h"

namespace pa {

constexpr int kHeadDim = 128;
constexpr int kDecodeChunk = 1024;  // tokens per work item
constexpr int kDecodeStep = 32;    // tokens per inner iteration
constexpr int kDecodeWaves = 4;    // items per workgroup

struct DecodeParams {
  const uint16_t* q;
  int64_t q_bs, q_hs;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int32_t num_pages, page_size;
  int64_t page_stride, slot_stride, head_stride;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t pages_per_seq;
  const int32_t* lengths;
  int32_t batch, num_heads, num_kv_heads, group;
  int32_t n_chunks;
  float logit_scale;  // scale * log2(e) when soft_cap is off, else scale
  float soft_cap;     // <= 0: off
  float* ws_o;        // [batch, Hkv, n_chunks, group, d]
  float* ws_ml;       // [batch, Hkv, n_chunks, group, 2] (max log2, sum)
};

// V rows are read exactly once and in whole 256-byte rows: stream them past
// the caches.  K rows are read 64 bytes per row per instruction, so their
// 128-byte lines are kept cacheable for the instruction that reads the rest.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

// Offset of token `t` of a sequence in the pool (without the head offset).
__device__ __forceinline__ int64_t token_offset(const DecodeParams& p, const int32_t* bt_row, int t) {
  const int lp = t / p.page_size;
  const int32_t page = safe_page(bt_row, lp, p.num_pages);
  return (int64_t)page * p.page_stride + (int64_t)(t - lp * p.page_size) * p.slot_stride;
}

__device__ __forceinline__ uint32_t perm_lo(uint32_t a, uint32_t b) {
  // (a.lo16) | (b.lo16 << 16)
  return __builtin_amdgcn_perm(b, a, 0x05040100u);
}
__device__ __forceinline__ uint32_t perm_hi(uint32_t a, uint32_t b) {
  // (a.hi16) | (b.hi16 << 16)
  return __builtin_amdgcn_perm(b, a, 0x07060302u);
}

template <bool kAligned>
__global__ void __launch_bounds__(256)
decode_split_kernel(DecodeParams p) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t item = (int64_t)blockIdx.x * kDecodeWaves + wave;
  const int hkv = p.num_kv_heads;
  const int64_t n_items = (int64_t)p.batch * p.n_chunks * hkv;
  if (item >= n_items) return;
  const int kvh = (int)(item % hkv);
  const int64_t rest = item / hkv;
  const int chunk = (int)(rest % p.n_chunks);
  const int b = (int)(rest / p.n_chunks);
  // lengths past the block table's span are clamped to it (no read beyond the table row)
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  const int t_begin = chunk * kDecodeChunk;
  if (t_begin >= len) return;
  const int t_end = min(t_begin + kDecodeChunk, len);

  const int n = lane & 15;   // q column of S/O; also the d-chunk of V loads
  const int g = lane >> 4;   // k group
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int64_t head_off = (int64_t)kvh * p.head_stride;

  // Q^T operand: k-step s uses d chunk (4s + g) for both Q and K.
  bf16x8 qt[4];
  {
    const bool live = n < p.group;
    const uint16_t* qrow = p.q + (int64_t)b * p.q_bs + (int64_t)(kvh * p.group + (live ? n : 0)) * p.q_hs;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 v = live ? ld16(qrow + 8 * (4 * s + g)) : u32x4{0, 0, 0, 0};
      qt[s] = as_bf16x8(v);
    }
  }

  f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f;  // finite so that exp2(x - m) never sees inf - inf
  float l_run = 0.f;

  // Token of V k-slot i of this lane's group within a 32-token step.
  auto vtok = [&](int i) { return (i < 4 ? 4 * g + i : 16 + 4 * g + (i - 4)); };

  u32x4 kreg[2][4], vreg[8];
  auto load_step = [&](int t0) {
    if constexpr (kAligned) {
      // A 32-token step never crosses a page; clamp tokens past the end onto
      // the last valid one (same page) so no stale or NaN data is read.
      const int lp = t0 / p.page_size;
      const int32_t page = safe_page(bt_row, lp, p.num_pages);
      const int64_t pbase = (int64_t)page * p.page_stride + head_off;
      const int pstart = lp * p.page_size;
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        const int t = min(t0 + 16 * tile + n, len - 1);
        const uint16_t* row = p.k_cache + pbase + (int64_t)(t - pstart) * p.slot_stride;
#pragma unroll
        for (int s = 0; s < 4; ++s) kreg[tile][s] = ld16(row + 8 * (4 * s + g));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int t = min(t0 + vtok(i), len - 1);
        vreg[i] = ld16_stream(p.v_cache + pbase + (int64_t)(t - pstart) * p.slot_stride + 8 * n);
      }
    } else {
#pragma unroll
      for (int tile = 0; tile < 2; ++tile) {
        const int t = min(t0 + 16 * tile + n, len - 1);
        const uint16_t* row = p.k_cache + token_offset(p, bt_row, t) + head_off;
#pragma unroll
        for (int s = 0; s < 4; ++s) kreg[tile][s] = ld16(row + 8 * (4 * s + g));
      }
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int t = min(t0 + vtok(i), len - 1);
        vreg[i] = ld16_stream(p.v_cache + token_offset(p, bt_row, t) + head_off + 8 * n);
      }
    }
  };

  load_step(t_begin);
  for (int t0 = t_begin; t0 < t_end; t0 += kDecodeStep) {
    u32x4 kc[2][4], vc[8];
#pragma unroll
    for (int tile = 0; tile < 2; ++tile)
#pragma unroll
      for (int s = 0; s < 4; ++s) kc[tile][s] = kreg[tile][s];
#pragma unroll
    for (int i = 0; i < 8; ++i) vc[i] = vreg[i];
    if (t0 + kDecodeStep < t_end) load_step(t0 + kDecodeStep);

    // ---- S^T = K . Q^T for tokens t0..t0+15 (sa) and t0+16..t0+31 (sb)
    f32x4 sa = {0.f, 0.f, 0.f, 0.f}, sb = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      sa = mfma16(as_bf16x8(kc[0][s]), qt[s], sa);
      sb = mfma16(as_bf16x8(kc[1][s]), qt[s], sb);
    }
    // lane holds S[q = n][token t0 + 4g + i] (sa) and [t0 + 16 + 4g + i] (sb)
    float x[8];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      x[i] = sa[i];
      x[4 + i] = sb[i];
    }
    float mx = -INFINITY;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      float v = x[i];
      if (p.soft_cap > 0.f) v = p.soft_cap * tanhf(v * p.logit_scale / p.soft_cap) * kLog2e;
      else v = v * p.logit_scale;
      const int t = t0 + vtok(i);
      v = t < len ? v : -INFINITY;
      x[i] = v;
      mx = fmaxf(mx, v);
    }
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    const float m_new = fmaxf(m_run, mx);
    const float corr = fast_exp2(m_run - m_new);
    m_run = m_new;
    float psum = 0.f;
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      x[i] = fast_exp2(x[i] - m_new);
      psum += x[i];
    }
    l_run = l_run * corr + psum;
    u32x4 pw;
    pw[0] = pack_bf16x2(x[0], x[1]);
    pw[1] = pack_bf16x2(x[2], x[3]);
    pw[2] = pack_bf16x2(x[4], x[5]);
    pw[3] = pack_bf16x2(x[6], x[7]);
    const bf16x8 pt = as_bf16x8(pw);

    // ---- transpose V pieces into the A layout of the 8 d-tiles
#pragma unroll
    for (int q2 = 0; q2 < 4; ++q2) {
      u32x4 lo, hi;
#pragma unroll
      for (int pp = 0; pp < 4; ++pp) {
        lo[pp] = perm_lo(vc[2 * pp][q2], vc[2 * pp + 1][q2]);
        hi[pp] = perm_hi(vc[2 * pp][q2], vc[2 * pp + 1][q2]);
      }
      acc[2 * q2] = acc[2 * q2] * corr;
      acc[2 * q2 + 1] = acc[2 * q2 + 1] * corr;
      acc[2 * q2] = mfma16(as_bf16x8(lo), pt, acc[2 * q2]);
      acc[2 * q2 + 1] = mfma16(as_bf16x8(hi), pt, acc[2 * q2 + 1]);
    }
  }

  l_run = sum_xor16(l_run);
  l_run = sum_xor32(l_run);

  if (n < p.group) {
    const int64_t part = (((int64_t)b * hkv + kvh) * p.n_chunks + chunk) * p.group + n;
    float* dst = p.ws_o + part * kHeadDim + 32 * g;
    // acc[j][r] = O^T[d = 32g + 8r + j][q = n]
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      f32x4 lo = {acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
      f32x4 hi = {acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
      *reinterpret_cast<f32x4*>(dst + 8 * r) = lo;
      *reinterpret_cast<f32x4*>(dst + 8 * r + 4) = hi;
    }
    if (g == 0) {
      p.ws_ml[2 * part] = m_run;
      p.ws_ml[2 * part + 1] = l_run;
    }
  }
}

// One wave per (sequence, q head): out = sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M).
__global__ void __launch_bounds__(256)
decode_merge_kernel(DecodeParams p, uint16_t* __restrict__ out, int64_t out_bs, int64_t out_hs) {
  const int lane = threadIdx.x & 63;
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= (int64_t)p.batch * p.num_heads) return;
  const int b = (int)(pair / p.num_heads);
  const int h = (int)(pair - (int64_t)b * p.num_heads);
  const int kvh = h / p.group;
  const int qi = h - kvh * p.group;
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  const int nc = len > 0 ? min((len + kDecodeChunk - 1) / kDecodeChunk, p.n_chunks) : 0;
  const int64_t base = ((int64_t)b * p.num_kv_heads + kvh) * p.n_chunks;
  float mmax = -INFINITY;
  for (int c = 0; c < nc; ++c) mmax = fmaxf(mmax, p.ws_ml[2 * ((base + c) * p.group + qi)]);
  float o0 = 0.f, o1 = 0.f, lsum = 0.f;
  for (int c = 0; c < nc; ++c) {
    const int64_t part = (base + c) * p.group + qi;
    const float w = fast_exp2(p.ws_ml[2 * part] - mmax);
    lsum += p.ws_ml[2 * part + 1] * w;
    const float2 o = *reinterpret_cast<const float2*>(p.ws_o + part * kHeadDim + 2 * lane);
    o0 += o.x * w;
    o1 += o.y * w;
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint32_t* dst = reinterpret_cast<uint32_t*>(out + (int64_t)b * out_bs + (int64_t)h * out_hs) + lane;
  *dst = pack_bf16x2(o0 * inv, o1 * inv);
}

static int decode_chunks(int32_t pages_per_seq, int32_t page_size) {
  const int64_t max_tokens = (int64_t)pages_per_seq * page_size;
  return (int)((max_tokens + kDecodeChunk - 1) / kDecodeChunk);
}

}  // namespace pa

using namespace pa;

extern "C" size_t pa_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t head_dim,
                                           int32_t pages_per_seq, int32_t page_size) {
  if (batch <= 0 || num_heads <= 0 || head_dim <= 0 || pages_per_seq <= 0 || page_size <= 0) return 0;
  const size_t parts = (size_t)batch * num_heads * decode_chunks(pages_per_seq, page_size);
  return parts * ((size_t)head_dim + 2) * sizeof(float);
}

extern "C" int pa_decode(const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
                         const uint16_t* k_cache, const uint16_t* v_cache,
                         int32_t num_pages, int32_t page_size,
                         int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                         const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                         const int32_t* lengths, int32_t batch,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                         float scale, float soft_cap,
                         uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride,
                         void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_pages <= 0 || page_size <= 0 ||
      pages_per_seq < 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_decode: bad sizes (batch=%d, num_heads=%d, num_kv_heads=%d, num_pages=%d, "
                "page_size=%d, pages_per_seq=%d)",
                batch, num_heads, num_kv_heads, num_pages, page_size, pages_per_seq);
  if (num_heads % num_kv_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_decode: Number of Q heads must be divisible by number of KV heads. Got %d and %d.",
                num_heads, num_kv_heads);
  if (head_dim != kHeadDim)
    return fail(PA_ERR_UNSUPPORTED, "pa_decode: head_dim %d not supported (only %d)", head_dim, kHeadDim);
  const int group = num_heads / num_kv_heads;
  if (group > 16)
    return fail(PA_ERR_UNSUPPORTED, "pa_decode: %d q heads per kv head not supported (max 16)", group);
  if (batch == 0) return PA_OK;
  if (!q || !k_cache || !v_cache || !block_tables || !lengths || !out)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_decode: null pointer");
  const uintptr_t align_bits = (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out;
  if ((align_bits & 15u) || (q_batch_stride | q_head_stride | page_stride | slot_stride | head_stride) % 8 ||
      (out_batch_stride | out_head_stride) % 2)
    return fail(PA_ERR_UNSUPPORTED, "pa_decode: operands must be 16-byte aligned with strides multiple of 8");
  const size_t need = pa_decode_workspace_size(batch, num_heads, head_dim, pages_per_seq, page_size);
  if (pages_per_seq > 0 && (!workspace || workspace_bytes < need))
    return fail(PA_ERR_WORKSPACE, "pa_decode: workspace of %zu bytes needed, %zu given", need, workspace_bytes);

  DecodeParams prm;
  prm.q = q;
  prm.q_bs = q_batch_stride;
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
  prm.lengths = lengths;
  prm.batch = batch;
  prm.num_heads = num_heads;
  prm.num_kv_heads = num_kv_heads;
  prm.group = group;
  prm.n_chunks = pages_per_seq > 0 ? decode_chunks(pages_per_seq, page_size) : 0;
  prm.soft_cap = soft_cap > 0.f ? soft_cap : 0.f;
  prm.logit_scale = prm.soft_cap > 0.f ? scale : scale * kLog2e;
  const size_t parts = (size_t)batch * num_heads * prm.n_chunks;
  prm.ws_o = reinterpret_cast<float*>(workspace);
  prm.ws_ml = prm.ws_o + parts * head_dim;

  hipStream_t s = (hipStream_t)stream;
  const int64_t items = (int64_t)batch * prm.n_chunks * num_kv_heads;
  const int64_t blocks = (items + kDecodeWaves - 1) / kDecodeWaves;
  if (blocks > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "pa_decode: grid of %lld workgroups too large", (long long)blocks);
  if (blocks > 0) {  // no table pages: every row is zero, only the merge pass runs
    if (page_size % kDecodeStep == 0)
      decode_split_kernel<true><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(prm);
    else
      decode_split_kernel<false><<<dim3((unsigned)blocks), dim3(256), 0, s>>>(prm);
    int rc = launch_status("pa_decode(split)");
    if (rc) return rc;
  }
  const int64_t pairs = (int64_t)batch * num_heads;
  decode_merge_kernel<<<dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, s>>>(prm, out, out_batch_stride,
                                                                           out_head_stride);
  return launch_status("pa_decode(merge)");
}
