// Split-K paged GQA decode for gfx950.
//
// Workgroup = (sequence b, kv head, chunk of 2048 context tokens; 1024 when
// pages hold 16 tokens), four wavefronts.  The chunk is cut into 16-token steps dealt round-robin to
// the waves (wave w takes steps w, w+4, ...), so the four waves stream
// adjacent token rows and finish together.  Each wave keeps kDecodeBufs steps
// of K and V in flight in VGPRs: the loads of step i+kDecodeBufs are issued as
// soon as step i has been consumed, so HBM always sees several 8 KiB requests
// per wave.  Per step:
//
//   S^T[t][q] = K[t][:] . Q[q][:]          4 x v_mfma_f32_16x16x32_bf16
//                                           (16 tokens x 16 q columns, K = d)
//   online softmax per q column (lane-local after two permlane swaps; the
//   accumulator is rescaled only when the running max grows by more than
//   2^kDecodeSlack)
//   O^T[d][q] += V^T[d][t] . P^T[t][q]      8 x v_mfma_f32_16x16x16_bf16
//
// The q heads of one kv head sit in the N dimension, so the softmax row of a
// lane is its accumulator column.  K is read as 64-byte row pieces in the MFMA
// A layout; V as 16-byte pieces where each 16-lane group reads one whole
// 256-byte token row, transposed in registers with v_perm_b32.  The M (d)
// dimension of the PV MFMA is permuted so that M-tile j row m holds
// d = 8m + j: a lane then owns the 8 contiguous d values of its V load.
//
// Workgroups are dealt round-robin to the 8 XCDs; the grid is renumbered so
// that each XCD runs a contiguous range of (sequence, chunk, kv head) items.
// The kv heads of one token row (adjacent in the pool) are then read by one
// XCD at nearly the same time, which keeps HBM accesses close together:
// measured 6.07 TB/s against 5.36 TB/s with the heads spread over all XCDs.
//
// The four waves combine (m, l, o) through LDS.  A sequence covered by one
// chunk is finished right there; longer sequences leave one f32 partial per
// chunk in the caller's workspace and decode_merge_kernel combines them with
// the log-sum-exp rule of decode_paged_attention.py:274-282.
#include "pa_common.h"
#include "pa_errors.h"

namespace pa {

constexpr int kHeadDim = 128;
constexpr int kDecodeStep = 16;     // tokens per wave step
constexpr int kDecodeWaves = 4;     // waves per workgroup
#ifndef PA_DECODE_BUFS
#define PA_DECODE_BUFS 4
#endif
constexpr int kDecodeBufs = PA_DECODE_BUFS;  // steps in flight per wave
constexpr float kDecodeSlack = 8.f;          // lazy-rescale threshold (log2 units)

typedef __attribute__((__vector_size__(4 * sizeof(__bf16)))) __bf16 bf16x4v;

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
  int32_t chunk;     // tokens per workgroup
  int32_t n_chunks;  // chunks of the widest block-table row
  float logit_scale;  // scale * log2(e) when soft_cap is off, else scale
  float soft_cap;     // <= 0: off
  float* ws_o;        // [batch, Hkv, n_chunks, group, d]
  float* ws_ml;       // [batch, Hkv, n_chunks, group, 2] (max log2, sum)
  uint16_t* out;
  int64_t out_bs, out_hs;
};

// V rows are read exactly once and as whole 256-byte rows: stream them past
// the caches.  K rows are read 64 bytes per row per instruction, so their
// 128-byte lines stay cacheable for the instruction that reads the other half.
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

__device__ __forceinline__ f32x4 mfma16k16(const bf16x4v& a, const bf16x4v& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// The bf16 halves selected by `hi` of a and b, packed as (a_half, b_half).
__device__ __forceinline__ uint32_t pick2(uint32_t a, uint32_t b, bool hi) {
  return hi ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
}

struct alignas(16) DecodeLds {
  float o[kDecodeWaves][16][kHeadDim];
  float m[kDecodeWaves][16];
  float l[kDecodeWaves][16];
};

// Tokens per workgroup: the aligned path keeps the chunk's page ids in one
// VGPR (one per lane), so a chunk spans at most 64 pages.
__host__ __device__ inline int decode_chunk_tokens(int page_size) { return page_size >= 32 ? 2048 : 1024; }

// kAligned: page_size % 16 == 0, so a 16-token step never crosses a page and
// the chunk's page ids (at most 64) are read once, one per lane.
template <bool kAligned, bool kSoftCap>
__global__ void __launch_bounds__(256, 2)
decode_split_kernel(DecodeParams p) {
  __shared__ DecodeLds red;
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hkv = p.num_kv_heads;
  // XCD x = blockIdx % 8 serves items [x*q8 + min(x, r8), ...) in order
  int item;
  {
    const int nb = gridDim.x, x = blockIdx.x & 7, k = blockIdx.x >> 3;
    const int q8 = nb >> 3, r8 = nb & 7;
    item = x * q8 + min(x, r8) + k;  // a bijection of [0, nb)
  }
  const int kvh = item % hkv;
  const int rest = item / hkv;
  const int chunk = rest % p.n_chunks;
  const int b = rest / p.n_chunks;
  // lengths past the block table's span are clamped to it (no read beyond the table row)
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  const int t_begin = chunk * p.chunk;
  if (t_begin >= len) return;  // uniform over the workgroup
  const int t_end = min(t_begin + p.chunk, len);
  const int n_steps = (t_end - t_begin + kDecodeStep - 1) / kDecodeStep;
  const int my_steps = n_steps > wave ? (n_steps - wave + kDecodeWaves - 1) / kDecodeWaves : 0;
  const int n_chunks_b = (len + p.chunk - 1) / p.chunk;

  const int n = lane & 15;  // q column of S/O; the d chunk of V loads; the token of K loads
  const int g = lane >> 4;  // 16-lane group
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int64_t head_off = (int64_t)kvh * p.head_stride;

  // Page ids of the chunk, one per lane (aligned path).
  const int lp_first = t_begin / p.page_size;
  int32_t my_page = 0;
  if constexpr (kAligned) {
    const int lp = lp_first + lane;
    if (lp < p.pages_per_seq) my_page = safe_page(bt_row, lp, p.num_pages);
  }

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

  u32x4 kb[kDecodeBufs][4], vb[kDecodeBufs][4];

  // Loads of wave step `ks` (tokens t0 .. t0+15) into one buffer.  Tokens past
  // the sequence end are clamped onto its last token (same page in the aligned
  // case), so no stale or NaN data reaches the accumulator.  A step past the
  // wave's last one still issues its 8 loads, all of the first 256 bytes of q
  // (cache hits): every buffer then sees the same number of loads issued
  // after it, and the compiler waits for exactly the buffer being consumed.
  auto issue = [&](u32x4 (&kd)[4], u32x4 (&vd)[4], int ks) __attribute__((always_inline)) {
    const bool valid = ks < my_steps;  // uniform
    const int t0 = t_begin + kDecodeStep * (kDecodeWaves * ks + wave);
    const int lim = len - 1 - t0;  // >= 0 when valid
    if constexpr (kAligned) {
      const uint16_t* kbase = p.q;
      const uint16_t* vbase = p.q;
      int64_t rs = 0;
      if (valid) {
        const int lp = t0 / p.page_size;
        const int32_t page = __builtin_amdgcn_readlane(my_page, lp - lp_first);
        const int64_t base = (int64_t)page * p.page_stride +
                             (int64_t)(t0 - lp * p.page_size) * p.slot_stride + head_off;
        kbase = p.k_cache + base;
        vbase = p.v_cache + base;
        rs = p.slot_stride;
      }
      const int64_t krow = (int64_t)min(n, lim) * rs;
#pragma unroll
      for (int s = 0; s < 4; ++s) kd[s] = ld16(kbase + krow + 8 * (4 * s + g));
#pragma unroll
      for (int i = 0; i < 4; ++i) vd[i] = ld16_stream(vbase + (int64_t)min(4 * g + i, lim) * rs + 8 * n);
    } else {
      if (!valid) {
#pragma unroll
        for (int s = 0; s < 4; ++s) kd[s] = ld16(p.q + 8 * (4 * s + g));
#pragma unroll
        for (int i = 0; i < 4; ++i) vd[i] = ld16_stream(p.q + 8 * n);
        return;
      }
      auto tok_off = [&](int t) {
        const int lp = t / p.page_size;
        const int32_t page = safe_page(bt_row, lp, p.num_pages);
        return (int64_t)page * p.page_stride + (int64_t)(t - lp * p.page_size) * p.slot_stride + head_off;
      };
      const uint16_t* krow = p.k_cache + tok_off(t0 + min(n, lim));
#pragma unroll
      for (int s = 0; s < 4; ++s) kd[s] = ld16(krow + 8 * (4 * s + g));
#pragma unroll
      for (int i = 0; i < 4; ++i) vd[i] = ld16_stream(p.v_cache + tok_off(t0 + min(4 * g + i, lim)) + 8 * n);
    }
  };

  auto consume = [&](const u32x4 (&kd)[4], const u32x4 (&vd)[4], int ks) __attribute__((always_inline)) {
    const int t0 = t_begin + kDecodeStep * (kDecodeWaves * ks + wave);
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int s = 0; s < 4; ++s) sc = mfma16(as_bf16x8(kd[s]), qt[s], sc);
    // lane holds S[q = n][token t0 + 4g + r]
    float x[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = sc[r];
      if constexpr (kSoftCap) v = p.soft_cap * tanhf(v * p.logit_scale / p.soft_cap) * kLog2e;
      else v = v * p.logit_scale;
      v = t0 + 4 * g + r < len ? v : -INFINITY;
      x[r] = v;
      mx = fmaxf(mx, v);
    }
    mx = max_xor16(mx);
    mx = max_xor32(mx);
    if (__builtin_amdgcn_ballot_w64(mx > m_run + kDecodeSlack)) {
      const float m_new = fmaxf(m_run, mx);
      const float corr = fast_exp2(m_run - m_new);
      m_run = m_new;
      l_run *= corr;
#pragma unroll
      for (int j = 0; j < 8; ++j) acc[j] = acc[j] * corr;
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      x[r] = fast_exp2(x[r] - m_run);
      l_run += x[r];
    }
    u32x2 pw;
    pw[0] = pack_bf16x2(x[0], x[1]);
    pw[1] = pack_bf16x2(x[2], x[3]);
    const bf16x4v pt = __builtin_bit_cast(bf16x4v, pw);
    // V^T tile j: lane (n, g) supplies d = 8n + j of tokens 4g .. 4g+3
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      u32x2 a;
      a[0] = pick2(vd[0][j >> 1], vd[1][j >> 1], j & 1);
      a[1] = pick2(vd[2][j >> 1], vd[3][j >> 1], j & 1);
      acc[j] = mfma16k16(__builtin_bit_cast(bf16x4v, a), pt, acc[j]);
    }
  };

#pragma unroll
  for (int j = 0; j < kDecodeBufs; ++j) issue(kb[j], vb[j], j);
  for (int k0 = 0; k0 < my_steps; k0 += kDecodeBufs) {
#pragma unroll
    for (int j = 0; j < kDecodeBufs; ++j) {
      const int ks = k0 + j;
      if (ks < my_steps) consume(kb[j], vb[j], ks);
      issue(kb[j], vb[j], ks + kDecodeBufs);
    }
  }

  // ---- combine the four waves through LDS
  l_run = sum_xor16(l_run);
  l_run = sum_xor32(l_run);
  // acc[j][r] = O^T[d = 8 * (4g + r) + j][q = n]
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float* dst = &red.o[wave][n][32 * g + 8 * r];
    *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
  }
  if (g == 0) {
    red.m[wave][n] = m_run;
    red.l[wave][n] = l_run;
  }
  __syncthreads();
  // wave w finishes d = 32w + 8g .. +7 of column n
  float mm = red.m[0][n];
#pragma unroll
  for (int w = 1; w < kDecodeWaves; ++w) mm = fmaxf(mm, red.m[w][n]);
  float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  float ll = 0.f;
  const int d0 = 32 * wave + 8 * g;
#pragma unroll
  for (int w = 0; w < kDecodeWaves; ++w) {
    const float sw = fast_exp2(red.m[w][n] - mm);
    ll += sw * red.l[w][n];
    const f32x4 a = *reinterpret_cast<const f32x4*>(&red.o[w][n][d0]);
    const f32x4 c = *reinterpret_cast<const f32x4*>(&red.o[w][n][d0 + 4]);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      o[i] += sw * a[i];
      o[4 + i] += sw * c[i];
    }
  }
  if (n >= p.group) return;
  if (n_chunks_b == 1) {
    const float inv = 1.f / ll;  // ll >= 1: the chunk holds a visible token
    u32x4 w;
#pragma unroll
    for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(o[2 * i] * inv, o[2 * i + 1] * inv);
    st16(p.out + (int64_t)b * p.out_bs + (int64_t)(kvh * p.group + n) * p.out_hs + d0, w);
  } else {
    const int64_t part = (((int64_t)b * hkv + kvh) * p.n_chunks + chunk) * p.group + n;
    float* dst = p.ws_o + part * kHeadDim + d0;
    *reinterpret_cast<f32x4*>(dst) = f32x4{o[0], o[1], o[2], o[3]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{o[4], o[5], o[6], o[7]};
    if (wave == 0 && g == 0) {
      p.ws_ml[2 * part] = mm;
      p.ws_ml[2 * part + 1] = ll;
    }
  }
}

// One wave per (sequence, q head): out = sum_c o_c 2^(m_c - M) / sum_c l_c 2^(m_c - M).
// Sequences of one chunk were finished by the split kernel; length 0 gives zeros.
__global__ void __launch_bounds__(256)
decode_merge_kernel(DecodeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= (int64_t)p.batch * p.num_heads) return;
  const int b = (int)(pair / p.num_heads);
  const int h = (int)(pair - (int64_t)b * p.num_heads);
  const int kvh = h / p.group;
  const int qi = h - kvh * p.group;
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  const int nc = len > 0 ? min((len + p.chunk - 1) / p.chunk, p.n_chunks) : 0;
  if (nc == 1) return;
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
  uint32_t* dst = reinterpret_cast<uint32_t*>(p.out + (int64_t)b * p.out_bs + (int64_t)h * p.out_hs) + lane;
  *dst = pack_bf16x2(o0 * inv, o1 * inv);
}

static int decode_chunks(int32_t pages_per_seq, int32_t page_size) {
  const int64_t max_tokens = (int64_t)pages_per_seq * page_size;
  const int chunk = decode_chunk_tokens(page_size);
  return (int)((max_tokens + chunk - 1) / chunk);
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
      (out_batch_stride | out_head_stride) % 8)
    return fail(PA_ERR_UNSUPPORTED, "pa_decode: operands must be 16-byte aligned with strides multiple of 8");
  if ((int64_t)pages_per_seq * page_size > 0x7fffffffLL)
    return fail(PA_ERR_UNSUPPORTED, "pa_decode: block table spans more than 2^31 tokens");
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
  prm.chunk = decode_chunk_tokens(page_size);
  prm.n_chunks = pages_per_seq > 0 ? decode_chunks(pages_per_seq, page_size) : 0;
  prm.soft_cap = soft_cap > 0.f ? soft_cap : 0.f;
  prm.logit_scale = prm.soft_cap > 0.f ? scale : scale * kLog2e;
  const size_t parts = (size_t)batch * num_heads * prm.n_chunks;
  prm.ws_o = reinterpret_cast<float*>(workspace);
  prm.ws_ml = prm.ws_o + parts * head_dim;
  prm.out = out;
  prm.out_bs = out_batch_stride;
  prm.out_hs = out_head_stride;

  hipStream_t s = (hipStream_t)stream;
  const int64_t blocks = (int64_t)batch * prm.n_chunks * num_kv_heads;
  if (blocks > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "pa_decode: grid of %lld workgroups too large", (long long)blocks);
  if (blocks > 0) {  // no table pages: every row is zero, only the merge pass runs
    const bool aligned = page_size % kDecodeStep == 0;
    const dim3 grid((unsigned)blocks), block(64 * kDecodeWaves);
    if (aligned && prm.soft_cap == 0.f) decode_split_kernel<true, false><<<grid, block, 0, s>>>(prm);
    else if (aligned) decode_split_kernel<true, true><<<grid, block, 0, s>>>(prm);
    else if (prm.soft_cap == 0.f) decode_split_kernel<false, false><<<grid, block, 0, s>>>(prm);
    else decode_split_kernel<false, true><<<grid, block, 0, s>>>(prm);
    int rc = launch_status("pa_decode(split)");
    if (rc) return rc;
  }
  const int64_t pairs = (int64_t)batch * num_heads;
  decode_merge_kernel<<<dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, s>>>(prm);
  return launch_status("pa_decode(merge)");
}
