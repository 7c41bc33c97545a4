// QK RMSNorm + RoPE + KV store for gfx950: the layer step between the q/k/v
// projections and attention (vllm/model/qwen3.py:286-299), in one pass over
// the new tokens.
//
// One wavefront per token.  Lane p first evaluates the rotation of pair p
// (d/2 = 64 pairs) for the token's position; then the wave walks the token's
// H + 2*Hkv rows four at a time, one row per 16-lane group, each lane owning
// 8 contiguous elements (4 rotation pairs) of the row:
//   q row:  RMSNorm (16-lane sum of squares), scale, RoPE -> q_out
//   k row:  RMSNorm, scale, RoPE -> k_cache[slot]
//   v row:  copy -> v_cache[slot]
// Every byte of q, k and v is read once and every output byte written once.
//
// Numerics follow the reference's bf16 evaluation: positions and
// inv_freq are bf16 values, freqs = bf16(pos * inv_freq), cos/sin are
// evaluated in float32 and rounded to bf16; the normalised row is rounded to
// bf16 before the rotation, which is evaluated in float32 and rounded once.
#include <cmath>
#include <cstring>

#include "pa_common.h"
#include "pa_errors.h"

namespace pa {

constexpr int kRopeDim = 128;
constexpr int kRopePairs = kRopeDim / 2;

struct RopeParams {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const uint16_t* k;
  int64_t k_ts, k_hs;
  const uint16_t* v;
  int64_t v_ts, v_hs;
  const uint16_t* q_w;
  const uint16_t* k_w;
  const int32_t* positions;
  const int32_t* slots;
  uint16_t* q_out;
  int64_t qo_ts, qo_hs;
  uint16_t* k_cache;
  uint16_t* v_cache;
  int64_t num_slots;
  int32_t page_size;
  int64_t page_stride, slot_stride, head_stride;
  int32_t num_tokens, num_heads, num_kv_heads;
  float eps;
  float pos_div;  // linear / dynamic rope scaling factor (positions / factor)
  int32_t scale_pos;
  uint32_t inv_freq[kRopePairs / 2];  // bf16 pairs: pair 2i in the low half
};

__device__ __forceinline__ float round_bf16f(float x) {
  const f32x2 v = {x, 0.f};
  return bf16_lo(__builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2)));
}

// q, k and v are read exactly once: non-temporal loads keep them from
// displacing lines other work still needs.
__device__ __forceinline__ u32x4 ld16_stream(const uint16_t* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}

template <bool kNtStore>
__device__ __forceinline__ void st16_stream(uint16_t* p, const u32x4& v) {
  if constexpr (kNtStore)
    __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p));
  else
    st16(p, v);
}

// kRowsInFlight: each lane has loads of that many rows outstanding (the wave
// 4x as many) before it computes on the first one.  Measured on the Qwen3-32B
// shape (80 rows a token) 4 rows with non-temporal stores streams fastest;
// for 32 rows a token 2 rows with plain stores does.
template <int kRowsInFlight, bool kNtStore>
__global__ void __launch_bounds__(256)
qk_norm_rope_store_kernel(RopeParams p) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= p.num_tokens) return;
  const int i16 = lane & 15;
  const int g = lane >> 4;
  const int nq = p.num_heads;
  const int nqk = p.num_heads + p.num_kv_heads;
  const int rows = nqk + p.num_kv_heads;

  // row r of this token: q heads, then k heads, then v heads
  auto row_src = [&](int r) -> const uint16_t* {
    if (r < nq) return p.q + t * p.q_ts + r * p.q_hs;
    if (r < nqk) return p.k + t * p.k_ts + (r - nq) * p.k_hs;
    return p.v + t * p.v_ts + (r - nqk) * p.v_hs;
  };

  // first batch of rows in flight before the rotation is evaluated
  u32x4 x[kRowsInFlight];
#pragma unroll
  for (int u = 0; u < kRowsInFlight; ++u) {
    const int r = 4 * u + g;
    if (r < rows) x[u] = ld16_stream(row_src(r) + 8 * i16);
  }

  // ---- rotation of pair `lane` for this token
  float pos = (float)p.positions[t];
  if (p.scale_pos) pos = pos / p.pos_div;
  pos = round_bf16f(pos);
  const uint32_t fw = p.inv_freq[lane >> 1];
  const float inv = (lane & 1) ? bf16_hi(fw) : bf16_lo(fw);
  const float f = round_bf16f(pos * inv);
  const float cs_own = round_bf16f(cosf(f));
  const float sn_own = round_bf16f(sinf(f));
  // lane (g, i) rotates pairs 4i .. 4i+3 of its row
  float cs[4], sn[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    cs[j] = __shfl(cs_own, 4 * i16 + j);
    sn[j] = __shfl(sn_own, 4 * i16 + j);
  }
  const u32x4 wq = ld16(p.q_w + 8 * i16);
  const u32x4 wk = ld16(p.k_w + 8 * i16);

  const int64_t slot = p.slots[t];
  const bool store_kv = slot >= 0 && slot < p.num_slots;
  int64_t cache_off = 0;
  if (store_kv) {
    const int64_t pg = slot / p.page_size;
    cache_off = pg * p.page_stride + (slot - pg * p.page_size) * p.slot_stride;
  }

  for (int r0 = 0; r0 < rows; r0 += 4 * kRowsInFlight) {
    u32x4 nx[kRowsInFlight];
    const int r1 = r0 + 4 * kRowsInFlight;
    // next batch in flight while this one is computed
#pragma unroll
    for (int u = 0; u < kRowsInFlight; ++u) {
      const int r = r1 + 4 * u + g;
      if (r < rows) nx[u] = ld16_stream(row_src(r) + 8 * i16);
    }
#pragma unroll
    for (int u = 0; u < kRowsInFlight; ++u) {
      const int r = r0 + 4 * u + g;
      if (r >= rows) break;  // whole 16-lane group
      if (r >= nqk) {
        if (store_kv) st16_stream<kNtStore>(p.v_cache + cache_off + (r - nqk) * p.head_stride + 8 * i16, x[u]);
        continue;
      }
      float xv[8];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        xv[2 * e] = bf16_lo(x[u][e]);
        xv[2 * e + 1] = bf16_hi(x[u][e]);
      }
      float ss = 0.f;
#pragma unroll
      for (int e = 0; e < 8; ++e) ss = __builtin_fmaf(xv[e], xv[e], ss);
      ss += __shfl_xor(ss, 1, 16);
      ss += __shfl_xor(ss, 2, 16);
      ss += __shfl_xor(ss, 4, 16);
      ss += __shfl_xor(ss, 8, 16);
      const float rs = 1.f / sqrtf(ss * (1.f / kRopeDim) + p.eps);
      const u32x4 w = r < nq ? wq : wk;
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        // RMSNorm output, rounded to bf16 as the reference stores it
        const float y1 = round_bf16f(xv[2 * e] * (rs * bf16_lo(w[e])));
        const float y2 = round_bf16f(xv[2 * e + 1] * (rs * bf16_hi(w[e])));
        o[e] = pack_bf16x2(y1 * cs[e] - y2 * sn[e], y1 * sn[e] + y2 * cs[e]);
      }
      if (r < nq) {
        st16_stream<kNtStore>(p.q_out + t * p.qo_ts + r * p.qo_hs + 8 * i16, o);
      } else if (store_kv) {
        st16_stream<kNtStore>(p.k_cache + cache_off + (r - nq) * p.head_stride + 8 * i16, o);
      }
    }
#pragma unroll
    for (int u = 0; u < kRowsInFlight; ++u) x[u] = nx[u];
  }
}

// bf16 value of x (round to nearest even), as float
static float host_round_bf16(float x) {
  uint32_t u;
  memcpy(&u, &x, 4);
  if ((u & 0x7f800000u) == 0x7f800000u) return x;
  u = (u + 0x7fffu + ((u >> 16) & 1u)) & 0xffff0000u;
  float r;
  memcpy(&r, &u, 4);
  return r;
}

}  // namespace pa

using namespace pa;

extern "C" int pa_qk_norm_rope_store(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                                     const uint16_t* k, int64_t k_tok_stride, int64_t k_head_stride,
                                     const uint16_t* v, int64_t v_tok_stride, int64_t v_head_stride,
                                     const uint16_t* q_norm_weight, const uint16_t* k_norm_weight,
                                     float eps, float rope_theta, float rope_scaling_factor,
                                     const int32_t* positions, const int32_t* slot_mapping,
                                     int32_t num_tokens, int32_t num_heads, int32_t num_kv_heads,
                                     int32_t head_dim,
                                     uint16_t* q_out, int64_t q_out_tok_stride, int64_t q_out_head_stride,
                                     uint16_t* k_cache, uint16_t* v_cache,
                                     int32_t num_pages, int32_t page_size,
                                     int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                                     void* stream) {
  if (num_tokens < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_pages <= 0 || page_size <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_qk_norm_rope_store: bad sizes (num_tokens=%d, num_heads=%d, num_kv_heads=%d, num_pages=%d, "
                "page_size=%d)",
                num_tokens, num_heads, num_kv_heads, num_pages, page_size);
  if (head_dim != kRopeDim)
    return fail(PA_ERR_UNSUPPORTED, "pa_qk_norm_rope_store: head_dim %d not supported (only %d)", head_dim,
                kRopeDim);
  if (!(rope_theta > 0.f) || !(rope_scaling_factor > 0.f) || !(eps >= 0.f))
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_qk_norm_rope_store: bad rope_theta/scaling factor/eps");
  if (num_tokens == 0) return PA_OK;
  if (!q || !k || !v || !q_norm_weight || !k_norm_weight || !positions || !slot_mapping || !q_out || !k_cache ||
      !v_cache)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_qk_norm_rope_store: null pointer");
  const uintptr_t align = (uintptr_t)q | (uintptr_t)k | (uintptr_t)v | (uintptr_t)q_norm_weight |
                          (uintptr_t)k_norm_weight | (uintptr_t)q_out | (uintptr_t)k_cache | (uintptr_t)v_cache;
  if ((align & 15u) || (q_tok_stride | q_head_stride | k_tok_stride | k_head_stride | v_tok_stride | v_head_stride |
                        q_out_tok_stride | q_out_head_stride | page_stride | slot_stride | head_stride) % 8)
    return fail(PA_ERR_UNSUPPORTED,
                "pa_qk_norm_rope_store: operands must be 16-byte aligned with strides multiple of 8");

  RopeParams prm;
  prm.q = q;
  prm.q_ts = q_tok_stride;
  prm.q_hs = q_head_stride;
  prm.k = k;
  prm.k_ts = k_tok_stride;
  prm.k_hs = k_head_stride;
  prm.v = v;
  prm.v_ts = v_tok_stride;
  prm.v_hs = v_head_stride;
  prm.q_w = q_norm_weight;
  prm.k_w = k_norm_weight;
  prm.positions = positions;
  prm.slots = slot_mapping;
  prm.q_out = q_out;
  prm.qo_ts = q_out_tok_stride;
  prm.qo_hs = q_out_head_stride;
  prm.k_cache = k_cache;
  prm.v_cache = v_cache;
  prm.num_slots = (int64_t)num_pages * page_size;
  prm.page_size = page_size;
  prm.page_stride = page_stride;
  prm.slot_stride = slot_stride;
  prm.head_stride = head_stride;
  prm.num_tokens = num_tokens;
  prm.num_heads = num_heads;
  prm.num_kv_heads = num_kv_heads;
  prm.eps = eps;
  prm.scale_pos = rope_scaling_factor != 1.f;
  prm.pos_div = rope_scaling_factor;
  // inv_freq = 1 / theta ** (arange(0, d, 2) / d) with bf16 operands and
  // results (qwen3.py:62-63): theta, the exponent, the power and the
  // reciprocal are each rounded to bf16.
  const float theta = host_round_bf16(rope_theta);
  for (int i = 0; i < kRopePairs / 2; ++i) {
    uint32_t w = 0;
    for (int h = 0; h < 2; ++h) {
      const float e = host_round_bf16((float)(2 * (2 * i + h)) / (float)head_dim);
      const float pw = host_round_bf16(powf(theta, e));
      const float inv = host_round_bf16(1.f / pw);
      uint32_t u;
      memcpy(&u, &inv, 4);
      w |= (u >> 16) << (16 * h);
    }
    prm.inv_freq[i] = w;
  }
  const int64_t blocks = ((int64_t)num_tokens + 3) / 4;
  if (num_heads + 2 * num_kv_heads >= 64)
    qk_norm_rope_store_kernel<4, true><<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(prm);
  else
    qk_norm_rope_store_kernel<2, false><<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(prm);
  return launch_status("pa_qk_norm_rope_store");
}
