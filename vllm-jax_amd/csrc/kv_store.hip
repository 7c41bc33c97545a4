// KV-cache store (scatter of new tokens into pages) and block-table gather.
//
// Both are pure data movement bound by HBM: one thread moves one 16-byte
// chunk (8 bf16) of a token's [Hkv, d] row, so a wave moves 1 KiB of
// consecutive source bytes per instruction.
#include "pa_common.h"
#include "pa_errors.h"

namespace pa {

// k/v rows are [Hkv, d]; one token = Hkv*d/8 chunks of 16 bytes.
__global__ void __launch_bounds__(256)
kv_store_vec_kernel(const uint16_t* __restrict__ k, int64_t k_ts, int64_t k_hs,
                    const uint16_t* __restrict__ v, int64_t v_ts, int64_t v_hs,
                    const int32_t* __restrict__ slot_mapping, int32_t num_tokens,
                    int32_t chunks_per_head, int32_t chunks_per_token,
                    uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                    int64_t num_slots, int32_t page_size,
                    int64_t page_stride, int64_t slot_stride, int64_t head_stride) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t t = gid / chunks_per_token;
  if (t >= num_tokens) return;
  const int32_t c = (int32_t)(gid - t * chunks_per_token);
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;  // padding token or dropped slot
  const int32_t h = c / chunks_per_head;
  const int32_t e = (c - h * chunks_per_head) * 8;
  const int64_t page = slot / page_size;
  const int64_t dst = page * page_stride + (slot - page * page_size) * slot_stride + h * head_stride + e;
  const u32x4 kv = ld16(k + t * k_ts + h * k_hs + e);
  const u32x4 vv = ld16(v + t * v_ts + h * v_hs + e);
  st16(k_cache + dst, kv);
  st16(v_cache + dst, vv);
}

// Element-wise fallback for operands that are not 16-byte aligned.
__global__ void __launch_bounds__(256)
kv_store_scalar_kernel(const uint16_t* __restrict__ k, int64_t k_ts, int64_t k_hs,
                       const uint16_t* __restrict__ v, int64_t v_ts, int64_t v_hs,
                       const int32_t* __restrict__ slot_mapping, int32_t num_tokens,
                       int32_t head_dim, int32_t elems_per_token,
                       uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache,
                       int64_t num_slots, int32_t page_size,
                       int64_t page_stride, int64_t slot_stride, int64_t head_stride) {
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t t = gid / elems_per_token;
  if (t >= num_tokens) return;
  const int32_t c = (int32_t)(gid - t * elems_per_token);
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;
  const int32_t h = c / head_dim;
  const int32_t e = c - h * head_dim;
  const int64_t page = slot / page_size;
  const int64_t dst = page * page_stride + (slot - page * page_size) * slot_stride + h * head_stride + e;
  k_cache[dst] = k[t * k_ts + h * k_hs + e];
  v_cache[dst] = v[t * v_ts + h * v_hs + e];
}

// out[b, j] = cache[page(b, j / page_size), j % page_size] for j < len[b], else 0.
__global__ void __launch_bounds__(256)
gather_kv_kernel(const uint16_t* __restrict__ cache, int32_t num_pages, int32_t page_size,
                 int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                 const int32_t* __restrict__ block_tables, int64_t bt_stride, int32_t pages_per_seq,
                 const int32_t* __restrict__ lengths, int32_t batch,
                 int32_t head_dim, int32_t elems_per_token, uint16_t* __restrict__ out) {
  const int64_t tokens_per_seq = (int64_t)pages_per_seq * page_size;
  const int64_t gid = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  const int64_t row = gid / elems_per_token;  // b * tokens_per_seq + j
  if (row >= (int64_t)batch * tokens_per_seq) return;
  const int32_t c = (int32_t)(gid - row * elems_per_token);
  const int32_t b = (int32_t)(row / tokens_per_seq);
  const int32_t j = (int32_t)(row - (int64_t)b * tokens_per_seq);
  uint16_t val = 0;
  if (j < lengths[b]) {
    const int32_t page = safe_page(block_tables + (int64_t)b * bt_stride, j / page_size, num_pages);
    const int32_t h = c / head_dim;
    const int32_t e = c - h * head_dim;
    val = cache[(int64_t)page * page_stride + (int64_t)(j % page_size) * slot_stride + h * head_stride + e];
  }
  out[gid] = val;
}

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

// Quantising KV store: one kLanes-lane group per (token, kv head) row, 8
// values per lane (lanes past the row's cph = d / 8 chunks hold none; 16
// lanes up to d = 128, 32 up to 256).  amax over the row (butterfly); the stored
// scale is the smallest power of two s with amax / s <= 448 (at least
// 2^-126), and the codes are e4m3(x / s) with round-to-nearest-even
// (v_cvt_pk_fp8_f32), x / s exact; an all-zero row stores scale 1.  A power
// of two lets the readers widen a code with its scale in one exact
// conversion (v_cvt_scalef32_pk_bf16_fp8 scales by a power of two).  Codes
// go to the (page, slot, head) byte pool, scales to a [Hkv, NB, BS]-strided
// float pool.
template <int kLanes>
__global__ void __launch_bounds__(256)
kv_store_fp8_kernel(const uint16_t* __restrict__ k, int64_t k_ts, int64_t k_hs,
                    const uint16_t* __restrict__ v, int64_t v_ts, int64_t v_hs,
                    const int32_t* __restrict__ slot_mapping, int32_t num_tokens, int32_t num_kv_heads, int32_t cph,
                    uint8_t* __restrict__ k_cache, uint8_t* __restrict__ v_cache,
                    float* __restrict__ k_scales, float* __restrict__ v_scales,
                    int64_t num_slots, int32_t page_size,
                    int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                    int64_t sc_page_stride, int64_t sc_slot_stride, int64_t sc_head_stride) {
  static_assert(kLanes == 16 || kLanes == 32, "row group");
  const int64_t row = ((int64_t)blockIdx.x * blockDim.x + threadIdx.x) / kLanes;  // (token, head)
  const int i16 = threadIdx.x & (kLanes - 1);
  const int64_t t = row / num_kv_heads;
  if (t >= num_tokens) return;  // whole group
  const int h = (int)(row - t * num_kv_heads);
  const int64_t slot = slot_mapping[t];
  if (slot < 0 || slot >= num_slots) return;
  const int64_t page = slot / page_size;
  const int64_t off = slot - page * page_size;
  const bool has = i16 < cph;  // the lane holds a chunk of the row
  const int ci = has ? i16 : 0;
  const int64_t dst = page * page_stride + off * slot_stride + h * head_stride + 8 * ci;
  const int64_t sdst = page * sc_page_stride + off * sc_slot_stride + h * sc_head_stride;
#pragma unroll
  for (int which = 0; which < 2; ++which) {
    const u32x4 x = ld16(which ? v + t * v_ts + h * v_hs + 8 * ci : k + t * k_ts + h * k_hs + 8 * ci);
    float f[8];
    float a = 0.f;
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      f[2 * e] = bf16_lo(x[e]);
      f[2 * e + 1] = bf16_hi(x[e]);
      a = fmaxf(a, fmaxf(fabsf(f[2 * e]), fabsf(f[2 * e + 1])));
    }
    if (!has) a = 0.f;
#pragma unroll
    for (int m = 1; m < kLanes; m <<= 1) a = fmaxf(a, __shfl_xor(a, m, kLanes));
    // a = 1.m * 2^E: a / 2^(E-8) = 1.m * 256 <= 448 iff 1.m <= 1.75, else
    // 2^(E-7) is the smallest; exponent fields below 1 are raised to 1
    const uint32_t ab = __float_as_uint(a);
    const int ef = (int)(ab >> 23) - 8 + ((ab & 0x7fffffu) > 0x600000u ? 1 : 0);
    const int e = ef < 1 ? 1 : ef;                                   // scale 2^(e - 127)
    const bool nz = a > 0.f;
    const float sc = nz ? __uint_as_float((uint32_t)e << 23) : 1.f;
    const float inv = nz ? __uint_as_float((uint32_t)(254 - e) << 23) : 1.f;  // 1 / sc, exact
    int lo = 0, hi = 0;
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[0] * inv, f[1] * inv, lo, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(f[2] * inv, f[3] * inv, lo, true);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[4] * inv, f[5] * inv, hi, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(f[6] * inv, f[7] * inv, hi, true);
    if (has) *reinterpret_cast<u32x2*>((which ? v_cache : k_cache) + dst) = u32x2{(uint32_t)lo, (uint32_t)hi};
    if (i16 == 0) (which ? v_scales : k_scales)[sdst] = sc;
  }
}

// Page copies for copy-on-write: page dst[i] <- page src[i] for K and V.
// blockIdx.y = pair, x covers the page's page_size * Hkv * d/8 chunks.
__global__ void __launch_bounds__(256)
copy_blocks_kernel(uint16_t* __restrict__ k_cache, uint16_t* __restrict__ v_cache, int32_t num_pages,
                   int32_t page_size, int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                   int32_t chunks_per_head, int32_t chunks_per_slot,
                   const int32_t* __restrict__ src, const int32_t* __restrict__ dst) {
  const int64_t c = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (c >= (int64_t)page_size * chunks_per_slot) return;
  const int32_t sp = src[blockIdx.y], dp = dst[blockIdx.y];
  if (sp < 0 || sp >= num_pages || dp < 0 || dp >= num_pages) return;
  const int32_t slot = (int32_t)(c / chunks_per_slot);
  const int32_t r = (int32_t)(c - (int64_t)slot * chunks_per_slot);
  const int32_t h = r / chunks_per_head;
  const int32_t e = (r - h * chunks_per_head) * 8;
  const int64_t off = (int64_t)slot * slot_stride + h * head_stride + e;
  st16(k_cache + dp * page_stride + off, ld16(k_cache + sp * page_stride + off));
  st16(v_cache + dp * page_stride + off, ld16(v_cache + sp * page_stride + off));
}

}  // namespace pa

using namespace pa;

extern "C" int pa_kv_store(const uint16_t* k, int64_t k_tok_stride, int64_t k_head_stride,
                           const uint16_t* v, int64_t v_tok_stride, int64_t v_head_stride,
                           const int32_t* slot_mapping, int32_t num_tokens,
                           int32_t num_kv_heads, int32_t head_dim,
                           uint16_t* k_cache, uint16_t* v_cache,
                           int32_t num_pages, int32_t page_size,
                           int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                           void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_pages <= 0 || page_size <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_kv_store: bad sizes (num_tokens=%d, num_kv_heads=%d, head_dim=%d, num_pages=%d, page_size=%d)",
                num_tokens, num_kv_heads, head_dim, num_pages, page_size);
  if (num_tokens == 0) return PA_OK;
  if (!k || !v || !slot_mapping || !k_cache || !v_cache)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_kv_store: null pointer");
  hipStream_t s = (hipStream_t)stream;
  const int64_t num_slots = (int64_t)num_pages * page_size;
  const bool vec = head_dim % 8 == 0 && aligned16(k) && aligned16(v) && aligned16(k_cache) &&
                   aligned16(v_cache) && k_tok_stride % 8 == 0 && k_head_stride % 8 == 0 &&
                   v_tok_stride % 8 == 0 && v_head_stride % 8 == 0 && page_stride % 8 == 0 &&
                   slot_stride % 8 == 0 && head_stride % 8 == 0;
  if (vec) {
    const int32_t cph = head_dim / 8;
    const int32_t cpt = cph * num_kv_heads;
    const int64_t threads = (int64_t)num_tokens * cpt;
    const int64_t blocks = (threads + 255) / 256;
    kv_store_vec_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        k, k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, slot_mapping, num_tokens,
        cph, cpt, k_cache, v_cache, num_slots, page_size, page_stride, slot_stride, head_stride);
  } else {
    const int32_t ept = head_dim * num_kv_heads;
    const int64_t threads = (int64_t)num_tokens * ept;
    const int64_t blocks = (threads + 255) / 256;
    kv_store_scalar_kernel<<<dim3((unsigned)blocks), dim3(256), 0, s>>>(
        k, k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, slot_mapping, num_tokens,
        head_dim, ept, k_cache, v_cache, num_slots, page_size, page_stride, slot_stride, head_stride);
  }
  return launch_status("pa_kv_store");
}

extern "C" int pa_gather_kv(const uint16_t* cache, int32_t num_pages, int32_t page_size,
                            int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                            const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                            const int32_t* lengths, int32_t batch,
                            int32_t num_kv_heads, int32_t head_dim, uint16_t* out, void* stream) {
  if (batch < 0 || pages_per_seq < 0 || num_kv_heads <= 0 || head_dim <= 0 || num_pages <= 0 ||
      page_size <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_gather_kv: bad sizes");
  if (batch == 0 || pages_per_seq == 0) return PA_OK;
  if (!cache || !block_tables || !lengths || !out)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_gather_kv: null pointer");
  const int32_t ept = head_dim * num_kv_heads;
  const int64_t threads = (int64_t)batch * pages_per_seq * page_size * ept;
  const int64_t blocks = (threads + 255) / 256;
  gather_kv_kernel<<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
      cache, num_pages, page_size, page_stride, slot_stride, head_stride, block_tables, bt_stride,
      pages_per_seq, lengths, batch, head_dim, ept, out);
  return launch_status("pa_gather_kv");
}

extern "C" int pa_copy_blocks(uint16_t* k_cache, uint16_t* v_cache, int32_t num_pages, int32_t page_size,
                              int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                              int32_t num_kv_heads, int32_t head_dim,
                              const int32_t* src_blocks, const int32_t* dst_blocks, int32_t num_copies, void* stream) {
  if (num_pages <= 0 || page_size <= 0 || num_kv_heads <= 0 || head_dim <= 0 || head_dim % 8 || num_copies < 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_copy_blocks: bad sizes (num_pages=%d, page_size=%d, num_kv_heads=%d, head_dim=%d, n=%d)",
                num_pages, page_size, num_kv_heads, head_dim, num_copies);
  if (num_copies == 0) return PA_OK;
  if (num_copies > 65535) return fail(PA_ERR_UNSUPPORTED, "pa_copy_blocks: at most 65535 copies per call");
  if (!k_cache || !v_cache || !src_blocks || !dst_blocks)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_copy_blocks: null pointer");
  if ((((uintptr_t)k_cache | (uintptr_t)v_cache) & 15u) || (page_stride | slot_stride | head_stride) % 8)
    return fail(PA_ERR_UNSUPPORTED, "pa_copy_blocks: pools must be 16-byte aligned with strides multiple of 8");
  const int32_t cph = head_dim / 8;
  const int32_t cps = cph * num_kv_heads;
  const int64_t chunks = (int64_t)page_size * cps;
  const dim3 grid((unsigned)((chunks + 255) / 256), (unsigned)num_copies);
  copy_blocks_kernel<<<grid, dim3(256), 0, (hipStream_t)stream>>>(k_cache, v_cache, num_pages, page_size, page_stride,
                                                                  slot_stride, head_stride, cph, cps, src_blocks,
                                                                  dst_blocks);
  return launch_status("pa_copy_blocks");
}

extern "C" int pa_kv_store_fp8(const uint16_t* k, int64_t k_tok_stride, int64_t k_head_stride,
                               const uint16_t* v, int64_t v_tok_stride, int64_t v_head_stride,
                               const int32_t* slot_mapping, int32_t num_tokens,
                               int32_t num_kv_heads, int32_t head_dim,
                               uint8_t* k_cache, uint8_t* v_cache, float* k_scales, float* v_scales,
                               int32_t num_pages, int32_t page_size,
                               int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                               int64_t scale_page_stride, int64_t scale_slot_stride, int64_t scale_head_stride,
                               void* stream) {
  if (num_tokens < 0 || num_kv_heads <= 0 || num_pages <= 0 || page_size <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_kv_store_fp8: bad sizes (num_tokens=%d, num_kv_heads=%d, num_pages=%d, page_size=%d)",
                num_tokens, num_kv_heads, num_pages, page_size);
  if (head_dim % 16 != 0 || head_dim < 16 || head_dim > 256)
    return fail(PA_ERR_UNSUPPORTED, "pa_kv_store_fp8: head_dim %d not supported (a multiple of 16 from 16 to 256)",
                head_dim);
  if (num_tokens == 0) return PA_OK;
  if (!k || !v || !slot_mapping || !k_cache || !v_cache || !k_scales || !v_scales)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_kv_store_fp8: null pointer");
  if (!aligned16(k) || !aligned16(v) || ((uintptr_t)k_cache | (uintptr_t)v_cache) & 7u ||
      ((uintptr_t)k_scales | (uintptr_t)v_scales) & 3u ||
      (k_tok_stride | k_head_stride | v_tok_stride | v_head_stride) % 8 || (page_stride | slot_stride | head_stride) % 8)
    return fail(PA_ERR_UNSUPPORTED, "pa_kv_store_fp8: bf16 rows must be 16-byte and code rows 8-byte aligned");
  const int64_t groups = (int64_t)num_tokens * num_kv_heads;
  const int32_t cph = head_dim / 8;
  const int lanes = cph <= 16 ? 16 : 32;
  const int64_t blocks = (groups * lanes + 255) / 256;
  if (blocks > 0x7fffffff) return fail(PA_ERR_UNSUPPORTED, "pa_kv_store_fp8: %d tokens too many", num_tokens);
  if (lanes == 16)
    kv_store_fp8_kernel<16><<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
        k, k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, slot_mapping, num_tokens, num_kv_heads, cph,
        k_cache, v_cache, k_scales, v_scales, (int64_t)num_pages * page_size, page_size, page_stride, slot_stride,
        head_stride, scale_page_stride, scale_slot_stride, scale_head_stride);
  else
    kv_store_fp8_kernel<32><<<dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream>>>(
        k, k_tok_stride, k_head_stride, v, v_tok_stride, v_head_stride, slot_mapping, num_tokens, num_kv_heads, cph,
        k_cache, v_cache, k_scales, v_scales, (int64_t)num_pages * page_size, page_size, page_stride, slot_stride,
        head_stride, scale_page_stride, scale_slot_stride, scale_head_stride);
  return launch_status("pa_kv_store_fp8");
}
