// Split-K paged GQA decode for gfx950.
//
// Workgroup = (sequence b, kv head, chunk of context tokens: 4096 on large
// launches with pages of 64+ tokens, else 2048, 1024 when pages hold 16
// tokens), four wavefronts.  The chunk is cut into 16-token steps dealt
// round-robin to the waves (wave w takes steps w, w+4, ...), so the four waves stream
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
// lane is its accumulator column.  K and V are read as 16-byte pieces where
// each 16-lane group reads one whole 256-byte token row (full cache lines,
// non-temporal).  V is transposed in registers with v_perm_b32: the M (d)
// dimension of the PV MFMA is permuted so that M-tile j row m holds
// d = 8m + j, and a lane then owns the 8 contiguous d values of its V load.
// K goes through the wave's LDS into the row-per-lane MFMA A layout (pages
// whose size is not a multiple of 16 read K in that layout directly).
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
#pragma once
#include <type_traits>

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
#ifndef PA_DECODE_BUFS_FP8
#define PA_DECODE_BUFS_FP8 4
#endif
constexpr int kDecodeBufsFp8 = PA_DECODE_BUFS_FP8;  // ... with float8 pages (half the bytes per step)
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
  // q heads of a kv head are taken 16 at a time (the MFMA's N columns): a
  // work item is one of hblocks = ceil(group / 16) blocks of them, and reads
  // its kv head's K/V itself
  int32_t hblocks;
  int32_t chunk;     // tokens per workgroup
  int32_t n_chunks;  // chunks of the widest block-table row
  float logit_scale;  // scale * log2(e) when soft_cap is off, else scale
  float soft_cap;     // <= 0: off
  float* ws_o;        // [batch, Hkv, n_chunks, group, d]
  float* ws_ml;       // [batch, Hkv, n_chunks, group, 2] (max log2, sum)
  uint16_t* out;
  int64_t out_bs, out_hs;
  // Optional row map (null: sequence b owns q / out row b).  Otherwise
  // rows[b] is the q / out row of sequence b and rows[b + 1] > rows[b] must
  // hold (a cu_seqlens array); a sequence without a row in [0, row_limit)
  // is skipped.
  const int32_t* rows;
  int32_t row_limit;
  int32_t zero_empty;  // write zeros for length-0 sequences here (no merge pass follows)
  // float8 pages: e4m3 codes addressed with the strides above (in bytes), and
  // per-token float scales addressed [page][head][slot] with slot stride 1
  const uint8_t* k8;
  const uint8_t* v8;
  const float* k_scales;
  const float* v_scales;
  int64_t sc_page_stride, sc_head_stride;
  // Work list (may be null): plan[0] = number of listed (sequence, chunk)
  // pairs, plan[kDecodePlanHeader + r] = pair index b * n_chunks + c of rank
  // r, most tokens first.
  const int32_t* plan;
};
constexpr int kDecodePlanHeader = 64;  // ints before the first entry (256 bytes)

__device__ __forceinline__ int64_t decode_row(const DecodeParams& p, int b) { return p.rows ? p.rows[b] : b; }

__device__ __forceinline__ bool decode_has_row(const DecodeParams& p, int b) {
  if (!p.rows) return true;
  const int r0 = p.rows[b];
  return r0 >= 0 && r0 < p.row_limit && p.rows[b + 1] > r0;
}

// K and V rows are read exactly once and as whole rows: stream them past the
// caches.  (Half-row K reads, 64 bytes per row per instruction, must stay
// cacheable for the instruction that reads the other half.)
__device__ __forceinline__ u32x4 ld16_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(p));
}
__device__ __forceinline__ u32x2 ld8_stream(const void* p) {
  return __builtin_nontemporal_load(reinterpret_cast<const u32x2*>(p));
}
// K/V loads of a decode item: streamed, unless kShared (more than 16 q heads
// per kv head: the item's q-head blocks are separate items on one XCD, run
// next to each other, and each reads the kv head's K and V; cacheable loads
// let the later blocks hit the XCD's L2 instead of HBM).
template <bool kShared>
__device__ __forceinline__ u32x4 ld16_kv(const void* p) {
  if constexpr (kShared) return *reinterpret_cast<const u32x4*>(p);
  else return ld16_stream(p);
}
template <bool kShared>
__device__ __forceinline__ u32x2 ld8_kv(const void* p) {
  if constexpr (kShared) return *reinterpret_cast<const u32x2*>(p);
  else return ld8_stream(p);
}

__device__ __forceinline__ f32x4 mfma16k16(const bf16x4v& a, const bf16x4v& b, const f32x4& c) {
  return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
}

// The bf16 halves selected by `hi` of a and b, packed as (a_half, b_half).
__device__ __forceinline__ uint32_t pick2(uint32_t a, uint32_t b, bool hi) {
  return hi ? __builtin_amdgcn_perm(b, a, 0x07060302u) : __builtin_amdgcn_perm(b, a, 0x05040100u);
}

// LDS of the cross-wave combine: o [waves][16 q columns][d], m and l [waves][16].
struct alignas(16) DecodeLds {
  float o[kDecodeWaves][16][kHeadDim];
  float m[kDecodeWaves][16];
  float l[kDecodeWaves][16];
};

// Workgroups are dealt round-robin to the 8 XCDs: XCD x = bid % 8 serves
// items [x*q8 + min(x, r8), ...) in order.  A bijection of [0, nb).
__device__ __forceinline__ int xcd_grouped_item(int bid, int nb) {
  const int x = bid & 7, k = bid >> 3;
  const int q8 = nb >> 3, r8 = nb & 7;
  return x * q8 + min(x, r8) + k;
}

// Tokens per workgroup (the shorter chunks; large launches over pages of 16+
// tokens that are a multiple of 16 take 4096): with one page id per lane
// (one VGPR) a chunk spans at most 64 pages.
__host__ __device__ inline int decode_chunk_tokens(int page_size) { return page_size >= 32 ? 2048 : 1024; }

// One decode work item (sequence, chunk, kv head) numbered `item`, run by
// kWaves wavefronts (threads 0 .. 64*kWaves-1 of the workgroup).  red_o /
// red_m / red_l are LDS arrays of [kWaves][16][d] and [kWaves][16] floats.
// kAligned: page_size % 16 == 0, so a 16-token step never crosses a page and
// the chunk's page ids are read once, kIds per lane (lane l holds the ids of
// the chunk's pages l, l + 64, ...): a chunk spans at most 64 kIds pages.
// kFp8: K/V pages hold 1-byte codes with per-token scales
// (decode_paged_attention.py:72-81,108-115), float8 e4m3 or integers by
// kCode: K is widened to bf16 exactly and its logits multiplied by the
// token's K scale; P is multiplied by the token's V scale before PV.  Half
// the K/V bytes of the bf16 path.
template <int kWaves, bool kAligned, bool kSoftCap, bool kFp8 = false, bool kShared = false, int kCode = kCodeE4M3,
          int kIds = 1>
__device__ __forceinline__ void decode_item(const DecodeParams& p, int item, float* red_o, float* red_m,
                                            float* red_l) {
  static_assert(kIds == 1 || kIds == 4, "one or four page ids per lane");
  static_assert(kWaves == 4 || kWaves == 8, "the combine splits d over the waves");
  static_assert(!kFp8 || kAligned, "float8 pages need 16-token aligned steps");
  constexpr int kBufs = kFp8 ? kDecodeBufsFp8 : kDecodeBufs;
  constexpr int kDPerWave = kHeadDim / kWaves;  // output d values each wave finishes
  constexpr int kDPerLane = kDPerWave / 4;      // ... each lane (4 lane groups)
  const int lane = threadIdx.x & 63;
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int hkv = p.num_kv_heads;
  const int vheads = hkv * p.hblocks;  // (kv head, block of 16 q heads) pairs
  const int vh = item % vheads;
  const int rest = item / vheads;
  const int kvh = vh / p.hblocks;
  const int qc0 = 16 * (vh - kvh * p.hblocks);  // first q column (head within the group) of this item
  const int g_end = min(p.group, qc0 + 16);
  const int chunk = rest % p.n_chunks;
  const int b = rest / p.n_chunks;
  // lengths past the block table's span are clamped to it (no read beyond the table row)
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  if (!decode_has_row(p, b)) return;  // uniform over the workgroup
  const int t_begin = chunk * p.chunk;
  if (t_begin >= len) {  // uniform over the workgroup
    if (chunk == 0 && p.zero_empty) {
      // length 0: the G output rows of this kv head are zero
      const int64_t orow = decode_row(p, b) * p.out_bs;
      for (int c = threadIdx.x; c < (g_end - qc0) * (kHeadDim / 8); c += 64 * kWaves)
        st16(p.out + orow + (int64_t)(kvh * p.group + qc0 + c / (kHeadDim / 8)) * p.out_hs + 8 * (c % (kHeadDim / 8)),
             u32x4{0, 0, 0, 0});
    }
    return;
  }
  const int t_end = min(t_begin + p.chunk, len);
  const int n_steps = (t_end - t_begin + kDecodeStep - 1) / kDecodeStep;
  const int my_steps = n_steps > wave ? (n_steps - wave + kWaves - 1) / kWaves : 0;
  const int n_chunks_b = (len + p.chunk - 1) / p.chunk;

  const int n = lane & 15;  // q column of S/O; the d chunk of V loads; the token of K loads
  const int g = lane >> 4;  // 16-lane group
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int64_t head_off = (int64_t)kvh * p.head_stride;

  // Page ids of the chunk, one per lane (aligned path).
  const int lp_first = t_begin / p.page_size;
  int32_t my_page = 0;
  int32_t my_page_hi[kIds == 4 ? 3 : 1] = {};  // (kIds == 4) page ids lp_first + 64 (j + 1) + lane
  if constexpr (kAligned) {
    const int lp = lp_first + lane;
    if (lp < p.pages_per_seq) my_page = safe_page(bt_row, lp, p.num_pages);
    if constexpr (kIds == 4) {
#pragma unroll
      for (int j = 0; j < 3; ++j)
        if (lp + 64 * (j + 1) < p.pages_per_seq) my_page_hi[j] = safe_page(bt_row, lp + 64 * (j + 1), p.num_pages);
    }
  }
  // the page id of the chunk's page idx (wave-uniform)
  auto chunk_page = [&](int idx) __attribute__((always_inline)) -> int32_t {
    if constexpr (kIds == 1) {
      return __builtin_amdgcn_readlane(my_page, idx);
    } else {
      const int k = idx >> 6;
      const int32_t v = k == 0 ? my_page : (k == 1 ? my_page_hi[0] : (k == 2 ? my_page_hi[1] : my_page_hi[2]));
      return __builtin_amdgcn_readlane(v, idx & 63);
    }
  };

  // Q^T operand: k-step s uses d chunk kchunk(s) for both Q and K (any
  // bijection works for a dot product).  bf16 pages: chunk 4s + g.  Float8
  // pages: chunk 8(s/2) + 2g + s%2, so that a lane's K chunks for steps
  // 2r, 2r+1 are 16 adjacent bytes (one 16-byte load per pair of steps).
  auto kchunk = [&](int s) __attribute__((always_inline)) {
    return kFp8 ? 8 * (s >> 1) + 2 * g + (s & 1) : 4 * s + g;
  };
  bf16x8 qt[4];
  {
    const bool live = qc0 + n < g_end;
    const uint16_t* qrow = p.q + decode_row(p, b) * p.q_bs + (int64_t)(kvh * p.group + qc0 + (live ? n : 0)) * p.q_hs;
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      u32x4 v = live ? ld16(qrow + 8 * kchunk(s)) : u32x4{0, 0, 0, 0};
      qt[s] = as_bf16x8(v);
    }
  }

  f32x4 acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float m_run = -1e30f;  // finite so that exp2(x - m) never sees inf - inf
  float l_run = 0.f;

  // K: 4 loads of 8 bf16, or 2 loads of 16 float8 codes; V: 4 loads of 8 values
  constexpr int kKLoads = kFp8 ? 2 : 4;
  using VBuf = std::conditional_t<kFp8, u32x2, u32x4>;
  u32x4 kb[kBufs][kKLoads];
  VBuf vb[kBufs][4];
  u32x4 sb[kFp8 ? kBufs : 1][2];  // K and V scales of tokens t0+4g .. t0+4g+3

  // Loads of wave step `ks` (tokens t0 .. t0+15) into one buffer.  Tokens past
  // the sequence end are clamped onto its last token (same page in the aligned
  // case), so no stale or NaN data reaches the accumulator.  A step past the
  // wave's last one still issues its 8 loads, all of the first 256 bytes of q
  // (cache hits): every buffer then sees the same number of loads issued
  // after it, and the compiler waits for exactly the buffer being consumed.
  auto issue = [&](int j, int ks) __attribute__((always_inline)) {
    u32x4(&kd)[kKLoads] = kb[j];
    VBuf(&vd)[4] = vb[j];
    const bool valid = ks < my_steps;  // uniform
    const int t0 = t_begin + kDecodeStep * (kWaves * ks + wave);
    const int lim = len - 1 - t0;  // >= 0 when valid
    if constexpr (kFp8) {
      const uint8_t* kbase = reinterpret_cast<const uint8_t*>(p.q);
      const uint8_t* vbase = kbase;
      const float* ksp = reinterpret_cast<const float*>(p.q);
      const float* vsp = ksp;
      int64_t rs = 0;
      if (valid) {
        const int lp = t0 / p.page_size;
        const int32_t page = chunk_page(lp - lp_first);
        const int off = t0 - lp * p.page_size;
        const int64_t base = (int64_t)page * p.page_stride + (int64_t)off * p.slot_stride + head_off;
        kbase = p.k8 + base;
        vbase = p.v8 + base;
        rs = p.slot_stride;
        const int64_t sbase = (int64_t)page * p.sc_page_stride + (int64_t)kvh * p.sc_head_stride + off + 4 * g;
        ksp = p.k_scales + sbase;
        vsp = p.v_scales + sbase;
      }
      // K rows whole (128 bytes of codes, eight lanes a row), streamed: load r
      // gives lane l row 8r + l / 8, 16-byte chunk l % 8
#pragma unroll
      for (int r = 0; r < kKLoads; ++r)
        kd[r] = ld16_kv<kShared>(kbase + (int64_t)min(8 * r + (lane >> 3), lim) * rs + 16 * (lane & 7));
#pragma unroll
      for (int i = 0; i < 4; ++i) vd[i] = ld8_kv<kShared>(vbase + (int64_t)min(4 * g + i, lim) * rs + 8 * n);
      sb[j][0] = ld16(ksp);
      sb[j][1] = ld16(vsp);
    } else if constexpr (kAligned) {
      const uint16_t* kbase = p.q;
      const uint16_t* vbase = p.q;
      int64_t rs = 0;
      if (valid) {
        const int lp = t0 / p.page_size;
        const int32_t page = chunk_page(lp - lp_first);
        const int64_t base = (int64_t)page * p.page_stride +
                             (int64_t)(t0 - lp * p.page_size) * p.slot_stride + head_off;
        kbase = p.k_cache + base;
        vbase = p.v_cache + base;
        rs = p.slot_stride;
      }
      // K rows whole (one 256-byte row per 16-lane group), streamed like V:
      // load i gives lane (n, g) row 4i + g, chunk n
#pragma unroll
      for (int i = 0; i < 4; ++i) kd[i] = ld16_kv<kShared>(kbase + (int64_t)min(4 * i + g, lim) * rs + 8 * n);
#pragma unroll
      for (int i = 0; i < 4; ++i) vd[i] = ld16_kv<kShared>(vbase + (int64_t)min(4 * g + i, lim) * rs + 8 * n);
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
      for (int i = 0; i < 4; ++i) vd[i] = ld16_kv<kShared>(p.v_cache + tok_off(t0 + min(4 * g + i, lim)) + 8 * n);
    }
  };

  auto consume = [&](int j, int ks) __attribute__((always_inline)) {
    const u32x4(&kd)[kKLoads] = kb[j];
    const VBuf(&vdr)[4] = vb[j];
    const int t0 = t_begin + kDecodeStep * (kWaves * ks + wave);
    f32x4 sc = {0.f, 0.f, 0.f, 0.f};
    if constexpr (kAligned) {
      // The K A operand wants row n per lane (chunks kchunk(s)); the loads
      // delivered whole rows across lanes.  The wave turns them round
      // through its own slice of red_o (free until the combine), with chunk c
      // of row r stored at c ^ (r mod rows-per-bank-cycle): conflict-free
      // 16-byte writes and reads.
      typedef u32x4 __attribute__((address_space(3))) * lds_u32x4;
      const uint32_t kst = (uint32_t)(uintptr_t)(float __attribute__((address_space(3)))*)(red_o) +
                           (uint32_t)(wave * 16 * kHeadDim * 4);
      if constexpr (kFp8) {
#pragma unroll
        for (int r = 0; r < kKLoads; ++r) {
          const int row = 8 * r + (lane >> 3);
          *(lds_u32x4)(uintptr_t)(kst + 128 * row + 16 * ((lane & 7) ^ (row & 7))) = kd[r];
        }
        u32x4 kr[kKLoads];
#pragma unroll
        for (int r = 0; r < kKLoads; ++r)  // row n, chunk 4r + g: the codes of k-steps 2r, 2r + 1
          kr[r] = *(lds_u32x4)(uintptr_t)(kst + 128 * n + 16 * ((4 * r + g) ^ (n & 7)));
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u32x4& w = kr[s >> 1];
          const u32x4 kk = codes8_to_bf16x8<kCode>((s & 1) ? u32x2{w[2], w[3]} : u32x2{w[0], w[1]});
          sc = mfma16(as_bf16x8(kk), qt[s], sc);
        }
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const int r = 4 * i + g;
          *(lds_u32x4)(uintptr_t)(kst + 256 * r + 16 * (n ^ (r & 15))) = kd[i];
        }
#pragma unroll
        for (int s = 0; s < 4; ++s) {
          const u32x4 kk = *(lds_u32x4)(uintptr_t)(kst + 256 * n + 16 * ((4 * s + g) ^ (n & 15)));
          sc = mfma16(as_bf16x8(kk), qt[s], sc);
        }
      }
    } else {
#pragma unroll
      for (int s = 0; s < 4; ++s) sc = mfma16(as_bf16x8(kd[s]), qt[s], sc);
    }
    // lane holds S[q = n][token t0 + 4g + r]
    float x[4];
    float mx = -INFINITY;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      float v = sc[r];
      if constexpr (kFp8) v *= __uint_as_float(sb[j][0][r]);
      if constexpr (kSoftCap) v = soft_cap_log2(v, soft_cap_s2(p.logit_scale, p.soft_cap), soft_cap_c(p.soft_cap));
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
    if constexpr (kFp8) {
#pragma unroll
      for (int r = 0; r < 4; ++r)  // past the length the scale slot is not data: select, never multiply
        x[r] = t0 + 4 * g + r < len ? x[r] * __uint_as_float(sb[j][1][r]) : 0.f;
    }
    u32x2 pw;
    pw[0] = pack_bf16x2(x[0], x[1]);
    pw[1] = pack_bf16x2(x[2], x[3]);
    const bf16x4v pt = __builtin_bit_cast(bf16x4v, pw);
    u32x4 vd[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if constexpr (kFp8) vd[i] = codes8_to_bf16x8<kCode>(vdr[i]);
      else vd[i] = vdr[i];
    }
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
  for (int j = 0; j < kBufs; ++j) issue(j, j);
  for (int k0 = 0; k0 < my_steps; k0 += kBufs) {
#pragma unroll
    for (int j = 0; j < kBufs; ++j) {
      const int ks = k0 + j;
      if (ks < my_steps) consume(j, ks);
      issue(j, ks + kBufs);
    }
  }

  // ---- combine the waves through LDS
  l_run = sum_xor16(l_run);
  l_run = sum_xor32(l_run);
  // acc[j][r] = O^T[d = 8 * (4g + r) + j][q = n]
  auto ro = [&](int w, int col, int d) __attribute__((always_inline)) -> float* {
    return red_o + ((w * 16 + col) * kHeadDim + d);
  };
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    float* dst = ro(wave, n, 32 * g + 8 * r);
    *reinterpret_cast<f32x4*>(dst) = f32x4{acc[0][r], acc[1][r], acc[2][r], acc[3][r]};
    *reinterpret_cast<f32x4*>(dst + 4) = f32x4{acc[4][r], acc[5][r], acc[6][r], acc[7][r]};
  }
  if (g == 0) {
    red_m[wave * 16 + n] = m_run;
    red_l[wave * 16 + n] = l_run;
  }
  __syncthreads();
  // wave w finishes d = kDPerWave*w + kDPerLane*g .. of column n
  float mm = red_m[n];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) mm = fmaxf(mm, red_m[w * 16 + n]);
  float o[kDPerLane];
#pragma unroll
  for (int i = 0; i < kDPerLane; ++i) o[i] = 0.f;
  float ll = 0.f;
  const int d0 = kDPerWave * wave + kDPerLane * g;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    const float sw = fast_exp2(red_m[w * 16 + n] - mm);
    ll += sw * red_l[w * 16 + n];
#pragma unroll
    for (int i4 = 0; i4 < kDPerLane / 4; ++i4) {
      const f32x4 a = *reinterpret_cast<const f32x4*>(ro(w, n, d0 + 4 * i4));
#pragma unroll
      for (int i = 0; i < 4; ++i) o[4 * i4 + i] += sw * a[i];
    }
  }
  if (qc0 + n >= g_end) return;
  if (n_chunks_b == 1) {
    const float inv = 1.f / ll;  // ll >= 1: the chunk holds a visible token
    uint16_t* dst = p.out + decode_row(p, b) * p.out_bs + (int64_t)(kvh * p.group + qc0 + n) * p.out_hs + d0;
    if constexpr (kDPerLane == 8) {
      u32x4 w;
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = pack_bf16x2(o[2 * i] * inv, o[2 * i + 1] * inv);
      st16(dst, w);
    } else {
      u32x2 w;
#pragma unroll
      for (int i = 0; i < 2; ++i) w[i] = pack_bf16x2(o[2 * i] * inv, o[2 * i + 1] * inv);
      *reinterpret_cast<u32x2*>(dst) = w;
    }
  } else {
    const int64_t part = (((int64_t)b * hkv + kvh) * p.n_chunks + chunk) * p.group + qc0 + n;
    float* dst = p.ws_o + part * kHeadDim + d0;
#pragma unroll
    for (int i4 = 0; i4 < kDPerLane / 4; ++i4)
      *reinterpret_cast<f32x4*>(dst + 4 * i4) = f32x4{o[4 * i4], o[4 * i4 + 1], o[4 * i4 + 2], o[4 * i4 + 3]};
    if (wave == 0 && g == 0) {
      p.ws_ml[2 * part] = mm;
      p.ws_ml[2 * part + 1] = ll;
    }
  }
}

// Host launch of decode_merge_kernel for the sequences of `p` (defined with
// the kernel in decode.hip).
void launch_decode_merge(const DecodeParams& p, hipStream_t s);

}  // namespace pa
