// Paged attention for head sizes other than 128 (multiples of 16 from 16 to
// 256): a prefill kernel and a split-K decode kernel with its merge.  The
// reference takes any head size as long as q and the pages agree
// (prefill_paged_attention.py:199-203, decode_paged_attention.py:356-360);
// the tuned kernels of prefill.hip / decode.hip are built for 128, and these
// cover the rest with the same arithmetic: S in f32 on the matrix core from
// bf16 q (scaled by scale * log2 e and rounded, without the soft cap) and K,
// exp2 online softmax with a lazily moved reference max, P rounded to bf16
// for PV, f32 O.
//
// Both kernels use v_mfma_f32_32x32x16_bf16 (lane layouts in pa_common.h)
// in the same two products per 32-token kv step:
//   S^T = K Q^T     A = K rows (m = token, from the staged K tile), B = Q^T
//                   (n = q row or head);
//                   lane (n, h = lane / 32) ends with column n's logits of
//                   tokens 8(i/4) + 4h + i%4, i < 16;
//   O^T += V^T P^T  A = V^T (m = d), B = P^T (n as above): the lane's own
//                   eight P values of k-step u, tokens 16u + 8(e/4) + 4h +
//                   e%4, fill its k slots 8h + e.
// K and V are staged row-major in LDS with whole-row 16-byte writes.  An
// A operand of V^T (d = the lane's row, the eight tokens of its k slots) is
// two transposing 8-byte reads (vt_operand).  The online-softmax state of a
// column lives in the two lanes (n, 0) and (n, 1), exactly where O^T's
// column n lives, so the rescale needs no exchange.
#include <climits>
#include <type_traits>

#include "any_head.h"
#include "decode_impl.h"
#include "prefill_impl.h"

namespace pa {
namespace {

// Prefill waves per workgroup (32 q rows each): 8 while the registers allow
// two waves per SIMD (head sizes up to 112), else 4.
__host__ __device__ constexpr int any_prefill_waves(int d) { return d <= 112 ? 8 : 4; }
// Up to head size 64 the prefill's registers are capped at 128 per lane
// (four waves per SIMD), so two workgroups share a CU; from 80 on the cap
// would spill.  Pages below 16 tokens are paged per chunk, and their page
// ids are read a step ahead only with one workgroup per CU (four waves,
// from head size 144 on; see prefill_any_kernel).
__host__ __device__ constexpr int any_prefill_wpe(int d) { return d <= 64 ? 4 : 1; }
__host__ __device__ constexpr bool any_pages_ahead(int d) { return any_prefill_waves(d) == 4; }
constexpr int kAnyStep = 32;                 // kv tokens per step (the MFMA's M)

template <int D>
struct AnyDims {
  static_assert(D % 16 == 0 && D >= 16 && D <= 256, "head size");
  static constexpr int kKs = D / 16;         // k-steps of S = K Q^T
  static constexpr int kDt = (D + 31) / 32;  // 32-row blocks of O^T
  static constexpr int kChunks = D / 8;      // 16-byte chunks of a K / V row
  // Bytes per K row in LDS: 16 bytes of padding put the 16 rows a K read
  // serves per pass (16 bytes each) on distinct banks.
  static constexpr int kRow = 2 * D + 16;
  // Bytes per V row: a transposing V^T read serves 32 lanes per pass, 4 rows
  // x 8 columns x 2 bytes wide and two 16-column groups; with a row stride of
  // 64 or 192 mod 256 bytes the 4 rows land on 4 disjoint quarters of the 64
  // banks (a stride of 2D + 16 put 2 to 4 lanes on a bank).  The smallest
  // padding of 0 / 32 / 64 / 96 bytes that gives it, which also keeps the
  // widest V^T operand (64 * kDt bytes from a row's start) inside its row.
  static constexpr int vpad() {
    for (int pad = 0; pad <= 96; pad += 32)
      if ((2 * D + pad) % 256 == 64 || (2 * D + pad) % 256 == 192) return pad;
    return 32;  // D = 16 (32-byte rows)
  }
  static constexpr int kVRow = 2 * D + vpad();
  static_assert(64 * kDt <= kVRow, "V^T operands stay inside their row");
  // the V tile, with 32 bytes of slack past its last row
  static constexpr int kVTile = kAnyStep * kVRow + 32;
};

typedef char __attribute__((address_space(3))) lds_char;

// Whether chunk c = tid + kThreads * i (i < kPer) of a step's kChunks
// exists.  Only the last i can fail, and none does when kChunks is a
// multiple of kThreads: a plain c < kChunks would leave a divergent branch
// around every chunk's load and LDS write (the compiler does not know the
// thread index is below kThreads), which keeps it from scheduling across
// them.
template <int kChunks, int kThreads, int kPer>
__device__ __forceinline__ bool any_chunk_live(int i, int c) {
  return kChunks % kThreads == 0 || i + 1 < kPer || c < kChunks;
}

// A operand of V^T for rows d0 .. d0 + 31 and k-step u from the row-major
// V tile (rows of `row` bytes): lane (m, h) takes d = d0 + m of the tokens
// 16u + 4h + {0,1,2,3} and 16u + 8 + 4h + {0,1,2,3}, in two transposing
// reads (ds_read_b64_tr_b16): in each 16-lane group, lane s addresses 4
// bf16 of token row s / 4 at columns 4 (s % 4) .. +3 of the group's 16
// columns and receives column s of the 4 rows.  Rows d >= the head size
// read the row padding or the next row: finite or not, they only feed rows
// of O^T that are never stored.
template <int kRowBytes>
__device__ __forceinline__ u32x4 vt_operand(const lds_char* v, int d0, int u, int lane) {
  const int sl = lane & 15;
  const lds_char* a =
      v + (16 * u + 4 * (lane >> 5) + (sl >> 2)) * kRowBytes + 2 * (d0 + 16 * ((lane >> 4) & 1) + 4 * (sl & 3));
  const u32x2 lo = __builtin_bit_cast(u32x2, ds_read_tr16((lds_cbytes)a));
  const u32x2 hi = __builtin_bit_cast(u32x2, ds_read_tr16((lds_cbytes)(a + 8 * kRowBytes)));
  return u32x4{lo[0], lo[1], hi[0], hi[1]};
}

__device__ __forceinline__ u32x4 lds_ld16(const lds_char* a) {
  return *reinterpret_cast<const u32x4 __attribute__((address_space(3)))*>(a);
}
__device__ __forceinline__ void lds_st16(lds_char* a, const u32x4& v) {
  *reinterpret_cast<u32x4 __attribute__((address_space(3)))*>(a) = v;
}

// Logit in log2 units.  Without the soft cap q arrives scaled by
// scale * log2 e (any_q_operand), so S already is; with it,
// cap * log2 e * tanh(x * scale / cap) (scale = logit_scale of the params).
template <bool kSoftCap>
__device__ __forceinline__ float any_logit(float x, float logit_scale, float cap) {
  if constexpr (kSoftCap) return soft_cap_log2(x, soft_cap_s2(logit_scale, cap), soft_cap_c(cap));
  else return x;
}

// A q operand (8 bf16), scaled by scale * log2 e and rounded to bf16 when
// the soft cap is off, as the tuned kernels do.
template <bool kSoftCap>
__device__ __forceinline__ bf16x8 any_q_operand(const u32x4& raw, float logit_scale) {
  if constexpr (kSoftCap) {
    return as_bf16x8(raw);
  } else {
    u32x4 o;
#pragma unroll
    for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(bf16_lo(raw[e]) * logit_scale, bf16_hi(raw[e]) * logit_scale);
    return as_bf16x8(o);
  }
}

// Logit in log2 units from an unscaled q: x * scale * log2 e, or the soft
// cap as above (decode, whose q is not scaled in bf16 first).
template <bool kSoftCap>
__device__ __forceinline__ float any_logit_f32(float x, float logit_scale, float cap) {
  if constexpr (kSoftCap) return soft_cap_log2(x, soft_cap_s2(logit_scale, cap), soft_cap_c(cap));
  else return x * logit_scale;
}

constexpr float kAnySlack = 8.f;  // lazy rescale: the reference max moves when a row max exceeds it by more

// The lazy reference max of the prefill: the column's reference m_run
// moves (and O and l are rescaled) only when some column of the wave
// exceeds its own by more than the slack; called when that holds for the
// step's row max mx.
template <int kDt>
__device__ __forceinline__ void any_lazy_rescale(float mx, float& m_run, float& l_run, f32x16 (&acc)[kDt]) {
  const float m_new = fmaxf(m_run, mx);
  const float corr = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
  m_run = m_new;
  l_run *= corr;
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt) acc[dt] = acc[dt] * corr;
}

// P of one step's logits relative to the reference max (lazy form: l and O
// already at m_run), its row sum into l_run, and O^T += V^T P^T from the
// staged V tile.
template <int kDt, int kRowBytes>
__device__ __forceinline__ void any_p_pv(const f32x16& s, float m_run, float& l_run, f32x16 (&acc)[kDt],
                                         const lds_char* v, int lane) {
  const float ms = m_run == -INFINITY ? 0.f : m_run;  // a column that has seen no key yet keeps P = 0
  float ls = 0.f;
  u32x4 pw[2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = fast_exp2(s[8 * u + 2 * e] - ms);
      const float b = fast_exp2(s[8 * u + 2 * e + 1] - ms);
      pw[u][e] = pack_bf16x2(a, b);
      ls += a + b;
    }
  l_run = l_run + ls;
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt)
#pragma unroll
    for (int u = 0; u < 2; ++u)
      acc[dt] = mfma32(as_bf16x8(vt_operand<kRowBytes>(v, 32 * dt, u, lane)), as_bf16x8(pw[u]), acc[dt]);
}

// Online softmax of one step's logits `s` (masked ones -inf) for the lane's
// column, then O^T += V^T P^T from the staged V tile (decode).  The running
// max moves every step: decode is bound by memory, and a lazy reference's
// branch costs registers at the large head sizes.
// kVs: quantized V pages, vs[i] the V scale of s[i]'s token: P is rounded to
// bf16 as p * vs for PV, while the row sum takes p itself.
template <int kDt, int kRowBytes, bool kVs = false>
__device__ __forceinline__ void any_softmax_pv(const f32x16& s, float& m_run, float& l_run, f32x16 (&acc)[kDt],
                                               const lds_char* v, int lane, const f32x16& vs = f32x16{}) {
  float mx = s[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
  mx = max_xor32(mx);
  const float m_new = fmaxf(m_run, mx);
  const float corr = fast_exp2(m_run - (m_new == -INFINITY ? 0.f : m_new));
  m_run = m_new;
  const float ms = m_run == -INFINITY ? 0.f : m_run;  // a column that has seen no key yet keeps P = 0
  float ls = 0.f;
  u32x4 pw[2];
#pragma unroll
  for (int u = 0; u < 2; ++u)
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      const float a = fast_exp2(s[8 * u + 2 * e] - ms);
      const float b = fast_exp2(s[8 * u + 2 * e + 1] - ms);
      if constexpr (kVs) pw[u][e] = pack_bf16x2(a * vs[8 * u + 2 * e], b * vs[8 * u + 2 * e + 1]);
      else pw[u][e] = pack_bf16x2(a, b);
      ls += a + b;
    }
  l_run = l_run * corr + ls;
#pragma unroll
  for (int dt = 0; dt < kDt; ++dt) {
    acc[dt] = acc[dt] * corr;
#pragma unroll
    for (int u = 0; u < 2; ++u)
      acc[dt] = mfma32(as_bf16x8(vt_operand<kRowBytes>(v, 32 * dt, u, lane)), as_bf16x8(pw[u]), acc[dt]);
  }
}

// ---- prefill: one workgroup of 8 or 4 waves per (q tile of 32 * waves / G tokens,
// sequence, kv head), grid order of prefill_item (no work list).  Row 32w + n
// of wave w is token row / G, head row % G of the kv head's group.  All
// waves share the step's K and V tiles (row-major); the next step's
// K / V chunks are loaded into registers while this step computes.
// kPaged3: pages of at least 16 tokens, so a 32-token step (clamped to the
// kv length) lies in at most three consecutive table entries: the step is
// paged once, with uniform values, instead of per lane and chunk.
template <int D, bool kSoftCap, bool kPaged3>
__global__ void __launch_bounds__(64 * any_prefill_waves(D)) __attribute__((amdgpu_waves_per_eu(any_prefill_wpe(D))))
prefill_any_kernel(PrefillParams p) {
  using A = AnyDims<D>;
  constexpr int kAnyWaves = any_prefill_waves(D);
  constexpr int kThreads = 64 * kAnyWaves;
  constexpr int kStepChunks = kAnyStep * A::kChunks;
  constexpr int kPer = (kStepChunks + kThreads - 1) / kThreads;  // chunks of K (and of V) per thread and step
  __shared__ __attribute__((aligned(16))) char k_tile_g[kAnyStep * A::kRow];
  __shared__ __attribute__((aligned(16))) char v_tile_g[A::kVTile];
  __shared__ int red_hi[kAnyWaves], red_lo[kAnyWaves];
  lds_char* k_tile = (lds_char*)k_tile_g;
  lds_char* v_tile = (lds_char*)v_tile_g;

  PrefillWork w;
  if (!prefill_resolve(p, blockIdx.x, w)) return;  // uniform across the workgroup
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = tid >> 6;
  const int n = lane & 31;
  const int h = lane >> 5;
  const int G = p.group;
  const int row = 32 * wave + n;
  const int rtok = w.qt * p.tile_tokens + row / G;
  const bool row_ok = row < p.tile_tokens * G && rtok < w.lq_rows;
  const int ltok = min(rtok, w.lq_rows - 1);  // lanes without a row compute on a real row, never stored
  const int head = w.kvh * G + row % G;
  const uint16_t* qrow = p.q + (int64_t)(w.q0 + ltok) * p.q_ts + (int64_t)head * p.q_hs;
  bf16x8 qb[A::kKs];
#pragma unroll
  for (int ks = 0; ks < A::kKs; ++ks) qb[ks] = any_q_operand<kSoftCap>(ld16(qrow + 16 * ks + 8 * h), p.logit_scale);
  const int qpos = p.positions[w.q0 + ltok];

  // kv index j is visible to some row iff j < lk and j + kv_pos_off <= the
  // tile's largest position
  int mx = row_ok ? qpos : INT_MIN, mn = row_ok ? qpos : INT_MAX;
  minmax32(mx, mn);
  if (lane == 0) {
    red_hi[wave] = mx;
    red_lo[wave] = mn;
  }
  __syncthreads();
  int qmax = red_hi[0], qmin = red_lo[0];
#pragma unroll
  for (int i = 1; i < kAnyWaves; ++i) {
    qmax = max(qmax, red_hi[i]);
    qmin = min(qmin, red_lo[i]);
  }
  const int64_t kv_hi64 = min((int64_t)w.lk, (int64_t)qmax - w.kv_pos_off + 1);
  const int kv_hi = kv_hi64 < 0 ? 0 : (int)kv_hi64;
  const int n_steps = (kv_hi + kAnyStep - 1) / kAnyStep;

  const int32_t* bt_row = p.block_tables + (int64_t)w.b * p.bt_stride;
  const int64_t head_off = (int64_t)w.kvh * p.head_stride;
  u32x4 kr[kPer], vr[kPer];
  // kPaged3: step_pages() reads the step's (up to) three page ids with
  // scalar loads, a step before its K / V loads, and turns them into scalar
  // row bases; a lane then finds its row with two compares and a select
  // (per chunk: no division by the page size, no block-table load, no 64-bit
  // multiply by the page stride).  For the next step to load: the in-page
  // offset of its first (clamped) token, and the element offsets of table
  // entries lp0 .. lp0 + 2 for this kv head; plain scalars, so that nothing
  // is placed in an array in memory.
  // The raw table entries are clamped and turned into row bases only when
  // the step is loaded (a step later): used at once, the scalar loads would
  // be waited for where they are issued.
  int sp_off0 = 0;
  int32_t sp_g0 = 0, sp_g1 = 0, sp_g2 = 0;  // raw table entries lp0 .. lp0 + 2
  auto step_pages = [&](int j0) __attribute__((always_inline)) {
    const int jc0 = min(j0, w.lk - 1);
    const int lp0 = __builtin_amdgcn_readfirstlane(jc0 / p.page_size);
    sp_off0 = __builtin_amdgcn_readfirstlane(jc0 - lp0 * p.page_size);
    // entries past the table row are never selected: the index is clamped
    const int last = p.pages_per_seq - 1;
    const __attribute__((address_space(4))) int32_t* c = (const __attribute__((address_space(4))) int32_t*)bt_row;
    sp_g0 = c[min(lp0, last)];
    sp_g1 = c[min(lp0 + 1, last)];
    sp_g2 = c[min(lp0 + 2, last)];
  };
  // (the entries come in by value: a select among captured references
  // became an indexed access to the closure, which put it in scratch memory)
  auto load3 = [&](int j0, int off0, int32_t g0, int32_t g1, int32_t g2) __attribute__((always_inline)) {
    // the entries clamped into the pool, as safe_page does
    auto base = [&](int32_t g) __attribute__((always_inline)) {
      const int32_t pg = g < 0 ? 0 : (g >= p.num_pages ? p.num_pages - 1 : g);
      return (int64_t)pg * p.page_stride + head_off;
    };
    const int64_t b0 = base(g0), b1 = base(g1), b2 = base(g2);
    const int jc0 = min(j0, w.lk - 1);
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = tid + kThreads * i;
      if (any_chunk_live<kStepChunks, kThreads, kPer>(i, c)) {
        const int t = c / A::kChunks;
        const int e = c - t * A::kChunks;
        // token min(j0 + t, lk - 1) = lp0 * page_size + x, x < 3 * page_size
        const int x = off0 + (min(j0 + t, w.lk - 1) - jc0);
        const int q = (x >= p.page_size ? 1 : 0) + (x >= 2 * p.page_size ? 1 : 0);
        const int64_t base = q == 0 ? b0 : (q == 1 ? b1 : b2);
        const int64_t off = base + (int64_t)(x - q * p.page_size) * p.slot_stride + 8 * e;
        kr[i] = ld16(p.k_cache + off);
        vr[i] = ld16(p.v_cache + off);
      }
    }
  };
  // Page sizes below 16 (!kPaged3): per lane and chunk.  kAhead: the page
  // ids of a step's chunks are read one step before its K / V loads
  // (pages()), so that no K / V load waits on its block-table read: with a
  // single workgroup per CU nothing else hides that second latency.
  // Otherwise load() reads them itself (fewer live registers).
  constexpr bool kAhead = any_pages_ahead(D);
  int32_t pg[kAhead ? kPer : 1];
  auto pages = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = tid + kThreads * i;
      if (any_chunk_live<kStepChunks, kThreads, kPer>(i, c)) {
        // tokens past the kv length read the last valid one (masked below)
        const int j = min(j0 + c / A::kChunks, w.lk - 1);
        pg[i] = safe_page(bt_row, j / p.page_size, p.num_pages);
      }
    }
  };
  auto load = [&](int j0) __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = tid + kThreads * i;
      if (any_chunk_live<kStepChunks, kThreads, kPer>(i, c)) {
        const int t = c / A::kChunks;
        const int e = c - t * A::kChunks;
        // tokens past the kv length read the last valid one (masked below)
        const int j = min(j0 + t, w.lk - 1);
        int32_t page;
        if constexpr (kAhead) page = pg[i];
        else page = safe_page(bt_row, j / p.page_size, p.num_pages);
        const int64_t off =
            (int64_t)page * p.page_stride + (int64_t)(j % p.page_size) * p.slot_stride + head_off + 8 * e;
        kr[i] = ld16(p.k_cache + off);
        vr[i] = ld16(p.v_cache + off);
      }
    }
  };
  auto store = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = tid + kThreads * i;
      if (any_chunk_live<kStepChunks, kThreads, kPer>(i, c)) {
        const int t = c / A::kChunks;
        const int e = c - t * A::kChunks;
        lds_st16(k_tile + t * A::kRow + 16 * e, kr[i]);
        lds_st16(v_tile + t * A::kVRow + 16 * e, vr[i]);
      }
    }
  };

  f32x16 acc[A::kDt];
#pragma unroll
  for (int dt = 0; dt < A::kDt; ++dt) acc[dt] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  // kPaged3 and kAhead: every step loads the next step's K / V and the page
  // ids of the one after, also past the last step (the token index is
  // clamped, so those loads read real rows, never used): loads under a
  // branch would make the compiler wait for them where the branch joins.
  if (n_steps > 0) {
    if constexpr (kPaged3) {
      step_pages(0);
      load3(0, sp_off0, sp_g0, sp_g1, sp_g2);
      step_pages(kAnyStep);
    } else {
      if constexpr (kAhead) pages(0);
      load(0);
      if constexpr (kAhead) pages(kAnyStep);
    }
  }
  // A step: step_head() stages its tiles, issues the next loads, computes its
  // masked logits into s and returns their row max; step_tail() takes P and PV.
  f32x16 s;
  auto step_head = [&](int st) __attribute__((always_inline)) {
    __syncthreads();  // every wave is done with the previous step's tiles
    store();
    __syncthreads();
    const int j0 = st * kAnyStep;
    if constexpr (kPaged3) {
      load3(j0 + kAnyStep, sp_off0, sp_g0, sp_g1, sp_g2);
      step_pages(j0 + 2 * kAnyStep);
    } else if constexpr (kAhead) {
      load(j0 + kAnyStep);
      pages(j0 + 2 * kAnyStep);
    } else if (st + 1 < n_steps) {
      load(j0 + kAnyStep);
    }
    s = f32x16{};
#pragma unroll
    for (int ks = 0; ks < A::kKs; ++ks)
      s = mfma32(as_bf16x8(lds_ld16(k_tile + n * A::kRow + 2 * (16 * ks + 8 * h))), qb[ks], s);
    if constexpr (kAnyWaves == 4) {
      // each K read four MFMAs ahead of the MFMA it feeds (left to itself
      // the compiler issued them one or two ahead: nothing else on the SIMD
      // hides the LDS latency)
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 4, 0);
#pragma unroll
      for (int i = 0; i < A::kKs; ++i) {
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (i + 4 < A::kKs) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) s[i] = any_logit<kSoftCap>(s[i], p.logit_scale, p.soft_cap);
    // a step below the length and below every row's causal limit needs no mask
    if (j0 + kAnyStep > w.lk || (int64_t)j0 + kAnyStep - 1 + w.kv_pos_off > qmin) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int j = j0 + 8 * (i >> 2) + 4 * h + (i & 3);
        s[i] = j < w.lk && (int64_t)j + w.kv_pos_off <= qpos ? s[i] : -INFINITY;
      }
    }
    float mx = s[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) mx = fmaxf(mx, s[i]);
    return max_xor32(mx);
  };
  auto step_tail = [&]() __attribute__((always_inline)) { any_p_pv<A::kDt, A::kVRow>(s, m_run, l_run, acc, v_tile, lane); };
  if constexpr (kAnyWaves == 4) {
    // O lives in AGPRs here (with one wave per SIMD the registers allow it),
    // and a rescale inside the loop made the compiler copy all of O into
    // VGPRs on every step; the loop is left for the (rare) rescale instead.
    int st = 0;
    while (st < n_steps) {
      float mx = step_head(st);
      while (!__any(mx > m_run + kAnySlack)) {
        step_tail();
        if (++st >= n_steps) break;
        mx = step_head(st);
      }
      if (st >= n_steps) break;
      any_lazy_rescale(mx, m_run, l_run, acc);
      step_tail();
      ++st;
    }
  } else {
    for (int st = 0; st < n_steps; ++st) {
      const float mx = step_head(st);
      if (__any(mx > m_run + kAnySlack)) any_lazy_rescale(mx, m_run, l_run, acc);
      step_tail();
    }
  }
  // a row that sees no key (its position precedes the sequence's first kv
  // position) is written as zeros
  const float l_tot = sum_xor32(l_run);
  const float inv = l_tot > 0.f ? 1.f / l_tot : 0.f;
  if (!row_ok) return;
  uint16_t* orow = p.out + (int64_t)(w.q0 + rtok) * p.o_ts + (int64_t)head * p.o_hs;
#pragma unroll
  for (int dt = 0; dt < A::kDt; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = 32 * dt + 8 * g4 + 4 * h;
      if (d0 < D)
        *reinterpret_cast<u32x2*>(orow + d0) =
            u32x2{pack_bf16x2(acc[dt][4 * g4] * inv, acc[dt][4 * g4 + 1] * inv),
                  pack_bf16x2(acc[dt][4 * g4 + 2] * inv, acc[dt][4 * g4 + 3] * inv)};
    }
}

// Rows of tokens [4 zb, 4 zb + 4) that no prefill item writes (outside every
// sequence or at offset >= max_seqlen_q): zeros, one wave per token.
__global__ void __launch_bounds__(256)
prefill_any_zero_kernel(PrefillParams p, int head_dim) {
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= p.num_tokens) return;
  bool covered = false;
  if (p.batch > 0 && t >= p.cu_q[0] && t < p.cu_q[p.batch]) {
    int lo = 0, hi = p.batch;  // invariant: cu_q[lo] <= t < cu_q[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (p.cu_q[mid] <= t) lo = mid;
      else hi = mid;
    }
    covered = t - p.cu_q[lo] < p.max_seqlen_q;
  }
  if (covered) return;
  const int per_head = head_dim / 8;
  for (int c = lane; c < p.num_heads * per_head; c += 64) {
    const int hh = c / per_head;
    st16(p.out + t * p.o_ts + (int64_t)hh * p.o_hs + 8 * (c - hh * per_head), u32x4{0u, 0u, 0u, 0u});
  }
}

// ---- decode: one wave per (sequence, chunk, kv head, block of 32 q heads),
// grid order item = ((b * n_chunks + chunk) * Hkv + kv head) * hblocks +
// block.  K and V rows are read with whole-row 16-byte loads (8 lanes per
// 128 bytes) and staged row-major in the wave's K and V tiles.
// The chunk's partial (O unnormalised, the log2 max and the sum per head)
// goes to the workspace; decode_any_merge_kernel combines the chunks of
// every sequence.
// Whole 128-byte lines per K / V row (head sizes multiple of 64): the
// generic decode can stream its K / V loads past the caches.
__host__ __device__ constexpr bool any_decode_streamable(int d) { return d % 64 == 0; }
// Tokens per load batch of the generic decode: up to head size 64 two
// 32-token steps (more bytes in flight per wave for one wave less per SIMD).
__host__ __device__ constexpr int any_decode_batch(int d) { return d <= 64 ? 2 * kAnyStep : kAnyStep; }

// Eight 1-byte codes of type `code` (uniform over the launch) to bf16, exactly.
__device__ __forceinline__ u32x4 codes8_to_bf16x8_rt(const u32x2& c, int code) {
  if (code == kCodeI8) return codes8_to_bf16x8<kCodeI8>(c);
  if (code == kCodeU8) return codes8_to_bf16x8<kCodeU8>(c);
  return codes8_to_bf16x8<kCodeE4M3>(c);
}

// kStream: K / V loads non-temporal (rows of whole 128-byte lines, each
// read by one item: one block of q heads per kv head).
// kQuant: the pages hold 1-byte codes of type `code` (p.k8 / p.v8, strides in
// bytes) with per-token scales (p.k_scales / p.v_scales).  Eight codes per
// lane and chunk are loaded (8 bytes) and widened to bf16 exactly as they are
// staged, so the tiles and the MFMAs are those of bf16 pages; the step's
// scales are staged beside them.  As in the tuned decode, the logit of token
// j is (q . k_j) * k_scale_j, and P is rounded to bf16 as p * v_scale_j.
// kPaged3: pages of at least half a load batch (any_decode_batch), so a
// batch (clamped to the chunk) lies in at most three consecutive table
// entries, paged once per batch with scalar loads as in the prefill.
template <int D, bool kSoftCap, bool kStream, bool kQuant, bool kPaged3>
__global__ void __launch_bounds__(64)
decode_any_kernel(DecodeParams p, int code) {
  using A = AnyDims<D>;
  // Up to head size 64 a load batch is two 32-token steps (more bytes in
  // flight per wave for one wave less per SIMD); the next batch is loaded
  // while this one computes, up to the head size whose registers still allow
  // it without spills.
  constexpr int kTok = any_decode_batch(D);         // tokens per load batch
  constexpr int kSub = kTok / kAnyStep;
  constexpr int kPer = kTok * A::kChunks / 64;      // chunks of K (and of V) per lane and batch
  constexpr bool kPrefetch = kSoftCap ? D <= 192 : D <= 224;
  __shared__ __attribute__((aligned(16))) char k_tile_g[kTok * A::kRow];
  __shared__ __attribute__((aligned(16))) char v_tile_g[kTok * A::kVRow + 32];
  __shared__ __attribute__((aligned(16))) float ksc_g[kQuant ? kTok : 4], vsc_g[kQuant ? kTok : 4];
  lds_char* k_tile = (lds_char*)k_tile_g;
  lds_char* v_tile = (lds_char*)v_tile_g;
  const int lane = threadIdx.x;
  const int n = lane & 31;
  const int h = lane >> 5;
  const int hkv = p.num_kv_heads;
  const int vheads = hkv * p.hblocks;
  int item;
  if (p.plan) {
    // the decode work list (pairs by token count, most first): XCD x = bid
    // % 8 takes ranks x, x + 8, ..., all kv heads (and q-head blocks) of a
    // rank in a row, so the XCDs get near-equal work and the kv heads of a
    // token row are read by one XCD together
    const int k = blockIdx.x >> 3;
    const int kr = k / vheads;
    const int r = 8 * kr + (blockIdx.x & 7);
    if (r >= p.plan[0]) return;
    item = p.plan[kDecodePlanHeader + r] * vheads + (k - kr * vheads);
  } else {
    // contiguous item ranges per XCD: the kv heads of a (sequence, chunk),
    // adjacent slices of each token row, are read by one XCD together
    item = xcd_grouped_item(blockIdx.x, gridDim.x);
  }
  const int vh = item % vheads;
  const int rest = item / vheads;
  const int kvh = vh / p.hblocks;
  const int qc0 = 32 * (vh - kvh * p.hblocks);  // first q head (within the group) of this item
  const int g_end = min(p.group, qc0 + 32);
  const int chunk = rest % p.n_chunks;
  const int b = rest / p.n_chunks;
  if (!decode_has_row(p, b)) return;
  // lengths past the block table's span are clamped to it
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  const int t0 = chunk * p.chunk;
  if (t0 >= len) return;  // the merge writes what this chunk would have held
  const int t1 = min(t0 + p.chunk, len);
  const bool live = qc0 + n < g_end;
  const uint16_t* qrow =
      p.q + decode_row(p, b) * p.q_bs + (int64_t)(kvh * p.group + qc0 + (live ? n : 0)) * p.q_hs;
  bf16x8 qb[A::kKs];
#pragma unroll
  for (int ks = 0; ks < A::kKs; ++ks) {
    const u32x4 v = ld16(qrow + 16 * ks + 8 * h);
    qb[ks] = as_bf16x8(live ? v : u32x4{0u, 0u, 0u, 0u});  // unscaled: the logits are scaled in f32
  }
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int64_t head_off = (int64_t)kvh * p.head_stride;
  using Raw = std::conditional_t<kQuant, u32x2, u32x4>;
  Raw kr[kPer], vr[kPer];
  float ksr = 0.f, vsr = 0.f;  // (kQuant) scales of token lane % kTok of the batch
  auto load = [&](int j0) __attribute__((always_inline)) {
    // (kPaged3) the batch's first (clamped) token is table entry lp0, offset
    // off0; entries lp0 .. lp0 + 2 as scalar element (and scale) offsets
    const int jc0 = min(j0, t1 - 1);
    int off0 = 0;
    int64_t b0 = 0, b1 = 0, b2 = 0, s0 = 0, s1 = 0, s2 = 0;
    if constexpr (kPaged3) {
      const int lp0 = __builtin_amdgcn_readfirstlane(jc0 / p.page_size);
      off0 = __builtin_amdgcn_readfirstlane(jc0 - lp0 * p.page_size);
      const int last = p.pages_per_seq - 1;  // entries past the row are never selected
      const int64_t g0 = safe_page_scalar(bt_row, min(lp0, last), p.num_pages);
      const int64_t g1 = safe_page_scalar(bt_row, min(lp0 + 1, last), p.num_pages);
      const int64_t g2 = safe_page_scalar(bt_row, min(lp0 + 2, last), p.num_pages);
      b0 = g0 * p.page_stride + head_off;
      b1 = g1 * p.page_stride + head_off;
      b2 = g2 * p.page_stride + head_off;
      if constexpr (kQuant) {
        const int64_t sh = (int64_t)kvh * p.sc_head_stride;
        s0 = g0 * p.sc_page_stride + sh;
        s1 = g1 * p.sc_page_stride + sh;
        s2 = g2 * p.sc_page_stride + sh;
      }
    }
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = lane + 64 * i;
      const int t = c / A::kChunks;
      const int e = c - t * A::kChunks;
      // tokens past the chunk read its last token (masked below)
      const int j = min(j0 + t, t1 - 1);
      int64_t off;
      if constexpr (kPaged3) {
        const int x = off0 + (j - jc0);  // j = lp0 * page_size + x, x < 3 * page_size
        const int q = (x >= p.page_size ? 1 : 0) + (x >= 2 * p.page_size ? 1 : 0);
        off = (q == 0 ? b0 : (q == 1 ? b1 : b2)) + (int64_t)(x - q * p.page_size) * p.slot_stride + 8 * e;
      } else {
        off = (int64_t)safe_page(bt_row, j / p.page_size, p.num_pages) * p.page_stride +
              (int64_t)(j % p.page_size) * p.slot_stride + head_off + 8 * e;
      }
      if constexpr (kQuant) {
        kr[i] = *reinterpret_cast<const u32x2*>(p.k8 + off);
        vr[i] = *reinterpret_cast<const u32x2*>(p.v8 + off);
      } else if constexpr (kStream) {
        kr[i] = ld16_stream(p.k_cache + off);
        vr[i] = ld16_stream(p.v_cache + off);
      } else {
        kr[i] = ld16(p.k_cache + off);
        vr[i] = ld16(p.v_cache + off);
      }
    }
    if constexpr (kQuant) {
      // past the chunk: the scales of its last token (a real one; those
      // tokens are masked, so their p is 0)
      const int j = min(j0 + (lane & (kTok - 1)), t1 - 1);
      int64_t si;
      if constexpr (kPaged3) {
        const int x = off0 + (j - jc0);
        const int q = (x >= p.page_size ? 1 : 0) + (x >= 2 * p.page_size ? 1 : 0);
        si = (q == 0 ? s0 : (q == 1 ? s1 : s2)) + (x - q * p.page_size);
      } else {
        si = (int64_t)safe_page(bt_row, j / p.page_size, p.num_pages) * p.sc_page_stride +
             (int64_t)kvh * p.sc_head_stride + j % p.page_size;
      }
      ksr = p.k_scales[si];
      vsr = p.v_scales[si];
    }
  };

  f32x16 acc[A::kDt];
#pragma unroll
  for (int dt = 0; dt < A::kDt; ++dt) acc[dt] = f32x16{};
  float m_run = -INFINITY, l_run = 0.f;
  if constexpr (kPrefetch) load(t0);
  for (int j0 = t0; j0 < t1; j0 += kTok) {
    if constexpr (!kPrefetch) load(j0);
    __syncthreads();  // the previous step's tile reads are done
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
      const int c = lane + 64 * i;
      const int t = c / A::kChunks;
      const int e = c - t * A::kChunks;
      if constexpr (kQuant) {
        lds_st16(k_tile + t * A::kRow + 16 * e, codes8_to_bf16x8_rt(kr[i], code));
        lds_st16(v_tile + t * A::kVRow + 16 * e, codes8_to_bf16x8_rt(vr[i], code));
      } else {
        lds_st16(k_tile + t * A::kRow + 16 * e, kr[i]);
        lds_st16(v_tile + t * A::kVRow + 16 * e, vr[i]);
      }
    }
    if constexpr (kQuant) {
      if (lane < kTok) {
        ksc_g[lane] = ksr;
        vsc_g[lane] = vsr;
      }
    }
    __syncthreads();
    if constexpr (kPrefetch) {
      if (j0 + kTok < t1) load(j0 + kTok);
    }
#pragma unroll
    for (int sub = 0; sub < kSub; ++sub) {
      const int js = j0 + kAnyStep * sub;
      if (sub == 0 || js < t1) {  // uniform: a batch's second step may hold no token
        f32x16 s = {};
#pragma unroll
        for (int ks = 0; ks < A::kKs; ++ks)
          s = mfma32(as_bf16x8(lds_ld16(k_tile + (kAnyStep * sub + n) * A::kRow + 2 * (16 * ks + 8 * h))), qb[ks],
                     s);
        // (kQuant) scales of the lane's 16 tokens 8(i/4) + 4h + i%4 of the step
        f32x16 ksc = {}, vsc = {};
        if constexpr (kQuant) {
#pragma unroll
          for (int q4 = 0; q4 < 4; ++q4) {
            const int o = kAnyStep * sub + 8 * q4 + 4 * h;
            const f32x4 a = __builtin_bit_cast(f32x4, lds_ld16((const lds_char*)ksc_g + 4 * o));
            const f32x4 c = __builtin_bit_cast(f32x4, lds_ld16((const lds_char*)vsc_g + 4 * o));
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              ksc[4 * q4 + r] = a[r];
              vsc[4 * q4 + r] = c[r];
            }
          }
        }
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          const int j = js + 8 * (i >> 2) + 4 * h + (i & 3);
          s[i] = j < t1 ? any_logit_f32<kSoftCap>(kQuant ? s[i] * ksc[i] : s[i], p.logit_scale, p.soft_cap)
                        : -INFINITY;
        }
        any_softmax_pv<A::kDt, A::kVRow, kQuant>(s, m_run, l_run, acc, v_tile + kAnyStep * sub * A::kVRow,
                                                       lane, vsc);
      }
    }
  }
  const float l_tot = sum_xor32(l_run);
  if (!live) return;
  const int64_t part = (((int64_t)b * hkv + kvh) * p.n_chunks + chunk) * p.group + qc0 + n;
  float* dst = p.ws_o + part * D;
#pragma unroll
  for (int dt = 0; dt < A::kDt; ++dt)
#pragma unroll
    for (int g4 = 0; g4 < 4; ++g4) {
      const int d0 = 32 * dt + 8 * g4 + 4 * h;
      if (d0 < D)
        *reinterpret_cast<f32x4*>(dst + d0) =
            f32x4{acc[dt][4 * g4], acc[dt][4 * g4 + 1], acc[dt][4 * g4 + 2], acc[dt][4 * g4 + 3]};
    }
  if (h == 0) {
    p.ws_ml[2 * part] = m_run;
    p.ws_ml[2 * part + 1] = l_tot;
  }
}

// One wave per (sequence, q head): out = sum_c o_c 2^(m_c - M) / sum_c l_c
// 2^(m_c - M) over the sequence's chunks; length 0 gives zeros.  Lane l
// finishes the d pairs 2l and 2l + 128.
__global__ void __launch_bounds__(256)
decode_any_merge_kernel(DecodeParams p, int head_dim) {
  const int lane = threadIdx.x & 63;
  const int64_t pair = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (pair >= (int64_t)p.batch * p.num_heads) return;
  const int b = (int)(pair / p.num_heads);
  const int hd = (int)(pair - (int64_t)b * p.num_heads);
  if (!decode_has_row(p, b)) return;
  const int kvh = hd / p.group;
  const int qi = hd - kvh * p.group;
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  const int nc = len > 0 ? min((len + p.chunk - 1) / p.chunk, p.n_chunks) : 0;
  const int64_t base = ((int64_t)b * p.num_kv_heads + kvh) * p.n_chunks;
  float mmax = -INFINITY;
  for (int c = 0; c < nc; ++c) mmax = fmaxf(mmax, p.ws_ml[2 * ((base + c) * p.group + qi)]);
  float o[2][2] = {{0.f, 0.f}, {0.f, 0.f}};
  float lsum = 0.f;
  for (int c = 0; c < nc; ++c) {
    const int64_t part = (base + c) * p.group + qi;
    const float wgt = fast_exp2(p.ws_ml[2 * part] - mmax);
    lsum += p.ws_ml[2 * part + 1] * wgt;
#pragma unroll
    for (int k = 0; k < 2; ++k) {
      const int d = 2 * lane + 128 * k;
      if (d < head_dim) {
        const float2 v = *reinterpret_cast<const float2*>(p.ws_o + part * head_dim + d);
        o[k][0] += v.x * wgt;
        o[k][1] += v.y * wgt;
      }
    }
  }
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  uint16_t* orow = p.out + decode_row(p, b) * p.out_bs + (int64_t)hd * p.out_hs;
#pragma unroll
  for (int k = 0; k < 2; ++k) {
    const int d = 2 * lane + 128 * k;
    if (d < head_dim) *reinterpret_cast<uint32_t*>(orow + d) = pack_bf16x2(o[k][0] * inv, o[k][1] * inv);
  }
}

#define PA_ANY_DIMS(X) \
  X(16) X(32) X(48) X(64) X(80) X(96) X(112) X(144) X(160) X(176) X(192) X(208) X(224) X(240) X(256)

}  // namespace

bool any_head_dim(int head_dim) {
  switch (head_dim) {
#define PA_ANY_CASE(d) case d:
    PA_ANY_DIMS(PA_ANY_CASE)
#undef PA_ANY_CASE
    return true;
    default:
      return false;
  }
}

int prefill_any_launch(const char* name, const PrefillParams& prm, int head_dim, hipStream_t s) {
  PrefillParams p = prm;
  const int waves = any_prefill_waves(head_dim);
  if (p.group > 32 * waves)
    return fail(PA_ERR_UNSUPPORTED, "%s: %d q heads per kv head not supported at head_dim %d (max %d)", name,
                p.group, head_dim, 32 * waves);
  p.plan = nullptr;
  p.pool = nullptr;
  p.tile_tokens = 32 * waves / p.group;
  p.n_qtiles = (p.max_seqlen_q + p.tile_tokens - 1) / p.tile_tokens;
  if (p.num_tokens > 0) {
    prefill_any_zero_kernel<<<dim3((unsigned)((p.num_tokens + 3) / 4)), dim3(256), 0, s>>>(p, head_dim);
    const int rc = launch_status(name);
    if (rc) return rc;
  }
  if (p.batch == 0 || p.max_seqlen_q == 0) return PA_OK;
  const int64_t items = (int64_t)p.n_qtiles * p.batch * p.num_kv_heads;
  if (items > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "%s: grid of %lld workgroups too large", name, (long long)items);
  const dim3 g((unsigned)items), blk(64 * waves);
  const bool cap = p.soft_cap > 0.f;
  const bool paged3 = p.page_size >= 16;
  switch (head_dim) {
#define PA_ANY_LAUNCH(d)                                                                       \
  case d:                                                                                      \
    if (cap && paged3) prefill_any_kernel<d, true, true><<<g, blk, 0, s>>>(p);                 \
    else if (cap) prefill_any_kernel<d, true, false><<<g, blk, 0, s>>>(p);                     \
    else if (paged3) prefill_any_kernel<d, false, true><<<g, blk, 0, s>>>(p);                  \
    else prefill_any_kernel<d, false, false><<<g, blk, 0, s>>>(p);                             \
    break;
    PA_ANY_DIMS(PA_ANY_LAUNCH)
#undef PA_ANY_LAUNCH
    default:
      return fail(PA_ERR_UNSUPPORTED, "%s: head_dim %d not supported", name, head_dim);
  }
  return launch_status(name);
}

int decode_any_launch(const char* name, const DecodeParams& prm, int head_dim, hipStream_t s, int code) {
  DecodeParams p = prm;
  p.hblocks = (p.group + 31) / 32;
  const int64_t pairs = (int64_t)p.batch * p.n_chunks;
  const int64_t vheads = (int64_t)p.num_kv_heads * p.hblocks;
  // with the work list (p.plan, from pa_decode), XCD x runs ranks x, x + 8, ...
  const int64_t items = p.plan ? (pairs + 7) / 8 * 8 * vheads : pairs * vheads;
  if (items > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "%s: grid of %lld workgroups too large", name, (long long)items);
  if (items > 0) {
    const dim3 g((unsigned)items), blk(64);
    const bool cap = p.soft_cap > 0.f;
    // one block of q heads per kv head: every K / V row is read once
    const bool stream = p.hblocks == 1;
    const bool quant = code >= 0;
    // a load batch spans at most three pages
    const bool paged3 = 2 * p.page_size >= any_decode_batch(head_dim);
    switch (head_dim) {
#define PA_ANY_DECODE(d, P)                                                                              \
    if (quant && cap) decode_any_kernel<d, true, false, true, P><<<g, blk, 0, s>>>(p, code);             \
    else if (quant) decode_any_kernel<d, false, false, true, P><<<g, blk, 0, s>>>(p, code);              \
    else if (cap && stream) decode_any_kernel<d, true, any_decode_streamable(d), false, P><<<g, blk, 0, s>>>(p, 0);  \
    else if (cap) decode_any_kernel<d, true, false, false, P><<<g, blk, 0, s>>>(p, 0);                   \
    else if (stream) decode_any_kernel<d, false, any_decode_streamable(d), false, P><<<g, blk, 0, s>>>(p, 0); \
    else decode_any_kernel<d, false, false, false, P><<<g, blk, 0, s>>>(p, 0);
#define PA_ANY_LAUNCH(d)     \
  case d:                    \
    if (paged3) {            \
      PA_ANY_DECODE(d, true) \
    } else {                 \
      PA_ANY_DECODE(d, false)\
    }                        \
    break;
      PA_ANY_DIMS(PA_ANY_LAUNCH)
      PA_ANY_LAUNCH(128)  // more than 16 q heads per kv head over bf16 pages (pa_decode)
#undef PA_ANY_LAUNCH
#undef PA_ANY_DECODE
      default:
        return fail(PA_ERR_UNSUPPORTED, "%s: head_dim %d not supported", name, head_dim);
    }
    const int rc = launch_status(name);
    if (rc) return rc;
  }
  const int64_t rows = (int64_t)p.batch * p.num_heads;  // (sequence, q head) pairs
  if (rows > 0) {
    decode_any_merge_kernel<<<dim3((unsigned)((rows + 3) / 4)), dim3(256), 0, s>>>(p, head_dim);
    return launch_status(name);
  }
  return PA_OK;
}

}  // namespace pa
