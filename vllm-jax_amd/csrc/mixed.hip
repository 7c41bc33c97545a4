// One launch for a mixed batch of decode and prefill sequences on gfx950.
//
// The reference runs a scheduler step as two jitted calls, decode then
// prefill, each padded to a power-of-two bucket (model_runner.py:310-333,
// 243-255, 286-292).  Here one kernel covers both halves of the batch with
// no padding: sequences 0 .. num_decodes-1 are decode sequences (one q row
// each, split-K over their kv length), the rest are prefill sequences (ragged
// causal q tiles).  Every workgroup has 512 threads and the prefill item's
// 128 KiB of LDS; the grid is cut into regions:
//
//   [0, r1)    prefill items of the longest q-tile levels
//   [r1, r2)   decode items (sequence, 4096-token chunk, kv head), 8 waves
//              each, numbered XCD-grouped like decode_split_kernel
//   [r2, r3)   the remaining prefill items
//   [r3, r4)   zero pass: 512 token rows per workgroup, rows no item writes
//
// The hardware starts workgroups in index order, so the costliest items
// (long causal q tiles) start first, the decode chunks (HBM streams) run
// while those tiles still occupy other CUs, and short tiles fill the tail.
// A decode item combines its 8 waves through the LDS of the prefill ring,
// which it does not otherwise use.  When a decode sequence can span more
// than one chunk, decode_merge_kernel follows as a second launch.
//
// Large steps instead take their items from a work list built by
// mixed_plan_kernel (a launch of one workgroup before the step): decode
// chunks and prefill q tiles priced on one measured time scale and sorted,
// costliest first, then dealt over the XCDs; the zero pass follows them.
#include <algorithm>

#include "any_head.h"
#include "decode_impl.h"
#include "prefill_impl.h"

namespace pa {

constexpr int kMixedDecodeWaves = kWaves;     // a decode item uses the whole workgroup
constexpr int kZeroRowsPerBlock = kThreads;   // one row per thread in the zero pass
#ifndef PA_MIXED_COST_RATIO
#define PA_MIXED_COST_RATIO 2.6f
#endif
// Time of a 64-token prefill tile (256 q rows on the MFMA) over the time of
// a 64-token decode step of one workgroup (HBM stream), both measured on
// MI355X: prefill levels whose items cost more than a decode chunk go first.
constexpr float kPrefillOverDecodeTile = PA_MIXED_COST_RATIO;

// Item costs of the work list in units of 1/8 us, from per-workgroup
// timestamps of the Qwen3-0.6B mixed step on MI355X: a decode item takes
// 8.0 us + 1.03 us per 64 tokens, a prefill item 11.2 us + 1.86 us per
// 64-token kv tile.
constexpr int kDecodeItemCost = 64;
constexpr int kDecodeStepCost = 2;  // per 16-token step
constexpr int kPrefillItemCost = 90;
constexpr int kPrefillTileCost = 15;
constexpr int kMixedPlanThreads = 1024;
constexpr int kMixedPlanBins = 4096;
constexpr int kMixedPlanMaxPrefill = 2048;          // prefill sequences the planner keeps in LDS
constexpr int64_t kMixedPlanMinItems = 2048;        // workgroups from which pa_mixed builds a work list

struct MixedParams {
  PrefillParams pre;  // the prefill sequences (arrays start at entry num_decodes)
  DecodeParams dec;   // the decode sequences (entries 0 .. num_decodes-1)
  // Work list (may be null): plan[0] = entries, records of 8 ints from
  // kPlanHeader on, costliest first: {0, b, qt, q0, lq_rows, lk, kv_pos_off}
  // for a prefill q tile, {1, b, chunk, hb} for block hb of 16 q heads (of
  // every kv head) of a decode chunk.  With a list,
  // [0, r3) are list items and [r3, r4) the zero pass.
  const int32_t* plan;
  int32_t r1, r2, r3, r4;
  int32_t pre_head;     // prefill items in region [0, r1)
  int32_t n_dec_items;  // decode items in region [r1, r2)
  // zero pass
  const int32_t* cu_q;
  int32_t batch, num_decodes, num_tokens, max_seqlen_q, num_heads;
  uint16_t* out;
  int64_t o_ts, o_hs;
};

// Rows of tokens [512 zb, 512 zb + 512) that no item writes: outside every
// sequence, past the first row of a decode sequence, or at offset >=
// max_seqlen_q in a prefill sequence.
__device__ __forceinline__ void mixed_zero_rows(const MixedParams& m, int zb) {
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int64_t base = (int64_t)zb * kZeroRowsPerBlock + 64 * wave;
  const int64_t t = base + lane;
  bool need = false;
  if (t < m.num_tokens) {
    bool covered = false;
    if (t >= m.cu_q[0] && t < m.cu_q[m.batch]) {
      int lo = 0, hi = m.batch;  // invariant: cu_q[lo] <= t < cu_q[hi]
      while (hi - lo > 1) {
        const int mid = (lo + hi) >> 1;
        if (m.cu_q[mid] <= t) lo = mid;
        else hi = mid;
      }
      const int64_t off = t - m.cu_q[lo];
      covered = lo < m.num_decodes ? off == 0 : off < m.max_seqlen_q;
    }
    need = !covered;
  }
  uint64_t todo = __builtin_amdgcn_ballot_w64(need);
  const int chunks = m.num_heads * (kPHeadDim / 8);
  while (todo) {
    const int l = __builtin_ctzll(todo);
    todo &= todo - 1;
    uint16_t* row = m.out + (base + l) * m.o_ts;
    for (int c = lane; c < chunks; c += 64)
      st16(row + (int64_t)(c / (kPHeadDim / 8)) * m.o_hs + 8 * (c % (kPHeadDim / 8)), u32x4{0, 0, 0, 0});
  }
}

// Work list of a mixed step (one workgroup).  Decode pairs (sequence b,
// chunk c) come first in the index space, then prefill pairs (sequence b,
// q tile qt); a pair is listed when it has work (chunk 0 of a decode
// sequence always: it writes the zeros of an empty one).  Counting sort by
// cost, largest first.
__global__ void __launch_bounds__(kMixedPlanThreads)
mixed_plan_kernel(MixedParams m, int32_t* __restrict__ plan) {
  __shared__ int32_t hist[kMixedPlanBins];
  __shared__ int4 seqs[kMixedPlanMaxPrefill];
  __shared__ int32_t lag[kMixedPlanMaxPrefill];
  __shared__ int32_t scan[kMixedPlanThreads];
  const int tid = threadIdx.x;
  const PrefillParams& pp = m.pre;
  const DecodeParams& dp = m.dec;
  for (int i = tid; i < kMixedPlanBins; i += kMixedPlanThreads) hist[i] = 0;
  for (int b = tid; b < pp.batch; b += kMixedPlanThreads) prefill_seq_geometry(pp, b, seqs[b], lag[b]);
  __syncthreads();
  const int nc = dp.n_chunks, nq = pp.n_qtiles, hb = dp.hblocks;
  const int dec_pairs = dp.batch * nc * hb;
  const int pairs = dec_pairs + pp.batch * nq;
  const int span = dp.pages_per_seq * dp.page_size;
  auto bin_of = [&](int i) -> int {  // 0: nothing to do
    int cost;
    if (i < dec_pairs) {
      const int bc = i / hb, b = bc / nc, c = bc - b * nc;
      const int t0 = c * dp.chunk;
      const int len = min(dp.lengths[b], span);
      if (t0 >= len && c > 0) return 0;
      const int steps = t0 >= len ? 0 : (min(len - t0, dp.chunk) + kDecodeStep - 1) / kDecodeStep;
      cost = kDecodeItemCost + kDecodeStepCost * steps;
    } else {
      const int j = i - dec_pairs, b = j / nq;
      const int tiles = prefill_pair_tiles(seqs[b], lag[b], j - b * nq, pp.tile_tokens);
      if (tiles < 0) return 0;
      cost = kPrefillItemCost + kPrefillTileCost * tiles;
    }
    return min(cost, kMixedPlanBins - 1);
  };
  for (int64_t ii = tid; ii < pairs; ii += kMixedPlanThreads) {
    const int i = (int)ii;
    const int c = bin_of(i);
    if (c) atomicAdd(&hist[c], 1);
  }
  __syncthreads();
  constexpr int kPer = kMixedPlanBins / kMixedPlanThreads;  // thread t owns bins from the top
  int cnt[kPer], local = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    cnt[j] = hist[kMixedPlanBins - 1 - (kPer * tid + j)];
    local += cnt[j];
  }
  int count;
  int run = block_exclusive_scan<kMixedPlanThreads>(local, scan, count);
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    hist[kMixedPlanBins - 1 - (kPer * tid + j)] = run;  // first rank of the bin
    run += cnt[j];
  }
  __syncthreads();
  for (int64_t ii = tid; ii < pairs; ii += kMixedPlanThreads) {
    const int i = (int)ii;
    const int c = bin_of(i);
    if (!c) continue;
    int32_t* r = plan + kPlanHeader + 8 * atomicAdd(&hist[c], 1);
    if (i < dec_pairs) {
      const int bc = i / hb, b = bc / nc;
      st16(r, u32x4{1u, (uint32_t)b, (uint32_t)(bc - b * nc), (uint32_t)(i - bc * hb)});
      st16(r + 4, u32x4{0u, 0u, 0u, 0u});
    } else {
      const int j = i - dec_pairs, b = j / nq;
      const int4 g = seqs[b];
      st16(r, u32x4{0u, (uint32_t)b, (uint32_t)(j - b * nq), (uint32_t)g.x});
      st16(r + 4, u32x4{(uint32_t)g.y, (uint32_t)g.z, (uint32_t)g.w, 0u});
    }
  }
  if (tid == 0) plan[0] = count;
}

template <bool kSoftCap, int kPagingP, bool kAlignedD, int kIdsD>
__global__ void __launch_bounds__(kThreads, 1)
mixed_kernel(MixedParams m) {
  const int bid = blockIdx.x;
  if (bid >= m.r3) {
    mixed_zero_rows(m, bid - m.r3);
    return;
  }
  // one call site each for the decode item and the prefill item (both are large)
  int dec = -1;
  PrefillWork w;
  bool pre = false;
  if (m.plan) {
    // With num_kv_heads % 8 == 0, XCD x = bid % 8 walks the whole list and
    // takes kv head 8j + ((x - b) mod 8) of every entry, as the prefill work
    // list does: every XCD sees the same cost sequence, and a (sequence, kv
    // head) stays on one XCD, so a prefill sequence's q tiles in flight share
    // that XCD's L2 (Qwen3-0.6B step 371 -> 361 us, same process).
    // Otherwise XCD x takes ranks x, x + 8, ... with all kv heads of a rank
    // in a row.
    const int hkv = m.pre.num_kv_heads;
    int r, hsub = 0, h = 0;
    const bool by_xcd = (hkv & 7) == 0;
    if (by_xcd) {
      const int per = hkv >> 3;
      const int k = bid >> 3;
      r = k / per;
      hsub = k - r * per;
    } else {
      const int k = bid >> 3;
      const int kr = k / hkv;
      r = 8 * kr + (bid & 7);
      h = k - kr * hkv;
    }
    const __attribute__((address_space(4))) int32_t* pl = (const __attribute__((address_space(4))) int32_t*)m.plan;
    const int count = pl[0];
    const __attribute__((address_space(4))) int32_t* e = pl + kPlanHeader + 8 * r;  // room for every rank
    const int kind = e[0], b = e[1], sub = e[2];
    if (r >= count) return;  // uniform over the workgroup
    if (by_xcd) h = 8 * hsub + (((bid & 7) - b) & 7);
    if (kind) {
      dec = ((b * m.dec.n_chunks + sub) * hkv + h) * m.dec.hblocks + e[3];
    } else {
      w = PrefillWork{b, sub, h, e[3], e[4], e[5], e[6]};
      pre = true;
    }
  } else if (bid >= m.r1 && bid < m.r2) {
    const int item = xcd_grouped_item(bid - m.r1, m.r2 - m.r1);
    if (item >= m.n_dec_items) return;
    dec = item;
  } else {
    const int pre_bid = bid < m.r1 ? bid : m.pre_head + (bid - m.r2);
    if (bid < m.r1 && bid >= m.pre_head) return;  // padding of region 1
    pre = prefill_resolve(m.pre, pre_bid, w);
  }
  if (dec >= 0) {
    // [8 waves][16][d] floats fill the K ring exactly; m and l go to the V ring
    float* red_o = reinterpret_cast<float*>(&k_lds[0][0]);
    float* red_m = reinterpret_cast<float*>(&v_lds[0][0]);
    decode_item<kMixedDecodeWaves, kAlignedD, kSoftCap, false, false, kCodeE4M3, kIdsD>(m.dec, dec, red_o, red_m,
                                                                                        red_m + 16 * kMixedDecodeWaves);
    return;
  }
  if (pre) prefill_run<kSoftCap, kPagingP>(m.pre, w);
}

static_assert(sizeof(float) * kMixedDecodeWaves * 16 * kPHeadDim <= sizeof(uint16_t) * kStages * kTileElems,
              "decode combine must fit the K ring");

// Tokens per decode item (a multiple of the 16-token step): eight waves take
// up to twice the chunk of the four-wave decode kernel.  With 16-aligned pages
// the chunk is the whole pages that fit 4096 tokens: up to 64 of them (one
// page id per lane) from 64-token pages on, up to 256 below (four per lane:
// 256 pages of 16 tokens, 128 of 32, 85 of 48).  Pages above 4096 tokens get
// 4096-token chunks inside one page (the aligned decode item walks a chunk
// that starts inside a page).
static int mixed_decode_chunk(int page_size) {
  constexpr int kMax = 4096;
  if (page_size % kDecodeStep != 0 || page_size >= kMax) return kMax;
  return (kMax / page_size) * page_size;
}

static int mixed_decode_chunks(int32_t pages_per_seq, int32_t page_size) {
  const int64_t max_tokens = (int64_t)pages_per_seq * page_size;
  const int chunk = mixed_decode_chunk(page_size);
  return (int)((max_tokens + chunk - 1) / chunk);
}

static int64_t round8(int64_t x) { return (x + 7) & ~(int64_t)7; }

}  // namespace pa

using namespace pa;

// Decode partials (none when every decode sequence fits one chunk), then at
// a 256-byte boundary the work list: a header and 8 ints per pair, the pair
// count rounded up to 8.
static size_t mixed_partials_bytes(int32_t num_decodes, int32_t num_heads, int32_t head_dim, int chunks) {
  if (num_decodes <= 0 || chunks <= 1) return 0;  // every decode sequence is finished inside its item
  return ((size_t)num_decodes * num_heads * chunks * ((size_t)head_dim + 2) * sizeof(float) + 255) / 256 * 256;
}

// Decode pairs (sequence, chunk, block of 16 q heads) and prefill pairs
// (sequence, q tile) of the work list; each pair is one item per kv head.
static int64_t mixed_pairs(int32_t batch, int32_t num_decodes, int32_t max_seqlen_q, int32_t num_heads,
                           int32_t num_kv_heads, int32_t pages_per_seq, int32_t page_size) {
  const int chunks = pages_per_seq > 0 ? mixed_decode_chunks(pages_per_seq, page_size) : 0;
  const int group = num_heads / num_kv_heads;
  const int64_t tile_tokens = kRows / group;
  const int64_t n_pre = batch - num_decodes;
  const int64_t n_qtiles = n_pre > 0 ? (max_seqlen_q + tile_tokens - 1) / tile_tokens : 0;
  return (int64_t)num_decodes * chunks * ((group + 15) / 16) + n_pre * n_qtiles;
}

extern "C" size_t pa_mixed_workspace_size(int32_t batch, int32_t num_decodes, int32_t max_seqlen_q,
                                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                          int32_t pages_per_seq, int32_t page_size) {
  if (batch < 0 || num_decodes < 0 || num_decodes > batch || max_seqlen_q < 0 || num_heads <= 0 ||
      num_kv_heads <= 0 || num_heads % num_kv_heads || num_heads / num_kv_heads > kRows || head_dim <= 0 ||
      pages_per_seq < 0 || page_size <= 0)
    return 0;
  const int chunks = pages_per_seq > 0 ? mixed_decode_chunks(pages_per_seq, page_size) : 0;
  if (head_dim != kPHeadDim) {
    // the generic kernels: decode partials of every chunk (no work list),
    // after 256 bytes that keep the size non-zero
    if (!any_head_dim(head_dim)) return 0;
    return 256 + ((size_t)num_decodes * num_heads * chunks * ((size_t)head_dim + 2) * sizeof(float) + 255) / 256 *
                     256;
  }
  const int64_t pairs = mixed_pairs(batch, num_decodes, max_seqlen_q, num_heads, num_kv_heads, pages_per_seq,
                                    page_size);
  return mixed_partials_bytes(num_decodes, num_heads, head_dim, chunks) +
         (size_t)(kPlanHeader + 8 * ((pairs + 7) / 8 * 8)) * sizeof(int32_t);
}

extern "C" int pa_mixed(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                        const uint16_t* k_cache, const uint16_t* v_cache,
                        int32_t num_pages, int32_t page_size,
                        int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                        const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                        const int32_t* cu_seqlens_q, const int32_t* kv_lens, const int32_t* input_positions,
                        int32_t batch, int32_t num_decodes, int32_t num_tokens, int32_t max_seqlen_q,
                        int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                        float prefill_scale, float decode_scale, float soft_cap,
                        uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride,
                        void* workspace, size_t workspace_bytes, void* stream) {
  if (batch < 0 || num_decodes < 0 || num_decodes > batch || num_tokens < 0 || max_seqlen_q < 0 ||
      num_heads <= 0 || num_kv_heads <= 0 || num_pages <= 0 || page_size <= 0 || pages_per_seq < 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_mixed: bad sizes (batch=%d, num_decodes=%d, num_tokens=%d, max_seqlen_q=%d, num_heads=%d, "
                "num_kv_heads=%d, num_pages=%d, page_size=%d, pages_per_seq=%d)",
                batch, num_decodes, num_tokens, max_seqlen_q, num_heads, num_kv_heads, num_pages, page_size,
                pages_per_seq);
  if (num_heads % num_kv_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "pa_mixed: Number of Q heads must be divisible by number of KV heads. Got %d and %d.", num_heads,
                num_kv_heads);
  const bool any_d = head_dim != kPHeadDim && any_head_dim(head_dim);
  if (head_dim != kPHeadDim && !any_d)
    return fail(PA_ERR_UNSUPPORTED, "pa_mixed: head_dim %d not supported (128, or a multiple of 16 from 16 to 256)",
                head_dim);
  const int group = num_heads / num_kv_heads;
  if (group > kRows)
    return fail(PA_ERR_UNSUPPORTED, "pa_mixed: %d q heads per kv head not supported (max %d)", group, kRows);
  if (num_tokens == 0) return PA_OK;
  if (!q || !out || !cu_seqlens_q || !input_positions ||
      (batch > 0 && (!k_cache || !v_cache || !block_tables || !kv_lens)))
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_mixed: null pointer");
  const uintptr_t align_bits = (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out;
  if ((align_bits & 15u) || (q_tok_stride | q_head_stride | page_stride | slot_stride | head_stride |
                             out_tok_stride | out_head_stride) % 8)
    return fail(PA_ERR_UNSUPPORTED, "pa_mixed: operands must be 16-byte aligned with strides multiple of 8");
  if ((int64_t)pages_per_seq * page_size > 0x7fffffffLL)
    return fail(PA_ERR_UNSUPPORTED, "pa_mixed: block table spans more than 2^31 tokens");
  if (!any_d && page_size % kTileN == 0 && !prefill_offsets_fit(slot_stride))
    return fail(PA_ERR_UNSUPPORTED, "pa_mixed: slot stride %lld too large for 32-bit tile offsets (max %lld)",
                (long long)slot_stride, (long long)((0x7fffffffLL - (kPHeadDim - 1)) / (kTileN - 1)));
  const int n_chunks = pages_per_seq > 0 ? mixed_decode_chunks(pages_per_seq, page_size) : 0;
  const size_t need = pa_mixed_workspace_size(batch, num_decodes, max_seqlen_q, num_heads, num_kv_heads, head_dim,
                                              pages_per_seq, page_size);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u))
    return fail(PA_ERR_WORKSPACE, "pa_mixed: 256-byte aligned workspace of %zu bytes needed, %zu given", need,
                workspace_bytes);
  const size_t partials = mixed_partials_bytes(num_decodes, num_heads, head_dim, n_chunks);
  const float cap = soft_cap > 0.f ? soft_cap : 0.f;

  MixedParams m{};
  // ---- prefill half: entries num_decodes .. batch-1
  const int n_pre = batch - num_decodes;
  PrefillParams& pp = m.pre;
  pp.q = q;
  pp.q_ts = q_tok_stride;
  pp.q_hs = q_head_stride;
  pp.k_cache = k_cache;
  pp.v_cache = v_cache;
  pp.num_pages = num_pages;
  pp.page_size = page_size;
  pp.page_stride = page_stride;
  pp.slot_stride = slot_stride;
  pp.head_stride = head_stride;
  pp.block_tables = block_tables ? block_tables + (int64_t)num_decodes * bt_stride : nullptr;
  pp.bt_stride = bt_stride;
  pp.pages_per_seq = pages_per_seq;
  pp.cu_q = cu_seqlens_q + num_decodes;
  pp.cu_k = nullptr;
  pp.kv_lens = kv_lens ? kv_lens + num_decodes : nullptr;
  pp.positions = input_positions;
  pp.batch = n_pre;
  pp.num_tokens = num_tokens;
  pp.num_heads = num_heads;
  pp.num_kv_heads = num_kv_heads;
  pp.group = group;
  pp.tile_tokens = kRows / group;
  pp.n_qtiles = n_pre > 0 ? (max_seqlen_q + pp.tile_tokens - 1) / pp.tile_tokens : 0;
  pp.max_seqlen_q = max_seqlen_q;
  pp.soft_cap = cap;
  pp.logit_scale = cap > 0.f ? prefill_scale : prefill_scale * kLog2e;
  pp.out = out;
  pp.o_ts = out_tok_stride;
  pp.o_hs = out_head_stride;
  // ---- decode half: entries 0 .. num_decodes-1
  DecodeParams& dp = m.dec;
  dp.q = q;
  dp.q_bs = q_tok_stride;
  dp.q_hs = q_head_stride;
  dp.k_cache = k_cache;
  dp.v_cache = v_cache;
  dp.num_pages = num_pages;
  dp.page_size = page_size;
  dp.page_stride = page_stride;
  dp.slot_stride = slot_stride;
  dp.head_stride = head_stride;
  dp.block_tables = block_tables;
  dp.bt_stride = bt_stride;
  dp.pages_per_seq = pages_per_seq;
  dp.lengths = kv_lens;
  dp.batch = num_decodes;
  dp.num_heads = num_heads;
  dp.num_kv_heads = num_kv_heads;
  dp.group = group;
  dp.hblocks = (group + 15) / 16;  // a decode item covers 16 q heads of one kv head
  dp.chunk = mixed_decode_chunk(page_size);
  dp.n_chunks = n_chunks;
  dp.soft_cap = cap;
  dp.logit_scale = cap > 0.f ? decode_scale : decode_scale * kLog2e;
  dp.ws_o = reinterpret_cast<float*>(workspace);
  dp.ws_ml = partials > 0 ? dp.ws_o + (size_t)num_decodes * num_heads * n_chunks * head_dim : nullptr;
  dp.out = out;
  dp.out_bs = out_tok_stride;
  dp.out_hs = out_head_stride;
  dp.rows = cu_seqlens_q;
  dp.row_limit = num_tokens;
  dp.zero_empty = 1;
  // ---- zero pass
  m.cu_q = cu_seqlens_q;
  m.batch = batch;
  m.num_decodes = num_decodes;
  m.num_tokens = num_tokens;
  m.max_seqlen_q = max_seqlen_q;
  m.num_heads = num_heads;
  m.out = out;
  m.o_ts = out_tok_stride;
  m.o_hs = out_head_stride;
  if (any_d) {
    // head sizes other than 128: the generic prefill (with its zero pass:
    // every row outside the prefill sequences or past max_seqlen_q, so also
    // the decode rows, which the decode merge then writes) and the generic
    // decode, which leaves partials for every chunk
    hipStream_t gs = (hipStream_t)stream;
    dp.ws_o = reinterpret_cast<float*>(workspace);
    dp.ws_ml = dp.ws_o + (size_t)num_decodes * num_heads * n_chunks * head_dim;
    const int rc = prefill_any_launch("pa_mixed", pp, head_dim, gs);
    if (rc || num_decodes == 0) return rc;
    return decode_any_launch("pa_mixed", dp, head_dim, gs);
  }

  // ---- regions.  Prefill level l (q tile n_qtiles-1-l) reaches kv index
  // (n_qtiles-l)*tile_tokens; it goes before the decode items while it costs
  // more than one decode chunk.
  const int64_t pairs = (int64_t)n_pre * num_kv_heads;
  const int64_t dec_tokens = std::min<int64_t>(dp.chunk, (int64_t)pages_per_seq * page_size);
  int head_levels = 0;
  while (head_levels < pp.n_qtiles &&
         (float)(pp.n_qtiles - head_levels) * pp.tile_tokens * kPrefillOverDecodeTile >= (float)dec_tokens)
    ++head_levels;
  if (num_decodes == 0) head_levels = pp.n_qtiles;
  const int64_t pre_items = (int64_t)pp.n_qtiles * pairs;
  const int64_t pre_head = (int64_t)head_levels * pairs;
  const int64_t dec_items = (int64_t)num_decodes * n_chunks * num_kv_heads * dp.hblocks;
  const int64_t r1 = round8(pre_head);
  const int64_t r2 = r1 + round8(dec_items);
  const int64_t r3 = r2 + (pre_items - pre_head);
  const int64_t zero_blocks = (num_tokens + kZeroRowsPerBlock - 1) / kZeroRowsPerBlock;
  // the work list: every (decode chunk | prefill q tile) pair, all kv heads
  const int64_t list_pairs = mixed_pairs(batch, num_decodes, max_seqlen_q, num_heads, num_kv_heads, pages_per_seq,
                                         page_size);
  const bool planned = list_pairs > 0 && list_pairs * num_kv_heads >= kMixedPlanMinItems &&
                       n_pre <= kMixedPlanMaxPrefill;
  const int64_t list_items = (list_pairs + 7) / 8 * 8 * num_kv_heads;
  const int64_t r4 = (planned ? list_items : r3) + zero_blocks;
  if (r4 > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "pa_mixed: grid of %lld workgroups too large", (long long)r4);
  m.r1 = (int32_t)r1;
  m.r2 = (int32_t)r2;
  m.r3 = (int32_t)(planned ? list_items : r3);
  m.r4 = (int32_t)r4;
  m.pre_head = (int32_t)pre_head;
  m.n_dec_items = (int32_t)dec_items;

  hipStream_t s = (hipStream_t)stream;
  if (planned) {
    int32_t* plan = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) + partials);
    mixed_plan_kernel<<<dim3(1), dim3(kMixedPlanThreads), 0, s>>>(m, plan);
    int rc = launch_status("pa_mixed(plan)");
    if (rc) return rc;
    m.plan = plan;
  }
  const dim3 grid((unsigned)r4), block(kThreads);
  const int paging_p = prefill_paging(page_size, slot_stride);
  const bool aligned_d = page_size % kDecodeStep == 0;  // every kPageTile / kPageWave size is
  // (aligned) a decode chunk of more than 64 pages: four page ids per lane
  // (pages below 64 tokens, so never with whole-tile prefill paging; always
  // with the per-wave paging of 16- and 32-token pages)
  const bool wide_d = aligned_d && dp.chunk / page_size > 64;
  if (cap > 0.f) {
    if (paging_p == kPageTile) mixed_kernel<true, kPageTile, true, 1><<<grid, block, 0, s>>>(m);
    else if (paging_p == kPageWave) mixed_kernel<true, kPageWave, true, 4><<<grid, block, 0, s>>>(m);
    else if (wide_d) mixed_kernel<true, kPageLane, true, 4><<<grid, block, 0, s>>>(m);
    else if (aligned_d) mixed_kernel<true, kPageLane, true, 1><<<grid, block, 0, s>>>(m);
    else mixed_kernel<true, kPageLane, false, 1><<<grid, block, 0, s>>>(m);
  } else {
    if (paging_p == kPageTile) mixed_kernel<false, kPageTile, true, 1><<<grid, block, 0, s>>>(m);
    else if (paging_p == kPageWave) mixed_kernel<false, kPageWave, true, 4><<<grid, block, 0, s>>>(m);
    else if (wide_d) mixed_kernel<false, kPageLane, true, 4><<<grid, block, 0, s>>>(m);
    else if (aligned_d) mixed_kernel<false, kPageLane, true, 1><<<grid, block, 0, s>>>(m);
    else mixed_kernel<false, kPageLane, false, 1><<<grid, block, 0, s>>>(m);
  }
  int rc = launch_status("pa_mixed");
  if (rc || partials == 0 || num_decodes == 0) return rc;
  launch_decode_merge(dp, s);
  return launch_status("pa_mixed(merge)");
}
