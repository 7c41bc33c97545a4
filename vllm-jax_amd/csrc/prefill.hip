// Ragged causal GQA paged prefill for gfx950: the kernel entry and its host
// launcher.  The work item (one q tile of one sequence and kv head) is
// prefill_body in prefill_impl.h.
#include <algorithm>

#include "any_head.h"
#include "prefill_impl.h"

namespace pa {

// Output rows the prefill items do not write, for 64 tokens t0 .. t0 + 63
// (one wave): rows outside all sequences (before cu_q[0], from cu_q[batch]
// on) and rows at offset >= max_seqlen_q inside their sequence (the
// reference drops those too: its scatter only covers the first
// max_seqlen_bucket rows, prefill...:384-388) are zeroed.  A lane checks one
// token; the wave zeroes the rows it found, one after the other.
__device__ void prefill_zero_rows(const PrefillParams& p, int64_t t0) {
  const int lane = threadIdx.x & 63;
  const int64_t t = t0 + lane;
  const int32_t* cu_q = p.cu_q;
  const int batch = p.batch;
  bool zero = t < p.num_tokens;
  if (zero && batch > 0 && t >= cu_q[0] && t < cu_q[batch]) {
    // last b with cu_q[b] <= t
    int lo = 0, hi = batch;  // invariant: cu_q[lo] <= t < cu_q[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cu_q[mid] <= t) lo = mid;
      else hi = mid;
    }
    zero = t - cu_q[lo] >= p.max_seqlen_q;
  }
  uint64_t todo = __ballot(zero);
  const int chunks = p.num_heads * (kPHeadDim / 8);
  while (todo) {
    const int k = __ffsll((unsigned long long)todo) - 1;
    todo &= todo - 1;
    uint16_t* row = p.out + (t0 + k) * p.o_ts;
    for (int c = lane; c < chunks; c += 64) {
      const int hh = c / (kPHeadDim / 8);
      st16(row + hh * p.o_hs + (c - hh * (kPHeadDim / 8)) * 8, u32x4{0, 0, 0, 0});
    }
  }
}

// kZero (launches without a work list): workgroups past the items zero the
// rows no item writes, 512 tokens each, in place of a launch of their own.
template <bool kSoftCap, int kPaging, bool kZero = false>
__global__ void __launch_bounds__(kThreads, 1)
prefill_kernel(PrefillParams p) {
  if constexpr (kZero) {
    const int64_t items = (int64_t)p.n_qtiles * p.batch * p.num_kv_heads;
    if (blockIdx.x >= items) {  // uniform over the workgroup
      prefill_zero_rows(p, ((int64_t)blockIdx.x - items) * kThreads + 64 * (threadIdx.x >> 6));
      return;
    }
  }
  prefill_body<kSoftCap, kPaging>(p, blockIdx.x);
}

// The item of workgroup `bid` with the pools: every XCD walks the whole list
// (n items, one kv head of every entry, as prefill_resolve deals them), but
// only its first n - s items statically (workgroup 8 k + x runs XCD x's k-th
// item).  The last s items of every XCD, the cheapest, form that XCD's pool,
// claimed in list order with one atomicAdd on its counter by the workgroups
// dispatched after the static ones.  A workgroup takes from its own XCD's
// pool first (its items' K/V is in that XCD's L2) and steals from the next
// XCDs' pools once it is empty.  The 8 XCDs finish identical static work up
// to 6 % apart (clock and memory differ per XCD); the XCDs that run ahead
// reach their pool workgroups first and take more.  -1: nothing left.
__device__ __forceinline__ int prefill_pooled_item(const PrefillParams& p, int bid) {
  const int n = p.plan[0] * (p.num_kv_heads >> 3);  // items of one XCD
  const int s = n >> 2;
  if (bid < 8 * (n - s)) return bid;
  const int x = bid & 7;
  for (int i = 0; i < 8; ++i) {
    const int y = (x + i) & 7;
    // a plain read first: a spent pool is passed without an atomic (the
    // counter only grows, so a stale value errs late)
    if (__hip_atomic_load(p.pool + y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) >= s) continue;
    const int j = atomicAdd(p.pool + y, 1);  // XCD y's item n - s + j
    if (j < s) return 8 * (n - s + j) + y;
  }
  return -1;
}

template <bool kSoftCap, int kPaging>
__global__ void __launch_bounds__(kThreads, 1)
prefill_kernel_pooled(PrefillParams p) {
  __shared__ int32_t s_item;
  if (threadIdx.x == 0) s_item = prefill_pooled_item(p, blockIdx.x);
  __syncthreads();
  const int item = __builtin_amdgcn_readfirstlane(s_item);  // the same in every lane
  if (item < 0) return;
  prefill_body<kSoftCap, kPaging>(p, item);
}

constexpr int kPrepThreads = 1024;
constexpr int64_t kPoolMinItems = 16384;  // smallest grid that uses prefill_kernel_pooled
constexpr int kPlanBins = 4096;       // cost classes of the work list (class + 1, clamped)
constexpr int kPlanClassTiles = 16;   // kv tiles per cost class
constexpr int kPlanMaxBatch = 2048;   // sequences whose geometry the planner keeps in LDS
// Launches below this many items run in grid order (longest q-tile levels
// first) even with a workspace: the list's one-workgroup build costs a few
// microseconds ahead of the prefill, which short launches do not earn back
// (same process, bit-identical: the Qwen3-0.6B single-layer prefill 23.0 ->
// 20.3 us, 4 x 512 tokens of the Qwen3-8B heads 25.4 -> 23.2 us, 1 x 2048
// 52.2 -> 49.2 us; 256 x 128 and 64 x 1024 tokens, above it, unchanged).
constexpr int64_t kPrefillPlanMinItems = 1024;

// Work list of the prefill (run by one workgroup).  A pair (sequence b,
// q tile qt) is listed when the tile has rows; its cost is the number of kv
// tiles its last row sees, estimated as if positions were contiguous (the
// list orders the work and changes no result).  Pairs are counting-sorted by
// cost in classes of kPlanClassTiles kv tiles, largest first, so the longest
// items start first and no long item is left for the end.  Inside a class a
// sequence's q tiles stay together (costliest first), in runs of up to 64
// pairs: the workgroups an XCD runs at one time then stream the K/V of a few
// sequences, which its L2 holds (Qwen3-32B long prefill -2.7 %, prefix-cached
// -2.2 % against a list sorted by exact cost with the sequences interleaved).
// Per sequence, q0 / lq_rows / lk / kv_pos_off are derived exactly as
// prefill_resolve derives them without a list.
__device__ void prefill_plan(const PrefillParams& p, int32_t* __restrict__ plan) {
  __shared__ int32_t hist[kPlanBins];
  __shared__ int4 seqs[kPlanMaxBatch];  // q0, lq_rows, lk, kv_pos_off
  __shared__ int32_t lag[kPlanMaxBatch];  // lk - lq
  __shared__ int32_t scan[kPrepThreads];
  const int tid = threadIdx.x;
  for (int i = tid; i < kPlanBins; i += kPrepThreads) hist[i] = 0;
  for (int b = tid; b < p.batch; b += kPrepThreads) prefill_seq_geometry(p, b, seqs[b], lag[b]);
  __syncthreads();
  const int nq = p.n_qtiles;
  const int pairs = p.batch * nq;
  // pair i: sequence i / nq, q tile nq - 1 - i % nq (a sequence's tiles in a
  // row, costliest first); bin: its cost class
  auto bin_of = [&](int i) -> int {  // 0: no rows
    const int b = i / nq;
    const int tiles = prefill_pair_tiles(seqs[b], lag[b], nq - 1 - (i - b * nq), p.tile_tokens);
    return tiles < 0 ? 0 : min(tiles / kPlanClassTiles + 1, kPlanBins - 1);
  };
  for (int64_t ii = tid; ii < pairs; ii += kPrepThreads) {
    const int i = (int)ii;
    const int c = bin_of(i);
    if (c) atomicAdd(&hist[c], 1);
  }
  __syncthreads();
  // thread t owns bins kPlanBins-1-4t .. kPlanBins-4-4t (largest first)
  constexpr int kPer = kPlanBins / kPrepThreads;
  int cnt[kPer], local = 0;
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    cnt[j] = hist[kPlanBins - 1 - (kPer * tid + j)];
    local += cnt[j];
  }
  int count;
  int run = block_exclusive_scan<kPrepThreads>(local, scan, count);  // pairs in larger bins
#pragma unroll
  for (int j = 0; j < kPer; ++j) {
    hist[kPlanBins - 1 - (kPer * tid + j)] = run;  // first rank of the bin
    run += cnt[j];
  }
  __syncthreads();
  const int lane = tid & 63;
  for (int64_t i0 = tid - lane; i0 < pairs; i0 += kPrepThreads) {  // whole waves (uniform trip count)
    const int i = (int)i0 + lane;
    const int c = i < pairs ? bin_of(i) : 0;
    // ranks for this wave's 64 consecutive pairs, class by class, in lane order
    uint64_t todo = __ballot(c != 0);
    int rank = 0;
    while (todo) {
      const int lead = __ffsll((unsigned long long)todo) - 1;
      const int cc = __shfl(c, lead);
      const uint64_t m = __ballot(c == cc);
      int base = 0;
      if (lane == lead) base = atomicAdd(&hist[cc], __popcll(m));
      base = __shfl(base, lead);
      if (c == cc) rank = base + __popcll(m & ((1ull << lane) - 1));
      todo &= ~m;
    }
    if (!c) continue;
    const int b = i / nq;
    const int4 sq = seqs[b];
    int32_t* r = plan + kPlanHeader + 8 * rank;
    st16(r, u32x4{(uint32_t)b, (uint32_t)(nq - 1 - (i - b * nq)), (uint32_t)sq.x, (uint32_t)sq.y});
    st16(r + 4, u32x4{(uint32_t)sq.z, (uint32_t)sq.w, 0u, 0u});
  }
  if (tid == 0) {
    plan[0] = count;
    for (int i = 8; i < 16; ++i) plan[i] = 0;  // the pools' counters (prefill_kernel_pooled)
  }
}

// Before the prefill: workgroup 0 builds the work list (when `plan` is
// given); the others zero every output row the prefill kernel does not write:
// rows outside all sequences (before cu_q[0], from cu_q[batch] on) and rows
// at offset >= max_seqlen_q inside their sequence (the reference drops those
// too: its scatter only covers the first max_seqlen_bucket rows,
// prefill...:384-388).  One wave per token row.
__global__ void __launch_bounds__(kPrepThreads)
prefill_prep_kernel(PrefillParams p, int32_t* __restrict__ plan) {
  int zb = blockIdx.x;
  if (plan) {
    if (zb == 0) {
      prefill_plan(p, plan);
      return;
    }
    --zb;
  }
  const int lane = threadIdx.x & 63;
  const int64_t t = (int64_t)zb * (kPrepThreads / 64) + (threadIdx.x >> 6);
  if (t >= p.num_tokens) return;
  const int32_t* cu_q = p.cu_q;
  const int batch = p.batch;
  bool covered = false;
  if (batch > 0 && t >= cu_q[0] && t < cu_q[batch]) {
    // last b with cu_q[b] <= t
    int lo = 0, hi = batch;  // invariant: cu_q[lo] <= t < cu_q[hi]
    while (hi - lo > 1) {
      const int mid = (lo + hi) >> 1;
      if (cu_q[mid] <= t) lo = mid;
      else hi = mid;
    }
    covered = t - cu_q[lo] < p.max_seqlen_q;
  }
  if (covered) return;
  const int chunks_per_head = kPHeadDim / 8;
  for (int c = lane; c < p.num_heads * chunks_per_head; c += 64) {
    const int hh = c / chunks_per_head;
    const int e = (c - hh * chunks_per_head) * 8;
    st16(p.out + t * p.o_ts + hh * p.o_hs + e, u32x4{0, 0, 0, 0});
  }
}

// Quantized pages for the prefill (float8 e4m3 or integer codes).  A
// block-table entry (b, lp) is in use when lp * page_size < the sequence's
// kv length.  Every distinct physical page in use is widened once into a
// compact bf16 pool (slot i of the pool holds the i-th distinct page), each
// element bf16(code value * scale of its token), one rounding (exact for an
// e4m3 code with a power-of-two scale); the remapped table points there (-1 for unused entries, which
// the prefill never reads).  Pages shared between sequences (cached
// prefixes) are widened once.
//
// fp8_pages_plan_kernel (one workgroup) finds the distinct pages with an
// open-addressing hash in LDS: keys are physical page ids, and the thread
// whose atomicCAS claims a key takes the next slot from an LDS counter and
// records its entry as the slot's owner.  The hash has 2^hbits slots, at
// least twice the table's entries up to 2^kFp8HashBits; a larger table
// keeps the largest hash, which holds up to 2^(hbits - 1) distinct pages
// (the table's entries repeat the pages of shared prefixes, and small pages
// make many entries).  A launch with more distinct pages than that (or
// hbits == 0) gives every used entry its own slot instead.
constexpr int kFp8HashBits = 14;  // LDS hash of 2^14 slots: up to 2^13 distinct pages

// Physical page of table entry e, or -1 when the entry is not in use.
__device__ __forceinline__ int32_t fp8_entry_page(const int32_t* __restrict__ bt, int64_t bt_stride,
                                                  int32_t pages_per_seq, int32_t page_size, int32_t num_pages,
                                                  const int32_t* __restrict__ cu_q, const int32_t* __restrict__ cu_k,
                                                  int64_t e) {
  const int b = (int)(e / pages_per_seq);
  const int lp = (int)(e - (int64_t)b * pages_per_seq);
  const int lk = cu_k ? cu_k[b + 1] - cu_k[b] : cu_q[b + 1] - cu_q[b];
  if ((int64_t)lp * page_size >= lk) return -1;
  const int32_t raw = bt[(int64_t)b * bt_stride + lp];
  return raw < 0 ? 0 : (raw >= num_pages ? num_pages - 1 : raw);
}

__device__ __forceinline__ uint32_t fp8_page_hash(int32_t page, int hbits) {
  return ((uint32_t)page * 0x9E3779B1u) >> (32 - hbits);
}

__global__ void __launch_bounds__(1024)
fp8_pages_plan_kernel(const int32_t* __restrict__ bt, int64_t bt_stride, int32_t pages_per_seq, int32_t batch,
                      int32_t page_size, int32_t num_pages, const int32_t* __restrict__ cu_q,
                      const int32_t* __restrict__ cu_k, int32_t hbits, int32_t* __restrict__ bt_out,
                      int32_t* __restrict__ owner, int32_t* __restrict__ count) {
  __shared__ int32_t keys[1 << kFp8HashBits];
  __shared__ int32_t slots[1 << kFp8HashBits];
  __shared__ int32_t n_slots;
  __shared__ int32_t overflow;
  const int tid = threadIdx.x;
  const int64_t entries = (int64_t)batch * pages_per_seq;
  const uint32_t hmask = hbits ? (1u << hbits) - 1u : 0u;
  const int32_t max_distinct = hbits ? 1 << (hbits - 1) : 0;
  if (hbits)
    for (uint32_t h = tid; h <= hmask; h += blockDim.x) keys[h] = -1;
  if (tid == 0) {
    n_slots = 0;
    overflow = hbits ? 0 : 1;
  }
  __syncthreads();
  if (hbits) {
    for (int64_t e = tid; e < entries; e += blockDim.x) {
      const int32_t page = fp8_entry_page(bt, bt_stride, pages_per_seq, page_size, num_pages, cu_q, cu_k, e);
      if (page < 0) continue;
      // at most one pass over the hash: a full hash ends the probe (the
      // launch then falls back to one slot per entry)
      uint32_t h = fp8_page_hash(page, hbits);
      for (uint32_t probe = 0; probe <= hmask; ++probe) {
        const int32_t prev = atomicCAS(&keys[h], -1, page);
        if (prev == -1) {
          const int32_t sl = atomicAdd(&n_slots, 1);
          slots[h] = sl;
          if (sl < max_distinct) owner[sl] = (int32_t)e;
          else overflow = 1;
          break;
        }
        if (prev == page) break;
        h = (h + 1) & hmask;
        if (probe == hmask) overflow = 1;
      }
    }
    __syncthreads();
  }
  if (!overflow) {
    // every page in use holds a key, so each lookup ends
    for (int64_t e = tid; e < entries; e += blockDim.x) {
      const int32_t page = fp8_entry_page(bt, bt_stride, pages_per_seq, page_size, num_pages, cu_q, cu_k, e);
      int32_t sl = -1;
      if (page >= 0) {
        uint32_t h = fp8_page_hash(page, hbits);
        while (keys[h] != page) h = (h + 1) & hmask;
        sl = slots[h];
      }
      bt_out[e] = sl;
    }
  } else {
    // one slot per used entry, in claim order
    __syncthreads();
    if (tid == 0) n_slots = 0;
    __syncthreads();
    for (int64_t e = tid; e < entries; e += blockDim.x) {
      const int32_t page = fp8_entry_page(bt, bt_stride, pages_per_seq, page_size, num_pages, cu_q, cu_k, e);
      if (page >= 0) owner[atomicAdd(&n_slots, 1)] = (int32_t)e;
      else bt_out[e] = -1;
    }
    __syncthreads();
    for (int32_t sl = tid; sl < n_slots; sl += blockDim.x) bt_out[owner[sl]] = sl;
  }
  if (tid == 0) *count = n_slots;
}

// Slot i of the compact pool: the page of entry owner[i], widened.  A page
// is widened in `split` parts, each a split-th of its (slot, head) rows (16
// codes per thread and step): with one workgroup per page too few loads
// were in flight (a 256-token page is 1 MiB of codes), so pages take up to
// kWidenSplit parts of at least one step each.  The grid strides over the
// (slot, part) units up to the slot count the plan left on the device.
constexpr int kWidenSplit = 16;        // parts of a page, at most
constexpr int kWidenMaxBlocks = 8192;  // workgroups of the widening pass, at most
__global__ void __launch_bounds__(256)
fp8_pages_widen_kernel(const uint8_t* __restrict__ k8, const uint8_t* __restrict__ v8,
                       const float* __restrict__ ks, const float* __restrict__ vs, int32_t num_pages,
                       int32_t page_size, int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                       int64_t sc_page_stride, int64_t sc_head_stride, const int32_t* __restrict__ bt,
                       int64_t bt_stride, int32_t pages_per_seq, const int32_t* __restrict__ cu_q,
                       const int32_t* __restrict__ cu_k, int32_t num_kv_heads, const int32_t* __restrict__ owner,
                       const int32_t* __restrict__ count, uint16_t* __restrict__ wk, uint16_t* __restrict__ wv,
                       int32_t code, int32_t head_dim, int32_t split) {
  const int64_t units = (int64_t)*count * split;
  for (int64_t u = blockIdx.x; u < units; u += gridDim.x) {
    const int32_t sl = (int32_t)(u / split);
    const int part_w = (int)(u - (int64_t)sl * split);
    const int64_t page =
        fp8_entry_page(bt, bt_stride, pages_per_seq, page_size, num_pages, cu_q, cu_k, owner[sl]);  // in use
    const int rows = page_size * num_kv_heads;  // (slot, head) rows of head_dim codes
    const int parts = head_dim >> 4;            // 16 codes per part
    const int64_t wbase = (int64_t)sl * rows * head_dim;
    const int c_lo = (int)((int64_t)rows * parts * part_w / split);
    const int c_hi = (int)((int64_t)rows * parts * (part_w + 1) / split);
#pragma unroll 4
    for (int c = c_lo + threadIdx.x; c < c_hi; c += 256) {
      const int r = c / parts, part = c - r * parts;  // 16 codes of row r
      const int slot = r / num_kv_heads, h = r - slot * num_kv_heads;
      const int64_t src = page * page_stride + (int64_t)slot * slot_stride + (int64_t)h * head_stride + 16 * part;
      const int64_t sidx = page * sc_page_stride + (int64_t)h * sc_head_stride + slot;
      const int64_t dst = wbase + (int64_t)r * head_dim + 16 * part;
#pragma unroll
      for (int which = 0; which < 2; ++which) {
        const u32x4 x = ld16((which ? v8 : k8) + src);
        const float sc = (which ? vs : ks)[sidx];
        u32x4 o[2];
        // A positive normal power-of-two scale (what pa_kv_store_fp8 writes):
        // v_cvt_scalef32_pk_bf16_fp8 multiplies by 2^exponent(sc), so one
        // conversion per pair gives code * sc exactly.  Any other scale:
        // widen to float32, multiply, round to bf16 once.  The two agree
        // wherever both apply.
        const uint32_t sb = __float_as_uint(sc);
        if (code != kCodeE4M3) {
          // integer codes (uniform over the launch): the integer times the
          // scale, rounded to bf16 once
          const uint32_t flip = code == kCodeI8 ? 0x80808080u : 0u;
          const float bias = code == kCodeI8 ? 128.f : 0.f;
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const uint32_t c = x[w] ^ flip;
            o[w >> 1][2 * (w & 1)] = pack_bf16x2(((float)(c & 0xffu) - bias) * sc, ((float)((c >> 8) & 0xffu) - bias) * sc);
            o[w >> 1][2 * (w & 1) + 1] =
                pack_bf16x2(((float)((c >> 16) & 0xffu) - bias) * sc, ((float)(c >> 24) - bias) * sc);
          }
        } else if ((sb & 0x807fffffu) == 0u && sb >= 0x00800000u && sb < 0x7f800000u) {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            o[w >> 1][2 * (w & 1)] =
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)x[w], sc, false));
            o[w >> 1][2 * (w & 1) + 1] =
                __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8((int)x[w], sc, true));
          }
        } else {
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            const auto lo = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[w], false);
            const auto hi = __builtin_amdgcn_cvt_pk_f32_fp8((int)x[w], true);
            o[w >> 1][2 * (w & 1)] = pack_bf16x2(lo[0] * sc, lo[1] * sc);
            o[w >> 1][2 * (w & 1) + 1] = pack_bf16x2(hi[0] * sc, hi[1] * sc);
          }
        }
        uint16_t* d = (which ? wv : wk) + dst;
        st16(d, o[0]);
        st16(d + 8, o[1]);
      }
    }
  }
}

}  // namespace pa

using namespace pa;

// Checks and launches of pa_prefill; pa_prefill_fp8 runs it on its bf16
// workspace pool.
static int prefill_launch(const char* name, const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
                          const uint16_t* k_cache, const uint16_t* v_cache, int32_t num_pages, int32_t page_size,
                          int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                          const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                          const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                          const int32_t* input_positions, int32_t batch, int32_t num_tokens, int32_t max_seqlen_q,
                          int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale, float soft_cap,
                          uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride, void* workspace,
                          size_t workspace_bytes, void* stream) {
  if (batch < 0 || num_tokens < 0 || max_seqlen_q < 0 || num_heads <= 0 || num_kv_heads <= 0 ||
      num_pages <= 0 || page_size <= 0 || pages_per_seq < 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes (batch=%d, num_tokens=%d, max_seqlen_q=%d, num_heads=%d, "
                "num_kv_heads=%d, num_pages=%d, page_size=%d, pages_per_seq=%d)",
                name, batch, num_tokens, max_seqlen_q, num_heads, num_kv_heads, num_pages, page_size,
                pages_per_seq);
  if (num_heads % num_kv_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "%s: Number of Q heads must be divisible by number of KV heads. Got %d and %d.", name,
                num_heads, num_kv_heads);
#ifdef PA_PREFILL_PHASES
  const bool any_d = false;  // the phase-timestamp build instruments the head_dim 128 kernel only
#else
  const bool any_d = head_dim != kPHeadDim && any_head_dim(head_dim);
#endif
  if (head_dim != kPHeadDim && !any_d)
    return fail(PA_ERR_UNSUPPORTED, "%s: head_dim %d not supported (128, or a multiple of 16 from 16 to 256)",
                name, head_dim);
  const int group = num_heads / num_kv_heads;
  if (group > kRows)
    return fail(PA_ERR_UNSUPPORTED, "%s: %d q heads per kv head not supported (max %d)", name, group, kRows);
  if (num_tokens == 0) return PA_OK;
  if (!q || !out || !cu_seqlens_q || !input_positions || (batch > 0 && (!k_cache || !v_cache || !block_tables)))
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  const uintptr_t align_bits = (uintptr_t)q | (uintptr_t)k_cache | (uintptr_t)v_cache | (uintptr_t)out;
  if ((align_bits & 15u) || (q_tok_stride | q_head_stride | page_stride | slot_stride | head_stride |
                             out_tok_stride | out_head_stride) % 8)
    return fail(PA_ERR_UNSUPPORTED, "%s: operands must be 16-byte aligned with strides multiple of 8", name);
  if (!any_d && page_size % kTileN == 0 && !prefill_offsets_fit(slot_stride))
    return fail(PA_ERR_UNSUPPORTED, "%s: slot stride %lld too large for 32-bit tile offsets (max %lld)", name,
                (long long)slot_stride, (long long)((0x7fffffffLL - (kPHeadDim - 1)) / (kTileN - 1)));
  if (workspace) {
    const size_t need = pa_prefill_workspace_size(batch, max_seqlen_q, num_heads, num_kv_heads);
    if (workspace_bytes < need || ((uintptr_t)workspace & 255u))
      return fail(PA_ERR_WORKSPACE, "%s: 256-byte aligned workspace of %zu bytes needed, %zu given", name, need,
                  workspace_bytes);
  }
  hipStream_t s = (hipStream_t)stream;

  PrefillParams prm{};
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
#ifndef PA_PREFILL_PHASES
  if (any_d) return prefill_any_launch(name, prm, head_dim, s);
#endif
  const int64_t items = (int64_t)prm.n_qtiles * batch * num_kv_heads;
  if (items > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "%s: grid of %lld workgroups too large", name, (long long)items);
  // the work list needs every sequence's geometry in the planner's LDS
  const bool planned = workspace && batch > 0 && max_seqlen_q > 0 && batch <= kPlanMaxBatch &&
                       items >= kPrefillPlanMinItems;
  int32_t* plan = planned ? reinterpret_cast<int32_t*>(workspace) : nullptr;
  if (planned) {  // the list and the zero rows, ahead of the prefill
    const int64_t zero_blocks = (num_tokens + kPrepThreads / 64 - 1) / (kPrepThreads / 64) + 1;
    prefill_prep_kernel<<<dim3((unsigned)zero_blocks), dim3(kPrepThreads), 0, s>>>(prm, plan);
    int rc = launch_status(name);
    if (rc) return rc;
  }
  prm.plan = plan;
  // the pool pays off on long launches (the XCDs' finishing spread grows with
  // the launch; the extra workgroups cost a dispatch each)
  prm.pool = plan && num_kv_heads % 8 == 0 && items >= kPoolMinItems ? plan + 8 : nullptr;
  // with a list, items past its count return at once; with the pool, a
  // quarter more workgroups than items lets the XCDs that run ahead take up
  // to twice their share of it; without a list, workgroups past the items
  // zero the rows no item writes (512 tokens each: no launch of their own)
  const int64_t blocks = prm.pool ? std::min<int64_t>(items + (items + 3) / 4, 0x7fffffff)
                                  : items + (planned ? 0 : (num_tokens + kThreads - 1) / kThreads);
  if (blocks > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "%s: grid of %lld workgroups too large", name, (long long)blocks);
  if (blocks == 0) return PA_OK;
  const int paging = prefill_paging(page_size, slot_stride);
  const dim3 g((unsigned)blocks), b(kThreads);
  // one instance per (soft cap, paging, pool | list | grid order with the zero rows)
  auto launch = [&](auto cap, auto pg) {
    constexpr bool kCap = decltype(cap)::value;
    constexpr int kPg = decltype(pg)::value;
    if (prm.pool) prefill_kernel_pooled<kCap, kPg><<<g, b, 0, s>>>(prm);
    else if (planned) prefill_kernel<kCap, kPg><<<g, b, 0, s>>>(prm);
    else prefill_kernel<kCap, kPg, true><<<g, b, 0, s>>>(prm);
  };
  auto with_paging = [&](auto cap) {
    if (paging == kPageTile) launch(cap, std::integral_constant<int, kPageTile>{});
    else if (paging == kPageWave) launch(cap, std::integral_constant<int, kPageWave>{});
    else launch(cap, std::integral_constant<int, kPageLane>{});
  };
  if (prm.soft_cap > 0.f) with_paging(std::true_type{});
  else with_paging(std::false_type{});
  return launch_status(name);
}

extern "C" size_t pa_prefill_workspace_size(int32_t batch, int32_t max_seqlen_q, int32_t num_heads,
                                            int32_t num_kv_heads) {
  if (batch < 0 || max_seqlen_q < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_heads % num_kv_heads ||
      num_heads / num_kv_heads > kRows)
    return 0;
  const int64_t tile_tokens = kRows / (num_heads / num_kv_heads);
  const int64_t pairs = (int64_t)batch * ((max_seqlen_q + tile_tokens - 1) / tile_tokens);
  return (size_t)(kPlanHeader + 8 * pairs) * sizeof(int32_t);
}

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
                          void* workspace, size_t workspace_bytes, void* stream) {
  return prefill_launch("pa_prefill", q, q_tok_stride, q_head_stride, k_cache, v_cache, num_pages, page_size,
                        page_stride, slot_stride, head_stride, block_tables, bt_stride, pages_per_seq, cu_seqlens_q,
                        cu_seqlens_k, input_positions, batch, num_tokens, max_seqlen_q, num_heads, num_kv_heads,
                        head_dim, scale, soft_cap, out, out_tok_stride, out_head_stride, workspace, workspace_bytes,
                        stream);
}

// Widened K and V pages (one per table entry at most), the remapped block
// table, the slots' owner entries and the slot count, then (256-byte
// aligned) the prefill's work list.
static size_t fp8_widened_bytes(int32_t batch, int32_t pages_per_seq, int32_t page_size, int32_t num_kv_heads,
                                int32_t head_dim) {
  const size_t entries = (size_t)batch * pages_per_seq;
  const size_t page_elems = (size_t)page_size * num_kv_heads * head_dim;
  return (2 * entries * page_elems * sizeof(uint16_t) + (2 * entries + 1) * sizeof(int32_t) + 255) / 256 * 256;
}

extern "C" size_t pa_prefill_fp8_workspace_size(int32_t batch, int32_t pages_per_seq, int32_t page_size,
                                                int32_t num_kv_heads, int32_t head_dim, int32_t max_seqlen_q,
                                                int32_t num_heads) {
  if (batch <= 0 || pages_per_seq <= 0 || page_size <= 0 || num_kv_heads <= 0 || head_dim <= 0) return 0;
  const size_t plan = pa_prefill_workspace_size(batch, max_seqlen_q, num_heads, num_kv_heads);
  if (!plan) return 0;
  return fp8_widened_bytes(batch, pages_per_seq, page_size, num_kv_heads, head_dim) + plan;
}

// pa_prefill over 1-byte codes of type `code` (pa_prefill_fp8, pa_prefill_quant).
static int prefill_quant(const char* name, int32_t code, const uint16_t* q, int64_t q_tok_stride,
                         int64_t q_head_stride, const uint8_t* k_cache, const uint8_t* v_cache,
                         const float* k_scales, const float* v_scales, int32_t num_pages, int32_t page_size,
                         int64_t page_stride, int64_t slot_stride, int64_t head_stride, int64_t scale_page_stride,
                         int64_t scale_head_stride, const int32_t* block_tables, int64_t bt_stride,
                         int32_t pages_per_seq, const int32_t* cu_seqlens_q, const int32_t* cu_seqlens_k,
                         const int32_t* input_positions, int32_t batch, int32_t num_tokens, int32_t max_seqlen_q,
                         int32_t num_heads, int32_t num_kv_heads, int32_t head_dim, float scale, float soft_cap,
                         uint16_t* out, int64_t out_tok_stride, int64_t out_head_stride, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (code != kCodeE4M3 && code != kCodeI8 && code != kCodeU8)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: code_type %d is not one of PA_CODE_E4M3 (0), PA_CODE_INT8 (1), "
                "PA_CODE_UINT8 (2)", name, code);
  if (batch < 0 || num_pages <= 0 || page_size <= 0 || pages_per_seq < 0 || num_kv_heads <= 0)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: bad sizes (batch=%d, num_pages=%d, page_size=%d, "
                "pages_per_seq=%d, num_kv_heads=%d)", name, batch, num_pages, page_size, pages_per_seq, num_kv_heads);
  if (head_dim != kPHeadDim && !any_head_dim(head_dim))
    return fail(PA_ERR_UNSUPPORTED, "%s: head_dim %d not supported (128, or a multiple of 16 from 16 to 256)", name,
                head_dim);
  if (batch == 0 || pages_per_seq == 0 || num_tokens == 0)  // nothing to widen: zero rows only
    return prefill_launch(name, q, q_tok_stride, q_head_stride, nullptr, nullptr, 1, page_size,
                          (int64_t)page_size * num_kv_heads * head_dim, (int64_t)num_kv_heads * head_dim, head_dim,
                          block_tables, bt_stride, pages_per_seq, cu_seqlens_q, cu_seqlens_k, input_positions, 0,
                          num_tokens, max_seqlen_q, num_heads, num_kv_heads, head_dim, scale, soft_cap, out,
                          out_tok_stride, out_head_stride, nullptr, 0, stream);
  if (!k_cache || !v_cache || !k_scales || !v_scales || !block_tables || !cu_seqlens_q)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  if (num_kv_heads == 1) {  // a size-1 dimension's stride is arbitrary (and never used)
    head_stride = 0;
    scale_head_stride = 0;
  }
  if ((((uintptr_t)k_cache | (uintptr_t)v_cache) & 15u) || (page_stride | slot_stride | head_stride) % 16 ||
      (((uintptr_t)k_scales | (uintptr_t)v_scales) & 3u))
    return fail(PA_ERR_UNSUPPORTED, "%s: code rows must be 16-byte aligned", name);
  const size_t need = pa_prefill_fp8_workspace_size(batch, pages_per_seq, page_size, num_kv_heads, head_dim,
                                                    max_seqlen_q, num_heads);
  if (!need)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: bad sizes (max_seqlen_q=%d, num_heads=%d, "
                "num_kv_heads=%d)", name, max_seqlen_q, num_heads, num_kv_heads);
  if (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u))
    return fail(PA_ERR_WORKSPACE, "%s: 256-byte aligned workspace of %zu bytes needed, %zu given", name, need,
                workspace_bytes);
  const int64_t entries = (int64_t)batch * pages_per_seq;
  if (entries > 0x7fffffff / kWidenSplit)
    return fail(PA_ERR_UNSUPPORTED, "%s: %lld table entries", name, (long long)entries);
  const int64_t page_elems = (int64_t)page_size * num_kv_heads * head_dim;
  uint16_t* wk = reinterpret_cast<uint16_t*>(workspace);
  uint16_t* wv = wk + entries * page_elems;
  int32_t* bt2 = reinterpret_cast<int32_t*>(wv + entries * page_elems);
  hipStream_t s = (hipStream_t)stream;
  int32_t* owner = bt2 + entries;
  int32_t* n_slots = owner + entries;
  // an LDS hash of at least twice the entries finds the distinct pages
  int hbits = 6;
  while (hbits <= kFp8HashBits && ((int64_t)1 << hbits) < 2 * entries) ++hbits;
  if (hbits > kFp8HashBits) hbits = kFp8HashBits;  // the plan falls back past 2^(hbits - 1) distinct pages
  fp8_pages_plan_kernel<<<dim3(1), dim3(1024), 0, s>>>(block_tables, bt_stride, pages_per_seq, batch, page_size,
                                                       num_pages, cu_seqlens_q, cu_seqlens_k, hbits, bt2, owner,
                                                       n_slots);
  int rc = launch_status(name);
  if (rc) return rc;
  // parts per page: a step (256 threads x 16 codes) each, at most kWidenSplit
  const int64_t page_steps = (int64_t)page_size * num_kv_heads * (head_dim / 16) / 256;
  const int split = (int)std::max<int64_t>(1, std::min<int64_t>(kWidenSplit, page_steps));
  const int64_t widen_blocks = std::min<int64_t>(entries * split, kWidenMaxBlocks);
  fp8_pages_widen_kernel<<<dim3((unsigned)widen_blocks), dim3(256), 0, s>>>(
      k_cache, v_cache, k_scales, v_scales, num_pages, page_size, page_stride, slot_stride, head_stride,
      scale_page_stride, scale_head_stride, block_tables, bt_stride, pages_per_seq, cu_seqlens_q, cu_seqlens_k,
      num_kv_heads, owner, n_slots, wk, wv, code, head_dim, split);
  rc = launch_status(name);
  if (rc) return rc;
  return prefill_launch(name, q, q_tok_stride, q_head_stride, wk, wv, (int32_t)std::min<int64_t>(entries, 0x7fffffff),
                        page_size, page_elems, (int64_t)num_kv_heads * head_dim, head_dim, bt2, pages_per_seq,
                        pages_per_seq, cu_seqlens_q, cu_seqlens_k, input_positions, batch, num_tokens, max_seqlen_q,
                        num_heads, num_kv_heads, head_dim, scale, soft_cap, out, out_tok_stride, out_head_stride,
                        (char*)workspace + fp8_widened_bytes(batch, pages_per_seq, page_size, num_kv_heads, head_dim),
                        need - fp8_widened_bytes(batch, pages_per_seq, page_size, num_kv_heads, head_dim), stream);
}

extern "C" int pa_prefill_quant(int32_t code_type, const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
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
                                void* workspace, size_t workspace_bytes, void* stream) {
  return prefill_quant("pa_prefill_quant", code_type, q, q_tok_stride, q_head_stride, k_cache, v_cache, k_scales,
                       v_scales, num_pages, page_size, page_stride, slot_stride, head_stride, scale_page_stride,
                       scale_head_stride, block_tables, bt_stride, pages_per_seq, cu_seqlens_q, cu_seqlens_k,
                       input_positions, batch, num_tokens, max_seqlen_q, num_heads, num_kv_heads, head_dim, scale,
                       soft_cap, out, out_tok_stride, out_head_stride, workspace, workspace_bytes, stream);
}

extern "C" int pa_prefill_fp8(const uint16_t* q, int64_t q_tok_stride, int64_t q_head_stride,
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
                              void* workspace, size_t workspace_bytes, void* stream) {
  return prefill_quant("pa_prefill_fp8", kCodeE4M3, q, q_tok_stride, q_head_stride, k_cache, v_cache, k_scales,
                       v_scales, num_pages, page_size, page_stride, slot_stride, head_stride, scale_page_stride,
                       scale_head_stride, block_tables, bt_stride, pages_per_seq, cu_seqlens_q, cu_seqlens_k,
                       input_positions, batch, num_tokens, max_seqlen_q, num_heads, num_kv_heads, head_dim, scale,
                       soft_cap, out, out_tok_stride, out_head_stride, workspace, workspace_bytes, stream);
}

#ifdef PA_PREFILL_PHASES
// (phase build only) Copies the first n words of the phase timestamps to
// host memory / clears them all.
extern "C" int pa_prefill_phases_read(unsigned long long* out, size_t n) {
  if (!out || n > (size_t)8 * kPhaseSlots) return fail(PA_ERR_INVALID_ARGUMENT, "pa_prefill_phases_read: bad size");
  return hipMemcpyFromSymbol(out, HIP_SYMBOL(g_prefill_phases), n * sizeof(unsigned long long)) == hipSuccess
             ? PA_OK
             : fail(PA_ERR_LAUNCH, "pa_prefill_phases_read: copy failed");
}
extern "C" int pa_prefill_phases_clear(void) {
  void* g = nullptr;
  if (hipGetSymbolAddress(&g, HIP_SYMBOL(g_prefill_phases)) != hipSuccess ||
      hipMemset(g, 0, sizeof(g_prefill_phases)) != hipSuccess || hipDeviceSynchronize() != hipSuccess)
    return fail(PA_ERR_LAUNCH, "pa_prefill_phases_clear: clear failed");
  return PA_OK;
}
#endif
