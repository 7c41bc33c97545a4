// Ragged causal GQA paged prefill for gfx950.
//
// Workgroup = (q tile, sequence, kv head); 8 waves x 32 rows = 256 rows, where
// a row is a (query token, q head of this kv head) pair: row n of the tile is
// token n / G, head n % G (G = q heads per kv head).  Packing the G heads into
// the MFMA dimension makes every K/V tile staged in LDS serve G x tokens rows.
// One workgroup per CU, two waves per SIMD.
//
// KV tiles of 64 tokens go through a 4-stage LDS ring filled by direct
// global->LDS loads (global_load_lds_dwordx4) through the block table, issued
// two to three tiles ahead of use.  Per tile and wave:
//   S^T[t][n] = K[t][:] . Q[n][:]      v_mfma_f32_32x32x16_bf16, K rows read
//                                       with ds_read_b128, Q^T kept in VGPRs
//   online softmax per row n            row n = lane % 32: the row max needs one
//                                       permlane32 swap and rescaling O is
//                                       lane-local; the reference max only
//                                       moves when a row max grows by more than
//                                       2^8, so O is rarely rescaled.  Q is
//                                       scaled by scale*log2 e once per item
//                                       and the QK accumulators start at
//                                       -m_ref, so S leaves the MFMAs as the
//                                       exponent itself (soft cap: raw S)
//   O^T[d][n] += V^T[d][t] . P^T[t][n]  V^T operand read from the row-major V
//                                       tile with ds_read_b64_tr_b16 (gfx950's
//                                       transposing LDS read), P^T straight from
//                                       the S^T accumulator registers
// The softmax runs per 32-token half so one half's VALU work overlaps the
// other half's MFMAs.  LDS tiles are 64 rows x 256 B with 16-byte chunks
// XOR-swizzled per row so that both the K reads and the transposing V reads
// are bank-conflict free.  KV tiles entirely above the causal diagonal of the
// q tile are never loaded; the mask is evaluated only on tiles that straddle
// it or the kv length.  The Q tile comes in and the O tile goes out through
// each wave's own LDS blocks, four whole 256-byte rows per load or store.
// Workgroups take their items from a work list sorted
// by cost (prefill_plan in prefill.hip), longest first; without a list, from
// the last q tile down.
#pragma once
#include <type_traits>

#include "pa_common.h"
#include "pa_errors.h"

namespace pa {

constexpr int kPHeadDim = 128;
constexpr int kWaves = 8;         // waves per workgroup, 32 rows each
constexpr int kThreads = 64 * kWaves;
constexpr int kRows = 32 * kWaves;  // rows per workgroup
constexpr int kTileN = 64;        // kv tokens per tile
constexpr int kStages = 4;        // LDS ring depth: loads run two tiles ahead
constexpr int kTileElems = kTileN * kPHeadDim;
constexpr float kRescaleSlack = 8.f;  // log2 units the running max may lag
// instruction classes of __builtin_amdgcn_sched_group_barrier
constexpr int kSchedMfma = 0x008;
constexpr int kSchedDsRead = 0x100;
#ifndef PA_AHEAD_MFMA
#define PA_AHEAD_MFMA 4
#endif
constexpr int kAheadMfma = PA_AHEAD_MFMA;  // MFMAs between an LDS read and the MFMA it feeds

struct PrefillParams {
  const uint16_t* q;
  int64_t q_ts, q_hs;
  const uint16_t* k_cache;
  const uint16_t* v_cache;
  int32_t num_pages, page_size;
  int64_t page_stride, slot_stride, head_stride;
  const int32_t* block_tables;
  int64_t bt_stride;
  int32_t pages_per_seq;
  const int32_t* cu_q;
  const int32_t* cu_k;     // may be null
  const int32_t* kv_lens;  // may be null; overrides cu_k: kv length of sequence b
  const int32_t* positions;
  int32_t batch, num_tokens, num_heads, num_kv_heads, group, tile_tokens, n_qtiles, max_seqlen_q;
  float logit_scale;  // scale*log2e (soft cap off) or scale
  float soft_cap;
  uint16_t* out;
  int64_t o_ts, o_hs;
  // Work list (may be null): plan[0] = number of (sequence, q tile) pairs with
  // rows, PrefillPair records from int kPlanHeader on, most kv tiles first.
  const int32_t* plan;
  // With the work list and num_kv_heads % 8 == 0: the counters of the eight
  // XCDs' pools (plan + 8 .. plan + 15, zeroed by the list builder), see
  // prefill_kernel_pooled; null otherwise.
  int32_t* pool;
};

// How the tile loads find their pages.  kPageLane: each lane looks up its
// row's page (any page size).  kPageTile: pages of a multiple of 64 tokens
// hold whole tiles, one scalar page base per tile.  kPageWave: pages of 16 or
// 32 tokens; a wave's 8 rows of a tile lie in one page, one scalar page base
// per wave and tile.
constexpr int kPageLane = 0, kPageTile = 1, kPageWave = 2;

// One entry of the work list: a (sequence, q tile) pair with the sequence's
// row range and kv geometry as prefill_body derives them.
struct PrefillPair {
  int32_t b, qt, q0, lq_rows, lk, kv_pos_off, pad0, pad1;
};
constexpr int kPlanHeader = 64;  // ints before the first record (256 bytes)

typedef s16x4 __attribute__((address_space(3))) * lds_s16x4_ptr;
typedef void __attribute__((address_space(3))) * lds_void_ptr;
typedef const char __attribute__((address_space(3))) * lds_cbytes;

// Transposing 8-byte LDS read (ds_read_b64_tr_b16) at LDS byte address `a`.
__device__ __forceinline__ s16x4 ds_read_tr16(lds_cbytes a) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4_ptr)(a));
}

// 16-byte LDS read (ds_read_b128) at LDS byte address `a`.
__device__ __forceinline__ u32x4 ds_read16(lds_cbytes a) {
  return *reinterpret_cast<const u32x4 __attribute__((address_space(3)))*>(a);
}

// Physical 16-byte chunk of logical chunk c in tile row r.
__device__ __forceinline__ int swz(int r, int c) {
  return c ^ (((r & 3) << 2) | ((r >> 2) & 3));
}

// Work item of workgroup `bid`: (q tile, sequence b, kv head).  Items are
// ordered from the last q tile down (longest causal rows first).  Within one
// q-tile level the (b, kv head) pairs are placed so that, with workgroups
// dealt round-robin to the 8 XCDs, an XCD always serves the same pairs and
// holds one kv head of every sequence: all q tiles of a (b, head) pair then
// share that XCD's L2, and every XCD carries the same mix of sequence lengths.
__device__ __forceinline__ void prefill_item(int bid, int batch, int hkv, int n_qtiles, int& qt, int& b, int& kvh) {
  const int pairs = batch * hkv;
  const int level = bid / pairs;
  const int j = bid - level * pairs;
  qt = n_qtiles - 1 - level;
  if (hkv % 8 == 0) {
    const int xcd = j & 7;
    const int k = j >> 3;             // 0 .. batch*hkv/8 - 1
    const int per_b = hkv >> 3;
    // An XCD deals its workgroups round-robin to its shader engines, so its
    // k-th workgroup of a level lands on the same engine at every level;
    // rotating the sequences by level gives every engine every sequence.
    const int bk = k / per_b;
    b = bk + level % batch;
    b = b >= batch ? b - batch : b;
    kvh = 8 * (k - bk * per_b) + ((xcd - b) & 7);
  } else {
    b = j / hkv;
    kvh = j - b * hkv;
  }
}

// One 16-byte-per-lane global->LDS load (global_load_lds_dwordx4): lane l's
// 16 bytes land at LDS byte address lds_block + 16*l.  Issued as inline asm so
// the compiler does not insert its conservative "wait for every LDS DMA"
// before unrelated LDS reads; completion is tracked explicitly with
// wait_vm_lgkm0 + s_barrier before any wave reads the stage.
__device__ __forceinline__ void dma16(const void* gptr, uint32_t lds_block) {
  asm volatile("s_mov_b32 m0, %1\n\tglobal_load_lds_dwordx4 %0, off" ::"v"(gptr), "s"(lds_block) : "memory", "m0");
}

// The same from a scalar base: lane l loads the 16 bytes at sbase + voff.
__device__ __forceinline__ void dma16s(uint32_t voff, const void* sbase, uint32_t lds_block) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1" ::"v"(voff), "s"(sbase), "s"(lds_block)
               : "memory", "m0");
}

// s_waitcnt with vmcnt = N (N < 16), lgkmcnt = 0, expcnt untouched (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vm_lgkm0() {
  static_assert(N >= 0 && N < 16, "vmcnt field");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (0 << 8));
}

// LDS of a prefill item, at file scope so that every kernel that runs prefill
// items (and may reuse the space for other work) refers to one allocation.
// One object per ring stage: the compiler's LDS-DMA wait tracking then sees
// that reads of stage s never alias loads in flight into the other stages
// (with a single array it waits for every DMA before any LDS read).
static __shared__ __attribute__((aligned(1024))) uint16_t k_lds[kStages][kTileElems];
static __shared__ __attribute__((aligned(1024))) uint16_t v_lds[kStages][kTileElems];
static __shared__ int red_max[kWaves], red_min[kWaves];

// Per-workgroup phase timestamps, only in a build with PA_PREFILL_PHASES
// (libpaged_attention_phases.so; the library proper has none): s_memrealtime
// (100 MHz) at the item's start, once its kv range is known, once its first
// tile is in LDS, after the loop and after the stores, then the workgroup's
// HW_ID | XCC_ID << 32, its tile count and its item (sequence | q tile << 24
// | kv head << 48), 8 words per workgroup id.
#ifdef PA_PREFILL_PHASES
constexpr int kPhaseSlots = 1 << 17;
__device__ unsigned long long g_prefill_phases[8 * kPhaseSlots];
#define PA_PHASE(t) const unsigned long long t = __builtin_amdgcn_s_memrealtime()
__device__ __forceinline__ void prefill_phases_store(unsigned long long t0, unsigned long long t1,
                                                     unsigned long long t2, unsigned long long t3,
                                                     unsigned long long t4, int n_tiles, int b, int qt,
                                                     int kvh) {
  if (threadIdx.x != 0 || blockIdx.x >= kPhaseSlots) return;
  unsigned long long* g = g_prefill_phases + 8 * (unsigned long long)blockIdx.x;
  g[0] = t0;
  g[1] = t1;
  g[2] = t2;
  g[3] = t3;
  g[4] = t4;
  const unsigned hw = __builtin_amdgcn_s_getreg((4) | (0 << 6) | (31 << 11));   // HW_ID
  const unsigned xcc = __builtin_amdgcn_s_getreg((20) | (0 << 6) | (3 << 11));  // XCC_ID
  g[5] = (unsigned long long)hw | ((unsigned long long)xcc << 32);
  g[6] = (unsigned long long)n_tiles;
  g[7] = (unsigned long long)b | ((unsigned long long)qt << 24) | ((unsigned long long)kvh << 48);
}
#else
#define PA_PHASE(t) \
  do {              \
  } while (0)
#endif

// The aligned tile loads address a K/V row as a 32-bit per-lane offset from
// a scalar page base: tile row r (< 64) plus a 16-byte chunk (< 128 elements)
// is r * slot_stride + 8 * chunk elements, 2x that in bytes.  True when that
// fits int32 for every row (so the byte offset fits uint32 as well).
inline bool prefill_offsets_fit(int64_t slot_stride) {
  return slot_stride >= 0 && (kTileN - 1) * slot_stride + kPHeadDim - 1 <= (int64_t)0x7fffffff;
}

// Row range and kv geometry of prefill sequence b, as prefill_resolve
// derives them without a work list: g = (q0, lq_rows, lk, kv_pos_off), and
// lag = lk - lq (kv index of the first q row when positions are contiguous).
__device__ __forceinline__ void prefill_seq_geometry(const PrefillParams& p, int b, int4& g, int& lag) {
  const int q0 = p.cu_q[b];
  const int lq = p.cu_q[b + 1] - q0;
  const int lq_rows = (q0 < 0 || q0 >= p.num_tokens) ? 0 : min(min(lq, p.max_seqlen_q), p.num_tokens - q0);
  const int lk = min(p.kv_lens ? p.kv_lens[b] : (p.cu_k ? p.cu_k[b + 1] - p.cu_k[b] : lq),
                     p.pages_per_seq * p.page_size);
  const int off = lq_rows > 0 ? p.positions[q0] - (lk - lq) : 0;
  g = make_int4(q0, lq_rows, lk, off);
  lag = lk - lq;
}

// kv tiles the last row of q tile qt of a sequence with geometry (g, lag)
// sees, if positions are contiguous; -1 when the tile has no rows.
__device__ __forceinline__ int prefill_pair_tiles(const int4& g, int lag, int qt, int tile_tokens) {
  const int rows = g.y;
  if (qt * tile_tokens >= rows) return -1;
  const int64_t kv_hi = min((int64_t)g.z, (int64_t)lag + min(qt * tile_tokens + tile_tokens, rows));
  return kv_hi <= 0 ? 0 : (int)((kv_hi + kTileN - 1) / kTileN);
}

// A resolved work item: kv head kvh of q tile qt of sequence b, with the
// sequence's row range and kv geometry.
struct PrefillWork {
  int b, qt, kvh, q0, lq_rows, lk, kv_pos_off;
};

// Work item of workgroup `bid` (from the work list when there is one);
// false when the workgroup has nothing to do.
__device__ __forceinline__ bool prefill_resolve(const PrefillParams& p, int bid, PrefillWork& w) {
  const int hkv = p.num_kv_heads;
  if (p.plan) {
    // Workgroups are dealt round-robin to the 8 XCDs, and an XCD deals its
    // own round-robin to its four shader engines, waiting whenever the next
    // engine has no free CU: workgroups an XCD receives in a row must cost
    // about the same.  With hkv % 8 == 0, XCD x = bid % 8 walks the whole
    // list (hkv / 8 heads per entry), taking head (x - b) mod 8 (+ 8j) of
    // sequence b: every XCD sees the same cost sequence, and a (sequence, kv
    // head) stays on one XCD, so its q tiles in flight share that XCD's L2.
    // Otherwise entry rank, head = bid / hkv, bid % hkv.
    int rank, sub = 0;
    const bool by_xcd = (hkv & 7) == 0;
    if (by_xcd) {
      const int per = hkv >> 3;
      const int r = bid >> 3;
      rank = r / per;
      sub = r - rank * per;
    } else {
      rank = bid / hkv;
      w.kvh = bid - rank * hkv;
    }
    const __attribute__((address_space(4))) int32_t* pl = (const __attribute__((address_space(4))) int32_t*)p.plan;
    const int count = pl[0];
    // the list has room for every rank of the grid; entries past count are
    // never used
    const __attribute__((address_space(4))) int32_t* r = pl + kPlanHeader + 8 * rank;
    w.b = r[0];
    w.qt = r[1];
    w.q0 = r[2];
    w.lq_rows = r[3];
    w.lk = r[4];
    w.kv_pos_off = r[5];
    if (rank >= count) return false;  // uniform across the workgroup
    if (by_xcd) w.kvh = 8 * sub + (((bid & 7) - w.b) & 7);
    return true;
  }
  prefill_item(bid, p.batch, hkv, p.n_qtiles, w.qt, w.b, w.kvh);
  w.q0 = p.cu_q[w.b];
  const int lq = p.cu_q[w.b + 1] - w.q0;
  // rows past max_seqlen_q are left to the zero pass; rows past the token
  // count (malformed cu_seqlens) are never touched
  w.lq_rows = (w.q0 < 0 || w.q0 >= p.num_tokens) ? 0 : min(min(lq, p.max_seqlen_q), p.num_tokens - w.q0);
  if (w.qt * p.tile_tokens >= w.lq_rows) return false;  // uniform across the workgroup
  // kv lengths past the block table's span are clamped to it
  w.lk = min(p.kv_lens ? p.kv_lens[w.b] : (p.cu_k ? p.cu_k[w.b + 1] - p.cu_k[w.b] : lq),
             p.pages_per_seq * p.page_size);
  w.kv_pos_off = p.positions[w.q0] - (w.lk - lq);
  return true;
}

// One prefill work item, run by a whole 512-thread workgroup.
template <bool kSoftCap, int kPaging>
__device__ __forceinline__ void prefill_run(const PrefillParams& p, const PrefillWork& w) {
  constexpr bool kAligned = kPaging != kPageLane;  // scalar page bases
  PA_PHASE(ph0);
  auto k_stage = [&](auto c) __attribute__((always_inline)) -> uint16_t* { return k_lds[decltype(c)::value]; };
  auto v_stage = [&](auto c) __attribute__((always_inline)) -> uint16_t* { return v_lds[decltype(c)::value]; };

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);  // wave-uniform
  const int b = w.b, qt = w.qt, kvh = w.kvh, q0 = w.q0, lq_rows = w.lq_rows, lk = w.lk, kv_pos_off = w.kv_pos_off;
  const int tok0 = qt * p.tile_tokens;

  // ---- this lane's row
  const int n = lane & 31;
  const int h = lane >> 5;
  const int row = wave * 32 + n;
  const int rtok = tok0 + row / p.group;
  const bool row_ok = row < p.tile_tokens * p.group && rtok < lq_rows;
  // Loads are unconditional from a clamped row (lq_rows >= 1 here): a load
  // under a branch makes the compiler wait for it at the branch join.  A lane
  // without a row computes on the clamped row's finite data; its column of S
  // and O never mixes with other rows and is not stored.
  const int ltok = min(rtok, lq_rows - 1);
  const int qpos_ld = p.positions[q0 + ltok];
  // rows grow with the token: a wave whose first row has no token has none
  const bool wave_live = 32 * wave < p.tile_tokens * p.group && tok0 + (32 * wave) / p.group < lq_rows;

  // Wave w stages its Q rows and, at the end, its O rows in its own LDS:
  // 1 KiB blocks 2w and 2w+1 of K and of V in every stage, the only blocks
  // its own tile loads write (so no other wave's loads or reads can touch
  // them at those times).  Piece j of stage pair st holds rows 8j .. 8j+7 of
  // the wave, 256 bytes per row, with 16-byte chunk c of row r stored at
  // chunk c ^ (r & 15) (conflict-free reads of one chunk from 16 rows).
  auto piece = [&](int st, int j) __attribute__((always_inline)) -> uint32_t {
    return (uint32_t)(uintptr_t)(lds_void_ptr)((j & 1) ? &v_lds[st + (j >> 1)][0] : &k_lds[st + (j >> 1)][0]) +
           (uint32_t)(2048 * wave);
  };
  // row / group for rows < 256 as (row * gm) >> 24 (exact for group <= 256)
  const uint32_t gm = (0x1000000u + (uint32_t)p.group - 1u) / (uint32_t)p.group;

  // Q tile rows into stages 2 and 3 (free until tile 2 is issued, after the
  // barrier below), four whole 256-byte rows per load: full cache lines, where
  // a lane-per-row load would touch 32 lines a quarter each.  Issued before
  // the position reduction below so that their latencies overlap.
  bf16x8 qt_op[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane >> 4);
    const int rw = wave * 32 + r;
    const int tk = (int)(((uint32_t)rw * gm) >> 24);
    const int hd = rw - tk * p.group;
    const int lt = min(tok0 + tk, lq_rows - 1);
    const int c = (lane & 15) ^ (r & 15);
    dma16(p.q + (int64_t)(q0 + lt) * p.q_ts + (int64_t)(kvh * p.group + hd) * p.q_hs + 8 * c,
          piece(2, i >> 1) + 1024 * (i & 1));
  }
  const int qpos = row_ok ? qpos_ld : 0;
  // raw page ids of the first three kv tiles, read while the loads above fly
  int32_t raw_pre[3] = {0, 0, 0};
  // (kPageWave) log2 of the page size, and the table entry of this wave's
  // rows of tile T: rows 8w .. 8w + 7, or the tile's last row inside the kv
  // length when they lie past it (a wave's rows never straddle a page)
  const int pg_sh = kPaging == kPageWave ? (p.page_size == 16 ? 4 : 5) : 0;
  auto wave_entry = [&](int T) __attribute__((always_inline)) {
    const int last = min(max(lk - 1 - T * kTileN, 0), kTileN - 1);
    return (T * kTileN + min(8 * wave, last)) >> pg_sh;
  };
  if constexpr (kAligned) {
    if (p.pages_per_seq > 0) {
      const __attribute__((address_space(4))) int32_t* c =
          (const __attribute__((address_space(4))) int32_t*)(p.block_tables + (int64_t)b * p.bt_stride);
#pragma unroll
      for (int i = 0; i < 3; ++i)
        raw_pre[i] = c[min(kPaging == kPageWave ? wave_entry(i) : i * kTileN / p.page_size, p.pages_per_seq - 1)];
    }
  }

  // ---- q tile position range -> kv tile range (lanes n and n + 32 hold the same row)
  {
    int mx = row_ok ? qpos : INT_MIN;
    int mn = row_ok ? qpos : INT_MAX;
    minmax32(mx, mn);
    if (lane == 0) {
      red_max[wave] = mx;
      red_min[wave] = mn;
    }
  }

  // Retire every vector load here: the Q rows are in LDS, and the tile DMAs
  // below are invisible to the compiler's wait tracking, so nothing it
  // issued may still be in flight when they start (else it would drain them
  // at the loop head).
  wait_vm_lgkm0<0>();
  asm volatile("" ::: "memory");  // the Q reads stay after the wait
  // Q^T operand (B of S^T): lane (n, h)'s k-step ks is row n, d = 16ks + 8h
  // .. +8, i.e. chunk 2ks + h
#pragma unroll
  for (int ks = 0; ks < 8; ++ks)
    qt_op[ks] = as_bf16x8(
        ds_read16((lds_cbytes)(uintptr_t)(piece(2, n >> 3) + 256 * (n & 7) + 16 * ((2 * ks + h) ^ (n & 15)))));
  // read before any wave passes the barrier below (then tile 2 may overwrite
  // stage 2)
  wait_vm_lgkm0<0>();
  if constexpr (!kSoftCap) {
    // Q^T scaled by scale * log2 e (rounded to bf16), so that S = K Q^T is in
    // log2 units
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
      const u32x4 w = __builtin_bit_cast(u32x4, qt_op[ks]);
      u32x4 o;
#pragma unroll
      for (int e = 0; e < 4; ++e) o[e] = pack_bf16x2(bf16_lo(w[e]) * p.logit_scale, bf16_hi(w[e]) * p.logit_scale);
      qt_op[ks] = as_bf16x8(o);
    }
  }
  __syncthreads();
  int qpos_max = red_max[0], qpos_min = red_min[0];
#pragma unroll
  for (int w = 1; w < kWaves; ++w) {
    qpos_max = max(qpos_max, red_max[w]);
    qpos_min = min(qpos_min, red_min[w]);
  }
  // kv index j is visible to some row iff j < lk and j + kv_pos_off <= qpos_max
  const int64_t kv_hi64 = min((int64_t)lk, (int64_t)qpos_max - kv_pos_off + 1);
  const int kv_hi = kv_hi64 < 0 ? 0 : (int)kv_hi64;
  const int n_tiles = (kv_hi + kTileN - 1) / kTileN;
  PA_PHASE(ph1);
  // tiles [0, n_free) need no mask: every token is < lk and visible to every row
  const int64_t free_hi = min((int64_t)lk, (int64_t)qpos_min - kv_pos_off + 1);
  const int n_free = free_hi < 0 ? 0 : (int)(free_hi / kTileN);

  // ---- direct global->LDS tile loader.  A tile is 16 blocks of 1 KiB
  // (4 rows each); wave w fills blocks kBlk*w .. kBlk*w + kBlk-1 of K and V.
  // Lane l writes LDS bytes 16*l of a block, i.e. row 4blk + l/16, physical
  // chunk l%16, so it loads the logical chunk swz(row, l%16) of that token.
  constexpr int kBlk = 16 / kWaves;
  const int32_t* bt_row = p.block_tables + (int64_t)b * p.bt_stride;
  const int ld_r = lane >> 4;            // row within a 1 KiB block
  const int ld_p = lane & 15;            // physical chunk
  const int64_t head_off = (int64_t)kvh * p.head_stride;
  // per-lane element offset of the row within a page; the host guarantees
  // 63 * slot_stride + 127 <= INT32_MAX (prefill_offsets_fit), so neither
  // this nor the byte offset 2 * ld_off below wraps
  uint32_t ld_off[kBlk];
  uint32_t ld_sw[kBlk];  // its swizzled chunk part alone
  static_assert(kPaging != kPageWave || kBlk == 2, "a wave's rows of a tile must lie in one 16-token page");
  // (kPageWave) tile rows are rows of the wave's page: r mod page size
  const int row_mask = kPaging == kPageWave ? p.page_size - 1 : kTileN - 1;
#pragma unroll
  for (int i = 0; i < kBlk; ++i) {
    const int r = 4 * (kBlk * wave + i) + ld_r;
    ld_sw[i] = (uint32_t)(8 * swz(r, ld_p));
    ld_off[i] = (uint32_t)((kPaging == kPageWave ? r & row_mask : r) * (int32_t)p.slot_stride) + ld_sw[i];
  }
  // Tile DMA in two steps: tile_addrs() computes this wave's 2*kBlk global
  // addresses (K block 0, V block 0, K block 1, ...), dma_issue() issues one
  // of them, so the loads can be spread through other work.  In the aligned
  // case the tile's page id comes in raw (read ahead of time by the caller).
  struct TileAddrs {
    const char* kb;         // (aligned) scalar K and V bases of the tile
    const char* vb;
    uint32_t vo[kBlk];      // (aligned) this lane's byte offsets from them
    const uint16_t* g[2 * kBlk];  // (unaligned) this lane's pointers
  };
  // Aligned pages hold tpp whole tiles: tile j0 = 64 (tpp lp + r) is tile r
  // of table entry lp.  The loop walks (lp, r) incrementally, so no division
  // sits on the softmax wave's path.
  const int tpp = kPaging == kPageTile ? p.page_size / kTileN : 1;
  const int64_t tile_stride = (int64_t)kTileN * p.slot_stride;
  auto page_raw_at = [&](int lp) __attribute__((always_inline)) {
    const __attribute__((address_space(4))) int32_t* c = (const __attribute__((address_space(4))) int32_t*)bt_row;
    // stays inside the table row (only called with n_tiles > 0, so the row
    // has an entry: lk <= pages_per_seq * page_size)
    return c[max(min(lp, p.pages_per_seq - 1), 0)];
  };
  // rin: (aligned) the tile's index inside its page
  auto tile_addrs = [&](int j0, int32_t raw, int rin) __attribute__((always_inline)) {
    TileAddrs a;
    if constexpr (kAligned) {
      // the whole tile (kPageTile) or this wave's rows of it (kPageWave) lie
      // in one page
      const int32_t page = raw < 0 ? 0 : (raw >= p.num_pages ? p.num_pages - 1 : raw);
      // One scalar base per tile and a per-lane offset: no per-lane 64-bit
      // address arithmetic on the softmax wave's path.
      const int64_t pbase = (int64_t)page * p.page_stride + rin * tile_stride + head_off;
      a.kb = (const char*)(p.k_cache + pbase);
      a.vb = (const char*)(p.v_cache + pbase);
      // rows past the kv length read the tile's last valid token (masked,
      // never stale); a tile wholly past it reads its row 0.  Selects, no
      // branch.
      const int last = __builtin_amdgcn_readfirstlane(max(lk - 1 - j0, 0));
      const int last_row = kPaging == kPageWave ? min(last, kTileN - 1) & row_mask : min(last, kTileN - 1);
      const uint32_t last_off = (uint32_t)(last_row * (int32_t)p.slot_stride);
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        const int r = 4 * (kBlk * wave + i) + ld_r;
        a.vo[i] = 2u * (r <= last ? ld_off[i] : last_off + ld_sw[i]);
      }
    } else {
      int32_t pages[kBlk];
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        const int r = 4 * (kBlk * wave + i) + ld_r;
        const int j = min(j0 + r, lk - 1);
        pages[i] = safe_page(bt_row, j / p.page_size, p.num_pages);
      }
#pragma unroll
      for (int i = 0; i < kBlk; ++i) {
        const int r = 4 * (kBlk * wave + i) + ld_r;
        const int j = min(j0 + r, lk - 1);
        const int64_t o = (int64_t)pages[i] * p.page_stride + (int64_t)(j % p.page_size) * p.slot_stride +
                          head_off + 8 * swz(r, ld_p);
        a.g[2 * i] = p.k_cache + o;
        a.g[2 * i + 1] = p.v_cache + o;
      }
    }
    return a;
  };
  const uint32_t k_lds0 = (uint32_t)(uintptr_t)(lds_void_ptr)(&k_lds[0][0]);
  const uint32_t v_lds0 = (uint32_t)(uintptr_t)(lds_void_ptr)(&v_lds[0][0]);
  auto dma_issue = [&](const TileAddrs& a, int i, int stage) __attribute__((always_inline)) {
    const uint32_t lds = ((i & 1) ? v_lds0 : k_lds0) + (uint32_t)(stage * kTileElems * 2 + (kBlk * wave + (i >> 1)) * 1024);
    if constexpr (kAligned) dma16s(a.vo[i >> 1], (i & 1) ? a.vb : a.kb, lds);
    else dma16(a.g[i], lds);
  };
  auto issue_tile_raw = [&](int j0, int32_t raw, int stage) __attribute__((always_inline)) {
    const TileAddrs a = tile_addrs(j0, raw, (j0 / kTileN) % tpp);
#pragma unroll
    for (int i = 0; i < 2 * kBlk; ++i) dma_issue(a, i, stage);
  };
  constexpr int kDmaPerTile = 2 * kBlk;  // vm instructions one wave issues per tile

  // ---- per-lane LDS read offsets (bytes), fixed for the whole kernel.
  // K (A of S^T): row 32mt + n, logical chunk 2ks + h; the swizzle of a row
  // only depends on its low 4 bits, i.e. on n.
  const int fn = ((n & 3) << 2) | ((n >> 2) & 3);
  uint32_t koff[8];
#pragma unroll
  for (int ks = 0; ks < 8; ++ks) koff[ks] = n * 256 + 16 * ((2 * ks + h) ^ fn);
  // V^T (tr16): lane = 16*gamma + s reads row tokbase + 4h + s/4 (+8) and
  // logical column 32dt + 16(gamma%2) + 4(s%4): chunk 4dt + 2(gamma%2) +
  // (s%4)/2, byte 8*(s%2) inside it.  tokbase is a multiple of 16, so the
  // row's swizzle is that of tr_row (or tr_row + 8).
  const int tr_s = lane & 15;
  const int tr_gamma = lane >> 4;
  const int tr_row = 4 * h + (tr_s >> 2);
  const int f0 = ((tr_row & 3) << 2) | ((tr_row >> 2) & 3);
  const int f1 = (((tr_row + 8) & 3) << 2) | (((tr_row + 8) >> 2) & 3);
  uint32_t voff0[4], voff1[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) {
    const int c = 4 * dt + 2 * (tr_gamma & 1) + ((tr_s & 3) >> 1);
    voff0[dt] = v_lds0 + tr_row * 256 + 16 * (c ^ f0) + 8 * (tr_s & 1);
    voff1[dt] = v_lds0 + (tr_row + 8) * 256 + 16 * (c ^ f1) + 8 * (tr_s & 1);
  }
#pragma unroll
  for (int dt = 0; dt < 4; ++dt) asm volatile("" : "+v"(voff0[dt]), "+v"(voff1[dt]));

  f32x16 acc_o[4];
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int i = 0; i < 16; ++i) acc_o[dt][i] = 0.f;
  float m_ref = 0.f;  // reference max (log2 units) of the accumulators
  f32x16 neg_mref = {};  // -m_ref in every element: the QK accumulators start from it
  // running row sums, one per quarter of a tile (four short add chains), of
  // the f32 exponentials: v_dot2c on the packed P would wait for the matrix
  // core, which the other wave of the SIMD keeps busy
  float l_part[4] = {0.f, 0.f, 0.f, 0.f};
  f32x16 s_acc[2];  // S^T of the tile between its QK and its softmax
  bf16x8 pt[4];     // P^T of the tile between its softmax and its PV

  // ---- work pieces.  M(t) = PV(t-1) + QK(t) is MFMA work, SM(t) = softmax of
  // tile t is VALU work.  Waves 0-3 (group A) and 4-7 (group B) share the
  // SIMDs pairwise and run the same sequence half a step apart:
  //   segment 2t:   A: M(t)    B: SM(t-1)
  //   segment 2t+1: A: SM(t)   B: M(t)
  // with a workgroup barrier after every segment, so on every SIMD one wave
  // feeds the matrix core while the other one does its softmax (ping-pong).
  auto qk = [&](auto kst) __attribute__((always_inline)) {
    const lds_cbytes kt = (lds_cbytes)(k_stage(kst));
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) {
#pragma unroll
      for (int mt = 0; mt < 2; ++mt) {
        const bf16x8 a = as_bf16x8(ds_read16(kt + koff[ks] + mt * 8192));
        // the first k-step starts from -m_ref (zero with the soft cap)
        s_acc[mt] = mfma32(a, qt_op[ks], ks == 0 ? (kSoftCap ? f32x16{} : neg_mref) : s_acc[mt]);
      }
    }
  };
  auto pv = [&](auto vst) __attribute__((always_inline)) {
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      // k-step u: tokens 32(u/2) + 16(u%2) + {4h + r, 8 + 4h + r}
      const int rb = decltype(vst)::value * kTileElems * 2 + (32 * (u >> 1) + 16 * (u & 1)) * 256;
#pragma unroll
      for (int dt = 0; dt < 4; ++dt) {
        const s16x4 lo = ds_read_tr16((lds_cbytes)(uintptr_t)voff0[dt] + rb);
        const s16x4 hi = ds_read_tr16((lds_cbytes)(uintptr_t)voff1[dt] + rb);
        const u32x2 lo2 = __builtin_bit_cast(u32x2, lo);
        const u32x2 hi2 = __builtin_bit_cast(u32x2, hi);
        const u32x4 a = {lo2[0], lo2[1], hi2[0], hi2[1]};
        acc_o[dt] = mfma32(as_bf16x8(a), pt[u], acc_o[dt]);
      }
    }
  };
  const float cap_s2 = kSoftCap ? soft_cap_s2(p.logit_scale, p.soft_cap) : 0.f;
  const float cap_c = kSoftCap ? soft_cap_c(p.soft_cap) : 0.f;
  const float cap_2c = 2.f * cap_c;
  auto softmax = [&](int t, auto&& between) __attribute__((always_inline)) {
    const int j0 = t * kTileN;
    if constexpr (kSoftCap) {
      // capped logits relative to m_ref, as the uncapped S leaves the MFMAs
      const float cap_cm = cap_c - m_ref;
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          s_acc[mt][i] = soft_cap_log2_rel(s_acc[mt][i], cap_s2, cap_2c, cap_cm);
    }
    // s_acc[mt][i] = S[row n][token j0 + 32mt + 8(i/4) + 4h + i%4]
    if (t >= n_free) {
      // token j = j0 + 4h + c is visible iff j < lk and j + kv_pos_off <=
      // qpos, i.e. iff c < lim: one compare and one select per element
      const int64_t hi = min((int64_t)lk, (int64_t)qpos - kv_pos_off + 1) - j0 - 4 * h;
      int lim = (int)max((int64_t)0, min(hi, (int64_t)kTileN));
      asm volatile("" : "+v"(lim));  // keeps the compares 32-bit (the compiler widens them otherwise)
#pragma unroll
      for (int mt = 0; mt < 2; ++mt)
#pragma unroll
        for (int i = 0; i < 16; ++i)
          s_acc[mt][i] = 32 * mt + 8 * (i >> 2) + (i & 3) < lim ? s_acc[mt][i] : -INFINITY;
    }
    // four independent max3 chains (one per 16-token quarter)
    float mq[4];
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const int mt = q4 >> 1, b0 = 8 * (q4 & 1);
      float m = __builtin_fmaxf(__builtin_fmaxf(s_acc[mt][b0], s_acc[mt][b0 + 1]), s_acc[mt][b0 + 2]);
      m = __builtin_fmaxf(__builtin_fmaxf(m, s_acc[mt][b0 + 3]), s_acc[mt][b0 + 4]);
      m = __builtin_fmaxf(__builtin_fmaxf(m, s_acc[mt][b0 + 5]), s_acc[mt][b0 + 6]);
      mq[q4] = __builtin_fmaxf(m, s_acc[mt][b0 + 7]);
    }
    float mx = __builtin_fmaxf(__builtin_fmaxf(mq[0], mq[1]), __builtin_fmaxf(mq[2], mq[3]));
    mx = max_xor32(mx);  // log2 units: S is computed from the scaled Q (soft cap: capped logits)
    {
      // S is already relative to m_ref.  The first tile sets m_ref to the row
      // max (a row that sees no key keeps 0); later the reference moves only
      // when a row max exceeds it by more than the slack (any lane).
      if (t == 0 || __any(mx > kRescaleSlack)) {
        const float d = t == 0 ? (mx == -INFINITY ? 0.f : mx) : fmaxf(mx, 0.f);
        if (t != 0) {
          const float corr = fast_exp2(-d);
#pragma unroll
          for (int u = 0; u < 4; ++u) l_part[u] *= corr;
#pragma unroll
          for (int dt = 0; dt < 4; ++dt) acc_o[dt] = acc_o[dt] * corr;
        }
        m_ref += d;
#pragma unroll
        for (int i = 0; i < 16; ++i) neg_mref[i] = -m_ref;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) s_acc[mt] = s_acc[mt] - d;
      }
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      between(u);
      const int mt = u >> 1;
      const int base = 8 * (u & 1);
      u32x4 w;
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const float a = fast_exp2(s_acc[mt][base + 2 * e]);
        const float c = fast_exp2(s_acc[mt][base + 2 * e + 1]);
        w[e] = pack_bf16x2(a, c);
        l_part[u] += a + c;
      }
      // Materialise P here: otherwise the compiler sinks the exp work past
      // the barrier into the next MFMA segment, undoing the ping-pong.
      pt[u] = as_bf16x8(w);
      asm volatile("" : "+v"(pt[u]));
    }
    asm volatile("" : "+v"(l_part[0]), "+v"(l_part[1]), "+v"(l_part[2]), "+v"(l_part[3]));
  };
  auto barrier = [&]() __attribute__((always_inline)) {
    __builtin_amdgcn_sched_barrier(0);
    __builtin_amdgcn_s_barrier();
    __builtin_amdgcn_sched_barrier(0);
  };

  // Every wave runs the same sequence  M(0) SM(0) M(1) SM(1) ... M(n)  with a
  // barrier after each piece; group B starts with one idle barrier (and group
  // A ends with one), which shifts B half a step behind A: A's M(t) runs in
  // global segment 2t, B's in 2t+1.
  //
  // Tile T sits in stage T % 4.  Tile DMAs are issued from the softmax
  // segment (VALU-bound, so the memory instructions cost nothing there),
  // never from the MFMA segment.  Group A issues its share of tile T during
  // SM(T-2) (segment 2T-3) and waits for it at the end of iteration T-1
  // (segment 2T-1); group B, half a step later, issues during SM(T-3)
  // (segment 2T-4) and waits at the end of iteration T-2 (segment 2T-2).  So
  // every share of tile T has landed before A's QK(T) in segment 2T, and the
  // stage's previous tile T-4 was last read by B's M(T-3) in segment 2T-5.
  const bool grp_b = wave >= kWaves / 2;
  const int ahead = grp_b ? 3 : 2;  // tile issued during SM(t) is t + ahead
  using T_ = std::true_type;
  using F_ = std::false_type;
  // One M segment + one SM segment.  kPv / kQk say whether PV(t-1) / QK(t)
  // exist (every iteration but the first and the last has both), so that the
  // steady-state M segment is a single block the scheduler can interleave.
  int32_t page_next = 0;  // raw block-table entry of the next tile to load (aligned path)
  int nx_lp = 0, nx_r = 0;  // (aligned) table entry and in-page index of that tile
  auto iteration = [&](int t, auto st, auto has_pv, auto has_qk) __attribute__((always_inline)) {
    constexpr int s = decltype(st)::value;
    constexpr bool kPv = decltype(has_pv)::value;
    constexpr bool kQk = decltype(has_qk)::value;
    using KS = std::integral_constant<int, s>;
    using VS = std::integral_constant<int, (s + kStages - 1) % kStages>;
    // A wave with no row (past the last token of a sequence's last q tile)
    // skips its MFMA and softmax work in the steady-state iterations; its
    // tile loads, waits and barriers stay.  Under the part's power limit the
    // energy it saves goes to the other waves.
    if (!(kPv && kQk) || wave_live) {
    if constexpr (kPv) pv(VS{});
    if constexpr (kQk) qk(KS{});
    if constexpr (kPv && kQk) {
      // 16 PV MFMAs (2 transposing V reads each) then 16 QK MFMAs (1 K read
      // each): every read is issued kAheadMfma MFMAs before the MFMA it feeds.
      constexpr int A = kAheadMfma;
      __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2 * A, 0);
#pragma unroll
      for (int i = 1; i <= 32; ++i) {
        const int next = i + A;  // MFMA whose operands are read now
        __builtin_amdgcn_sched_group_barrier(kSchedMfma, 1, 0);
        if (next <= 16) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 2, 0);
        else if (next <= 32) __builtin_amdgcn_sched_group_barrier(kSchedDsRead, 1, 0);
      }
    }
    }
    wait_vm_lgkm0<15>();  // LDS reads of this segment retired (vmcnt untouched)
    barrier();
    // Tile t + ahead, also when it is past the last tile (into a stage
    // nobody reads again): every iteration issues the same loads, so the
    // softmax has no branch around them and the waits count the same.
    const int ti = t + ahead;
    const int dstage = grp_b ? (s + 3) % kStages : (s + 2) % kStages;
    TileAddrs ta;
    if constexpr (kPv || kQk) ta = tile_addrs(ti * kTileN, page_next, nx_r);
    if constexpr (kPaging == kPageTile && (kPv || kQk)) {  // for the next iteration: tile ti + 1
      if (++nx_r == tpp) {
        nx_r = 0;
        ++nx_lp;
      }
      page_next = page_raw_at(nx_lp);
    } else if constexpr (kPaging == kPageWave && (kPv || kQk)) {
      page_next = page_raw_at(wave_entry(ti + 1));
    }
    // one DMA before each quarter of the softmax: a burst of them would
    // stall on the address queue
    auto between = [&](int u) __attribute__((always_inline)) {
      if constexpr (kPv || kQk) dma_issue(ta, u, dstage);
    };
    if constexpr (kQk) {
      if (!kPv || wave_live) {
        softmax(t, between);
      } else {
#pragma unroll
        for (int u = 0; u < 4; ++u) between(u);
      }
    } else {
#pragma unroll
      for (int u = 0; u < 4; ++u) between(u);
    }
    // this wave's share of tile t + ahead - 1 has landed: at most the loads of
    // tile t + ahead (issued above) may still be outstanding
    wait_vm_lgkm0<kDmaPerTile>();
    barrier();
  };
  using S0 = std::integral_constant<int, 0>;
  using S1 = std::integral_constant<int, 1>;
  using S2 = std::integral_constant<int, 2>;
  using S3 = std::integral_constant<int, 3>;

  // Prologue: A issues tiles 0 and 1, B tiles 0, 1 and 2.  Everyone waits for
  // tile 0 before the first barrier; B also waits for tile 1 before its idle
  // barrier (which ends segment 0, i.e. before A's M(1) in segment 2).
  if (n_tiles > 0) {
    issue_tile_raw(0, raw_pre[0], 0);
    issue_tile_raw(kTileN, raw_pre[1], 1);
    if (grp_b) issue_tile_raw(2 * kTileN, raw_pre[2], 2);
  }
  // raw page id of the first tile the loop loads (tile `ahead`)
  if (kPaging == kPageTile && n_tiles > 0) {
    nx_lp = ahead / tpp;
    nx_r = ahead - nx_lp * tpp;
    page_next = page_raw_at(nx_lp);
  } else if (kPaging == kPageWave && n_tiles > 0) {
    page_next = page_raw_at(wave_entry(ahead));
  }
  const int issued = n_tiles > 0 ? (grp_b ? 3 : 2) : 0;
  if (issued == 3) wait_vm_lgkm0<2 * kDmaPerTile>();
  else if (issued == 2) wait_vm_lgkm0<kDmaPerTile>();
  else wait_vm_lgkm0<0>();
  __builtin_amdgcn_s_barrier();
  if (grp_b) {
    if (issued == 3) wait_vm_lgkm0<kDmaPerTile>();
    else wait_vm_lgkm0<0>();
    barrier();
  }
  PA_PHASE(ph2);

  // iterations t = 0 .. n_tiles: QK(0) alone, then PV(t-1) + QK(t), then
  // PV(n_tiles-1) alone.  Tile t sits in stage t % 4.
  if (n_tiles == 0) {
    iteration(0, S0{}, F_{}, F_{});
  } else {
    iteration(0, S0{}, F_{}, T_{});
    int t = 1;
    for (; t + 4 <= n_tiles; t += 4) {
      iteration(t, S1{}, T_{}, T_{});
      iteration(t + 1, S2{}, T_{}, T_{});
      iteration(t + 2, S3{}, T_{}, T_{});
      iteration(t + 3, S0{}, T_{}, T_{});
    }
    if (t < n_tiles) iteration(t, S1{}, T_{}, T_{});
    if (t + 1 < n_tiles) iteration(t + 1, S2{}, T_{}, T_{});
    if (t + 2 < n_tiles) iteration(t + 2, S3{}, T_{}, T_{});
    switch (n_tiles & 3) {
      case 0: iteration(n_tiles, S0{}, T_{}, F_{}); break;
      case 1: iteration(n_tiles, S1{}, T_{}, F_{}); break;
      case 2: iteration(n_tiles, S2{}, T_{}, F_{}); break;
      default: iteration(n_tiles, S3{}, T_{}, F_{}); break;
    }
  }
  if (!grp_b) barrier();
  wait_vm_lgkm0<0>();  // loads of tiles past the end may still be in flight
  PA_PHASE(ph3);

  // ---- epilogue.  acc_o[dt][i] of lane (n, h) holds row n, d = 32dt +
  // 8(i/4) + 4h + i%4: four consecutive d per i/4, i.e. the h-th half of
  // 16-byte chunk 4dt + i/4.  The normalised bf16 rows go to the wave's own
  // blocks of stages 0 and 1 (every LDS read ended at the loop's last
  // barrier, and this wave's own tile loads have landed), then out four
  // whole 256-byte rows per store.
  const float l_run = sum_xor32((l_part[0] + l_part[1]) + (l_part[2] + l_part[3]));
  const float inv = l_run > 0.f ? 1.f / l_run : 0.f;
#pragma unroll
  for (int dt = 0; dt < 4; ++dt)
#pragma unroll
    for (int q4 = 0; q4 < 4; ++q4) {
      const f32x16& a = acc_o[dt];
      const int i = 4 * q4;
      const u32x2 v = {pack_bf16x2(a[i] * inv, a[i + 1] * inv), pack_bf16x2(a[i + 2] * inv, a[i + 3] * inv)};
      *reinterpret_cast<u32x2 __attribute__((address_space(3)))*>(
          (uintptr_t)(piece(0, n >> 3) + 256 * (n & 7) + 16 * ((4 * dt + q4) ^ (n & 15)) + 8 * h)) = v;
    }
  // A fresh lane index: the row arithmetic below repeats the Q loads'
  // expressions, which the compiler would otherwise carry through the loop.
  int lane_e = lane;
  asm volatile("" : "+v"(lane_e));
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    const int r = 4 * i + (lane_e >> 4);
    const u32x4 v = ds_read16((lds_cbytes)(uintptr_t)(piece(0, r >> 3) + 256 * (r & 7) + 16 * (lane_e & 15)));
    const int rw = wave * 32 + r;
    const int tk = (int)(((uint32_t)rw * gm) >> 24);
    const int hd = rw - tk * p.group;
    const int c = (lane_e & 15) ^ (r & 15);
    if (rw < p.tile_tokens * p.group && tok0 + tk < lq_rows)
      st16(p.out + (int64_t)(q0 + tok0 + tk) * p.o_ts + (int64_t)(kvh * p.group + hd) * p.o_hs + 8 * c, v);
  }
#ifdef PA_PREFILL_PHASES
  PA_PHASE(ph4);
  prefill_phases_store(ph0, ph1, ph2, ph3, ph4, n_tiles, b, qt, kvh);
#endif
}

// The work item numbered `bid`, resolved and run.
template <bool kSoftCap, int kPaging>
__device__ __forceinline__ void prefill_body(const PrefillParams& p, int bid) {
  PrefillWork w;
  if (prefill_resolve(p, bid, w)) prefill_run<kSoftCap, kPaging>(p, w);
}

// Tile paging of a launch (kPageLane / kPageTile / kPageWave).
inline int prefill_paging(int32_t page_size, int64_t slot_stride) {
  if (page_size % kTileN == 0) return kPageTile;
  if ((page_size == 16 || page_size == 32) && prefill_offsets_fit(slot_stride)) return kPageWave;
  return kPageLane;
}

}  // namespace pa
