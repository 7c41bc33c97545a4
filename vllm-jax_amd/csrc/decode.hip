// Split-K paged GQA decode for gfx950: the kernel entries and the host
// launcher.  The work item (one chunk of one sequence and kv head) is
// decode_item in decode_impl.h.
#include <mutex>

#include "any_head.h"
#include "decode_impl.h"

namespace pa {

constexpr int kPlanThreads = 1024;
constexpr int kPlanBins = 512;  // cost classes: 16-token steps of the pair + 1, clamped

// Work list of the decode (one workgroup).  Pair (b, c) = chunk c of
// sequence b is listed when it holds tokens (and chunk 0 of an empty
// sequence when its zeros are written here); its cost is its number of
// 16-token steps.  Pairs are counting-sorted by cost, largest first.
__global__ void __launch_bounds__(kPlanThreads)
decode_plan_kernel(DecodeParams p, int32_t* __restrict__ plan) {
  __shared__ int32_t hist[kPlanBins];
  __shared__ int32_t scan[kPlanThreads];
  const int tid = threadIdx.x;
  for (int i = tid; i < kPlanBins; i += kPlanThreads) hist[i] = 0;
  __syncthreads();
  const int nc = p.n_chunks;
  const int pairs = p.batch * nc;
  const int span = p.pages_per_seq * p.page_size;
  auto bin_of = [&](int i) -> int {  // 0: not listed
    const int b = i / nc, c = i - b * nc;
    const int len = min(p.lengths[b], span);
    const int t0 = c * p.chunk;
    if (t0 >= len) return (c == 0 && p.zero_empty) ? 1 : 0;
    const int steps = (min(len - t0, p.chunk) + kDecodeStep - 1) / kDecodeStep;
    return min(steps + 1, kPlanBins - 1);
  };
  for (int64_t ii = tid; ii < pairs; ii += kPlanThreads) {
    const int i = (int)ii;
    const int c = bin_of(i);
    if (c) atomicAdd(&hist[c], 1);
  }
  __syncthreads();
  // thread t < kPlanBins owns bin kPlanBins - 1 - t (largest first)
  const int local = tid < kPlanBins ? hist[kPlanBins - 1 - tid] : 0;
  int count;
  const int first = block_exclusive_scan<kPlanThreads>(local, scan, count);
  if (tid < kPlanBins) hist[kPlanBins - 1 - tid] = first;  // first rank of the bin
  __syncthreads();
  for (int64_t ii = tid; ii < pairs; ii += kPlanThreads) {
    const int i = (int)ii;
    const int c = bin_of(i);
    if (c) plan[kDecodePlanHeader + atomicAdd(&hist[c], 1)] = i;
  }
  if (tid == 0) plan[0] = count;
}

template <bool kAligned, bool kSoftCap, bool kFp8 = false, bool kShared = false, int kCode = kCodeE4M3,
          int kIds = 1>
__global__ void __launch_bounds__(256, 2)
decode_split_kernel(DecodeParams p) {
  __shared__ DecodeLds red;
  int item;
  if (p.plan) {
    // XCD x = bid % 8 takes ranks x, x + 8, x + 16, ... of the list, all
    // kv heads (and their q-head blocks) of a rank in a row: the XCDs get
    // near-equal token counts, and the kv heads of a token row (adjacent
    // slices of one pool row) are read by one XCD at nearly the same time.
    const int hkv = p.num_kv_heads * p.hblocks;
    const int k = blockIdx.x >> 3;
    const int kr = k / hkv;
    const int r = 8 * kr + (blockIdx.x & 7);
    const __attribute__((address_space(4))) int32_t* pl = (const __attribute__((address_space(4))) int32_t*)p.plan;
    const int count = pl[0];
    const int pair = pl[kDecodePlanHeader + r];  // the list has room for every rank of the grid
    if (r >= count) return;  // uniform over the workgroup
    item = pair * hkv + (k - kr * hkv);
  } else {
    item = xcd_grouped_item(blockIdx.x, gridDim.x);
  }
  decode_item<kDecodeWaves, kAligned, kSoftCap, kFp8, kShared, kCode, kIds>(p, item, &red.o[0][0][0],
                                                                            &red.m[0][0], &red.l[0][0]);
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
  if (!decode_has_row(p, b)) return;
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
  uint32_t* dst = reinterpret_cast<uint32_t*>(p.out + decode_row(p, b) * p.out_bs + (int64_t)h * p.out_hs) + lane;
  *dst = pack_bf16x2(o0 * inv, o1 * inv);
}

// The merge of launches with many chunks per sequence (a few long
// sequences): one workgroup per (sequence, q head), so that its partials are
// read in parallel.  Eight groups of 32 threads take every eighth chunk, a
// thread four d values of it (16 bytes); the sums of the groups meet in LDS.
constexpr int kMergeWideChunks = 4;  // launches with more chunks per sequence take the wide merge
__global__ void __launch_bounds__(256)
decode_merge_wide_kernel(DecodeParams p) {
  __shared__ float red[8][kHeadDim];
  __shared__ float red_m[4], red_l[4];
  const int tid = threadIdx.x;
  const int lane = tid & 63, wave = tid >> 6;
  const int b = (int)(blockIdx.x / p.num_heads);
  const int h = (int)(blockIdx.x - (int64_t)b * p.num_heads);
  if (!decode_has_row(p, b)) return;  // uniform over the workgroup
  const int kvh = h / p.group;
  const int qi = h - kvh * p.group;
  const int len = min(p.lengths[b], p.pages_per_seq * p.page_size);
  const int nc = len > 0 ? min((len + p.chunk - 1) / p.chunk, p.n_chunks) : 0;
  if (nc == 1) return;
  const int64_t base = ((int64_t)b * p.num_kv_heads + kvh) * p.n_chunks;
  auto ml = [&](int c) __attribute__((always_inline)) { return p.ws_ml + 2 * ((base + c) * p.group + qi); };
  // M = the largest chunk max; L = sum_c l_c 2^(m_c - M)
  float mx = -INFINITY;
  for (int c = tid; c < nc; c += 256) mx = fmaxf(mx, ml(c)[0]);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o));
  if (lane == 0) red_m[wave] = mx;
  __syncthreads();
  const float mmax = fmaxf(fmaxf(red_m[0], red_m[1]), fmaxf(red_m[2], red_m[3]));
  float ls = 0.f;
  for (int c = tid; c < nc; c += 256) ls += ml(c)[1] * fast_exp2(ml(c)[0] - mmax);
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) ls += __shfl_xor(ls, o);
  if (lane == 0) red_l[wave] = ls;
  // O = sum_c o_c 2^(m_c - M): group g = tid / 32 takes chunks g, g + 8, ...
  const int g = tid >> 5, e = tid & 31;
  float4 o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll 4
  for (int c = g; c < nc; c += 8) {
    const int64_t part = (base + c) * p.group + qi;
    const float w = fast_exp2(p.ws_ml[2 * part] - mmax);
    const float4 v = *reinterpret_cast<const float4*>(p.ws_o + part * kHeadDim + 4 * e);
    o.x += v.x * w;
    o.y += v.y * w;
    o.z += v.z * w;
    o.w += v.w * w;
  }
  *reinterpret_cast<float4*>(&red[g][4 * e]) = o;
  __syncthreads();
  if (tid >= 32) return;
  const float lsum = red_l[0] + red_l[1] + red_l[2] + red_l[3];
  const float inv = lsum > 0.f ? 1.f / lsum : 0.f;
  float4 t = *reinterpret_cast<const float4*>(&red[0][4 * e]);
#pragma unroll
  for (int k = 1; k < 8; ++k) {
    const float4 v = *reinterpret_cast<const float4*>(&red[k][4 * e]);
    t.x += v.x;
    t.y += v.y;
    t.z += v.z;
    t.w += v.w;
  }
  uint16_t* dst = p.out + decode_row(p, b) * p.out_bs + (int64_t)h * p.out_hs + 4 * e;
  *reinterpret_cast<u32x2*>(dst) = u32x2{pack_bf16x2(t.x * inv, t.y * inv), pack_bf16x2(t.z * inv, t.w * inv)};
}

void launch_decode_merge(const DecodeParams& p, hipStream_t s) {
  const int64_t pairs = (int64_t)p.batch * p.num_heads;
  if (p.n_chunks > kMergeWideChunks) decode_merge_wide_kernel<<<dim3((unsigned)pairs), dim3(256), 0, s>>>(p);
  else decode_merge_kernel<<<dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, s>>>(p);
}

constexpr int64_t kDecodePlanMinItems = 2048;  // workgroups from which pa_decode builds a work list

constexpr int kDecodeLongChunk = 4096;  // tokens per item on large launches
constexpr int kDecodeShortChunk = 1024;  // tokens per item of the generic decode at small head sizes

// The generic decode (one wave per item) at head sizes below 128 other than
// 64 runs best with 1024-token items; same-process A/B on the Qwen3-8B
// batch's contexts, 1024 against 2048 tokens: 48 -5.6 %, 80 -0.2 %, 96
// -1.3 %, 112 -1.2 %; 64 +1.6 %, 160 +1.6 %, 192 +3.6 %, 224 +1.9 %.
static bool decode_any_short_chunk(int head_dim) { return head_dim < 128 && head_dim != 64; }

constexpr int kDecodeMinChunk = 512;        // shortest item of a small launch
constexpr int64_t kDecodeFillPairs = 64;  // (sequence, chunk) pairs of a launch that fills the CUs

// A small launch (fewer than kDecodeFillPairs pairs over the widest table
// row: a few long sequences) halves its chunk, down to kDecodeMinChunk
// tokens, until it has that many: with 8 kv heads, 512 items of four waves,
// one per workgroup slot (two per CU).  One 32 768-token sequence of the
// Qwen3-8B heads took 2048-token items, 128 workgroups for 256 CUs: 38.8 ->
// 29.0 us with 512-token ones (same process).  Halving launches that
// already hold 512 items cost 1-2 % (16 x 8192 and 64 x 2048 tokens).
// Depends on the batch and the table only, so the workspace size gives the
// same chunk.
static int decode_fill_chunk(int chunk, int32_t batch, int64_t span) {
  while (chunk > kDecodeMinChunk && (int64_t)batch * ((span + chunk - 1) / chunk) < kDecodeFillPairs) chunk /= 2;
  return chunk;
}

// Chunks of the widest table row at the shortest chunk a launch can take:
// the workspace holds one partial per (sequence, q head, chunk) for them.
static int decode_chunks(int32_t batch, int32_t pages_per_seq, int32_t page_size, int32_t head_dim) {
  const int64_t max_tokens = (int64_t)pages_per_seq * page_size;
  int chunk = decode_chunk_tokens(page_size);
  if (head_dim != kHeadDim && decode_any_short_chunk(head_dim)) chunk = min(chunk, kDecodeShortChunk);
  if (head_dim == kHeadDim) chunk = decode_fill_chunk(chunk, batch, max_tokens);  // decode_split_kernel
  return (int)((max_tokens + chunk - 1) / chunk);
}

// Tokens per work item of decode_split_kernel.  An item pays a fixed cost
// (q, the chunk's page ids, the waves' combine, a partial and its merge),
// so on launches that still hold kDecodePlanMinItems items of 4096 tokens
// the chunk is 4096; else decode_chunk_tokens.  Pages of 64+ tokens keep a
// 4096-token chunk within 64 page ids (one per lane); pages of 16, 32 or 48
// tokens span 256, 128 or up to 87 and take the four-ids-per-lane kernels
// (decode_chunk_span).  The workspace is sized for the shorter chunks, so
// either fits it.
static int decode_split_chunk(int32_t page_size, int32_t batch, int32_t pages_per_seq, int64_t vheads) {
  const int base = decode_chunk_tokens(page_size);
  if (page_size < 64 && page_size % kDecodeStep != 0) return base;
  const int64_t chunks = ((int64_t)pages_per_seq * page_size + kDecodeLongChunk - 1) / kDecodeLongChunk;
  return (int64_t)batch * chunks * vheads >= kDecodePlanMinItems ? kDecodeLongChunk : base;
}

// Pages a chunk of `chunk` tokens spans at most (aligned pages).  Chunks
// start at multiples of `chunk`: when page_size divides it a chunk spans
// chunk / page_size pages, else at most floor((chunk + page_size - 2) /
// page_size) + 1.  decode_split_kernel holds one page id per lane up to 64
// pages and four (kIds = 4) up to 256: every chunk of 4096 tokens or less
// over pages of 16+ tokens.
static int decode_chunk_span(int32_t page_size, int chunk) {
  return chunk % page_size == 0 ? chunk / page_size : (chunk + page_size - 2) / page_size + 1;
}

// Tokens per work item of the generic decode (decode_any_kernel, one wave
// per item): 1024 at the head sizes of decode_any_short_chunk; 4096 at head
// size 256 on launches that still hold kDecodePlanMinItems such items (-1.7 %
// there over 256-token pages, -3.4 % over 16-token ones, where 4096 cost
// 4-9 % at 64, 96 and 32 q heads per kv head; its page ids are scalar loads
// per step, so any chunk fits); else decode_chunk_tokens.
static int decode_any_chunk(int32_t head_dim, int32_t page_size, int32_t batch, int32_t pages_per_seq,
                            int64_t vheads) {
  const int base = decode_chunk_tokens(page_size);
  if (decode_any_short_chunk(head_dim)) return min(base, kDecodeShortChunk);
  if (head_dim == 256) return decode_split_chunk(page_size, batch, pages_per_seq, vheads);
  return base;
}

}  // namespace pa

using namespace pa;

// ---- pa_decode_noalloc: pa_decode with its workspace in a static device
// array, for callers that cannot allocate device memory.  Every GPU the
// library runs on holds its own copy of `scratch` until the process ends;
// the host refers to it only through the address hipGetSymbolAddress returns
// for the current device (the symbol's host-side name is not a device
// address).  The decode workspace needs no clearing (the merge reads only the
// partials of chunks a launch wrote, and a listed launch rewrites the list),
// so nothing is zeroed between calls.  Calls that overlap on one GPU share
// the array and race.
constexpr size_t kNoAllocScratchBytes = (size_t)64 << 20;
static __device__ __align__(256) char scratch[kNoAllocScratchBytes];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxScratchDevices];  // per device, set once with that device current

// Device address of `scratch` on the current device (looked up on the first
// call per device).
int noalloc_scratch(const char* name, void** out) {
  int dev = -1;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return fail(PA_ERR_LAUNCH, "%s: hipGetDevice failed: %s", name, hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxScratchDevices)
    return fail(PA_ERR_UNSUPPORTED, "%s: device %d beyond the %d devices the scratch table holds", name, dev,
                kMaxScratchDevices);
  std::lock_guard<std::mutex> g(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* ptr = nullptr;
    e = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !ptr)
      return fail(PA_ERR_LAUNCH, "%s: hipGetSymbolAddress(scratch) failed on device %d: %s", name, dev,
                  hipGetErrorString(e));
    g_scratch_ptr[dev] = ptr;
  }
  *out = g_scratch_ptr[dev];
  return PA_OK;
}
}  // namespace

// Partials (o, then max / sum), then at a 256-byte boundary the work list:
// a header and one int per pair, the pair count rounded up to 8.
static size_t decode_partials_bytes(int32_t batch, int32_t num_heads, int32_t head_dim, int32_t n_chunks) {
  const size_t parts = (size_t)batch * num_heads * n_chunks;
  return (parts * ((size_t)head_dim + 2) * sizeof(float) + 255) / 256 * 256;
}

extern "C" size_t pa_decode_workspace_size(int32_t batch, int32_t num_heads, int32_t head_dim,
                                           int32_t pages_per_seq, int32_t page_size) {
  if (batch <= 0 || num_heads <= 0 || head_dim <= 0 || pages_per_seq <= 0 || page_size <= 0) return 0;
  const int n_chunks = decode_chunks(batch, pages_per_seq, page_size, head_dim);
  const size_t pairs8 = ((size_t)batch * n_chunks + 7) / 8 * 8;
  return decode_partials_bytes(batch, num_heads, head_dim, n_chunks) + (kDecodePlanHeader + pairs8) * sizeof(int32_t);
}

// Shared argument checks and launch of pa_decode / pa_decode_fp8.  `prm`
// arrives with the cache pointers (and scales) set; the rest is filled here.
// Launch of the split kernel over 1-byte codes of type `code` (kCodeE4M3,
// kCodeI8, kCodeU8).
template <int kCode, int kIds>
static void launch_decode_codes(const DecodeParams& prm, bool cap, bool shared, dim3 grid, dim3 block,
                                hipStream_t s) {
  if (!cap && shared) decode_split_kernel<true, false, true, true, kCode, kIds><<<grid, block, 0, s>>>(prm);
  else if (!cap) decode_split_kernel<true, false, true, false, kCode, kIds><<<grid, block, 0, s>>>(prm);
  else decode_split_kernel<true, true, true, false, kCode, kIds><<<grid, block, 0, s>>>(prm);
}

template <int kCode>
static void launch_decode_codes(const DecodeParams& prm, bool cap, bool shared, bool wide, dim3 grid, dim3 block,
                                hipStream_t s) {
  if (wide) launch_decode_codes<kCode, 4>(prm, cap, shared, grid, block, s);
  else launch_decode_codes<kCode, 1>(prm, cap, shared, grid, block, s);
}

static int decode_common(const char* name, DecodeParams& prm, bool fp8, const uint16_t* q, int64_t q_batch_stride,
                         int64_t q_head_stride, int32_t num_pages, int32_t page_size, int64_t page_stride,
                         int64_t slot_stride, int64_t head_stride, const int32_t* block_tables, int64_t bt_stride,
                         int32_t pages_per_seq, const int32_t* lengths, int32_t batch, int32_t num_heads,
                         int32_t num_kv_heads, int32_t head_dim, float scale, float soft_cap, uint16_t* out,
                         int64_t out_batch_stride, int64_t out_head_stride, void* workspace, size_t workspace_bytes,
                         void* stream, int code = kCodeE4M3) {
  if (fp8 && code != kCodeE4M3 && code != kCodeI8 && code != kCodeU8)
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: code_type %d is not one of PA_CODE_E4M3 (0), PA_CODE_INT8 (1), "
                "PA_CODE_UINT8 (2)", name, code);
  if (batch < 0 || num_heads <= 0 || num_kv_heads <= 0 || num_pages <= 0 || page_size <= 0 ||
      pages_per_seq < 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "%s: bad sizes (batch=%d, num_heads=%d, num_kv_heads=%d, num_pages=%d, "
                "page_size=%d, pages_per_seq=%d)",
                name, batch, num_heads, num_kv_heads, num_pages, page_size, pages_per_seq);
  if (num_heads % num_kv_heads != 0)
    return fail(PA_ERR_INVALID_ARGUMENT,
                "%s: Number of Q heads must be divisible by number of KV heads. Got %d and %d.", name,
                num_heads, num_kv_heads);
  if (head_dim != kHeadDim && !any_head_dim(head_dim))
    return fail(PA_ERR_UNSUPPORTED, "%s: head_dim %d not supported (128, or a multiple of 16 from 16 to 256)", name,
                head_dim);
  const int group = num_heads / num_kv_heads;
  // The generic kernels (any_head.hip) take every head size but 128, and
  // also 128 over bf16 pages with more than 16 q heads per kv head: their
  // items cover 32 q heads (one 32-wide MFMA column block), where this
  // kernel's cover 16, so each kv head's K/V is read half as often (32 q
  // heads per kv head: 261 -> 236 us for the Qwen3-8B batch's contexts).
  // Over float8 pages this kernel stays faster (155 vs 284 us).
  const bool any_d = head_dim != kHeadDim || (!fp8 && group > 16);
  if (fp8 && !any_d && page_size % kDecodeStep != 0)
    return fail(PA_ERR_UNSUPPORTED, "%s: quantized pages need page_size %% %d == 0 (got %d)", name, kDecodeStep,
                page_size);
  if (batch == 0) return PA_OK;
  if (num_kv_heads == 1) {  // a size-1 dimension's stride is arbitrary (and never used)
    head_stride = 0;
    prm.sc_head_stride = 0;
  }
  const void* kc = fp8 ? (const void*)prm.k8 : (const void*)prm.k_cache;
  const void* vc = fp8 ? (const void*)prm.v8 : (const void*)prm.v_cache;
  if (!q || !kc || !vc || !block_tables || !lengths || !out || (fp8 && (!prm.k_scales || !prm.v_scales)))
    return fail(PA_ERR_INVALID_ARGUMENT, "%s: null pointer", name);
  const uintptr_t align_bits = (uintptr_t)q | (uintptr_t)kc | (uintptr_t)vc | (uintptr_t)out |
                               (fp8 ? ((uintptr_t)prm.k_scales | (uintptr_t)prm.v_scales) : 0);
  if ((align_bits & 15u) || (q_batch_stride | q_head_stride | page_stride | slot_stride | head_stride) % 8 ||
      (out_batch_stride | out_head_stride) % 8 ||
      (fp8 && ((page_stride | slot_stride | head_stride) % 16 || (prm.sc_page_stride | prm.sc_head_stride) % 4)))
    return fail(PA_ERR_UNSUPPORTED, "%s: operands must be 16-byte aligned with strides multiple of 8", name);
  if ((int64_t)pages_per_seq * page_size > 0x7fffffffLL)
    return fail(PA_ERR_UNSUPPORTED, "%s: block table spans more than 2^31 tokens", name);
  if ((int64_t)batch * num_heads > 0x7fffffffLL)  // the merge grid: up to one workgroup per (sequence, q head)
    return fail(PA_ERR_UNSUPPORTED, "%s: %lld (sequence, q head) rows, more than 2^31", name,
                (long long)batch * num_heads);
  const size_t need = pa_decode_workspace_size(batch, num_heads, head_dim, pages_per_seq, page_size);
  if (pages_per_seq > 0 && (!workspace || workspace_bytes < need || ((uintptr_t)workspace & 255u)))
    return fail(PA_ERR_WORKSPACE, "%s: 256-byte aligned workspace of %zu bytes needed, %zu given", name, need,
                workspace_bytes);

  prm.q = q;
  prm.q_bs = q_batch_stride;
  prm.q_hs = q_head_stride;
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
  prm.hblocks = (group + 15) / 16;
  // work items per (sequence, chunk): one per kv head and block of q heads
  // (16 per item here, 32 in the generic kernels)
  const int64_t vheads = (int64_t)num_kv_heads * (any_d ? (group + 31) / 32 : prm.hblocks);
  prm.chunk = any_d ? decode_any_chunk(head_dim, page_size, batch, pages_per_seq, vheads)
                    : decode_fill_chunk(decode_split_chunk(page_size, batch, pages_per_seq, vheads), batch,
                                        (int64_t)pages_per_seq * page_size);
  prm.n_chunks =
      pages_per_seq > 0 ? (int)(((int64_t)pages_per_seq * page_size + prm.chunk - 1) / prm.chunk) : 0;
  // (this kernel, aligned pages) the chunk's page ids, one or four per lane
  const int span = !any_d && page_size % kDecodeStep == 0 ? decode_chunk_span(page_size, prm.chunk) : 0;
  if (span > 4 * 64)
    return fail(PA_ERR_UNSUPPORTED, "%s: a %d-token chunk spans %d pages of %d tokens (max 256)", name, prm.chunk,
                span, page_size);
  prm.soft_cap = soft_cap > 0.f ? soft_cap : 0.f;
  prm.logit_scale = prm.soft_cap > 0.f ? scale : scale * kLog2e;
  const size_t parts = (size_t)batch * num_heads * prm.n_chunks;
  prm.ws_o = reinterpret_cast<float*>(workspace);
  prm.ws_ml = prm.ws_o + parts * head_dim;
  prm.out = out;
  prm.out_bs = out_batch_stride;
  prm.out_hs = out_head_stride;
  prm.rows = nullptr;
  prm.row_limit = 0;
  prm.zero_empty = 0;

  hipStream_t s = (hipStream_t)stream;
  const int64_t pairs = (int64_t)batch * prm.n_chunks;
  // The work list pays for its launch once the grid is several waves of
  // workgroups deep (two per CU, 256 CUs).
  const bool planned = pairs > 0 && pairs * vheads >= kDecodePlanMinItems;
  const int64_t blocks = planned ? (pairs + 7) / 8 * 8 * vheads : pairs * vheads;
  if (blocks > 0x7fffffff)
    return fail(PA_ERR_UNSUPPORTED, "%s: grid of %lld workgroups too large", name, (long long)blocks);
  if (planned) {
    int32_t* plan = reinterpret_cast<int32_t*>(reinterpret_cast<char*>(workspace) +
                                               decode_partials_bytes(batch, num_heads, head_dim, prm.n_chunks));
    decode_plan_kernel<<<dim3(1), dim3(kPlanThreads), 0, s>>>(prm, plan);
    int rc = launch_status(name);
    if (rc) return rc;
    prm.plan = plan;
  }
  if (any_d) return decode_any_launch(name, prm, head_dim, s, fp8 ? code : -1);
  if (blocks > 0) {  // no table pages: every row is zero, only the merge pass runs
    const bool aligned = page_size % kDecodeStep == 0;
    const bool cap = prm.soft_cap > 0.f;
    const dim3 grid((unsigned)blocks), block(64 * kDecodeWaves);
    // (quantized pages) more than 16 q heads per kv head: several items read
    // each kv head's K/V, so the loads stay cacheable (the soft cap keeps the
    // streaming form); bf16 pages with more than 16 went to the generic kernel
    const bool shared = prm.hblocks > 1;
    const bool wide = span > 64;
    if (fp8 && code == kCodeI8) launch_decode_codes<kCodeI8>(prm, cap, shared, wide, grid, block, s);
    else if (fp8 && code == kCodeU8) launch_decode_codes<kCodeU8>(prm, cap, shared, wide, grid, block, s);
    else if (fp8) launch_decode_codes<kCodeE4M3>(prm, cap, shared, wide, grid, block, s);
    else if (wide && !cap) decode_split_kernel<true, false, false, false, kCodeE4M3, 4><<<grid, block, 0, s>>>(prm);
    else if (wide) decode_split_kernel<true, true, false, false, kCodeE4M3, 4><<<grid, block, 0, s>>>(prm);
    else if (aligned && !cap) decode_split_kernel<true, false><<<grid, block, 0, s>>>(prm);
    else if (aligned) decode_split_kernel<true, true><<<grid, block, 0, s>>>(prm);
    else if (!cap) decode_split_kernel<false, false><<<grid, block, 0, s>>>(prm);
    else decode_split_kernel<false, true><<<grid, block, 0, s>>>(prm);
    int rc = launch_status(name);
    if (rc) return rc;
  }
  launch_decode_merge(prm, s);
  return launch_status(name);
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
  DecodeParams prm{};
  prm.k_cache = k_cache;
  prm.v_cache = v_cache;
  return decode_common("pa_decode", prm, false, q, q_batch_stride, q_head_stride, num_pages, page_size, page_stride,
                       slot_stride, head_stride, block_tables, bt_stride, pages_per_seq, lengths, batch, num_heads,
                       num_kv_heads, head_dim, scale, soft_cap, out, out_batch_stride, out_head_stride, workspace,
                       workspace_bytes, stream);
}

extern "C" size_t pa_decode_noalloc_max_workspace(void) { return kNoAllocScratchBytes; }

extern "C" int pa_decode_noalloc(const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
                                 const uint16_t* k_cache, const uint16_t* v_cache,
                                 int32_t num_pages, int32_t page_size,
                                 int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                                 const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                                 const int32_t* lengths, int32_t batch,
                                 int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                                 float scale, float soft_cap,
                                 uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride, void* stream) {
  // the size limit is checked before the device is touched
  const size_t need = pa_decode_workspace_size(batch, num_heads, head_dim, pages_per_seq, page_size);
  if (need > kNoAllocScratchBytes)
    return fail(PA_ERR_WORKSPACE,
                "pa_decode_noalloc: this launch needs %zu bytes of workspace, more than the %zu bytes of its static "
                "scratch (batch=%d, num_heads=%d, pages_per_seq=%d, page_size=%d); use pa_decode with a workspace",
                need, kNoAllocScratchBytes, batch, num_heads, pages_per_seq, page_size);
  void* ws = nullptr;
  if (need > 0 && batch > 0) {
    int rc = noalloc_scratch("pa_decode_noalloc", &ws);
    if (rc) return rc;
  }
  DecodeParams prm{};
  prm.k_cache = k_cache;
  prm.v_cache = v_cache;
  return decode_common("pa_decode_noalloc", prm, false, q, q_batch_stride, q_head_stride, num_pages, page_size,
                       page_stride, slot_stride, head_stride, block_tables, bt_stride, pages_per_seq, lengths, batch,
                       num_heads, num_kv_heads, head_dim, scale, soft_cap, out, out_batch_stride, out_head_stride, ws,
                       ws ? kNoAllocScratchBytes : 0, stream);
}

extern "C" int pa_decode_quant(int32_t code_type, const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
                               const uint8_t* k_cache, const uint8_t* v_cache,
                               const float* k_scales, const float* v_scales,
                               int32_t num_pages, int32_t page_size,
                               int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                               int64_t scale_page_stride, int64_t scale_head_stride,
                               const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                               const int32_t* lengths, int32_t batch,
                               int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                               float scale, float soft_cap,
                               uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride,
                               void* workspace, size_t workspace_bytes, void* stream) {
  DecodeParams prm{};
  prm.k8 = k_cache;
  prm.v8 = v_cache;
  prm.k_scales = k_scales;
  prm.v_scales = v_scales;
  prm.sc_page_stride = scale_page_stride;
  prm.sc_head_stride = scale_head_stride;
  return decode_common("pa_decode_quant", prm, true, q, q_batch_stride, q_head_stride, num_pages, page_size,
                       page_stride, slot_stride, head_stride, block_tables, bt_stride, pages_per_seq, lengths, batch,
                       num_heads, num_kv_heads, head_dim, scale, soft_cap, out, out_batch_stride, out_head_stride,
                       workspace, workspace_bytes, stream, code_type);
}

extern "C" int pa_decode_fp8(const uint16_t* q, int64_t q_batch_stride, int64_t q_head_stride,
                             const uint8_t* k_cache, const uint8_t* v_cache,
                             const float* k_scales, const float* v_scales,
                             int32_t num_pages, int32_t page_size,
                             int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                             int64_t scale_page_stride, int64_t scale_head_stride,
                             const int32_t* block_tables, int64_t bt_stride, int32_t pages_per_seq,
                             const int32_t* lengths, int32_t batch,
                             int32_t num_heads, int32_t num_kv_heads, int32_t head_dim,
                             float scale, float soft_cap,
                             uint16_t* out, int64_t out_batch_stride, int64_t out_head_stride,
                             void* workspace, size_t workspace_bytes, void* stream) {
  DecodeParams prm{};
  prm.k8 = k_cache;
  prm.v8 = v_cache;
  prm.k_scales = k_scales;
  prm.v_scales = v_scales;
  prm.sc_page_stride = scale_page_stride;
  prm.sc_head_stride = scale_head_stride;
  return decode_common("pa_decode_fp8", prm, true, q, q_batch_stride, q_head_stride, num_pages, page_size,
                       page_stride, slot_stride, head_stride, block_tables, bt_stride, pages_per_seq, lengths, batch,
                       num_heads, num_kv_heads, head_dim, scale, soft_cap, out, out_batch_stride, out_head_stride,
                       workspace, workspace_bytes, stream, kCodeE4M3);
}
