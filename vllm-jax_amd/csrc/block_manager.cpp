// Host-side KV block manager: the reference's FIFO block allocator
// (vllm/src/kv_cache_manager.py:14-70) with two additions, both off the
// reference's path unless asked for:
//
//   * prefix caching: a full block is keyed by a chained 64-bit hash of its
//     tokens and its predecessor; a prefill whose leading full blocks match
//     cached ones takes them (reference count + 1) instead of new blocks.
//     A hit is verified against the stored tokens and predecessor block, so a
//     hash collision can never share the wrong block.  Freed cached blocks
//     stay reusable in the free queue until they are handed out again.
//   * fork + copy-on-write: a forked sequence shares every block of its
//     parent; the first write into a shared block moves the writer to a
//     fresh block and records a (src, dst) page copy for the device
//     (pa_copy_blocks).
//
// With prefix caching off and no forks, every call returns exactly what the
// reference returns for the same sequence of calls (block ids, order,
// reference counts, free-queue order).
#include <cstdint>
#include <cstring>
#include <mutex>
#include <unordered_map>
#include <vector>

#include "pa_errors.h"

namespace pa {
namespace {

struct SeqState {
  std::vector<int32_t> table;
  int32_t cached_tokens = 0;  // prompt tokens found in cached blocks at the last prefill
};

constexpr uint64_t kHashSeed = 0x9e3779b97f4a7c15ull;

// splitmix64 finaliser: a bijective 64-bit mixer.
inline uint64_t mix64(uint64_t x) {
  x += 0x9e3779b97f4a7c15ull;
  x = (x ^ (x >> 30)) * 0xbf58476d1ce4e5b9ull;
  x = (x ^ (x >> 27)) * 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

}  // namespace

struct BlockManager {
  int32_t num_blocks = 0, block_size = 0;
  bool prefix = false;
  std::mutex mu;
  std::vector<int32_t> ref;
  // free queue: intrusive doubly-linked FIFO over block ids
  std::vector<int32_t> prev, next;
  std::vector<uint8_t> in_free;
  int32_t head = -1, tail = -1, nfree = 0;
  // prefix cache
  std::vector<uint8_t> hashed;
  std::vector<uint64_t> bhash;
  std::vector<int32_t> parent;   // predecessor block of a cached block (-1: first block)
  std::vector<int32_t> btokens;  // [num_blocks][block_size] tokens of cached blocks
  std::unordered_map<uint64_t, int32_t> cache;
  std::unordered_map<int64_t, SeqState> seqs;
  std::vector<int32_t> copy_src, copy_dst;

  void push_back(int32_t b) {
    prev[b] = tail;
    next[b] = -1;
    if (tail >= 0) next[tail] = b;
    else head = b;
    tail = b;
    in_free[b] = 1;
    ++nfree;
  }
  void unlink(int32_t b) {
    if (prev[b] >= 0) next[prev[b]] = next[b];
    else head = next[b];
    if (next[b] >= 0) prev[next[b]] = prev[b];
    else tail = prev[b];
    in_free[b] = 0;
    --nfree;
  }
  // kv_cache_manager.py:48 / :58: take the oldest free block
  int32_t pop_front() {
    const int32_t b = head;
    unlink(b);
    if (hashed[b]) {  // the block's cached contents are about to be overwritten
      auto it = cache.find(bhash[b]);
      if (it != cache.end() && it->second == b) cache.erase(it);
      hashed[b] = 0;
    }
    return b;
  }
  uint64_t chain(uint64_t h, const int32_t* toks) const {
    for (int32_t i = 0; i < block_size; ++i) h = mix64(h ^ (uint32_t)toks[i]);
    return h;
  }
  // cached block holding tokens `toks` after block `par`, or -1
  int32_t lookup(uint64_t h, int32_t par, const int32_t* toks) const {
    auto it = cache.find(h);
    if (it == cache.end()) return -1;
    const int32_t c = it->second;
    if (parent[c] != par || std::memcmp(&btokens[(size_t)c * block_size], toks, sizeof(int32_t) * block_size) != 0)
      return -1;
    return c;
  }
  void remember(int32_t b, uint64_t h, int32_t par, const int32_t* toks) {
    if (hashed[b] || cache.count(h)) return;  // first writer keeps the key
    cache.emplace(h, b);
    hashed[b] = 1;
    bhash[b] = h;
    parent[b] = par;
    std::memcpy(&btokens[(size_t)b * block_size], toks, sizeof(int32_t) * block_size);
  }
  // leading full blocks (before the last token) found in the cache
  int32_t prefix_hits(const int32_t* toks, int64_t n, std::vector<int32_t>* out) const {
    if (!prefix || !toks || n <= 0) return 0;
    const int64_t full = (n - 1) / block_size;
    uint64_t h = kHashSeed;
    int32_t par = -1, hits = 0;
    for (int64_t i = 0; i < full; ++i) {
      const int32_t* t = toks + i * block_size;
      h = chain(h, t);
      const int32_t c = lookup(h, par, t);
      if (c < 0) break;
      if (out) out->push_back(c);
      par = c;
      ++hits;
    }
    return hits;
  }
};

}  // namespace pa

using namespace pa;

struct pa_block_manager {
  BlockManager m;
};

extern "C" pa_block_manager* pa_bm_create(int32_t num_blocks, int32_t block_size, int32_t enable_prefix_caching) {
  if (num_blocks <= 0 || block_size <= 0) {
    fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_create: bad sizes (num_blocks=%d, block_size=%d)", num_blocks, block_size);
    return nullptr;
  }
  auto* h = new pa_block_manager;
  BlockManager& m = h->m;
  m.num_blocks = num_blocks;
  m.block_size = block_size;
  m.prefix = enable_prefix_caching != 0;
  m.ref.assign(num_blocks, 0);
  m.prev.assign(num_blocks, -1);
  m.next.assign(num_blocks, -1);
  m.in_free.assign(num_blocks, 0);
  m.hashed.assign(num_blocks, 0);
  m.bhash.assign(num_blocks, 0);
  m.parent.assign(num_blocks, -1);
  if (m.prefix) m.btokens.assign((size_t)num_blocks * block_size, 0);
  for (int32_t b = 0; b < num_blocks; ++b) m.push_back(b);  // :17-18, id order
  return h;
}

extern "C" void pa_bm_destroy(pa_block_manager* h) { delete h; }

extern "C" int32_t pa_bm_num_free_blocks(pa_block_manager* h) {
  if (!h) return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_num_free_blocks: null manager");
  std::lock_guard<std::mutex> g(h->m.mu);
  return h->m.nfree;
}

extern "C" int pa_bm_can_allocate(pa_block_manager* h, int64_t seq_id, const int32_t* token_ids, int32_t num_tokens,
                                  int32_t is_prefill) {
  if (!h || num_tokens < 0) return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_can_allocate: bad arguments");
  BlockManager& m = h->m;
  std::lock_guard<std::mutex> g(m.mu);
  SeqState& s = m.seqs[seq_id];  // :24-27 creates the table
  const int32_t bs = m.block_size;
  if (is_prefill) {
    // :34-36, minus the blocks a prefix hit takes from the cache
    const int64_t needed = ((int64_t)num_tokens + bs - 1) / bs;
    std::vector<int32_t> hits;
    if (s.table.empty()) m.prefix_hits(token_ids, num_tokens, &hits);
    int64_t from_free = needed - (int64_t)hits.size();
    for (int32_t c : hits) from_free += m.in_free[c];  // a free cached block leaves the queue too
    return from_free <= m.nfree ? 1 : 0;
  }
  if (s.table.empty()) return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_can_allocate: decode of sequence %lld without blocks",
                                   (long long)seq_id);
  int64_t needed = num_tokens % bs == 0 ? 1 : 0;  // :38-41
  const int64_t idx = ((int64_t)num_tokens - 1) / bs;
  if (num_tokens > 0 && idx < (int64_t)s.table.size() && m.ref[s.table[idx]] > 1) ++needed;  // copy-on-write
  return needed <= m.nfree ? 1 : 0;
}

extern "C" int pa_bm_allocate(pa_block_manager* h, int64_t seq_id, const int32_t* token_ids, int32_t num_tokens,
                              int32_t is_prefill) {
  if (!h || num_tokens < 0) return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_allocate: bad arguments");
  BlockManager& m = h->m;
  std::lock_guard<std::mutex> g(m.mu);
  SeqState& s = m.seqs[seq_id];
  const int32_t bs = m.block_size;
  if (is_prefill) {
    // :46-51, with cached leading blocks taken first
    // Every check comes before the first change of state: a refused
    // allocation leaves the table, the reference counts and the queue as
    // they were (as pa_bm_can_allocate counts it).
    const int64_t needed = ((int64_t)num_tokens + bs - 1) / bs;
    std::vector<int32_t> hits;
    if (s.table.empty()) m.prefix_hits(token_ids, num_tokens, &hits);
    int64_t from_free = needed - (int64_t)s.table.size() - (int64_t)hits.size();
    for (int32_t c : hits) from_free += m.in_free[c];  // a free cached block leaves the queue too
    if (from_free > m.nfree)
      return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_allocate: %lld blocks needed, %d free", (long long)from_free,
                  m.nfree);
    for (int32_t c : hits) {
      if (m.in_free[c]) m.unlink(c);
      ++m.ref[c];
      s.table.push_back(c);
    }
    s.cached_tokens = (int32_t)hits.size() * bs;
    while ((int64_t)s.table.size() < needed) {
      const int32_t b = m.pop_front();
      ++m.ref[b];
      s.table.push_back(b);
    }
    if (m.prefix && token_ids) {  // make this prompt's full blocks findable
      uint64_t hh = kHashSeed;
      int32_t par = -1;
      for (int64_t i = 0; i < (int64_t)num_tokens / bs; ++i) {
        const int32_t* t = token_ids + i * bs;
        hh = m.chain(hh, t);
        m.remember(s.table[i], hh, par, t);
        par = s.table[i];
      }
    }
    return PA_OK;
  }
  // decode (:53-60): the token at position num_tokens-1 is written now
  if (s.table.empty())
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_allocate: decode of sequence %lld without blocks", (long long)seq_id);
  const int64_t idx = ((int64_t)num_tokens - 1) / bs;
  const bool cow = num_tokens > 0 && idx < (int64_t)s.table.size() && m.ref[s.table[idx]] > 1;
  const int32_t want = (cow ? 1 : 0) + (num_tokens % bs == 0 ? 1 : 0);
  if (want > m.nfree)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_allocate: %d blocks needed (copy-on-write %d), %d free", want,
                cow ? 1 : 0, m.nfree);
  if (cow) {
    const int32_t old = s.table[idx];
    const int32_t b = m.pop_front();
    ++m.ref[b];
    --m.ref[old];
    s.table[idx] = b;
    m.copy_src.push_back(old);
    m.copy_dst.push_back(b);
  }
  if (num_tokens % bs == 0) {
    const int32_t b = m.pop_front();
    ++m.ref[b];
    s.table.push_back(b);
  }
  return PA_OK;
}

extern "C" int32_t pa_bm_num_cached_tokens(pa_block_manager* h, int64_t seq_id) {
  if (!h) return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_num_cached_tokens: null manager");
  std::lock_guard<std::mutex> g(h->m.mu);
  auto it = h->m.seqs.find(seq_id);
  return it == h->m.seqs.end() ? 0 : it->second.cached_tokens;
}

extern "C" int32_t pa_bm_block_table(pa_block_manager* h, int64_t seq_id, int32_t* out, int32_t capacity) {
  if (!h || capacity < 0 || (capacity > 0 && !out))
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_block_table: bad arguments");
  std::lock_guard<std::mutex> g(h->m.mu);
  const std::vector<int32_t>& t = h->m.seqs[seq_id].table;
  const int32_t n = (int32_t)t.size();
  for (int32_t i = 0; i < n && i < capacity; ++i) out[i] = t[i];
  return n;
}

extern "C" int pa_bm_fork(pa_block_manager* h, int64_t parent_id, int64_t child_id) {
  if (!h || parent_id == child_id) return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_fork: bad arguments");
  BlockManager& m = h->m;
  std::lock_guard<std::mutex> g(m.mu);
  auto it = m.seqs.find(parent_id);
  if (it == m.seqs.end() || it->second.table.empty())
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_fork: sequence %lld has no blocks", (long long)parent_id);
  SeqState& c = m.seqs[child_id];
  if (!c.table.empty())
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_fork: sequence %lld already has blocks", (long long)child_id);
  c.table = m.seqs[parent_id].table;
  c.cached_tokens = 0;
  for (int32_t b : c.table) ++m.ref[b];
  return PA_OK;
}

extern "C" int pa_bm_deallocate(pa_block_manager* h, int64_t seq_id) {
  if (!h) return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_deallocate: null manager");
  BlockManager& m = h->m;
  std::lock_guard<std::mutex> g(m.mu);
  SeqState& s = m.seqs[seq_id];
  for (int32_t b : s.table)  // :62-70, in table order
    if (--m.ref[b] == 0) m.push_back(b);
  m.seqs.erase(seq_id);
  return PA_OK;
}

extern "C" int32_t pa_bm_ref_count(pa_block_manager* h, int32_t block_id) {
  if (!h || block_id < 0 || block_id >= h->m.num_blocks)
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_ref_count: bad block id");
  std::lock_guard<std::mutex> g(h->m.mu);
  return h->m.ref[block_id];
}

extern "C" int32_t pa_bm_take_copies(pa_block_manager* h, int32_t* src, int32_t* dst, int32_t capacity) {
  if (!h || capacity < 0 || (capacity > 0 && (!src || !dst)))
    return fail(PA_ERR_INVALID_ARGUMENT, "pa_bm_take_copies: bad arguments");
  BlockManager& m = h->m;
  std::lock_guard<std::mutex> g(m.mu);
  const int32_t n = (int32_t)m.copy_src.size();
  if (n > capacity) return n;  // caller retries with a larger buffer; nothing is taken
  for (int32_t i = 0; i < n; ++i) {
    src[i] = m.copy_src[i];
    dst[i] = m.copy_dst[i];
  }
  m.copy_src.clear();
  m.copy_dst.clear();
  return n;
}
