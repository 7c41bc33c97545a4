/*
 * C ABI of the host-side KV block manager and the device page copy that
 * serves its copy-on-write (part of libpaged_attention.so).
 *
 * The manager hands out pool blocks to sequences the way the reference's
 * KVCacheManager does (vllm/src/kv_cache_manager.py:14-70): a FIFO queue of
 * free blocks, one block table per sequence, reference counts.  With prefix
 * caching off and no forks, every call sequence yields the reference's block
 * ids, order and counts.  Two additions (no reference counterpart):
 *   - prefix caching: leading full blocks of a prompt whose tokens (and
 *     predecessor block) match a cached block are shared, not reallocated;
 *     only blocks before the prompt's last token are taken from the cache;
 *   - fork + copy-on-write: a forked sequence shares its parent's blocks;
 *     a decode write into a shared block moves the writer to a fresh block
 *     and queues a (src, dst) page copy, executed with pa_copy_blocks.
 * Host functions are thread-safe per manager; return codes follow
 * paged_attention.h (negative = error, pa_last_error() has the message).
 */
#ifndef VLLM_JAX_AMD_BLOCK_MANAGER_H_
#define VLLM_JAX_AMD_BLOCK_MANAGER_H_

#include <stddef.h>
#include <stdint.h>

#include "paged_attention.h"

#ifdef __cplusplus
extern "C" {
#endif

typedef struct pa_block_manager pa_block_manager;

/* KVCacheManager.__init__ (kv_cache_manager.py:16-22): blocks 0..num_blocks-1
 * free, queued in id order.  NULL on bad sizes. */
pa_block_manager* pa_bm_create(int32_t num_blocks, int32_t block_size, int32_t enable_prefix_caching);
void pa_bm_destroy(pa_block_manager* bm);

/* len(free_block_queue). */
int32_t pa_bm_num_free_blocks(pa_block_manager* bm);

/* can_allocate (kv_cache_manager.py:29-41): 1 = yes, 0 = no.  num_tokens is
 * len(request); token_ids (may be NULL) are the request's tokens, used for
 * prefix-cache lookups. */
int pa_bm_can_allocate(pa_block_manager* bm, int64_t seq_id, const int32_t* token_ids, int32_t num_tokens,
                       int32_t is_prefill);

/* allocate_slots (kv_cache_manager.py:43-60).  Prefill: the table grows to
 * ceil(num_tokens / block_size) blocks, cached leading blocks first.
 * Decode: a shared block about to be written is copied (queued), and a block
 * is appended when num_tokens % block_size == 0. */
int pa_bm_allocate(pa_block_manager* bm, int64_t seq_id, const int32_t* token_ids, int32_t num_tokens,
                   int32_t is_prefill);

/* Prompt tokens covered by cached blocks at the sequence's last prefill
 * (a multiple of block_size; 0 without prefix caching). */
int32_t pa_bm_num_cached_tokens(pa_block_manager* bm, int64_t seq_id);

/* get_block_table (kv_cache_manager.py:24-27): copies up to `capacity` block
 * ids to `out` and returns the table length. */
int32_t pa_bm_block_table(pa_block_manager* bm, int64_t seq_id, int32_t* out, int32_t capacity);

/* Share every block of `parent_id` with the empty sequence `child_id`. */
int pa_bm_fork(pa_block_manager* bm, int64_t parent_id, int64_t child_id);

/* deallocate (kv_cache_manager.py:62-70). */
int pa_bm_deallocate(pa_block_manager* bm, int64_t seq_id);

/* Reference count of one block. */
int32_t pa_bm_ref_count(pa_block_manager* bm, int32_t block_id);

/* Queued copy-on-write page copies: returns their count n; if n <= capacity
 * they are written to src/dst (host arrays) and the queue is cleared,
 * otherwise nothing is taken. */
int32_t pa_bm_take_copies(pa_block_manager* bm, int32_t* src, int32_t* dst, int32_t capacity);

/* Device page copy for copy-on-write: page dst_blocks[i] <- page
 * src_blocks[i] in both K and V pools (device int32 arrays, num_copies <=
 * 65535), the pool addressed as in pa_kv_store.  Destinations must be
 * distinct and must not be sources.  Block ids outside [0, num_pages) are
 * skipped. */
int pa_copy_blocks(uint16_t* k_cache, uint16_t* v_cache, int32_t num_pages, int32_t page_size,
                   int64_t page_stride, int64_t slot_stride, int64_t head_stride,
                   int32_t num_kv_heads, int32_t head_dim,
                   const int32_t* src_blocks, const int32_t* dst_blocks, int32_t num_copies, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* VLLM_JAX_AMD_BLOCK_MANAGER_H_ */
