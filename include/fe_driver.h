/*
 * fe_driver.h - host side of the MI355X attention path: what FlashEngine.cpp's
 * model runner does around the fe_attn.h calls each step.
 *
 *   fe_graph_buckets     batch sizes that get a captured HIP graph
 *                        (reference src/common.cpp:45-51)
 *   fe_blocks_*          FIFO KV page allocator, per sequence page tables,
 *                        and its prefix cache of shared read-only pages
 *                        (reference src/scheduler.cpp:5-36, BlockManager)
 *   fe_prepare_metadata  per-step positions / slots and the CSR metadata that
 *                        fe_attn_plan_prepare consumes, graph padding included
 *                        (reference src/cuda_model.cpp:131-142)
 *   fe_rope_table        the [max_len][dim] cos | sin table that fe_rope and
 *                        fe_rope_append read (reference src/cuda_model.cpp:44-47)
 *
 * Everything except fe_rope_table is host-only (no device needed).  Errors
 * follow fe_attn.h: FE_OK or a negative FE_E* code, message in
 * fe_attn_last_error().
 */
#ifndef FE_DRIVER_H
#define FE_DRIVER_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Replaces fe::graph_buckets (reference src/common.cpp:45-51): 1, 2, 4, 8
 * (those <= maximum), then every multiple of 16 up to maximum, then maximum
 * itself if not yet listed.  Writes at most `cap` values to `out` (may be
 * NULL to query) and the full count to *n_out.  maximum must be > 0. */
int fe_graph_buckets(int64_t maximum, int64_t* out, int cap, int* n_out);

/* KV page allocator, the page-table side of fe::BlockManager (reference
 * src/scheduler.cpp:5 constructor, :31 ensure, :36 release, :6 probe, :18
 * publish, :30 snapshot).  Free pages form a FIFO queue that starts as
 * 0, 1, ..., total-1; ensure takes pages from its front, release returns a
 * sequence's pages to its back once no sequence holds them.  With the prefix
 * cache on, a page published under the token prefix it ends stays resident
 * after release until ensure takes it from the queue again (an eviction),
 * and probe hands it, shared and read-only, to every later sequence whose
 * tokens start with that prefix.  Sequences are integer ids.  Not
 * thread-safe. */
typedef struct fe_blocks fe_blocks;

/* total in (0, INT32_MAX), block_size > 0; no prefix cache (reference:
 * BlockManager(total, block_size)). */
int fe_blocks_create(int64_t total, int64_t block_size, fe_blocks** out);
/* Same, with the prefix cache on when caching != 0 (reference:
 * BlockManager(total, block_size, caching), src/scheduler.cpp:5). */
int fe_blocks_create_ex(int64_t total, int64_t block_size, int caching, fe_blocks** out);
int fe_blocks_destroy(fe_blocks* blocks);
/* Grows sequence `seq`'s table to ceil(target_tokens / block_size) pages.
 * *ok_out = 1 on success (or nothing to do); 0, with nothing allocated, when
 * too few pages are free (reference: ensure returns false).  A page taken
 * from the queue that is still resident in the prefix cache is evicted
 * first (the evict hook is told). */
int fe_blocks_ensure(fe_blocks* blocks, int64_t seq, int64_t target_tokens, int* ok_out);
/* Drops `seq`'s hold on its pages; a page no sequence holds any more goes to
 * the back of the free queue (no-op for an unknown seq).  The sequence's
 * probe may run again afterwards (reference: release resets cached and
 * prefix_probed, src/scheduler.cpp:36); its request counters are kept, so a
 * preempted request counts once in the statistics. */
int fe_blocks_release(fe_blocks* blocks, int64_t seq);
/* release, then forget the sequence's request counters: call it when the
 * request finishes (the reference's Sequence object goes away). */
int fe_blocks_forget(fe_blocks* blocks, int64_t seq);
/* Copies up to `cap` page ids of `seq` to `out` (may be NULL) and the table
 * length to *n_out. */
int fe_blocks_table(const fe_blocks* blocks, int64_t seq, int32_t* out, int cap, int* n_out);
/* Pages held by at least one sequence (reference: BlockManager::used). */
int64_t fe_blocks_used(const fe_blocks* blocks);
/* Pages in the free queue, resident cached pages included (reference:
 * BlockManager::free). */
int64_t fe_blocks_free_pages(const fe_blocks* blocks);

/* Prefix-cache hooks (reference: BlockManager::prefix_page_ready and
 * on_evict_page, bound to the model by bind_model, include/fe/model.hpp:22-26).
 * ready(user, key, n, page) returns nonzero when the page cached under the
 * n-token prefix `key` may be reused (probe) or published (publish); evict
 * (user, key, n, page) is told before ensure reuses a resident page.  Either
 * may be NULL (always ready / nothing to tell).  Hooks must not call back
 * into the same allocator. */
typedef int (*fe_prefix_ready_fn)(void* user, const int64_t* key, int64_t n, int32_t page);
typedef void (*fe_prefix_evict_fn)(void* user, const int64_t* key, int64_t n, int32_t page);
int fe_blocks_set_prefix_hooks(fe_blocks* blocks, fe_prefix_ready_fn ready, fe_prefix_evict_fn evict,
                               void* user);

/* Reference BlockManager::probe (src/scheduler.cpp:6-17): before `seq` has
 * pages, give it the resident pages of the longest published prefix of
 * tokens[0 .. n_tokens) that ends at least one token short of n_tokens (the
 * last prompt token is always computed), walking block by block and stopping
 * at the first prefix that is not resident or not ready.  *cached_out = the
 * tokens covered (a multiple of block_size).  No-op (returning the earlier
 * result) after a probe since the last release, and 0 with the prefix cache
 * off.  FE_EINVAL when `seq` already holds pages. */
int fe_blocks_probe(fe_blocks* blocks, int64_t seq, const int64_t* tokens, int64_t n_tokens, int64_t* cached_out);
/* Reference BlockManager::publish (src/scheduler.cpp:18-29): for every full
 * block of tokens[0 .. min(computed, n_tokens)), publish the sequence's page
 * under the prefix it ends, unless the prefix is already resident or the
 * ready hook says no.  FE_EINVAL (pages before it stay published) when the
 * page is not allocated or already published under another prefix.  No-op
 * with the prefix cache off. */
int fe_blocks_publish(fe_blocks* blocks, int64_t seq, const int64_t* tokens, int64_t n_tokens, int64_t computed);

/* Counters of BlockManager::snapshot (src/scheduler.cpp:30). */
typedef struct fe_prefix_stats {
  int64_t requests;        /* prefix_requests: sequences probed, once each */
  int64_t hit_requests;    /* prefix_hit_requests: of those, with a hit */
  int64_t cached_blocks;   /* prefix_cached_blocks: pages handed out by probe */
  int64_t new_blocks;      /* prefix_new_blocks: pages published */
  int64_t resident_blocks; /* prefix_resident_blocks: published, not evicted */
  int64_t evictions;       /* prefix_evictions */
} fe_prefix_stats;
int fe_blocks_prefix_stats(const fe_blocks* blocks, fe_prefix_stats* out);

/* Replaces CudaModel::prepare's metadata loop (reference
 * src/cuda_model.cpp:131-142).  Sequence i < n_seqs contributes rows[i]
 * query rows at positions start[i] .. start[i]+rows[i]-1 over a context of
 * start[i]+rows[i] tokens, with page table tables[table_off[i] ..
 * table_off[i+1]).  Entries n_seqs .. count-1 are graph padding: entry_rows
 * rows at positions 0 .. entry_rows-1, slot -1 (not stored), one page
 * `dummy_page`, last = entry_rows.
 * Outputs (caller-allocated; pass NULL pointers with zero caps to query the
 * sizes): positions / slots int64 [rows], qo / kv int32 [count+1], pages
 * int32 [n_pages], last int32 [count]; slot = table[pos / page] * page +
 * pos % page.  Fails (FE_EINVAL) when a context exceeds max_model_len or a
 * page table does not cover a written slot or the context, as the reference
 * does; FE_ECAPACITY when an output is too small. */
int fe_prepare_metadata(int n_seqs, const int64_t* start, const int32_t* rows, const int32_t* table_off,
                        const int32_t* tables, int count, int entry_rows, int page, int64_t max_model_len,
                        int32_t dummy_page, int64_t* positions, int64_t* slots, int rows_cap, int32_t* qo,
                        int32_t* kv, int32_t* pages, int pages_cap, int32_t* last, int* n_rows_out,
                        int* n_pages_out);

/* Fills the device table [max_len][dim] fp32 with cos | sin halves
 * (reference src/cuda_model.cpp:44-47):
 *   inv[i] = 1 / theta^((2i)/dim) (fp32), f = p * inv[i] (fp32),
 *   table[p][i] = cos(f), table[p][dim/2 + i] = sin(f).
 * Transcendentals are the device library's, so the table is not bit-identical
 * to another device's; dim even, max_len > 0. */
int fe_rope_table(float* table, int max_len, int dim, double theta, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* FE_DRIVER_H */
