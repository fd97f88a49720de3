/*
 * fe_driver.h - host side of the MI355X attention path: what FlashEngine.cpp's
 * model runner does around the fe_attn.h calls each step.
 *
 *   fe_graph_buckets     batch sizes that get a captured HIP graph
 *                        (reference src/common.cpp:45-51)
 *   fe_blocks_*          FIFO KV page allocator, per sequence page tables
 *                        (reference src/scheduler.cpp:5,31-35, BlockManager
 *                        without the prefix cache)
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
 * src/scheduler.cpp:5 constructor, :31 ensure, :35 release; the prefix cache
 * is not part of this path).  Free pages form a FIFO queue that starts as
 * 0, 1, ..., total-1; ensure takes pages from its front, release returns a
 * sequence's pages to its back. */
typedef struct fe_blocks fe_blocks;

/* total in (0, INT32_MAX), block_size > 0. */
int fe_blocks_create(int64_t total, int64_t block_size, fe_blocks** out);
int fe_blocks_destroy(fe_blocks* blocks);
/* Grows sequence `seq`'s table to ceil(target_tokens / block_size) pages.
 * *ok_out = 1 on success (or nothing to do); 0, with nothing allocated, when
 * too few pages are free (reference: ensure returns false). */
int fe_blocks_ensure(fe_blocks* blocks, int64_t seq, int64_t target_tokens, int* ok_out);
/* Returns all pages of `seq` to the free queue (no-op for an unknown seq). */
int fe_blocks_release(fe_blocks* blocks, int64_t seq);
/* Copies up to `cap` page ids of `seq` to `out` (may be NULL) and the table
 * length to *n_out. */
int fe_blocks_table(const fe_blocks* blocks, int64_t seq, int32_t* out, int cap, int* n_out);
/* Pages currently allocated (reference: BlockManager::used). */
int64_t fe_blocks_used(const fe_blocks* blocks);

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
