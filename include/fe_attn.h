/*
 * fe_attn.h - C ABI of the MI355X (gfx950) paged-KV attention path.
 *
 * This is the drop-in boundary for FlashEngine.cpp's native attention ops.
 * Each entry point replaces one function of the reference's `fe::cuda`
 * boundary (include/fe/native_cuda.hpp:6-14) and keeps its argument meaning:
 * plain device pointers, host metadata arrays, an opaque plan and a `void*`
 * stream that is a `hipStream_t` (NULL = the legacy default stream).
 *
 * Memory contract (reference src/cuda_model.cpp:60,94-96,131-142):
 *   q, out       [rows][hq][dim]                      bf16 or fp16, device
 *   k/v cache    [blocks+1][page][hkv][dim]           bf16 or fp16, device
 *                (page index `blocks` is the padding ("dummy") page)
 *   qo, kv       int32 [batch+1] CSR offsets,        host
 *   pages        int32 [kv[batch]] page ids,          host
 *   last         int32 [batch] tokens in last page,   host, 1..page
 *   pos, slots   int64 [rows],                        device
 *   rope table   fp32 [max_positions][dim] = cos | sin halves, device
 * Sequence b has length len_b = (kv[b+1]-kv[b]-1)*page + last[b] tokens and
 * qlen_b = qo[b+1]-qo[b] query rows; token t lives at cache slot
 * pages[kv[b] + t/page]*page + t%page.  With causal masking, local query row
 * i sees tokens t <= len_b - qlen_b + i (end-aligned: a chunk attends fully to
 * its cached prefix and causally to itself); without it, every t < len_b.
 *
 * Errors: every function returns FE_OK (0) or a negative FE_E* code and
 * leaves a message readable through fe_attn_last_error() on the calling
 * thread.  A plan is not thread-safe; all device work is ordered on the
 * stream passed in.  fe_attn_run, fe_rope, fe_store and fe_rope_append do no
 * allocation, no host synchronisation and launch a grid fixed by the plan's
 * capacity, so they may be captured into a HIP graph; fe_attn_plan_prepare
 * must run outside capture.
 */
#ifndef FE_ATTN_H
#define FE_ATTN_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

enum {
  FE_OK = 0,
  FE_EINVAL = -1,    /* bad argument or metadata (reference: std::runtime_error) */
  FE_ECAPACITY = -2, /* metadata exceeds the capacity fixed at create time */
  FE_EDEVICE = -3,   /* HIP runtime error */
  FE_ENOMEM = -4     /* device, pinned or host allocation failed */
};

typedef struct fe_attn_plan fe_attn_plan;

/* Replaces fe::cuda::create_plan (reference include/fe/native_cuda.hpp:7,
 * src/flashinfer_attention.cu:22-27, src/portable_gpu_ops.cpp:23-25).
 * Allocates capacity-sized metadata, work lists and the split-KV workspace on
 * the current device.  Rejects dim != 128, page not a power of two >= 16,
 * hq not a multiple of hkv. */
int fe_attn_plan_create(int hq, int hkv, int dim, int page, int max_batch,
                        int max_pages, int bf16, int blocks,
                        fe_attn_plan** plan_out);

/* Replaces fe::cuda::destroy_plan (native_cuda.hpp:8). NULL is a no-op. */
int fe_attn_plan_destroy(fe_attn_plan* plan);

/* Replaces fe::cuda::prepare_plan (native_cuda.hpp:9,
 * flashinfer_attention.cu:29-34, portable_gpu_ops.cpp:27-38).  On a stream
 * that is capturing a graph it returns FE_EINVAL and enqueues nothing.
 * Validates the host CSR metadata (batch <= max_batch, kv[batch] <=
 * max_batch*max_pages, qlen <= len <= (max_pages-1)*page, page ids in
 * [0, blocks], last in [1, page]), builds the decode / tile / merge work
 * lists and copies them to the plan's device buffers on `stream` (one small
 * kernel on `stream` reads the plan's pinned staging memory; the call waits
 * for the previous prepare's transfer before reusing that memory).
 * `graph` != 0 pins the launch grids to the plan capacity so that a graph
 * captured once replays correctly after later prepares.  `stream` must be
 * on the device that was current when the plan was created (FE_EDEVICE
 * otherwise), here and in fe_attn_run. */
int fe_attn_plan_prepare(fe_attn_plan* plan, const int32_t* qo,
                         const int32_t* kv, const int32_t* pages,
                         const int32_t* last, int batch, int rows, int graph,
                         void* stream);

/* Replaces fe::cuda::attention (native_cuda.hpp:10,
 * flashinfer_attention.cu:35-44, portable_gpu_ops.cpp:39-44).
 * out[r,h,:] = softmax_t(q[r,h].K[t,h/(hq/hkv)] / sqrt(dim) + mask) . V.
 * `lse` (may be NULL; the reference has no such output) receives
 * [rows][hq] fp32 natural-log log-sum-exp of the scaled logits over the
 * visible keys.  causal = 0 is DFlash's non-causal block attention.
 * q, k_cache, v_cache and out must be 16-byte aligned (FE_EINVAL otherwise),
 * as the contiguous tensors of a caching allocator are. */
int fe_attn_run(fe_attn_plan* plan, const void* q, const void* k_cache,
                const void* v_cache, void* out, float* lse, int causal,
                void* stream);

/* Replaces fe::cuda::rope (native_cuda.hpp:13, cuda_kernels.cu:19-23,33,
 * portable_gpu_ops.cpp:50-53).  In-place NeoX rotate-half on q [rows][hq][dim]
 * and k [rows][hkv][dim] in fp32 without FMA contraction:
 *   x'_j = rn(rn(a*c) - rn(b*s)), x'_{j+d/2} = rn(rn(b*c) + rn(a*s)),
 * c = cache[pos*dim + j], s = cache[pos*dim + d/2 + j], then round-to-nearest-
 * even back to bf16/fp16.  Rows whose pos is outside [0, max_positions) are
 * left unchanged.  q and k must not alias. */
int fe_rope(void* q, void* k, const int64_t* pos, const float* cache, int rows,
            int hq, int hkv, int dim, int bf16, void* stream,
            int max_positions);

/* Replaces fe::cuda::store (native_cuda.hpp:14, cuda_kernels.cu:24,34,
 * portable_gpu_ops.cpp:54).  kc[slot*width + c] = k[row*width + c] and the
 * same for v; rows with slot < 0 (padding) or slot >= cache_slots are
 * skipped. */
int fe_store(const void* k, const void* v, void* k_cache, void* v_cache,
             const int64_t* slots, int rows, int width, int bf16, void* stream,
             int cache_slots);

/* Fused paged-KV append with RoPE: equivalent to fe_rope(q, k, ...) followed
 * by fe_store(k, v, ...) on the cache, in one pass over the new tokens
 * (composition of reference src/cuda_model.cpp:94-95).  q is rotated in
 * place; k and v are read only (the rotated k goes straight to the cache).
 * Rows with slot < 0 still rotate q but write nothing to the cache. */
int fe_rope_append(void* q, const void* k, const void* v, void* k_cache,
                   void* v_cache, const int64_t* pos, const int64_t* slots,
                   const float* cache, int rows, int hq, int hkv, int dim,
                   int bf16, int max_positions, int cache_slots, void* stream);

/* No counterpart in the reference.  For callers that cannot allocate device
 * memory (serving loops and harnesses that forbid hipMalloc):
 * fe_attn_plan_prepare + fe_attn_run in one call, without a plan.  Same arguments and results as a plan of (hq, hkv, dim, page,
 * blocks, bf16) prepared with (qo, kv, pages, last, batch, rows) and run
 * with (q, k_cache, v_cache, out, lse, causal): the same work lists, kernels
 * and bits.  The work lists and split-KV partials live in a 48 MiB device
 * array of the library (one per device, reserved when the library's code
 * object loads on that device, whether or not this entry point is ever
 * called, and kept until the process ends): enough for the full split-KV
 * budget of any plan with up to 128 query heads plus 15.5 MiB of work lists
 * and page table; a call that needs more returns FE_ECAPACITY.  Allocates no device or pinned
 * memory; the metadata goes to the device by one copy from pageable host
 * memory on `stream`, which HIP performs synchronously: the call returns
 * after the stream's earlier work and the copy have run.  For the same
 * reason it cannot be captured into a HIP graph (a replay would copy from
 * host memory the call has released): on a capturing stream it returns
 * FE_EINVAL and enqueues nothing; capture the plan entry points instead.
 * Every call on a device shares that device's array.  Calls ordered on one
 * stream are safe.  Calls that overlap on one device (other streams, other
 * threads) are not: a later call's copy overwrites the page table and work
 * lists that an earlier call's kernels are still reading, so those kernels
 * can read page ids of the other call, i.e. outside their own caches, and
 * fault the device.  Order such calls on one stream or with events. */
int fe_attn_run_noalloc(const void* q, const void* k_cache, const void* v_cache,
                        void* out, float* lse, int causal, const int32_t* qo,
                        const int32_t* kv, const int32_t* pages,
                        const int32_t* last, int batch, int rows, int hq,
                        int hkv, int dim, int page, int blocks, int bf16,
                        void* stream);

/* Message of the last failed call on this thread ("" if none). */
const char* fe_attn_last_error(void);

/* Host-only planner introspection (no device needed): runs the same
 * validation and work-list construction as fe_attn_plan_prepare and reports
 * the counts.  Used by tests and by the benchmark to report the split-KV
 * layout.  counts_out[0..3] = decode items, tile items, merge rows,
 * partial rows. */
int fe_attn_plan_describe(int hq, int hkv, int dim, int page, int max_batch,
                          int max_pages, int blocks, const int32_t* qo,
                          const int32_t* kv, const int32_t* pages,
                          const int32_t* last, int batch, int rows,
                          int32_t* counts_out);

/* Host-only planner dump: writes up to `cap` work items (8 int32 each:
 * kind(0 decode,1 tile), seq, q0, nq, kvh, t0, t1, part) and returns the
 * number written in *n_out.  Lets CPU tests check that every visible
 * (row, head, token) triple is covered exactly once. */
int fe_attn_plan_dump(int hq, int hkv, int dim, int page, int max_batch,
                      int max_pages, int blocks, const int32_t* qo,
                      const int32_t* kv, const int32_t* pages,
                      const int32_t* last, int batch, int rows, int causal,
                      int32_t* items_out, int cap, int* n_out);

/* Host-only: the share assignment fe_attn_plan_prepare gives tile items
 * (one share per tile workgroup), on caller-chosen costs, for tests.  Longest
 * processing time: items in decreasing cost order (equal costs keep their
 * input order) each go to the least-loaded share, the lowest index among
 * equals.  When 0 <= fast < the number of shares in use, the loads of shares
 * [0, fast) count at 2/3 (they stand for the first-dispatched workgroup of
 * each CU's pair, which runs faster), so they receive 3/2 of the work;
 * fe_attn_plan_prepare passes the device's CU count.  fast < 0 (or >= the
 * shares in use) weighs all shares alike.  costs[n] >= 0, total below 2^43,
 * 1 <= slots < 2^20.  Writes order_out[n] (input index of each item, share by
 * share) and off_out[0..*n_shares_out] (CSR offsets of the
 * max(1, min(slots, n)) shares; off_out must hold min(slots, n) + 2
 * entries). */
int fe_attn_assign_shares(const int32_t* costs, int n, int slots, int fast,
                          int32_t* order_out, int32_t* off_out,
                          int* n_shares_out);

/* Library identification, e.g. "feattn-hip-gfx950 <version>". */
const char* fe_attn_version(void);

#ifdef __cplusplus
}
#endif

#endif /* FE_ATTN_H */
