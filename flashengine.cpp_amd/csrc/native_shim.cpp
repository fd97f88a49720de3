// fe::cuda:: entry points over the C ABI: status codes become
// std::runtime_error, matching the reference's check() behaviour
// (src/flashinfer_attention.cu:13, src/cuda_kernels.cu:10).
#include <new>
#include <stdexcept>
#include <string>

#include "fe_attn.h"
#include "fe_ops.h"
#include "fe_native_hip.hpp"

namespace fe::cuda {

struct AttentionPlan {
  fe_attn_plan* plan = nullptr;
};

namespace {
void check(int rc) {
  if (rc != FE_OK) throw std::runtime_error(std::string("feattn: ") + fe_attn_last_error());
}
}  // namespace

AttentionPlan* create_plan(int hq, int hkv, int dim, int page, int max_batch, int max_pages, bool bf16, int blocks) {
  fe_attn_plan* p = nullptr;
  check(fe_attn_plan_create(hq, hkv, dim, page, max_batch, max_pages, bf16 ? 1 : 0, blocks, &p));
  auto* handle = new (std::nothrow) AttentionPlan{p};
  if (handle == nullptr) {
    fe_attn_plan_destroy(p);
    throw std::bad_alloc();
  }
  return handle;
}

void destroy_plan(AttentionPlan* plan) {
  if (plan == nullptr) return;
  fe_attn_plan_destroy(plan->plan);
  delete plan;
}

void prepare_plan(AttentionPlan* plan, const int32_t* qo, const int32_t* kv, const int32_t* pages,
                  const int32_t* last, int batch, int rows, bool graph, void* stream) {
  if (plan == nullptr) throw std::runtime_error("feattn: null plan");
  check(fe_attn_plan_prepare(plan->plan, qo, kv, pages, last, batch, rows, graph ? 1 : 0, stream));
}

void attention(AttentionPlan* plan, void* q, void* k, void* v, void* output, bool causal, void* stream) {
  attention_lse(plan, q, k, v, output, nullptr, causal, stream);
}

void attention_lse(AttentionPlan* plan, void* q, void* k, void* v, void* output, float* lse, bool causal,
                   void* stream) {
  if (plan == nullptr) throw std::runtime_error("feattn: null plan");
  check(fe_attn_run(plan->plan, q, k, v, output, lse, causal ? 1 : 0, stream));
}

void norm(const void* x, const void* residual, const void* weight, void* output, void* new_residual, int rows,
          int width, float eps, bool bf16, void* stream) {
  check(fe_norm(x, residual, weight, output, new_residual, rows, width, eps, bf16 ? 1 : 0, stream));
}

void silu_mul(const void* gu, void* output, int rows, int width, bool bf16, void* stream) {
  check(fe_silu_mul(gu, output, rows, width, bf16 ? 1 : 0, stream));
}

void accept(const int64_t* draft, const int64_t* verify, int64_t* committed, int batch, int k, void* stream) {
  check(fe_accept(draft, verify, committed, batch, k, stream));
}

void norm_rope_store(const void* qkv, int64_t row_stride, const void* q_weight, const void* k_weight, float eps,
                     void* q_out, void* kc, void* vc, const int64_t* pos, const int64_t* slots, const float* cache,
                     int rows, int hq, int hkv, int dim, bool bf16, void* stream, int max_positions,
                     int cache_slots) {
  check(fe_norm_rope_append(qkv, row_stride, q_weight, k_weight, eps, q_out, kc, vc, pos, slots, cache, rows, hq, hkv,
                            dim, bf16 ? 1 : 0, max_positions, cache_slots, stream));
}

void rope(void* q, void* k, const int64_t* pos, const float* cache, int rows, int hq, int hkv, int dim, bool bf16,
          void* stream, int max_positions) {
  check(fe_rope(q, k, pos, cache, rows, hq, hkv, dim, bf16 ? 1 : 0, stream, max_positions));
}

void store(const void* k, const void* v, void* kc, void* vc, const int64_t* slots, int rows, int width, bool bf16,
           void* stream, int cache_slots) {
  check(fe_store(k, v, kc, vc, slots, rows, width, bf16 ? 1 : 0, stream, cache_slots));
}

void rope_store(void* q, const void* k, const void* v, void* kc, void* vc, const int64_t* pos, const int64_t* slots,
                const float* cache, int rows, int hq, int hkv, int dim, bool bf16, void* stream, int max_positions,
                int cache_slots) {
  check(fe_rope_append(q, k, v, kc, vc, pos, slots, cache, rows, hq, hkv, dim, bf16 ? 1 : 0, max_positions,
                       cache_slots, stream));
}

}  // namespace fe::cuda
