// fe_native_hip.hpp - the reference's `fe::cuda` attention-path boundary,
// implemented for MI355X on top of the C ABI in fe_attn.h.
//
// Same namespace, names, parameter lists and error behaviour (std::runtime_error)
// as the reference declaration in include/fe/native_cuda.hpp:5-15 (every
// function it declares), so that src/cuda_model.cpp's call sites link against
// libfeattn.so unchanged.  `void* stream` is a hipStream_t.
// The `bool causal` attention call is the reference's; attention_lse adds the
// optional [rows][hq] natural-log log-sum-exp output.
#pragma once
#include <cstddef>
#include <cstdint>

namespace fe::cuda {
struct AttentionPlan;
AttentionPlan* create_plan(int hq, int hkv, int dim, int page, int max_batch, int max_pages, bool bf16, int blocks);
void destroy_plan(AttentionPlan* plan);
void prepare_plan(AttentionPlan* plan, const int32_t* qo, const int32_t* kv, const int32_t* pages,
                  const int32_t* last, int batch, int rows, bool graph, void* stream);
void attention(AttentionPlan* plan, void* q, void* k, void* v, void* output, bool causal, void* stream);
void attention_lse(AttentionPlan* plan, void* q, void* k, void* v, void* output, float* lse, bool causal,
                   void* stream);
void norm(const void* x, const void* residual, const void* weight, void* output, void* new_residual, int rows,
          int width, float eps, bool bf16, void* stream);
void silu_mul(const void* gu, void* output, int rows, int width, bool bf16, void* stream);
void rope(void* q, void* k, const int64_t* pos, const float* cache, int rows, int hq, int hkv, int dim, bool bf16,
          void* stream, int max_positions);
void store(const void* k, const void* v, void* kc, void* vc, const int64_t* slots, int rows, int width, bool bf16,
           void* stream, int cache_slots);
void rope_store(void* q, const void* k, const void* v, void* kc, void* vc, const int64_t* pos, const int64_t* slots,
                const float* cache, int rows, int hq, int hkv, int dim, bool bf16, void* stream, int max_positions,
                int cache_slots);
void accept(const int64_t* draft, const int64_t* verify, int64_t* committed, int batch, int k, void* stream);
// q = norm(q), k = norm(k), rope(q, k), store(k, v) in one pass over a fused
// [rows][q | k | v heads] projection (see fe_norm_rope_append).
void norm_rope_store(const void* qkv, int64_t row_stride, const void* q_weight, const void* k_weight, float eps,
                     void* q_out, void* kc, void* vc, const int64_t* pos, const int64_t* slots, const float* cache,
                     int rows, int hq, int hkv, int dim, bool bf16, void* stream, int max_positions, int cache_slots);
}  // namespace fe::cuda
