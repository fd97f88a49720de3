// ORACLE (test infrastructure only): extern "C" entry points over the
// reference's own fe::cuda ATen implementation (src/portable_gpu_ops.cpp,
// compiled unmodified from the reference tree by oracle/Makefile), so the GPU
// tests can run the reference's attention, rope and store on identical
// inputs.  The reference code runs its ATen ops on at::kCUDA, which on a
// ROCm LibTorch is the HIP device; the calling process must have loaded
// torch first.
#include <exception>
#include <string>

#include "fe/native_cuda.hpp"

namespace {
thread_local std::string g_err;
template <typename F>
int guard(F&& f) {
  try {
    f();
    return 0;
  } catch (const std::exception& e) {
    g_err = e.what();
    return -1;
  }
}
}  // namespace

extern "C" {
const char* ref_last_error() { return g_err.c_str(); }

void* ref_create_plan(int hq, int hkv, int dim, int page, int max_batch, int max_pages, int bf16, int blocks) {
  void* out = nullptr;
  guard([&] { out = fe::cuda::create_plan(hq, hkv, dim, page, max_batch, max_pages, bf16 != 0, blocks); });
  return out;
}

int ref_destroy_plan(void* plan) {
  return guard([&] { fe::cuda::destroy_plan(static_cast<fe::cuda::AttentionPlan*>(plan)); });
}

int ref_prepare_plan(void* plan, const int32_t* qo, const int32_t* kv, const int32_t* pages, const int32_t* last,
                     int batch, int rows, int graph, void* stream) {
  return guard([&] {
    fe::cuda::prepare_plan(static_cast<fe::cuda::AttentionPlan*>(plan), qo, kv, pages, last, batch, rows, graph != 0,
                           stream);
  });
}

int ref_attention(void* plan, void* q, void* k, void* v, void* out, int causal, void* stream) {
  return guard([&] {
    fe::cuda::attention(static_cast<fe::cuda::AttentionPlan*>(plan), q, k, v, out, causal != 0, stream);
  });
}

int ref_rope(void* q, void* k, const int64_t* pos, const float* cache, int rows, int hq, int hkv, int dim, int bf16,
             void* stream, int max_positions) {
  return guard([&] { fe::cuda::rope(q, k, pos, cache, rows, hq, hkv, dim, bf16 != 0, stream, max_positions); });
}

int ref_store(const void* k, const void* v, void* kc, void* vc, const int64_t* slots, int rows, int width, int bf16,
              void* stream, int cache_slots) {
  return guard([&] { fe::cuda::store(k, v, kc, vc, slots, rows, width, bf16 != 0, stream, cache_slots); });
}
}
