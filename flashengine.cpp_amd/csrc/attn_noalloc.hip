// Attention entry point that allocates nothing: plan metadata and split-KV
// partials live in a fixed device array of this library instead of memory
// that fe_attn_plan_create allocates.  For callers that may not allocate
// device memory (serving loops and harnesses that forbid hipMalloc).  Not
// capturable: each call copies its work lists from host memory it releases.
#include <hip/hip_runtime.h>

#include <atomic>
#include <cstdint>
#include <string>

#include "fe_attn.h"

namespace feattn {
int report_error(int code, const std::string& msg);
int attn_oneshot(uint8_t* arena, size_t bytes, int device, const void* q, const void* k_cache, const void* v_cache,
                 void* out, float* lse, int causal, const int32_t* qo, const int32_t* kv, const int32_t* pages,
                 const int32_t* last, int batch, int rows, int hq, int hkv, int dim, int page, int blocks, int bf16,
                 hipStream_t st);
}  // namespace feattn

namespace {

// 48 MiB.  A plan's split-KV budget is max(1024, 64 MiB / (hq * 516 B))
// partial slots of hq * 260 B each (fe_attn.cpp: partial_cap_for): at most
// 32.25 MiB below 128 query heads and 1024 * hq * 260 B from 128 on, so the
// full budget of any plan with up to 128 query heads (32.5 MiB) fits beside
// 15.5 MiB of work lists and page table.  Each device the library runs on
// holds its own copy from the time the library's code object is loaded
// until the process ends, whether or not this entry point is called.
constexpr size_t kScratchBytes = 48u << 20;
constexpr size_t kFullBudgetHeads = 128;
constexpr size_t kPartialSlotsFloor = 1024;
constexpr size_t kPartialBytesPerHead = 128 * 2 + 4;  // 16-bit partial row + fp32 log2-LSE
static_assert(kScratchBytes >= kPartialSlotsFloor * kFullBudgetHeads * kPartialBytesPerHead + (15u << 20),
              "scratch must hold the split-KV budget of a 128-head plan plus 15 MiB of metadata");
constexpr int kMaxDevices = 64;

// Device address of each device's copy of `scratch`, looked up on the first
// call made with that device current.
std::atomic<uint8_t*> g_scratch[kMaxDevices];

}  // namespace

// In host code `scratch` names a host-side stand-in, not device memory: only
// the address hipGetSymbolAddress returns may reach a kernel or a copy.
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

extern "C" int fe_attn_run_noalloc(const void* q, const void* k_cache, const void* v_cache, void* out, float* lse,
                                   int causal, const int32_t* qo, const int32_t* kv, const int32_t* pages,
                                   const int32_t* last, int batch, int rows, int hq, int hkv, int dim, int page,
                                   int blocks, int bf16, void* stream) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return feattn::report_error(FE_EDEVICE, std::string("hipGetDevice: ") + hipGetErrorString(e));
  if (dev < 0 || dev >= kMaxDevices)
    return feattn::report_error(FE_EDEVICE, "attention (no-alloc): device ordinal beyond " +
                                                std::to_string(kMaxDevices - 1));
  uint8_t* ptr = g_scratch[dev].load(std::memory_order_acquire);
  if (ptr == nullptr) {
    e = hipGetSymbolAddress(reinterpret_cast<void**>(&ptr), HIP_SYMBOL(scratch));
    if (e != hipSuccess || ptr == nullptr)
      return feattn::report_error(FE_EDEVICE,
                                  std::string("hipGetSymbolAddress(scratch): ") + hipGetErrorString(e));
    g_scratch[dev].store(ptr, std::memory_order_release);
  }
  return feattn::attn_oneshot(ptr, kScratchBytes, dev, q, k_cache, v_cache, out, lse, causal, qo, kv, pages, last,
                              batch, rows, hq, hkv, dim, page, blocks, bf16, static_cast<hipStream_t>(stream));
}
