// Device helpers shared by the attention kernels: plan-metadata reads
// through the scalar cache, HBM -> LDS direct copies, wait counters and LDS
// operand reads (gfx950).
#pragma once
#include <atomic>
#include <type_traits>

#include "attn_types.hpp"
#include "device_util.hpp"

namespace feattn {

constexpr int kLdsBytes = 163840;  // LDS per compute unit (gfx950)

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// Reads of plan metadata (work items, sequence table, page table) through
// the constant address space: these buffers are not written while a kernel
// runs, so wave-uniform indices become scalar loads.
typedef const __attribute__((address_space(4))) int32_t* const_i32p;

__device__ __forceinline__ int32_t ldc(const int32_t* p, int i) { return ((const_i32p)p)[uniform(i)]; }

__device__ __forceinline__ WorkItem ldc_item(const WorkItem* items, int i) {
  const int32_t* p = reinterpret_cast<const int32_t*>(items + uniform(i));
  return WorkItem{ldc(p, 0), ldc(p, 1), ldc(p, 2), ldc(p, 3), ldc(p, 4), ldc(p, 5), ldc(p, 6), ldc(p, 7)};
}

__device__ __forceinline__ SeqInfo ldc_seq(const SeqInfo* seqs, int i) {
  const int32_t* p = reinterpret_cast<const int32_t*>(seqs + uniform(i));
  return SeqInfo{ldc(p, 0), ldc(p, 1), ldc(p, 2), ldc(p, 3)};
}

// STREAM: the non-temporal hint, for data that no other work of the launch
// reads again (K/V rows streamed once).  Such reads then neither displace
// reused lines nor cost cache allocation on their way: the decode kernel
// streams 6.4-6.9 TB/s with it against 5.7-6.1 without.
template <bool STREAM = false>
__device__ __forceinline__ void lds_dma16(const void* gaddr, uint32_t lds_addr) {
  uint32_t saved;
  if constexpr (STREAM) {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %1, off nt\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(gaddr), "s"(__builtin_amdgcn_readfirstlane(lds_addr))  // wave-uniform by construction
        : "memory");
  } else {
    asm volatile(
        "s_mov_b32 %0, m0\n\t"
        "s_mov_b32 m0, %2\n\t"
        "global_load_lds_dwordx4 %1, off\n\t"
        "s_mov_b32 m0, %0"
        : "=&s"(saved)
        : "v"(gaddr), "s"(__builtin_amdgcn_readfirstlane(lds_addr))  // wave-uniform by construction
        : "memory");
  }
}

template <int N>
__device__ __forceinline__ void wait_vmem() {
  asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// Waits until at most `n` units (4 copy instructions each) issued after the
// awaited one are still in flight; n is wave-uniform.  vmcnt holds 6 bits,
// so n is clamped to 15 (a longer wait, never a shorter one).
template <int MAXU>
__device__ __forceinline__ void wait_units(int n) {
  static_for<0, (MAXU < 15 ? MAXU : 15) + 1>([&](auto i) {
    constexpr int I = decltype(i)::value;
    if (I == (MAXU < 15 ? MAXU : 15)) {
      if (n >= I) wait_vmem<4 * I>();
    } else if (n == I) {
      wait_vmem<4 * I>();
    }
  });
}

__device__ __forceinline__ void wait_lds() { asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory"); }

typedef short s16x4 __attribute__((ext_vector_type(4)));

template <bool BF16>
__device__ __forceinline__ f32x4 mfma16k16(u32x2 a, u32x2 b, f32x4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                      0, 0, 0);
  } else {
    typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
    return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                                 0, 0);
  }
}

__device__ __forceinline__ u32x2 lds_read_tr16(uint32_t lds_addr) {
  typedef __attribute__((address_space(3))) s16x4 lds_s16x4;
  const s16x4 v = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)lds_addr);
  return __builtin_bit_cast(u32x2, v);
}

__device__ __forceinline__ u32x4 lds_read16(uint32_t lds_addr) {
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  return *(lds_u32x4*)(uintptr_t)lds_addr;
}

__device__ __forceinline__ void lds_zero16(uint32_t lds_addr) {
  typedef __attribute__((address_space(3))) u32x4 lds_u32x4;
  *(lds_u32x4*)(uintptr_t)lds_addr = u32x4{0u, 0u, 0u, 0u};
}

// Raises a kernel's dynamic LDS limit (the rings exceed the 64 KB default)
// once per device; `done` holds one bit per device id.  Safe to call from
// several host threads.
inline hipError_t allow_lds(const void* fn, size_t bytes, std::atomic<uint64_t>& done) {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return e;
  const uint64_t bit = dev >= 0 && dev < 64 ? uint64_t(1) << dev : 0;
  if (bit != 0 && (done.load(std::memory_order_acquire) & bit) != 0) return hipSuccess;
  e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, (int)bytes);
  if (e == hipSuccess && bit != 0) done.fetch_or(bit, std::memory_order_acq_rel);
  return e;
}

}  // namespace feattn
