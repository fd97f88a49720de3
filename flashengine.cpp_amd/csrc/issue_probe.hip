// Issue-overlap and LDS-throughput reference kernels for the benchmark
// (lib/libfeprobe.so, with read_probe.hip); not part of the attention path.  Each wavefront runs a
// loop of four independent v_mfma_f32_16x16x32_bf16 accumulator chains with
// K independent VALU instructions (v_fma_f32, or v_exp_f32) after every
// MFMA, the interleave pinned by sched_group_barrier, and records the shader
// clock (s_memtime) around the loop.  With one wavefront per SIMD the cycles
// per (MFMA + K VALU) show whether a wavefront's VALU work overlaps its own
// MFMAs; with two per SIMD, whether it overlaps the other wavefront's.
//
// sink[b * 64] receives workgroup b's loop cycles; the other lanes' slots
// receive values that depend on every accumulator, so nothing is dead.
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

template <int K, bool EXP>
__global__ __launch_bounds__(64) void issue_kernel(float* __restrict__ sink, int iters, float seed) {
  const int lane = threadIdx.x;
  bf16x8 a, b;
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(seed * (lane + i));
    b[i] = (__bf16)(seed * (lane - i));
  }
  f32x4 c0 = {0.f, 0.f, 0.f, 0.f}, c1 = c0, c2 = c0, c3 = c0;
  float x[8];
  for (int i = 0; i < 8; ++i) x[i] = seed * (lane + 3 * i);
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#define FE_PROBE_STEP(C)                                             \
  C = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, C, 0, 0, 0);     \
  _Pragma("unroll") for (int k = 0; k < K; ++k) {                    \
    if (EXP) x[k % 8] = __builtin_amdgcn_exp2f(x[k % 8]);            \
    else x[k % 8] = __builtin_fmaf(x[k % 8], 0.999f, 0.001f);        \
  }
    FE_PROBE_STEP(c0)
    FE_PROBE_STEP(c1)
    FE_PROBE_STEP(c2)
    FE_PROBE_STEP(c3)
#undef FE_PROBE_STEP
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);  // one MFMA
      __builtin_amdgcn_sched_group_barrier(0x002, K, 0);  // then K VALU
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  float s = c0[0] + c1[1] + c2[2] + c3[3];
  for (int i = 0; i < 8; ++i) s += x[i];
  sink[(size_t)blockIdx.x * 64 + lane] = lane == 0 ? (float)(t1 - t0) : s;
}

}  // namespace

// Launches `grid` single-wavefront workgroups (grid = 4 x CUs: one wavefront
// per SIMD; 8 x CUs: two).  K VALU per MFMA: 2, 4, 8 or 16 (v_fma_f32), 2 or 4
// (v_exp_f32).  Returns 0, -1 for an unsupported K (nothing launched), or the
// HIP error of the launch.  `sink` holds grid * 64 floats.
extern "C" int fe_probe_issue(float* sink, int iters, int k, int exp, int grid, void* stream) {
  if (sink == nullptr || iters < 1 || grid < 1) return -1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
#define FE_PROBE_LAUNCH(KK, E) \
  hipLaunchKernelGGL((issue_kernel<KK, E>), dim3(grid), dim3(64), 0, st, sink, iters, 0.001f)
  if (exp) {
    switch (k) {
      case 2: FE_PROBE_LAUNCH(2, true); break;
      case 4: FE_PROBE_LAUNCH(4, true); break;
      default: return -1;
    }
  } else {
    switch (k) {
      case 2: FE_PROBE_LAUNCH(2, false); break;
      case 4: FE_PROBE_LAUNCH(4, false); break;
      case 8: FE_PROBE_LAUNCH(8, false); break;
      case 16: FE_PROBE_LAUNCH(16, false); break;
      default: return -1;
    }
  }
#undef FE_PROBE_LAUNCH
  return (int)hipGetLastError();
}

// LDS read throughput: W wavefronts per workgroup (one workgroup per CU,
// 64 KB of LDS), each looping over groups of 8 independent reads of its own
// 8 KB region -- ds_read_b128 (16 bytes per lane) or ds_read_b64_tr_b16 (8
// bytes per lane, the transposing read of the tile kernel's V operand) --
// then a wait; lane i reads bytes [16 i, 16 i + 16) (or [8 i, 8 i + 8)) of
// each 1 KB block, so no two lanes of a read share a bank.  sink[b * 64 * W]
// receives workgroup b's wavefront-0 loop cycles (s_memtime).
namespace {

typedef uint32_t u32x4p __attribute__((ext_vector_type(4)));
typedef short s16x4p __attribute__((ext_vector_type(4)));

template <bool TR>
__global__ __launch_bounds__(1024) void lds_kernel(float* __restrict__ sink, int iters) {
  extern __shared__ __attribute__((aligned(16))) uint8_t lds[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  // fill this wavefront's 8 KB
  for (int i = lane; i < 2048; i += 64) reinterpret_cast<uint32_t*>(lds + wave * 8192)[i] = (uint32_t)(i * 2654435761u);
  __syncthreads();
  const uint32_t base = (uint32_t)(uintptr_t)lds + (uint32_t)(wave * 8192) + (uint32_t)(lane * (TR ? 8 : 16));
  uint32_t acc = 0;
  const uint64_t t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
    asm volatile("" ::: "memory");  // the reads are issued every iteration
    if constexpr (TR) {
      typedef __attribute__((address_space(3))) s16x4p lds_s16x4;
      s16x4p v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k)
        v[k] = __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_s16x4*)(uintptr_t)(base + 1024 * k));
#pragma unroll
      for (int k = 0; k < 8; ++k) asm volatile("" ::"v"(v[k]));
      acc ^= (uint32_t)(uint16_t)v[0][0];
    } else {
      typedef __attribute__((address_space(3))) u32x4p lds_u32x4;
      u32x4p v[8];
#pragma unroll
      for (int k = 0; k < 8; ++k) v[k] = *(lds_u32x4*)(uintptr_t)(base + 1024 * k);
#pragma unroll
      for (int k = 0; k < 8; ++k) asm volatile("" ::"v"(v[k]));  // used whole, no ALU work
      acc ^= v[0][0];
    }
  }
  const uint64_t t1 = __builtin_amdgcn_s_memtime();
  sink[(size_t)blockIdx.x * blockDim.x + t] = t == 0 ? (float)(t1 - t0) : (float)acc;
}

}  // namespace

// waves in 1..16 (one workgroup of 64 * waves threads per CU, grid = CUs),
// tr: 0 = ds_read_b128, 1 = ds_read_b64_tr_b16.  Returns 0, -1 for bad
// arguments (nothing launched), or the HIP error of the launch.  `sink`
// holds grid * 64 * waves floats.
extern "C" int fe_probe_lds(float* sink, int iters, int waves, int tr, int grid, void* stream) {
  if (sink == nullptr || iters < 1 || waves < 1 || waves > 16 || grid < 1) return -1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const void* fn = tr ? (const void*)lds_kernel<true> : (const void*)lds_kernel<false>;
  hipError_t e = hipFuncSetAttribute(fn, hipFuncAttributeMaxDynamicSharedMemorySize, 131072);
  if (e != hipSuccess) return (int)e;
  const size_t lds = (size_t)waves * 8192;
  if (tr) hipLaunchKernelGGL(lds_kernel<true>, dim3(grid), dim3(64 * waves), lds, st, sink, iters);
  else hipLaunchKernelGGL(lds_kernel<false>, dim3(grid), dim3(64 * waves), lds, st, sink, iters);
  return (int)hipGetLastError();
}
