// Issue-overlap reference kernel for the benchmark (lib/libfeprobe.so, with
// read_probe.hip); not part of the attention path.  Each wavefront runs a
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
