// Shared by the RoPE / append kernels: 16-byte row accesses and the NeoX
// rotate-half of 8 pairs in fp32 with every product and sum rounded
// separately (reference src/cuda_kernels.cu:19-23), rounded to nearest even
// into the 16-bit storage type.  Files that include this header are compiled
// with -ffp-contract=off.
#pragma once
#include "device_util.hpp"

namespace feattn {

__device__ __forceinline__ u32x4 ldv(const uint16_t* p) { return *reinterpret_cast<const u32x4*>(p); }
// Stores carry the non-temporal hint: the rotated rows and cache slots are
// not read again by this kernel, and the 8192-token paged store streams
// 6.2-6.5 TB/s so against 5.6-5.7 (RoPE and the fused appends unchanged).
// Loads keep the default policy (the hint on them cost 5-20 %).
__device__ __forceinline__ void stv(uint16_t* p, u32x4 v) { __builtin_nontemporal_store(v, reinterpret_cast<u32x4*>(p)); }

// Rotates 8 pairs: x = first-half chunk, y = second-half chunk, cs / sn =
// the matching cos and sin entries.
template <bool BF16>
__device__ __forceinline__ void rotate8(u32x4& x, u32x4& y, const float* cs, const float* sn) {
  const f32x4 c0 = reinterpret_cast<const f32x4*>(cs)[0];
  const f32x4 c1 = reinterpret_cast<const f32x4*>(cs)[1];
  const f32x4 s0 = reinterpret_cast<const f32x4*>(sn)[0];
  const f32x4 s1 = reinterpret_cast<const f32x4*>(sn)[1];
  const float c[8] = {c0[0], c0[1], c0[2], c0[3], c1[0], c1[1], c1[2], c1[3]};
  const float s[8] = {s0[0], s0[1], s0[2], s0[3], s1[0], s1[1], s1[2], s1[3]};
  float na[8], nb[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const int e = 2 * i + h;
      const float a = h ? hi_f32<BF16>(x[i]) : lo_f32<BF16>(x[i]);
      const float b = h ? hi_f32<BF16>(y[i]) : lo_f32<BF16>(y[i]);
      na[e] = __fsub_rn(__fmul_rn(a, c[e]), __fmul_rn(b, s[e]));
      nb[e] = __fadd_rn(__fmul_rn(b, c[e]), __fmul_rn(a, s[e]));
    }
  }
  x = pack8_rne<BF16>(na);
  y = pack8_rne<BF16>(nb);
}

}  // namespace feattn
