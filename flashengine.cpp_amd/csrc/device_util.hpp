// Device helpers for gfx950 (CDNA4): element conversions, MFMA wrappers and
// wavefront (64-lane) exchanges.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace feattn {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
typedef int32_t i32x16 __attribute__((ext_vector_type(16)));

// ---- element conversions -------------------------------------------------
// Storage is raw 16-bit; BF16 selects bfloat16 vs IEEE binary16.

template <bool BF16>
__device__ __forceinline__ float to_f32(uint32_t h16) {
  if constexpr (BF16) {
    return __uint_as_float(h16 << 16);
  } else {
    return (float)__builtin_bit_cast(_Float16, (uint16_t)h16);
  }
}

// Low / high half of a packed pair.
template <bool BF16>
__device__ __forceinline__ float lo_f32(uint32_t w) {
  if constexpr (BF16) return __uint_as_float(w << 16);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)(w & 0xffffu));
}
template <bool BF16>
__device__ __forceinline__ float hi_f32(uint32_t w) {
  if constexpr (BF16) return __uint_as_float(w & 0xffff0000u);
  else return (float)__builtin_bit_cast(_Float16, (uint16_t)(w >> 16));
}

// fp32 -> 16-bit, round to nearest even.  The bf16 path is written out in
// integer arithmetic so it is the same function as ATen's CPU conversion
// (NaN -> 0x7fc0); the fp16 path is the hardware RNE conversion of the
// already-rounded fp32 value.  The empty asm pins that value in a register:
// otherwise the backend may fold a preceding multiply into the conversion
// (v_fma_mixlo_f16), which rounds the exact product straight to fp16 and
// differs from rounding to fp32 first whenever the fp32 product is a tie.
template <bool BF16>
__device__ __forceinline__ uint32_t from_f32_rne(float f) {
  if constexpr (BF16) {
    uint32_t u = __float_as_uint(f);
    if ((u & 0x7fffffffu) > 0x7f800000u) return 0x7fc0u;
    u += 0x7fffu + ((u >> 16) & 1u);
    return u >> 16;
  } else {
    asm("" : "+v"(f));
    return (uint32_t)__builtin_bit_cast(uint16_t, (_Float16)f);
  }
}

// Eight fp32 values -> four packed 16-bit pairs (out[i] = v[2i] | v[2i+1] <<
// 16), bit-identical to from_f32_rne on every element.  bf16: the hardware
// converter (v_cvt_pk_bf16_f32, round to nearest even, one instruction per
// pair) gives the same bits for every non-NaN input; it would keep NaN
// payload bits, so a lane holding a NaN redoes its packing with
// from_f32_rne (0x7fc0).  fp16: from_f32_rne per element.
template <bool BF16>
__device__ __forceinline__ u32x4 pack8_rne(const float (&v)[8]) {
  u32x4 out;
  if constexpr (BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    bool nan = false;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float a = v[2 * i], b = v[2 * i + 1];
      asm("" : "+v"(a));  // the rounded fp32 values, not a folded product
      asm("" : "+v"(b));
      nan = nan || __builtin_isnan(a) || __builtin_isnan(b);
      out[i] = __builtin_bit_cast(uint32_t, __builtin_convertvector((f32x2){a, b}, bf16x2));
    }
    if (nan) {
#pragma unroll
      for (int i = 0; i < 4; ++i) out[i] = from_f32_rne<true>(v[2 * i]) | (from_f32_rne<true>(v[2 * i + 1]) << 16);
    }
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) out[i] = from_f32_rne<false>(v[2 * i]) | (from_f32_rne<false>(v[2 * i + 1]) << 16);
  }
  return out;
}

// Two fp32 -> packed 16-bit pair using the hardware converter (RNE); used for
// softmax probabilities and attention outputs, where the tolerance, not bit
// identity, is the contract.
template <bool BF16>
__device__ __forceinline__ uint32_t pack2(float a, float b) {
  // one v_cvt_pk_{bf16,f16}_f32 (round to nearest even) for both halves
  typedef float f32x2 __attribute__((ext_vector_type(2)));
  const f32x2 v = {a, b};
  if constexpr (BF16) {
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
  } else {
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, f16x2));
  }
}

// ---- MFMA ----------------------------------------------------------------
// v_mfma_f32_16x16x32_{bf16,f16}.  Operand layout (64 lanes, lane = 16*J + L):
//   A (16 x 32): lane holds row L, 8 reduction elements selected by (J, e)
//   B (32 x 16): lane holds column L, the same 8 reduction elements
//   C (16 x 16): lane holds rows 4*J + r (r = 0..3) of column L
// Which reduction index (J, e) denotes is the same for A and B, so callers
// may assign reduction indices to data freely as long as both operands agree.
template <bool BF16>
__device__ __forceinline__ f32x4 mfma16(u32x4 a, u32x4 b, f32x4 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a),
                                                    __builtin_bit_cast(bf16x8, b), c, 0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a),
                                                   __builtin_bit_cast(f16x8, b), c, 0, 0, 0);
  }
}

// ---- wavefront exchanges -------------------------------------------------
// Value of lane (lane & ~15) + src within each 16-lane row (ds_swizzle,
// bit-mask mode: and 0x10, or src).
template <int SRC>
__device__ __forceinline__ float row_bcast(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x10 | (SRC << 5)));
}

__device__ __forceinline__ float xor16(float v) {
  return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (16 << 10) | 0x1f));
}

__device__ __forceinline__ float xor32(float v) {
  return __shfl_xor(v, 32, 64);
}

// Reductions over lane pairs (i, i ^ 16) and (i, i ^ 32) on the VALU with
// gfx950's v_permlane{16,32}_swap (no LDS round trip).  Swapping a value
// with itself yields {rows 0,0,2,2} and {rows 1,1,3,3} (16-lane rows) for
// permlane16, {lower, lower} and {upper, upper} (32-lane halves) for
// permlane32, so combining the two results gives every lane the reduction
// of its pair, with the same operand order in both lanes of the pair.
__device__ __forceinline__ float max_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_x16(float v) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_x32(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

__device__ __forceinline__ int uniform(int v) { return __builtin_amdgcn_readfirstlane(v); }

constexpr float kNegInf = -__builtin_huge_valf();
constexpr float kLn2 = 0.69314718055994530942f;

}  // namespace feattn
