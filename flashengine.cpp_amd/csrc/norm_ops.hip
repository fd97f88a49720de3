// RMSNorm, the fused q/k RMSNorm + RoPE + paged-KV append, the SiLU-gated
// product and greedy draft acceptance for gfx950.
//
// RMSNorm follows the reference kernel's arithmetic (src/cuda_kernels.cu:11-17)
// so that results are reproducible bit for bit:
//   * thread t of a 256-thread row accumulates v_j^2 for j = t, t+256, ... in
//     order with one FMA per term (nvcc contracts `sum += v*v` by default);
//   * the 256 partial sums are combined by the pairwise tree
//     p[t] += p[t + s] for s = 128, 64, ..., 1 (p[0] is the total);
//   * scale = rsqrt(total / width + eps), here 1 / sqrt evaluated in double
//     precision and rounded once to float (the reference calls the device's
//     approximate rsqrtf);
//   * out_j = T(rn(rn(v_j * scale) * w_j)), new_residual_j = T(v_j).
// A butterfly (v + v[lane ^ s]) over the lanes that hold the tree's partial
// sums leaves the tree's total in every lane (addition commutes and each step
// pairs exactly the tree's operands), which is how the kernels below evaluate
// the tree inside a wavefront.
//
// This file is compiled with -ffp-contract=off; every fused multiply-add is
// written out.
#include "rope_math.hpp"

namespace feattn {

__device__ __forceinline__ float rsqrt_rn(float x) { return (float)(1.0 / __dsqrt_rn((double)x)); }

template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, true));
}
constexpr int kDppHalfMirror = 0x141;   // lane i <- lane 7 - i within each 8-lane half row
constexpr int kDppQuadXor2 = 0x4e;      // quad_perm [2, 3, 0, 1]
constexpr int kDppQuadXor1 = 0xb1;      // quad_perm [1, 0, 3, 2]

// ---------------------------------------------------------------------------
// fe_norm: one 256-thread block per row, any width.
// ---------------------------------------------------------------------------
template <bool BF16>
__global__ __launch_bounds__(256) void norm_kernel(const uint16_t* __restrict__ x, const uint16_t* __restrict__ res,
                                                   const uint16_t* __restrict__ w, uint16_t* __restrict__ out,
                                                   uint16_t* __restrict__ new_res, int width, float eps) {
  __shared__ float part[256];
  const int t = threadIdx.x;
  const size_t base = (size_t)blockIdx.x * width;
  float sum = 0.f;
  for (int j = t; j < width; j += 256) {
    float v = to_f32<BF16>(x[base + j]);
    if (res != nullptr) v = __fadd_rn(v, to_f32<BF16>(res[base + j]));
    sum = __builtin_fmaf(v, v, sum);
  }
  part[t] = sum;
  __syncthreads();
  if (t < 128) part[t] = __fadd_rn(part[t], part[t + 128]);
  __syncthreads();
  if (t < 64) {
    float s = __fadd_rn(part[t], part[t + 64]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) s = __fadd_rn(s, __shfl_xor(s, o, 64));
    if (t == 0) part[0] = s;
  }
  __syncthreads();
  const float scale = rsqrt_rn(__fadd_rn(__fdiv_rn(part[0], (float)width), eps));
  for (int j = t; j < width; j += 256) {
    float v = to_f32<BF16>(x[base + j]);
    if (res != nullptr) v = __fadd_rn(v, to_f32<BF16>(res[base + j]));
    if (new_res != nullptr) new_res[base + j] = (uint16_t)from_f32_rne<BF16>(v);
    out[base + j] = (uint16_t)from_f32_rne<BF16>(__fmul_rn(__fmul_rn(v, scale), to_f32<BF16>(w[j])));
  }
}

// ---------------------------------------------------------------------------
// Fused q/k RMSNorm + RoPE + paged-KV append (head dim 128).
// ---------------------------------------------------------------------------
// Eight lanes (one 8-lane half row) own a 128-element head: lane c holds
// chunk ch = c (c < 4) or 11 - c (c >= 4) of each half, i.e. elements
// 8ch .. 8ch+7 and 64+8ch .. 64+8ch+7 -- the RoPE pairs.  With that chunk
// order the tree's partner at distance 32 is the half-row mirror lane and the
// partners at distances 16 and 8 are lane ^ 2 and lane ^ 1, so the whole
// reduction is three DPP exchanges.
template <bool BF16>
__device__ __forceinline__ void normalize_head(u32x4& x, u32x4& y, u32x4 wl, u32x4 wh, float eps) {
  float a[8], b[8], s[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    a[2 * i] = lo_f32<BF16>(x[i]);
    a[2 * i + 1] = hi_f32<BF16>(x[i]);
    b[2 * i] = lo_f32<BF16>(y[i]);
    b[2 * i + 1] = hi_f32<BF16>(y[i]);
  }
  // tree step 64 (steps 128 and above add zeros): position 8ch + e
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = __fadd_rn(__fmul_rn(a[e], a[e]), __fmul_rn(b[e], b[e]));
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = __fadd_rn(s[e], dpp<kDppHalfMirror>(s[e]));   // step 32
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = __fadd_rn(s[e], dpp<kDppQuadXor2>(s[e]));     // step 16
#pragma unroll
  for (int e = 0; e < 8; ++e) s[e] = __fadd_rn(s[e], dpp<kDppQuadXor1>(s[e]));     // step 8
#pragma unroll
  for (int e = 0; e < 4; ++e) s[e] = __fadd_rn(s[e], s[e + 4]);                     // step 4
#pragma unroll
  for (int e = 0; e < 2; ++e) s[e] = __fadd_rn(s[e], s[e + 2]);                     // step 2
  const float total = __fadd_rn(s[0], s[1]);                                         // step 1
  const float scale = rsqrt_rn(__fadd_rn(__fdiv_rn(total, 128.f), eps));
  float na[8], nb[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    na[2 * i] = __fmul_rn(__fmul_rn(a[2 * i], scale), lo_f32<BF16>(wl[i]));
    na[2 * i + 1] = __fmul_rn(__fmul_rn(a[2 * i + 1], scale), hi_f32<BF16>(wl[i]));
    nb[2 * i] = __fmul_rn(__fmul_rn(b[2 * i], scale), lo_f32<BF16>(wh[i]));
    nb[2 * i + 1] = __fmul_rn(__fmul_rn(b[2 * i + 1], scale), hi_f32<BF16>(wh[i]));
  }
  x = pack8_rne<BF16>(na);
  y = pack8_rne<BF16>(nb);
}

// Work unit = (row, head in [0, hq + 2 hkv)): query heads are normalized with
// qw, rotated and written to q_out [rows][hq][128]; key heads are normalized
// with kw, rotated and written to the K cache at the row's slot; value heads
// are copied to the V cache.  Row r of the input holds q | k | v heads at
// qkv + r * row_stride.  Rows whose slot is outside [0, cache_slots) write
// no cache entry; rows whose position is outside [0, max_pos) are normalized
// but not rotated.  I: index type of the flat work range (uint32_t when it
// fits, which keeps the (row, head) split a 32-bit division).
template <bool BF16, typename I>
__global__ __launch_bounds__(256) void norm_rope_append_kernel(
    const uint16_t* __restrict__ qkv, int64_t row_stride, const uint16_t* __restrict__ qw,
    const uint16_t* __restrict__ kw, float eps, uint16_t* __restrict__ q_out, uint16_t* __restrict__ kc,
    uint16_t* __restrict__ vc, const int64_t* __restrict__ pos, const int64_t* __restrict__ slots,
    const float* __restrict__ cache, int rows, int hq, int hkv, int max_pos, int64_t cache_slots) {
  constexpr int D = 128, H = 64;
  const int heads = hq + 2 * hkv;
  const int64_t total = (int64_t)rows * heads * 8;   // a multiple of 8: groups never straddle the end
  const int c = threadIdx.x & 7;
  const int ch = c < 4 ? c : 11 - c;
  for (I idx = (I)blockIdx.x * blockDim.x + threadIdx.x; idx < (I)total; idx += (I)gridDim.x * blockDim.x) {
    const I unit = idx >> 3;
    const int head = (int)(unit % (I)heads);
    const int64_t row = (int64_t)(unit / (I)heads);
    int64_t slot = 0;
    if (head >= hq) {
      slot = slots[row];
      if (slot < 0 || slot >= cache_slots) continue;   // the whole 8-lane group skips together
    }
    const uint16_t* src = qkv + row * row_stride + (int64_t)head * D;
    u32x4 x = ldv(src + 8 * ch);
    u32x4 y = ldv(src + H + 8 * ch);
    if (head >= hq + hkv) {
      uint16_t* vd = vc + (slot * hkv + (head - hq - hkv)) * D;
      stv(vd + 8 * ch, x);
      stv(vd + H + 8 * ch, y);
      continue;
    }
    const uint16_t* w = head < hq ? qw : kw;
    normalize_head<BF16>(x, y, ldv(w + 8 * ch), ldv(w + H + 8 * ch), eps);
    const int64_t p = pos[row];
    if (p >= 0 && p < max_pos) {
      const float* cs = cache + p * D + 8 * ch;
      rotate8<BF16>(x, y, cs, cs + H);
    }
    uint16_t* dst = head < hq ? q_out + (row * hq + head) * D : kc + (slot * hkv + (head - hq)) * D;
    stv(dst + 8 * ch, x);
    stv(dst + H + 8 * ch, y);
  }
}

// ---------------------------------------------------------------------------
// SiLU-gated product (src/cuda_kernels.cu:18): out[r][c] = T(rn(x / (1 +
// exp(-x))) * up) with x = gu[r][c], up = gu[r][width + c].
// ---------------------------------------------------------------------------
template <bool BF16>
__global__ __launch_bounds__(256) void silu_mul_kernel(const uint16_t* __restrict__ gu, uint16_t* __restrict__ out,
                                                       int width, int64_t total) {
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = idx / width;
    const int64_t col = idx - row * width;
    const float xv = to_f32<BF16>(gu[row * 2 * width + col]);
    const float up = to_f32<BF16>(gu[row * 2 * width + width + col]);
    const float sig = __fdiv_rn(xv, __fadd_rn(1.f, expf(-xv)));
    out[idx] = (uint16_t)from_f32_rne<BF16>(__fmul_rn(sig, up));
  }
}

// ---------------------------------------------------------------------------
// Greedy acceptance (src/cuda_kernels.cu:25; src/scheduler.cpp:110), one
// thread per sequence: m = length of the longest prefix on which draft and
// verify agree; out[b][0..k] = verify[b][0..k] (equal to the draft on the
// accepted prefix, then the bonus token verify[m]), out[b][k+1] = m + 1.
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void accept_kernel(const int64_t* __restrict__ draft,
                                                     const int64_t* __restrict__ verify, int64_t* __restrict__ out,
                                                     int batch, int k) {
  const int b = blockIdx.x * blockDim.x + threadIdx.x;
  if (b >= batch) return;
  const int64_t* d = draft + (int64_t)b * k;
  const int64_t* v = verify + (int64_t)b * (k + 1);
  int64_t* o = out + (int64_t)b * (k + 2);
  int m = 0;
  while (m < k && d[m] == v[m]) ++m;
  for (int j = 0; j <= k; ++j) o[j] = v[j];
  o[k + 1] = m + 1;
}

static int grid_for(int64_t work) {
  int64_t g = (work + 255) / 256;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

hipError_t launch_norm(const void* x, const void* res, const void* w, void* out, void* new_res, int rows, int width,
                       float eps, bool bf16, hipStream_t st) {
  if (rows == 0) return hipSuccess;
  if (bf16)
    hipLaunchKernelGGL(norm_kernel<true>, dim3(rows), dim3(256), 0, st, (const uint16_t*)x, (const uint16_t*)res,
                       (const uint16_t*)w, (uint16_t*)out, (uint16_t*)new_res, width, eps);
  else
    hipLaunchKernelGGL(norm_kernel<false>, dim3(rows), dim3(256), 0, st, (const uint16_t*)x, (const uint16_t*)res,
                       (const uint16_t*)w, (uint16_t*)out, (uint16_t*)new_res, width, eps);
  return hipGetLastError();
}

hipError_t launch_norm_rope_append(const void* qkv, int64_t row_stride, const void* qw, const void* kw, float eps,
                                   void* q_out, void* kc, void* vc, const int64_t* pos, const int64_t* slots,
                                   const float* cache, int rows, int hq, int hkv, bool bf16, int max_pos,
                                   int64_t cache_slots, hipStream_t st) {
  const int64_t work = (int64_t)rows * (hq + 2 * hkv) * 8;
  if (work == 0) return hipSuccess;
  const int grid = grid_for(work);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, st, (const uint16_t*)qkv, row_stride, (const uint16_t*)qw,
                       (const uint16_t*)kw, eps, (uint16_t*)q_out, (uint16_t*)kc, (uint16_t*)vc, pos, slots, cache,
                       rows, hq, hkv, max_pos, cache_slots);
  };
  const bool narrow = work <= INT32_MAX;  // idx + grid stride stays below 2^32
  if (bf16) narrow ? go(norm_rope_append_kernel<true, uint32_t>) : go(norm_rope_append_kernel<true, int64_t>);
  else narrow ? go(norm_rope_append_kernel<false, uint32_t>) : go(norm_rope_append_kernel<false, int64_t>);
  return hipGetLastError();
}

hipError_t launch_silu_mul(const void* gu, void* out, int rows, int width, bool bf16, hipStream_t st) {
  const int64_t total = (int64_t)rows * width;
  if (total == 0) return hipSuccess;
  if (bf16)
    hipLaunchKernelGGL(silu_mul_kernel<true>, dim3(grid_for(total)), dim3(256), 0, st, (const uint16_t*)gu,
                       (uint16_t*)out, width, total);
  else
    hipLaunchKernelGGL(silu_mul_kernel<false>, dim3(grid_for(total)), dim3(256), 0, st, (const uint16_t*)gu,
                       (uint16_t*)out, width, total);
  return hipGetLastError();
}

hipError_t launch_accept(const int64_t* draft, const int64_t* verify, int64_t* out, int batch, int k,
                         hipStream_t st) {
  if (batch == 0) return hipSuccess;
  hipLaunchKernelGGL(accept_kernel, dim3((batch + 255) / 256), dim3(256), 0, st, draft, verify, out, batch, k);
  return hipGetLastError();
}

}  // namespace feattn
