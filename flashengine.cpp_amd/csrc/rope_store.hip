// RoPE, paged-KV store and the fused RoPE + paged-KV append for gfx950.
//
// Bit-exact with the reference (src/cuda_kernels.cu:19-24; ATen statement
// src/portable_gpu_ops.cpp:50-54): NeoX rotate-half in fp32 with every
// product and sum rounded separately, then round-to-nearest-even to the
// 16-bit storage type.  This file is compiled with -ffp-contract=off and the
// arithmetic is additionally spelled with the _rn intrinsics so that no
// product is fused into an FMA.
//
// Each thread owns 8 consecutive pairs (j, j + dim/2) of one (row, head):
// two 16-byte loads, two 16-byte stores, so a 128-dim head is 8 threads and
// every wavefront touches whole 256-byte head rows.
#include "rope_math.hpp"

namespace feattn {

// In-place rope on q [rows][hq][dim] and k [rows][hkv][dim].  I: index type
// of the flat work range (uint32_t when it fits: 32-bit divisions).
template <bool BF16, typename I>
__global__ __launch_bounds__(256) void rope_kernel(uint16_t* __restrict__ q, uint16_t* __restrict__ k,
                                                   const int64_t* __restrict__ pos,
                                                   const float* __restrict__ cache, int rows, int hq, int hkv,
                                                   int dim, int max_pos) {
  const int cpr = dim >> 4;  // 8-pair chunks per head
  const int64_t total = (int64_t)rows * (hq + hkv) * cpr;
  for (I idx = (I)blockIdx.x * blockDim.x + threadIdx.x; idx < (I)total; idx += (I)gridDim.x * blockDim.x) {
    const int c = (int)(idx % (I)cpr);
    const I rh = idx / (I)cpr;
    const int head = (int)(rh % (I)(hq + hkv));
    const int64_t row = (int64_t)(rh / (I)(hq + hkv));
    const int64_t p = pos[row];
    if (p < 0 || p >= max_pos) continue;
    uint16_t* base = head < hq ? q + (row * hq + head) * dim : k + (row * hkv + (head - hq)) * dim;
    const int half = dim >> 1;
    u32x4 x = ldv(base + 8 * c);
    u32x4 y = ldv(base + half + 8 * c);
    const float* cs = cache + p * dim + 8 * c;
    rotate8<BF16>(x, y, cs, cs + half);
    stv(base + 8 * c, x);
    stv(base + half + 8 * c, y);
  }
}

// kc[slot][:] = k[row][:], vc[slot][:] = v[row][:]; padding rows (slot < 0)
// and out-of-range slots are skipped.  `chunks` = width / 8.  I: index type
// of the flat work range (uint32_t when it fits).
template <typename I>
__global__ __launch_bounds__(256) void store_kernel(const uint16_t* __restrict__ k, const uint16_t* __restrict__ v,
                                                    uint16_t* __restrict__ kc, uint16_t* __restrict__ vc,
                                                    const int64_t* __restrict__ slots, int rows, int chunks,
                                                    int64_t cache_slots) {
  const int64_t total = (int64_t)rows * chunks;
  const int64_t width = (int64_t)chunks * 8;
  for (I idx = (I)blockIdx.x * blockDim.x + threadIdx.x; idx < (I)total; idx += (I)gridDim.x * blockDim.x) {
    const int64_t row = (int64_t)(idx / (I)chunks);
    const int64_t c = (int64_t)idx - row * chunks;
    const int64_t slot = slots[row];
    if (slot < 0 || slot >= cache_slots) continue;
    stv(kc + slot * width + 8 * c, ldv(k + row * width + 8 * c));
    stv(vc + slot * width + 8 * c, ldv(v + row * width + 8 * c));
  }
}

// Element-wise store for widths that are not a multiple of 8.
__global__ __launch_bounds__(256) void store_kernel_scalar(const uint16_t* __restrict__ k,
                                                           const uint16_t* __restrict__ v, uint16_t* __restrict__ kc,
                                                           uint16_t* __restrict__ vc,
                                                           const int64_t* __restrict__ slots, int rows, int width,
                                                           int64_t cache_slots) {
  const int64_t total = (int64_t)rows * width;
  for (int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x; idx < total;
       idx += (int64_t)gridDim.x * blockDim.x) {
    const int64_t row = idx / width;
    const int64_t c = idx - row * width;
    const int64_t slot = slots[row];
    if (slot < 0 || slot >= cache_slots) continue;
    kc[slot * width + c] = k[idx];
    vc[slot * width + c] = v[idx];
  }
}

// Fused rope + append.  Work unit = (row, head in [0, hq + hkv), chunk):
// query heads rotate q in place; kv heads rotate k into the K cache at the
// row's slot and copy both halves of v into the V cache.  I: index type of
// the flat work range (uint32_t when it fits: 32-bit divisions).
template <bool BF16, typename I>
__global__ __launch_bounds__(256) void rope_append_kernel(uint16_t* __restrict__ q, const uint16_t* __restrict__ k,
                                                          const uint16_t* __restrict__ v, uint16_t* __restrict__ kc,
                                                          uint16_t* __restrict__ vc, const int64_t* __restrict__ pos,
                                                          const int64_t* __restrict__ slots,
                                                          const float* __restrict__ cache, int rows, int hq, int hkv,
                                                          int dim, int max_pos, int64_t cache_slots) {
  const int cpr = dim >> 4;
  const int half = dim >> 1;
  const int64_t total = (int64_t)rows * (hq + hkv) * cpr;
  for (I idx = (I)blockIdx.x * blockDim.x + threadIdx.x; idx < (I)total; idx += (I)gridDim.x * blockDim.x) {
    const int c = (int)(idx % (I)cpr);
    const I rh = idx / (I)cpr;
    const int head = (int)(rh % (I)(hq + hkv));
    const int64_t row = (int64_t)(rh / (I)(hq + hkv));
    const int64_t p = pos[row];
    const bool rot = p >= 0 && p < max_pos;
    const float* cs = cache + (rot ? p : 0) * dim + 8 * c;
    if (head < hq) {
      if (!rot) continue;
      uint16_t* base = q + (row * hq + head) * dim;
      u32x4 x = ldv(base + 8 * c);
      u32x4 y = ldv(base + half + 8 * c);
      rotate8<BF16>(x, y, cs, cs + half);
      stv(base + 8 * c, x);
      stv(base + half + 8 * c, y);
    } else {
      const int64_t slot = slots[row];
      if (slot < 0 || slot >= cache_slots) continue;
      const int g = head - hq;
      const uint16_t* kb = k + (row * hkv + g) * dim;
      u32x4 x = ldv(kb + 8 * c);
      u32x4 y = ldv(kb + half + 8 * c);
      if (rot) rotate8<BF16>(x, y, cs, cs + half);
      uint16_t* kd = kc + (slot * hkv + g) * dim;
      stv(kd + 8 * c, x);
      stv(kd + half + 8 * c, y);
      const uint16_t* vb = v + (row * hkv + g) * dim;
      uint16_t* vd = vc + (slot * hkv + g) * dim;
      stv(vd + 8 * c, ldv(vb + 8 * c));
      stv(vd + half + 8 * c, ldv(vb + half + 8 * c));
    }
  }
}

static int grid_for(int64_t work) {
  int64_t g = (work + 255) / 256;
  if (g > 65536) g = 65536;
  if (g < 1) g = 1;
  return (int)g;
}

hipError_t launch_rope(void* q, void* k, const int64_t* pos, const float* cache, int rows, int hq, int hkv, int dim,
                       bool bf16, int max_pos, hipStream_t st) {
  const int64_t work = (int64_t)rows * (hq + hkv) * (dim >> 4);
  if (work == 0) return hipSuccess;
  const int grid = grid_for(work);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, st, (uint16_t*)q, (uint16_t*)k, pos, cache, rows, hq, hkv,
                       dim, max_pos);
  };
  const bool narrow = work <= INT32_MAX;  // idx + grid stride stays below 2^32
  if (bf16) narrow ? go(rope_kernel<true, uint32_t>) : go(rope_kernel<true, int64_t>);
  else narrow ? go(rope_kernel<false, uint32_t>) : go(rope_kernel<false, int64_t>);
  return hipGetLastError();
}

hipError_t launch_store(const void* k, const void* v, void* kc, void* vc, const int64_t* slots, int rows, int width,
                        int64_t cache_slots, hipStream_t st) {
  if (rows == 0 || width == 0) return hipSuccess;
  if (width % 8 == 0) {
    const int chunks = width / 8;
    const int64_t work = (int64_t)rows * chunks;
    if (work <= INT32_MAX)  // idx + grid stride stays below 2^32
      hipLaunchKernelGGL(store_kernel<uint32_t>, dim3(grid_for(work)), dim3(256), 0, st, (const uint16_t*)k,
                         (const uint16_t*)v, (uint16_t*)kc, (uint16_t*)vc, slots, rows, chunks, cache_slots);
    else
      hipLaunchKernelGGL(store_kernel<int64_t>, dim3(grid_for(work)), dim3(256), 0, st, (const uint16_t*)k,
                         (const uint16_t*)v, (uint16_t*)kc, (uint16_t*)vc, slots, rows, chunks, cache_slots);
  } else {
    hipLaunchKernelGGL(store_kernel_scalar, dim3(grid_for((int64_t)rows * width)), dim3(256), 0, st,
                       (const uint16_t*)k, (const uint16_t*)v, (uint16_t*)kc, (uint16_t*)vc, slots, rows, width,
                       cache_slots);
  }
  return hipGetLastError();
}

hipError_t launch_rope_append(void* q, const void* k, const void* v, void* kc, void* vc, const int64_t* pos,
                              const int64_t* slots, const float* cache, int rows, int hq, int hkv, int dim, bool bf16,
                              int max_pos, int64_t cache_slots, hipStream_t st) {
  const int64_t work = (int64_t)rows * (hq + hkv) * (dim >> 4);
  if (work == 0) return hipSuccess;
  const int grid = grid_for(work);
  auto go = [&](auto kernel) {
    hipLaunchKernelGGL(kernel, dim3(grid), dim3(256), 0, st, (uint16_t*)q, (const uint16_t*)k, (const uint16_t*)v,
                       (uint16_t*)kc, (uint16_t*)vc, pos, slots, cache, rows, hq, hkv, dim, max_pos, cache_slots);
  };
  const bool narrow = work <= INT32_MAX;  // idx + grid stride stays below 2^32
  if (bf16) narrow ? go(rope_append_kernel<true, uint32_t>) : go(rope_append_kernel<true, int64_t>);
  else narrow ? go(rope_append_kernel<false, uint32_t>) : go(rope_append_kernel<false, int64_t>);
  return hipGetLastError();
}

// RoPE table (reference src/cuda_model.cpp:44-47), one thread per (position,
// frequency): inv = 1 / theta^((2i)/dim), f = p * inv in fp32 (this file is
// compiled without FMA contraction), cos | sin halves.
__global__ void rope_table_kernel(float* table, int max_len, int dim, float theta) {
  const int half = dim / 2;
  const int64_t idx = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
  if (idx >= (int64_t)max_len * half) return;
  const int p = (int)(idx / half);
  const int i = (int)(idx % half);
  const float inv = 1.0f / powf(theta, (float)(2 * i) / (float)dim);
  const float f = (float)p * inv;
  table[(size_t)p * dim + i] = cosf(f);
  table[(size_t)p * dim + half + i] = sinf(f);
}

hipError_t launch_rope_table(float* table, int max_len, int dim, float theta, hipStream_t st) {
  const int64_t n = (int64_t)max_len * (dim / 2);
  const int grid = (int)((n + 255) / 256);
  hipLaunchKernelGGL(rope_table_kernel, dim3(grid), dim3(256), 0, st, table, max_len, dim, theta);
  return hipGetLastError();
}

}  // namespace feattn
