// Read-throughput reference kernels for the benchmark, built into their own
// library (lib/libfeprobe.so); not part of the attention path.  They stream a
// paged cache laid out like the engine's K / V pools -- 32 KB pages of 16
// token rows, each row 8 kv heads x 128 16-bit values (2 KB) -- in the
// patterns the attention kernels use, with no arithmetic, so that the
// benchmark can report what the memory system delivers for each pattern:
//
//  * fe_probe_rows: work units of (chain of pages, kv head group); a unit
//    reads 256 B (one kv head, as one tile workgroup reads the cache) or
//    2 KB (all eight kv heads, as the wavefronts of one decode workgroup read
//    it together) of every row of its pages, with plain 16-byte loads and
//    32 KB per workgroup in flight.
//  * fe_probe_tile_copy: the tile kernel's copy stream without its compute.
//    Per 64-token tile, wavefront w copies page w's 16 rows of one kv head
//    from the K pool and from the V pool into a two-stage 32 KB LDS ring with
//    direct-to-LDS loads; the next tile's copy is issued after the barrier
//    that ends the wait for the current one.
//
// Page ids come from a table of chains (chain c = pages[c * chain_len ..]);
// every id must be below the pool's page count, which the caller guarantees
// (the benchmark passes a permutation of the pool's pages).
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace {

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

constexpr int kPageBytes = 32768;  // 16 rows x 2 KB
constexpr int kRowChunks = 128;    // 16-byte chunks per 2 KB row

// HPU kv heads (of 8) per unit: 1 or 8.  Thread t reads chunk t % CH of row
// t / CH (+ RPP per pass) of each of the step's K pages; every thread keeps
// 8 loads (32 KB per workgroup) in flight.
template <int HPU>
__global__ __launch_bounds__(256) void probe_rows_kernel(const u32x4* __restrict__ cache,
                                                         const int* __restrict__ pages, int n_chains,
                                                         int chain_len, uint32_t* __restrict__ sink) {
  constexpr int G = 8 / HPU;        // units per chain
  constexpr int CH = 16 * HPU;      // chunks per row read by a unit
  constexpr int RPP = 256 / CH;     // rows per pass of 256 threads
  constexpr int PASSES = 16 / RPP;  // passes per page
  constexpr int K = 8 / HPU;        // pages per step
  const int t = threadIdx.x;
  const int row0 = t / CH, ch = t % CH;
  const int n_units = n_chains * G;
  uint32_t acc = 0;
  for (int u = blockIdx.x; u < n_units; u += gridDim.x) {
    const int chain = u / G, g = u % G;
    const int* pp = pages + (size_t)chain * chain_len;
    for (int p0 = 0; p0 < chain_len; p0 += K) {
      u32x4 v[K][PASSES];
#pragma unroll
      for (int k = 0; k < K; ++k) {
        const size_t page = (size_t)pp[p0 + k];
#pragma unroll
        for (int s = 0; s < PASSES; ++s)
          v[k][s] = cache[(page * 16 + row0 + s * RPP) * kRowChunks + g * CH + ch];
      }
#pragma unroll
      for (int k = 0; k < K; ++k)
#pragma unroll
        for (int s = 0; s < PASSES; ++s) acc ^= v[k][s].x ^ v[k][s].y ^ v[k][s].z ^ v[k][s].w;
    }
  }
  sink[(size_t)blockIdx.x * 256 + t] = acc;
}

// Direct-to-LDS copy of 16 bytes per lane: lane i lands at lds_addr + 16 i.
__device__ __forceinline__ void copy16(const void* gaddr, uint32_t lds_addr) {
  uint32_t saved;
  asm volatile(
      "s_mov_b32 %0, m0\n\t"
      "s_mov_b32 m0, %2\n\t"
      "global_load_lds_dwordx4 %1, off\n\t"
      "s_mov_b32 m0, %0"
      : "=&s"(saved)
      : "v"(gaddr), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
      : "memory");
}

// Tile `tile` of a chain (pages 4 tile .. 4 tile + 3), kv head h: wavefront
// `wave` copies its page's 16 rows x 256 B of K, then of V, into stage `st`
// (K blocks at 4 KB x wave, V blocks at 16 KB + 4 KB x wave).
__device__ __forceinline__ void copy_tile(const char* kc, const char* vc, const int* pp, int tile, int h, int lane,
                                          int wave, uint32_t st) {
  const int pg = __builtin_amdgcn_readfirstlane(pp[tile * 4 + wave]);
  const size_t blk = (size_t)pg * kPageBytes + (size_t)h * 256;
  const int J = lane >> 4, L = lane & 15;
#pragma unroll
  for (int r = 0; r < 4; ++r) copy16(kc + blk + (4 * r + J) * 2048 + 16 * L, st + wave * 4096 + 1024 * r);
#pragma unroll
  for (int r = 0; r < 4; ++r) copy16(vc + blk + (4 * r + J) * 2048 + 16 * L, st + (4 + wave) * 4096 + 1024 * r);
}

__global__ __launch_bounds__(256, 2) void probe_tile_copy_kernel(const char* __restrict__ kc,
                                                                 const char* __restrict__ vc,
                                                                 const int* __restrict__ pages, int n_chains,
                                                                 int chain_len, uint32_t* __restrict__ sink) {
  extern __shared__ __attribute__((aligned(16))) uint32_t ring[];
  const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
  const uint32_t lbase = (uint32_t)(uintptr_t)ring;
  const int n_units = n_chains * 8;
  const int tiles = chain_len / 4;
  uint32_t acc = 0;
  int stage = 0;
  for (int u = blockIdx.x; u < n_units; u += gridDim.x) {
    const int chain = u / 8, h = u % 8;
    const int* pp = pages + (size_t)chain * chain_len;
    copy_tile(kc, vc, pp, 0, h, lane, wave, lbase + stage * 32768u);
    for (int j = 0; j < tiles; ++j) {
      asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // this wavefront's copies of tile j
      __syncthreads();                                   // every wavefront's; stage ^ 1 is free
      if (j + 1 < tiles) copy_tile(kc, vc, pp, j + 1, h, lane, wave, lbase + (stage ^ 1) * 32768u);
      acc ^= ring[stage * 8192 + t * 32];
      stage ^= 1;
    }
  }
  sink[(size_t)blockIdx.x * 256 + t] = acc;
}

}  // namespace

// Returns 0, -1 for bad arguments (nothing launched), or the HIP error of the
// launch.  `sink` holds grid * 256 words.
extern "C" int fe_probe_rows(const void* cache, const int* pages, int n_chains, int chain_len, int heads_per_unit,
                             int grid, uint32_t* sink, void* stream) {
  if (cache == nullptr || pages == nullptr || sink == nullptr || n_chains < 1 || chain_len < 8 ||
      chain_len % 8 != 0 || grid < 1)
    return -1;
  const hipStream_t st = static_cast<hipStream_t>(stream);
  const u32x4* c = static_cast<const u32x4*>(cache);
  if (heads_per_unit == 1)
    hipLaunchKernelGGL(probe_rows_kernel<1>, dim3(grid), dim3(256), 0, st, c, pages, n_chains, chain_len, sink);
  else if (heads_per_unit == 8)
    hipLaunchKernelGGL(probe_rows_kernel<8>, dim3(grid), dim3(256), 0, st, c, pages, n_chains, chain_len, sink);
  else
    return -1;
  return (int)hipGetLastError();
}

extern "C" int fe_probe_tile_copy(const void* k_pool, const void* v_pool, const int* pages, int n_chains,
                                  int chain_len, int grid, uint32_t* sink, void* stream) {
  if (k_pool == nullptr || v_pool == nullptr || pages == nullptr || sink == nullptr || n_chains < 1 ||
      chain_len < 4 || chain_len % 4 != 0 || grid < 1)
    return -1;
  hipLaunchKernelGGL(probe_tile_copy_kernel, dim3(grid), dim3(256), 65536, static_cast<hipStream_t>(stream),
                     static_cast<const char*>(k_pool), static_cast<const char*>(v_pool), pages, n_chains, chain_len,
                     sink);
  return (int)hipGetLastError();
}
