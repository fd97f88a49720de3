// Wide-item attention kernel for gfx950: chunked prefill and other query
// blocks wider than 128 (query row, head) columns.
//
// Semantics as in attn_kernels.hip (reference include/fe/native_cuda.hpp:10;
// ATen statement src/portable_gpu_ops.cpp:39-44): fp32 softmax and
// accumulation, scores pre-multiplied by log2(e)/sqrt(128) and exponentiated
// with exp2, log-sum-exp kept in log2 units and converted on output.
//
// One workgroup per compute unit, eight wavefronts (two per SIMD).  A work
// item is (sequence, kv head, up to 256 (query row, head) columns, token
// range); wavefront w owns columns 32w .. 32w+31.  The workgroup walks the
// items of its share (longest first, from the planner) as one stream of
// 64-token tiles: K and V rows of a tile (one kv head, 256 bytes a row) are
// copied HBM -> LDS with direct-to-LDS loads into a four-stage ring, each
// wavefront copying 8 of the 64 rows, two tiles ahead of use; one barrier per
// tile publishes a landed tile and frees the stage read two tiles before.
//
// Per 32-token block, with v_mfma_f32_32x32x16 (lane l: n = l % 32, h = l / 32):
//   S^T = K Q^T: A = K rows (lane: token n, dims 16s+8h..+7, ds_read_b128),
//                B = Q^T in registers (lane: column n, the same dims),
//                8 k-steps; D: lane holds tokens 8(i/4)+4h+(i%4) of column n.
//   O^T += V^T P^T: k-step ks covers tokens 16ks..16ks+15; element e of the
//                operands is token 16ks+8(e/4)+4h+(e%4), which is the lane's
//                own S^T value i = 8ks+e, and the V^T operand reads the same
//                tokens with two ds_read_b64_tr_b16; D: lane holds dims
//                32db+8(i/4)+4h+(i%4) of column n.
// A column's scores sit in one lane pair (l, l^32), so the row maximum and sum
// take one permlane32 exchange.  The next block's S^T MFMAs are issued before
// the current block's softmax, so the MFMA pipe has independent work while
// the exponentials run.
#include "attn_types.hpp"
#include "device_util.hpp"
#include "kernel_util.hpp"

namespace feattn {

constexpr int kWideWaves = kWideCols / 32;          // 8
constexpr int kWideStages = 4;
constexpr int kWideHalf = kTileTokens * 256;        // K (or V) rows of one tile: 16 KB
constexpr int kWideStage = 2 * kWideHalf;           // K rows, then V rows
constexpr int kWideLds = kWideStages * kWideStage;  // 128 KB
static_assert(kWideLds <= kLdsBytes, "wide ring exceeds LDS");
static_assert(kTileTokens == 64, "a tile is two 32-token blocks");

typedef float f32x16 __attribute__((ext_vector_type(16)));

// max(a, b, c) in one v_max3_f32 (fmaxf chains make the compiler quiet each
// operand first, one extra instruction per MFMA result).
__device__ __forceinline__ float max3f(float a, float b, float c) {
  float r;
  asm("v_max3_f32 %0, %1, %2, %3" : "=v"(r) : "v"(a), "v"(b), "v"(c));
  return r;
}

template <bool BF16>
__device__ __forceinline__ f32x16 mfma32(u32x4 a, u32x4 b, f32x16 c) {
  if constexpr (BF16) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                    0, 0, 0);
  } else {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c, 0,
                                                   0, 0);
  }
}

// Position in a workgroup's stream: item `it` (record w, sequence s) at
// token `tok` (a tile start for the copy cursor, a block start otherwise).
struct WideCursor {
  int it;
  WorkItem w;
  SeqInfo s;
  int tok;
};

__device__ __forceinline__ bool wide_item(const AttnArgs& a, WideCursor& c, int it, int end) {
  c.it = it;
  if (it >= end) return false;
  c.w = ldc_item(a.items, it);
  c.s = ldc_seq(a.seqs, c.w.seq);
  c.tok = c.w.t0;
  return true;
}

// Next 64-token tile of the stream.
__device__ __forceinline__ bool wide_next_tile(const AttnArgs& a, WideCursor& c, int end) {
  c.tok += kTileTokens;
  if (c.tok < c.w.t1) return true;
  return wide_item(a, c, c.it + 1, end);
}

// HBM -> LDS direct copy of 16 bytes per lane from a scalar base plus a
// per-lane 32-bit offset (the LDS destination, lane i at base + 16 i, comes
// from M0).
__device__ __forceinline__ void lds_dma16_sb(const void* sbase, uint32_t voff, uint32_t lds_addr) {
  asm volatile("s_mov_b32 m0, %2\n\tglobal_load_lds_dwordx4 %0, %1"
               :
               : "v"(voff), "s"(sbase), "s"(__builtin_amdgcn_readfirstlane(lds_addr))
               : "memory", "m0");
}

// Group-0 wavefront w's share of one tile copy: the 16-token page holding
// K and V rows 16w .. 16w+15 of the tile (one kv head, 256 bytes a row),
// eight 1 KB direct-to-LDS loads issued one at a time between MFMAs (a burst
// of all of a tile's loads stalls the issuing wavefronts).  Load r of K / V
// moves rows 4r .. 4r+3 of the page (lane i: row 4r + i/16, 16-byte slot
// i%16).  Chunk c of tile row t sits at slot c ^ (t % 16) (K) or c ^ 4(t % 4)
// (V), which keeps the operand reads free of bank conflicts; the lane offsets
// lo_k / lo_v (row and chunk of load r) are loop invariants.  Rows at or past
// the item end read the item's last token instead (a live slot; its scores
// are masked and its probabilities are zero), so stale cache slots are never
// read and every tile costs the same eight loads.
struct WideCopy {
  const char* kbase;  // page base of K / V (kv head offset included)
  const char* vbase;
  uint32_t roff;      // byte offset of the first row in the page
  uint32_t dst;       // LDS address of tile row 16w of the stage
  int tok0, t1;       // first token of the share, item end
  bool clamp;         // the share reaches the item end
};

__device__ __forceinline__ WideCopy wide_copy_plan(const AttnArgs& a, const WideCursor& c, int pg,
                                                   uint32_t stage_addr, int wave) {
  const int row_bytes = a.hkv * kHeadDim * 2;
  const int pshift = a.page_shift;
  WideCopy p;
  p.tok0 = c.tok + 16 * wave;
  p.t1 = c.w.t1;
  p.clamp = p.tok0 + 15 >= p.t1;
  const size_t page_base = ((size_t)pg << pshift) * row_bytes + (size_t)c.w.kvh * kHeadDim * 2;
  p.kbase = reinterpret_cast<const char*>(a.kc) + page_base;
  p.vbase = reinterpret_cast<const char*>(a.vc) + page_base;
  p.roff = (uint32_t)((p.tok0 & ((1 << pshift) - 1)) * row_bytes);
  p.dst = stage_addr + (uint32_t)(16 * wave) * 256;
  return p;
}

// Load i of a tile copy: i = 0..3 K rows 4i.., i = 4..7 V rows 4(i-4)..
__device__ __forceinline__ void wide_copy_piece(const AttnArgs& a, const WideCopy& p, int i, int lane,
                                                const uint32_t (&lo)[8]) {
  const int r = i & 3;
  uint32_t off = p.roff + lo[i];
  if (p.clamp) {
    // rows clamped to the item's last token (same page as tok0 when tok0 <
    // t1, else the page of t1 - 1, which `pg` then is)
    const int row_bytes = a.hkv * kHeadDim * 2;
    const int pmask = (1 << a.page_shift) - 1;
    const int j = 4 * r + (lane >> 4);
    const int tok = min(p.tok0 + j, p.t1 - 1);
    off += (uint32_t)(((tok & pmask) - ((p.tok0 & pmask) + j)) * row_bytes);
  }
  lds_dma16_sb(i < 4 ? p.kbase : p.vbase, off, p.dst + 1024 * r + (i < 4 ? 0u : (uint32_t)kWideHalf));
}

// Page id of group-0 wavefront `wave`'s page of the copy cursor's tile.
__device__ __forceinline__ int wide_copy_page(const AttnArgs& a, const WideCursor& c, int wave) {
  const int ptok = min(c.tok + 16 * wave, c.w.t1 - 1);
  return ldc(a.pages, c.s.page_off + (ptok >> a.page_shift));
}

// Workgroup barrier without the memory fence of __syncthreads (whose release
// would wait for every copy in flight); the callers wait for their own copies
// first.  The memory clobber keeps LDS reads below it; the sched_barrier
// fences keep the scheduler from moving MFMA / VALU work across it, which
// would blur the phases the barriers separate.
__device__ __forceinline__ void wide_barrier() {
  __builtin_amdgcn_sched_barrier(0);
  asm volatile("s_barrier" ::: "memory");
  __builtin_amdgcn_sched_barrier(0);
}

// Cursor over the tiles of a workgroup's stream with the item they belong to:
// tile jt of item `it` (nt tiles).
struct WideTile {
  int it;
  WorkItem w;
  SeqInfo s;
  int jt;
  int nt;
};

__device__ __forceinline__ bool wide_tile_item(const AttnArgs& a, WideTile& t, int it, int end) {
  t.it = it;
  if (it >= end) return false;
  t.w = ldc_item(a.items, it);
  t.s = ldc_seq(a.seqs, t.w.seq);
  t.jt = 0;
  t.nt = (t.w.t1 - t.w.t0 + kTileTokens - 1) / kTileTokens;
  return true;
}

template <bool BF16, bool CAUSAL>
__global__ __launch_bounds__(64 * kWideWaves, 1) __attribute__((amdgpu_waves_per_eu(2, 2))) void attn_wide_kernel(
    AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dsm[];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  // Waves 0-3 and 4-7 each hold one wavefront per SIMD; group 1 runs one
  // phase behind group 0, so each SIMD pairs an MFMA phase of one group with
  // a softmax (VALU) phase of the other.
  const int grp = wave >> 2;
  const int n = lane & 31;
  const int h = lane >> 5;
  const int G = a.group;
  const uint32_t lbase = (uint32_t)(uintptr_t)dsm;
  const int n_items = uniform(*a.n_items);
  const int it0 = ldc(a.tile_off, blockIdx.x);
  const int end = min(ldc(a.tile_off, blockIdx.x + 1), n_items);
  if (it0 >= end) return;

  // LDS operand offsets inside a 32-token block of a stage.
  uint32_t koff[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) koff[st] = (uint32_t)(n * 256 + 16 * ((2 * st + h) ^ (n & 15)));
  uint32_t voff[4];
  {
    // ds_read_b64_tr_b16 source lane (g = lane/16, 4k + m = lane%16): token
    // 4(g/2) + k of the 8-row group, dims 16(g%2) + 4m .. +3 of dim block db
    // (chunk 4db + 2(g%2) + m/2 at slot chunk ^ 4k, half m%2).
    const int g = lane >> 4, k = (lane >> 2) & 3, m = lane & 3;
    const int vl = (4 * (g >> 1) + k) * 256 + 32 * (g & 1) + 8 * m;
#pragma unroll
    for (int db = 0; db < 4; ++db) voff[db] = (uint32_t)(vl + 64 * (db ^ k));
  }

  // Copy cursor: every wavefront issues its share of stream tile T at the
  // start of phase slot 2T-4 (an even slot) into stage T % 4 and waits for it
  // at the end of slot 2T-1, before the barrier that opens the first phase
  // reading it.
  // Copies (group 0 only): wavefront w copies one page of stream tile T in
  // its MFMA phase of slot 2T-4 (pieces among the MFMAs) into stage T % 4 and
  // waits for it at the end of slot 2T-1 (its softmax phase), before the
  // barrier that opens the first phase reading it.
  uint32_t copy_lo[8];
  {
    const int row_bytes = a.hkv * kHeadDim * 2;
    const int cJ = lane >> 4, cL = lane & 15;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const int j = 4 * r + cJ;  // row of the page = tile row mod 16
      copy_lo[r] = (uint32_t)(j * row_bytes + 16 * (cL ^ j));
      copy_lo[4 + r] = (uint32_t)(j * row_bytes + 16 * (cL ^ (4 * (j & 3))));
    }
  }
  WideCursor cc;
  wide_item(a, cc, it0, end);
  int cpg = grp == 0 ? wide_copy_page(a, cc, wave) : 0;  // page id of the cursor's tile, read one tile ahead
  int cj = 0;  // tiles issued
  bool c_live = grp == 0;
  auto copy_plan = [&]() {
    return wide_copy_plan(a, cc, cpg, lbase + (uint32_t)((cj & (kWideStages - 1)) * kWideStage), wave);
  };
  auto copy_done = [&]() {
    ++cj;
    c_live = wide_next_tile(a, cc, end);
    if (c_live) cpg = wide_copy_page(a, cc, wave);
  };
  // VMEM operations issued after the newest tile's copies: 0, 8 (a Q load)
  // or -1 (stores: unknown count)
  int after = 0;
  auto wait_tile = [&](int T) {
    if (cj <= T) return;  // past the stream end (or group 1: no copies)
    const int n = cj > T + 1 ? 8 : 0;  // tile T+1's copies may stay in flight
    if (after < 0 || n == 0) wait_vmem<0>();
    else if (after == 0) wait_vmem<8>();
    else wait_vmem<16>();
  };

  // Q rows of an item, B operands of the eight k-steps.  They are loaded with
  // asm loads that the compiler does not track, so it inserts no wait of its
  // own for them (such a wait would also cover the tile copies in flight);
  // the kernel waits for them explicitly and q_ready() marks the point.
  u32x4 qf[8] = {};
  auto load_q = [&](const WorkItem& w) {
    const int ncols = w.nq * G;
    const int col = min(32 * wave + n, ncols - 1);
    const int row = w.q0 + col / G;
    const int head = w.kvh * G + col % G;
    const uint16_t* qp = a.q + ((size_t)row * a.hq + head) * kHeadDim + 8 * h;
#pragma unroll
    for (int st = 0; st < 8; ++st)
      asm volatile("global_load_dwordx4 %0, %1, off" : "+v"(qf[st]) : "v"(qp + 16 * st) : "memory");
  };
  auto q_ready = [&]() {
#pragma unroll
    for (int st = 0; st < 8; ++st) asm volatile("" : "+v"(qf[st]));
  };

  // softmax / output state of the item of the tile being softmaxed
  WideTile nx;  // the tile whose S^T the next MFMA phase computes
  wide_tile_item(a, nx, it0, end);
  WorkItem w = nx.w;
  SeqInfo sq = nx.s;
  int ncols = 0, col = 0, crow = 0, chead = 0, lim = 0, lim_min = 0;
  float m = kNegInf, lsum = 0.f;
  f32x16 o[4];
  auto start_item = [&]() {
    ncols = w.nq * G;
    col = 32 * wave + n;
    const int ce = min(col, ncols - 1);
    crow = w.q0 + ce / G;
    chead = w.kvh * G + ce % G;
    lim = min(CAUSAL ? sq.len - sq.qlen + (crow - sq.qo) : sq.len - 1, w.t1 - 1);
    // the wavefront's smallest limit is its first column's (rows grow with columns)
    const int c0 = min(32 * wave, ncols - 1);
    lim_min = uniform(min(CAUSAL ? sq.len - sq.qlen + (w.q0 + c0 / G - sq.qo) : sq.len - 1, w.t1 - 1));
    m = kNegInf;
    lsum = 0.f;
  };

  // prologue: tiles 0 and 1 and the first item's Q land before the first
  // barrier; group 1 then runs one phase behind
  if (grp == 0) {
#pragma unroll 1
    for (int t = 0; t < 2 && c_live; ++t) {
      const WideCopy cp = copy_plan();
#pragma unroll
      for (int i = 0; i < 8; ++i) wide_copy_piece(a, cp, i, lane, copy_lo);
      copy_done();
    }
  }
  load_q(w);
  wait_vmem<0>();
  q_ready();
  wide_barrier();
  start_item();
#pragma unroll
  for (int db = 0; db < 4; ++db) o[db] = f32x16{};
  int slot = grp;
  if (grp) wide_barrier();

  f32x16 s0 = {}, s1 = {};  // S^T of tile j+1 (tokens 0-31, 32-63)
  u32x4 pf[4] = {};         // P^T of tile j, one u32x4 per 16-token k-step
  bool q_pending = false;
  int q_tail = 0;        // VMEM loads issued after the pending Q loads
  bool cu_last = false;  // tile j is its item's last
  bool nx_live = true;   // tile j+1 exists
  for (int j = -1;; ++j) {
    // ==== MFMA phase: S^T of tile j+1, O^T += V^T P^T of tile j =============
    {
      // the SIMD's oldest-first arbitration would otherwise let the partner
      // wave's softmax VALU delay these MFMAs
      asm volatile("s_setprio 2" ::: "memory");
      // group 0 copies tile j+3 in pieces among this phase's MFMAs
      const bool cp_on = c_live;
      WideCopy cp{};
      if (cp_on) cp = copy_plan();
      after = 0;
      if (q_pending) {
        // the next item's Q loads, then q_tail (0 or 4) copy pieces of group 0
        if (q_tail == 4) wait_vmem<4>();
        else wait_vmem<0>();
        q_ready();
        q_pending = false;
      }
      // (past the stream end the S^T MFMAs read a stage of the ring and the
      // result is dropped)
      const uint32_t kb = lbase + (uint32_t)(((j + 1) & (kWideStages - 1)) * kWideStage);
      const uint32_t vb = lbase + (uint32_t)((j & (kWideStages - 1)) * kWideStage) + kWideHalf;
      // per-lane operand addresses of this phase; the block / k-step offsets
      // are immediates of the reads
      uint32_t ka[8], va[4];
#pragma unroll
      for (int st = 0; st < 8; ++st) ka[st] = kb + koff[st];
#pragma unroll
      for (int db = 0; db < 4; ++db) va[db] = vb + voff[db];
      s0 = f32x16{};
      s1 = f32x16{};
      // K fragments four k-steps ahead of their MFMAs
      constexpr int kAhead = 4;
      u32x4 k0[8], k1[8];
#pragma unroll
      for (int st = 0; st < kAhead; ++st) {
        k0[st] = lds_read16(ka[st]);
        k1[st] = lds_read16(ka[st] + 32 * 256);
      }
#pragma unroll
      for (int st = 0; st < 8; ++st) {
        if (st + kAhead < 8) {
          k0[st + kAhead] = lds_read16(ka[st + kAhead]);
          k1[st + kAhead] = lds_read16(ka[st + kAhead] + 32 * 256);
        }
        s0 = mfma32<BF16>(k0[st], qf[st], s0);
        s1 = mfma32<BF16>(k1[st], qf[st], s1);
        if (cp_on && (st & 1)) wide_copy_piece(a, cp, st >> 1, lane, copy_lo);
        __builtin_amdgcn_sched_barrier(0);
      }
      // the next phase's S^T is of the following item: load its Q now that
      // this phase's S^T MFMAs have read the current one
      if (nx_live && nx.jt + 1 == nx.nt && nx.it + 1 < end) {
        load_q(ldc_item(a.items, nx.it + 1));
        q_pending = true;
        q_tail = cp_on ? 4 : 0;  // copy pieces 4-7 follow
        after = 8;
      }
      if (j >= 0) {
        // V^T fragments four MFMAs ahead of their use; MFMA i is k-step i/4
        // (16 tokens) and dim block i%4
        u32x4 vf[16];
        auto read_v = [&](int i) {
          const int ks = i >> 2, db = i & 3;
          const u32x2 lo = lds_read_tr16(va[db] + ks * 4096);
          const u32x2 hi = lds_read_tr16(va[db] + ks * 4096 + 2048);
          vf[i] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        };
#pragma unroll
        for (int i = 0; i < 4; ++i) read_v(i);
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if (i + 4 < 16) read_v(i + 4);
          o[i & 3] = mfma32<BF16>(vf[i], pf[i >> 2], o[i & 3]);
          if (cp_on && (i & 3) == 3) wide_copy_piece(a, cp, 4 + (i >> 2), lane, copy_lo);
          __builtin_amdgcn_sched_barrier(0);
        }
      } else if (cp_on) {
#pragma unroll
        for (int i = 4; i < 8; ++i) wide_copy_piece(a, cp, i, lane, copy_lo);
      }
      if (cp_on) copy_done();
      // The item of tile j ends with this phase's O^T update: write its rows
      // and switch the softmax state to tile j+1's item.
      if (j >= 0 && cu_last) {
        const float ls = sum_x32(lsum);
        if (col < ncols) {
          const float inv = ls > 0.f ? 1.f / ls : 0.f;
          const float l2 = ls > 0.f ? m + __log2f(ls) : kNegInf;
          uint16_t* dst;
          if (w.part < 0) {
            dst = a.out + ((size_t)crow * a.hq + chead) * kHeadDim + 4 * h;
            if (a.lse != nullptr && h == 0) a.lse[(size_t)crow * a.hq + chead] = l2 * kLn2;
          } else {
            const size_t pslot = (size_t)(w.part + col / G);
            dst = a.part_o + (pslot * a.hq + chead) * kHeadDim + 4 * h;
            if (h == 0) a.part_lse[pslot * a.hq + chead] = l2;
          }
#pragma unroll
          for (int db = 0; db < 4; ++db)
#pragma unroll
            for (int qq = 0; qq < 4; ++qq) {
              const u32x2 v = {pack2<BF16>(o[db][4 * qq] * inv, o[db][4 * qq + 1] * inv),
                               pack2<BF16>(o[db][4 * qq + 2] * inv, o[db][4 * qq + 3] * inv)};
              *reinterpret_cast<u32x2*>(dst + 32 * db + 8 * qq) = v;
            }
        }
        after = -1;
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] = f32x16{};
        if (nx_live) {
          w = nx.w;
          sq = nx.s;
          start_item();
        }
      }
      asm volatile("s_setprio 0" ::: "memory");
      wide_barrier();
      ++slot;
    }

    // ==== softmax phase: softmax of tile j+1 =================================
    {
      bool up = false;
      float alpha = 1.f;
      if (nx_live) {
        const int T = nx.w.t0 + kTileTokens * nx.jt;
        if (T + 63 > lim_min) {
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int t = T + 8 * (i >> 2) + 4 * h + (i & 3);
            if (t > lim) s0[i] = kNegInf;
            if (t + 32 > lim) s1[i] = kNegInf;
          }
        }
        // row maximum with v_max3 (fmaxf would first quiet every MFMA result)
        float mx0 = max3f(s0[0], s0[1], s0[2]), mx1 = max3f(s1[0], s1[1], s1[2]);
#pragma unroll
        for (int i = 3; i < 15; i += 2) {
          mx0 = max3f(mx0, s0[i], s0[i + 1]);
          mx1 = max3f(mx1, s1[i], s1[i + 1]);
        }
        float mx = max3f(mx0, mx1, max3f(s0[15], s1[15], kNegInf));
        mx = max_x32(mx);
        const float mt = mx * a.scale_log2;
        up = mt > m + 8.f;
        alpha = fast_exp2(up ? m - mt : 0.f);
        m = up ? mt : m;
        const float m_use = m == kNegInf ? 0.f : m;
        float ps = 0.f;
#pragma unroll
        for (int ks = 0; ks < 2; ++ks)
#pragma unroll
          for (int jj = 0; jj < 4; ++jj) {
            const int i = 8 * ks + 2 * jj;
            const float a0 = fast_exp2(__builtin_fmaf(s0[i], a.scale_log2, -m_use));
            const float a1 = fast_exp2(__builtin_fmaf(s0[i + 1], a.scale_log2, -m_use));
            const float b0 = fast_exp2(__builtin_fmaf(s1[i], a.scale_log2, -m_use));
            const float b1 = fast_exp2(__builtin_fmaf(s1[i + 1], a.scale_log2, -m_use));
            ps += (a0 + a1) + (b0 + b1);
            pf[ks][jj] = pack2<BF16>(a0, a1);
            pf[2 + ks][jj] = pack2<BF16>(b0, b1);
          }
        lsum = lsum * alpha + ps;
      }
      if (__builtin_amdgcn_ballot_w64(up) != 0) {
#pragma unroll
        for (int db = 0; db < 4; ++db) o[db] *= alpha;
      }
      if (slot & 1) wait_tile((slot + 1) >> 1);
      wide_barrier();
      ++slot;
    }
    if (!nx_live) break;
    cu_last = nx.jt + 1 == nx.nt;
    if (!cu_last) ++nx.jt;
    else nx_live = wide_tile_item(a, nx, nx.it + 1, end);
  }
  // group 0's barrier for the slot group 1 still runs
  if (grp == 0) wide_barrier();
}

template <bool BF16, bool CAUSAL>
static hipError_t wide_launch(const AttnArgs& a, int grid, hipStream_t st) {
  static std::atomic<uint64_t> lds_ok{0};
  const hipError_t e = allow_lds((const void*)attn_wide_kernel<BF16, CAUSAL>, kWideLds, lds_ok);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_wide_kernel<BF16, CAUSAL>), dim3(grid), dim3(64 * kWideWaves), kWideLds, st, a);
  return hipGetLastError();
}

hipError_t launch_wide(const AttnArgs& a, bool bf16, bool causal, int grid, hipStream_t st) {
  if (bf16) return causal ? wide_launch<true, true>(a, grid, st) : wide_launch<true, false>(a, grid, st);
  return causal ? wide_launch<false, true>(a, grid, st) : wide_launch<false, false>(a, grid, st);
}

}  // namespace feattn
