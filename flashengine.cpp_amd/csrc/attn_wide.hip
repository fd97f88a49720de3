// Wide tile kernel: chunked prefill and other tile work whose items carry
// more than 64 (query row, head) columns, on v_mfma_f32_32x32x16_{bf16,f16}.
//
// Semantics as the other attention kernels (the reference's attention
// boundary, include/fe/native_cuda.hpp:10; ATen statement
// src/portable_gpu_ops.cpp:39-44): per (query row, head) column, an fp32
// softmax over its visible tokens of q.k / sqrt(128), in the exp2 domain,
// accumulated in fp32.
//
// Workgroup: eight wavefronts, one workgroup per CU (two wavefronts per
// SIMD); wavefront w owns columns 32 w .. 32 w + 31 of an item of up to 256
// (query row, head) columns.  K and V stream through LDS in 64-token stages
// of four 16-token blocks, copied HBM -> LDS by direct-to-LDS loads:
// wavefront w < 4 copies K block w, wavefront w >= 4 V block w - 4.  Four K
// slots (LDS bytes 0 .. 65535) and four V slots (65536 .. 131071) let the
// copies run three stages ahead of the compute.
//
// Per wavefront an item is a software pipeline over 32-token sub-tiles.
// Iteration s issues the MFMAs of S(s + 1) = K(s + 1) Q^T (eight k-steps of
// 16 dims into one 32x32 accumulator) and of O^T += V^T(s - 1) P^T(s - 1)
// (four 32-dim blocks x two 16-token k-steps) in alternation, with the
// softmax of S(s) -- row maximum, exponentials, row sum, packing of P(s) --
// placed between them, so that the two wavefronts sharing a SIMD always have
// MFMA and VALU work to overlap.  Operands are read from LDS two MFMA slots
// ahead.
//
// Lane layout (lane = 32 h + n): the S^T accumulator holds tokens
// 8 j + 4 h + i (register 4 j + i) of column n; the P^T operand of k-step kk
// is the lane's own values j = 2 kk, 2 kk + 1 packed to 16 bits, and the V^T
// operand reads the same token order with two ds_read_b64_tr_b16.  The O^T
// accumulator of dim block db holds dims 32 db + 8 j + 4 h + i of column n.
//
// Synchronisation: one barrier per 64-token stage.  Barrier g sits before
// the first S MFMAs of stage g (stages numbered across the workgroup's
// items): each wavefront first waits for the copy set it issued three
// barriers earlier (K(g) for the K copiers, V(g - 1) for the V copiers),
// zeroes V rows past the item end, and after the barrier -- which also
// guarantees that K(g - 1) and V(g - 2) are no longer read -- requests
// K(g + 3) or V(g + 2) into those slots.  The copy side walks the
// workgroup's stage stream across item boundaries.
#include <atomic>
#include <type_traits>

#include "attn_types.hpp"
#include "device_util.hpp"
#include "kernel_util.hpp"

namespace feattn {

typedef float f32x16 __attribute__((ext_vector_type(16)));

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

constexpr int kWideStage = 64;     // tokens per stage: four 16-token blocks
constexpr int kWideWavesMax = 8;
constexpr int kWideKSlot = 16384;  // bytes of one K (or V) slot
constexpr int kWideSlots = 4;      // K slots, and V slots
constexpr int kWideVBase = kWideSlots * kWideKSlot;
constexpr int kWidePages = 2 * kWideSlots * kWideKSlot;  // per wavefront: a ring of 4 page ids
constexpr int kWideLds = kWidePages + kWideWavesMax * 16;
constexpr int kWideCols = 32;      // columns per wavefront
constexpr int kWideWaves = 8;
static_assert(kWideWaves * kWideCols == kWideItemCols, "eight wavefronts of 32 columns");

// The workgroup's stage stream (items of its share, 64-token stages each),
// walked by the copy side.  All fields are wavefront-uniform.
struct WideStream {
  int it;        // item index of the current stage
  int end;       // end of the share
  int t1;        // end token of the item
  int kvh;       // kv head of the item
  int page_off;  // first page id of the item's sequence
  int tok;       // first token of the current stage
  int live;      // 0 once past the last stage
};

// The stream at the first stage of item `it` (< end) of the share.
__device__ __forceinline__ WideStream stream_at(const AttnArgs& a, int it, int end) {
  const int32_t* p = reinterpret_cast<const int32_t*>(a.items + uniform(it));
  WideStream c;
  c.it = it;
  c.end = end;
  c.kvh = ldc(p, 3);
  c.tok = ldc(p, 4);
  c.t1 = ldc(p, 5);
  c.page_off = ldc(reinterpret_cast<const int32_t*>(a.seqs + uniform(ldc(p, 0))), 3);
  c.live = 1;
  return c;
}

// The stream one stage on.  Written in value form (a new cursor, every
// field assigned on each path) so the cursor stays in scalar registers.
__device__ __forceinline__ WideStream stream_next(const AttnArgs& a, WideStream c) {
  if (!c.live) return c;
  if (c.tok + kWideStage < c.t1) {
    c.tok += kWideStage;
    return c;
  }
  if (c.it + 1 < c.end) return stream_at(a, c.it + 1, c.end);
  c.live = 0;
  return c;
}

// A 16-token block (tokens tok + 16 blk ..) of K or V is copied into its
// LDS block by four direct-to-LDS copies: lane (J, L) of copy r fetches row
// 4 r + J, chunk L ^ t (K) or L ^ (2 t mod 16) (V), so LDS chunk position c
// holds that swizzled chunk; `goff` is the lane's offset of copy 0.
// Rows of block `blk` of the stream's current stage inside its item (<= 0:
// none, 16 when the stream has ended).
__device__ __forceinline__ int stream_rows(const WideStream& c, int blk) {
  return c.live ? c.t1 - (c.tok + 16 * blk) : 16;
}

// The page id of block `blk` of the stream's current stage is fetched into
// LDS word `lds` (one lane, direct-to-LDS) when the block is inside its item.
// Returns the instructions issued (0 or 1).
__device__ __forceinline__ int stream_page_fetch(const AttnArgs& a, const WideStream& c, int blk, uint32_t lds,
                                                 int lane) {
  if (!c.live) return 0;
  const int tok = c.tok + 16 * blk;
  if (tok >= c.t1) return 0;
  if (lane == 0) lds_dma4(a.pages + c.page_off + (tok >> a.page_shift), lds);
  return 1;
}

// Source of block `blk` of the stream's current stage (page id `pg`).
__device__ __forceinline__ const char* stream_src(const AttnArgs& a, const WideStream& c, const uint16_t* cache,
                                                  int blk, int pg) {
  const int tok = c.tok + 16 * blk;
  const int pshift = a.page_shift;
  const size_t off = (((size_t)pg << pshift) + (size_t)(tok & ((1 << pshift) - 1))) * (size_t)(a.hkv * kHeadDim * 2) +
                     (size_t)c.kvh * kHeadDim * 2;
  return reinterpret_cast<const char*>(cache) + off;
}

// Copies R0 .. R1 - 1 of a block (four rows each) from `src` to `lds`.
template <bool V, int R0, int R1>
__device__ __forceinline__ void block_copy(const char* src, int goff, int row4, uint32_t lds) {
#pragma unroll
  for (int r = R0; r < R1; ++r) {
    const int x = V ? ((r & 1) ? 128 : 0) : 64 * r;
    lds_dma16(src + r * row4 + (goff ^ x), lds + 1024 * r);
  }
}

template <bool BF16, bool CAUSAL>
__global__ __launch_bounds__(64 * kWideWaves, 1) void attn_wide_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dsm[];
  const int lane = threadIdx.x & 63;
  const int wave = uniform(threadIdx.x >> 6);
  const int n_items = uniform(*a.n_items);
  const int row_bytes = a.hkv * kHeadDim * 2;
  const uint32_t lbase = (uint32_t)(uintptr_t)dsm;
  const int n = lane & 31, h = lane >> 5;
  const bool vcopier = wave >= 4;  // copies V blocks (else K blocks)
  const int cblk = wave & 3;       // the 16-token block of each stage it copies

  // Per-lane LDS and global offsets.  The chunk swizzles only touch address
  // bits 4-7 of 256-byte rows (lbase is 256-byte aligned: the dynamic LDS
  // allocation starts there), so the operand addresses of every k-step /
  // dim block, and the copy offsets of every copy, are one base XORed with
  // a constant:
  //   K operand of k-step ks (sub-tile half 0 of K slot 0):  kofs ^ (32 ks)
  //   V^T operand of dim block db (first read, V slot 0):   vofs ^ (64 db)
  //   K copy r (row 4 r + J):  r * 4 rows + (goff ^ (64 r))
  //   V copy r:                r * 4 rows + (goff ^ (128 (r & 1)))
  // Slot s adds 16384 s, sub-tile half 8192, V k-step 4096, the second V^T
  // read 2048.
  uint32_t kofs, vofs;
  int goff;
  {
    const int t16 = n & 15;
    kofs = lbase + (uint32_t)((n >> 4) * 4096 + t16 * 256 + 16 * ((h ^ t16) & 15));
    const int gg = (lane >> 4) & 1, L = lane & 15;
    const int tv = 4 * h + (L >> 2);
    const int c0 = 2 * gg + ((L & 3) >> 1);
    vofs = lbase + (uint32_t)(kWideVBase + tv * 256 + 16 * ((c0 ^ (2 * tv)) & 15) + 8 * (L & 1));
    const int J = lane >> 4;
    goff = vcopier ? J * row_bytes + 16 * (L ^ ((2 * J) & 15)) : J * row_bytes + 16 * (L ^ J);
  }
  const int row4 = 4 * row_bytes;

  int it = ldc(a.tile_off, blockIdx.x);
  const int end = min(ldc(a.tile_off, blockIdx.x + 1), n_items);
  if (it >= end) return;

  // ---- copy side ---------------------------------------------------------
  // One cursor per wavefront over the stage stream: K copiers run three
  // stages ahead of the barriers, V copiers two.  A second cursor runs three
  // stages ahead of the first and fetches the page ids (into a ring of four
  // LDS words per wavefront), so a copy never waits on a page-table load.
  // A copy set is the stage's four copies and the page id three stages on;
  // the last three sets are remembered (instructions issued; for V the rows
  // inside the item and the LDS block) so that a barrier waits for exactly
  // the set three barriers back, which also holds the page id the next set
  // needs.
  WideStream cs = stream_at(a, it, end);
  WideStream ps = cs;
  const uint32_t ring = lbase + (uint32_t)(kWidePages + 16 * wave);
  int cslot = 0;                     // slot of the cursor's stage
  int nset = 0;                      // sets issued (ring position)
  int cnt1 = 0, cnt2 = 0;            // instructions of the last two sets (0 .. 5)
  int vr1 = 16, vr2 = 16, vr3 = 16;  // V rows inside the item of the last three sets
  uint32_t vz1 = lbase, vz2 = lbase, vz3 = lbase;
  auto shift = [&](int cnt, int rows, uint32_t dst) {
    vr3 = vr2;
    vz3 = vz2;
    vr2 = vr1;
    vz2 = vz1;
    vr1 = rows;
    vz1 = dst;
    cnt2 = cnt1;
    cnt1 = cnt;
  };
  // page ids of the first three stages
  for (int k = 0; k < 3; ++k) {
    stream_page_fetch(a, ps, cblk, ring + 4 * k, lane);
    ps = stream_next(a, ps);
  }
  wait_vmem<0>();
  // The two wavefronts of a SIMD issue their sets at different times, so
  // that one computes while the other queues copies on the CU's memory
  // pipeline: K copiers (the wavefronts that run ahead in the SIMD's issue
  // order) right after the barrier, V copiers one iteration later.  A set is
  // issue_a (page id, addresses, first two copies) then issue_b (last two
  // copies, the page id three stages on, the cursor step).
  const char* csrc = nullptr;  // source of the set being issued
  uint32_t cdst = 0;
  int crows = 16, ccopy = 0;
  auto issue_a = [&]() {
    cdst = lbase + (uint32_t)((vcopier ? kWideVBase : 0) + cslot * kWideKSlot + cblk * 4096);
    crows = stream_rows(cs, cblk);
    ccopy = cs.live && crows > 0;
    if (ccopy) {
      const int pg = uniform((int)lds_read4(ring + 4 * (nset & 3)));
      csrc = stream_src(a, cs, vcopier ? a.vc : a.kc, cblk, pg);
      if (vcopier) block_copy<true, 0, 2>(csrc, goff, row4, cdst);
      else block_copy<false, 0, 2>(csrc, goff, row4, cdst);
    }
  };
  auto issue_b = [&]() {
    if (ccopy) {
      if (vcopier) block_copy<true, 2, 4>(csrc, goff, row4, cdst);
      else block_copy<false, 2, 4>(csrc, goff, row4, cdst);
    }
    int cnt = ccopy ? 4 : 0;
    // the page id of the stage three sets on goes to the ring word just read
    cnt += stream_page_fetch(a, ps, cblk, ring + 4 * ((nset + 3) & 3), lane);
    ps = stream_next(a, ps);
    if (cs.live) cslot = (cslot + 1) & (kWideSlots - 1);
    cs = stream_next(a, cs);
    ++nset;
    shift(cnt, vcopier ? crows : 16, cdst);
  };
  auto issue = [&]() {
    issue_a();
    issue_b();
  };
  // the sets of barriers -3, -2, -1: K(0), K(1), K(2) / none, V(0), V(1)
  if (vcopier) {
    shift(0, 16, lbase);
    // the V cursor's first page id sits at ring word 0: start the ring there
  } else {
    issue();
  }
  issue();
  issue();

  // Barrier of one stage: the set issued three barriers back has landed (V
  // rows past their item zeroed: 0 * stale must stay 0); every wavefront is
  // past its reads of the slots about to be refilled; then the K copiers'
  // next set (the caller issues the V copiers' one, issue_mid).
  auto stage_barrier = [&]() {
    const int younger = cnt1 + cnt2;
    switch (younger) {
      case 0: wait_vmem<0>(); break;
      case 1: wait_vmem<1>(); break;
      case 2: wait_vmem<2>(); break;
      case 3: wait_vmem<3>(); break;
      case 4: wait_vmem<4>(); break;
      case 5: wait_vmem<5>(); break;
      case 6: wait_vmem<6>(); break;
      case 7: wait_vmem<7>(); break;
      case 8: wait_vmem<8>(); break;
      case 9: wait_vmem<9>(); break;
      default: wait_vmem<10>(); break;
    }
    if (vr3 < 16) {
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int q = lane + 64 * u;
        if ((q >> 4) >= vr3) lds_zero16(vz3 + 16 * q);
      }
    }
    __syncthreads();
    if (!vcopier) {
      issue_a();
      issue_b();
    }
  };
  // the V copiers' set, one iteration after the barrier
  auto issue_mid = [&]() {
    if (vcopier) {
      issue_a();
      issue_b();
    }
  };

  // ---- compute side ------------------------------------------------------
  u32x4 qf[8];
  f32x16 o[4];
  f32x16 sc;
  u32x4 pp[2];
  float m = kNegInf, lsum = 0.f;
  int lim = -1, lim_min = 0;
  uint32_t kb = kofs, vb = vofs;  // operand bases of the K / V slots in use

  // S^T of the sub-tile in half HALF of the K slot at kb.
  auto s_tile = [&](auto half_) -> f32x16 {
    constexpr int HALF = decltype(half_)::value;
    f32x16 acc{};
#pragma unroll
    for (int ks = 0; ks < 8; ++ks) acc = mfma32<BF16>(lds_read16((kb ^ (32 * ks)) + HALF * 8192), qf[ks], acc);
    return acc;
  };

  // Softmax step of one sub-tile (first token T): P in the two k-step
  // operands, returns whether any lane raised its reference maximum (then O
  // must be scaled by `alpha` once the PV MFMAs in flight are done).
  auto softmax = [&](auto mask_, const f32x16& s_in, int T, u32x4(&p)[2], float& alpha) -> bool {
    constexpr bool MASK = decltype(mask_)::value;
    f32x16 sv = s_in;
    if constexpr (MASK) {
      // token of register 4 j + i is T + 8 j + 4 h + i
      const int d = lim - (T + 4 * h);
#pragma unroll
      for (int r = 0; r < 16; ++r)
        if (8 * (r >> 2) + (r & 3) > d) sv[r] = kNegInf;
    }
    float mx = __builtin_fmaxf(__builtin_fmaxf(sv[0], sv[1]), sv[2]);
#pragma unroll
    for (int i = 3; i < 15; i += 2) mx = __builtin_fmaxf(__builtin_fmaxf(mx, sv[i]), sv[i + 1]);
    mx = __builtin_fmaxf(mx, sv[15]);
    mx = max_x32(mx);
    // Lazy reference maximum: raised (with l and O rescaled) only when the
    // sub-tile maximum exceeds it by more than 8, so p <= 2^8.
    const float mt = mx * a.scale_log2;
    const bool up = mt > m + 8.f;
    alpha = up ? fast_exp2(m - mt) : 1.f;
    if (up) m = mt;
    const float mu = m == kNegInf ? 0.f : m;
    float x[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) x[i] = fast_exp2(__builtin_fmaf(sv[i], a.scale_log2, -mu));
    float ps = x[0];
#pragma unroll
    for (int i = 1; i < 16; ++i) ps += x[i];
    lsum = lsum * alpha + ps;
#pragma unroll
    for (int kk = 0; kk < 2; ++kk)
#pragma unroll
      for (int e = 0; e < 4; ++e) p[kk][e] = pack2<BF16>(x[8 * kk + 2 * e], x[8 * kk + 2 * e + 1]);
    return __builtin_amdgcn_ballot_w64(up) != 0;
  };

  // One pipeline iteration of sub-tile s: S(s + 1) from half HALF of the K
  // slot at kb (unless LAST), PV(s - 1) from half HALF of the V slot at vb
  // (unless FIRST), softmax of S(s) (first token T).
  auto iter = [&](auto half_, auto first_, auto last_, auto mask_, int T) {
    constexpr int HALF = decltype(half_)::value;
    constexpr bool HS = !decltype(last_)::value, HP = !decltype(first_)::value;
    f32x16 sn{};
    u32x4 pn[2];
    float alpha;
    // MFMA slots: 2 i = S k-step i, 2 i + 1 = PV block (db = i & 3,
    // kk = i >> 2); operands read two slots ahead
    u32x4 opnd[16];
    auto rd = [&](int j) {
      if (j & 1) {
        if constexpr (HP) {
          const int i = j >> 1;
          const uint32_t va = (vb ^ (64 * (i & 3))) + HALF * 8192 + (i >> 2) * 4096;
          const u32x2 lo = lds_read_tr16(va);
          const u32x2 hi = lds_read_tr16(va + 2048);
          opnd[j] = u32x4{lo[0], lo[1], hi[0], hi[1]};
        }
      } else {
        if constexpr (HS) opnd[j] = lds_read16((kb ^ (32 * (j >> 1))) + HALF * 8192);
      }
    };
    rd(0);
    rd(1);
#pragma unroll
    for (int j = 0; j < 16; ++j) {
      if (j + 2 < 16) rd(j + 2);
      const int i = j >> 1;
      if (j & 1) {
        if constexpr (HP) o[i & 3] = mfma32<BF16>(opnd[j], pp[i >> 2], o[i & 3]);
      } else {
        if constexpr (HS) sn = mfma32<BF16>(opnd[j], qf[i], sn);
      }
    }
    const bool any_up = softmax(mask_, sc, T, pn, alpha);
    // the softmax is complete before the rescale branch, so the scheduler
    // interleaves all of it with the MFMAs above
    asm volatile("" : "+v"(pn[0]), "+v"(pn[1]), "+v"(alpha), "+v"(lsum));
    constexpr int NM = (HS ? 8 : 0) + (HP ? 8 : 0);
    constexpr int NR = (HS ? 8 : 0) + (HP ? 16 : 0);
    if constexpr (NM == 16) {
      __builtin_amdgcn_sched_group_barrier(0x100, 3, 0);
      static_for<0, 16>([&](auto j_) {
        constexpr int j = decltype(j_)::value;
        constexpr int r = (j + 2 < 16) ? (((j + 2) & 1) ? 2 : 1) : 0;
        if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 5, 0);
      });
    } else if constexpr (NM == 8) {
      __builtin_amdgcn_sched_group_barrier(0x100, NR / 4, 0);
      static_for<0, 8>([&](auto j_) {
        constexpr int j = decltype(j_)::value;
        constexpr int r = (j < 6) ? (NR / 8) : 0;
        if constexpr (r > 0) __builtin_amdgcn_sched_group_barrier(0x100, r, 0);
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, 9, 0);
      });
    }
    if (any_up) {
#pragma unroll
      for (int db = 0; db < 4; ++db) o[db] *= alpha;
    }
    pp[0] = pn[0];
    pp[1] = pn[1];
    sc = sn;
    // keep each iteration's reads and softmax inside its own schedule
    __builtin_amdgcn_sched_barrier(0);
  };
  using F = std::false_type;
  using Tr = std::true_type;
  using H0 = std::integral_constant<int, 0>;
  using H1 = std::integral_constant<int, 1>;


  int g0 = 0;  // stage number (mod 4) of the current item's first stage
  bool first = true;
  for (; it < end; ++it) {
    const WorkItem w = ldc_item(a.items, it);
    const SeqInfo s = ldc_seq(a.seqs, w.seq);
    const int G = a.group;
    const int ncols = w.nq * G;
    const bool wave_on = wave * kWideCols < ncols;
    const int t0 = w.t0;
    const int NS = (w.t1 - t0 + 31) >> 5;  // 32-token sub-tiles
    {
      const int col = wave * kWideCols + n;
      const bool ok = col < ncols;
      const int crow = w.q0 + (ok ? col / G : 0);
      const int chead = w.kvh * G + (ok ? col % G : 0);
      lim = -1;
      if (ok) lim = min(CAUSAL ? s.len - s.qlen + (crow - s.qo) : s.len - 1, w.t1 - 1);
      lim_min = ok ? lim : (1 << 30);
#pragma unroll
      for (int o_ = 32; o_ >= 1; o_ >>= 1) lim_min = min(lim_min, __shfl_xor(lim_min, o_, 64));
      lim_min = uniform(lim_min);
      const uint16_t* qp = a.q + ((size_t)crow * a.hq + chead) * kHeadDim + 8 * h;
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) qf[ks] = ld16(qp + 16 * ks);
#pragma unroll
      for (int ks = 0; ks < 8; ++ks) {
        if (!ok) qf[ks] = u32x4{0u, 0u, 0u, 0u};
        asm volatile("" : "+v"(qf[ks]));
      }
    }
#pragma unroll
    for (int db = 0; db < 4; ++db) o[db] = f32x16{};
    m = kNegInf;
    lsum = 0.f;
    // barrier of the item's first stage: the previous item's last one, or
    // (first item) here
    if (first) {
      stage_barrier();
      issue_mid();
    }
    first = false;
    // iteration s reads K of sub-tile s + 1 (stage (s + 1) / 2) and V of
    // sub-tile s - 1 (stage (s - 1) / 2): stage j of the item sits in slot
    // (g0 + j) mod 4
    auto set_bases = [&](int ks_stage, int vs_stage) {
      kb = kofs + (uint32_t)(kWideKSlot * ((g0 + ks_stage) & (kWideSlots - 1)));
      vb = vofs + (uint32_t)(kWideKSlot * ((g0 + vs_stage) & (kWideSlots - 1)));
    };
    set_bases(0, 0);
    auto masked = [&](int T) { return T + 31 > lim_min; };
    // The last iteration also computes an S of the sub-tile past the item
    // (in-bounds LDS, result unused): one MFMA shape for every iteration
    // keeps the register allocation to a few schedules.
    if (wave_on) {
      // S(0), then iteration 0: S(1) beside the softmax of S(0)
      sc = s_tile(H0{});
      iter(H1{}, Tr{}, F{}, Tr{}, t0);
    }
    int s_ = 1;
    // pairs of iterations (odd s, then s + 1): unmasked while the later
    // sub-tile ends at or before every column's limit, masked after that
    // (the mask test is monotone in the sub-tile)
    for (; s_ + 1 < NS && !masked(t0 + 32 * (s_ + 1)); s_ += 2) {
      stage_barrier();
      set_bases((s_ + 1) >> 1, (s_ - 1) >> 1);
      if (wave_on) iter(H0{}, F{}, F{}, F{}, t0 + 32 * s_);
      issue_mid();
      if (wave_on) iter(H1{}, F{}, F{}, F{}, t0 + 32 * (s_ + 1));
    }
    for (; s_ + 1 < NS; s_ += 2) {
      stage_barrier();
      set_bases((s_ + 1) >> 1, (s_ - 1) >> 1);
      if (wave_on) iter(H0{}, F{}, F{}, Tr{}, t0 + 32 * s_);
      issue_mid();
      if (wave_on) iter(H1{}, F{}, F{}, Tr{}, t0 + 32 * (s_ + 1));
    }
    if (s_ < NS) {  // a last, odd iteration
      stage_barrier();
      set_bases((s_ + 1) >> 1, (s_ - 1) >> 1);
      if (wave_on) iter(H0{}, F{}, F{}, Tr{}, t0 + 32 * s_);
      issue_mid();
    }
    if (NS & 1) {
      // the last sub-tile opened a stage: its V is past the next barrier
      stage_barrier();
      issue_mid();
      set_bases(0, (NS - 1) >> 1);
    }
    g0 = (g0 + ((w.t1 - t0 + kWideStage - 1) / kWideStage)) & (kWideSlots - 1);
    if (!wave_on) continue;
    // PV of the last sub-tile (half (NS - 1) & 1 of the V slot at vb)
    auto pv_last = [&](auto half_) {
      constexpr int HALF = decltype(half_)::value;
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const uint32_t va = (vb ^ (64 * (i & 3))) + HALF * 8192 + (i >> 2) * 4096;
        const u32x2 lo = lds_read_tr16(va);
        const u32x2 hi = lds_read_tr16(va + 2048);
        o[i & 3] = mfma32<BF16>(u32x4{lo[0], lo[1], hi[0], hi[1]}, pp[i >> 2], o[i & 3]);
      }
    };
    if (NS & 1) pv_last(H0{});
    else pv_last(H1{});

    const float ln = sum_x32(lsum);
    const int col = wave * kWideCols + n;
    if (col >= ncols) continue;
    const int crow = w.q0 + col / G;
    const int chead = w.kvh * G + col % G;
    const float inv = ln > 0.f ? 1.f / ln : 0.f;
    const float l2 = ln > 0.f ? m + __log2f(ln) : kNegInf;
    uint16_t* op;
    if (w.part < 0) op = a.out + ((size_t)crow * a.hq + chead) * kHeadDim;
    else op = a.part_o + ((size_t)(w.part + col / G) * a.hq + chead) * kHeadDim;
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const u32x2 v = {pack2<BF16>(o[db][4 * j] * inv, o[db][4 * j + 1] * inv),
                         pack2<BF16>(o[db][4 * j + 2] * inv, o[db][4 * j + 3] * inv)};
        *reinterpret_cast<u32x2*>(op + 32 * db + 8 * j + 4 * h) = v;
      }
    if (h == 0) {
      if (w.part < 0) {
        if (a.lse != nullptr) a.lse[(size_t)crow * a.hq + chead] = l2 * kLn2;
      } else {
        a.part_lse[(size_t)(w.part + col / G) * a.hq + chead] = l2;
      }
    }
  }
  // Copies of stages past the share may still be in flight (cursor ahead of
  // the compute): let them land before the workgroup's LDS is released.
  wait_vmem<0>();
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
