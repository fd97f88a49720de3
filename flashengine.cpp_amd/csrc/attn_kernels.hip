// Paged-KV attention kernels for gfx950.
//
// Semantics follow the reference's attention boundary
// (include/fe/native_cuda.hpp:10; ATen statement src/portable_gpu_ops.cpp:39-44):
// out[r,h] = softmax_t(q[r,h].K[t, h/(hq/hkv)] / sqrt(128) + mask) . V[t, h/(hq/hkv)]
// with fp32 softmax and accumulation.  Softmax runs in the exp2 domain
// (scores pre-multiplied by log2(e)/sqrt(128)); log-sum-exp is kept in log2
// units internally and converted to natural log on output.
//
// Three kernels:
//  * attn_decode_kernel: persistent; each wavefront walks one share of the
//    decode token stream for one kv head (pieces of <= 16 (query row, head)
//    columns: decode rows x GQA heads along the MFMA N dimension), copying
//    Q / K / V units straight into a small LDS ring and computing
//    S^T = K Q^T and O^T = V^T P^T on the MFMA.
//  * attn_tile_kernel: four wavefronts share 64-token K / V tiles staged in
//    LDS; each wavefront owns 16 or 32 (query row, head) columns and
//    computes S^T = K Q^T and O^T = V^T P^T on the bf16/fp16 MFMA with fp32
//    accumulation (chunked prefill, DFlash blocks, verify rows).
//  * attn_merge_kernel: combines split-KV partials by their log-sum-exp, one
//    wavefront per (query row, head) with a batch of splits in flight.
// and stage_copy_kernel, which moves a prepared plan's metadata from pinned
// host memory into its device arena on the caller's stream.
#include <algorithm>
#include <atomic>
#include <type_traits>

#include "attn_types.hpp"
#include "device_util.hpp"
#include "kernel_util.hpp"

namespace feattn {


// ===========================================================================
// Decode kernel
// ===========================================================================
// Each wavefront slot owns one kv head and one share of the decode token
// stream (the planner's equal cut of all decode sequences, each piece a
// sequence's work item of <= 16 (query row, head) columns).  Consecutive
// slots are consecutive kv heads of the same share, so the WAVES wavefronts
// of a workgroup stream the same cache pages together.
//
// HBM -> LDS copies use direct-to-LDS loads (global_load_lds_dwordx4: lane i
// of an instruction lands at LDS base + 16 i).  A wavefront's share is one
// stream of 4 KB units -- per item: its Q (16 columns x 256 bytes), then
// K and V of each 16-token block -- copied into a ring of U unit slots that
// the wavefront owns.  Copies run up to U units ahead of the unit being
// computed, across item boundaries, so a wavefront keeps U - 2 units in
// flight while it computes.  Every copy instruction moves
// four whole 256-byte rows; inside a unit, 16-byte chunk c of row t sits at
// chunk position c ^ t (K, Q) or c ^ (2t mod 16) (V), which makes the
// operand reads below free of LDS bank conflicts.  Page ids and item
// metadata are read with scalar loads one block / one item ahead of use.
//
// Lane = 16*J + L.  Per block:
//   S^T = K Q^T:  A = K rows (lane: token L, dims 32s+8J..+8, ds_read_b128),
//                 B = Q^T (lane: column L, the same dims), 4 x 16x16x32 MFMA;
//                 C: lane holds tokens 4J+r (r = 0..3) of column L.
//   O^T += V^T P^T: A = V^T (lane: dim 16db+L, tokens 4J..4J+3, one
//                 ds_read_b64_tr_b16), B = P^T (lane: column L, tokens
//                 4J..4J+3 = its own S^T values), 8 x 16x16x16 MFMA;
//                 C: lane holds dims 16db+4J+r of column L.
// Softmax statistics are per column, i.e. per lane (reduced over J).
constexpr int kDecUnit = 4096;  // 16 rows x 256 bytes: one K or V block, or one item's Q

// Ring slots per wavefront.  Three (one unit in flight while a K/V pair is
// computed) measured fastest: with 8 wavefronts per CU, deeper rings only
// add queueing in the memory system (with the non-temporal K/V reads too:
// four slots took 99.5 against 98.7 us per headline step).
#ifndef FEATTN_DECODE_UNITS
#define FEATTN_DECODE_UNITS 3
#endif
template <int WAVES>
constexpr int dec_units() {
  static_assert(FEATTN_DECODE_UNITS * WAVES * kDecUnit <= kLdsBytes, "decode ring exceeds LDS");
  return FEATTN_DECODE_UNITS;
}


__device__ __forceinline__ DecodeItem ldc_ditem(const DecodeItem* items, int i) {
  const int32_t* p = reinterpret_cast<const int32_t*>(items + uniform(i));
  return DecodeItem{ldc(p, 0), ldc(p, 1), ldc(p, 2), ldc(p, 3), ldc(p, 4), ldc(p, 5), ldc(p, 6), ldc(p, 7)};
}

__device__ __forceinline__ ShareStart ldc_share(const ShareStart* shares, int i) {
  typedef const __attribute__((address_space(4))) i32x16* const_i32x16p;
  const i32x16 v = *(const_i32x16p)(shares + uniform(i));
  ShareStart r;
  r.it_begin = v[0];
  r.it_end = v[1];
  r.first = DecodeItem{v[2], v[3], v[4], v[5], v[6], v[7], v[8], v[9]};
  r.pg0 = v[10];
  r.pg1 = v[11];
  return r;
}

// NCB: 16-column blocks per item (1 or 2: up to 32 (query row, head)
// columns, e.g. 8 verify rows with 4 heads per kv head).  Four blocks would
// need more than the 256 registers of two wavefronts per SIMD.
template <bool BF16, int WAVES, int NCB>
__global__ __launch_bounds__(64 * WAVES) void attn_decode_kernel(AttnArgs a, int causal) {
  constexpr int U = dec_units<WAVES>();
  static_assert(U >= 2, "the ring must hold one K/V pair");
  extern __shared__ __attribute__((aligned(16))) uint8_t dsm[];
  const int lane = threadIdx.x & 63;
  const int J = lane >> 4;
  const int L = lane & 15;
  const int wave = uniform(threadIdx.x >> 6);
  const int G = a.group;
  const int pshift = a.page_shift;
  const int pmask = (1 << pshift) - 1;
  const uint32_t ring = (uint32_t)(uintptr_t)dsm + (uint32_t)(wave * U * kDecUnit);

  // Wavefront slot -> (kv head, share): consecutive slots are consecutive
  // kv heads of one share (WAVES divides hkv, so a workgroup holds one
  // share and its wavefronts walk the same blocks).  Records past the
  // shares in use are empty.
  const int slot = blockIdx.x * WAVES + wave;
  const int kvh = slot % a.hkv;
  const int share = slot / a.hkv;
  if (share >= a.n_share_cap) return;
  const ShareStart rec = ldc_share(a.shares, share);
  const int it_begin = rec.it_begin;
  const int it_end = rec.it_end;
  if (it_begin >= it_end) return;

  // Per-lane pieces of the copy and read addresses (fixed for the kernel).
  // Copy instruction r, lane i = 16*J + L: row 4r + J, chunk position L.
  const int row_bytes = a.hkv * kHeadDim * 2;
  int k_goff[4], v_goff[4];
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = 4 * r + J;
    k_goff[r] = t * row_bytes + 16 * (L ^ t);
    v_goff[r] = t * row_bytes + 16 * (L ^ ((2 * t) & 15));
  }
  // K operand for k-step s: token L, chunk 4s + J; Q operand: column L, same chunk.
  uint32_t k_lds[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) k_lds[s] = (uint32_t)(16 * (16 * L + (((4 * s + J) ^ L) & 15)));
  // V^T operand for dim block db: lane (J, L = 4k + m) points at token 4J + k,
  // dims 16 db + 4m .. +3 (chunk 2 db + m/2, half m%2).
  uint32_t v_lds[8];
  {
    const int k = L >> 2, m = L & 3, t = 4 * J + k;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int c = 2 * db + (m >> 1);
      v_lds[db] = (uint32_t)(16 * (16 * t + ((c ^ (2 * t)) & 15)) + 8 * (m & 1));
    }
  }

  const size_t head_off = (size_t)kvh * kHeadDim * 2;
  auto page_id = [&](const DecodeItem& d, int tok) { return ldc(a.pages, d.page_off + (tok >> pshift)); };
  auto block_addr = [&](const void* cache, int tok, int pg) {
    const size_t blk = (((size_t)pg << pshift) + (size_t)(tok & pmask)) * (size_t)row_bytes;
    return reinterpret_cast<const char*>(cache) + head_off + blk;
  };

  // ---- copy side: the next unit of the share's stream --------------------
  // kind 0 = Q of item c_it, 1 = K / 2 = V of block c_tok.  The following
  // item (nw) and the next K block's page id (pg_next) are requested one
  // item / one block before they are needed; the share record supplies the
  // first two page ids.
  int c_it = it_begin;
  DecodeItem cw = rec.first;
  DecodeItem nw = cw;
  if (c_it + 1 < it_end) nw = ldc_ditem(a.ditems, c_it + 1);
  int c_kind = 0;
  int c_qb = 0;  // column block of the next Q unit
  int c_tok = cw.t0;
  int pg_next = rec.pg0;
  int pg_after = rec.pg1;  // page of the block after pg_next's, valid while first_k
  bool first_k = true;
  int pg_cur = pg_next;
  bool c_live = true;
  int issued = 0;  // units copied so far
  int c_slot = 0;  // ring slot of the next copy

  auto issue_one = [&]() {
    const uint32_t dst = ring + (uint32_t)(c_slot * kDecUnit);
    if (c_kind == 0) {
      const int nc = cw.nq * G;
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int n = 4 * r + J;  // row of the unit = column within the block
        const int col = 16 * c_qb + n;
        const int nn = col < nc ? col : 0;  // columns past the item repeat column 0
        const int row = cw.q0 + nn / G;
        const int head = kvh * G + nn % G;
        lds_dma16(a.q + ((size_t)row * a.hq + head) * kHeadDim + 8 * (L ^ n), dst + 1024 * r);
      }
      if (++c_qb == NCB) {
        c_qb = 0;
        c_kind = 1;
      }
    } else if (c_kind == 1) {
      pg_cur = pg_next;
      const char* kb = block_addr(a.kc, c_tok, pg_cur);
#pragma unroll
      for (int r = 0; r < 4; ++r) lds_dma16<true>(kb + k_goff[r], dst + 1024 * r);
      // page of the next K block: later in this item, or the next item's first
      if (first_k) {
        pg_next = pg_after;
        first_k = false;
      } else if (c_tok + 16 < cw.t1) {
        pg_next = page_id(cw, c_tok + 16);
      } else if (c_it + 1 < it_end) {
        pg_next = page_id(nw, nw.t0);
      }
      c_kind = 2;
    } else {
      const char* vb = block_addr(a.vc, c_tok, pg_cur);
#pragma unroll
      for (int r = 0; r < 4; ++r) lds_dma16<true>(vb + v_goff[r], dst + 1024 * r);
      c_tok += 16;
      c_kind = 1;
      if (c_tok >= cw.t1) {
        ++c_it;
        if (c_it < it_end) {
          cw = nw;
          c_tok = cw.t0;
          c_kind = 0;
          if (c_it + 1 < it_end) nw = ldc_ditem(a.ditems, c_it + 1);
        } else {
          c_live = false;
        }
      }
    }
    ++issued;
    c_slot = c_slot + 1 == U ? 0 : c_slot + 1;
  };

  // ---- compute side --------------------------------------------------------
  int consumed = 0;  // units whose reads are complete
  int r_slot = 0;    // ring slot of the next unit to compute on
  // Refills every free slot; the slots freed last were read one step ago.
  auto refill = [&]() {
    wait_lds();
    while (c_live && issued - consumed < U) issue_one();
  };

  for (int it = it_begin; it < it_end; ++it) {
    refill();
    // the copy side read this item's record before (a scalar cache hit)
    const DecodeItem w = it == it_begin ? rec.first : ldc_ditem(a.ditems, it);
    const int t0 = w.t0;
    const int t1 = w.t1;
    const int ncols = w.nq * G;
    bool col_ok[NCB];
    int crow[NCB], chead[NCB], lim[NCB];  // lim: last visible token of the lane's column
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const int n = 16 * cb + L;
      col_ok[cb] = n < ncols;
      crow[cb] = w.q0 + (col_ok[cb] ? n / G : 0);
      chead[cb] = kvh * G + (col_ok[cb] ? n % G : 0);
      lim[cb] = -1;
      if (col_ok[cb]) lim[cb] = min(causal ? w.len - w.nq + (crow[cb] - w.q0) : w.len - 1, t1 - 1);
    }

    // Q units, one per column block
    u32x4 qf[NCB][4];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      if (cb > 0) refill();
      wait_units<U>(issued - consumed - 1);
      const uint32_t qb = ring + (uint32_t)(r_slot * kDecUnit);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        qf[cb][k] = lds_read16(qb + k_lds[k]);
        if (!col_ok[cb]) qf[cb][k] = u32x4{0u, 0u, 0u, 0u};
      }
      consumed += 1;
      r_slot = r_slot + 1 == U ? 0 : r_slot + 1;
    }

    float m[NCB], lsum[NCB];
    f32x4 o[8][NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      m[cb] = kNegInf;
      lsum[cb] = 0.f;
#pragma unroll
      for (int db = 0; db < 8; ++db) o[db][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
    }

    for (int tok = t0; tok < t1; tok += 16) {
      // The workgroup's wavefronts (consecutive kv heads of one share, the
      // same blocks in the same order) are brought back in step every four
      // blocks, so each page is requested by all of them at about the same
      // time (every block: 0.3 % slower; never: 0.8 % slower).
      if (((tok - t0) & 48) == 0) __builtin_amdgcn_s_barrier();
      refill();
      wait_units<U>(issued - consumed - 2);
      const uint32_t kst = ring + (uint32_t)(r_slot * kDecUnit);
      const int v_slot = r_slot + 1 == U ? 0 : r_slot + 1;
      const uint32_t vst = ring + (uint32_t)(v_slot * kDecUnit);

      f32x4 sc[NCB];
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) sc[cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const u32x4 kf = lds_read16(kst + k_lds[k]);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) sc[cb] = mfma16<BF16>(kf, qf[cb][k], sc[cb]);
      }

      u32x2 pf[NCB];
      float alpha[NCB];
      bool any_up = false;
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) {
        float x[4];
        float mx = kNegInf;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[r] = tok + 4 * J + r <= lim[cb] ? sc[cb][r] * a.scale_log2 : kNegInf;
          mx = fmaxf(mx, x[r]);
        }
        mx = max_x32(max_x16(mx));
        // Lazy reference maximum: raised (with l and o rescaled) only when the
        // block maximum exceeds it by more than 8, so p <= 2^8.
        const bool up = mx > m[cb] + 8.f;
        alpha[cb] = up ? fast_exp2(m[cb] - mx) : 1.f;
        if (up) m[cb] = mx;
        any_up = any_up || up;
        const float m_use = m[cb] == kNegInf ? 0.f : m[cb];
        float ps = 0.f;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[r] = fast_exp2(x[r] - m_use);
          ps += x[r];
        }
        lsum[cb] = lsum[cb] * alpha[cb] + ps;
        pf[cb] = u32x2{pack2<BF16>(x[0], x[1]), pack2<BF16>(x[2], x[3])};
      }

      if (t1 - tok < 16) {
        // Rows past the item end hold stale cache contents: zero them so that
        // 0 * (stale) can never become NaN.  (16-byte slot q holds part of
        // token row q / 16.)
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int q = lane + 64 * u;
          if ((q >> 4) >= t1 - tok) lds_zero16(vst + 16 * q);
        }
      }
      if (__builtin_amdgcn_ballot_w64(any_up) != 0) {
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb)
#pragma unroll
          for (int db = 0; db < 8; ++db) o[db][cb] *= alpha[cb];
      }
      u32x2 vf[8];
#pragma unroll
      for (int db = 0; db < 8; ++db) vf[db] = lds_read_tr16(vst + v_lds[db]);
#pragma unroll
      for (int db = 0; db < 8; ++db)
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) o[db][cb] = mfma16k16<BF16>(vf[db], pf[cb], o[db][cb]);
      consumed += 2;
      r_slot = v_slot + 1 == U ? 0 : v_slot + 1;
    }

#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      const float ls = sum_x32(sum_x16(lsum[cb]));
      if (col_ok[cb]) {
        const float inv = ls > 0.f ? 1.f / ls : 0.f;
        const float l2 = ls > 0.f ? m[cb] + __log2f(ls) : kNegInf;
        if (w.part < 0) {
          uint16_t* op = a.out + ((size_t)crow[cb] * a.hq + chead[cb]) * kHeadDim + 4 * J;
#pragma unroll
          for (int db = 0; db < 8; ++db) {
            const u32x2 v = {pack2<BF16>(o[db][cb][0] * inv, o[db][cb][1] * inv),
                             pack2<BF16>(o[db][cb][2] * inv, o[db][cb][3] * inv)};
            *reinterpret_cast<u32x2*>(op + 16 * db) = v;
          }
          if (a.lse != nullptr && J == 0) a.lse[(size_t)crow[cb] * a.hq + chead[cb]] = l2 * kLn2;
        } else {
          const size_t pslot = (size_t)(w.part + (16 * cb + L) / G);
          uint16_t* po = a.part_o + (pslot * a.hq + chead[cb]) * kHeadDim + 4 * J;
#pragma unroll
          for (int db = 0; db < 8; ++db) {
            const u32x2 v = {pack2<BF16>(o[db][cb][0] * inv, o[db][cb][1] * inv),
                             pack2<BF16>(o[db][cb][2] * inv, o[db][cb][3] * inv)};
            *reinterpret_cast<u32x2*>(po + 16 * db) = v;
          }
          if (J == 0) a.part_lse[pslot * a.hq + chead[cb]] = l2;
        }
      }
    }
  }
}

// ===========================================================================
// Tile kernel (MFMA for both products)
// ===========================================================================
// Four wavefronts share 64-token K and V tiles in LDS (two-stage ring of
// 32 KB stages: K blocks then V blocks, 16 tokens x 256 bytes each, chunk
// swizzles as in the decode kernel).  Wavefront w copies block w of each
// tile with direct-to-LDS loads; after its own copy lands and a barrier,
// the next tile's copy is issued and the current tile is computed.
//
// Columns: an item of <= 64 (query row, head) columns gives each wavefront
// NCB = 1 block of 16 columns, a larger item (<= 128) NCB = 2.  The item
// body is instantiated per NCB, and per tile for masked (diagonal / last)
// and unmasked tiles, so the unrolled MFMA sequences carry no branches.
// Per wavefront and tile:
//   S^T = K Q^T: A = K rows from LDS (lane: token 16tb+L, dims 32s+8J..+8),
//                B = Q^T in registers; C: lane holds tokens 16tb+4J+r of
//                column L.
//   O^T += V^T P^T with 16x16x32 MFMA over 32-token k-steps: the P^T operand
//                element e of lane (J, L) is token 32ks+4J+e (e < 4) or
//                32ks+16+4J+(e-4) (e >= 4) -- the lane's own S^T values of
//                blocks 2ks, 2ks+1 -- and the V^T operand reads the same
//                token order with one ds_read_b64_tr_b16 per block.
constexpr int kTileBlock = 4096;               // 16 tokens x 256 bytes
constexpr int kTileStage = 8 * kTileBlock;     // K blocks 0..3, then V blocks 0..3

struct TileLanes {
  int k_goff[4], v_goff[4];
  uint32_t k_lds[4], v_lds[8];
};

// Copies this wavefront's 16-token block (tokens T + 16 wave ..) of item
// w's tile starting at token T into ring stage `stage`; blocks at or past the
// item end are skipped.
template <bool STREAM>
__device__ __forceinline__ void tile_copy(const AttnArgs& a, const WorkItem& w, const SeqInfo& s,
                                          const TileLanes& tl, uint32_t lbase, int wave, int T, int stage) {
  const int tok = T + 16 * wave;
  if (tok >= w.t1) return;
  const int pshift = a.page_shift;
  const int row_bytes = a.hkv * kHeadDim * 2;
  const int pg = ldc(a.pages, s.page_off + (tok >> pshift));
  const size_t blk = (((size_t)pg << pshift) + (size_t)(tok & ((1 << pshift) - 1))) * (size_t)row_bytes +
                     (size_t)w.kvh * kHeadDim * 2;
  const char* kb = reinterpret_cast<const char*>(a.kc) + blk;
  const char* vb = reinterpret_cast<const char*>(a.vc) + blk;
  const uint32_t st = lbase + (uint32_t)(stage * kTileStage);
#pragma unroll
  for (int r = 0; r < 4; ++r) lds_dma16<STREAM>(kb + tl.k_goff[r], st + wave * kTileBlock + 1024 * r);
#pragma unroll
  for (int r = 0; r < 4; ++r) lds_dma16<STREAM>(vb + tl.v_goff[r], st + (4 + wave) * kTileBlock + 1024 * r);
}

// Computes item w whose first tile was already requested into stage
// `stage0`; during its last tile the first tile of the next item (wn, sn) is
// requested into the other stage, whose index is returned.
template <bool BF16, bool CAUSAL, int NCB, bool STREAM>
__device__ __forceinline__ int tile_item(const AttnArgs& a, const WorkItem& w, const SeqInfo& s, bool has_next,
                                         const WorkItem& wn, const SeqInfo& sn, const TileLanes& tl, uint32_t lbase,
                                         int wave, int lane, int stage0) {
  const int J = lane >> 4;
  const int L = lane & 15;
  const int G = a.group;
  const int kvh = w.kvh;
  const int t0 = w.t0;
  const int t1 = w.t1;
  const int ncols = w.nq * G;
  constexpr int kWcols = 16 * NCB;  // columns per wavefront
  const bool wave_on = wave * kWcols < ncols;


  int lim[NCB], crow[NCB], chead[NCB];
  u32x4 qf[NCB][4];
  int lim_min = 1 << 30;
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    const int n = wave * kWcols + 16 * cb + L;
    const bool ok = n < ncols;
    crow[cb] = w.q0 + (ok ? n / G : 0);
    chead[cb] = kvh * G + (ok ? n % G : 0);
    lim[cb] = -1;
    if (ok) lim[cb] = min(CAUSAL ? s.len - s.qlen + (crow[cb] - s.qo) : s.len - 1, t1 - 1);
    if (ok) lim_min = min(lim_min, lim[cb]);
    const uint16_t* qp = a.q + ((size_t)crow[cb] * a.hq + chead[cb]) * kHeadDim + 8 * J;
#pragma unroll
    for (int k = 0; k < 4; ++k) qf[cb][k] = ld16(qp + 32 * k);
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      if (!ok) qf[cb][k] = u32x4{0u, 0u, 0u, 0u};
      // Q (and the first tile's copy, issued before it) have landed past this
      // point; the registers are then plain values, so no wait for them falls
      // inside the tile loop while the next copy is in flight.
      asm volatile("" : "+v"(qf[cb][k]));
    }
  }
  // Tiles ending at or before every column's limit of the wavefront need no mask.
#pragma unroll
  for (int o_ = 32; o_ >= 1; o_ >>= 1) lim_min = min(lim_min, __shfl_xor(lim_min, o_, 64));

  float m[NCB], lsum[NCB];
  f32x4 o[8][NCB];
#pragma unroll
  for (int cb = 0; cb < NCB; ++cb) {
    m[cb] = kNegInf;
    lsum[cb] = 0.f;
#pragma unroll
    for (int db = 0; db < 8; ++db) o[db][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
  }

  auto compute = [&](uint32_t st, int T, auto masked) {
    constexpr bool MASK = decltype(masked)::value;
    f32x4 sc[4][NCB];
#pragma unroll
    for (int tb = 0; tb < 4; ++tb)
#pragma unroll
      for (int cb = 0; cb < NCB; ++cb) sc[tb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      // one base per k-step; the block offsets fold into the instruction
      const uint32_t kb = st + tl.k_lds[k];
#pragma unroll
      for (int tb = 0; tb < 4; ++tb) {
        const u32x4 kf = lds_read16(kb + tb * kTileBlock);
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) sc[tb][cb] = mfma16<BF16>(kf, qf[cb][k], sc[tb][cb]);
      }
    }

    u32x4 pf[2][NCB];
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      // Row max on raw scores (the scale is positive), then
      // p = exp2(s * scale - max * scale) with one FMA per element.
      float mx = kNegInf;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          if constexpr (MASK) {
            if (T + 16 * tb + 4 * J + r > lim[cb]) sc[tb][cb][r] = kNegInf;
          }
          mx = fmaxf(mx, sc[tb][cb][r]);
        }
      mx = max_x32(max_x16(mx));
      // Lazy reference maximum: raised (with l and o rescaled) only when the
      // tile maximum exceeds it by more than 8, so p <= 2^8.
      const float mt = mx * a.scale_log2;
      const bool up = mt > m[cb] + 8.f;
      const float alpha = up ? fast_exp2(m[cb] - mt) : 1.f;
      if (up) m[cb] = mt;
      const float m_use = m[cb] == kNegInf ? 0.f : m[cb];
      float x[4][4];
      float ps = 0.f;
#pragma unroll
      for (int tb = 0; tb < 4; ++tb)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[tb][r] = fast_exp2(__builtin_fmaf(sc[tb][cb][r], a.scale_log2, -m_use));
          ps += x[tb][r];
        }
      lsum[cb] = lsum[cb] * alpha + ps;
      if (__builtin_amdgcn_ballot_w64(up) != 0) {
#pragma unroll
        for (int db = 0; db < 8; ++db) o[db][cb] *= alpha;
      }
#pragma unroll
      for (int ks = 0; ks < 2; ++ks) {
        pf[ks][cb][0] = pack2<BF16>(x[2 * ks][0], x[2 * ks][1]);
        pf[ks][cb][1] = pack2<BF16>(x[2 * ks][2], x[2 * ks][3]);
        pf[ks][cb][2] = pack2<BF16>(x[2 * ks + 1][0], x[2 * ks + 1][1]);
        pf[ks][cb][3] = pack2<BF16>(x[2 * ks + 1][2], x[2 * ks + 1][3]);
      }
    }

    // k-step outer: the two MFMAs into one accumulator are 8 * NCB apart
#pragma unroll
    for (int ks = 0; ks < 2; ++ks)
#pragma unroll
      for (int db = 0; db < 8; ++db) {
        // one base per dim block; the block offsets fold into the instruction
        const uint32_t vb = st + tl.v_lds[db];
        const u32x2 lo = lds_read_tr16(vb + (4 + 2 * ks) * kTileBlock);
        const u32x2 hi = lds_read_tr16(vb + (5 + 2 * ks) * kTileBlock);
        const u32x4 vf = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
        for (int cb = 0; cb < NCB; ++cb) o[db][cb] = mfma16<BF16>(vf, pf[ks][cb], o[db][cb]);
      }
    // V^T operand reads three blocks ahead of their MFMAs (LDS latency)
    __builtin_amdgcn_sched_group_barrier(0x100, 6, 0);
#pragma unroll
    for (int i = 0; i < 13; ++i) {
      __builtin_amdgcn_sched_group_barrier(0x008, NCB, 0);
      __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
    }
    __builtin_amdgcn_sched_group_barrier(0x008, 3 * NCB, 0);
  };

  int stage = stage0;
  for (int T = t0; T < t1; T += kTileTokens) {
    wait_vmem<0>();  // this wavefront's block of the tile has landed
    const uint32_t st = lbase + (uint32_t)(stage * kTileStage);
    {
      // rows at or past the item end: zero V (0 * stale must stay 0)
      const int valid = t1 - (T + 16 * wave);
      if (valid < 16) {
        const uint32_t vblk = st + (4 + wave) * kTileBlock;
#pragma unroll
        for (int u = 0; u < 4; ++u) {
          const int q = lane + 64 * u;
          if ((q >> 4) >= valid) lds_zero16(vblk + 16 * q);
        }
      }
    }
    __syncthreads();  // every block of the tile is in LDS; the other stage is free
    if (T + kTileTokens < t1) tile_copy<STREAM>(a, w, s, tl, lbase, wave, T + kTileTokens, stage ^ 1);
    else if (has_next) tile_copy<STREAM>(a, wn, sn, tl, lbase, wave, wn.t0, stage ^ 1);
    if (wave_on) {
      if (T + kTileTokens - 1 <= lim_min) compute(st, T, std::false_type{});
      else compute(st, T, std::true_type{});
    }
    stage ^= 1;
  }

  if (wave_on) {
#pragma unroll
    for (int cb = 0; cb < NCB; ++cb) {
      float ln = lsum[cb];
      ln = sum_x32(sum_x16(ln));
      const int n = wave * kWcols + 16 * cb + L;
      if (n < ncols) {
        const float inv = ln > 0.f ? 1.f / ln : 0.f;
        const float l2 = ln > 0.f ? m[cb] + __log2f(ln) : kNegInf;
        if (w.part < 0) {
          uint16_t* op = a.out + ((size_t)crow[cb] * a.hq + chead[cb]) * kHeadDim + 4 * J;
#pragma unroll
          for (int db = 0; db < 8; ++db) {
            u32x2 v = {pack2<BF16>(o[db][cb][0] * inv, o[db][cb][1] * inv),
                       pack2<BF16>(o[db][cb][2] * inv, o[db][cb][3] * inv)};
            *reinterpret_cast<u32x2*>(op + 16 * db) = v;
          }
          if (a.lse != nullptr && J == 0) a.lse[(size_t)crow[cb] * a.hq + chead[cb]] = l2 * kLn2;
        } else {
          const size_t slot = (size_t)(w.part + (n / G));
          uint16_t* po = a.part_o + (slot * a.hq + chead[cb]) * kHeadDim + 4 * J;
#pragma unroll
          for (int db = 0; db < 8; ++db) {
            const u32x2 v = {pack2<BF16>(o[db][cb][0] * inv, o[db][cb][1] * inv),
                             pack2<BF16>(o[db][cb][2] * inv, o[db][cb][3] * inv)};
            *reinterpret_cast<u32x2*>(po + 16 * db) = v;
          }
          if (J == 0) a.part_lse[slot * a.hq + chead[cb]] = l2;
        }
      }
    }
  }
  return stage;
}

template <bool BF16, bool CAUSAL, bool STREAM>
__global__ __launch_bounds__(256, 2) void attn_tile_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t dsm[];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int J = lane >> 4;
  const int L = lane & 15;
  const int n_items = uniform(*a.n_items);
  const int row_bytes = a.hkv * kHeadDim * 2;
  const uint32_t lbase = (uint32_t)(uintptr_t)dsm;

  TileLanes tl;
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int t = 4 * r + J;
    tl.k_goff[r] = t * row_bytes + 16 * (L ^ t);
    tl.v_goff[r] = t * row_bytes + 16 * (L ^ ((2 * t) & 15));
  }
#pragma unroll
  for (int s = 0; s < 4; ++s) tl.k_lds[s] = (uint32_t)(16 * (16 * L + (((4 * s + J) ^ L) & 15)));
  {
    const int k = L >> 2, m = L & 3, t = 4 * J + k;
#pragma unroll
    for (int db = 0; db < 8; ++db) {
      const int c = 2 * db + (m >> 1);
      tl.v_lds[db] = (uint32_t)(16 * (16 * t + ((c ^ (2 * t)) & 15)) + 8 * (m & 1));
    }
  }

  // The workgroup's share of the item list (assigned by the planner,
  // longest items first); each item's first tile is requested during the
  // previous item's last tile.
  int it = ldc(a.tile_off, blockIdx.x);
  const int end = min(ldc(a.tile_off, blockIdx.x + 1), n_items);
  if (it >= end) return;
  WorkItem w = ldc_item(a.items, it);
  SeqInfo s = ldc_seq(a.seqs, w.seq);
  tile_copy<STREAM>(a, w, s, tl, lbase, wave, w.t0, 0);
  int stage = 0;
  for (;;) {
    const int nit = it + 1;
    const bool has_next = nit < end;
    WorkItem wn = w;
    SeqInfo sn = s;
    if (has_next) {
      wn = ldc_item(a.items, nit);
      sn = ldc_seq(a.seqs, wn.seq);
    }
    if (w.nq * a.group <= 64)
      stage = tile_item<BF16, CAUSAL, 1, STREAM>(a, w, s, has_next, wn, sn, tl, lbase, wave, lane, stage);
    else
      stage = tile_item<BF16, CAUSAL, 2, STREAM>(a, w, s, has_next, wn, sn, tl, lbase, wave, lane, stage);
    if (!has_next) break;
    it = nit;
    w = wn;
    s = sn;
  }
}

// ===========================================================================
// Split-KV merge
// ===========================================================================
// One wavefront per (merged row, pair of heads): lanes 0-31 take head 2hp,
// lanes 32-63 head 2hp + 1, each lane 4 of the 128 dims, so every partial-row
// load is one 8-byte access per lane.  Splits are folded in batches of
// kMergeBatch whose log-sum-exps and partial rows are all in flight
// together; loads past a row's split count are not issued.
template <bool BF16>
__global__ __launch_bounds__(256) void attn_merge_kernel(MergeArgs a) {
  const int lane = threadIdx.x & 63;
  const int hq = a.hq;
  const int hpairs = (hq + 1) >> 1;
  const int stride = gridDim.x * 4;
  // A graph launch folds the list of the latest prepare, found through the
  // header; an eager launch is handed the list and its length.
  const MergeRow* rows = a.rows;
  int n_rows = a.n_rows;
  if (a.count_base != nullptr) {
    n_rows = uniform(a.count_base[0]);
    rows += uniform(a.count_base[1]);
  }
  const int n_pairs = n_rows * hpairs;
  const int d = 4 * (lane & 31);
  for (int pair = blockIdx.x * 4 + uniform(threadIdx.x >> 6); pair < n_pairs; pair += stride) {
    const MergeRow mr = rows[pair / hpairs];
    const int h = 2 * (pair % hpairs) + (lane >> 5);
    const bool on = h < hq;
    const int hh = on ? h : hq - 1;
    constexpr int kMergeBatch = 8;
    float m = kNegInf, wsum = 0.f;
    f32x4 acc = {0.f, 0.f, 0.f, 0.f};
    for (int sp0 = 0; sp0 < mr.nsplit; sp0 += kMergeBatch) {
      float l[kMergeBatch];
      u32x2 rv[kMergeBatch];  // four 16-bit partial values
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        l[u] = kNegInf;
        rv[u] = u32x2{0u, 0u};
        if (sp0 + u < mr.nsplit) {  // wave-uniform
          const size_t slot = (size_t)(mr.part + (sp0 + u) * mr.stride);
          l[u] = a.part_lse[slot * hq + hh];
          rv[u] = *reinterpret_cast<const u32x2*>(a.part_o + (slot * hq + hh) * kHeadDim + d);
        }
      }
      float bm = m;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) bm = fmaxf(bm, l[u]);
      const float mu = bm == kNegInf ? 0.f : bm;
      const float sc = fast_exp2(m - mu);
      wsum *= sc;
      acc *= sc;
#pragma unroll
      for (int u = 0; u < kMergeBatch; ++u) {
        const float wt = fast_exp2(l[u] - mu);
        const f32x4 v = {lo_f32<BF16>(rv[u][0]), hi_f32<BF16>(rv[u][0]), lo_f32<BF16>(rv[u][1]),
                         hi_f32<BF16>(rv[u][1])};
        wsum += wt;
        acc += wt * v;
      }
      m = bm;
    }
    if (on) {
      const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
      const size_t oi = (size_t)mr.row * hq + h;
      const u32x2 o = {pack2<BF16>(acc[0] * inv, acc[1] * inv), pack2<BF16>(acc[2] * inv, acc[3] * inv)};
      *reinterpret_cast<u32x2*>(a.out + oi * kHeadDim + d) = o;
      if (a.lse != nullptr && (lane & 31) == 0) a.lse[oi] = wsum > 0.f ? (m + __log2f(wsum)) * kLn2 : kNegInf;
    }
  }
}

// ===========================================================================
// Launchers
// ===========================================================================
// Wavefronts per decode workgroup: consecutive kv heads of one share, as
// many as divide hkv (at most kDecodeWavesPerCu).
int decode_wg_waves(int hkv) {
  for (int w = kDecodeWavesPerCu; w > 1; w >>= 1)
    if (hkv % w == 0) return w;
  return 1;
}

template <bool BF16, int WAVES, int NCB>
static hipError_t decode_launch(const AttnArgs& a, int causal, int grid, hipStream_t st) {
  const size_t lds = (size_t)WAVES * dec_units<WAVES>() * kDecUnit + 16;
  static std::atomic<uint64_t> lds_ok{0};
  const hipError_t e = allow_lds((const void*)attn_decode_kernel<BF16, WAVES, NCB>, lds, lds_ok);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_decode_kernel<BF16, WAVES, NCB>), dim3(grid), dim3(64 * WAVES), lds, st, a, causal);
  return hipGetLastError();
}

template <bool BF16, int WAVES>
static hipError_t decode_launch_ncb(const AttnArgs& a, int ncb, int causal, int grid, hipStream_t st) {
  switch (ncb) {
    case 1: return decode_launch<BF16, WAVES, 1>(a, causal, grid, st);
    case 2: return decode_launch<BF16, WAVES, 2>(a, causal, grid, st);
    default: return hipErrorInvalidValue;
  }
}

template <bool BF16>
static hipError_t decode_launch_waves(const AttnArgs& a, int waves, int ncb, int causal, int grid, hipStream_t st) {
  switch (waves) {
    case 8: return decode_launch_ncb<BF16, 8>(a, ncb, causal, grid, st);
    case 4: return decode_launch_ncb<BF16, 4>(a, ncb, causal, grid, st);
    case 2: return decode_launch_ncb<BF16, 2>(a, ncb, causal, grid, st);
    case 1: return decode_launch_ncb<BF16, 1>(a, ncb, causal, grid, st);
    default: return hipErrorInvalidValue;
  }
}

hipError_t launch_decode(const AttnArgs& a, bool bf16, int waves, int ncb, int causal, int grid, hipStream_t st) {
  return bf16 ? decode_launch_waves<true>(a, waves, ncb, causal, grid, st)
              : decode_launch_waves<false>(a, waves, ncb, causal, grid, st);
}

// Plan staging: copies a prepared metadata image from pinned host memory
// (read through its device mapping) into the plan's device arena, as a
// kernel on the caller's stream.  A copy-engine transfer there costs about
// 20 us a step: the copy engine waits for the compute queue's previous
// kernels and the next kernel waits for the copy engine.  16 bytes per lane.
__global__ __launch_bounds__(256) void stage_copy_kernel(u32x4* dst, const u32x4* src, int n16) {
  for (int i = blockIdx.x * 256 + threadIdx.x; i < n16; i += gridDim.x * 256) dst[i] = src[i];
}

hipError_t launch_stage_copy(void* dst, const void* src, size_t bytes, hipStream_t st) {
  if (bytes % 16 != 0 || bytes / 16 > (size_t)INT32_MAX) return hipErrorInvalidValue;
  const int n16 = (int)(bytes / 16);
  const int grid = std::max(1, std::min(256, (n16 + 255) / 256));
  hipLaunchKernelGGL(stage_copy_kernel, dim3(grid), dim3(256), 0, st, static_cast<u32x4*>(dst),
                     static_cast<const u32x4*>(src), n16);
  return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, bool bf16, int grid, hipStream_t st) {
  if (bf16) hipLaunchKernelGGL((attn_merge_kernel<true>), dim3(grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL((attn_merge_kernel<false>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

template <bool BF16, bool CAUSAL, bool STREAM>
static hipError_t tile_launch(const AttnArgs& a, int grid, hipStream_t st) {
  const size_t lds = 2 * kTileStage;
  static std::atomic<uint64_t> lds_ok{0};
  const hipError_t e = allow_lds((const void*)attn_tile_kernel<BF16, CAUSAL, STREAM>, lds, lds_ok);
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL((attn_tile_kernel<BF16, CAUSAL, STREAM>), dim3(grid), dim3(256), lds, st, a);
  return hipGetLastError();
}

template <bool BF16, bool CAUSAL>
static hipError_t tile_launch(const AttnArgs& a, bool stream, int grid, hipStream_t st) {
  return stream ? tile_launch<BF16, CAUSAL, true>(a, grid, st) : tile_launch<BF16, CAUSAL, false>(a, grid, st);
}

hipError_t launch_tile(const AttnArgs& a, bool bf16, bool causal, bool stream, int grid, hipStream_t st) {
  if (bf16) return causal ? tile_launch<true, true>(a, stream, grid, st) : tile_launch<true, false>(a, stream, grid, st);
  return causal ? tile_launch<false, true>(a, stream, grid, st) : tile_launch<false, false>(a, stream, grid, st);
}

}  // namespace feattn
