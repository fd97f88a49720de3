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
//  * attn_decode_kernel: one wavefront per work item of at most 16
//    (query row, head) columns (decode rows, GQA heads packed along the MFMA
//    N dimension).  K streams straight from HBM into MFMA A-operand registers
//    (S^T = K Q^T); P.V runs on the VALU with coalesced 256-byte V row loads.
//  * attn_tile_kernel: four wavefronts share 64-token K / V^T tiles staged in
//    LDS; each wavefront owns 32 (query row, head) columns and computes
//    S^T = K Q^T and O^T = V^T P^T on the bf16/fp16 MFMA with fp32
//    accumulation (chunked prefill, DFlash blocks, verify rows).
//  * attn_merge_kernel: combines split-KV partials by their log-sum-exp.
#include <type_traits>

#include "attn_types.hpp"
#include "device_util.hpp"

namespace feattn {

template <int I, int N, typename F>
__device__ __forceinline__ void static_for(F&& f) {
  if constexpr (I < N) {
    f(std::integral_constant<int, I>{});
    static_for<I + 1, N>(f);
  }
}

__device__ __forceinline__ u32x4 ld16(const uint16_t* p) {
  return *reinterpret_cast<const u32x4*>(p);
}

// ===========================================================================
// Decode kernel
// ===========================================================================
// Lane = 16*J + L.  For a 16-token block starting at token `tok`:
//   K operand: lane loads token tok+L, elements 32*s + 8*J .. +8 for k-step s
//              (each instruction reads 64 contiguous bytes of 16 token rows);
//   Q operand: lane holds column L, the same elements;
//   S^T (C):   lane holds tokens tok + 4*J + r (r = 0..3) of column L;
//   V:         lane group J handles tokens tok + 4*J + r, lane L owns the
//              head dims 8*L .. 8*L+7 (one 16-byte load per token row,
//              16 lanes cover the 256-byte row).
template <bool BF16, int NC, int NB>
__global__ __launch_bounds__(256) void attn_decode_kernel(AttnArgs a, int causal) {
  const int lane = threadIdx.x & 63;
  const int J = lane >> 4;
  const int L = lane & 15;
  const int wave = uniform(threadIdx.x >> 6);
  const int n_items = uniform(*a.n_items);
  const int G = a.group;
  const int pshift = a.page_shift;
  const int pmask = (1 << pshift) - 1;

  for (int it = blockIdx.x * 4 + wave; it < n_items; it += gridDim.x * 4) {
    const WorkItem w = a.items[it];
    const SeqInfo s = a.seqs[uniform(w.seq)];
    const int kvh = uniform(w.kvh);
    const int t0 = uniform(w.t0);
    const int t1 = uniform(w.t1);
    const int ncols = uniform(w.nq) * G;

    const bool col_ok = L < ncols;
    const int crow = w.q0 + (col_ok ? L / G : 0);
    const int chead = kvh * G + (col_ok ? L % G : 0);
    int lim = -1;  // last visible token of column L
    if (col_ok) {
      lim = causal ? s.len - s.qlen + (crow - s.qo) : s.len - 1;
      lim = min(lim, t1 - 1);
    }

    u32x4 qf[4];
    {
      const uint16_t* qp = a.q + ((size_t)crow * a.hq + chead) * kHeadDim + 8 * J;
#pragma unroll
      for (int k = 0; k < 4; ++k) qf[k] = col_ok ? ld16(qp + 32 * k) : u32x4{0u, 0u, 0u, 0u};
    }

    float m = kNegInf;
    float lsum = 0.f;
    float acc[NC][8];
#pragma unroll
    for (int n = 0; n < NC; ++n)
#pragma unroll
      for (int e = 0; e < 8; ++e) acc[n][e] = 0.f;

    const size_t row_elems = (size_t)a.hkv * kHeadDim;
    const uint16_t* kbase = a.kc + (size_t)kvh * kHeadDim;
    const uint16_t* vbase = a.vc + (size_t)kvh * kHeadDim;

    for (int t = t0; t < t1; t += 16 * NB) {
      u32x4 kf[NB][4];
      u32x4 vf[NB][4];
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        const int tok = t + 16 * b;
        if (tok < t1) {
          const int pg = uniform(a.pages[s.page_off + (tok >> pshift)]);
          const size_t slot0 = ((size_t)pg << pshift) + (size_t)(tok & pmask);
          const uint16_t* kp = kbase + (slot0 + L) * row_elems + 8 * J;
#pragma unroll
          for (int k = 0; k < 4; ++k) kf[b][k] = ld16(kp + 32 * k);
#pragma unroll
          for (int r = 0; r < 4; ++r) {
            const uint16_t* vp = vbase + (slot0 + 4 * J + r) * row_elems + 8 * L;
            u32x4 v = ld16(vp);
            // Tokens past the item end hold stale cache contents; zero them so
            // that 0 * (stale) can never become NaN.
            if (tok + 4 * J + r >= t1) v = u32x4{0u, 0u, 0u, 0u};
            vf[b][r] = v;
          }
        } else {
#pragma unroll
          for (int k = 0; k < 4; ++k) {
            kf[b][k] = u32x4{0u, 0u, 0u, 0u};
            vf[b][k] = u32x4{0u, 0u, 0u, 0u};
          }
        }
      }

      // S^T = K Q^T, 16 tokens x 16 columns per block.
      float x[NB][4];
      float mx = kNegInf;
#pragma unroll
      for (int b = 0; b < NB; ++b) {
        f32x4 sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k) sc = mfma16<BF16>(kf[b][k], qf[k], sc);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          const int tok = t + 16 * b + 4 * J + r;
          const float v = tok <= lim ? sc[r] * a.scale_log2 : kNegInf;
          x[b][r] = v;
          mx = fmaxf(mx, v);
        }
      }
      mx = fmaxf(mx, xor16(mx));
      mx = fmaxf(mx, xor32(mx));
      const float m_new = fmaxf(m, mx);
      const float m_use = m_new == kNegInf ? 0.f : m_new;
      const float alpha = fast_exp2(m - m_use);
      float ps = 0.f;
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          x[b][r] = fast_exp2(x[b][r] - m_use);
          ps += x[b][r];
        }
      lsum = lsum * alpha + ps;
      m = m_new;

      static_for<0, NC>([&](auto n) {
        const float an = row_bcast<n>(alpha);
#pragma unroll
        for (int e = 0; e < 8; ++e) acc[n][e] *= an;
      });

      // O += P V on the VALU: lane group J owns tokens 4*J + r of each block.
#pragma unroll
      for (int b = 0; b < NB; ++b)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
          float v[8];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            v[2 * i] = lo_f32<BF16>(vf[b][r][i]);
            v[2 * i + 1] = hi_f32<BF16>(vf[b][r][i]);
          }
          const float pv = x[b][r];
          static_for<0, NC>([&](auto n) {
            const float pn = row_bcast<n>(pv);
#pragma unroll
            for (int e = 0; e < 8; ++e) acc[n][e] += pn * v[e];
          });
        }
    }

    // Combine the four lane groups (disjoint token subsets).
    lsum += xor16(lsum);
    lsum += xor32(lsum);
#pragma unroll
    for (int n = 0; n < NC; ++n)
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        acc[n][e] += xor16(acc[n][e]);
        acc[n][e] += xor32(acc[n][e]);
      }

    static_for<0, NC>([&](auto n) {
      const float ln = row_bcast<n>(lsum);
      const float mn = row_bcast<n>(m);
      if (n < ncols && J == (n & 3)) {
        const int row = w.q0 + n / G;
        const int head = kvh * G + n % G;
        const float inv = ln > 0.f ? 1.f / ln : 0.f;
        const float l2 = ln > 0.f ? mn + __log2f(ln) : kNegInf;
        if (w.part < 0) {
          u32x4 o;
#pragma unroll
          for (int i = 0; i < 4; ++i) o[i] = pack2<BF16>(acc[n][2 * i] * inv, acc[n][2 * i + 1] * inv);
          *reinterpret_cast<u32x4*>(a.out + ((size_t)row * a.hq + head) * kHeadDim + 8 * L) = o;
          if (a.lse != nullptr && L == 0) a.lse[(size_t)row * a.hq + head] = l2 * kLn2;
        } else {
          const size_t slot = (size_t)(w.part + n / G);
          float* po = a.part_o + (slot * a.hq + head) * kHeadDim + 8 * L;
          f32x4 o0 = {acc[n][0] * inv, acc[n][1] * inv, acc[n][2] * inv, acc[n][3] * inv};
          f32x4 o1 = {acc[n][4] * inv, acc[n][5] * inv, acc[n][6] * inv, acc[n][7] * inv};
          reinterpret_cast<f32x4*>(po)[0] = o0;
          reinterpret_cast<f32x4*>(po)[1] = o1;
          if (L == 0) a.part_lse[slot * a.hq + head] = l2;
        }
      }
    });
  }
}

// ===========================================================================
// Tile kernel (MFMA for both products)
// ===========================================================================
// LDS: K tile [64 tokens][128 dims] with rows padded to 272 bytes and a
// transposed V tile [128 dims][64 tokens] with rows padded to 136 bytes, so
// the 16 rows read by one MFMA operand fetch fall in distinct banks.
constexpr int kKStride = 272;
constexpr int kVStride = 136;
constexpr int kLdsK = kTileTokens * kKStride;
constexpr int kLdsV = kHeadDim * kVStride;

// Per wavefront: columns 32*wave + 16*cb + L (cb = 0, 1).
// S^T block (tb, cb): lane holds tokens 16*tb + 4*J + r of its column.
// P^T operand for k-step ks covers tokens 32*ks .. 32*ks+31; lane element e
// is token 32*ks + 4*J + e (e < 4) or 32*ks + 16 + 4*J + (e-4) (e >= 4), which
// is exactly what the lane holds of S^T blocks 2*ks and 2*ks+1.  The V^T
// operand reads the same token order from LDS.
template <bool BF16, bool CAUSAL>
__global__ __launch_bounds__(256, 2) void attn_tile_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint8_t lds[kLdsK + kLdsV];
  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = uniform(tid >> 6);
  const int J = lane >> 4;
  const int L = lane & 15;
  const int n_items = uniform(*a.n_items);
  const int G = a.group;
  const int pshift = a.page_shift;
  const int pmask = (1 << pshift) - 1;
  const size_t row_elems = (size_t)a.hkv * kHeadDim;

  for (int it = blockIdx.x; it < n_items; it += gridDim.x) {
    const WorkItem w = a.items[it];
    const SeqInfo s = a.seqs[uniform(w.seq)];
    const int kvh = uniform(w.kvh);
    const int t0 = uniform(w.t0);
    const int t1 = uniform(w.t1);
    const int ncols = uniform(w.nq) * G;
    const bool wave_on = 32 * wave < ncols;

    int lim[2];
    int crow[2];
    int chead[2];
    u32x4 qf[2][4];
#pragma unroll
    for (int cb = 0; cb < 2; ++cb) {
      const int n = 32 * wave + 16 * cb + L;
      const bool ok = n < ncols;
      crow[cb] = w.q0 + (ok ? n / G : 0);
      chead[cb] = kvh * G + (ok ? n % G : 0);
      lim[cb] = -1;
      if (ok) lim[cb] = min(CAUSAL ? s.len - s.qlen + (crow[cb] - s.qo) : s.len - 1, t1 - 1);
      const uint16_t* qp = a.q + ((size_t)crow[cb] * a.hq + chead[cb]) * kHeadDim + 8 * J;
#pragma unroll
      for (int k = 0; k < 4; ++k) qf[cb][k] = ok ? ld16(qp + 32 * k) : u32x4{0u, 0u, 0u, 0u};
    }

    float m[2] = {kNegInf, kNegInf};
    float lsum[2] = {0.f, 0.f};
    f32x4 o[8][2];
#pragma unroll
    for (int db = 0; db < 8; ++db)
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) o[db][cb] = f32x4{0.f, 0.f, 0.f, 0.f};

    // Global -> register staging of one 64-token tile.
    u32x4 kr[4];
    u32x4 v0[2];
    u32x4 v1[2];
    auto gload = [&](int T) {
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int qd = tid + 256 * k;
        const int tok = T + (qd >> 4);
        const int c = qd & 15;
        u32x4 val = {0u, 0u, 0u, 0u};
        if (tok < t1) {
          const int pg = a.pages[s.page_off + (tok >> pshift)];
          const size_t slot = ((size_t)pg << pshift) + (size_t)(tok & pmask);
          val = ld16(a.kc + slot * row_elems + (size_t)kvh * kHeadDim + 8 * c);
        }
        kr[k] = val;
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int qd = tid + 256 * k;
        const int tok = T + 2 * (qd >> 4);
        const int c = qd & 15;
        u32x4 x0 = {0u, 0u, 0u, 0u};
        u32x4 x1 = {0u, 0u, 0u, 0u};
        if (tok < t1) {
          const int pg = a.pages[s.page_off + (tok >> pshift)];
          const size_t slot = ((size_t)pg << pshift) + (size_t)(tok & pmask);
          const uint16_t* vp = a.vc + slot * row_elems + (size_t)kvh * kHeadDim + 8 * c;
          x0 = ld16(vp);
          // tok is even and pages hold a multiple of 16 tokens, so tok+1 is
          // in the same page.
          if (tok + 1 < t1) x1 = ld16(vp + row_elems);
        }
        v0[k] = x0;
        v1[k] = x1;
      }
    };

    gload(t0);
    for (int T = t0; T < t1; T += kTileTokens) {
      __syncthreads();
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        const int qd = tid + 256 * k;
        *reinterpret_cast<u32x4*>(lds + (qd >> 4) * kKStride + 16 * (qd & 15)) = kr[k];
      }
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const int qd = tid + 256 * k;
        const int pr = qd >> 4;
        const int c = qd & 15;
        uint8_t* vt = lds + kLdsK + 4 * pr;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const uint32_t x0 = v0[k][i];
          const uint32_t x1 = v1[k][i];
          *reinterpret_cast<uint32_t*>(vt + (8 * c + 2 * i) * kVStride) = (x0 & 0xffffu) | (x1 << 16);
          *reinterpret_cast<uint32_t*>(vt + (8 * c + 2 * i + 1) * kVStride) = (x0 >> 16) | (x1 & 0xffff0000u);
        }
      }
      __syncthreads();
      if (T + kTileTokens < t1) gload(T + kTileTokens);

      if (wave_on) {
        f32x4 sc[4][2];
#pragma unroll
        for (int tb = 0; tb < 4; ++tb)
#pragma unroll
          for (int cb = 0; cb < 2; ++cb) sc[tb][cb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int k = 0; k < 4; ++k)
#pragma unroll
          for (int tb = 0; tb < 4; ++tb) {
            const u32x4 kfrag =
                *reinterpret_cast<const u32x4*>(lds + (16 * tb + L) * kKStride + 64 * k + 16 * J);
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) sc[tb][cb] = mfma16<BF16>(kfrag, qf[cb][k], sc[tb][cb]);
          }

        u32x4 pf[2][2];
#pragma unroll
        for (int cb = 0; cb < 2; ++cb) {
          float x[4][4];
          float mx = kNegInf;
#pragma unroll
          for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              const int tok = T + 16 * tb + 4 * J + r;
              const float v = tok <= lim[cb] ? sc[tb][cb][r] * a.scale_log2 : kNegInf;
              x[tb][r] = v;
              mx = fmaxf(mx, v);
            }
          mx = fmaxf(mx, xor16(mx));
          mx = fmaxf(mx, xor32(mx));
          const float m_new = fmaxf(m[cb], mx);
          const float m_use = m_new == kNegInf ? 0.f : m_new;
          const float alpha = fast_exp2(m[cb] - m_use);
          float ps = 0.f;
#pragma unroll
          for (int tb = 0; tb < 4; ++tb)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
              x[tb][r] = fast_exp2(x[tb][r] - m_use);
              ps += x[tb][r];
            }
          lsum[cb] = lsum[cb] * alpha + ps;
          m[cb] = m_new;
#pragma unroll
          for (int db = 0; db < 8; ++db) o[db][cb] *= alpha;
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            pf[ks][cb][0] = pack2<BF16>(x[2 * ks][0], x[2 * ks][1]);
            pf[ks][cb][1] = pack2<BF16>(x[2 * ks][2], x[2 * ks][3]);
            pf[ks][cb][2] = pack2<BF16>(x[2 * ks + 1][0], x[2 * ks + 1][1]);
            pf[ks][cb][3] = pack2<BF16>(x[2 * ks + 1][2], x[2 * ks + 1][3]);
          }
        }

#pragma unroll
        for (int db = 0; db < 8; ++db)
#pragma unroll
          for (int ks = 0; ks < 2; ++ks) {
            const uint8_t* vb = lds + kLdsK + (16 * db + L) * kVStride + 64 * ks + 8 * J;
            const u32x2 lo = *reinterpret_cast<const u32x2*>(vb);
            const u32x2 hi = *reinterpret_cast<const u32x2*>(vb + 32);
            const u32x4 vfrag = {lo[0], lo[1], hi[0], hi[1]};
#pragma unroll
            for (int cb = 0; cb < 2; ++cb) o[db][cb] = mfma16<BF16>(vfrag, pf[ks][cb], o[db][cb]);
          }
      }
    }

    if (wave_on) {
#pragma unroll
      for (int cb = 0; cb < 2; ++cb) {
        float ln = lsum[cb];
        ln += xor16(ln);
        ln += xor32(ln);
        const int n = 32 * wave + 16 * cb + L;
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
            float* po = a.part_o + (slot * a.hq + chead[cb]) * kHeadDim + 4 * J;
#pragma unroll
            for (int db = 0; db < 8; ++db) *reinterpret_cast<f32x4*>(po + 16 * db) = o[db][cb] * inv;
            if (J == 0) a.part_lse[slot * a.hq + chead[cb]] = l2;
          }
        }
      }
    }
    __syncthreads();  // LDS reuse by the next item
  }
}

// ===========================================================================
// Split-KV merge
// ===========================================================================
// One workgroup per merged row; thread handles 4 dims of one head per pass.
template <bool BF16>
__global__ __launch_bounds__(256) void attn_merge_kernel(MergeArgs a) {
  const int n_rows = uniform(*a.n_rows);
  const int hq = a.hq;
  for (int idx = blockIdx.x; idx < n_rows; idx += gridDim.x) {
    const MergeRow mr = a.rows[idx];
    for (int e = threadIdx.x; e < hq * 32; e += blockDim.x) {
      const int h = e >> 5;
      const int d = (e & 31) * 4;
      float mx = kNegInf;
      for (int sp = 0; sp < mr.nsplit; ++sp)
        mx = fmaxf(mx, a.part_lse[(size_t)(mr.part + sp * mr.stride) * hq + h]);
      const float mu = mx == kNegInf ? 0.f : mx;
      float wsum = 0.f;
      f32x4 acc = {0.f, 0.f, 0.f, 0.f};
      for (int sp = 0; sp < mr.nsplit; ++sp) {
        const size_t slot = (size_t)(mr.part + sp * mr.stride);
        const float wgt = fast_exp2(a.part_lse[slot * hq + h] - mu);
        wsum += wgt;
        acc += wgt * *reinterpret_cast<const f32x4*>(a.part_o + (slot * hq + h) * kHeadDim + d);
      }
      const float inv = wsum > 0.f ? 1.f / wsum : 0.f;
      u32x2 v = {pack2<BF16>(acc[0] * inv, acc[1] * inv), pack2<BF16>(acc[2] * inv, acc[3] * inv)};
      *reinterpret_cast<u32x2*>(a.out + ((size_t)mr.row * hq + h) * kHeadDim + d) = v;
      if (a.lse != nullptr && d == 0)
        a.lse[(size_t)mr.row * hq + h] = wsum > 0.f ? (mu + __log2f(wsum)) * kLn2 : kNegInf;
    }
  }
}

// ===========================================================================
// Launchers
// ===========================================================================
template <bool BF16>
static hipError_t decode_dispatch(const AttnArgs& a, int nc, int causal, int grid, hipStream_t st) {
  switch (nc) {
    case 4:
      hipLaunchKernelGGL((attn_decode_kernel<BF16, 4, 4>), dim3(grid), dim3(256), 0, st, a, causal);
      break;
    case 8:
      hipLaunchKernelGGL((attn_decode_kernel<BF16, 8, 2>), dim3(grid), dim3(256), 0, st, a, causal);
      break;
    case 16:
      hipLaunchKernelGGL((attn_decode_kernel<BF16, 16, 2>), dim3(grid), dim3(256), 0, st, a, causal);
      break;
    default:
      return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t launch_decode(const AttnArgs& a, bool bf16, int nc, int causal, int grid, hipStream_t st) {
  return bf16 ? decode_dispatch<true>(a, nc, causal, grid, st) : decode_dispatch<false>(a, nc, causal, grid, st);
}

hipError_t launch_tile(const AttnArgs& a, bool bf16, bool causal, int grid, hipStream_t st) {
  if (bf16) {
    if (causal) hipLaunchKernelGGL((attn_tile_kernel<true, true>), dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((attn_tile_kernel<true, false>), dim3(grid), dim3(256), 0, st, a);
  } else {
    if (causal) hipLaunchKernelGGL((attn_tile_kernel<false, true>), dim3(grid), dim3(256), 0, st, a);
    else hipLaunchKernelGGL((attn_tile_kernel<false, false>), dim3(grid), dim3(256), 0, st, a);
  }
  return hipGetLastError();
}

hipError_t launch_merge(const MergeArgs& a, bool bf16, int grid, hipStream_t st) {
  if (bf16) hipLaunchKernelGGL((attn_merge_kernel<true>), dim3(grid), dim3(256), 0, st, a);
  else hipLaunchKernelGGL((attn_merge_kernel<false>), dim3(grid), dim3(256), 0, st, a);
  return hipGetLastError();
}

}  // namespace feattn
