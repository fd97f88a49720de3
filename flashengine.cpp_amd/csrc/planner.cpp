// Host planner.  Validation mirrors the reference's checks
// (src/flashinfer_attention.cu:23,30; src/portable_gpu_ops.cpp:28-30) and adds
// the ones a raw-pointer kernel needs to stay in bounds (page ids, `last`).
#include "planner.hpp"

#include <algorithm>
#include <new>

#include "fe_attn.h"

namespace feattn {

namespace {

// Shortest decode share: below this, per-piece start-up and merge cost more
// than the extra wavefronts gain.
constexpr int64_t kMinShareTokens = 64;

bool is_pow2(int v) { return v > 0 && (v & (v - 1)) == 0; }

int round_up(int v, int m) { return (v + m - 1) / m * m; }

int ceil_div(int a, int b) { return (a + b - 1) / b; }

// Share boundaries (token offsets into the decode stream, multiples of 16):
// equal shares of `quota` tokens.
std::vector<int64_t> cut_uniform(int64_t stream, int64_t quota) {
  std::vector<int64_t> cuts;
  for (int64_t c = 0; c < stream; c += quota) cuts.push_back(c);
  cuts.push_back(stream);
  return cuts;
}

}  // namespace

// Assigns items to `slots` shares (one per tile workgroup) by the longest
// processing time rule -- in decreasing cost order, each item goes to the
// least-loaded share -- and regroups them share by share (longest first
// inside a share).  off receives the CSR offsets of the shares in use.
void assign_shares(std::vector<WorkItem>& items, int slots, std::vector<int32_t>& off, int fast) {
  // Stable sort by decreasing cost: a counting sort over the (small,
  // non-negative) costs, else the comparison sort.
  int32_t cmin = 0, cmax = 0;
  for (const WorkItem& w : items) {
    cmin = std::min(cmin, w.cost);
    cmax = std::max(cmax, w.cost);
  }
  if (cmin >= 0 && cmax <= (1 << 16)) {
    std::vector<int32_t> start((size_t)cmax + 2, 0);
    for (const WorkItem& w : items) ++start[(size_t)(cmax - w.cost) + 1];
    for (size_t c = 1; c < start.size(); ++c) start[c] += start[c - 1];
    std::vector<WorkItem> sorted(items.size());
    for (const WorkItem& w : items) sorted[start[(size_t)(cmax - w.cost)]++] = w;
    items.swap(sorted);
  } else {
    std::stable_sort(items.begin(), items.end(),
                     [](const WorkItem& x, const WorkItem& y) { return x.cost > y.cost; });
  }
  const int n = std::max(1, std::min<int>(slots, (int)items.size()));
  std::vector<int> share(items.size());
  // Binary min-heap of (load << 20 | share) keys: the root is the least-loaded
  // share, the lowest index among equals.  Each item raises the root's load
  // and sifts it down (one pass instead of a pop and a push).  Shares below
  // `fast` count their load at kFastShareWeight / kSlowShareWeight (2/3): they
  // end up with 3/2 of the others' work.
  constexpr int kShareBits = 20;  // shares (tile workgroups) < 2^20; loads < 2^43
  const bool weighted = fast < n;
  std::vector<uint64_t> heap(n);
  for (int k = 0; k < n; ++k) heap[k] = (uint64_t)k;  // ascending: already a heap
  for (size_t i = 0; i < items.size(); ++i) {
    const int k = (int)(heap[0] & ((uint64_t(1) << kShareBits) - 1));
    share[i] = k;
    const uint64_t w = !weighted ? 1 : (k < fast ? kFastShareWeight : kSlowShareWeight);
    const uint64_t key = heap[0] + (((uint64_t)items[i].cost * w) << kShareBits);
    size_t h = 0;
    for (;;) {
      size_t c = 2 * h + 1;
      if (c >= (size_t)n) break;
      if (c + 1 < (size_t)n && heap[c + 1] < heap[c]) ++c;
      if (heap[c] >= key) break;
      heap[h] = heap[c];
      h = c;
    }
    heap[h] = key;
  }
  off.assign(n + 1, 0);
  for (size_t i = 0; i < items.size(); ++i) ++off[share[i] + 1];
  for (int k = 0; k < n; ++k) off[k + 1] += off[k];
  std::vector<WorkItem> grouped(items.size());
  std::vector<int32_t> pos(off.begin(), off.end() - 1);
  for (size_t i = 0; i < items.size(); ++i) grouped[pos[share[i]]++] = items[i];
  items.swap(grouped);
}

namespace {

// Tile work list by an equal cut of the tile stream: the query-row chunks of
// the tile sequences (qr rows each, over their visible token ranges), in
// batch order, are laid end to end and cut at tile boundaries into `slots /
// hkv` shares of equal cost (tiles x 16-column blocks per wavefront).  Every
// kv head uses the same cut, and share k of kv head h goes to workgroup
// k * hkv + h, so the workgroups of one share read the same pages at the same
// time.  A chunk cut into several pieces gets partial slots and merge rows
// as in the longest-first list.  Returns false, leaving `ml` alone, when the
// cut needs more partial slots or items than `slot_budget` / `item_cap`.
bool cut_tile_stream(const std::vector<SeqInfo>& seqs, int G, int hkv, bool causal, int slots, int partial_base,
                     int slot_budget, int item_cap, ModeLists& ml) {
  const int qr = kTileCols / G;
  const int n_shares = slots / hkv;
  if (n_shares < 1) return false;
  struct Chunk {
    int seq, q0, nq, extent, tiles, c;
  };
  std::vector<Chunk> ch;
  int64_t total = 0;
  for (int b = 0; b < (int)seqs.size(); ++b) {
    const SeqInfo& s = seqs[b];
    if (s.qlen * G <= kDecodeCols) continue;
    for (int i0 = 0; i0 < s.qlen; i0 += qr) {
      const int nq = std::min(qr, s.qlen - i0);
      const int extent = causal ? std::min(s.len, s.len - s.qlen + i0 + nq) : s.len;
      const int tiles = ceil_div(extent, kTileTokens);
      const int c = nq * G > kTileCols / 2 ? 2 : 1;
      ch.push_back(Chunk{b, s.qo + i0, nq, extent, tiles, c});
      total += (int64_t)tiles * c;
    }
  }
  if (ch.empty()) return false;
  // Pieces in stream order: (chunk, first tile, tiles, share).  Share k ends
  // at the first tile boundary where the cumulative cost reaches
  // (k + 1) * total / n_shares, so a tile's granularity never accumulates
  // from share to share; the last share ends with the stream.
  struct Piece {
    int chunk, tile0, ntiles, share;
  };
  std::vector<Piece> pcs;
  std::vector<int> npc(ch.size(), 0);
  int share = 0;
  int64_t cum = 0;
  auto target = [&](int k) { return ((int64_t)(k + 1) * total + n_shares - 1) / n_shares; };
  for (int i = 0; i < (int)ch.size(); ++i) {
    int done = 0;
    while (done < ch[i].tiles) {
      while (share < n_shares - 1 && cum >= target(share)) ++share;
      int take = ch[i].tiles - done;
      if (share < n_shares - 1) {
        const int64_t need = (target(share) - cum + ch[i].c - 1) / ch[i].c;  // >= 1 tile
        take = (int)std::min<int64_t>(need, take);
      }
      pcs.push_back(Piece{i, done, take, share});
      ++npc[i];
      done += take;
      cum += (int64_t)take * ch[i].c;
    }
  }
  if ((int64_t)pcs.size() * hkv > item_cap) return false;
  std::vector<int> base(ch.size(), -1);
  int64_t rows = partial_base;
  for (size_t i = 0; i < ch.size(); ++i)
    if (npc[i] > 1) {
      base[i] = (int)rows;
      rows += (int64_t)npc[i] * ch[i].nq;
    }
  if (rows > slot_budget) return false;

  ModeLists out;
  out.partial_rows = (int)rows;
  for (size_t i = 0; i < ch.size(); ++i)
    if (base[i] >= 0)
      for (int r = 0; r < ch[i].nq; ++r) out.merge.push_back(MergeRow{ch[i].q0 + r, base[i] + r, npc[i], ch[i].nq});
  // Piece p's index within its chunk (pieces of a chunk are consecutive).
  std::vector<int> sp(pcs.size());
  for (size_t p = 0; p < pcs.size(); ++p) sp[p] = (p > 0 && pcs[p - 1].chunk == pcs[p].chunk) ? sp[p - 1] + 1 : 0;
  const int used = pcs.back().share + 1;
  out.tile.reserve(pcs.size() * (size_t)hkv);
  out.tile_off.assign((size_t)used * hkv + 1, 0);
  size_t p0 = 0;
  for (int k = 0; k < used; ++k) {
    size_t p1 = p0;
    while (p1 < pcs.size() && pcs[p1].share == k) ++p1;
    for (int h = 0; h < hkv; ++h) {
      for (size_t p = p0; p < p1; ++p) {
        const Chunk& c = ch[pcs[p].chunk];
        const int t0 = pcs[p].tile0 * kTileTokens;
        const int t1 = std::min(c.extent, (pcs[p].tile0 + pcs[p].ntiles) * kTileTokens);
        const int part = base[pcs[p].chunk] < 0 ? -1 : base[pcs[p].chunk] + sp[p] * c.nq;
        out.tile.push_back(WorkItem{c.seq, c.q0, c.nq, h, t0, t1, part, pcs[p].ntiles * c.c});
      }
      out.tile_off[(size_t)k * hkv + h + 1] = (int32_t)out.tile.size();
    }
    p0 = p1;
  }
  ml = std::move(out);
  return true;
}

}  // namespace

int validate_shape(const PlanShape& sh, std::string& err) {
  if (sh.dim != kHeadDim) {
    err = "attention supports head_dim 128 only (got " + std::to_string(sh.dim) + ")";
    return FE_EINVAL;
  }
  if (sh.hq <= 0 || sh.hkv <= 0 || sh.hq % sh.hkv != 0) {
    err = "hq must be a positive multiple of hkv";
    return FE_EINVAL;
  }
  if (sh.hq / sh.hkv > kTileCols) {
    err = "GQA group larger than 128 query heads per kv head";
    return FE_EINVAL;
  }
  if (!is_pow2(sh.page) || sh.page < 16) {
    err = "page size must be a power of two >= 16";
    return FE_EINVAL;
  }
  if (sh.max_batch <= 0 || sh.max_pages <= 0 || sh.blocks < 0) {
    err = "max_batch and max_pages must be positive, blocks non-negative";
    return FE_EINVAL;
  }
  return FE_OK;
}

static int build_plan_impl(const PlanShape& sh, const int32_t* qo, const int32_t* kv, const int32_t* pages,
               const int32_t* last, int batch, int rows, BuiltPlan& out, std::string& err) {
  int rc = validate_shape(sh, err);
  if (rc != FE_OK) return rc;
  if (batch < 0 || rows < 0) {
    err = "negative batch or rows";
    return FE_EINVAL;
  }
  if (batch > sh.max_batch) {
    err = "attention metadata exceeds capacity: batch " + std::to_string(batch) + " > max_batch " +
          std::to_string(sh.max_batch);
    return FE_ECAPACITY;
  }
  out = BuiltPlan();
  if (batch > 0 && (qo == nullptr || kv == nullptr || last == nullptr)) {
    err = "null metadata pointer";
    return FE_EINVAL;
  }
  const int64_t max_context = (int64_t)(sh.max_pages - 1) * sh.page;
  if (batch > 0) {
    if (qo[0] < 0 || kv[0] < 0) {
      err = "qo[0] and kv[0] must be non-negative";
      return FE_EINVAL;
    }
    if ((int64_t)kv[batch] > (int64_t)sh.max_batch * sh.max_pages) {
      err = "attention metadata exceeds capacity: kv[batch] > max_batch * max_pages";
      return FE_ECAPACITY;
    }
    if (kv[batch] > 0 && pages == nullptr) {
      err = "null page table";
      return FE_EINVAL;
    }
  }
  out.seqs.resize(batch);
  for (int b = 0; b < batch; ++b) {
    const int np = kv[b + 1] - kv[b];
    const int ql = qo[b + 1] - qo[b];
    if (np < 1 || ql < 0) {
      err = "sequence " + std::to_string(b) + ": qo/kv offsets must be non-decreasing with >= 1 page";
      return FE_EINVAL;
    }
    if (last[b] < 1 || last[b] > sh.page) {
      err = "sequence " + std::to_string(b) + ": last must be in [1, page]";
      return FE_EINVAL;
    }
    const int64_t len = (int64_t)(np - 1) * sh.page + last[b];
    if (len < ql || len > max_context) {
      err = "attention context out of range for sequence " + std::to_string(b) + " (len " + std::to_string(len) +
            ", query rows " + std::to_string(ql) + ", max_context " + std::to_string(max_context) + ")";
      return FE_EINVAL;
    }
    for (int i = kv[b]; i < kv[b + 1]; ++i) {
      if (pages[i] < 0 || pages[i] > sh.blocks) {
        err = "page id " + std::to_string(pages[i]) + " outside [0, blocks]";
        return FE_EINVAL;
      }
    }
    out.seqs[b] = SeqInfo{qo[b], ql, (int32_t)len, kv[b]};
  }
  if (batch > 0 && qo[batch] > rows) {
    err = "qo[batch] exceeds rows";
    return FE_EINVAL;
  }

  const int G = sh.hq / sh.hkv;
  const int slot_budget = sh.partial_cap;

  // ---- decode pieces: sequences whose (rows x group) fit one MFMA column
  // block.  Each kv head's token stream -- the decode sequences one after
  // another, each padded to whole 16-token blocks -- is cut into equal
  // shares, one per decode wavefront slot (decode_waves / hkv shares); a
  // share's pieces are its intersections with the sequences.  Every kv head
  // uses the same cut, so the wavefronts of one workgroup (consecutive kv
  // heads of one share) read the same pages at the same time.  A sequence
  // cut into several pieces is merged by log-sum-exp afterwards; when the
  // partials would not fit, shares grow (fewer wavefronts busy).
  int max_cols = 0;
  int64_t stream = 0;
  for (int b = 0; b < batch; ++b) {
    const SeqInfo& s = out.seqs[b];
    if (s.qlen > 0 && s.qlen * G <= kDecodeCols) {
      stream += round_up(s.len, 16);
      max_cols = std::max(max_cols, s.qlen * G);
    }
  }
  // columns per decode item, in 16-column MFMA blocks: 1 or 2 blocks
  out.decode_nc = max_cols <= 16 ? 16 : 32;
  const int n_static = std::max(1, sh.decode_waves / sh.hkv);
  if (stream > 0) {
    // Partial slots and pieces that a cut needs (a sequence overlapping
    // several shares is cut into pieces, each with qlen partial rows).
    auto cost_of = [&](const std::vector<int64_t>& cuts, int64_t& slots, int64_t& pieces) {
      slots = pieces = 0;
      int64_t off = 0;
      size_t k = 0;
      for (int b = 0; b < batch; ++b) {
        const SeqInfo& s = out.seqs[b];
        if (s.qlen == 0 || s.qlen * G > kDecodeCols) continue;
        const int64_t end = off + round_up(s.len, 16);
        while (cuts[k + 1] <= off) ++k;
        size_t k1 = k;
        while (cuts[k1 + 1] < end) ++k1;
        const int64_t np = (int64_t)(k1 - k + 1);
        if (np > 1) slots += np * s.qlen;
        pieces += np;
        off = end;
      }
    };
    auto fits = [&](const std::vector<int64_t>& cuts) {
      int64_t slots, pieces;
      cost_of(cuts, slots, pieces);
      return slots <= slot_budget && pieces <= sh.item_cap;
    };
    std::vector<int64_t> cuts;
    int64_t quota = std::max<int64_t>(kMinShareTokens, round_up((int)((stream + n_static - 1) / n_static), 16));
    for (;;) {
      cuts = cut_uniform(stream, quota);
      if (fits(cuts)) break;
      if (quota >= stream) {
        err = "attention metadata exceeds capacity: decode work list";
        return FE_ECAPACITY;
      }
      quota *= 2;
    }
    const int used = (int)cuts.size() - 1;
    out.decode_share_off.assign(used + 1, 0);
    int64_t off = 0;
    int share = 0;
    size_t k = 0;
    for (int b = 0; b < batch; ++b) {
      const SeqInfo& s = out.seqs[b];
      if (s.qlen == 0 || s.qlen * G > kDecodeCols) continue;
      const int64_t end = off + round_up(s.len, 16);
      while (cuts[k + 1] <= off) ++k;
      size_t k1 = k;
      while (cuts[k1 + 1] < end) ++k1;
      const int np = (int)(k1 - k + 1);
      int base = -1;
      if (np > 1) {
        base = out.decode_partials;
        out.decode_partials += np * s.qlen;
        for (int r = 0; r < s.qlen; ++r) out.decode_merge.push_back(MergeRow{s.qo + r, base + r, np, s.qlen});
      }
      for (size_t j = k; j <= k1; ++j) {
        while (share < (int)j) out.decode_share_off[++share] = (int32_t)out.decode.size();
        const int t0 = (int)(std::max<int64_t>(off, cuts[j]) - off);
        const int t1 = (int)std::min<int64_t>(s.len, std::min<int64_t>(end, cuts[j + 1]) - off);
        out.decode.push_back(
            WorkItem{b, s.qo, s.qlen, 0, t0, t1, base < 0 ? -1 : base + (int)(j - k) * s.qlen, t1 - t0});
      }
      off = end;
    }
    while (share < used) out.decode_share_off[++share] = (int32_t)out.decode.size();
    out.decode_items.resize(out.decode.size());
    for (size_t i = 0; i < out.decode.size(); ++i) {
      const WorkItem& w = out.decode[i];
      const SeqInfo& sq = out.seqs[w.seq];
      out.decode_items[i] = DecodeItem{w.q0, w.nq, sq.len, sq.page_off, w.t0, w.t1, w.part, w.seq};
    }
    auto page_of = [&](const DecodeItem& d, int tok) { return pages[d.page_off + tok / sh.page]; };
    out.decode_starts.assign(used, ShareStart{});
    for (int k = 0; k < used; ++k) {
      ShareStart& ss = out.decode_starts[k];
      ss.it_begin = out.decode_share_off[k];
      ss.it_end = out.decode_share_off[k + 1];
      if (ss.it_begin >= ss.it_end) continue;
      const DecodeItem& d = out.decode_items[ss.it_begin];
      ss.first = d;
      ss.pg0 = page_of(d, d.t0);
      if (d.t0 + 16 < d.t1) ss.pg1 = page_of(d, d.t0 + 16);
      else if (ss.it_begin + 1 < ss.it_end) {
        const DecodeItem& d2 = out.decode_items[ss.it_begin + 1];
        ss.pg1 = page_of(d2, d2.t0);
      }
    }
  }

  // ---- tile items, per mask mode.
  const int qr = kTileCols / G;  // query rows per tile item
  for (int causal = 0; causal < 2; ++causal) {
    ModeLists& ml = out.mode[causal];
    ml.partial_rows = out.decode_partials;
    // (q tile, kv head) pairs before splitting, to size the split factor.
    int64_t pairs = 0;
    for (int b = 0; b < batch; ++b) {
      const SeqInfo& s = out.seqs[b];
      if (s.qlen * G > kDecodeCols) pairs += (int64_t)ceil_div(s.qlen, qr) * sh.hkv;
    }
    if (pairs == 0) continue;
    // Aim for about 8 items per compute unit (2 resident workgroups, several
    // rounds in longest-first order); never split below 256 tokens.
    int want = (int)std::max<int64_t>(1, ((int64_t)sh.num_cus * 8 + pairs - 1) / pairs);
    for (;;) {
      ml.tile.clear();
      ml.tile.reserve((size_t)std::min<int64_t>(pairs * want, sh.item_cap + 1));  // at most want pieces per pair
      ml.merge.clear();
      ml.partial_rows = out.decode_partials;
      for (int b = 0; b < batch; ++b) {
        const SeqInfo& s = out.seqs[b];
        if (s.qlen * G <= kDecodeCols) continue;
        for (int i0 = 0; i0 < s.qlen; i0 += qr) {
          const int nq = std::min(qr, s.qlen - i0);
          const int extent = causal ? std::min(s.len, s.len - s.qlen + i0 + nq) : s.len;
          int ns = std::max(1, std::min(want, extent / 256));
          int chunk = round_up(ceil_div(extent, ns), kTileTokens);
          ns = ceil_div(extent, chunk);
          int base = -1;
          if (ns > 1) {
            base = ml.partial_rows;
            ml.partial_rows += ns * nq;
            for (int r = 0; r < nq; ++r) ml.merge.push_back(MergeRow{s.qo + i0 + r, base + r, ns, nq});
          }
          for (int sp = 0; sp < ns; ++sp) {
            const int t0 = sp * chunk;
            const int t1 = std::min(extent, t0 + chunk);
            // Cost ~ tiles times the 16-column blocks each wavefront
            // computes (1 for items of <= 64 columns, else 2).
            const int cost = ceil_div(t1 - t0, kTileTokens) * (nq * G > kTileCols / 2 ? 2 : 1);
            for (int h = 0; h < sh.hkv; ++h)
              ml.tile.push_back(WorkItem{b, s.qo + i0, nq, h, t0, t1, base < 0 ? -1 : base + sp * nq, cost});
          }
        }
      }
      if (ml.partial_rows <= slot_budget && ml.tile.size() <= (size_t)sh.item_cap) break;
      if (want == 1) {
        err = "attention metadata exceeds capacity: tile work list (" + std::to_string(ml.tile.size()) + " items)";
        return FE_ECAPACITY;
      }
      want = std::max(1, want / 2);
    }
    // Two tile workgroups share each CU; the first of the pair to be
    // dispatched (workgroup b < num_cus) wins the SIMDs' issue arbitration
    // and, at equal work, finished the 8192-token prefill in 184 us against
    // 230 us for the second.  The first ones therefore get more of the work:
    // 3/2 of the second's measured fastest (0.261 against 0.267 ms for equal
    // shares; 4/3 gained 1 %, 2/1 lost), since the second speeds up once its
    // partner has finished.
    assign_shares(ml.tile, sh.tile_slots, ml.tile_off, sh.num_cus);
    // When the longest-first list had to split chunks anyway, an equal cut
    // of the tile stream balances the workgroups to within a tile, usually
    // with fewer pieces; it replaces the list if it needs no more partial rows.
    if (ml.partial_rows > out.decode_partials) {
      ModeLists cut;
      if (cut_tile_stream(out.seqs, G, sh.hkv, causal != 0, sh.tile_slots, out.decode_partials, slot_budget,
                          sh.item_cap, cut) &&
          cut.partial_rows <= ml.partial_rows)
        ml = std::move(cut);
    }
  }
  for (int causal = 0; causal < 2; ++causal) {
    std::vector<MergeRow>& m = out.mode[causal].merge;
    m.insert(m.begin(), out.decode_merge.begin(), out.decode_merge.end());
    if (m.size() > (size_t)slot_budget) {
      err = "attention metadata exceeds capacity: merge rows";
      return FE_ECAPACITY;
    }
  }
  return FE_OK;
}

int build_plan(const PlanShape& sh, const int32_t* qo, const int32_t* kv, const int32_t* pages,
               const int32_t* last, int batch, int rows, BuiltPlan& out, std::string& err) {
  try {
    return build_plan_impl(sh, qo, kv, pages, last, batch, rows, out, err);
  } catch (const std::bad_alloc&) {
    err = "out of host memory while building the work lists";
    return FE_ENOMEM;
  }
}

}  // namespace feattn

