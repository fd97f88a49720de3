// Host planner under AddressSanitizer / UndefinedBehaviorSanitizer: random
// valid batches (decode rows, verify rows, 16-row blocks, prefill chunks;
// several head layouts and page sizes) must plan into work lists whose every
// index stays inside the lists, the sequences and the partial workspace, and
// whose pieces cover each (query rows, kv head) token range exactly once;
// corrupted metadata must be refused with an error code.  A second pass runs
// serving steps through the host driver (the FIFO page allocator and the
// per-step metadata builder, graph padding included) into the planner.
// Built and run by tests/test_planner_sanitized.py (g++ with
// -fsanitize=address,undefined).
#include <stdint.h>
#include <stdio.h>

#include <algorithm>
#include <random>
#include <string>
#include <unordered_map>
#include <vector>

#include "fe_attn.h"
#include "fe_driver.h"
#include "planner.hpp"

namespace feattn {
// The library's error reporter lives with the HIP entry points; the host
// code under test only needs its contract (returns `code`).
int report_error(int code, const std::string& msg) {
  (void)msg;
  return code;
}
}  // namespace feattn

using namespace feattn;

namespace {

int g_fail = 0;

#define CHECK(cond, ...)                                   \
  do {                                                     \
    if (!(cond)) {                                         \
      fprintf(stderr, "check failed: %s: ", #cond);        \
      fprintf(stderr, __VA_ARGS__);                        \
      fprintf(stderr, "\n");                               \
      ++g_fail;                                            \
      return false;                                        \
    }                                                      \
  } while (0)

struct Batch {
  int hq, hkv, page, blocks, max_batch, max_pages, rows;
  std::vector<int32_t> qo, kv, pages, last;
  int batch() const { return (int)last.size(); }
};

Batch random_batch(std::mt19937& rng) {
  static const int heads[][2] = {{32, 8}, {32, 4}, {16, 16}, {64, 8}, {8, 1}, {40, 8}, {28, 4}, {128, 1}};
  static const int pages_sz[] = {16, 16, 32, 64};
  Batch b;
  const auto& h = heads[rng() % 8];
  b.hq = h[0];
  b.hkv = h[1];
  b.page = pages_sz[rng() % 4];
  const int n = (int)(rng() % 49);
  std::vector<int> starts(n), qlens(n);
  for (int i = 0; i < n; ++i) {
    const int kind = (int)(rng() % 10);
    int q = 1;
    if (kind == 6) q = 2 + (int)(rng() % 7);
    else if (kind == 7) q = 16;
    else if (kind == 8) q = 17 + (int)(rng() % 300);
    else if (kind == 9) q = 300 + (int)(rng() % 1300);
    qlens[i] = q;
    starts[i] = (int)(rng() % 3) == 0 ? 0 : (int)(rng() % 9000);
  }
  b.qo.assign(1, 0);
  b.kv.assign(1, 0);
  int maxp = 1;
  for (int i = 0; i < n; ++i) {
    const int len = starts[i] + qlens[i];
    const int np = (len + b.page - 1) / b.page;
    b.qo.push_back(b.qo.back() + qlens[i]);
    b.kv.push_back(b.kv.back() + np);
    b.last.push_back(len - (np - 1) * b.page);
    maxp = std::max(maxp, np);
  }
  const int total = b.kv.back();
  b.blocks = total + (int)(rng() % 5);
  std::vector<int32_t> perm(b.blocks + 1);
  for (int i = 0; i <= b.blocks; ++i) perm[i] = i;
  std::shuffle(perm.begin(), perm.end(), rng);
  b.pages.assign(perm.begin(), perm.begin() + total);
  if (total > 0 && rng() % 4 == 0) b.pages[rng() % total] = b.pages[0];  // shared pages are allowed
  b.max_batch = std::max(1, n + (int)(rng() % 3));
  b.max_pages = maxp + 1 + (int)(rng() % 3);
  b.rows = b.qo.back() + (int)(rng() % 4);
  return b;
}

PlanShape shape_of(const Batch& b) {
  PlanShape sh;
  sh.hq = b.hq;
  sh.hkv = b.hkv;
  sh.dim = 128;
  sh.page = b.page;
  sh.max_batch = b.max_batch;
  sh.max_pages = b.max_pages;
  sh.blocks = b.blocks;
  sh.partial_cap = std::max<int>(1024, (int)((64u << 20) / ((size_t)b.hq * 129 * 4)));
  return sh;
}

// Pieces [t0, t1) of one (rows, kv head) unit must tile [0, extent) exactly.
bool covers(std::vector<std::pair<int, int>> pcs, int extent, const char* what, int key) {
  std::sort(pcs.begin(), pcs.end());
  int at = 0;
  for (const auto& p : pcs) {
    CHECK(p.first == at, "%s %d: piece starts at %d, expected %d", what, key, p.first, at);
    CHECK(p.second > p.first, "%s %d: empty piece at %d", what, key, p.first);
    at = p.second;
  }
  CHECK(at == extent, "%s %d: pieces end at %d, extent %d", what, key, at, extent);
  return true;
}

bool check_plan(const Batch& b, const PlanShape& sh, const BuiltPlan& bp) {
  const int G = sh.hq / sh.hkv;
  const int nb = b.batch();
  CHECK((int)bp.seqs.size() == nb, "seqs %zu", bp.seqs.size());
  // decode pieces
  const size_t nd = bp.decode.size();
  CHECK(bp.decode_items.size() == nd, "decode items %zu vs %zu", bp.decode_items.size(), nd);
  if (!bp.decode_share_off.empty()) {
    CHECK(bp.decode_share_off.front() == 0 && (size_t)bp.decode_share_off.back() == nd, "decode share offsets");
    for (size_t k = 0; k + 1 < bp.decode_share_off.size(); ++k)
      CHECK(bp.decode_share_off[k] <= bp.decode_share_off[k + 1], "decode share %zu", k);
    CHECK(bp.decode_starts.size() + 1 == bp.decode_share_off.size(), "decode starts %zu", bp.decode_starts.size());
  }
  std::vector<std::vector<std::pair<int, int>>> dcov(nb);
  for (size_t i = 0; i < nd; ++i) {
    const WorkItem& w = bp.decode[i];
    CHECK(w.seq >= 0 && w.seq < nb, "decode item %zu seq %d", i, w.seq);
    const SeqInfo& s = bp.seqs[w.seq];
    CHECK(s.qlen * G <= kDecodeCols, "decode item %zu has %d columns", i, s.qlen * G);
    CHECK(w.t0 >= 0 && w.t0 < w.t1 && w.t1 <= s.len, "decode item %zu tokens [%d, %d) of %d", i, w.t0, w.t1, s.len);
    CHECK(w.part < 0 || (w.part >= 0 && w.part + s.qlen <= bp.decode_partials), "decode item %zu part %d", i, w.part);
    const DecodeItem& d = bp.decode_items[i];
    CHECK(d.q0 == s.qo && d.nq == s.qlen && d.len == s.len && d.page_off == s.page_off && d.t0 == w.t0 &&
              d.t1 == w.t1 && d.part == w.part,
          "decode item %zu record", i);
    CHECK(d.page_off + (d.t1 - 1) / sh.page < b.kv[w.seq + 1], "decode item %zu page range", i);
    dcov[w.seq].push_back({w.t0, w.t1});
  }
  for (int s = 0; s < nb; ++s)
    if (bp.seqs[s].qlen > 0 && bp.seqs[s].qlen * G <= kDecodeCols && !covers(dcov[s], bp.seqs[s].len, "decode seq", s))
      return false;
  for (size_t k = 0; k < bp.decode_starts.size(); ++k) {
    const ShareStart& ss = bp.decode_starts[k];
    CHECK(ss.it_begin >= 0 && ss.it_begin <= ss.it_end && (size_t)ss.it_end <= nd, "share %zu range", k);
    if (ss.it_begin < ss.it_end) {
      const DecodeItem& d = bp.decode_items[ss.it_begin];
      CHECK(ss.pg0 == b.pages[d.page_off + d.t0 / sh.page], "share %zu first page", k);
    }
  }
  // tile lists of both masks
  for (int m = 0; m < 2; ++m) {
    const ModeLists& ml = bp.mode[m];
    const bool causal = m == 1;
    CHECK(ml.partial_rows >= bp.decode_partials && ml.partial_rows <= sh.partial_cap, "mode %d partial rows %d", m,
          ml.partial_rows);
    if (!ml.tile_off.empty()) {
      CHECK(ml.tile_off.front() == 0 && (size_t)ml.tile_off.back() == ml.tile.size(), "mode %d tile offsets", m);
      for (size_t k = 0; k + 1 < ml.tile_off.size(); ++k)
        CHECK(ml.tile_off[k] <= ml.tile_off[k + 1], "mode %d share %zu", m, k);
      CHECK((int)ml.tile_off.size() - 1 <= sh.tile_slots, "mode %d shares %zu", m, ml.tile_off.size());
    } else {
      CHECK(ml.tile.empty(), "mode %d items without shares", m);
    }
    // unit key: (first row, kv head) -> pieces
    std::vector<std::vector<std::pair<int, int>>> tcov((size_t)std::max(1, b.rows) * sh.hkv);
    std::vector<int> ext((size_t)std::max(1, b.rows) * sh.hkv, -1);
    for (size_t i = 0; i < ml.tile.size(); ++i) {
      const WorkItem& w = ml.tile[i];
      CHECK(w.seq >= 0 && w.seq < nb, "tile item %zu seq %d", i, w.seq);
      const SeqInfo& s = bp.seqs[w.seq];
      CHECK(s.qlen * G > kDecodeCols, "tile item %zu of a decode sequence", i);
      CHECK(w.kvh >= 0 && w.kvh < sh.hkv, "tile item %zu kv head %d", i, w.kvh);
      CHECK(w.nq >= 1 && w.nq * G <= kTileCols && w.q0 >= s.qo && w.q0 + w.nq <= s.qo + s.qlen,
            "tile item %zu rows [%d, +%d)", i, w.q0, w.nq);
      const int extent = causal ? std::min(s.len, s.len - s.qlen + (w.q0 - s.qo) + w.nq) : s.len;
      CHECK(w.t0 >= 0 && w.t0 < w.t1 && w.t1 <= extent, "tile item %zu tokens [%d, %d) of %d", i, w.t0, w.t1, extent);
      CHECK(w.t0 % kTileTokens == 0, "tile item %zu starts off a tile boundary", i);
      CHECK(w.part < 0 || (w.part >= bp.decode_partials && w.part + w.nq <= ml.partial_rows), "tile item %zu part %d", i,
            w.part);
      const size_t key = (size_t)w.q0 * sh.hkv + w.kvh;
      tcov[key].push_back({w.t0, w.t1});
      ext[key] = extent;
    }
    for (size_t key = 0; key < tcov.size(); ++key)
      if (!tcov[key].empty() && !covers(tcov[key], ext[key], "tile unit", (int)key)) return false;
    for (size_t r = 0; r < ml.merge.size(); ++r) {
      const MergeRow& mr = ml.merge[r];
      CHECK(mr.row >= 0 && mr.row < b.rows && mr.nsplit >= 2 && mr.stride >= 1, "merge row %zu", r);
      CHECK(mr.part >= 0 && (int64_t)mr.part + (int64_t)(mr.nsplit - 1) * mr.stride < ml.partial_rows, "merge row %zu slots",
            r);
    }
  }
  return true;
}

// A copy of a valid batch with one field corrupted; build_plan must refuse it.
bool check_refused(const Batch& good, std::mt19937& rng) {
  if (good.batch() == 0) return true;
  Batch b = good;
  const int s = (int)(rng() % b.batch());
  const int kind = (int)(rng() % 5);
  if (kind == 0) b.last[s] = 0;
  else if (kind == 1) b.last[s] = b.page + 1;
  else if (kind == 2 && b.kv[s + 1] > b.kv[s]) b.pages[b.kv[s]] = b.blocks + 1;
  else if (kind == 3) b.kv[s + 1] = b.kv[s];  // a sequence with no page
  else b.max_batch = b.batch() - 1;
  const PlanShape sh = shape_of(b);
  BuiltPlan bp;
  std::string err;
  const int rc = build_plan(sh, b.qo.data(), b.kv.data(), b.pages.data(), b.last.data(), b.batch(), b.rows, bp, err);
  CHECK(rc != FE_OK, "corruption %d of sequence %d was accepted", kind, s);
  CHECK(!err.empty(), "corruption %d refused without a message", kind);
  return true;
}

// Serving steps: sequences arrive with prompts that share prefixes, take the
// longest cached prefix from the allocator's prefix cache, prefill the rest
// in chunks, decode a token per step, publish what they computed, are
// preempted (their pages released and probed again) or finish; every step's
// metadata comes from the page allocator and fe_prepare_metadata (padded to a
// graph bucket at times) and must plan cleanly.
bool serve(std::mt19937& rng, int steps, int& planned) {
  const int page = 16, pool = 1200;  // small enough for the free queue to wrap: evictions
  fe_blocks* blocks = nullptr;
  CHECK(fe_blocks_create_ex(pool, page, 1, &blocks) == FE_OK, "allocator");
  struct Seq {
    int64_t id, len;
    std::vector<int64_t> tokens;
    bool probed;
  };
  std::vector<std::vector<int64_t>> stems(4);
  for (auto& st : stems) {
    st.resize(rng() % 700);
    for (auto& t : st) t = (int64_t)(rng() % 4);
  }
  std::vector<Seq> live;
  int64_t next_id = 0, hits = 0;
  for (int step = 0; step < steps; ++step) {
    // arrivals, departures and preemptions
    if (live.size() < 40 && rng() % 2 == 0) {
      Seq q{next_id++, 0, {}, false};
      const auto& st = stems[rng() % stems.size()];
      q.tokens.assign(st.begin(), st.begin() + (long)(rng() % (st.size() + 1)));
      for (int t = 1 + (int)(rng() % 200); t > 0; --t) q.tokens.push_back((int64_t)(rng() % 4));
      live.push_back(std::move(q));
    }
    if (!live.empty() && rng() % 5 == 0) {
      const size_t k = rng() % live.size();
      CHECK(fe_blocks_forget(blocks, live[k].id) == FE_OK, "forget");
      live.erase(live.begin() + (long)k);
    }
    if (!live.empty() && rng() % 11 == 0) {
      Seq& q = live[rng() % live.size()];
      CHECK(fe_blocks_release(blocks, q.id) == FE_OK, "release");
      q.len = 0;
      q.probed = false;
    }
    std::vector<int64_t> start;
    std::vector<int32_t> rows, table_off(1, 0), tables;
    std::vector<size_t> in_step;
    for (size_t k = 0; k < live.size(); ++k) {
      Seq& q = live[k];
      if (!q.probed) {
        int64_t cached = -1;
        CHECK(fe_blocks_probe(blocks, q.id, q.tokens.data(), (int64_t)q.tokens.size(), &cached) == FE_OK, "probe");
        CHECK(cached % page == 0 && cached < (int64_t)q.tokens.size(), "probe covered %lld of %zu tokens",
              (long long)cached, q.tokens.size());
        q.len = cached;
        q.probed = true;
        hits += cached > 0;
      }
      const int64_t prompt_left = (int64_t)q.tokens.size() - q.len;
      int r = 1;
      if (prompt_left > 0) r = (int)std::min<int64_t>(prompt_left, 1 + (int64_t)(rng() % 700));
      int ok = 0;
      CHECK(fe_blocks_ensure(blocks, q.id, q.len + r, &ok) == FE_OK, "ensure");
      if (!ok) continue;  // the pool is full: the sequence waits
      int n = 0;
      CHECK(fe_blocks_table(blocks, q.id, nullptr, 0, &n) == FE_OK, "table size");
      const size_t at = tables.size();
      tables.resize(at + (size_t)n);
      int n2 = 0;
      CHECK(fe_blocks_table(blocks, q.id, tables.data() + at, n, &n2) == FE_OK && n2 == n, "table");
      start.push_back(q.len);
      rows.push_back(r);
      table_off.push_back((int32_t)tables.size());
      in_step.push_back(k);
    }
    std::unordered_map<int32_t, int> holders;  // page -> live tables holding it
    for (const Seq& q : live) {
      int n = 0;
      fe_blocks_table(blocks, q.id, nullptr, 0, &n);
      std::vector<int32_t> t((size_t)n);
      fe_blocks_table(blocks, q.id, t.data(), n, &n);
      for (int32_t id : t) ++holders[id];
    }
    CHECK((int64_t)holders.size() == fe_blocks_used(blocks) &&
              fe_blocks_free_pages(blocks) == pool - (int64_t)holders.size(),
          "allocator: %zu pages in tables, %lld used, %lld free", holders.size(), (long long)fe_blocks_used(blocks),
          (long long)fe_blocks_free_pages(blocks));
    const int n_seqs = (int)start.size();
    const int count = n_seqs + (rng() % 3 == 0 ? (int)(rng() % 4) : 0);  // graph padding entries
    if (count == 0) continue;
    int n_rows = 0, n_pages = 0;
    CHECK(fe_prepare_metadata(n_seqs, start.data(), rows.data(), table_off.data(), tables.data(), count, 1, page,
                              1 << 20, pool, nullptr, nullptr, 0, nullptr, nullptr, nullptr, 0, nullptr, &n_rows,
                              &n_pages) == FE_OK,
          "metadata size");
    Batch b;
    std::vector<int64_t> pos((size_t)n_rows), slots((size_t)n_rows);
    b.qo.resize((size_t)count + 1);
    b.kv.resize((size_t)count + 1);
    b.pages.resize((size_t)n_pages);
    b.last.resize((size_t)count);
    CHECK(fe_prepare_metadata(n_seqs, start.data(), rows.data(), table_off.data(), tables.data(), count, 1, page,
                              1 << 20, pool, pos.data(), slots.data(), n_rows, b.qo.data(), b.kv.data(), b.pages.data(),
                              n_pages, b.last.data(), nullptr, nullptr) == FE_OK,
          "metadata");
    // each written slot lies in a page of its own sequence's table that no
    // other sequence holds (shared prefix pages are read-only)
    for (int i = 0; i < n_seqs; ++i)
      for (int j = 0; j < rows[i]; ++j) {
        const int64_t r = b.qo[i] + j;
        CHECK(pos[r] == start[i] + j, "position of row %lld", (long long)r);
        const int32_t id = tables[table_off[i] + pos[r] / page];
        CHECK(slots[r] == (int64_t)id * page + pos[r] % page, "slot of row %lld", (long long)r);
        CHECK(holders[id] == 1, "row %lld writes page %d, held by %d sequences", (long long)r, id, holders[id]);
      }
    b.hq = 32;
    b.hkv = 8;
    b.page = page;
    b.blocks = pool;  // the padding entries' dummy page
    b.max_batch = count;
    int maxp = 1;
    for (int i = 0; i < count; ++i) maxp = std::max(maxp, b.kv[i + 1] - b.kv[i]);
    b.max_pages = maxp + 1;
    b.rows = n_rows;
    const PlanShape sh = shape_of(b);
    BuiltPlan bp;
    std::string err;
    const int rc = build_plan(sh, b.qo.data(), b.kv.data(), b.pages.data(), b.last.data(), count, n_rows, bp, err);
    if (rc == FE_ECAPACITY) continue;
    CHECK(rc == FE_OK, "step %d: metadata refused by the planner: %s", step, err.c_str());
    if (!check_plan(b, sh, bp)) return false;
    ++planned;
    for (size_t i = 0; i < in_step.size(); ++i) {
      Seq& q = live[in_step[i]];
      q.len += rows[i];
      if (q.len > (int64_t)q.tokens.size()) q.tokens.push_back((int64_t)(rng() % 4));  // the decoded token
      CHECK(fe_blocks_publish(blocks, q.id, q.tokens.data(), (int64_t)q.tokens.size(), q.len) == FE_OK, "publish");
    }
  }
  fe_prefix_stats st{};
  CHECK(fe_blocks_prefix_stats(blocks, &st) == FE_OK && st.hit_requests > 0 && st.evictions > 0,
        "prefix cache unexercised: %lld hits, %lld evictions", (long long)st.hit_requests, (long long)st.evictions);
  printf("prefix cache: %lld of %lld requests hit, %lld pages reused, %lld published, %lld evicted\n",
         (long long)st.hit_requests, (long long)st.requests, (long long)st.cached_blocks, (long long)st.new_blocks,
         (long long)st.evictions);
  fe_blocks_destroy(blocks);
  return true;
}

}  // namespace

int main(int argc, char** argv) {
  const int n = argc > 1 ? atoi(argv[1]) : 400;
  std::mt19937 rng(12345);
  int planned = 0, refused = 0;
  for (int i = 0; i < n && g_fail == 0; ++i) {
    const Batch b = random_batch(rng);
    const PlanShape sh = shape_of(b);
    BuiltPlan bp;
    std::string err;
    const int rc = build_plan(sh, b.qo.data(), b.kv.data(), b.pages.data(), b.last.data(), b.batch(), b.rows, bp, err);
    if (rc == FE_ECAPACITY) continue;  // a batch beyond the workspace: refused, nothing to check
    if (rc != FE_OK) {
      fprintf(stderr, "case %d: valid batch refused (%d): %s\n", i, rc, err.c_str());
      return 1;
    }
    if (!check_plan(b, sh, bp)) {
      fprintf(stderr, "case %d (hq %d hkv %d page %d batch %d)\n", i, b.hq, b.hkv, b.page, b.batch());
      return 1;
    }
    ++planned;
    if (!check_refused(b, rng)) return 1;
    ++refused;
  }
  if (g_fail) return 1;
  const int steps = argc > 2 ? atoi(argv[2]) : 300;
  int served = 0;
  if (!serve(rng, steps, served)) return 1;
  printf("ok: %d batches planned and checked, %d corruptions refused, %d of %d serving steps planned\n", planned,
         refused, served, steps);
  return 0;
}
