// Host side of the attention path (C ABI declared in include/fe_driver.h):
// graph batch buckets, the FIFO KV page allocator with its prefix cache and
// the per-step metadata builder of FlashEngine.cpp's model runner.  Pure host code.
#include "fe_driver.h"

#include <algorithm>
#include <deque>
#include <memory>
#include <new>
#include <string>
#include <unordered_map>
#include <vector>

#include "fe_attn.h"

namespace feattn {
int report_error(int code, const std::string& msg);
}  // namespace feattn

using feattn::report_error;

// Reference src/common.cpp:45-51.
extern "C" int fe_graph_buckets(int64_t maximum, int64_t* out, int cap, int* n_out) {
  if (maximum <= 0) return report_error(FE_EINVAL, "graph bucket maximum must be positive");
  if (n_out == nullptr) return report_error(FE_EINVAL, "n_out is null");
  std::vector<int64_t> b;
  for (int64_t n : {1, 2, 4, 8})
    if (n <= maximum) b.push_back(n);
  for (int64_t n = 16; n <= maximum; n += 16) b.push_back(n);
  if (b.empty() || b.back() != maximum) b.push_back(maximum);
  *n_out = (int)b.size();
  if (out != nullptr) std::copy(b.begin(), b.begin() + std::min<size_t>(b.size(), (size_t)std::max(cap, 0)), out);
  return FE_OK;
}

// Reference src/scheduler.cpp:5-36 (BlockManager).
//
// Free queue: FIFO order as in the reference, but a page that probe takes
// out of the middle of the queue is not searched for: each queue entry
// carries the page's free generation at the time it was queued, and an entry
// whose page is no longer free, or was queued again since, is skipped when it
// reaches the front.  The surviving order is the reference's erase +
// push_back order.
//
// Prefix cache: the reference keys published pages by their whole token
// prefix.  Here a prefix is a node of a trie of block_size-token blocks (its
// parent is the prefix one block shorter), found through a hash of (parent,
// block) and confirmed by comparing the block's tokens, so lookups are exact
// and no prefix is stored more than once.  A node lives while it caches a
// page or has a child: a prefix whose page was evicted stays reachable for
// its longer cached prefixes, as the reference's map keeps them.
namespace {

struct SeqState {
  std::vector<int32_t> table;
  int64_t cached = 0;
  bool probed = false, counted = false, hit_counted = false;
  bool idle() const { return table.empty() && cached == 0 && !probed && !counted && !hit_counted; }
};

struct PrefixNode {
  int32_t parent = -1;  // -1: the empty prefix
  int32_t page = -1;    // page caching this prefix, or -1
  int32_t children = 0;
  uint64_t hash = 0;
  std::vector<int64_t> block;  // the prefix's last block_size tokens
};

uint64_t mix64(uint64_t x) {
  x ^= x >> 30;
  x *= 0xbf58476d1ce4e5b9ull;
  x ^= x >> 27;
  x *= 0x94d049bb133111ebull;
  return x ^ (x >> 31);
}

}  // namespace

struct fe_blocks {
  int64_t block_size = 0;
  bool caching = false;
  std::deque<std::pair<int32_t, uint32_t>> queue;  // (page, free generation)
  std::vector<uint32_t> free_gen;
  std::vector<uint8_t> is_free;
  int64_t n_free = 0;
  std::vector<uint32_t> refs;  // sequences holding each page
  int64_t n_used = 0;
  std::unordered_map<int64_t, SeqState> seqs;
  std::vector<PrefixNode> nodes;
  std::vector<int32_t> spare_nodes;
  std::unordered_multimap<uint64_t, int32_t> children;  // hash(parent, block) -> node
  std::vector<int32_t> page_node;                       // node a page caches, or -1
  int64_t resident = 0;
  int64_t requests = 0, hits = 0, hit_blocks = 0, new_blocks = 0, evictions = 0;
  fe_prefix_ready_fn ready = nullptr;
  fe_prefix_evict_fn evict = nullptr;
  void* user = nullptr;

  uint64_t block_hash(int32_t parent, const int64_t* tokens) const {
    uint64_t h = mix64((uint64_t)(int64_t)parent + 0x9e3779b97f4a7c15ull);
    for (int64_t i = 0; i < block_size; ++i) h = mix64(h ^ (uint64_t)tokens[i]);
    return h;
  }
  int32_t find_child(int32_t parent, const int64_t* tokens) const {
    const auto range = children.equal_range(block_hash(parent, tokens));
    for (auto it = range.first; it != range.second; ++it) {
      const PrefixNode& n = nodes[it->second];
      if (n.parent == parent && std::equal(n.block.begin(), n.block.end(), tokens)) return it->second;
    }
    return -1;
  }
  int32_t add_child(int32_t parent, const int64_t* tokens) {
    int32_t id;
    if (!spare_nodes.empty()) {
      id = spare_nodes.back();
      spare_nodes.pop_back();
    } else {
      if (nodes.size() >= (size_t)INT32_MAX) throw std::bad_alloc();
      id = (int32_t)nodes.size();
      nodes.emplace_back();
    }
    PrefixNode& n = nodes[id];
    n.parent = parent;
    n.page = -1;
    n.children = 0;
    n.hash = block_hash(parent, tokens);
    n.block.assign(tokens, tokens + block_size);
    children.emplace(n.hash, id);
    if (parent >= 0) ++nodes[parent].children;
    return id;
  }
  // Removes `id` and then its ancestors while they cache no page and have no
  // child left.
  void prune(int32_t id) {
    while (id >= 0 && nodes[id].page < 0 && nodes[id].children == 0) {
      const auto range = children.equal_range(nodes[id].hash);
      for (auto it = range.first; it != range.second; ++it)
        if (it->second == id) {
          children.erase(it);
          break;
        }
      const int32_t parent = nodes[id].parent;
      nodes[id].parent = -1;
      spare_nodes.push_back(id);
      if (parent >= 0) --nodes[parent].children;
      id = parent;
    }
  }
  std::vector<int64_t> prefix_of(int32_t id) const {
    std::vector<int32_t> path;
    for (; id >= 0; id = nodes[id].parent) path.push_back(id);
    std::vector<int64_t> key;
    key.reserve(path.size() * (size_t)block_size);
    for (auto it = path.rbegin(); it != path.rend(); ++it) key.insert(key.end(), nodes[*it].block.begin(), nodes[*it].block.end());
    return key;
  }
  void evict_page(int32_t page) {
    const int32_t id = page_node[page];
    if (evict != nullptr) {
      const std::vector<int64_t> key = prefix_of(id);
      evict(user, key.data(), (int64_t)key.size(), page);
    }
    nodes[id].page = -1;
    page_node[page] = -1;
    --resident;
    ++evictions;
    prune(id);
  }

  void push_free(int32_t page) {
    is_free[page] = 1;
    queue.emplace_back(page, ++free_gen[page]);
    ++n_free;
  }
  int32_t pop_free() {  // n_free > 0
    for (;;) {
      const auto [page, gen] = queue.front();
      queue.pop_front();
      if (is_free[page] && gen == free_gen[page]) {
        is_free[page] = 0;
        --n_free;
        return page;
      }
    }
  }
  void take_free(int32_t page) {  // out of the middle of the queue
    is_free[page] = 0;
    --n_free;
    if (queue.size() > 2 * (size_t)n_free + 1024) {  // drop skipped entries
      std::deque<std::pair<int32_t, uint32_t>> live;
      for (const auto& e : queue)
        if (is_free[e.first] && e.second == free_gen[e.first]) live.push_back(e);
      queue.swap(live);
    }
  }
};

extern "C" int fe_blocks_create_ex(int64_t total, int64_t block_size, int caching, fe_blocks** out) {
  try {
    if (out == nullptr) return report_error(FE_EINVAL, "out is null");
    *out = nullptr;
    if (total <= 0 || total >= INT32_MAX || block_size <= 0) return report_error(FE_EINVAL, "invalid KV page pool");
    std::unique_ptr<fe_blocks> b(new fe_blocks());
    b->block_size = block_size;
    b->caching = caching != 0;
    b->free_gen.assign((size_t)total, 0);
    b->is_free.assign((size_t)total, 1);
    b->refs.assign((size_t)total, 0);
    b->page_node.assign((size_t)total, -1);
    for (int32_t i = 0; i < (int32_t)total; ++i) b->queue.emplace_back(i, 0u);
    b->n_free = total;
    *out = b.release();
    return FE_OK;
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

extern "C" int fe_blocks_create(int64_t total, int64_t block_size, fe_blocks** out) {
  return fe_blocks_create_ex(total, block_size, 0, out);
}

extern "C" int fe_blocks_destroy(fe_blocks* b) {
  delete b;
  return FE_OK;
}

extern "C" int fe_blocks_set_prefix_hooks(fe_blocks* b, fe_prefix_ready_fn ready, fe_prefix_evict_fn evict,
                                          void* user) {
  if (b == nullptr) return report_error(FE_EINVAL, "null argument");
  b->ready = ready;
  b->evict = evict;
  b->user = user;
  return FE_OK;
}

// Reference src/scheduler.cpp:31-34.
extern "C" int fe_blocks_ensure(fe_blocks* b, int64_t seq, int64_t target, int* ok_out) {
  try {
    if (b == nullptr || ok_out == nullptr) return report_error(FE_EINVAL, "null argument");
    if (target < 0) return report_error(FE_EINVAL, "negative token target");
    auto it = b->seqs.try_emplace(seq).first;
    std::vector<int32_t>& t = it->second.table;
    const size_t needed = (size_t)((target + b->block_size - 1) / b->block_size);
    *ok_out = 1;
    if (needed <= t.size()) return FE_OK;
    if (needed - t.size() > (size_t)b->n_free) {  // all or nothing
      *ok_out = 0;
      if (it->second.idle()) b->seqs.erase(it);
      return FE_OK;
    }
    t.reserve(needed);
    while (t.size() < needed) {
      const int32_t id = b->pop_free();
      if (b->page_node[id] >= 0) b->evict_page(id);
      if (b->refs[id] != 0) return report_error(FE_EINVAL, "KV page allocated twice");
      b->refs[id] = 1;
      ++b->n_used;
      t.push_back(id);
    }
    return FE_OK;
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

// Reference src/scheduler.cpp:36.
static int release_pages(fe_blocks* b, int64_t seq, bool forget) {
  auto it = b->seqs.find(seq);
  if (it == b->seqs.end()) return FE_OK;
  SeqState& s = it->second;
  for (int32_t id : s.table) {
    if (b->refs[id] == 0) return report_error(FE_EINVAL, "KV page released twice");
    if (--b->refs[id] == 0) {
      --b->n_used;
      b->push_free(id);
    }
  }
  s.table.clear();
  s.cached = 0;
  s.probed = false;
  if (forget || s.idle()) b->seqs.erase(it);
  return FE_OK;
}

extern "C" int fe_blocks_release(fe_blocks* b, int64_t seq) {
  try {
    if (b == nullptr) return report_error(FE_EINVAL, "null argument");
    return release_pages(b, seq, false);
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

extern "C" int fe_blocks_forget(fe_blocks* b, int64_t seq) {
  try {
    if (b == nullptr) return report_error(FE_EINVAL, "null argument");
    return release_pages(b, seq, true);
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

// Reference src/scheduler.cpp:6-17.
extern "C" int fe_blocks_probe(fe_blocks* b, int64_t seq, const int64_t* tokens, int64_t n_tokens,
                               int64_t* cached_out) {
  try {
    if (b == nullptr || cached_out == nullptr || n_tokens < 0 || (tokens == nullptr && n_tokens > 0))
      return report_error(FE_EINVAL, "null or negative argument");
    *cached_out = 0;
    if (!b->caching) return FE_OK;
    auto it = b->seqs.try_emplace(seq).first;
    SeqState& s = it->second;
    if (s.probed) {
      *cached_out = s.cached;
      return FE_OK;
    }
    if (!s.table.empty() || s.cached != 0) return report_error(FE_EINVAL, "prefix probe must come before the sequence's pages are allocated");
    s.probed = true;
    if (!s.counted) {
      ++b->requests;
      s.counted = true;
    }
    int32_t node = -1;
    for (int64_t end = b->block_size; end < n_tokens; end += b->block_size) {
      const int32_t child = b->find_child(node, tokens + (end - b->block_size));
      if (child < 0) break;
      const int32_t id = b->nodes[child].page;
      if (id < 0 || (b->ready != nullptr && !b->ready(b->user, tokens, end, id))) break;
      if (b->refs[id]++ == 0) {
        b->take_free(id);
        ++b->n_used;
      }
      s.table.push_back(id);
      s.cached = end;
      ++b->hit_blocks;
      node = child;
    }
    if (s.cached != 0 && !s.hit_counted) {
      ++b->hits;
      s.hit_counted = true;
    }
    *cached_out = s.cached;
    return FE_OK;
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

// Reference src/scheduler.cpp:18-29.
extern "C" int fe_blocks_publish(fe_blocks* b, int64_t seq, const int64_t* tokens, int64_t n_tokens,
                                 int64_t computed) {
  try {
    if (b == nullptr || n_tokens < 0 || (tokens == nullptr && n_tokens > 0))
      return report_error(FE_EINVAL, "null or negative argument");
    if (!b->caching) return FE_OK;
    computed = std::max<int64_t>(0, std::min(computed, n_tokens));
    static const std::vector<int32_t> none;
    auto it = b->seqs.find(seq);
    const std::vector<int32_t>& table = it == b->seqs.end() ? none : it->second.table;
    int32_t node = -1;  // node of the prefix one block shorter than `end`
    for (int64_t end = b->block_size; end <= computed; end += b->block_size) {
      const size_t index = (size_t)((end - 1) / b->block_size);
      if (index >= table.size()) {
        b->prune(node);
        return report_error(FE_EINVAL, "publishing a KV page that is not allocated");
      }
      const int32_t id = table[index];
      const int64_t* block = tokens + (end - b->block_size);
      int32_t child = b->find_child(node, block);
      if (child < 0) child = b->add_child(node, block);
      node = child;
      if (b->ready != nullptr && !b->ready(b->user, tokens, end, id)) continue;
      if (b->nodes[node].page >= 0) continue;  // prefix already resident
      if (b->page_node[id] >= 0) {
        b->prune(node);
        return report_error(FE_EINVAL, "a published KV page cannot be published again under another prefix");
      }
      b->nodes[node].page = id;
      b->page_node[id] = node;
      ++b->resident;
      ++b->new_blocks;
    }
    b->prune(node);  // trailing prefixes that got no page
    return FE_OK;
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

extern "C" int fe_blocks_table(const fe_blocks* b, int64_t seq, int32_t* out, int cap, int* n_out) {
  if (b == nullptr || n_out == nullptr) return report_error(FE_EINVAL, "null argument");
  auto it = b->seqs.find(seq);
  if (it == b->seqs.end()) {
    *n_out = 0;
    return FE_OK;
  }
  const std::vector<int32_t>& t = it->second.table;
  *n_out = (int)t.size();
  if (out != nullptr) std::copy(t.begin(), t.begin() + std::min<size_t>(t.size(), (size_t)std::max(cap, 0)), out);
  return FE_OK;
}

extern "C" int64_t fe_blocks_used(const fe_blocks* b) { return b == nullptr ? 0 : b->n_used; }

extern "C" int64_t fe_blocks_free_pages(const fe_blocks* b) { return b == nullptr ? 0 : b->n_free; }

// Reference src/scheduler.cpp:30.
extern "C" int fe_blocks_prefix_stats(const fe_blocks* b, fe_prefix_stats* out) {
  if (b == nullptr || out == nullptr) return report_error(FE_EINVAL, "null argument");
  out->requests = b->requests;
  out->hit_requests = b->hits;
  out->cached_blocks = b->hit_blocks;
  out->new_blocks = b->new_blocks;
  out->resident_blocks = b->resident;
  out->evictions = b->evictions;
  return FE_OK;
}

// Reference src/cuda_model.cpp:131-142 (token ids are the model's, not the
// attention path's, and are not produced here).
extern "C" int fe_prepare_metadata(int n_seqs, const int64_t* start, const int32_t* rows, const int32_t* table_off,
                                   const int32_t* tables, int count, int entry_rows, int page, int64_t max_model_len,
                                   int32_t dummy_page, int64_t* positions, int64_t* slots, int rows_cap, int32_t* qo,
                                   int32_t* kv, int32_t* pages, int pages_cap, int32_t* last, int* n_rows_out,
                                   int* n_pages_out) {
  if (n_seqs < 0 || count < n_seqs) return report_error(FE_EINVAL, "count must be >= the number of sequences");
  if (page <= 0) return report_error(FE_EINVAL, "page size must be positive");
  if (count > n_seqs && entry_rows <= 0) return report_error(FE_EINVAL, "padding entries need entry_rows > 0");
  if (n_seqs > 0 && (start == nullptr || rows == nullptr || table_off == nullptr))
    return report_error(FE_EINVAL, "null sequence arrays");
  // Sizes and validation first: nothing is written on failure.
  int64_t n_rows = 0, n_pages = 0;
  for (int i = 0; i < n_seqs; ++i) {
    if (rows[i] < 0 || start[i] < 0) return report_error(FE_EINVAL, "negative rows or start");
    const int64_t length = start[i] + rows[i];
    if (length > max_model_len) return report_error(FE_EINVAL, "context exceeds max_model_len");
    const int64_t have = (int64_t)table_off[i + 1] - table_off[i];
    if (rows[i] > 0 && (start[i] + rows[i] - 1) / page >= have)
      return report_error(FE_EINVAL, "page table does not cover the write slot");
    const int64_t n = (length + page - 1) / page;
    if (n > have) return report_error(FE_EINVAL, "page table does not cover the context");
    n_rows += rows[i];
    n_pages += n;
  }
  n_rows += (int64_t)(count - n_seqs) * entry_rows;
  n_pages += count - n_seqs;
  if (n_rows > INT32_MAX || n_pages > INT32_MAX) return report_error(FE_ECAPACITY, "metadata too large");
  if (n_rows_out) *n_rows_out = (int)n_rows;
  if (n_pages_out) *n_pages_out = (int)n_pages;
  if (positions == nullptr && slots == nullptr && qo == nullptr && kv == nullptr && pages == nullptr &&
      last == nullptr)
    return FE_OK;  // size query
  if (positions == nullptr || slots == nullptr || qo == nullptr || kv == nullptr || pages == nullptr ||
      last == nullptr)
    return report_error(FE_EINVAL, "null output array");
  if (n_rows > rows_cap || n_pages > pages_cap) return report_error(FE_ECAPACITY, "output arrays too small");

  int64_t r = 0, pg = 0;
  qo[0] = 0;
  kv[0] = 0;
  for (int i = 0; i < count; ++i) {
    if (i < n_seqs) {
      const int32_t* tab = tables + table_off[i];
      for (int j = 0; j < rows[i]; ++j) {
        const int64_t pos = start[i] + j;
        positions[r] = pos;
        slots[r] = (int64_t)tab[pos / page] * page + pos % page;
        ++r;
      }
      const int64_t length = start[i] + rows[i];
      const int64_t n = (length + page - 1) / page;
      for (int64_t k = 0; k < n; ++k) pages[pg++] = tab[k];
      qo[i + 1] = qo[i] + rows[i];
      kv[i + 1] = (int32_t)pg;
      last[i] = (int32_t)((length - 1) % page + 1);
    } else {
      for (int j = 0; j < entry_rows; ++j) {
        positions[r] = j;
        slots[r] = -1;
        ++r;
      }
      pages[pg++] = dummy_page;
      qo[i + 1] = qo[i] + entry_rows;
      kv[i + 1] = (int32_t)pg;
      last[i] = entry_rows;
    }
  }
  return FE_OK;
}
