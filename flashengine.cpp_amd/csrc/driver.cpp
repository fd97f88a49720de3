// Host side of the attention path (C ABI declared in include/fe_driver.h):
// graph batch buckets, the FIFO KV page allocator and the per-step metadata
// builder of FlashEngine.cpp's model runner.  Pure host code.
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

// Reference src/scheduler.cpp:5 (constructor), :31 (ensure), :35 (release).
struct fe_blocks {
  int64_t block_size = 0;
  std::deque<int32_t> free;
  std::vector<uint8_t> used;  // per page: allocated to some sequence
  int64_t n_used = 0;
  std::unordered_map<int64_t, std::vector<int32_t>> tables;
};

extern "C" int fe_blocks_create(int64_t total, int64_t block_size, fe_blocks** out) {
  try {
    if (out == nullptr) return report_error(FE_EINVAL, "out is null");
    *out = nullptr;
    if (total <= 0 || total >= INT32_MAX || block_size <= 0) return report_error(FE_EINVAL, "invalid KV page pool");
    std::unique_ptr<fe_blocks> b(new fe_blocks());
    b->block_size = block_size;
    b->used.assign((size_t)total, 0);
    for (int32_t i = 0; i < (int32_t)total; ++i) b->free.push_back(i);
    *out = b.release();
    return FE_OK;
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

extern "C" int fe_blocks_destroy(fe_blocks* b) {
  delete b;
  return FE_OK;
}

extern "C" int fe_blocks_ensure(fe_blocks* b, int64_t seq, int64_t target, int* ok_out) {
  try {
    if (b == nullptr || ok_out == nullptr) return report_error(FE_EINVAL, "null argument");
    if (target < 0) return report_error(FE_EINVAL, "negative token target");
    std::vector<int32_t>& t = b->tables[seq];
    const size_t needed = (size_t)((target + b->block_size - 1) / b->block_size);
    *ok_out = 1;
    if (needed <= t.size()) return FE_OK;
    if (needed - t.size() > b->free.size()) {  // all or nothing
      *ok_out = 0;
      if (t.empty()) b->tables.erase(seq);
      return FE_OK;
    }
    while (t.size() < needed) {
      const int32_t id = b->free.front();
      b->free.pop_front();
      if (b->used[id]) return report_error(FE_EINVAL, "KV page allocated twice");
      b->used[id] = 1;
      ++b->n_used;
      t.push_back(id);
    }
    return FE_OK;
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

extern "C" int fe_blocks_release(fe_blocks* b, int64_t seq) {
  try {
    if (b == nullptr) return report_error(FE_EINVAL, "null argument");
    auto it = b->tables.find(seq);
    if (it == b->tables.end()) return FE_OK;
    for (int32_t id : it->second) {
      if (!b->used[id]) return report_error(FE_EINVAL, "KV page released twice");
      b->used[id] = 0;
      --b->n_used;
      b->free.push_back(id);
    }
    b->tables.erase(it);
    return FE_OK;
  } catch (const std::bad_alloc&) {
    return report_error(FE_ENOMEM, "out of host memory");
  }
}

extern "C" int fe_blocks_table(const fe_blocks* b, int64_t seq, int32_t* out, int cap, int* n_out) {
  if (b == nullptr || n_out == nullptr) return report_error(FE_EINVAL, "null argument");
  auto it = b->tables.find(seq);
  if (it == b->tables.end()) {
    *n_out = 0;
    return FE_OK;
  }
  *n_out = (int)it->second.size();
  if (out != nullptr)
    std::copy(it->second.begin(), it->second.begin() + std::min<size_t>(it->second.size(), (size_t)std::max(cap, 0)),
              out);
  return FE_OK;
}

extern "C" int64_t fe_blocks_used(const fe_blocks* b) { return b == nullptr ? 0 : b->n_used; }

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
