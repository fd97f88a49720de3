// C ABI of the MI355X attention path (declared in include/fe_attn.h).
//
// The plan owns one device arena (sequence table, page table, work lists,
// counts) plus the split-KV partial buffers, all allocated once at create
// time from the capacity arguments, like the reference's FlashInfer plan
// (src/flashinfer_attention.cu:14-27).  prepare() builds the work lists on
// the host into a pinned mirror of the arena and stages them with one copy
// on the caller's stream; run() only launches kernels, whose grids depend on
// the plan capacity in graph mode, so a captured graph stays valid across
// prepares.
#include "fe_attn.h"
#include "fe_driver.h"
#include "fe_ops.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstring>
#include <new>
#include <string>
#include <vector>

#include "attn_types.hpp"
#include "planner.hpp"

namespace feattn {
hipError_t launch_decode(const AttnArgs& a, bool bf16, int waves, int ncb, int causal, int grid, hipStream_t st);
int decode_wg_waves(int hkv);
hipError_t launch_tile(const AttnArgs& a, bool bf16, bool causal, bool stream, int grid, hipStream_t st);
hipError_t launch_merge(const MergeArgs& a, bool bf16, int grid, hipStream_t st);
hipError_t launch_stage_copy(void* dst, const void* src, size_t bytes, hipStream_t st);
hipError_t launch_rope(void* q, void* k, const int64_t* pos, const float* cache, int rows, int hq, int hkv, int dim,
                       bool bf16, int max_pos, hipStream_t st);
hipError_t launch_store(const void* k, const void* v, void* kc, void* vc, const int64_t* slots, int rows, int width,
                        int64_t cache_slots, hipStream_t st);
hipError_t launch_rope_table(float* table, int max_len, int dim, float theta, hipStream_t st);
hipError_t launch_norm(const void* x, const void* res, const void* w, void* out, void* new_res, int rows, int width,
                       float eps, bool bf16, hipStream_t st);
hipError_t launch_norm_rope_append(const void* qkv, int64_t row_stride, const void* qw, const void* kw, float eps,
                                   void* q_out, void* kc, void* vc, const int64_t* pos, const int64_t* slots,
                                   const float* cache, int rows, int hq, int hkv, bool bf16, int max_pos,
                                   int64_t cache_slots, hipStream_t st);
hipError_t launch_silu_mul(const void* gu, void* out, int rows, int width, bool bf16, hipStream_t st);
hipError_t launch_accept(const int64_t* draft, const int64_t* verify, int64_t* out, int batch, int k,
                         hipStream_t st);
hipError_t launch_rope_append(void* q, const void* k, const void* v, void* kc, void* vc, const int64_t* pos,
                              const int64_t* slots, const float* cache, int rows, int hq, int hkv, int dim, bool bf16,
                              int max_pos, int64_t cache_slots, hipStream_t st);
}  // namespace feattn

using namespace feattn;

namespace {

thread_local std::string g_error;

int fail(int code, const std::string& msg) {
  g_error = msg;
  return code;
}

int hip_fail(hipError_t e, const char* what) {
  return fail(FE_EDEVICE, std::string(what) + ": " + hipGetErrorString(e));
}

size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

// Decode share records: one per share the planner may cut (decode_waves / hkv).
int share_cap(const PlanShape& sh) { return std::max(1, sh.decode_waves / sh.hkv); }

// Split-KV slot budget: as many (row, all heads) partial slots as 64 MiB of
// fp32 rows would hold; the rows are stored in 16 bits, so they take half.
constexpr size_t kPartialBytes = 64u << 20;

int partial_cap_for(int hq) {
  return hq > 0 ? (int)std::max<size_t>(1024, kPartialBytes / ((size_t)hq * (kHeadDim + 1) * sizeof(float))) : 1024;
}

// A metadata arena is
//   [header | seqs | tshare[0] | tshare[1] | shares | heap ......]
// The first five regions have fixed sizes.  The heap holds the lists whose
// lengths vary from prepare to prepare (page table, decode pieces, tile
// items and merge records of both masks), packed one after another; every
// index a kernel follows into them (a share's item range, page_off, tile
// offsets, the header's tile ends and merge bases) is stored relative to
// the heap start.  So one prepare stages the arena with a single copy of
// [0, end of the heap's used part) (each small host-to-device copy costs
// several microseconds on the stream), and the region pointers of a
// captured launch stay valid.
//
// Record counts of the fixed regions and bytes of the heap.  A plan sizes
// them from its capacity, the one-shot entry from the call's own lists (a
// mode with no tshare records is not staged).
struct Regions {
  size_t seqs, tshare[2], shares, heap;
};

struct Layout {
  Regions n;
  size_t header, seqs, tshare[2], shares, heap, total;  // byte offsets
};

Layout make_layout(const Regions& r) {
  Layout l;
  l.n = r;
  size_t off = 0;
  l.header = off;
  off = align256(off + sizeof(int32_t) * 16);
  l.seqs = off;
  off = align256(off + sizeof(SeqInfo) * r.seqs);
  for (int m = 0; m < 2; ++m) {
    l.tshare[m] = off;
    off = align256(off + sizeof(int32_t) * r.tshare[m]);
  }
  l.shares = off;
  off = align256(off + sizeof(ShareStart) * r.shares);
  l.heap = off;
  off = align256(off + r.heap);
  l.total = off;
  return l;
}

// Byte offsets of the lists inside the heap (each 256-byte aligned, so a
// list's first record index is its offset over the record size).
struct HeapPlace {
  size_t pages, decode, tile[2], merge[2], used;
};

HeapPlace place_heap(size_t pages, size_t decode, const size_t tile[2], const size_t merge[2]) {
  HeapPlace p;
  size_t off = 0;
  auto put = [&](size_t bytes) {
    const size_t at = off;
    off = align256(off + bytes);
    return at;
  };
  p.pages = put(sizeof(int32_t) * pages);
  p.decode = put(sizeof(DecodeItem) * decode);
  for (int m = 0; m < 2; ++m) p.tile[m] = put(sizeof(WorkItem) * tile[m]);
  for (int m = 0; m < 2; ++m) p.merge[m] = put(sizeof(MergeRow) * merge[m]);
  p.used = off;
  return p;
}

// Places the lists of `bp` for the staged mask modes.
HeapPlace place_lists(const BuiltPlan& bp, int npages, const bool staged[2]) {
  size_t tile[2], merge[2];
  for (int m = 0; m < 2; ++m) {
    tile[m] = staged[m] ? bp.mode[m].tile.size() : 0;
    merge[m] = staged[m] ? bp.mode[m].merge.size() : 0;
  }
  return place_heap((size_t)npages, bp.decode_items.size(), tile, merge);
}

Regions capacity_regions(const PlanShape& sh) {
  Regions r;
  r.seqs = (size_t)sh.max_batch;
  r.shares = (size_t)share_cap(sh);
  const size_t tile[2] = {(size_t)sh.item_cap, (size_t)sh.item_cap};
  const size_t merge[2] = {(size_t)sh.partial_cap, (size_t)sh.partial_cap};
  for (int m = 0; m < 2; ++m) r.tshare[m] = (size_t)sh.tile_slots + 1;
  r.heap = place_heap((size_t)sh.max_batch * sh.max_pages, (size_t)sh.item_cap, tile, merge).used;
  return r;
}

// header[] indices.  Tile ends are heap indices (a workgroup's items end at
// min(tile_off[b + 1], end)); each merge count is followed by its base.
enum {
  kHdrDecodeShares = 0,
  kHdrTileEnd0 = 2,
  kHdrTileEnd1 = 3,
  kHdrMerge0 = 4,  // count, base
  kHdrMerge1 = 6,  // count, base
};

// Validated shape (host-only sizes).
int make_shape(int hq, int hkv, int dim, int page, int max_batch, int max_pages, int blocks, PlanShape& sh,
               std::string& err) {
  sh.hq = hq;
  sh.hkv = hkv;
  sh.dim = dim;
  sh.page = page;
  sh.max_batch = max_batch;
  sh.max_pages = max_pages;
  sh.blocks = blocks;
  if (validate_shape(sh, err) != FE_OK) return FE_EINVAL;
  sh.partial_cap = partial_cap_for(hq);
  return FE_OK;
}

// Launch sizes of `device`: the work a grid of resident workgroups covers.
int device_sizes(PlanShape& sh, int device, std::string& err) {
  int cus = 0;
  const hipError_t e = hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, device);
  if (e != hipSuccess) {
    err = std::string("hipDeviceGetAttribute: ") + hipGetErrorString(e);
    return FE_EDEVICE;
  }
  sh.num_cus = cus > 0 ? cus : 256;
  sh.decode_waves = sh.num_cus * kDecodeWavesPerCu;
  sh.tile_slots = sh.num_cus * 2;  // 2 resident 256-thread tile workgroups per CU
  return FE_OK;
}

// Writes the lists of `bp` into the host image `h` of the arena layout `l`,
// the heap lists at `hp`, every heap index shifted by its list's start.
// Returns the bytes to copy (the image up to the end of the heap's used
// part) in `bytes`.
int write_image(uint8_t* h, const Layout& l, const HeapPlace& hp, const PlanShape& sh, const BuiltPlan& bp,
                const int32_t* pages, int npages, size_t& bytes, std::string& err) {
  const int n_shares = (int)bp.decode_starts.size();
  const int scap = (int)l.n.shares;
  if (n_shares > scap) {
    err = "attention metadata exceeds capacity: decode shares";
    return FE_ECAPACITY;
  }
  if (bp.seqs.size() > l.n.seqs || hp.used > l.n.heap) {
    err = "attention metadata exceeds capacity: work lists";
    return FE_ECAPACITY;
  }
  uint8_t* heap = h + l.heap;
  const int32_t pages_base = (int32_t)(hp.pages / sizeof(int32_t));
  const int32_t decode_base = (int32_t)(hp.decode / sizeof(DecodeItem));

  int32_t* hdr = reinterpret_cast<int32_t*>(h + l.header);
  std::memset(hdr, 0, sizeof(int32_t) * 16);
  hdr[kHdrDecodeShares] = n_shares;

  SeqInfo* seqs = reinterpret_cast<SeqInfo*>(h + l.seqs);
  for (size_t b = 0; b < bp.seqs.size(); ++b) {
    seqs[b] = bp.seqs[b];
    seqs[b].page_off += pages_base;
  }
  if (npages > 0) std::memcpy(heap + hp.pages, pages, sizeof(int32_t) * npages);

  auto shift_piece = [&](DecodeItem d) {
    d.page_off += pages_base;
    return d;
  };
  DecodeItem* items = reinterpret_cast<DecodeItem*>(heap + hp.decode);
  for (size_t i = 0; i < bp.decode_items.size(); ++i) items[i] = shift_piece(bp.decode_items[i]);
  // Every share record up to the capacity is written: a graph launch covers
  // them all, and records past the shares in use must read as empty.
  ShareStart* ss = reinterpret_cast<ShareStart*>(h + l.shares);
  for (int k = 0; k < n_shares; ++k) {
    ss[k] = bp.decode_starts[k];
    ss[k].it_begin += decode_base;
    ss[k].it_end += decode_base;
    ss[k].first = shift_piece(ss[k].first);
  }
  std::memset(ss + n_shares, 0, sizeof(ShareStart) * (size_t)(scap - n_shares));

  const int tslots = sh.tile_slots;
  for (int m = 0; m < 2; ++m) {
    if (l.n.tshare[m] == 0) continue;  // mode not staged
    const int32_t tile_base = (int32_t)(hp.tile[m] / sizeof(WorkItem));
    const int32_t n_tile = (int32_t)bp.mode[m].tile.size();
    const size_t n_merge = bp.mode[m].merge.size();
    hdr[m ? kHdrTileEnd1 : kHdrTileEnd0] = tile_base + n_tile;
    hdr[(m ? kHdrMerge1 : kHdrMerge0) + 0] = (int32_t)n_merge;
    hdr[(m ? kHdrMerge1 : kHdrMerge0) + 1] = (int32_t)(hp.merge[m] / sizeof(MergeRow));
    if (n_tile > 0) std::memcpy(heap + hp.tile[m], bp.mode[m].tile.data(), sizeof(WorkItem) * n_tile);
    if (n_merge > 0) std::memcpy(heap + hp.merge[m], bp.mode[m].merge.data(), sizeof(MergeRow) * n_merge);
    // share offsets up to the launch capacity: shares past those in use are
    // empty (a graph launch covers every slot)
    const std::vector<int32_t>& off = bp.mode[m].tile_off;
    const int used = off.empty() ? 0 : (int)off.size() - 1;
    if (used > tslots) {
      err = "attention metadata exceeds capacity: tile shares";
      return FE_ECAPACITY;
    }
    int32_t* dst = reinterpret_cast<int32_t*>(h + l.tshare[m]);
    for (int k = 0; k <= tslots; ++k) dst[k] = tile_base + (k <= used && !off.empty() ? off[k] : n_tile);
  }
  bytes = l.heap + hp.used;
  return FE_OK;
}

// What the kernels of one prepared plan are launched from.
struct Launch {
  PlanShape sh;
  Layout lay{};
  const uint8_t* dev = nullptr;  // metadata arena on the device
  uint16_t* part_o = nullptr;    // 16-bit split-KV partial rows
  float* part_lse = nullptr;
  bool bf16 = true;
  bool graph = false;
  int graph_tile = -1;  // graph plans: the first graph prepare had tile work (1) or not (0)
  bool tile_stream[2] = {true, true};  // tile K/V reads with the non-temporal hint, per mask mode
  int graph_stream[2] = {-1, -1};      // graph plans: that choice at the first graph prepare
  int n_decode = 0, n_tile[2] = {0, 0}, n_merge[2] = {0, 0};
  size_t merge_off[2] = {0, 0};  // heap offsets of the merge lists just staged
  int n_tshare[2] = {0, 0};  // tile shares (workgroups) in use per mask mode
  int decode_wg = 8;         // wavefronts per decode workgroup
  int decode_nc = 16;
  int grid_decode_cap = 0, grid_tile_cap = 0, grid_merge_cap = 0;
};

void init_launch(Launch& L, const PlanShape& sh, bool bf16) {
  L.sh = sh;
  L.bf16 = bf16;
  L.decode_wg = decode_wg_waves(sh.hkv);
  L.grid_decode_cap = sh.num_cus * kDecodeWavesPerCu / L.decode_wg;  // persistent: every workgroup resident
  L.grid_tile_cap = sh.tile_slots;
  L.grid_merge_cap = sh.num_cus * 8;  // 4 (row, head pair) units per workgroup
}

// Launch sizes of the lists just staged.
// Whether the tile lists read each K/V token once per kv head: no sequence
// with tile work is cut into several column blocks (the planner gives such a
// sequence ceil(qlen / (kTileCols / group)) blocks, every one over the same
// tokens).  Chunked prefill is cut so, and those re-reads are L2 hits with
// the default policy (the 8192-token prefill takes 0.257 ms so, 0.282 ms
// streamed); DFlash blocks and short verify rows are one block each.
bool reads_tokens_once(const BuiltPlan& bp, const PlanShape& sh) {
  const int group = sh.hq / sh.hkv;
  const int rows_per_block = kTileCols / group;
  for (const SeqInfo& s : bp.seqs)
    if (s.qlen * group > kDecodeCols && s.qlen > rows_per_block) return false;
  return true;
}

void record_lists(Launch& L, const BuiltPlan& bp, const HeapPlace& hp, int nc) {
  L.decode_nc = nc;
  for (int m = 0; m < 2; ++m) L.merge_off[m] = hp.merge[m];
  L.n_decode = (int)bp.decode_starts.size() * L.sh.hkv;  // busy decode wavefronts
  for (int m = 0; m < 2; ++m) {
    L.n_tile[m] = (int)bp.mode[m].tile.size();
    L.n_tshare[m] = bp.mode[m].tile_off.empty() ? 0 : (int)bp.mode[m].tile_off.size() - 1;
    L.n_merge[m] = (int)bp.mode[m].merge.size();
    // Graph plans keep the policy their tile launch was captured with (a
    // cache hint: results do not depend on it).
    const bool once = reads_tokens_once(bp, L.sh);
    if (L.graph && L.graph_stream[m] < 0) L.graph_stream[m] = once ? 1 : 0;
    L.tile_stream[m] = L.graph ? L.graph_stream[m] > 0 : once;
  }
}

// The work of a call runs on the device of its stream (the current device
// for the null stream); a plan's memory lives on the device it was created
// on, and the two must agree.
int check_stream_device(hipStream_t st, int device) {
  int dev = -1;
  const hipError_t e = hipStreamGetDevice(st, &dev);
  if (e != hipSuccess) return hip_fail(e, "hipStreamGetDevice");
  if (dev != device)
    return fail(FE_EDEVICE, "attention: stream on device " + std::to_string(dev) + ", plan memory on device " +
                                std::to_string(device));
  return FE_OK;
}

int check_tensors(const void* q, const void* k_cache, const void* v_cache, const void* out, const float* lse) {
  if (q == nullptr || k_cache == nullptr || v_cache == nullptr || out == nullptr)
    return fail(FE_EINVAL, "null tensor pointer");
  // The kernels move q rows and K/V cache rows in 16-byte pieces (direct
  // to LDS) and write 8-byte pieces of out.
  const void* rows16[] = {q, k_cache, v_cache, out};
  for (const void* ptr : rows16)
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0)
      return fail(FE_EINVAL, "attention: q, k_cache, v_cache and out must be 16-byte aligned");
  if (reinterpret_cast<uintptr_t>(lse) % 4 != 0) return fail(FE_EINVAL, "attention: lse must be 4-byte aligned");
  return FE_OK;
}

int launch_all(const Launch& L, const void* q, const void* k_cache, const void* v_cache, void* out, float* lse,
               int causal, hipStream_t st) {
  const int mode = causal ? 1 : 0;
  const int32_t* hdr = reinterpret_cast<const int32_t*>(L.dev + L.lay.header);
  const uint8_t* heap = L.dev + L.lay.heap;
  AttnArgs a{};
  a.q = static_cast<const uint16_t*>(q);
  a.kc = static_cast<const uint16_t*>(k_cache);
  a.vc = static_cast<const uint16_t*>(v_cache);
  a.out = static_cast<uint16_t*>(out);
  a.lse = lse;
  a.seqs = reinterpret_cast<const SeqInfo*>(L.dev + L.lay.seqs);
  a.pages = reinterpret_cast<const int32_t*>(heap);
  a.part_o = L.part_o;
  a.part_lse = L.part_lse;
  a.hq = L.sh.hq;
  a.hkv = L.sh.hkv;
  a.group = L.sh.hq / L.sh.hkv;
  int shift = 0;
  while ((1 << shift) < L.sh.page) ++shift;
  a.page_shift = shift;
  a.scale_log2 = 1.4426950408889634f / 11.313708498984761f;  // log2(e) / sqrt(128)
  hipError_t e;
  if (L.graph || L.n_decode > 0) {
    AttnArgs d = a;
    d.ditems = reinterpret_cast<const DecodeItem*>(heap);
    d.shares = reinterpret_cast<const ShareStart*>(L.dev + L.lay.shares);
    d.n_share_cap = (int)L.lay.n.shares;
    const int wv = L.decode_wg;
    const int grid = L.graph ? L.grid_decode_cap : std::min(L.grid_decode_cap, (L.n_decode + wv - 1) / wv);
    e = launch_decode(d, L.bf16, L.decode_wg, L.decode_nc / 16, causal ? 1 : 0, std::max(grid, 1), st);
    if (e != hipSuccess) return hip_fail(e, "decode kernel launch");
  }
  if (L.graph ? L.graph_tile > 0 : L.n_tile[mode] > 0) {
    AttnArgs t = a;
    t.items = reinterpret_cast<const WorkItem*>(heap);
    t.n_items = hdr + (mode ? kHdrTileEnd1 : kHdrTileEnd0);
    t.tile_off = reinterpret_cast<const int32_t*>(L.dev + L.lay.tshare[mode]);
    const int grid = L.graph ? L.grid_tile_cap : L.n_tshare[mode];
    e = launch_tile(t, L.bf16, causal != 0, L.tile_stream[mode], std::max(grid, 1), st);
    if (e != hipSuccess) return hip_fail(e, "tile kernel launch");
  }
  if (L.graph || L.n_merge[mode] > 0) {
    MergeArgs m{};
    m.out = static_cast<uint16_t*>(out);
    m.lse = lse;
    if (L.graph) {
      m.rows = reinterpret_cast<const MergeRow*>(heap);
      m.count_base = hdr + (mode ? kHdrMerge1 : kHdrMerge0);
    } else {
      m.rows = reinterpret_cast<const MergeRow*>(heap + L.merge_off[mode]);
      m.n_rows = L.n_merge[mode];
    }
    m.part_o = L.part_o;
    m.part_lse = L.part_lse;
    m.hq = L.sh.hq;
    const int pairs4 = (int)(((int64_t)L.n_merge[mode] * ((L.sh.hq + 1) / 2) + 3) / 4);
    const int grid = L.graph ? L.grid_merge_cap : std::min(L.grid_merge_cap, pairs4);
    e = launch_merge(m, L.bf16, std::max(grid, 1), st);
    if (e != hipSuccess) return hip_fail(e, "merge kernel launch");
  }
  return FE_OK;
}

}  // namespace

namespace feattn {
// Shared with the host driver (driver.cpp): sets the message returned by
// fe_attn_last_error() on this thread and returns `code`.
int report_error(int code, const std::string& msg) { return fail(code, msg); }

// One-shot attention whose metadata arena and split-KV partials are carved
// out of `arena` (`bytes` of device memory on `device`): plans exactly as
// fe_attn_plan_prepare does for a plan of the same heads, page and blocks
// (so the results are identical), stages the metadata with one copy on `st`
// and launches as fe_attn_run does.  Allocates no device or pinned memory.
int attn_oneshot(uint8_t* arena, size_t bytes, int device, const void* q, const void* k_cache, const void* v_cache,
                 void* out, float* lse, int causal, const int32_t* qo, const int32_t* kv, const int32_t* pages,
                 const int32_t* last, int batch, int rows, int hq, int hkv, int dim, int page, int blocks, int bf16,
                 hipStream_t st) {
  // A capture would record the metadata copy below with a source in host
  // memory that is released when this call returns: a replay would then
  // read freed memory as work lists and page ids.  Refused before anything
  // is enqueued.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  hipError_t ce = hipStreamIsCapturing(st, &cap);
  if (ce != hipSuccess) return hip_fail(ce, "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(FE_EINVAL, "attention (no-alloc): the stream is capturing a graph; capture the plan entry "
                           "points (fe_attn_plan_prepare outside the capture, fe_attn_run inside) instead");
  if (batch < 0) return fail(FE_EINVAL, "batch must be non-negative");
  if (batch > 0 && kv == nullptr) return fail(FE_EINVAL, "null metadata pointer");
  // Capacity from the call itself: every sequence fits (the planner checks
  // len <= (max_pages - 1) * page) and so does the page table
  // (kv[batch] <= batch * max_pages).
  int64_t most = 1;
  for (int b = 0; b < batch; ++b) most = std::max<int64_t>(most, (int64_t)kv[b + 1] - kv[b]);
  most += 1;
  if (batch > 0) most = std::max<int64_t>(most, ((int64_t)kv[batch] + batch - 1) / batch);
  const int max_pages = (int)std::min<int64_t>(most, INT32_MAX / 2);
  PlanShape sh;
  std::string err;
  int rc = make_shape(hq, hkv, dim, page, std::max(batch, 1), max_pages, blocks, sh, err);
  if (rc == FE_OK) rc = device_sizes(sh, device, err);
  if (rc != FE_OK) return fail(rc, err);
  rc = check_tensors(q, k_cache, v_cache, out, lse);
  if (rc != FE_OK) return rc;
  rc = check_stream_device(st, device);
  if (rc != FE_OK) return rc;
  BuiltPlan bp;
  rc = build_plan(sh, qo, kv, pages, last, batch, rows, bp, err);
  if (rc != FE_OK) return fail(rc, err);
  const int mode = causal ? 1 : 0;
  const int npages = batch > 0 ? kv[batch] : 0;
  const bool staged[2] = {mode == 0, mode == 1};
  const HeapPlace hp = place_lists(bp, npages, staged);
  Regions r{};
  r.seqs = bp.seqs.size();
  r.tshare[mode] = (size_t)sh.tile_slots + 1;
  r.shares = (size_t)share_cap(sh);
  r.heap = hp.used;
  Launch L;
  init_launch(L, sh, bf16 != 0);
  L.lay = make_layout(r);
  const size_t parts = (size_t)bp.mode[mode].partial_rows * hq;
  const size_t o_off = L.lay.total;
  const size_t lse_off = align256(o_off + parts * kHeadDim * sizeof(uint16_t));
  const size_t need = lse_off + parts * sizeof(float);
  if (need > bytes)
    return fail(FE_ECAPACITY, "attention (no-alloc): this call needs " + std::to_string(need) +
                                  " bytes of device scratch, more than the " + std::to_string(bytes) + " it holds");
  // Nothing in the arena has to start at zero, whatever an earlier call
  // left there: the copy below writes every metadata field the kernels read
  // (header, share records, lists), and every partial slot a merge reads is
  // written by this call's decode or tile kernel first.
  std::vector<uint8_t> image(L.lay.total);
  size_t stage_bytes = 0;
  rc = write_image(image.data(), L.lay, hp, sh, bp, pages, npages, stage_bytes, err);
  if (rc != FE_OK) return fail(rc, err);
  // The image is pageable host memory, which HIP copies synchronously (the
  // call returns once the copy has run on `st`), so it may be released right
  // after.
  hipError_t e = hipMemcpyAsync(arena, image.data(), stage_bytes, hipMemcpyHostToDevice, st);
  if (e != hipSuccess) return hip_fail(e, "hipMemcpyAsync(attention metadata)");
  L.dev = arena;
  L.part_o = reinterpret_cast<uint16_t*>(arena + o_off);
  L.part_lse = reinterpret_cast<float*>(arena + lse_off);
  record_lists(L, bp, hp, bp.decode_nc);
  return launch_all(L, q, k_cache, v_cache, out, lse, causal, st);
}
}  // namespace feattn

struct fe_attn_plan {
  Launch run;                  // arena pointers, shape and launch sizes
  uint8_t* dev = nullptr;      // metadata arena
  uint8_t* host = nullptr;     // pinned mirror
  uint8_t* host_dev = nullptr; // its address in the device's view
  uint16_t* part_o = nullptr;  // 16-bit partial rows
  float* part_lse = nullptr;
  hipEvent_t staged = nullptr;
  bool staged_pending = false;
  int device = 0;
  bool prepared = false;
  int graph_nc = 0;  // graph plans: the decode column variant of the first graph prepare
};

extern "C" {

const char* fe_attn_last_error(void) { return g_error.c_str(); }

const char* fe_attn_version(void) { return "feattn-hip-gfx950 0.1.0"; }

int fe_attn_plan_create(int hq, int hkv, int dim, int page, int max_batch, int max_pages, int bf16, int blocks,
                        fe_attn_plan** plan_out) {
  if (plan_out == nullptr) return fail(FE_EINVAL, "plan_out is null");
  *plan_out = nullptr;
  PlanShape sh;
  std::string err;
  int rc = make_shape(hq, hkv, dim, page, max_batch, max_pages, blocks, sh, err);
  if (rc != FE_OK) return fail(rc, err);
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) return hip_fail(e, "hipGetDevice");
  rc = device_sizes(sh, dev, err);
  if (rc != FE_OK) return fail(rc, err);

  auto* p = new (std::nothrow) fe_attn_plan();
  if (p == nullptr) return fail(FE_ENOMEM, "out of host memory");
  p->device = dev;
  init_launch(p->run, sh, bf16 != 0);
  p->run.lay = make_layout(capacity_regions(sh));
  const size_t total = p->run.lay.total;
  auto cleanup = [&](int code, const std::string& msg) {
    fe_attn_plan_destroy(p);
    return fail(code, msg);
  };
  if (hipMalloc(&p->dev, total) != hipSuccess) return cleanup(FE_ENOMEM, "hipMalloc(plan metadata) failed");
  // Coherent and mapped: the staging kernel reads the mirror over the bus,
  // and no device cache may keep a previous prepare's image.
  if (hipHostMalloc(&p->host, total, hipHostMallocMapped | hipHostMallocCoherent) != hipSuccess)
    return cleanup(FE_ENOMEM, "hipHostMalloc(plan staging) failed");
  std::memset(p->host, 0, total);
  if (hipHostGetDevicePointer(reinterpret_cast<void**>(&p->host_dev), p->host, 0) != hipSuccess ||
      p->host_dev == nullptr)
    return cleanup(FE_EDEVICE, "hipHostGetDevicePointer(plan staging) failed");
  if (hipMalloc(&p->part_o, (size_t)sh.partial_cap * hq * kHeadDim * sizeof(uint16_t)) != hipSuccess)
    return cleanup(FE_ENOMEM, "hipMalloc(split-KV partials) failed");
  if (hipMalloc(&p->part_lse, (size_t)sh.partial_cap * hq * sizeof(float)) != hipSuccess)
    return cleanup(FE_ENOMEM, "hipMalloc(split-KV lse) failed");
  if (hipEventCreateWithFlags(&p->staged, hipEventDisableTiming) != hipSuccess)
    return cleanup(FE_EDEVICE, "hipEventCreate failed");
  // Counts start at zero so a run before any prepare does nothing.
  if (hipMemset(p->dev, 0, total) != hipSuccess) return cleanup(FE_EDEVICE, "hipMemset(plan) failed");
  if (hipDeviceSynchronize() != hipSuccess) return cleanup(FE_EDEVICE, "hipDeviceSynchronize failed");
  p->run.dev = p->dev;
  p->run.part_o = p->part_o;
  p->run.part_lse = p->part_lse;
  *plan_out = p;
  return FE_OK;
}

int fe_attn_plan_destroy(fe_attn_plan* p) {
  if (p == nullptr) return FE_OK;
  if (p->staged_pending) (void)hipEventSynchronize(p->staged);
  if (p->staged) (void)hipEventDestroy(p->staged);
  if (p->dev) (void)hipFree(p->dev);
  if (p->host) (void)hipHostFree(p->host);
  if (p->part_o) (void)hipFree(p->part_o);
  if (p->part_lse) (void)hipFree(p->part_lse);
  delete p;
  return FE_OK;
}

int fe_attn_plan_prepare(fe_attn_plan* p, const int32_t* qo, const int32_t* kv, const int32_t* pages,
                         const int32_t* last, int batch, int rows, int graph, void* stream) {
  if (p == nullptr) return fail(FE_EINVAL, "plan is null");
  Launch& L = p->run;
  BuiltPlan bp;
  std::string err;
  int rc = check_stream_device(static_cast<hipStream_t>(stream), p->device);
  if (rc != FE_OK) return rc;
  // A captured prepare would leave its staging kernel in the graph, reading
  // whatever the pinned image holds at each replay, and the wait on the
  // previous transfer would name an event recorded inside the capture.
  hipStreamCaptureStatus cap = hipStreamCaptureStatusNone;
  const hipError_t ce = hipStreamIsCapturing(static_cast<hipStream_t>(stream), &cap);
  if (ce != hipSuccess) return hip_fail(ce, "hipStreamIsCapturing");
  if (cap != hipStreamCaptureStatusNone)
    return fail(FE_EINVAL, "prepare_plan: the stream is capturing a graph; prepare outside the capture and "
                           "capture only the attention calls");
  rc = build_plan(L.sh, qo, kv, pages, last, batch, rows, bp, err);
  if (rc != FE_OK) return fail(rc, err);
  int nc = bp.decode_nc;
  int graph_nc = p->graph_nc, graph_tile = L.graph_tile;
  if (graph) {
    // Captured launches bake in the decode column variant; a later prepare
    // may not need a wider one (the reference refuses layout changes under
    // graph capture too: src/flashinfer_attention.cu:32).
    // (the layout is fixed by the first graph prepare that succeeds: it is
    // stored in the plan only after every check and copy below)
    if (graph_nc == 0) graph_nc = nc;
    if (nc > graph_nc)
      return fail(FE_EINVAL, "graph plan layout changed: decode rows per sequence grew after capture");
    nc = graph_nc;
    // Likewise whether the tile kernel is launched at all: a graph of
    // decode-only steps carries no tile launch, and a later prepare may not
    // bring tile work to it.
    const int tile = bp.mode[0].tile.empty() && bp.mode[1].tile.empty() ? 0 : 1;
    if (graph_tile < 0) graph_tile = tile;
    if (tile > graph_tile)
      return fail(FE_EINVAL, "graph plan layout changed: multi-row tile work after a capture without it");
  }
  hipStream_t st = static_cast<hipStream_t>(stream);
  // The pinned mirror may still be read by the previous prepare's copies.
  if (p->staged_pending) {
    hipError_t e = hipEventSynchronize(p->staged);
    if (e != hipSuccess) return hip_fail(e, "hipEventSynchronize");
    p->staged_pending = false;
  }
  const Layout& l = L.lay;
  uint8_t* h = p->host;
  const int npages = batch > 0 ? kv[batch] : 0;
  const bool staged[2] = {true, true};  // the mask is chosen at run time
  const HeapPlace hp = place_lists(bp, npages, staged);
  size_t bytes = 0;
  if (write_image(h, l, hp, L.sh, bp, pages, npages, bytes, err) != FE_OK) return fail(FE_ECAPACITY, err);
  // One transfer of the fixed regions and the used part of the heap, by a
  // kernel on `st` that reads the mirror (no copy-engine handoff).
  hipError_t e = launch_stage_copy(p->dev, p->host_dev, bytes, st);
  if (e != hipSuccess) return hip_fail(e, "plan staging kernel launch");
  e = hipEventRecord(p->staged, st);
  if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
  p->staged_pending = true;
  p->prepared = true;
  L.graph = graph != 0;
  if (graph) {
    p->graph_nc = graph_nc;
    L.graph_tile = graph_tile;
  }
  record_lists(L, bp, hp, nc);
  return FE_OK;
}

int fe_attn_run(fe_attn_plan* p, const void* q, const void* k_cache, const void* v_cache, void* out, float* lse,
                int causal, void* stream) {
  if (p == nullptr) return fail(FE_EINVAL, "plan is null");
  if (!p->prepared) return fail(FE_EINVAL, "attention called before prepare_plan");
  int rc = check_tensors(q, k_cache, v_cache, out, lse);
  if (rc != FE_OK) return rc;
  rc = check_stream_device(static_cast<hipStream_t>(stream), p->device);
  if (rc != FE_OK) return rc;
  return launch_all(p->run, q, k_cache, v_cache, out, lse, causal, static_cast<hipStream_t>(stream));
}

int fe_rope_table(float* table, int max_len, int dim, double theta, void* stream) {
  if (table == nullptr) return fail(FE_EINVAL, "rope table: null pointer");
  if (max_len <= 0 || dim <= 0 || dim % 2 != 0) return fail(FE_EINVAL, "rope table: max_len > 0 and even dim required");
  if (!(theta > 0.0)) return fail(FE_EINVAL, "rope table: theta must be positive");
  if ((int64_t)max_len * (dim / 2) > (int64_t)INT32_MAX * 128)
    return fail(FE_EINVAL, "rope table: max_len * dim / 2 exceeds the launch range");
  const hipError_t e = launch_rope_table(table, max_len, dim, (float)theta, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "rope table kernel launch");
}

int fe_rope(void* q, void* k, const int64_t* pos, const float* cache, int rows, int hq, int hkv, int dim, int bf16,
            void* stream, int max_positions) {
  if (rows < 0 || hq < 0 || hkv < 0) return fail(FE_EINVAL, "rope: negative size");
  if (dim <= 0 || dim % 16 != 0) return fail(FE_EINVAL, "rope: dim must be a positive multiple of 16");
  if (rows == 0) return FE_OK;
  if (q == nullptr || (hkv > 0 && k == nullptr) || pos == nullptr || cache == nullptr)
    return fail(FE_EINVAL, "rope: null pointer");
  if (q == k) return fail(FE_EINVAL, "rope: q and k must not alias");
  const hipError_t e = launch_rope(q, k, pos, cache, rows, hq, hkv, dim, bf16 != 0, max_positions,
                                   static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "rope kernel launch");
}

int fe_store(const void* k, const void* v, void* k_cache, void* v_cache, const int64_t* slots, int rows, int width,
             int bf16, void* stream, int cache_slots) {
  (void)bf16;  // a 16-bit copy is the same for both types
  if (rows < 0 || width < 0 || cache_slots < 0) return fail(FE_EINVAL, "store: negative size");
  if (rows == 0 || width == 0) return FE_OK;
  if (k == nullptr || v == nullptr || k_cache == nullptr || v_cache == nullptr || slots == nullptr)
    return fail(FE_EINVAL, "store: null pointer");
  const hipError_t e =
      launch_store(k, v, k_cache, v_cache, slots, rows, width, cache_slots, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "store kernel launch");
}

int fe_rope_append(void* q, const void* k, const void* v, void* k_cache, void* v_cache, const int64_t* pos,
                   const int64_t* slots, const float* cache, int rows, int hq, int hkv, int dim, int bf16,
                   int max_positions, int cache_slots, void* stream) {
  if (rows < 0 || hq < 0 || hkv < 0 || cache_slots < 0) return fail(FE_EINVAL, "rope_append: negative size");
  if (dim <= 0 || dim % 16 != 0) return fail(FE_EINVAL, "rope_append: dim must be a positive multiple of 16");
  if (rows == 0) return FE_OK;
  if (q == nullptr || k == nullptr || v == nullptr || k_cache == nullptr || v_cache == nullptr || pos == nullptr ||
      slots == nullptr || cache == nullptr)
    return fail(FE_EINVAL, "rope_append: null pointer");
  const hipError_t e = launch_rope_append(q, k, v, k_cache, v_cache, pos, slots, cache, rows, hq, hkv, dim,
                                          bf16 != 0, max_positions, cache_slots, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "rope_append kernel launch");
}

int fe_norm(const void* x, const void* residual, const void* weight, void* output, void* new_residual, int rows,
            int width, float eps, int bf16, void* stream) {
  if (rows < 0 || width <= 0) return fail(FE_EINVAL, "norm: rows >= 0 and width > 0 required");
  if (rows == 0) return FE_OK;
  if (x == nullptr || weight == nullptr || output == nullptr) return fail(FE_EINVAL, "norm: null pointer");
  const hipError_t e = launch_norm(x, residual, weight, output, new_residual, rows, width, eps, bf16 != 0,
                                   static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "norm kernel launch");
}

int fe_silu_mul(const void* gate_up, void* output, int rows, int width, int bf16, void* stream) {
  if (rows < 0 || width < 0) return fail(FE_EINVAL, "silu_mul: negative size");
  if ((int64_t)rows * width == 0) return FE_OK;
  if (gate_up == nullptr || output == nullptr) return fail(FE_EINVAL, "silu_mul: null pointer");
  const hipError_t e = launch_silu_mul(gate_up, output, rows, width, bf16 != 0, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "silu_mul kernel launch");
}

int fe_accept(const int64_t* draft, const int64_t* verify, int64_t* out, int batch, int k, void* stream) {
  if (batch < 0 || k < 0) return fail(FE_EINVAL, "accept: negative size");
  if (batch == 0) return FE_OK;
  if (draft == nullptr || verify == nullptr || out == nullptr) return fail(FE_EINVAL, "accept: null pointer");
  const hipError_t e = launch_accept(draft, verify, out, batch, k, static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "accept kernel launch");
}

int fe_norm_rope_append(const void* qkv, int64_t row_stride, const void* q_weight, const void* k_weight, float eps,
                        void* q_out, void* k_cache, void* v_cache, const int64_t* pos, const int64_t* slots,
                        const float* cache, int rows, int hq, int hkv, int dim, int bf16, int max_positions,
                        int cache_slots, void* stream) {
  if (rows < 0 || hq < 0 || hkv < 0 || cache_slots < 0) return fail(FE_EINVAL, "norm_rope_append: negative size");
  if (dim != kHeadDim) return fail(FE_EINVAL, "norm_rope_append: head dim must be 128");
  if (rows == 0 || hq + hkv == 0) return FE_OK;
  if (row_stride < (int64_t)(hq + 2 * hkv) * dim || row_stride % 8 != 0)
    return fail(FE_EINVAL, "norm_rope_append: row_stride must cover hq + 2*hkv heads and be a multiple of 8");
  if (qkv == nullptr || pos == nullptr || cache == nullptr || (hq > 0 && (q_out == nullptr || q_weight == nullptr)) ||
      (hkv > 0 && (k_weight == nullptr || k_cache == nullptr || v_cache == nullptr || slots == nullptr)))
    return fail(FE_EINVAL, "norm_rope_append: null pointer");
  const void* ptrs[] = {qkv, q_weight, k_weight, q_out, k_cache, v_cache};
  for (const void* ptr : ptrs)
    if (reinterpret_cast<uintptr_t>(ptr) % 16 != 0)
      return fail(FE_EINVAL, "norm_rope_append: tensors must be 16-byte aligned");
  const hipError_t e = launch_norm_rope_append(qkv, row_stride, q_weight, k_weight, eps, q_out, k_cache, v_cache, pos,
                                               slots, cache, rows, hq, hkv, bf16 != 0, max_positions, cache_slots,
                                               static_cast<hipStream_t>(stream));
  return e == hipSuccess ? FE_OK : hip_fail(e, "norm_rope_append kernel launch");
}

int fe_attn_plan_describe(int hq, int hkv, int dim, int page, int max_batch, int max_pages, int blocks,
                          const int32_t* qo, const int32_t* kv, const int32_t* pages, const int32_t* last, int batch,
                          int rows, int32_t* counts_out) {
  PlanShape sh;
  sh.hq = hq;
  sh.hkv = hkv;
  sh.dim = dim;
  sh.page = page;
  sh.max_batch = max_batch;
  sh.max_pages = max_pages;
  sh.blocks = blocks;
  sh.partial_cap = partial_cap_for(hq);
  BuiltPlan bp;
  std::string err;
  const int rc = build_plan(sh, qo, kv, pages, last, batch, rows, bp, err);
  if (rc != FE_OK) return fail(rc, err);
  if (counts_out) {
    counts_out[0] = (int32_t)bp.decode.size() * hkv;
    counts_out[1] = (int32_t)bp.mode[1].tile.size();
    counts_out[2] = (int32_t)bp.mode[1].merge.size();
    counts_out[3] = bp.mode[1].partial_rows;
  }
  return FE_OK;
}

int fe_attn_plan_dump(int hq, int hkv, int dim, int page, int max_batch, int max_pages, int blocks, const int32_t* qo,
                      const int32_t* kv, const int32_t* pages, const int32_t* last, int batch, int rows, int causal,
                      int32_t* items_out, int cap, int* n_out) {
  PlanShape sh;
  sh.hq = hq;
  sh.hkv = hkv;
  sh.dim = dim;
  sh.page = page;
  sh.max_batch = max_batch;
  sh.max_pages = max_pages;
  sh.blocks = blocks;
  sh.partial_cap = partial_cap_for(hq);
  BuiltPlan bp;
  std::string err;
  const int rc = build_plan(sh, qo, kv, pages, last, batch, rows, bp, err);
  if (rc != FE_OK) return fail(rc, err);
  int n = 0;
  auto emit = [&](int kind, const WorkItem& w) {
    if (items_out != nullptr && n < cap) {
      int32_t* o = items_out + 8 * n;
      o[0] = kind;
      o[1] = w.seq;
      o[2] = w.q0;
      o[3] = w.nq;
      o[4] = w.kvh;
      o[5] = w.t0;
      o[6] = w.t1;
      o[7] = w.part;
    }
    ++n;
  };
  for (size_t k = 0; k + 1 < bp.decode_share_off.size(); ++k)
    for (int h = 0; h < hkv; ++h)
      for (int i = bp.decode_share_off[k]; i < bp.decode_share_off[k + 1]; ++i) {
        WorkItem w = bp.decode[i];
        w.kvh = h;
        emit(0, w);
      }
  for (const WorkItem& w : bp.mode[causal ? 1 : 0].tile) emit(1, w);
  if (n_out) *n_out = n;
  return FE_OK;
}

int fe_attn_assign_shares(const int32_t* costs, int n, int slots, int fast, int32_t* order_out,
                          int32_t* off_out, int* n_shares_out) {
  if (n < 0 || slots < 1 || slots >= (1 << 20)) return fail(FE_EINVAL, "assign_shares: n >= 0 and 1 <= slots < 2^20");
  if (n > 0 && (costs == nullptr || order_out == nullptr)) return fail(FE_EINVAL, "assign_shares: null pointer");
  if (off_out == nullptr || n_shares_out == nullptr) return fail(FE_EINVAL, "assign_shares: null pointer");
  std::vector<WorkItem> items((size_t)n);
  int64_t total = 0;
  for (int i = 0; i < n; ++i) {
    if (costs[i] < 0) return fail(FE_EINVAL, "assign_shares: negative cost");
    total += costs[i];
    items[i] = WorkItem{i, 0, 0, 0, 0, 0, -1, costs[i]};  // seq carries the input index
  }
  if (total >= (int64_t(1) << 43)) return fail(FE_EINVAL, "assign_shares: total cost must stay below 2^43");
  std::vector<int32_t> off;
  assign_shares(items, slots, off, fast < 0 ? (1 << 30) : fast);
  for (int i = 0; i < n; ++i) order_out[i] = items[i].seq;
  for (size_t k = 0; k < off.size(); ++k) off_out[k] = off[k];
  *n_shares_out = (int)off.size() - 1;
  return FE_OK;
}

}  // extern "C"
