// Host-side planner: validates the reference's CSR metadata and turns it into
// decode / tile / merge work lists.  Pure host code (no HIP calls), so it is
// also exercised by the CPU tests through fe_attn_plan_describe / _dump.
#pragma once
#include <stdint.h>

#include <string>
#include <vector>

#include "attn_types.hpp"

namespace feattn {

struct PlanShape {
  int hq = 0;
  int hkv = 0;
  int dim = 0;
  int page = 0;
  int max_batch = 0;
  int max_pages = 0;
  int blocks = 0;
  int num_cus = 256;        // compute units on the device (sizes split-KV)
  int decode_waves = 2048;  // wavefront slots of one decode launch
  int tile_slots = 512;     // workgroups of one tile launch (two resident per CU)
  int item_cap = 1 << 16;   // work items per list
  int partial_cap = 4096;   // split-KV partial slots ([hq][128] fp32 each)
};

struct ModeLists {
  std::vector<WorkItem> tile;            // grouped by share: share k = [tile_off[k], tile_off[k+1])
  std::vector<int32_t> tile_off;         // CSR over shares (one share per tile workgroup)
  std::vector<MergeRow> merge;
  int partial_rows = 0;  // decode partials followed by this mode's tile partials
};

struct BuiltPlan {
  std::vector<SeqInfo> seqs;
  std::vector<WorkItem> decode;  // decode pieces (kvh unset), identical for both masks
  std::vector<int32_t> decode_share_off;  // CSR: pieces of share k = [off[k], off[k+1])
  std::vector<DecodeItem> decode_items;   // `decode` in the decode kernel's format
  std::vector<ShareStart> decode_starts;  // one per share in use
  int decode_partials = 0;
  std::vector<MergeRow> decode_merge;
  int decode_nc = 16;            // 16 or 32 columns per decode item (MFMA column blocks x 16)
  ModeLists mode[2];             // [0] full (non-causal), [1] causal
};

// Longest-processing-time assignment of items (by `cost`, >= 0) to at most
// `slots` (< 2^20) shares: items in decreasing cost order (ties keep their
// order) each go to the least-loaded share, the lowest index among equals;
// `items` is regrouped share by share and `off` gets the CSR offsets.  When
// `fast` is below the number of shares in use, shares [0, fast) are taken to
// work kSlowShareWeight / kFastShareWeight times as fast as the rest: their
// loads are counted at that ratio, so they receive that much more work.
constexpr uint64_t kFastShareWeight = 2;
constexpr uint64_t kSlowShareWeight = 3;
void assign_shares(std::vector<WorkItem>& items, int slots, std::vector<int32_t>& off, int fast = 1 << 30);

// Returns 0 (FE_OK) or a negative FE_E* code with `err` set.
int validate_shape(const PlanShape& sh, std::string& err);
int build_plan(const PlanShape& sh, const int32_t* qo, const int32_t* kv, const int32_t* pages,
               const int32_t* last, int batch, int rows, BuiltPlan& out, std::string& err);

}  // namespace feattn
