// Shared host/device layout of the attention plan's device metadata.
//
// The reference hands attention a FlashInfer plan (src/flashinfer_attention.cu:14-34)
// or, in the ATen build, per-sequence gather indices and masks
// (src/portable_gpu_ops.cpp:27-38).  Here the host planner turns the same
// CSR metadata (qo / kv / pages / last) into flat work lists that the HIP
// kernels walk with a grid fixed by the plan capacity.
#pragma once
#include <stdint.h>

namespace feattn {

constexpr int kHeadDim = 128;  // the only head size the reference builds (flashinfer_attention.cu:23)
constexpr int kTileTokens = 64;  // tokens per KV tile of the MFMA tile kernel (4 pages of 16)
constexpr int kTileCols = 128;   // (q row, head) columns per tile work item (4 waves x 32)
constexpr int kDecodeCols = 32;  // max (q row, head) columns of one decode work item (2 MFMA N blocks)
constexpr int kDecodeWavesPerCu = 8;  // decode wavefronts resident per CU (one kv head each)

// Per sequence, derived from the CSR metadata exactly as the reference ATen
// plan does (portable_gpu_ops.cpp:30): len = (kv[b+1]-kv[b]-1)*page + last[b].
struct SeqInfo {
  int32_t qo;        // first query row of the sequence (qo[b])
  int32_t qlen;      // query rows (qo[b+1]-qo[b])
  int32_t len;       // tokens in the KV cache for this sequence, current chunk included
  int32_t page_off;  // index of the sequence's first page id in the page table (kv[b])
};

// One unit of kernel work: query rows [q0, q0+nq) of sequence `seq` (all the
// query heads of kv head `kvh`) against tokens [t0, t1).  part < 0 writes
// the normalised result to `out`; part >= 0 writes it, with its log2
// log-sum-exp, to partial slot part + (row - q0) for the merge kernel.
struct WorkItem {
  int32_t seq;
  int32_t q0;
  int32_t nq;
  int32_t kvh;
  int32_t t0;
  int32_t t1;
  int32_t part;
  int32_t cost;  // planner's cost estimate; unused on the device
};

// Decode piece as the decode kernel reads it: every query row of sequence
// `seq` (rows [q0, q0+nq), len tokens, page ids from page_off) against
// tokens [t0, t1); part as in WorkItem.  Carries the sequence fields itself
// so that a piece costs one metadata read.
struct DecodeItem {
  int32_t q0;
  int32_t nq;
  int32_t len;
  int32_t page_off;
  int32_t t0;
  int32_t t1;
  int32_t part;
  int32_t seq;
};

// Start of one decode share (one wavefront per kv head walks it): the range
// of its pieces in the decode list plus everything the first copies need,
// so that a wavefront issues its first loads after a single metadata read.
// pg0 / pg1 are the page ids of the share's first two 16-token blocks (pg1
// = 0 when there is no second block).  An empty share has it_begin ==
// it_end.
struct alignas(64) ShareStart {
  int32_t it_begin;
  int32_t it_end;
  DecodeItem first;
  int32_t pg0;
  int32_t pg1;
  int32_t pad[4];
};
static_assert(sizeof(ShareStart) == 64, "one 64-byte scalar load");
static_assert(sizeof(DecodeItem) == 32, "two pieces per 64 bytes");

// One query row whose tokens were split over `nsplit` work items.  Split s
// of this row lives in partial slot part + s*stride.
struct MergeRow {
  int32_t row;
  int32_t part;
  int32_t nsplit;
  int32_t stride;
};

// Kernel arguments shared by the decode and tile kernels.
struct AttnArgs {
  const uint16_t* q;
  const uint16_t* kc;
  const uint16_t* vc;
  uint16_t* out;
  float* lse;             // [rows][hq] natural log, may be null
  const SeqInfo* seqs;
  const int32_t* pages;
  const WorkItem* items;
  const int32_t* n_items;  // tile only, device-resident: end of the item list (graph replays read the current one)
  const int32_t* tile_off;   // tile only: items of workgroup b = [tile_off[b], min(tile_off[b+1], *n_items))
  const DecodeItem* ditems;  // decode only: the pieces, share by share
  const ShareStart* shares;  // decode only: one record per share
  int n_share_cap;           // decode only: records in `shares`
  uint16_t* part_o;        // [slots][hq][128] in the attention's 16-bit type, normalised per split
  float* part_lse;         // [slots][hq] log2 domain
  int hq;
  int hkv;
  int group;               // hq / hkv
  int page_shift;          // log2(page)
  float scale_log2;        // log2(e) / sqrt(128)
};

struct MergeArgs {
  uint16_t* out;
  float* lse;
  const MergeRow* rows;       // the records (eager launches) or the list they are indexed from (graph launches)
  int n_rows;                 // eager launches: records at `rows`
  const int32_t* count_base;  // graph launches, device-resident: records to fold, index of the first in `rows`
  const uint16_t* part_o;
  const float* part_lse;
  int hq;
};

}  // namespace feattn
