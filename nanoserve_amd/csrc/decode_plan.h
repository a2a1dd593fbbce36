// Decode work plan shared by the plan kernel (decode_plan.hip) and the decode
// kernel (paged_attention.hip).
//
// A plan cuts the decode rows of one batch into items: an item is a range of
// context tokens of one (sequence, kv head) pair.  It is built on the device
// from the device lengths (and, for mixed batches, the device query offsets),
// so a captured HIP graph replays a plan that follows the step's lengths.  The
// token count per item is chosen so the items about fill the device once (one
// per CU) when the batch's work is small, and split into several rounds of
// items, longest pairs first, when it is large.
#pragma once

#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>

namespace ns {

// Waves of a decode workgroup, and the block ids an item carries: those of
// the first kItemBlocks / (kItemWaves * tiles per step) steps of every wave
// (two steps of four 16-token tiles at head_dim 64, four steps of two at 128).
constexpr int kItemWaves = 4;
constexpr int kItemBlocks = 32;

struct DecodeItem {
  uint32_t s;       // sequence
  uint32_t qtok;    // its query row
  uint32_t t0, t1;  // context tokens [t0, t1) of this item
  uint32_t first;   // plan index of the pair's first item
  uint32_t nsplit;  // items of the pair
  uint32_t kvh;     // kv head
  uint32_t split;   // this item's index within the pair (first + split is its plan index)
  // Block ids of the first steps of every wave (entry (w * steps + st) *
  // tiles_per_step + j: tile j of step st of wave w), copied from the block
  // table when the block size is at least 16 (a tile then lies in one
  // block), so those K/V loads need no table round trip.  Entries past a
  // wave's range are 0.
  int32_t blk[kItemBlocks];
};
static_assert(sizeof(DecodeItem) == 160, "items are ten 16-byte rows");

struct DecodePlanHeader {
  uint32_t n_items;
  uint32_t num_seqs, num_kv_heads;
  uint32_t item_tokens;  // tokens per item the plan chose (a multiple of 16)
  uint32_t item_cap;     // items the buffer holds
  uint32_t pad[11];
};
static_assert(sizeof(DecodePlanHeader) == 64, "header is one 64-byte row");

// Planning constants.  kPlanCUs bounds the CU count the plan assumes (MI355X
// has 256); kMaxRounds bounds how many items per CU a large batch is cut into.
constexpr int kPlanCUs = 256;
constexpr int kMaxRounds = 16;
// Tokens per item at most: a decode wave then has at most 1024 tokens, whose
// block ids the decode kernel loads in one vector load (one per lane).
constexpr int kMaxItemTokens = 4096;

// Tokens per item below which an item is not cut further, and the tokens per
// CU a round of items is sized for: 1 MiB of K and V per CU and round.  An
// item costs about 5 us beside its streaming (first loads, the cross-wave
// reduce, the merge and the dispatch of the next workgroup), so rounds are
// kept few and items long; the longest-first order balances what is left.
inline int plan_min_tokens(int head_dim) { return head_dim == 64 ? 128 : 64; }
inline int plan_round_tokens(int head_dim) { return head_dim == 64 ? 4096 : 2048; }
// One-round plans keep items at least this long (0: no such floor) while the
// batch still gives half of the CUs an item at that length: shorter items then
// add split-K merges faster than they add streaming CUs (c2, B = 32 around 1k
// tokens: 12.31 -> 12.23 us per call with 512-token items), and batches that
// need the short items' parallelism (the c5 engine's decode steps, under half
// the CUs at 512 tokens) keep them.  A batch whose every context fits one
// such item takes it too: no split-K merge at all (c1, B = 8 up to 512
// tokens: 8.59 -> 8.16 us; B = 8 / 32 at 512 tokens: -13% / -9%).
inline int plan_long_tokens(int head_dim) { return head_dim == 64 ? 512 : 0; }

// Rounds of items per CU the decode grid provides for a batch whose work is at
// most num_seqs * num_kv_heads * max_ctx tokens (the host does not know the
// actual lengths; the plan uses fewer rounds when the batch is lighter).
inline int plan_max_rounds(int64_t num_seqs, int num_kv_heads, int64_t max_ctx, int head_dim) {
  const int64_t bound = num_seqs * num_kv_heads * (max_ctx > 0 ? max_ctx : 1);
  const int64_t per_round = static_cast<int64_t>(kPlanCUs) * plan_round_tokens(head_dim);
  const int64_t r = (bound + per_round - 1) / per_round;
  return static_cast<int>(r < 1 ? 1 : (r > kMaxRounds ? kMaxRounds : r));
}

// Items a plan can hold: the round target, or every token cut into items of
// kMaxItemTokens when that is more, plus one rounding item per pair.
inline int64_t plan_item_cap(int64_t num_seqs, int num_kv_heads, int64_t max_ctx, int rounds) {
  const int64_t pairs = num_seqs * num_kv_heads;
  const int64_t by_tokens = (pairs * (max_ctx > 0 ? max_ctx : 1) + kMaxItemTokens - 1) / kMaxItemTokens;
  const int64_t by_rounds = static_cast<int64_t>(kPlanCUs) * rounds;
  return (by_tokens > by_rounds ? by_tokens : by_rounds) + pairs;
}

// Bytes of a plan buffer: header, items, then four int32 scratch arrays of
// num_seqs (the last num_seqs + 1) entries the plan kernel works in.
inline size_t plan_bytes(int64_t num_seqs, int64_t item_cap) {
  return sizeof(DecodePlanHeader) + static_cast<size_t>(item_cap) * sizeof(DecodeItem) +
         static_cast<size_t>(num_seqs) * 16 + 16;
}

struct DecodePlanArgs {
  void* plan;
  uint32_t item_cap;
  const void* block_tables;  // read for the inline block ids when bs_shift >= 4
  int64_t bt_stride;
  int bt64;
  int bs_shift;
  int tiles_per_step;  // 16-token tiles of one wave step of the decode kernel
  const void* seq_lens;
  int sl64;
  const void* qsl;  // read unless decode_only
  int qsl64;
  int decode_only;
  int num_seqs, num_kv_heads;
  int64_t max_ctx;  // lengths are clamped to this (tokens addressable through a table row)
  int cus;          // CUs of the device, at most kPlanCUs
  int rounds;       // upper bound on items per CU (plan_max_rounds)
  int min_tokens, round_tokens, long_tokens;
};

// Launch the (single-workgroup) plan kernel on `stream`.
hipError_t launch_decode_plan(const DecodePlanArgs& a, hipStream_t stream);

}  // namespace ns
