// Internal interface shared by the attention kernels.
#pragma once

#include "common.h"

namespace mvllm {

// One decode work-list record: split `split` (of `ns`) of request `r`, whose
// single query is token `qs` with visible keys [lo, hi]; the split streams
// keys [begin, end]. Positions fit in int32 (the launcher checks the block
// table's reach). r = -1 marks an empty slot.
struct DecodeItem {
  int32_t r, split, qs, ns;
  int32_t lo, hi, begin, end;
};

// One prefill work-list record: query tokens [t0, t1) of request `r` (whose
// first query is token `qs`); lo is the first visible key of row t0 and hi
// the last visible key of row t1 - 1 (their hull covers every row when
// visible ranges grow with the token, which the kernel checks). r = -1
// marks an empty slot.
struct PrefillItem {
  int32_t r, t0, t1, qs;
  int32_t lo, hi, pad0, pad1;
};

// Everything a ragged paged-attention launch needs. Strides are in elements.
struct AttnArgs {
  const void* q;
  int64_t q_s0, q_s1, q_s2;
  const void* cache;
  int64_t c_s[5];
  void* out;
  int64_t o_s0, o_s1, o_s2;
  const int64_t* positions;
  const int64_t* cstarts;
  const int64_t* qsl;
  const int64_t* lengths;
  const int64_t* table;
  int64_t t_s0, t_s1, width;
  int64_t num_tokens, num_requests, num_blocks, block_size;
  int32_t num_q_heads, num_kv_heads, group, head_dim;
  float scale_log2;  // softmax scale * log2(e): scores live in the exp2 domain
  // log2(block_size / 16) when block_size is a multiple of 16 whose
  // quotient is a power of two (16-key pages are then found with shifts),
  // else -1.
  int32_t page_shift = -1;
  // Split-KV decode partials: acc [R][max_splits][Hq][D], (max, sum) [R][max_splits][Hq].
  float* ws_acc;
  float2* ws_ml;
  int32_t split_tokens, max_splits;
  int32_t mode;  // generic kernel: 0 = every token; 1 = only requests with > 1 query
  // Prefill work list: one record per (request, query block) slot, heaviest
  // first; r = -1 marks an empty slot. Written by the item kernel before the
  // prefill kernel reads it.
  PrefillItem* items;
  // Decode work list: one record per (request, split) slot, full splits
  // first, then the partial last splits from the largest; r = -1 marks an
  // empty slot.
  DecodeItem* decode_items;
  // Per request, written with the decode work list: (query token, number of
  // splits), or (0, -1) for a request that is not a single-query decode. The
  // combine kernel reads it instead of re-deriving the visible range.
  int2* decode_req;
  // Host side only: the work lists and the per-request table are already in
  // the workspace (planned once for a step), so the launches skip the
  // work-list kernels.
  int32_t lists_ready;
  // The caller's max_query_len hint said 1 (no prefill launch): the combine
  // kernel makes the rows of any request with another query count NaN.
  int32_t decode_only;
};

// Visible key positions [lo, hi] of query `t` in request `r` whose first
// query is `qs`: the reference gathers [start(first query), length) and
// masks keys outside [start(t), pos(t)] (reference.py:101-138, 49-68).
// Positions past the block table's reach cannot be mapped and are clipped.
__device__ __forceinline__ void visible_range(const AttnArgs& a, int64_t r, int64_t qs,
                                              int64_t t, int64_t& lo, int64_t& hi) {
  const int64_t first = a.cstarts[qs];
  const int64_t own = a.cstarts[t];
  lo = own > first ? own : first;
  if (lo < 0) lo = 0;
  hi = a.positions[t];
  const int64_t last = a.lengths[r] - 1;
  if (last < hi) hi = last;
  const int64_t reach = a.width * a.block_size - 1;
  if (reach < hi) hi = reach;
}

// Physical block holding position p of request r, or -1 when the table
// entry is not a valid block id (such keys are treated as masked).
__device__ __forceinline__ int64_t block_of(const AttnArgs& a, int64_t r, int64_t p) {
  const int64_t b = a.table[r * a.t_s0 + (p / a.block_size) * a.t_s1];
  return (b >= 0 && b < a.num_blocks) ? b : -1;
}

// Number of split-KV partitions of a decode query with visible range [lo, hi].
__device__ __forceinline__ int64_t decode_num_splits(int64_t lo, int64_t hi, int32_t split) {
  if (hi < lo) return 0;
  const int64_t base = lo & ~int64_t(15);
  return (hi - base + split) / split;
}

// Host-side launchers (one per kernel family).
// Launchers; `start`/`stop` (may be null) bracket the main kernel's launch.
int launch_generic(const AttnArgs& a, int32_t dtype, hipStream_t s);
int launch_decode(const AttnArgs& a, int32_t dtype, hipStream_t s, hipEvent_t start,
                  hipEvent_t stop);
// The work-list kernels alone (decode list + per-request table; prefill list).
int launch_decode_lists(const AttnArgs& a, hipStream_t s);
int launch_prefill_lists(const AttnArgs& a, hipStream_t s);
int launch_prefill(const AttnArgs& a, int32_t dtype, hipStream_t s, hipEvent_t start,
                   hipEvent_t stop);
bool prefill_supported(const AttnArgs& a, int32_t dtype);

// The one-launch attention step: decode and prefill workgroups in one grid
// (attention_prefill.hip), for batches whose decode part runs the pipelined
// kernel with its default shape (kStepDecodeWaves waves, two stages).
constexpr int kStepDecodeWaves = 4;
bool decode_step_eligible(const AttnArgs& a);
int64_t decode_step_blocks(const AttnArgs& a);  // decode workgroups of the step grid
int launch_decode_combine(const AttnArgs& a, int32_t dtype, hipStream_t s);
// `prefill_first`: the prefill workgroups lead the grid (else the decode ones).
int launch_step(const AttnArgs& a, int32_t dtype, bool prefill_first, hipStream_t s, hipEvent_t start,
                hipEvent_t stop);

// Device properties used for launch shapes (cached per device).
int device_cu_count();

}  // namespace mvllm
