// Work-list builders of the attention kernels and the KV-row copy, as
// device functions: each runs in one 1024-thread workgroup (the list
// builders) or a part of one (the row copy), either in its own kernel or in
// the fused prologue of a forward (attention_api.hip), which builds both
// lists and writes the step's K/V rows in a single launch.
#pragma once

#include "attention.h"

namespace mvllm {

// One token's K and V rows copied into its cache slot (bit-exact), 16 bytes
// per step: whole token rows, because all KV heads of one token are
// contiguous in the cache layout (2, blocks, block_size, heads, dim).
struct KvRowArgs {
  const char* key;
  const char* value;
  char* cache;
  const int64_t* slots;
  int64_t key_token_stride;    // bytes
  int64_t value_token_stride;  // bytes
  int64_t plane_stride;        // bytes
  int64_t block_stride;        // bytes
  int64_t offset_stride;       // bytes
  int64_t block_size;
  int64_t num_slots;
  int32_t chunks;              // 16-byte chunks per token row
};

// Validates a KV write (mvllm_kv_write's checks) and, when the rows can be
// copied 16 bytes at a time, fills `rows` and sets `*vectorised` (kv_cache.hip).
int kv_write_prepare(const mvllm_tensor3* key, const mvllm_tensor3* value, const mvllm_kv_cache* cache,
                     const int64_t* slot_mapping, int64_t num_tokens, KvRowArgs* rows, bool* vectorised);

namespace {

// Rows of one prefill workgroup: (query head of a KV head's group, token)
// pairs; a work item then covers T = kRows / G query tokens, and
// prefill_lg_tok gives log2(T).
constexpr int kRows = 128;

inline int prefill_lg_tok(const AttnArgs& a) {
  int lg_tok = 0;
  while ((kRows >> lg_tok) > a.group) ++lg_tok;
  return lg_tok;
}

// Chunks c = first, first + step, ... of token `token`'s K row then V row.
// A slot < 0 or >= num_slots writes nothing.
__device__ inline void copy_kv_row(const KvRowArgs& a, int64_t token, int first, int step) {
  const int64_t slot = a.slots[token];
  const char* ksrc = a.key + token * a.key_token_stride;
  const char* vsrc = a.value + token * a.value_token_stride;
  if (first < 2 * a.chunks && first + step >= 2 * a.chunks) {
    // One chunk per thread: its load does not depend on the slot, so it is
    // issued before the slot is known and the two latencies overlap (a
    // padding token's row exists too; only its store is skipped).
    const bool is_value = first >= a.chunks;
    const int chunk = is_value ? first - a.chunks : first;
    const uint4 data = *reinterpret_cast<const uint4*>((is_value ? vsrc : ksrc) + 16 * chunk);
    // Keep the slot's checks (and their wait) after the load is issued.
    __builtin_amdgcn_sched_barrier(0);
    if (slot < 0 || slot >= a.num_slots) return;
    const int64_t block = slot / a.block_size;
    const int64_t offset = slot - block * a.block_size;
    char* dst = a.cache + block * a.block_stride + offset * a.offset_stride;
    *reinterpret_cast<uint4*>(dst + (is_value ? a.plane_stride : 0) + 16 * chunk) = data;
    return;
  }
  if (slot < 0 || slot >= a.num_slots) return;
  const int64_t block = slot / a.block_size;
  const int64_t offset = slot - block * a.block_size;
  char* dst = a.cache + block * a.block_stride + offset * a.offset_stride;
  for (int c = first; c < 2 * a.chunks; c += step) {
    const bool is_value = c >= a.chunks;
    const int chunk = is_value ? c - a.chunks : c;
    const uint4 data = *reinterpret_cast<const uint4*>((is_value ? vsrc : ksrc) + 16 * chunk);
    *reinterpret_cast<uint4*>(dst + (is_value ? a.plane_stride : 0) + 16 * chunk) = data;
  }
}

// ---- decode work list --------------------------------------------------------
//
// One workgroup lists the (request, split) items of the single-query
// requests: every full split first (in any order), then the partial last
// splits from the largest down, so the in-order dispatch of the decode grid
// ends on the shortest items. Empty slots (up to R * max_splits) get
// request -1.
constexpr int kDecodeListThreads = 1024;
constexpr int kSizeBuckets = 64;  // sizes of a partial split, split / 64 tokens (rounded up to a power of two) each

__device__ inline void build_decode_list(const AttnArgs& a) {
  __shared__ int32_t full_count, full_pos;
  __shared__ int32_t bucket[kSizeBuckets];
  const int tid = threadIdx.x;
  const int64_t R = a.num_requests;
  const int64_t capacity = R * a.max_splits;
  // 64 buckets of 2^bucket_shift sizes span every split length: the
  // smallest shift with 64 << shift >= split_tokens (a partial split holds
  // 1 .. split_tokens - 1 keys, so its bucket index stays below 64).
  int bucket_shift = 0;
  while ((kSizeBuckets << bucket_shift) < a.split_tokens) ++bucket_shift;
  if (tid == 0) full_count = full_pos = 0;
  if (tid < kSizeBuckets) bucket[tid] = 0;
  // A decode request: its query token, visible keys, split count and the
  // size of its last split (ns = 0: not a decode request, or no visible key;
  // dec = 1 marks a decode request).
  struct Desc {
    int32_t qs, lo, hi, ns, last, dec;
  };
  auto describe = [&](int64_t r) {
    Desc d = {0, 0, -1, 0, 0, 0};
    const int64_t qs = a.qsl[r];
    if (qs < 0 || qs >= a.num_tokens || a.qsl[r + 1] - qs != 1) return d;
    d.qs = static_cast<int32_t>(qs);
    d.dec = 1;
    int64_t lo, hi;
    visible_range(a, r, qs, qs, lo, hi);
    const int64_t n = decode_num_splits(lo, hi, a.split_tokens);
    if (n <= 0) return d;
    d.lo = static_cast<int32_t>(lo);
    d.hi = static_cast<int32_t>(hi);
    d.ns = static_cast<int32_t>(n);
    d.last = static_cast<int32_t>((hi - (lo & ~int64_t(15)) + 1) - (n - 1) * a.split_tokens);
    return d;
  };
  auto record = [&](int64_t r, const Desc& d, int32_t sp) {
    const int32_t begin = (d.lo & ~15) + sp * a.split_tokens;
    const int32_t end = begin + a.split_tokens - 1 < d.hi ? begin + a.split_tokens - 1 : d.hi;
    return DecodeItem{static_cast<int32_t>(r), sp, d.qs, d.ns, d.lo, d.hi, begin, end};
  };
  // The thread's first request stays in registers between the passes.
  Desc d0 = {0, 0, -1, 0, 0, 0};
  if (tid < R) d0 = describe(tid);
  __syncthreads();
  const int lane = tid & 63;
  // Exclusive prefix of v over the wave and the wave's total.
  auto wave_scan = [&](int32_t v, int32_t& total) {
    int32_t incl = v;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int32_t y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    total = __shfl(incl, 63, 64);
    return incl - v;
  };
  // Pass 1: count full splits (one LDS atomic per wave), histogram the
  // partial ones by size. The loop bound is uniform per wave.
  for (int64_t r0 = tid - lane; r0 < R; r0 += kDecodeListThreads) {
    const int64_t r = r0 + lane;
    Desc d = {0, 0, -1, 0, 0, 0};
    if (r < R) d = r == tid ? d0 : describe(r);
    const int32_t ns = d.ns, last = d.last;
    const bool partial = ns > 0 && last < a.split_tokens;
    int32_t total;
    wave_scan(partial ? ns - 1 : ns, total);
    if (lane == 0 && total) atomicAdd(&full_count, total);
    if (partial) atomicAdd(&bucket[(last - 1) >> bucket_shift], 1);
  }
  __syncthreads();
  // Partial splits start after the full ones, largest bucket first: an
  // exclusive scan over the buckets in descending order, one lane each.
  static_assert(kSizeBuckets == 64, "one wave scans the buckets");
  if (tid < 64) {
    const int32_t c = bucket[63 - tid];
    int32_t incl = c;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int32_t y = __shfl_up(incl, d, 64);
      if (tid >= d) incl += y;
    }
    const int32_t fulls = full_count;
    bucket[63 - tid] = fulls + incl - c;
    if (tid == 63) full_count = fulls + incl;  // total number of items
  }
  __syncthreads();
  // Pass 2: place the items (one LDS atomic per wave for the full splits).
  for (int64_t r0 = tid - lane; r0 < R; r0 += kDecodeListThreads) {
    const int64_t r = r0 + lane;
    Desc d = {0, 0, -1, 0, 0, 0};
    if (r < R) d = r == tid ? d0 : describe(r);
    const int32_t ns = d.ns, last = d.last;
    const bool partial = ns > 0 && last < a.split_tokens;
    const int32_t nfull = partial ? ns - 1 : ns;
    int32_t total;
    const int32_t excl = wave_scan(nfull, total);
    int32_t at = 0;
    if (lane == 0 && total) at = atomicAdd(&full_pos, total);
    at = __shfl(at, 0, 64) + excl;
    for (int32_t sp = 0; sp < nfull; ++sp) a.decode_items[at + sp] = record(r, d, sp);
    if (partial) a.decode_items[atomicAdd(&bucket[(last - 1) >> bucket_shift], 1)] = record(r, d, ns - 1);
    if (r < R) a.decode_req[r] = int2{d.qs, d.dec ? ns : -1};
  }
  for (int64_t j = full_count + tid; j < capacity; j += kDecodeListThreads)
    a.decode_items[j] = DecodeItem{-1, -1, 0, 0, 0, -1, 0, -1};
}


// ---- prefill work list ------------------------------------------------------
//
// Request r's query blocks of T tokens occupy work-list slots
// [qsl[r] / T + r, qsl[r] / T + r + ceil(n_r / T)), which never overlap and
// stay below N / T + R. One workgroup lists every (request, block) item of
// the multi-query requests, sorted by the number of 64-key tiles it visits,
// heaviest first, so that the hardware's in-order dispatch of the prefill
// grid approximates longest-processing-time-first scheduling. Empty slots
// (single-query requests) go last as request -1. Items within a cost
// bucket come in any order; every item writes only its own output rows.
constexpr int kItemThreads = 1024;
constexpr int kItemSlots = 8192;    // larger batches keep slot order (late slots first)
constexpr int kCostBuckets = 2048;  // tiles per item, clamped
static_assert(kCostBuckets == 2 * kItemThreads, "the bucket scan gives each thread two buckets");

__device__ inline void build_prefill_list(const AttnArgs& a, int32_t lg_tok) {
  __shared__ int32_t owner[kItemSlots];
  __shared__ uint16_t bucket_of[kItemSlots];
  __shared__ int32_t start[kCostBuckets];
  __shared__ int32_t wave_sums[kItemThreads / 64];
  __shared__ int32_t total;
  const int tid = threadIdx.x;
  const int64_t tpb = int64_t{1} << lg_tok;
  const int64_t R = a.num_requests;
  const int64_t nslots = a.num_tokens / tpb + R;
  // Record of query block b of request r (its first query is qs, its last
  // query token qe - 1).
  auto record = [&](int64_t r, int64_t qs, int64_t qe, int64_t b) {
    const int64_t t0 = qs + b * tpb;
    const int64_t t1 = t0 + tpb < qe ? t0 + tpb : qe;
    int64_t lo0, hi0, lo1, hi1;
    visible_range(a, r, qs, t0, lo0, hi0);
    visible_range(a, r, qs, t1 - 1, lo1, hi1);
    return PrefillItem{static_cast<int32_t>(r), static_cast<int32_t>(t0), static_cast<int32_t>(t1),
                       static_cast<int32_t>(qs), static_cast<int32_t>(lo0), static_cast<int32_t>(hi1), 0, 0};
  };
  const PrefillItem empty = {-1, 0, 0, 0, 0, -1, 0, 0};
  if (nslots > kItemSlots) {
    for (int64_t j = tid; j < nslots; j += kItemThreads) {
      int64_t rl = 0, rh = R - 1;
      while (rl < rh) {
        const int64_t mid = (rl + rh + 1) >> 1;
        if (a.qsl[mid] / tpb + mid <= j) rl = mid; else rh = mid - 1;
      }
      const int64_t qs = a.qsl[rl], qe = a.qsl[rl + 1];
      const int64_t b = j - (qs / tpb + rl);
      const bool ok = qs >= 0 && qe <= a.num_tokens && qe - qs > 1 && b >= 0 && qs + b * tpb < qe;
      a.items[nslots - 1 - j] = ok ? record(rl, qs, qe, b) : empty;
    }
    return;
  }
  for (int j = tid; j < nslots; j += kItemThreads) owner[j] = -1;
  for (int k = tid; k < kCostBuckets; k += kItemThreads) start[k] = 0;
  __syncthreads();
  for (int64_t r = tid; r < R; r += kItemThreads) {
    const int64_t qs = a.qsl[r], qe = a.qsl[r + 1];
    if (qs < 0 || qe > a.num_tokens || qe - qs <= 1) continue;
    const int64_t first = qs / tpb + r;
    const int64_t nb = (qe - qs + tpb - 1) / tpb;
    for (int64_t b = 0; b < nb && first + b < nslots; ++b) owner[first + b] = static_cast<int32_t>(r);
  }
  __syncthreads();
  // Cost of an item: 64-key tiles between its first row's first visible key
  // and its last row's last one.
  for (int j = tid; j < nslots; j += kItemThreads) {
    const int32_t r = owner[j];
    if (r < 0) continue;
    const int64_t qs = a.qsl[r], qe = a.qsl[r + 1];
    const int64_t t0 = qs + (j - (qs / tpb + r)) * tpb;
    const int64_t t1 = (t0 + tpb < qe ? t0 + tpb : qe) - 1;
    int64_t lo0, hi0, lo1, hi1;
    visible_range(a, r, qs, t0, lo0, hi0);
    visible_range(a, r, qs, t1, lo1, hi1);
    const int64_t tiles = hi1 >= lo0 ? (hi1 - lo0 + 64) / 64 : 0;
    const int bucket = static_cast<int>(tiles < kCostBuckets - 1 ? tiles : kCostBuckets - 1);
    bucket_of[j] = static_cast<uint16_t>(bucket);
    atomicAdd(&start[bucket], 1);
  }
  __syncthreads();
  // start[k] = number of items in buckets above k (exclusive scan, heaviest
  // first). Thread t owns buckets K - 1 - 2 t and K - 2 - 2 t.
  {
    const int k0 = kCostBuckets - 1 - 2 * tid;
    const int v0 = start[k0], v1 = start[k0 - 1];
    const int own = v0 + v1;
    int incl = own;
    const int lane = tid & 63, w = tid >> 6;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
      const int y = __shfl_up(incl, d, 64);
      if (lane >= d) incl += y;
    }
    if (lane == 63) wave_sums[w] = incl;
    __syncthreads();
    int before = 0;
    for (int i = 0; i < w; ++i) before += wave_sums[i];
    const int excl = before + incl - own;
    if (tid == kItemThreads - 1) total = excl + own;
    __syncthreads();
    start[k0] = excl;
    start[k0 - 1] = excl + v0;
  }
  __syncthreads();
  for (int j = tid; j < nslots; j += kItemThreads) {
    const int32_t r = owner[j];
    if (r < 0) continue;
    const int pos = atomicAdd(&start[bucket_of[j]], 1);
    const int64_t qs = a.qsl[r], qe = a.qsl[r + 1];
    a.items[pos] = record(r, qs, qe, j - (qs / tpb + r));
  }
  for (int64_t j = total + tid; j < nslots; j += kItemThreads) a.items[j] = empty;
}


}  // namespace
}  // namespace mvllm
