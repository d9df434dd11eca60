// Ragged-batch packing on the GPU.
//
// Replaces the reference ModelRunner's per-step Python loops
// (model_runner.py:751-900: flattened ids/positions, prefix-sum query
// starts, context lengths, slot mapping per token, null-padded block table,
// sampling rows; attention.py:68-75: per-token context starts) and the
// graph-padding copy (model_runner.py:78-122) with two launches:
//   1. a one-workgroup scan over requests (token / block / sampling prefix
//      sums, query_start_locations, context_lengths, sampling rows);
//   2. one workgroup per request filling its tokens and block-table row,
//      plus padding workgroups for the capacity tail.
#include "common.h"

namespace mvllm {
namespace {

constexpr int kScanThreads = 1024;
constexpr int kFillThreads = 256;

__device__ __forceinline__ int64_t spec_start(int32_t kind, int64_t param, int64_t pos) {
  if (kind == MVLLM_SPEC_SLIDING_WINDOW) {
    const int64_t s = pos - param + 1;
    return s > 0 ? s : 0;
  }
  if (kind == MVLLM_SPEC_CHUNKED_LOCAL) return (pos / param) * param;
  return 0;
}

// Device-resident block rows (mvllm_pack_batch_rows); rows == nullptr: the
// block ids of every request are in the payload.
struct Rows {
  int32_t* rows;
  int64_t num_slots, width;
  const int32_t* updates;
  int64_t num_updates;
};

__global__ __launch_bounds__(kScanThreads) void pack_scan_kernel(mvllm_pack_args a, Rows rw) {
  __shared__ int64_t tok[kScanThreads], blk[kScanThreads], smp[kScanThreads];
  const int tid = threadIdx.x;
  // Row updates first: the fill kernel that follows reads the rows. Each
  // record is range-checked; a bad one is skipped.
  if (rw.rows) {
    for (int64_t u = 0; u < rw.num_updates; ++u) {
      const int32_t* rec = rw.updates + 4 * u;
      const int64_t slot = rec[0], first = rec[1], count = rec[2], offset = rec[3];
      if (slot < 0 || slot >= rw.num_slots || first < 0 || count < 0 || first + count > rw.width ||
          offset < 0 || offset + count > a.num_block_ids)
        continue;
      int32_t* dst = rw.rows + slot * rw.width + first;
      for (int64_t i = tid; i < count; i += kScanThreads) dst[i] = a.block_ids[offset + i];
    }
    __syncthreads();
  }
  int64_t carry_tok = 0, carry_blk = 0, carry_smp = 0;
  for (int64_t base = 0; base < a.num_requests; base += kScanThreads) {
    const int64_t r = base + tid;
    int32_t* info = a.request_info + r * MVLLM_PACK_FIELDS;
    int64_t v_tok = 0, v_blk = 0, v_smp = 0, computed = 0;
    if (r < a.num_requests) {
      computed = info[0];
      v_tok = info[1];
      v_blk = info[2];
      v_smp = info[3] != 0 ? 1 : 0;
    }
    tok[tid] = v_tok;
    blk[tid] = v_blk;
    smp[tid] = v_smp;
    __syncthreads();
    for (int step = 1; step < kScanThreads; step <<= 1) {  // Hillis-Steele inclusive scan
      int64_t x_tok = 0, x_blk = 0, x_smp = 0;
      if (tid >= step) {
        x_tok = tok[tid - step];
        x_blk = blk[tid - step];
        x_smp = smp[tid - step];
      }
      __syncthreads();
      tok[tid] += x_tok;
      blk[tid] += x_blk;
      smp[tid] += x_smp;
      __syncthreads();
    }
    if (r < a.num_requests) {
      const int64_t t0 = carry_tok + tok[tid] - v_tok;
      const int64_t b0 = carry_blk + blk[tid] - v_blk;
      const int64_t s0 = carry_smp + smp[tid] - v_smp;
      info[4] = static_cast<int32_t>(t0);
      info[5] = static_cast<int32_t>(b0);
      if (a.query_start_locations) a.query_start_locations[r] = t0;
      if (a.context_lengths) a.context_lengths[r] = computed + v_tok;
      if (v_smp && a.sampling_rows) a.sampling_rows[s0] = t0 + v_tok - 1;
    }
    carry_tok += tok[kScanThreads - 1];
    carry_blk += blk[kScanThreads - 1];
    carry_smp += smp[kScanThreads - 1];
    __syncthreads();
  }
  if (a.query_start_locations)
    for (int64_t i = a.num_requests + tid; i <= a.request_capacity; i += kScanThreads)
      a.query_start_locations[i] = a.num_tokens;
}

__global__ __launch_bounds__(kFillThreads) void pack_fill_kernel(mvllm_pack_args a, Rows rw,
                                                                int64_t pad_blocks) {
  const int tid = threadIdx.x;
  const int64_t R = a.num_requests;
  const int64_t W = a.block_table_width;
  if (static_cast<int64_t>(blockIdx.x) < R) {
    const int64_t r = blockIdx.x;
    const int32_t* info = a.request_info + r * MVLLM_PACK_FIELDS;
    const int64_t computed = info[0], scheduled = info[1];
    int64_t nblocks = info[2];
    const int64_t t0 = info[4], b0 = info[5];
    const int32_t* ids = a.block_ids + b0;
    if (rw.rows) {
      // A request's ids come from its row; an out-of-range slot or a list
      // longer than the row has no block ids (null entries, slot -1).
      const int64_t slot = info[6];
      const bool ok = slot >= 0 && slot < rw.num_slots && nblocks <= rw.width;
      ids = rw.rows + (ok ? slot : 0) * rw.width;
      if (!ok) nblocks = 0;
    }
    for (int64_t i = tid; i < scheduled; i += kFillThreads) {
      const int64_t t = t0 + i;
      const int64_t pos = computed + i;
      if (a.positions) a.positions[t] = pos;
      if (a.input_ids) a.input_ids[t] = a.token_ids[t];
      if (a.context_starts) a.context_starts[t] = spec_start(a.spec_kind, a.spec_parameter, pos);
      if (a.slot_mapping) {
        const int64_t logical = pos / a.block_size;
        a.slot_mapping[t] = logical < nblocks
                                ? static_cast<int64_t>(ids[logical]) * a.block_size +
                                      (pos - logical * a.block_size)
                                : -1;
      }
    }
    if (a.block_table)
      for (int64_t j = tid; j < W; j += kFillThreads)
        a.block_table[r * W + j] = j < nblocks ? static_cast<int64_t>(ids[j]) : a.null_block_id;
    return;
  }
  // Padding: the capacity tail of every output.
  const int64_t stride = pad_blocks * kFillThreads;
  const int64_t first = (static_cast<int64_t>(blockIdx.x) - R) * kFillThreads + tid;
  for (int64_t t = a.num_tokens + first; t < a.token_capacity; t += stride) {
    if (a.input_ids) a.input_ids[t] = 0;
    if (a.positions) a.positions[t] = 0;
    if (a.context_starts) a.context_starts[t] = 0;
    if (a.slot_mapping) a.slot_mapping[t] = -1;
  }
  for (int64_t r = R + first; r < a.request_capacity; r += stride)
    if (a.context_lengths) a.context_lengths[r] = 0;
  if (a.block_table) {
    const int64_t begin = R * W, end = a.request_capacity * W;
    for (int64_t i = begin + first; i < end; i += stride) a.block_table[i] = a.null_block_id;
  }
}

__global__ __launch_bounds__(256) void context_starts_kernel(const int64_t* positions, int64_t n,
                                                             int32_t kind, int64_t param,
                                                             int64_t* out) {
  const int64_t i = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
  if (i < n) out[i] = spec_start(kind, param, positions[i]);
}

int check_spec(int32_t kind, int64_t param) {
  if (kind != MVLLM_SPEC_FULL && kind != MVLLM_SPEC_SLIDING_WINDOW &&
      kind != MVLLM_SPEC_CHUNKED_LOCAL)
    return fail(MVLLM_ERR_INVALID, "unknown attention spec kind %d", kind);
  if (kind != MVLLM_SPEC_FULL && param <= 0)
    return fail(MVLLM_ERR_INVALID, "spec parameter must be positive, got %lld", (long long)param);
  return MVLLM_OK;
}

}  // namespace
}  // namespace mvllm

using namespace mvllm;

extern "C" int mvllm_context_starts(const int64_t* positions, int64_t num_tokens,
                                    int32_t spec_kind, int64_t spec_parameter, int64_t* out,
                                    void* stream) {
  clear_error();
  if (int rc = check_spec(spec_kind, spec_parameter)) return rc;
  if (num_tokens < 0) return fail(MVLLM_ERR_INVALID, "negative num_tokens");
  if (num_tokens == 0) return MVLLM_OK;
  if (!positions || !out) return fail(MVLLM_ERR_INVALID, "null positions/out");
  const int64_t blocks = ceil_div(num_tokens, 256);
  if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "too many tokens");
  hipLaunchKernelGGL(context_starts_kernel, dim3(static_cast<unsigned>(blocks)), dim3(256), 0,
                     reinterpret_cast<hipStream_t>(stream), positions, num_tokens, spec_kind,
                     spec_parameter, out);
  MVLLM_LAUNCH_CHECK("context_starts_kernel");
  return MVLLM_OK;
}

namespace mvllm {
namespace {

int pack_batch(const mvllm_pack_args* args, const mvllm_block_rows* rows, void* stream) {
  if (!args) return fail(MVLLM_ERR_INVALID, "pack args are null");
  const mvllm_pack_args& a = *args;
  Rows rw = {nullptr, 0, 0, nullptr, 0};
  if (rows) {
    if (!rows->rows || rows->num_slots <= 0 || rows->width <= 0)
      return fail(MVLLM_ERR_INVALID, "block rows need a table of positive size");
    if (rows->num_updates < 0 || (rows->num_updates > 0 && !rows->updates))
      return fail(MVLLM_ERR_INVALID, "block-row updates are null");
    if (rows->num_slots > INT32_MAX || rows->width > INT32_MAX)
      return fail(MVLLM_ERR_INVALID, "block rows too large");
    rw = Rows{rows->rows, rows->num_slots, rows->width, rows->updates, rows->num_updates};
  }
  if (int rc = check_spec(a.spec_kind, a.spec_parameter)) return rc;
  if (a.num_requests < 0 || a.num_tokens < 0 || a.num_block_ids < 0 || a.block_size <= 0 ||
      a.block_table_width < 0)
    return fail(MVLLM_ERR_INVALID, "negative size or non-positive block_size");
  if (a.token_capacity < a.num_tokens || a.request_capacity < a.num_requests)
    return fail(MVLLM_ERR_INVALID, "capacity (%lld tokens, %lld requests) below actual (%lld, %lld)",
                (long long)a.token_capacity, (long long)a.request_capacity,
                (long long)a.num_tokens, (long long)a.num_requests);
  if (a.num_requests > 0 && !a.request_info) return fail(MVLLM_ERR_INVALID, "request_info is null");
  if (a.num_block_ids > 0 && !a.block_ids) return fail(MVLLM_ERR_INVALID, "block_ids is null");
  if (a.input_ids && a.num_tokens > 0 && !a.token_ids)
    return fail(MVLLM_ERR_INVALID, "input_ids requested without token_ids");
  if (a.num_requests > INT32_MAX / 2) return fail(MVLLM_ERR_INVALID, "too many requests");
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  hipLaunchKernelGGL(pack_scan_kernel, dim3(1), dim3(kScanThreads), 0, s, a, rw);
  MVLLM_LAUNCH_CHECK("pack_scan_kernel");
  const int64_t pad_elems = std::max<int64_t>(
      std::max<int64_t>(a.token_capacity - a.num_tokens, a.request_capacity - a.num_requests),
      (a.request_capacity - a.num_requests) * a.block_table_width);
  int64_t pad_blocks = ceil_div(pad_elems, kFillThreads);
  if (pad_blocks < 1) pad_blocks = 1;
  if (pad_blocks > 1024) pad_blocks = 1024;
  hipLaunchKernelGGL(pack_fill_kernel, dim3(static_cast<unsigned>(a.num_requests + pad_blocks)),
                     dim3(kFillThreads), 0, s, a, rw, pad_blocks);
  MVLLM_LAUNCH_CHECK("pack_fill_kernel");
  return MVLLM_OK;
}

}  // namespace
}  // namespace mvllm

extern "C" int mvllm_pack_batch(const mvllm_pack_args* args, void* stream) {
  clear_error();
  return pack_batch(args, nullptr, stream);
}

extern "C" int mvllm_pack_batch_rows(const mvllm_pack_args* args, const mvllm_block_rows* rows,
                                     void* stream) {
  clear_error();
  if (!rows) return fail(MVLLM_ERR_INVALID, "block rows are null");
  return pack_batch(args, rows, stream);
}
