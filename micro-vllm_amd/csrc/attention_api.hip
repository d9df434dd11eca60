// C-ABI entry points of ragged paged attention: validation, workspace
// sizing and dispatch to the decode / prefill / generic kernels.
#include <cmath>
#include <cstdlib>
#include <cstring>
#include <mutex>

#include "worklists.h"

namespace mvllm {

int device_cu_count() {
  static std::mutex mu;
  static int cached[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  std::lock_guard<std::mutex> lock(mu);
  if (cached[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess ||
        cus <= 0)
      cus = 256;
    cached[dev] = cus;
  }
  return cached[dev];
}

namespace {

// Split size (tokens) of the split-KV decode partition. It depends only on
// shapes so that the workspace can be sized before a graph is captured.
int32_t decode_split_tokens(int64_t num_requests, int64_t max_context) {
  if (const char* env = std::getenv("MVLLM_DECODE_SPLIT")) {
    const long v = std::strtol(env, nullptr, 10);
    if (v >= 16 && v % 16 == 0 && v <= (1 << 20)) return static_cast<int32_t>(v);
  }
  // Aim for roughly 2 (request, split) items per CU when every request
  // reaches half of the table's reach; never below 64 tokens per split.
  // (The sorted decode work list balances the grid; fewer, longer items
  // spend less on dispatch and per-item setup: 1,024-token splits on the
  // 256-sequence Qwen3 batch ran at 357-361 us against 371 us for 512.)
  const int64_t target_items = 2LL * device_cu_count();
  const int64_t est_tokens = num_requests * (max_context / 2 > 16 ? max_context / 2 : 16);
  int64_t split = (est_tokens + target_items - 1) / target_items;
  split = (split + 15) / 16 * 16;
  if (split < 64) split = 64;
  // The pipelined decode kernel reads a split's block ids once, two 16-token
  // tiles per lane, so it takes splits of up to 2048 tokens; longer splits
  // would fall back to the general kernel, which streams ~15% slower
  // (64 contexts of 8k-33k tokens: 916 vs 1097 us).
  if (split > 2048) split = 2048;
  return static_cast<int32_t>(split);
}

struct DecodeLayout {
  int32_t split_tokens;
  int32_t max_splits;
  int64_t acc_bytes;
  int64_t ml_bytes;
  int64_t items_bytes;  // prefill work list: one 32-byte record per slot, N / 8 + R slots at most
  int64_t decode_items_bytes;  // decode work list: one 32-byte record per (request, split)
  int64_t decode_req_bytes;  // per request (query token, splits) for the combine kernel
  int64_t total() const { return acc_bytes + ml_bytes + items_bytes + decode_items_bytes + decode_req_bytes; }
};

DecodeLayout decode_layout(const mvllm_batch* b, int64_t num_q_heads, int64_t head_dim) {
  DecodeLayout d;
  const int64_t reach = b->block_table_width * b->block_size;
  d.split_tokens = decode_split_tokens(b->num_requests, reach);
  // Visible ranges start at a 16-aligned base at most 15 tokens early.
  const int64_t splits = (reach + 15 + d.split_tokens) / d.split_tokens;
  d.max_splits = static_cast<int32_t>(splits < 1 ? 1 : splits);
  const int64_t items = b->num_requests * d.max_splits * num_q_heads;
  d.acc_bytes = (items * head_dim * 4 + 255) / 256 * 256;
  d.ml_bytes = (items * 8 + 255) / 256 * 256;
  // Prefill query blocks hold T = 128 / G >= 8 tokens.
  d.items_bytes = ((b->num_tokens / 8 + b->num_requests) * static_cast<int64_t>(sizeof(PrefillItem)) + 255) / 256 * 256;
  d.decode_items_bytes = (b->num_requests * d.max_splits * static_cast<int64_t>(sizeof(DecodeItem)) + 255) / 256 * 256;
  d.decode_req_bytes = (b->num_requests * 8 + 255) / 256 * 256;
  return d;
}

int check_tensor(const mvllm_tensor3* t, const char* name) {
  if (!t) return fail(MVLLM_ERR_INVALID, "%s descriptor is null", name);
  if (dtype_bytes(t->dtype) == 0) return fail(MVLLM_ERR_UNSUPPORTED, "%s has unsupported dtype", name);
  for (int i = 0; i < 3; ++i)
    if (t->size[i] < 0 || t->stride[i] < 0)
      return fail(MVLLM_ERR_INVALID, "%s has a negative size or stride", name);
  if (t->size[0] > 0 && t->size[1] > 0 && t->size[2] > 0 && !t->data)
    return fail(MVLLM_ERR_INVALID, "%s data pointer is null", name);
  return MVLLM_OK;
}

int check_batch(const mvllm_batch* b, const mvllm_kv_cache* c) {
  if (!b) return fail(MVLLM_ERR_INVALID, "batch is null");
  if (b->num_tokens < 0 || b->num_requests < 0 || b->block_table_width < 0)
    return fail(MVLLM_ERR_INVALID, "negative batch size");
  if (b->block_size != c->block_size)
    return fail(MVLLM_ERR_INVALID, "metadata block_size %lld != cache block_size %lld",
                (long long)b->block_size, (long long)c->block_size);
  if (!b->query_start_locations) return fail(MVLLM_ERR_INVALID, "query_start_locations is null");
  if (b->num_tokens > 0 && (!b->query_positions || !b->query_context_start_positions))
    return fail(MVLLM_ERR_INVALID, "query_positions/context starts are null");
  if (b->num_requests > 0 && (!b->context_lengths || (b->block_table_width > 0 && !b->block_table)))
    return fail(MVLLM_ERR_INVALID, "context_lengths/block_table are null");
  return MVLLM_OK;
}

bool vec16(int64_t stride_elems, int64_t esize) { return (stride_elems * esize) % 16 == 0; }

}  // namespace
}  // namespace mvllm

using namespace mvllm;

extern "C" int64_t mvllm_attention_workspace_bytes(const mvllm_batch* batch, int64_t num_q_heads,
                                                   int64_t head_dim) {
  if (!batch || num_q_heads <= 0 || head_dim <= 0 || batch->num_requests <= 0 ||
      batch->block_size <= 0)
    return 0;
  return decode_layout(batch, num_q_heads, head_dim).total();
}

namespace mvllm {
namespace {

// A second stream per device for the prefill launch of a mixed batch: the
// MFMA-bound prefill kernel then runs beside the HBM-bound decode kernel
// instead of after it (a CU holds one workgroup of each). Default priority,
// non-blocking; created on the first eager call and never destroyed. The
// caller's stream forks to it after the KV write and joins it before the
// call returns, so the call behaves like one launch sequence on the
// caller's stream (and a graph capture records two branches). Calls are
// expected from one host thread at a time per device, as the operator's.
struct SideStream {
  hipStream_t stream = nullptr;
  hipEvent_t fork = nullptr, join = nullptr;
};

SideStream* side_stream(hipStream_t caller) {
  if (const char* env = std::getenv("MVLLM_PREFILL_CONCURRENT"))
    if (std::atoi(env) == 0) return nullptr;
  static std::mutex mu;
  static SideStream per_device[64];
  // The caller's stream decides the device (the null stream: the current one).
  int dev = 0;
  if (caller ? hipStreamGetDevice(caller, &dev) != hipSuccess : hipGetDevice(&dev) != hipSuccess) return nullptr;
  if (dev < 0 || dev >= 64) return nullptr;
  std::lock_guard<std::mutex> lock(mu);
  SideStream& ss = per_device[dev];
  if (!ss.stream) {
    // Creating streams or events during a graph capture may be refused:
    // such a call stays on the caller's stream.
    hipStreamCaptureStatus status = hipStreamCaptureStatusNone;
    if (hipStreamIsCapturing(caller, &status) != hipSuccess || status != hipStreamCaptureStatusNone) return nullptr;
    int current = 0;
    if (hipGetDevice(&current) != hipSuccess) return nullptr;
    if (current != dev && hipSetDevice(dev) != hipSuccess) return nullptr;
    hipStream_t st = nullptr;
    hipEvent_t f = nullptr, j = nullptr;
    bool ok = hipStreamCreateWithFlags(&st, hipStreamNonBlocking) == hipSuccess;
    ok = ok && hipEventCreateWithFlags(&f, hipEventDisableTiming) == hipSuccess;
    ok = ok && hipEventCreateWithFlags(&j, hipEventDisableTiming) == hipSuccess;
    if (current != dev) (void)hipSetDevice(current);
    if (!ok) {
      if (st) (void)hipStreamDestroy(st);
      if (f) (void)hipEventDestroy(f);
      return nullptr;
    }
    ss.stream = st;
    ss.fork = f;
    ss.join = j;
  }
  return &ss;
}

// When the one-launch attention step replaces the separate decode and
// prefill launches. MVLLM_STEP_KERNEL: 0 never, 1 for batches without the
// max_query_len hint only, 2 (default) for every batch that may hold prefill
// work. MVLLM_STEP_ORDER=prefill puts the prefill workgroups first in the
// grid. Decode first is the default: the decode workgroups fill the chip,
// and the MFMA-bound prefill workgroups take the slots that the decode
// grid's tail leaves idle. On the Llama-3 mixed batch (8 chunks of 512 and
// 248 decodes) that step took 770 us, against 819 us with prefill first,
// 777 us with the prefill kernel on a second stream and 804 us serially.
struct StepPolicy {
  int mode = 2;
  bool prefill_first = false;
};

StepPolicy step_policy() {
  StepPolicy p;
  if (const char* env = std::getenv("MVLLM_STEP_KERNEL")) {
    const int v = std::atoi(env);
    if (v >= 0 && v <= 2) p.mode = v;
  }
  if (const char* env = std::getenv("MVLLM_STEP_ORDER")) p.prefill_first = std::strcmp(env, "prefill") == 0;
  return p;
}

// The fused prologue of a forward: workgroup 0 builds the decode work list
// and the per-request table, workgroup 1 (when the batch may hold
// multi-query requests) the prefill work list, and every later workgroup
// copies the K/V rows of `rows_per_wg` tokens into their cache slots. One
// launch instead of three: the lists depend only on the metadata, never on
// the cache, so they may be built while the rows are written.
constexpr int kPrologueThreads = 1024;
static_assert(kPrologueThreads == kDecodeListThreads && kPrologueThreads == kItemThreads,
              "the list builders run on one full prologue workgroup");

__global__ __launch_bounds__(kPrologueThreads) void forward_prologue_kernel(AttnArgs a, KvRowArgs kv,
                                                                            int32_t lg_tok, int32_t lists,
                                                                            int32_t rows_per_wg) {
  const int64_t wg = blockIdx.x;
  if (wg < lists) {
    if (wg == 0) build_decode_list(a);
    else build_prefill_list(a, lg_tok);
    return;
  }
  const int span = kPrologueThreads / rows_per_wg;  // threads per token row
  const int64_t token = (wg - lists) * rows_per_wg + threadIdx.x / span;
  if (token < a.num_tokens) copy_kv_row(kv, token, threadIdx.x % span, span);
}

// Batch and cache fields of the kernel arguments.
void fill_batch_args(AttnArgs& a, const mvllm_batch* batch, const mvllm_kv_cache* cache, int64_t Hq) {
  a.cache = cache->data;
  for (int i = 0; i < 5; ++i) a.c_s[i] = cache->stride[i];
  a.positions = batch->query_positions;
  a.cstarts = batch->query_context_start_positions;
  a.qsl = batch->query_start_locations;
  a.lengths = batch->context_lengths;
  a.table = batch->block_table;
  a.t_s0 = batch->block_table_stride[0];
  a.t_s1 = batch->block_table_stride[1];
  a.width = batch->block_table_width;
  a.num_tokens = batch->num_tokens;
  a.num_requests = batch->num_requests;
  a.num_blocks = cache->num_blocks;
  a.block_size = cache->block_size;
  a.page_shift = -1;
  if (cache->block_size >= 16 && cache->block_size % 16 == 0) {
    const int64_t pages = cache->block_size / 16;
    if ((pages & (pages - 1)) == 0) a.page_shift = __builtin_ctzll(static_cast<unsigned long long>(pages));
  }
  a.num_q_heads = static_cast<int32_t>(Hq);
  a.num_kv_heads = static_cast<int32_t>(cache->num_kv_heads);
  a.group = static_cast<int32_t>(Hq / cache->num_kv_heads);
  a.head_dim = static_cast<int32_t>(cache->head_dim);
}

// The cache-side conditions of the MFMA kernels (the query and output add
// their own): a plan is built whenever a planned call can take that path.
bool fast_cache(const mvllm_kv_cache* cache, int64_t group) {
  const int32_t dtype = cache->dtype;
  const int64_t es = dtype_bytes(dtype);
  return (dtype == MVLLM_DTYPE_BF16 || dtype == MVLLM_DTYPE_F16) && cache->head_dim == 128 && group <= 16 &&
         cache->stride[4] == 1 && cache->stride[3] == cache->head_dim && vec16(cache->stride[0], es) &&
         vec16(cache->stride[1], es) && vec16(cache->stride[2], es) && aligned16(cache->data);
}

// The MFMA decode / prefill path (with work lists) applies: 16-byte aligned
// rows of query, output and cache, head_dim 128, a supported group size and
// at least one request; otherwise the generic kernel runs.
bool attention_fast_path(const mvllm_tensor3* query, const mvllm_kv_cache* cache, const mvllm_tensor3* out,
                         const mvllm_batch* batch) {
  if (!query || !cache || !out || !batch || batch->num_requests <= 0) return false;
  const int64_t Hkv = cache->num_kv_heads;
  if (Hkv <= 0 || query->size[1] % Hkv != 0) return false;
  const int64_t es = dtype_bytes(query->dtype);
  return fast_cache(cache, query->size[1] / Hkv) && query->stride[2] == 1 && vec16(query->stride[0], es) &&
         vec16(query->stride[1], es) && aligned16(query->data) && out->stride[2] == 1 &&
         vec16(out->stride[0], es) && vec16(out->stride[1], es) && aligned16(out->data);
}

// Split-KV partials, work lists and the per-request table in the workspace.
int bind_workspace(AttnArgs& a, const mvllm_batch* batch, int64_t Hq, int64_t D, void* workspace,
                   int64_t workspace_bytes) {
  const DecodeLayout d = decode_layout(batch, Hq, D);
  if (workspace_bytes < d.total() || (!workspace && d.total() > 0))
    return fail(MVLLM_ERR_WORKSPACE, "workspace of %lld bytes is smaller than the %lld required",
                (long long)workspace_bytes, (long long)d.total());
  if (!aligned16(workspace)) return fail(MVLLM_ERR_INVALID, "workspace must be 16-byte aligned");
  char* const w = static_cast<char*>(workspace);
  a.split_tokens = d.split_tokens;
  a.max_splits = d.max_splits;
  a.decode_only = batch->max_query_len == 1 ? 1 : 0;
  a.ws_acc = reinterpret_cast<float*>(w);
  a.ws_ml = reinterpret_cast<float2*>(w + d.acc_bytes);
  a.items = reinterpret_cast<PrefillItem*>(w + d.acc_bytes + d.ml_bytes);
  a.decode_items = reinterpret_cast<DecodeItem*>(w + d.acc_bytes + d.ml_bytes + d.items_bytes);
  a.decode_req = reinterpret_cast<int2*>(w + d.acc_bytes + d.ml_bytes + d.items_bytes + d.decode_items_bytes);
  return MVLLM_OK;
}

int attention_plan(const mvllm_batch* batch, int64_t Hq, const mvllm_kv_cache* cache, void* workspace,
                   int64_t workspace_bytes, void* stream) {
  if (!cache || !cache->data) return fail(MVLLM_ERR_INVALID, "cache is null");
  if (int rc = check_batch(batch, cache)) return rc;
  const int64_t Hkv = cache->num_kv_heads, D = cache->head_dim;
  if (Hq <= 0 || Hkv <= 0 || Hq % Hkv != 0)
    return fail(MVLLM_ERR_INVALID, "query heads %lld not a multiple of KV heads %lld", (long long)Hq,
                (long long)Hkv);
  if (batch->num_tokens == 0 || batch->num_requests == 0 || !fast_cache(cache, Hq / Hkv)) return MVLLM_OK;
  AttnArgs a = {};
  fill_batch_args(a, batch, cache, Hq);
  if (int rc = bind_workspace(a, batch, Hq, D, workspace, workspace_bytes)) return rc;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (int rc = launch_decode_lists(a, s)) return rc;
  if (batch->max_query_len == 1 || !prefill_supported(a, cache->dtype)) return MVLLM_OK;
  return launch_prefill_lists(a, s);
}

int paged_attention(const mvllm_tensor3* query, const mvllm_kv_cache* cache,
                    const mvllm_batch* batch, const mvllm_tensor3* out, float scale,
                    void* workspace, int64_t workspace_bytes, const mvllm_timing* timing,
                    void* stream, bool planned = false, bool single_stream = false,
                    const KvRowArgs* fused_kv = nullptr) {
  if (int rc = check_tensor(query, "query")) return rc;
  if (int rc = check_tensor(out, "out")) return rc;
  if (!cache || !cache->data) return fail(MVLLM_ERR_INVALID, "cache is null");
  if (int rc = check_batch(batch, cache)) return rc;
  const int32_t dtype = query->dtype;
  if (cache->dtype != dtype || out->dtype != dtype)
    return fail(MVLLM_ERR_INVALID, "query/cache/out dtypes differ (%s/%s/%s)", dtype_name(dtype),
                dtype_name(cache->dtype), dtype_name(out->dtype));
  const int64_t N = batch->num_tokens;
  const int64_t Hq = query->size[1], D = query->size[2], Hkv = cache->num_kv_heads;
  if (query->size[0] != N || out->size[0] != N || out->size[1] != Hq || out->size[2] != D)
    return fail(MVLLM_ERR_INVALID, "query/out shapes do not match [%lld, %lld, %lld]",
                (long long)N, (long long)Hq, (long long)D);
  if (cache->head_dim != D) return fail(MVLLM_ERR_INVALID, "cache head_dim %lld != query head_dim %lld",
                                        (long long)cache->head_dim, (long long)D);
  if (Hkv <= 0 || Hq % Hkv != 0)
    return fail(MVLLM_ERR_INVALID, "query heads %lld not a multiple of KV heads %lld",
                (long long)Hq, (long long)Hkv);
  if (N == 0) return MVLLM_OK;
  if (Hq > 65535 || D > 65535) return fail(MVLLM_ERR_INVALID, "head count or head_dim too large");

  AttnArgs a = {};
  fill_batch_args(a, batch, cache, Hq);
  a.q = query->data;
  a.q_s0 = query->stride[0]; a.q_s1 = query->stride[1]; a.q_s2 = query->stride[2];
  a.out = out->data;
  a.o_s0 = out->stride[0]; a.o_s1 = out->stride[1]; a.o_s2 = out->stride[2];
  a.scale_log2 = scale * 1.4426950408889634f;  // log2(e)
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);

  const bool fast = attention_fast_path(query, cache, out, batch);
  if (!fast) {
    if (fused_kv) {
      // Only the rows: the generic kernel needs no work lists.
      const int64_t blocks = ceil_div(N, 1);
      hipLaunchKernelGGL(forward_prologue_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kPrologueThreads), 0, s,
                         a, *fused_kv, 0, 0, 1);
      MVLLM_LAUNCH_CHECK("forward_prologue_kernel");
    }
    a.mode = 0;
    return launch_generic(a, dtype, s);
  }
  if (int rc = bind_workspace(a, batch, Hq, D, workspace, workspace_bytes)) return rc;
  a.lists_ready = planned ? 1 : 0;
  const bool wants_prefill = batch->max_query_len != 1 && prefill_supported(a, dtype);
  if (fused_kv) {
    // The step's K/V rows and the work lists in one launch; the decode and
    // prefill launches below then find the lists ready.
    const int64_t chunks2 = 2 * static_cast<int64_t>(fused_kv->chunks);
    int32_t rows_per_wg = 1;
    while (rows_per_wg < 64 && 2 * rows_per_wg * chunks2 <= kPrologueThreads) rows_per_wg *= 2;
    if (chunks2 > kPrologueThreads) rows_per_wg = 1;
    const int32_t lists = a.lists_ready ? 0 : (wants_prefill ? 2 : 1);
    if (a.lists_ready) {
      // Lists were planned: only the rows (the planned decode launch checks its reach).
    } else if (a.width * a.block_size > INT32_MAX || a.num_tokens > INT32_MAX) {
      return fail(MVLLM_ERR_UNSUPPORTED, "decode positions beyond 2^31 are not supported");
    }
    const int64_t blocks = lists + ceil_div(N, rows_per_wg);
    if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "prologue grid too large");
    hipLaunchKernelGGL(forward_prologue_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kPrologueThreads), 0, s,
                       a, *fused_kv, static_cast<int32_t>(prefill_lg_tok(a)), lists, rows_per_wg);
    MVLLM_LAUNCH_CHECK("forward_prologue_kernel");
    a.lists_ready = 1;
  }
  hipEvent_t ds = timing ? static_cast<hipEvent_t>(timing->decode_start) : nullptr;
  hipEvent_t de = timing ? static_cast<hipEvent_t>(timing->decode_stop) : nullptr;
  hipEvent_t ps = timing ? static_cast<hipEvent_t>(timing->prefill_start) : nullptr;
  hipEvent_t pe = timing ? static_cast<hipEvent_t>(timing->prefill_stop) : nullptr;
  // A batch known to hold only single-query requests needs no prefill launch.
  if (wants_prefill) {
    // The one-launch step runs both kinds of workgroup in one grid. Without
    // the hint, a decode-only batch then pays only for empty prefill
    // workgroups at the grid's tail instead of a second launch. A caller that
    // times the prefill kernel on its own gets the separate launches; the
    // decode events then bracket the step kernel.
    const bool hinted = batch->max_query_len > 1;
    const bool prefill_timed = timing && (timing->prefill_start || timing->prefill_stop);
    const StepPolicy policy = step_policy();
    if (!prefill_timed && (policy.mode == 2 || (policy.mode == 1 && !hinted)) && decode_step_eligible(a))
      return launch_step(a, dtype, policy.prefill_first, s, ds, de);
    // A fork and join cost ~10 us: the prefill moves to the side stream only
    // when the hint says that the batch holds multi-query requests.
    SideStream* side = batch->max_query_len > 1 && !single_stream ? side_stream(s) : nullptr;
    hipStream_t pst = s;
    if (side) {
      MVLLM_HIP_TRY(hipEventRecord(side->fork, s));
      MVLLM_HIP_TRY(hipStreamWaitEvent(side->stream, side->fork, 0));
      pst = side->stream;
    }
    // The prefill goes first so that its workgroups are queued before the
    // decode grid fills the chip. Both branches are joined even on error.
    int rc = launch_prefill(a, dtype, pst, ps, pe);
    if (rc == MVLLM_OK) rc = launch_decode(a, dtype, s, ds, de);
    if (side) {
      MVLLM_HIP_TRY(hipEventRecord(side->join, side->stream));
      MVLLM_HIP_TRY(hipStreamWaitEvent(s, side->join, 0));
    }
    return rc;
  }
  if (int rc = launch_decode(a, dtype, s, ds, de)) return rc;
  if (batch->max_query_len == 1) return MVLLM_OK;
  a.mode = 1;
  return launch_generic(a, dtype, s);
}

int attention_forward(const mvllm_tensor3* query, const mvllm_tensor3* key,
                      const mvllm_tensor3* value, const mvllm_kv_cache* cache,
                      const mvllm_batch* batch, const mvllm_tensor3* out, float scale,
                      void* workspace, int64_t workspace_bytes, const mvllm_timing* timing,
                      void* stream, bool single_stream = false) {
  if (!batch) return fail(MVLLM_ERR_INVALID, "batch is null");
  if (batch->num_tokens > 0) {
    if (!batch->slot_mapping) return fail(MVLLM_ERR_INVALID, "slot_mapping is null");
    KvRowArgs rows;
    bool vectorised = false;
    if (int rc = kv_write_prepare(key, value, cache, batch->slot_mapping, batch->num_tokens, &rows, &vectorised))
      return rc;
    // The fused prologue needs the attention's MFMA path (the work lists)
    // and 16-byte rows; everything else writes the rows first, on its own.
    if (vectorised && attention_fast_path(query, cache, out, batch))
      return paged_attention(query, cache, batch, out, scale, workspace, workspace_bytes, timing, stream, false,
                             single_stream, &rows);
    if (int rc = mvllm_kv_write(key, value, cache, batch->slot_mapping, batch->num_tokens, stream))
      return rc;
  }
  return paged_attention(query, cache, batch, out, scale, workspace, workspace_bytes, timing,
                         stream, false, single_stream);
}

}  // namespace
}  // namespace mvllm

// ---- the allocation-free entry point ------------------------------------------
//
// mvllm_attention_forward_noalloc takes its workspace (split-KV partials and
// work lists) from this file-scope device array instead of a caller
// argument. Each device holds its own copy from the library's first use on
// it until the process ends. In host code `scratch` names a host-side
// stand-in, never the device memory: its device address comes from
// hipGetSymbolAddress, once per device, and only that address is passed on.
static __device__ __align__(256) unsigned char scratch[MVLLM_NOALLOC_SCRATCH_BYTES];

namespace mvllm {
namespace {

// Device address of `scratch` on the device that `stream` belongs to,
// looked up on the first call for that device (with it current) and kept.
// The lookup may load the library's code on that device, which a stream
// capture must not record: a first call made while `stream` is capturing is
// refused (MVLLM_ERR_INVALID) before any runtime call but the capture query.
int scratch_address(hipStream_t stream, void** out) {
  static std::mutex mu;
  static void* per_device[64] = {nullptr};
  int dev = 0;
  if (stream) {
    MVLLM_HIP_TRY(hipStreamGetDevice(stream, &dev));
  } else {
    MVLLM_HIP_TRY(hipGetDevice(&dev));
  }
  if (dev < 0 || dev >= 64) return fail(MVLLM_ERR_INVALID, "device %d out of range", dev);
  std::lock_guard<std::mutex> lock(mu);
  if (!per_device[dev]) {
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    MVLLM_HIP_TRY(hipStreamIsCapturing(stream, &capture));
    if (capture != hipStreamCaptureStatusNone)
      return fail(MVLLM_ERR_INVALID,
                  "mvllm_attention_forward_noalloc: the first call on device %d is under stream capture; "
                  "call it once outside capture on that device (it looks up its workspace then)", dev);
    int current = 0;
    MVLLM_HIP_TRY(hipGetDevice(&current));
    if (current != dev) MVLLM_HIP_TRY(hipSetDevice(dev));
    void* p = nullptr;
    const hipError_t status = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (current != dev) MVLLM_HIP_TRY(hipSetDevice(current));
    if (status != hipSuccess || !p)
      return fail(MVLLM_ERR_HIP, "hipGetSymbolAddress(scratch) failed on device %d: %s", dev,
                  hipGetErrorString(status));
    per_device[dev] = p;
  }
  *out = per_device[dev];
  return MVLLM_OK;
}

}  // namespace
}  // namespace mvllm

extern "C" int mvllm_paged_attention(const mvllm_tensor3* query, const mvllm_kv_cache* cache,
                                     const mvllm_batch* batch, const mvllm_tensor3* out,
                                     float scale, void* workspace, int64_t workspace_bytes,
                                     void* stream) {
  clear_error();
  return paged_attention(query, cache, batch, out, scale, workspace, workspace_bytes, nullptr,
                         stream);
}

extern "C" int mvllm_attention_plan(const mvllm_batch* batch, int64_t num_q_heads,
                                    const mvllm_kv_cache* cache, void* workspace,
                                    int64_t workspace_bytes, void* stream) {
  clear_error();
  return attention_plan(batch, num_q_heads, cache, workspace, workspace_bytes, stream);
}

extern "C" int mvllm_paged_attention_planned(const mvllm_tensor3* query, const mvllm_kv_cache* cache,
                                             const mvllm_batch* batch, const mvllm_tensor3* out,
                                             float scale, void* workspace, int64_t workspace_bytes,
                                             void* stream) {
  clear_error();
  return paged_attention(query, cache, batch, out, scale, workspace, workspace_bytes, nullptr, stream,
                         true);
}

extern "C" int mvllm_attention_forward(const mvllm_tensor3* query, const mvllm_tensor3* key,
                                       const mvllm_tensor3* value, const mvllm_kv_cache* cache,
                                       const mvllm_batch* batch, const mvllm_tensor3* out,
                                       float scale, void* workspace, int64_t workspace_bytes,
                                       void* stream) {
  clear_error();
  return attention_forward(query, key, value, cache, batch, out, scale, workspace,
                           workspace_bytes, nullptr, stream);
}

extern "C" int mvllm_attention_forward_timed(const mvllm_tensor3* query,
                                             const mvllm_tensor3* key,
                                             const mvllm_tensor3* value,
                                             const mvllm_kv_cache* cache,
                                             const mvllm_batch* batch, const mvllm_tensor3* out,
                                             float scale, void* workspace,
                                             int64_t workspace_bytes, const mvllm_timing* timing,
                                             void* stream) {
  clear_error();
  return attention_forward(query, key, value, cache, batch, out, scale, workspace,
                           workspace_bytes, timing, stream);
}

extern "C" int mvllm_attention_forward_noalloc(const mvllm_tensor3* query,
                                               const mvllm_tensor3* key,
                                               const mvllm_tensor3* value,
                                               const mvllm_kv_cache* cache,
                                               const mvllm_batch* batch,
                                               const mvllm_tensor3* out, float scale,
                                               void* stream) {
  clear_error();
  if (!query || !batch || !cache) return fail(MVLLM_ERR_INVALID, "query, batch or cache is null");
  const int64_t need = mvllm_attention_workspace_bytes(batch, query->size[1], query->size[2]);
  if (need > MVLLM_NOALLOC_SCRATCH_BYTES)
    return fail(MVLLM_ERR_WORKSPACE,
                "batch needs %lld bytes of workspace; mvllm_attention_forward_noalloc holds at most %lld "
                "(use mvllm_attention_forward with a caller workspace)",
                (long long)need, (long long)MVLLM_NOALLOC_SCRATCH_BYTES);
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  void* ws = nullptr;
  if (int rc = scratch_address(s, &ws)) return rc;
  // Everything stays on the caller's stream: no side stream is created.
  return attention_forward(query, key, value, cache, batch, out, scale, ws, MVLLM_NOALLOC_SCRATCH_BYTES,
                           nullptr, stream, true);
}
