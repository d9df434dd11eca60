/*
 * mvllm_amd.h — C ABI of the MI355X (gfx950) ragged paged-attention library.
 *
 * The library implements the tensor work of micro-vLLM's attention operator
 * (src/micro_vllm/attention/operators/base.py:30-40) as hand-written HIP
 * kernels: the paged KV-cache write, ragged causal GQA attention over the
 * paged cache (split-KV decode and MFMA prefill), a bit-exact block gather,
 * and the ragged-batch packing that the reference ModelRunner performs in
 * Python loops.
 *
 * Conventions
 *  - Every pointer is a device pointer unless noted; every size and stride is
 *    in elements (not bytes) and is a plain int64_t.
 *  - `stream` is a hipStream_t passed as void* (NULL = the null stream).
 *    Calls only enqueue work: nothing synchronises with the host, no device
 *    memory is allocated, so every entry point may be recorded into a HIP
 *    graph. A batch that may hold multi-query requests runs its decode and
 *    prefill workgroups in one launch on `stream` (the step kernel). Only a
 *    caller that times the prefill kernel on its own (mvllm_timing's prefill
 *    events), or a decode shape the step kernel does not take, gets separate
 *    launches; with max_query_len > 1 the prefill kernel then runs on a
 *    second, library-owned stream (one per device, default priority, created
 *    by the first call made outside a graph capture), forked from and joined
 *    back into `stream` within the call. MVLLM_PREFILL_CONCURRENT=0 keeps all
 *    work on `stream`; MVLLM_STEP_KERNEL=0 turns the step kernel off.
 *  - Return value: 0 on success, a negative MVLLM_ERR_* code on failure;
 *    mvllm_last_error() then describes the failure (thread-local text).
 *  - Index tensors are int64, as in the reference (AttentionMetadata,
 *    attention.py:12-28). Padding conventions follow the reference: slot -1
 *    writes nothing; a request with an empty query range does nothing;
 *    tokens outside every request get zero output; block-table entries past a
 *    request's visible context are never read.
 *  - The paged cache is the reference's tensor of shape
 *    (2, num_blocks, block_size, num_kv_heads, head_dim): plane 0 holds keys,
 *    plane 1 values (model_runner.py:688-703).
 */
#ifndef MVLLM_AMD_H
#define MVLLM_AMD_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

/* Element types (torch.float32 / torch.float16 / torch.bfloat16). */
enum {
  MVLLM_DTYPE_F32 = 0,
  MVLLM_DTYPE_F16 = 1,
  MVLLM_DTYPE_BF16 = 2
};

/* Status codes. */
enum {
  MVLLM_OK = 0,
  MVLLM_ERR_INVALID = -1,     /* bad shape, stride, pointer or size */
  MVLLM_ERR_UNSUPPORTED = -2, /* dtype / geometry the library does not handle */
  MVLLM_ERR_HIP = -3,         /* a HIP runtime call failed */
  MVLLM_ERR_WORKSPACE = -4    /* workspace smaller than required */
};

/* Attention visibility kinds (spec.py:13-51). */
enum {
  MVLLM_SPEC_FULL = 0,           /* start = 0 */
  MVLLM_SPEC_SLIDING_WINDOW = 1, /* start = max(0, pos - window + 1) */
  MVLLM_SPEC_CHUNKED_LOCAL = 2   /* start = (pos / chunk) * chunk */
};

/* A strided [tokens, heads, dim] device tensor (query, key, value, output). */
typedef struct mvllm_tensor3 {
  void* data;
  int32_t dtype;
  int32_t reserved;
  int64_t size[3];
  int64_t stride[3];
} mvllm_tensor3;

/* The paged cache (2, num_blocks, block_size, num_kv_heads, head_dim). */
typedef struct mvllm_kv_cache {
  void* data;
  int32_t dtype;
  int32_t reserved;
  int64_t num_blocks;
  int64_t block_size;
  int64_t num_kv_heads;
  int64_t head_dim;
  int64_t stride[5];
} mvllm_kv_cache;

/* AttentionMetadata (attention.py:12-28) as device int64 arrays. */
typedef struct mvllm_batch {
  const int64_t* query_positions;               /* [num_tokens] */
  const int64_t* query_context_start_positions; /* [num_tokens] */
  const int64_t* query_start_locations;         /* [num_requests + 1] */
  const int64_t* context_lengths;               /* [num_requests] */
  const int64_t* block_table;                   /* [num_requests, width] */
  const int64_t* slot_mapping;                  /* [num_tokens] */
  int64_t num_tokens;
  int64_t num_requests;
  int64_t block_table_width;
  int64_t block_table_stride[2];
  int64_t block_size;
  int64_t max_query_len; /* largest query count of a request, if the caller
                            knows it (<= 0: unknown). 1 lets a decode-only
                            batch skip the prefill launch; the rows of any
                            request with another query count then come back
                            NaN. */
} mvllm_batch;

/*
 * Scatter key/value rows into their physical cache slots:
 *   cache[0|1, slot / block_size, slot % block_size, h, :] = key|value[t, h, :]
 * Bit-exact copy; slot < 0 (padding) and slot >= num_blocks * block_size
 * write nothing. Slots must be distinct (the KV-cache manager guarantees it).
 * Replaces write_kv_cache (reference.py:84-98) and triton_write_kv_cache /
 * _write_kv_cache_kernel (triton_paged.py:293-325, 11-68).
 */
int mvllm_kv_write(const mvllm_tensor3* key, const mvllm_tensor3* value,
                   const mvllm_kv_cache* cache, const int64_t* slot_mapping,
                   int64_t num_tokens, void* stream);

/*
 * Bytes of device workspace mvllm_paged_attention / mvllm_attention_forward
 * need for this batch geometry: the split-KV partial results of the decode
 * kernel and the decode and prefill work lists, which the library writes
 * before it reads them (the caller need not initialise the workspace).
 * Decode positions must stay below 2^31 (block-table width * block size).
 * Depends only on
 * shapes, never on device data, so it can be sized before graph capture.
 */
int64_t mvllm_attention_workspace_bytes(const mvllm_batch* batch,
                                        int64_t num_q_heads, int64_t head_dim);

/*
 * Ragged causal GQA attention over the paged cache (the cache must already
 * hold every visible key, including the batch's own tokens). For query t of
 * request r, key positions [max(start(t), start(first query of r)),
 * min(pos(t), context_length(r) - 1)] are visible; softmax(q.k * scale) . v
 * in fp32, written in out's dtype. Tokens outside every request get zeros.
 * Replaces the attention part of ReferenceAttentionOperator.forward
 * (reference.py:26-81) and triton_paged_attention / _paged_attention_kernel
 * (triton_paged.py:328-389, 97-290).
 */
int mvllm_paged_attention(const mvllm_tensor3* query,
                          const mvllm_kv_cache* cache,
                          const mvllm_batch* batch, const mvllm_tensor3* out,
                          float scale, void* workspace,
                          int64_t workspace_bytes, void* stream);

/*
 * Writes the work lists of `batch` (the decode split list, the per-request
 * decode table and the prefill query-block list) into `workspace`, for
 * mvllm_paged_attention_planned. The workspace is sized by
 * mvllm_attention_workspace_bytes(batch, num_q_heads, head_dim) for the
 * cache's head_dim. No counterpart in the reference, whose operator runs per
 * layer (qwen.py:89-99): its callers are models whose layers share one batch
 * and one cache geometry, which then plan once per step instead of once per
 * layer (the lists depend only on the batch). Graph-capturable.
 */
int mvllm_attention_plan(const mvllm_batch* batch, int64_t num_q_heads,
                         const mvllm_kv_cache* cache, void* workspace,
                         int64_t workspace_bytes, void* stream);

/*
 * mvllm_paged_attention over the work lists that mvllm_attention_plan wrote
 * into the same workspace. The caller guarantees that the plan was made for
 * this batch, head count and cache geometry, and that nothing overwrote the
 * workspace since (calls in one stream may share it: each rewrites only the
 * split-KV partials). This is not checked; a mismatched plan gives wrong
 * results but every record field is range-checked before it is used as an
 * index.
 */
int mvllm_paged_attention_planned(const mvllm_tensor3* query,
                                  const mvllm_kv_cache* cache,
                                  const mvllm_batch* batch,
                                  const mvllm_tensor3* out, float scale,
                                  void* workspace, int64_t workspace_bytes,
                                  void* stream);

/*
 * The whole operator: mvllm_kv_write(key, value, slot_mapping) followed by
 * mvllm_paged_attention. Replaces AttentionOperator.forward
 * (base.py:30-40) as implemented by ReferenceAttentionOperator.forward
 * (reference.py:14-81) and TritonPagedAttentionOperator.forward
 * (triton_paged.py:395-418).
 */
int mvllm_attention_forward(const mvllm_tensor3* query,
                            const mvllm_tensor3* key,
                            const mvllm_tensor3* value,
                            const mvllm_kv_cache* cache,
                            const mvllm_batch* batch, const mvllm_tensor3* out,
                            float scale, void* workspace,
                            int64_t workspace_bytes, void* stream);

/*
 * Device workspace held by mvllm_attention_forward_noalloc: 32 MiB per device.
 * It covers the split-KV partials and work lists of batches such as 256
 * decodes over a 512-block table with 32 query heads (about 21 MB).
 */
#define MVLLM_NOALLOC_SCRATCH_BYTES (32LL * 1024 * 1024)

/*
 * mvllm_attention_forward without a workspace argument: for callers that
 * cannot allocate device memory (code under HIP graph capture that may not
 * grow a pool, tight serving loops, harnesses that forbid hipMalloc). No
 * counterpart in the reference. The workspace is a library-owned device
 * array of MVLLM_NOALLOC_SCRATCH_BYTES per device (its address is looked up
 * once per device on the first call there); the call allocates nothing and
 * runs all of its work on `stream` (no side stream). Graph capture: make the
 * first call on a device outside capture; a first call under capture is
 * refused with MVLLM_ERR_INVALID (the address lookup may load code), later
 * calls capture and replay like mvllm_attention_forward. A batch that needs more
 * workspace (mvllm_attention_workspace_bytes) is rejected with
 * MVLLM_ERR_WORKSPACE. Every call on one device shares that array: calls
 * that overlap on one device (other streams, other threads) race and give
 * wrong results. The array needs no initialisation: every call writes what
 * it reads.
 */
int mvllm_attention_forward_noalloc(const mvllm_tensor3* query,
                                    const mvllm_tensor3* key,
                                    const mvllm_tensor3* value,
                                    const mvllm_kv_cache* cache,
                                    const mvllm_batch* batch,
                                    const mvllm_tensor3* out, float scale,
                                    void* stream);

/*
 * Optional kernel timing for measurement: hipEvent_t handles (as void*,
 * NULL = not wanted) recorded on the launch stream immediately before and
 * after the decode kernel and the prefill kernel (hipExtLaunchKernel). With
 * prefill events set, the decode and prefill kernels are launched
 * separately; without them, the decode events bracket the step kernel when
 * that runs.
 */
typedef struct mvllm_timing {
  void* decode_start;
  void* decode_stop;
  void* prefill_start;
  void* prefill_stop;
} mvllm_timing;

/*
 * mvllm_attention_forward with per-kernel timing events. No counterpart in
 * the reference: it exists so a benchmark can time the dominant kernel of
 * a step on the stream it runs on.
 */
int mvllm_attention_forward_timed(const mvllm_tensor3* query,
                                  const mvllm_tensor3* key,
                                  const mvllm_tensor3* value,
                                  const mvllm_kv_cache* cache,
                                  const mvllm_batch* batch,
                                  const mvllm_tensor3* out, float scale,
                                  void* workspace, int64_t workspace_bytes,
                                  const mvllm_timing* timing, void* stream);

/*
 * Bit-exact gather of each request's visible K/V history into padded,
 * contiguous [num_requests, capacity, num_kv_heads, head_dim] buffers (same
 * dtype as the cache): row i of request r is the cache row of position
 * start(first query of r) + i, for i < context_length(r) - that start; rows
 * past it are left untouched. Replaces gather_kv_cache (reference.py:101-138);
 * the padded layout is the one of the reference's teaching gather kernel
 * (benchmarks/spike_triton_paged.py:52-174).
 */
int mvllm_gather_kv(const mvllm_kv_cache* cache, const mvllm_batch* batch,
                    int64_t capacity, void* out_key, void* out_value,
                    void* stream);

/*
 * Per-query visibility start for an attention spec:
 *   out[i] = start(positions[i]) for spec kind `spec_kind` with parameter
 *   `spec_parameter` (window size or chunk size; ignored for FULL).
 * Replaces the host loop in Attention.build_metadata (attention.py:68-75)
 * over AttentionSpec.context_start (spec.py:13-51).
 */
int mvllm_context_starts(const int64_t* positions, int64_t num_tokens,
                         int32_t spec_kind, int64_t spec_parameter,
                         int64_t* out, void* stream);

/*
 * Ragged-batch packing on the GPU. Input is a compact per-step payload in
 * device memory (int32, MVLLM_PACK_FIELDS values per request):
 *   request_info[r * 8 + 0] = num_computed_tokens
 *   request_info[r * 8 + 1] = num_scheduled_tokens
 *   request_info[r * 8 + 2] = number of block ids of request r (this group)
 *   request_info[r * 8 + 3] = 1 if the request requires sampling, else 0
 *   request_info[r * 8 + 4 .. 5] = scratch, overwritten by the call (the
 *                                  per-request prefix sums)
 *   request_info[r * 8 + 6] = the request's row of a device-resident block
 *                             table (mvllm_pack_batch_rows only)
 *   request_info[r * 8 + 7] = unused
 *   block_ids   = concatenation of every request's block ids (this group)
 *   token_ids   = concatenation of every request's input token ids (may be
 *                 NULL when input_ids is NULL)
 * Outputs (int64, NULL = not wanted) are written at the given capacities,
 * padded exactly as a captured graph expects (model_runner.py:78-122):
 *   input_ids[token_capacity]       (pad 0)
 *   positions[token_capacity]       (pad 0)
 *   context_starts[token_capacity]  (pad 0)
 *   query_start_locations[request_capacity + 1] (pad num_tokens)
 *   context_lengths[request_capacity]           (pad 0)
 *   block_table[request_capacity, block_table_width] (pad null_block_id)
 *   slot_mapping[token_capacity]    (pad -1; also -1 for a position whose
 *                                    logical block has no block id)
 *   sampling_rows[num_sampling]     (last flattened row of each sampling
 *                                    request, in request order)
 * With capacities equal to the actual sizes this is the unpadded output of
 * ModelRunner._flatten_model_input / _build_slot_mapping / _build_block_table
 * (model_runner.py:751-900) plus Attention.build_metadata's context starts.
 */
typedef struct mvllm_pack_args {
  int32_t* request_info;
  const int32_t* block_ids;
  const int32_t* token_ids;
  int64_t num_requests;
  int64_t num_tokens;
  int64_t num_block_ids;
  int64_t block_size;
  int64_t null_block_id;
  int32_t spec_kind;
  int32_t reserved;
  int64_t spec_parameter;
  int64_t token_capacity;
  int64_t request_capacity;
  int64_t block_table_width;
  int64_t* input_ids;
  int64_t* positions;
  int64_t* context_starts;
  int64_t* query_start_locations;
  int64_t* context_lengths;
  int64_t* block_table;
  int64_t* slot_mapping;
  int64_t* sampling_rows;
} mvllm_pack_args;

#define MVLLM_PACK_FIELDS 8

int mvllm_pack_batch(const mvllm_pack_args* args, void* stream);

/*
 * A device-resident copy of every live request's block ids, kept across
 * steps and updated by deltas (no counterpart in the reference, whose
 * ModelRunner rebuilds the table from full Python lists with one host-to-
 * device copy per request row every step, model_runner.py:871-900):
 *   rows[slot * width + i] = block id i of the request that owns `slot`;
 *   updates = num_updates records of 4 int32 each, (slot, first, count,
 *             offset): rows[slot * width + first + j] = block_ids[offset + j]
 *             for j < count, where block_ids is the pack call's payload.
 */
typedef struct mvllm_block_rows {
  int32_t* rows;
  int64_t num_slots;
  int64_t width;
  const int32_t* updates;
  int64_t num_updates;
} mvllm_block_rows;

/*
 * mvllm_pack_batch over a device-resident block table: the call first
 * applies `rows`' updates (args->block_ids / num_block_ids hold only the
 * updated ids), then packs as mvllm_pack_batch does, reading request r's
 * block ids from rows[request_info[r * 8 + 6] * width ...]
 * (request_info[r * 8 + 2] of them; a slot out of range or a list longer
 * than `width` is an error the kernels turn into null / -1 entries).
 * Single cache group per call. Replaces the per-step table rebuild of
 * ModelRunner._build_block_table / _build_slot_mapping (model_runner.py:
 * 833-900) for a caller that knows which block ids changed.
 */
int mvllm_pack_batch_rows(const mvllm_pack_args* args,
                          const mvllm_block_rows* rows, void* stream);

/*
 * Fused residual add + RMSNorm over `rows` rows of `dim` bf16/fp16 values
 * (dim <= 8192, strides in elements):
 *   if residual != NULL: h = round(residual + x), residual <- h; else h = x
 *   out = round(weight * round(h * rsqrt(mean(h^2) + eps)))
 * float32 math with the reference's rounding points. Replaces RMSNorm
 * (layers/normalization.py:7-22) and the decoder layer's residual adds
 * (models/qwen.py:136-156, models/llama.py:120-140).
 */
int mvllm_add_rms_norm(const void* x, int64_t x_stride, void* residual,
                       int64_t residual_stride, const void* weight, void* out,
                       int64_t out_stride, int64_t rows, int64_t dim,
                       float eps, int32_t dtype, void* stream);

/*
 * Pre-attention step of one layer, head_dim 128: per token, per-head RMSNorm
 * of query and key (weights may both be NULL: no norm), rotary embedding with
 * float32 cos/sin tables of 128 values per row (both NULL: none; rotate-half
 * convention), the rotated query to q_out ([num_tokens, Hq, 128],
 * contiguous), and the rotated key and the value into their paged-cache slot
 * (slot < 0 or out of range writes nothing). With positions == NULL the
 * tables hold one row per token; otherwise they hold table_rows rows, token t
 * uses row positions[t], and a position outside [0, table_rows) rotates to
 * NaN (never an out-of-bounds read). Replaces Qwen3Attention's q/k norm +
 * RotaryEmbedding (models/qwen.py:89-91, layers/rotary_embedding.py:14-52)
 * followed by write_kv_cache (operators/reference.py:84-98); the attention
 * that follows is mvllm_paged_attention.
 */
int mvllm_qk_norm_rope_kv_write(const mvllm_tensor3* query,
                                const mvllm_tensor3* key,
                                const mvllm_tensor3* value,
                                const void* q_weight, const void* k_weight,
                                const float* cos_table, const float* sin_table,
                                const int64_t* positions, int64_t table_rows,
                                float eps, void* q_out,
                                const mvllm_kv_cache* cache,
                                const int64_t* slot_mapping, void* stream);

/*
 * SwiGLU activation: gate_up rows hold [gate | up] (2 * intermediate values),
 * out[r, i] = round(round(silu(gate[r, i])) * up[r, i]). Replaces
 * SwiGLUMLP's silu(gate_proj(x)) * up_proj(x) (layers/mlp.py:10-21).
 */
int mvllm_silu_mul(const void* gate_up, int64_t in_stride, void* out,
                   int64_t out_stride, int64_t rows, int64_t intermediate,
                   int32_t dtype, void* stream);

/*
 * Embedding lookup + the first decoder layer's input RMSNorm, bf16/fp16:
 * residual_out[t] = embedding[id_t] and out[t] = RMSNorm(residual_out[t])
 * with the rounding of mvllm_add_rms_norm (residual == NULL), where id_t =
 * ids[t], or last_tokens[r] when ids[t] = -(1 + r) (a placeholder for the
 * token sampled at row r of the previous step, r < last_count). An id
 * outside [0, vocab) gives a zero row. Needs dim and the row strides in
 * multiples of 8 elements and 16-byte aligned rows. Replaces embed_tokens
 * and the first input_layernorm (models/qwen.py:227 and :144,
 * layers/normalization.py:7-22).
 */
int mvllm_embed_rms_norm(const int64_t* ids, int64_t num_tokens,
                         const int64_t* last_tokens, int64_t last_count,
                         const void* embedding, int64_t vocab,
                         int64_t embedding_stride, const void* weight,
                         void* residual_out, int64_t residual_stride,
                         void* out, int64_t out_stride, int64_t dim,
                         float eps, int32_t dtype, void* stream);

/*
 * Greedy sampling: out[r] = torch.argmax(logits[r, :cols]) for each of
 * `rows` rows (row_stride in elements; bf16, fp16 or fp32), the first index
 * of the maximum, a NaN counting as the maximum. out_copy (may be NULL)
 * receives the same indices. Replaces the sampler's per-row argmax
 * (sampling/sampler.py:24-31, 39-46); one launch, no host sync.
 */
int mvllm_argmax_rows(const void* logits, int64_t rows, int64_t cols,
                      int64_t row_stride, int32_t dtype, int64_t* out,
                      int64_t* out_copy, void* stream);

/* Text of the last failure on this thread ("" if none). */
const char* mvllm_last_error(void);

/* ABI version of this header (bumped on incompatible change). */
int mvllm_abi_version(void);

#define MVLLM_ABI_VERSION 5

#ifdef __cplusplus
}
#endif

#endif /* MVLLM_AMD_H */
