// Paged KV-cache write (slot scatter) and the bit-exact block gather.
//
// Both are pure HBM copies: no arithmetic touches the payload, so results
// are bit-exact for every element type. The fast paths move 16-byte chunks
// of whole token rows (all KV heads of one token are contiguous in the
// reference cache layout (2, blocks, block_size, heads, dim)); the generic
// paths handle arbitrary strides element by element.
#include "worklists.h"

namespace mvllm {
namespace {

// One workgroup per token: its K row then its V row.
__global__ __launch_bounds__(256) void kv_write_rows_kernel(KvRowArgs a) {
  copy_kv_row(a, blockIdx.x, threadIdx.x, blockDim.x);
}

struct WriteGenericArgs {
  const char* key;
  const char* value;
  char* cache;
  const int64_t* slots;
  int64_t ks[3], vs[3];   // element strides of key / value
  int64_t cs[5];          // element strides of the cache
  int64_t heads, dim, block_size, num_slots;
  int32_t esize;
};

template <int ESIZE>
__device__ __forceinline__ void copy_elem(char* dst, const char* src) {
  if constexpr (ESIZE == 4) {
    *reinterpret_cast<uint32_t*>(dst) = *reinterpret_cast<const uint32_t*>(src);
  } else {
    *reinterpret_cast<uint16_t*>(dst) = *reinterpret_cast<const uint16_t*>(src);
  }
}

template <int ESIZE>
__global__ __launch_bounds__(256) void kv_write_generic_kernel(WriteGenericArgs a) {
  const int64_t token = blockIdx.x;
  const int64_t slot = a.slots[token];
  if (slot < 0 || slot >= a.num_slots) return;
  const int64_t block = slot / a.block_size;
  const int64_t offset = slot - block * a.block_size;
  const int64_t total = a.heads * a.dim;
  for (int64_t i = threadIdx.x; i < total; i += blockDim.x) {
    const int64_t h = i / a.dim;
    const int64_t d = i - h * a.dim;
    const int64_t c = block * a.cs[1] + offset * a.cs[2] + h * a.cs[3] + d * a.cs[4];
    copy_elem<ESIZE>(a.cache + ESIZE * c,
                     a.key + ESIZE * (token * a.ks[0] + h * a.ks[1] + d * a.ks[2]));
    copy_elem<ESIZE>(a.cache + ESIZE * (c + a.cs[0]),
                     a.value + ESIZE * (token * a.vs[0] + h * a.vs[1] + d * a.vs[2]));
  }
}

struct GatherArgs {
  const char* cache;
  char* out_key;
  char* out_value;
  const int64_t* cstarts;
  const int64_t* qsl;
  const int64_t* lengths;
  const int64_t* table;
  int64_t table_s0, table_s1, width;
  int64_t cs[5];  // element strides
  int64_t heads, dim, block_size, num_blocks, capacity, num_tokens;
  int32_t esize;
  int32_t vector;  // 1: rows are contiguous and 16-byte aligned
};

// One workgroup per (gathered row, request).
__global__ __launch_bounds__(256) void gather_kernel(GatherArgs a) {
  const int64_t row = blockIdx.x;
  const int64_t r = blockIdx.y;
  const int64_t qs = a.qsl[r];
  if (qs < 0 || qs >= a.num_tokens || a.qsl[r + 1] <= qs) return;
  const int64_t first = a.cstarts[qs];
  const int64_t position = first + row;
  if (row >= a.capacity || position < 0 || position >= a.lengths[r]) return;
  const int64_t logical = position / a.block_size;
  if (logical >= a.width) return;
  const int64_t block = a.table[r * a.table_s0 + logical * a.table_s1];
  if (block < 0 || block >= a.num_blocks) return;
  const int64_t offset = position - logical * a.block_size;
  const int64_t row_elems = a.heads * a.dim;
  const int64_t src = block * a.cs[1] + offset * a.cs[2];
  const int64_t dst = (r * a.capacity + row) * row_elems;
  if (a.vector) {
    const int64_t chunks = row_elems * a.esize / 16;
    for (int64_t c = threadIdx.x; c < 2 * chunks; c += blockDim.x) {
      const bool is_value = c >= chunks;
      const int64_t chunk = is_value ? c - chunks : c;
      const uint4 data = *reinterpret_cast<const uint4*>(
          a.cache + a.esize * (src + (is_value ? a.cs[0] : 0)) + 16 * chunk);
      *reinterpret_cast<uint4*>((is_value ? a.out_value : a.out_key) +
                                a.esize * dst + 16 * chunk) = data;
    }
    return;
  }
  for (int64_t i = threadIdx.x; i < row_elems; i += blockDim.x) {
    const int64_t h = i / a.dim;
    const int64_t d = i - h * a.dim;
    const int64_t c = src + h * a.cs[3] + d * a.cs[4];
    if (a.esize == 4) {
      copy_elem<4>(a.out_key + 4 * (dst + i), a.cache + 4 * c);
      copy_elem<4>(a.out_value + 4 * (dst + i), a.cache + 4 * (c + a.cs[0]));
    } else {
      copy_elem<2>(a.out_key + 2 * (dst + i), a.cache + 2 * c);
      copy_elem<2>(a.out_value + 2 * (dst + i), a.cache + 2 * (c + a.cs[0]));
    }
  }
}

int check_cache(const mvllm_kv_cache* cache) {
  if (!cache || !cache->data) return fail(MVLLM_ERR_INVALID, "cache is null");
  if (dtype_bytes(cache->dtype) == 0)
    return fail(MVLLM_ERR_UNSUPPORTED, "unsupported cache dtype code %d", cache->dtype);
  if (cache->num_blocks < 1 || cache->block_size < 1 || cache->num_kv_heads < 1 ||
      cache->head_dim < 1)
    return fail(MVLLM_ERR_INVALID, "cache dimensions must be positive");
  for (int i = 0; i < 5; ++i)
    if (cache->stride[i] < 0) return fail(MVLLM_ERR_INVALID, "negative cache stride");
  return MVLLM_OK;
}

}  // namespace
}  // namespace mvllm

using namespace mvllm;

namespace mvllm {

int kv_write_prepare(const mvllm_tensor3* key, const mvllm_tensor3* value, const mvllm_kv_cache* cache,
                     const int64_t* slot_mapping, int64_t num_tokens, KvRowArgs* rows, bool* vectorised) {
  *vectorised = false;
  if (int rc = check_cache(cache)) return rc;
  if (!key || !value) return fail(MVLLM_ERR_INVALID, "key/value descriptor is null");
  if (num_tokens < 0) return fail(MVLLM_ERR_INVALID, "negative num_tokens");
  if (num_tokens == 0) return MVLLM_OK;
  if (!key->data || !value->data || !slot_mapping)
    return fail(MVLLM_ERR_INVALID, "null key/value/slot_mapping pointer");
  if (key->dtype != cache->dtype || value->dtype != cache->dtype)
    return fail(MVLLM_ERR_INVALID, "key/value dtype (%s/%s) must equal the cache dtype (%s)",
                dtype_name(key->dtype), dtype_name(value->dtype), dtype_name(cache->dtype));
  const int64_t H = cache->num_kv_heads, D = cache->head_dim;
  for (const mvllm_tensor3* t : {key, value}) {
    if (t->size[0] < num_tokens || t->size[1] != H || t->size[2] != D)
      return fail(MVLLM_ERR_INVALID,
                  "key/value shape [%lld, %lld, %lld] does not match [%lld, %lld, %lld]",
                  (long long)t->size[0], (long long)t->size[1], (long long)t->size[2],
                  (long long)num_tokens, (long long)H, (long long)D);
  }
  if (num_tokens > INT32_MAX) return fail(MVLLM_ERR_INVALID, "too many tokens");
  const int64_t es = dtype_bytes(cache->dtype);
  const int64_t row_bytes = H * D * es;
  const bool rows_contiguous = key->stride[2] == 1 && key->stride[1] == D &&
                               value->stride[2] == 1 && value->stride[1] == D &&
                               cache->stride[4] == 1 && cache->stride[3] == D;
  const bool vec_ok = rows_contiguous && row_bytes % 16 == 0 && aligned16(key->data) &&
                      aligned16(value->data) && aligned16(cache->data) &&
                      (key->stride[0] * es) % 16 == 0 && (value->stride[0] * es) % 16 == 0 &&
                      (cache->stride[0] * es) % 16 == 0 && (cache->stride[1] * es) % 16 == 0 &&
                      (cache->stride[2] * es) % 16 == 0;
  if (!vec_ok) return MVLLM_OK;
  KvRowArgs& a = *rows;
  a.key = static_cast<const char*>(key->data);
  a.value = static_cast<const char*>(value->data);
  a.cache = static_cast<char*>(cache->data);
  a.slots = slot_mapping;
  a.key_token_stride = key->stride[0] * es;
  a.value_token_stride = value->stride[0] * es;
  a.plane_stride = cache->stride[0] * es;
  a.block_stride = cache->stride[1] * es;
  a.offset_stride = cache->stride[2] * es;
  a.block_size = cache->block_size;
  a.num_slots = cache->num_blocks * cache->block_size;
  a.chunks = static_cast<int32_t>(row_bytes / 16);
  *vectorised = true;
  return MVLLM_OK;
}

}  // namespace mvllm

extern "C" int mvllm_kv_write(const mvllm_tensor3* key, const mvllm_tensor3* value,
                              const mvllm_kv_cache* cache, const int64_t* slot_mapping,
                              int64_t num_tokens, void* stream) {
  clear_error();
  KvRowArgs a;
  bool vec = false;
  if (int rc = kv_write_prepare(key, value, cache, slot_mapping, num_tokens, &a, &vec)) return rc;
  if (num_tokens == 0) return MVLLM_OK;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (vec) {
    int threads = static_cast<int>(std::min<int64_t>(256, ceil_div(2 * a.chunks, 64) * 64));
    hipLaunchKernelGGL(kv_write_rows_kernel, dim3(static_cast<unsigned>(num_tokens)),
                       dim3(threads), 0, s, a);
    MVLLM_LAUNCH_CHECK("kv_write_rows_kernel");
    return MVLLM_OK;
  }
  const int64_t H = cache->num_kv_heads, D = cache->head_dim;
  const int64_t es = dtype_bytes(cache->dtype);
  WriteGenericArgs g;
  g.key = static_cast<const char*>(key->data);
  g.value = static_cast<const char*>(value->data);
  g.cache = static_cast<char*>(cache->data);
  g.slots = slot_mapping;
  for (int i = 0; i < 3; ++i) {
    g.ks[i] = key->stride[i];
    g.vs[i] = value->stride[i];
  }
  for (int i = 0; i < 5; ++i) g.cs[i] = cache->stride[i];
  g.heads = H;
  g.dim = D;
  g.block_size = cache->block_size;
  g.num_slots = cache->num_blocks * cache->block_size;
  g.esize = static_cast<int32_t>(es);
  if (es == 4)
    hipLaunchKernelGGL(kv_write_generic_kernel<4>, dim3(static_cast<unsigned>(num_tokens)),
                       dim3(256), 0, s, g);
  else
    hipLaunchKernelGGL(kv_write_generic_kernel<2>, dim3(static_cast<unsigned>(num_tokens)),
                       dim3(256), 0, s, g);
  MVLLM_LAUNCH_CHECK("kv_write_generic_kernel");
  return MVLLM_OK;
}

extern "C" int mvllm_gather_kv(const mvllm_kv_cache* cache, const mvllm_batch* batch,
                               int64_t capacity, void* out_key, void* out_value,
                               void* stream) {
  clear_error();
  if (int rc = check_cache(cache)) return rc;
  if (!batch) return fail(MVLLM_ERR_INVALID, "batch is null");
  if (capacity < 0) return fail(MVLLM_ERR_INVALID, "negative capacity");
  if (batch->num_requests == 0 || capacity == 0) return MVLLM_OK;
  if (!out_key || !out_value || !batch->query_context_start_positions ||
      !batch->query_start_locations || !batch->context_lengths || !batch->block_table)
    return fail(MVLLM_ERR_INVALID, "null pointer in gather arguments");
  if (batch->block_size != cache->block_size)
    return fail(MVLLM_ERR_INVALID, "batch block_size %lld != cache block_size %lld",
                (long long)batch->block_size, (long long)cache->block_size);
  if (capacity > INT32_MAX || batch->num_requests > 65535)
    return fail(MVLLM_ERR_INVALID, "gather grid too large");
  const int64_t es = dtype_bytes(cache->dtype);
  GatherArgs a;
  a.cache = static_cast<const char*>(cache->data);
  a.out_key = static_cast<char*>(out_key);
  a.out_value = static_cast<char*>(out_value);
  a.cstarts = batch->query_context_start_positions;
  a.qsl = batch->query_start_locations;
  a.lengths = batch->context_lengths;
  a.table = batch->block_table;
  a.table_s0 = batch->block_table_stride[0];
  a.table_s1 = batch->block_table_stride[1];
  a.width = batch->block_table_width;
  for (int i = 0; i < 5; ++i) a.cs[i] = cache->stride[i];
  a.heads = cache->num_kv_heads;
  a.dim = cache->head_dim;
  a.block_size = cache->block_size;
  a.num_blocks = cache->num_blocks;
  a.capacity = capacity;
  a.num_tokens = batch->num_tokens;
  a.esize = static_cast<int32_t>(es);
  const int64_t row_bytes = a.heads * a.dim * es;
  a.vector = (cache->stride[4] == 1 && cache->stride[3] == a.dim && row_bytes % 16 == 0 &&
              aligned16(cache->data) && aligned16(out_key) && aligned16(out_value) &&
              (cache->stride[0] * es) % 16 == 0 && (cache->stride[1] * es) % 16 == 0 &&
              (cache->stride[2] * es) % 16 == 0)
                 ? 1
                 : 0;
  hipLaunchKernelGGL(gather_kernel,
                     dim3(static_cast<unsigned>(capacity), static_cast<unsigned>(batch->num_requests)),
                     dim3(256), 0, reinterpret_cast<hipStream_t>(stream), a);
  MVLLM_LAUNCH_CHECK("gather_kernel");
  return MVLLM_OK;
}
