// Fused elementwise steps of the decoder layer around the attention call,
// for bf16 / fp16 activations. Each replaces a chain of framework kernels
// with one HBM pass and keeps the reference's numerics: float32 math, the
// same rounding points to the activation type, and the rotary embedding's
// separately rounded multiplies and add.
//
// * add_rms_norm: h = residual + x (rounded), residual <- h,
//   out = weight * round(h * rsqrt(mean(h^2) + eps))
//   (layers/normalization.py:7-22; the residual adds of qwen.py:136-156).
// * qk_norm_rope_kv_write: per token, per-head RMSNorm of q and k (qwen.py:
//   89-90), rotary embedding with precomputed cos/sin (rotary_embedding.py:
//   14-52), q to its output, rotated k and v straight into their paged-cache
//   slot (reference.py:84-98; slot < 0 writes nothing).
// * silu_mul: out = round(round(silu(gate)) * up) (layers/mlp.py:10-21).
// * embed_rms_norm: the embedding rows of a step's token ids (models/qwen.py:
//   227 embed_tokens) and the first layer's input RMSNorm (:144), one pass.
// * argmax_rows: greedy sampling, torch.argmax(logits, dim=-1) per row
//   (sampling/sampler.py:24-31, 39-46): the first index of the row's maximum, NaN
//   counted as the maximum.
#include <cmath>

#include "common.h"

namespace mvllm {
namespace {

template <typename T> struct Act;
template <> struct Act<bf16_t> {
  __device__ static float load(uint16_t b) { return bf16_bits_to_float(b); }
  __device__ static uint16_t store(float v) { return static_cast<uint16_t>(float_to_bf16_bits(v)); }
  __device__ static float round(float v) { return load(store(v)); }
};
template <> struct Act<f16_t> {
  __device__ static float load(uint16_t b) { return f16_bits_to_float(b); }
  __device__ static uint16_t store(float v) { return static_cast<uint16_t>(float_to_f16_bits(v)); }
  __device__ static float round(float v) { return load(store(v)); }
};

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// ------------------------------------------------------------ add_rms_norm

struct NormArgs {
  const uint16_t* x;
  uint16_t* residual;  // null: no residual add
  const uint16_t* weight;
  uint16_t* out;
  int64_t x_stride, res_stride, out_stride;
  int64_t rows;
  int32_t dim;
  float eps;
  // Gather mode only: row t of x is row ids[t] of the embedding table x; an
  // id -(1 + r) is a placeholder for last[r]. Ids outside [0, vocab) after
  // that give a zero row. The gathered rows also go to copy_out.
  const int64_t* ids;
  const int64_t* last;
  int64_t last_count;
  int64_t vocab;
  uint16_t* copy_out;
  int64_t copy_stride;
};

constexpr int kNormThreads = 256;
constexpr int kNormMaxPerThread = 32;  // dim <= 8192

template <typename T>
__global__ __launch_bounds__(kNormThreads) void add_rms_norm_kernel(NormArgs a) {
  const int64_t row = blockIdx.x;
  const int tid = threadIdx.x;
  const uint16_t* x = a.x + row * a.x_stride;
  uint16_t* res = a.residual ? a.residual + row * a.res_stride : nullptr;
  float h[kNormMaxPerThread];
  float sq = 0.f;
#pragma unroll
  for (int i = 0; i < kNormMaxPerThread; ++i) {
    const int d = tid + i * kNormThreads;
    h[i] = 0.f;
    if (d < a.dim) {
      float v = Act<T>::load(x[d]);
      if (res) {
        v = Act<T>::round(Act<T>::load(res[d]) + v);
        res[d] = Act<T>::store(v);
      }
      h[i] = v;
      sq = __builtin_fmaf(v, v, sq);
    }
  }
  __shared__ float partial[kNormThreads / 64];
  sq = wave_sum(sq);
  if ((tid & 63) == 0) partial[tid >> 6] = sq;
  __syncthreads();
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < kNormThreads / 64; ++w) total += partial[w];
  const float inv = 1.f / sqrtf(total / static_cast<float>(a.dim) + a.eps);
  uint16_t* out = a.out + row * a.out_stride;
#pragma unroll
  for (int i = 0; i < kNormMaxPerThread; ++i) {
    const int d = tid + i * kNormThreads;
    if (d < a.dim) {
      const float normed = Act<T>::round(h[i] * inv);
      out[d] = Act<T>::store(Act<T>::load(a.weight[d]) * normed);
    }
  }
}

// Vectorised form: one wave per row, lane l holds dims 8 (l + 64 c) .. +8
// for chunk c < CHUNKS (dim <= 512 CHUNKS), 16-byte loads and stores. Needs
// dim % 8 == 0 and 16-byte aligned rows; the kernel above covers the rest.
// GATHER: x rows come from the embedding table by token id (no residual);
// the normalisation is the same code, so it rounds as add_rms_norm does.
template <typename T, int CHUNKS, bool GATHER>
__global__ __launch_bounds__(256) void add_rms_norm_rows_kernel(NormArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  if (row >= a.rows) return;
  const uint16_t* x = a.x + row * a.x_stride;
  bool x_ok = true;
  if constexpr (GATHER) {
    int64_t id = a.ids[row];
    if (id < 0) {
      const int64_t r = -(id + 1);
      id = (a.last != nullptr && r < a.last_count) ? a.last[r] : -1;
    }
    x_ok = id >= 0 && id < a.vocab;
    x = a.x + (x_ok ? id : 0) * a.x_stride;
  }
  uint16_t* res = a.residual ? a.residual + row * a.res_stride : nullptr;
  float h[CHUNKS][8];
  float sq = 0.f;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int d = 8 * (lane + 64 * c);
#pragma unroll
    for (int e = 0; e < 8; ++e) h[c][e] = 0.f;
    if (d < a.dim) {
      uint4 xv = uint4{0u, 0u, 0u, 0u};
      if (x_ok) xv = *reinterpret_cast<const uint4*>(x + d);
      if constexpr (GATHER) *reinterpret_cast<uint4*>(a.copy_out + row * a.copy_stride + d) = xv;
      const uint32_t xw[4] = {xv.x, xv.y, xv.z, xv.w};
#pragma unroll
      for (int e = 0; e < 8; ++e) h[c][e] = Act<T>::load((xw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      if (res) {
        const uint4 rv = *reinterpret_cast<const uint4*>(res + d);
        const uint32_t rw[4] = {rv.x, rv.y, rv.z, rv.w};
        uint32_t ow[4];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          h[c][e] = Act<T>::round(Act<T>::load((rw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) + h[c][e]);
          if (e & 1) ow[e >> 1] |= static_cast<uint32_t>(Act<T>::store(h[c][e])) << 16;
          else ow[e >> 1] = Act<T>::store(h[c][e]);
        }
        *reinterpret_cast<uint4*>(res + d) = uint4{ow[0], ow[1], ow[2], ow[3]};
      }
#pragma unroll
      for (int e = 0; e < 8; ++e) sq = __builtin_fmaf(h[c][e], h[c][e], sq);
    }
  }
  sq = wave_sum(sq);
  const float inv = 1.f / sqrtf(sq / static_cast<float>(a.dim) + a.eps);
  uint16_t* out = a.out + row * a.out_stride;
#pragma unroll
  for (int c = 0; c < CHUNKS; ++c) {
    const int d = 8 * (lane + 64 * c);
    if (d < a.dim) {
      const uint4 wv = *reinterpret_cast<const uint4*>(a.weight + d);
      const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
      uint32_t ow[4];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        const float normed = Act<T>::round(h[c][e] * inv);
        const uint32_t o = Act<T>::store(Act<T>::load((ww[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) * normed);
        if (e & 1) ow[e >> 1] |= o << 16;
        else ow[e >> 1] = o;
      }
      *reinterpret_cast<uint4*>(out + d) = uint4{ow[0], ow[1], ow[2], ow[3]};
    }
  }
}

// --------------------------------------------------- qk_norm_rope_kv_write

struct QkArgs {
  const uint16_t* q;  // [N, Hq, D] strided
  const uint16_t* k;  // [N, Hkv, D] strided
  const uint16_t* v;  // [N, Hkv, D] strided
  int64_t q_s0, q_s1, k_s0, k_s1, v_s0, v_s1;
  const uint16_t* q_weight;  // [D] or null (no q/k norm)
  const uint16_t* k_weight;
  const float* cos;  // [table_rows, D] or null (no rotary embedding)
  const float* sin;
  const int64_t* pos;  // table row of token t: pos[t] (null: row t)
  int64_t table_rows;
  uint16_t* q_out;  // [N, Hq, D] contiguous
  uint16_t* cache;
  int64_t c_s[5];
  const int64_t* slots;
  int64_t num_tokens, num_slots, block_size;
  int32_t num_q_heads, num_kv_heads;
  float eps;
};

// One wave per (token, row); rows 0..Hq-1 are query heads, then Hkv key
// heads, then Hkv value heads. head_dim 128: lane l holds dims 2l, 2l+1, so
// the rotate-half partner of lane l's pair sits in lane l ^ 32.
template <typename T>
__global__ __launch_bounds__(256) void qk_norm_rope_kernel(QkArgs a) {
  const int lane = threadIdx.x & 63;
  const int64_t item = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int rows = a.num_q_heads + 2 * a.num_kv_heads;
  const int64_t t = item / rows;
  const int row = static_cast<int>(item % rows);
  if (t >= a.num_tokens) return;
  const bool is_q = row < a.num_q_heads;
  const bool is_v = row >= a.num_q_heads + a.num_kv_heads;
  const int head = is_q ? row : is_v ? row - a.num_q_heads - a.num_kv_heads : row - a.num_q_heads;
  const uint16_t* src = is_q ? a.q + t * a.q_s0 + head * a.q_s1
                      : is_v ? a.v + t * a.v_s0 + head * a.v_s1
                             : a.k + t * a.k_s0 + head * a.k_s1;
  const uint32_t pair = *reinterpret_cast<const uint32_t*>(src + 2 * lane);
  uint32_t result = pair;
  if (!is_v) {
    float x0 = Act<T>::load(pair & 0xFFFFu), x1 = Act<T>::load(pair >> 16);
    const uint16_t* w = is_q ? a.q_weight : a.k_weight;
    if (w) {
      const float sq = wave_sum(__builtin_fmaf(x0, x0, x1 * x1));
      const float inv = 1.f / sqrtf(sq / 128.f + a.eps);
      const uint32_t wp = *reinterpret_cast<const uint32_t*>(w + 2 * lane);
      x0 = Act<T>::round(Act<T>::load(wp & 0xFFFFu) * Act<T>::round(x0 * inv));
      x1 = Act<T>::round(Act<T>::load(wp >> 16) * Act<T>::round(x1 * inv));
    }
    if (a.cos) {
      const float p0 = __shfl_xor(x0, 32, 64), p1 = __shfl_xor(x1, 32, 64);
      // rotate_half: dims < 64 take -x[d + 64], dims >= 64 take x[d - 64].
      const float r0 = lane < 32 ? -p0 : p0, r1 = lane < 32 ? -p1 : p1;
      const int64_t tr = a.pos ? a.pos[t] : t;
      float2 c = make_float2(NAN, NAN), s = c;  // a position outside the table gives NaN
      if (tr >= 0 && tr < a.table_rows) {
        c = *reinterpret_cast<const float2*>(a.cos + tr * 128 + 2 * lane);
        s = *reinterpret_cast<const float2*>(a.sin + tr * 128 + 2 * lane);
      }
      x0 = __fadd_rn(__fmul_rn(x0, c.x), __fmul_rn(r0, s.x));
      x1 = __fadd_rn(__fmul_rn(x1, c.y), __fmul_rn(r1, s.y));
    }
    result = static_cast<uint32_t>(Act<T>::store(x0)) | (static_cast<uint32_t>(Act<T>::store(x1)) << 16);
  }
  if (is_q) {
    *reinterpret_cast<uint32_t*>(a.q_out + (t * a.num_q_heads + head) * 128 + 2 * lane) = result;
    return;
  }
  const int64_t slot = a.slots[t];
  if (slot < 0 || slot >= a.num_slots) return;
  const int64_t block = slot / a.block_size;
  const int64_t off = slot - block * a.block_size;
  uint16_t* dst = a.cache + (is_v ? a.c_s[0] : 0) + block * a.c_s[1] + off * a.c_s[2] + head * a.c_s[3];
  *reinterpret_cast<uint32_t*>(dst + 2 * lane) = result;
}

// Vectorised form: a token's rows in passes of four. Lanes 16 g .. 16 g + 15
// hold row 4 p + g; lane j of a row holds dims 8 j .. +8 (16-byte loads and
// stores), whose rotate-half partners sit in lane j ^ 8. WHOLE_TOKEN: one
// wave takes all of a token's passes, loading its cos/sin values and cache
// slot once (large batches); otherwise each wave takes one pass (small
// batches, which need the parallelism). Needs 16-byte aligned rows; the
// kernel above covers the rest.
template <typename T, bool WHOLE_TOKEN>
__global__ __launch_bounds__(256) void qk_norm_rope_token_kernel(QkArgs a) {
  const int lane = threadIdx.x & 63;
  const int rows = a.num_q_heads + 2 * a.num_kv_heads;
  const int64_t w = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
  const int passes = (rows + 3) / 4;
  const int64_t t = WHOLE_TOKEN ? w : w / passes;
  const int p_first = WHOLE_TOKEN ? 0 : static_cast<int>(w % passes) * 4;
  const int p_end = WHOLE_TOKEN ? rows : p_first + 4;
  if (t >= a.num_tokens) return;
  const int g = lane >> 4, j = lane & 15;
  float cv[8], sv[8];
  if (a.cos) {
    const int64_t tr = a.pos ? a.pos[t] : t;
    float4 c0 = make_float4(NAN, NAN, NAN, NAN), c1 = c0, s0 = c0, s1 = c0;  // outside the table: NaN
    if (tr >= 0 && tr < a.table_rows) {
      const float4* cp = reinterpret_cast<const float4*>(a.cos + tr * 128 + 8 * j);
      const float4* sp = reinterpret_cast<const float4*>(a.sin + tr * 128 + 8 * j);
      c0 = cp[0]; c1 = cp[1]; s0 = sp[0]; s1 = sp[1];
    }
    cv[0] = c0.x; cv[1] = c0.y; cv[2] = c0.z; cv[3] = c0.w; cv[4] = c1.x; cv[5] = c1.y; cv[6] = c1.z; cv[7] = c1.w;
    sv[0] = s0.x; sv[1] = s0.y; sv[2] = s0.z; sv[3] = s0.w; sv[4] = s1.x; sv[5] = s1.y; sv[6] = s1.z; sv[7] = s1.w;
  }
  const int64_t slot = a.slots[t];
  const bool slot_ok = slot >= 0 && slot < a.num_slots;
  const int64_t block = slot_ok ? slot / a.block_size : 0;
  uint16_t* const kv_row = a.cache + block * a.c_s[1] + (slot_ok ? slot - block * a.block_size : 0) * a.c_s[2];
  for (int p = p_first; p < p_end; p += 4) {
    const int row = p + g;
    const bool live = row < rows;
    const int rr = live ? row : rows - 1;  // idle groups repeat a valid row and store nothing
    const bool is_q = rr < a.num_q_heads;
    const bool is_v = rr >= a.num_q_heads + a.num_kv_heads;
    const int head = is_q ? rr : is_v ? rr - a.num_q_heads - a.num_kv_heads : rr - a.num_q_heads;
    const uint16_t* src = is_q ? a.q + t * a.q_s0 + head * a.q_s1
                        : is_v ? a.v + t * a.v_s0 + head * a.v_s1
                               : a.k + t * a.k_s0 + head * a.k_s1;
    const uint4 raw = *reinterpret_cast<const uint4*>(src + 8 * j);
    uint4 result = raw;
    if (!is_v) {
      const uint32_t rw[4] = {raw.x, raw.y, raw.z, raw.w};
      float x[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) x[e] = Act<T>::load((rw[e >> 1] >> (16 * (e & 1))) & 0xFFFFu);
      const uint16_t* w = is_q ? a.q_weight : a.k_weight;
      if (w) {
        float sq = 0.f;
#pragma unroll
        for (int e = 0; e < 8; ++e) sq = __builtin_fmaf(x[e], x[e], sq);
#pragma unroll
        for (int m = 8; m >= 1; m >>= 1) sq += __shfl_xor(sq, m, 64);  // within the row's 16 lanes
        const float inv = 1.f / sqrtf(sq / 128.f + a.eps);
        const uint4 wv = *reinterpret_cast<const uint4*>(w + 8 * j);
        const uint32_t ww[4] = {wv.x, wv.y, wv.z, wv.w};
#pragma unroll
        for (int e = 0; e < 8; ++e)
          x[e] = Act<T>::round(Act<T>::load((ww[e >> 1] >> (16 * (e & 1))) & 0xFFFFu) * Act<T>::round(x[e] * inv));
      }
      if (a.cos) {
        // rotate_half: dims < 64 take -x[d + 64], dims >= 64 take x[d - 64].
        float r[8];
#pragma unroll
        for (int e = 0; e < 8; ++e) {
          const float pe = __shfl_xor(x[e], 8, 64);
          r[e] = j < 8 ? -pe : pe;
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) x[e] = __fadd_rn(__fmul_rn(x[e], cv[e]), __fmul_rn(r[e], sv[e]));
      }
      uint32_t ow[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        ow[e] = static_cast<uint32_t>(Act<T>::store(x[2 * e])) | (static_cast<uint32_t>(Act<T>::store(x[2 * e + 1])) << 16);
      result = uint4{ow[0], ow[1], ow[2], ow[3]};
    }
    if (!live) continue;
    if (is_q) {
      *reinterpret_cast<uint4*>(a.q_out + (t * a.num_q_heads + head) * 128 + 8 * j) = result;
    } else if (slot_ok) {
      uint16_t* dst = kv_row + (is_v ? a.c_s[0] : 0) + head * a.c_s[3];
      *reinterpret_cast<uint4*>(dst + 8 * j) = result;
    }
  }
}

// --------------------------------------------------------------- silu_mul

struct SiluArgs {
  const uint16_t* gate_up;  // [N, 2I]: gate then up
  uint16_t* out;            // [N, I]
  int64_t in_stride, out_stride;
  int64_t rows;
  int32_t inter;
};

template <typename T>
__global__ __launch_bounds__(256) void silu_mul_kernel(SiluArgs a) {
  const int64_t row = blockIdx.y;
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x) * 2;
  if (i >= a.inter) return;
  const uint16_t* g = a.gate_up + row * a.in_stride;
  const uint32_t gp = *reinterpret_cast<const uint32_t*>(g + i);
  const uint32_t up = *reinterpret_cast<const uint32_t*>(g + a.inter + i);
  float r[2];
#pragma unroll
  for (int e = 0; e < 2; ++e) {
    const float x = Act<T>::load(e ? gp >> 16 : gp & 0xFFFFu);
    const float s = Act<T>::round(x / (1.f + expf(-x)));
    r[e] = s * Act<T>::load(e ? up >> 16 : up & 0xFFFFu);
  }
  *reinterpret_cast<uint32_t*>(a.out + row * a.out_stride + i) =
      static_cast<uint32_t>(Act<T>::store(r[0])) | (static_cast<uint32_t>(Act<T>::store(r[1])) << 16);
}

// ------------------------------------------------------------ argmax_rows

struct ArgmaxArgs {
  const uint8_t* logits;
  int64_t rows, cols, row_stride;  // strides in elements
  int64_t* out;
  int64_t* out_copy;  // null: none
  int32_t esize;
  bool vec;  // 16-byte aligned rows: 16-byte loads
};

constexpr int kArgmaxThreads = 1024;
constexpr uint32_t kNoIndex = 0xFFFFFFFFu;

template <typename T> struct Logit;
template <> struct Logit<bf16_t> {
  static constexpr int kPerVec = 8;
  __device__ static float get(const uint4& v, int e) {
    const uint32_t w = (&v.x)[e >> 1];
    return bf16_bits_to_float((w >> (16 * (e & 1))) & 0xFFFFu);
  }
  __device__ static float get1(const uint8_t* p) { return bf16_bits_to_float(*reinterpret_cast<const uint16_t*>(p)); }
};
template <> struct Logit<f16_t> {
  static constexpr int kPerVec = 8;
  __device__ static float get(const uint4& v, int e) {
    const uint32_t w = (&v.x)[e >> 1];
    return f16_bits_to_float((w >> (16 * (e & 1))) & 0xFFFFu);
  }
  __device__ static float get1(const uint8_t* p) { return f16_bits_to_float(*reinterpret_cast<const uint16_t*>(p)); }
};
template <> struct Logit<float> {
  static constexpr int kPerVec = 4;
  __device__ static float get(const uint4& v, int e) { return __uint_as_float((&v.x)[e]); }
  __device__ static float get1(const uint8_t* p) { return *reinterpret_cast<const float*>(p); }
};

// Running (maximum, first index) of one lane over indices in increasing
// order: a value replaces the maximum only if strictly greater, so the first
// of equal values stays (-0 and +0 compare equal, as in torch); the first
// NaN is kept aside, since NaN is the maximum.
struct ArgmaxLane {
  float best = -INFINITY;
  uint32_t best_idx = kNoIndex;
  uint32_t nan_idx = kNoIndex;
  __device__ void see(float v, uint32_t idx) {
    if (best_idx == kNoIndex || v > best) {
      best = v != v ? best : v;
      best_idx = v != v ? best_idx : idx;
    }
    if (v != v && nan_idx == kNoIndex) nan_idx = idx;
  }
  // One 64-bit key that orders candidates across lanes: the value, mapped to
  // an unsigned integer that sorts like the float (NaN above +inf, -0 = +0),
  // then the complement of the index, so that equal values prefer the
  // smaller index. 0 = no candidate.
  __device__ uint64_t key() const {
    if (nan_idx != kNoIndex) return (0xFFFFFFFFull << 32) | (0xFFFFFFFFu - nan_idx);
    if (best_idx == kNoIndex) return 0;
    uint32_t b = __float_as_uint(best);
    if ((b & 0x7FFFFFFFu) == 0) b = 0;
    const uint32_t ord = (b & 0x80000000u) ? ~b : (b | 0x80000000u);
    return (static_cast<uint64_t>(ord) << 32) | (0xFFFFFFFFu - best_idx);
  }
};

__device__ __forceinline__ uint64_t max_u64(uint64_t a, uint64_t b) { return a > b ? a : b; }

// One workgroup per row: 16-byte loads, four in flight per lane, then a
// 64-bit maximum over the workgroup.
template <typename T>
__global__ __launch_bounds__(kArgmaxThreads) void argmax_rows_kernel(ArgmaxArgs a) {
  const int64_t row = blockIdx.x;
  const uint8_t* base = a.logits + row * a.row_stride * a.esize;
  ArgmaxLane lane_state;
  const int tid = threadIdx.x;
  if (a.vec) {
    constexpr int P = Logit<T>::kPerVec;
    const int64_t nvec = a.cols / P;
    const uint4* vp = reinterpret_cast<const uint4*>(base);
    for (int64_t v0 = tid; v0 < nvec; v0 += 4LL * kArgmaxThreads) {
      uint4 buf[4];
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + static_cast<int64_t>(u) * kArgmaxThreads;
        buf[u] = v < nvec ? vp[v] : uint4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int u = 0; u < 4; ++u) {
        const int64_t v = v0 + static_cast<int64_t>(u) * kArgmaxThreads;
        if (v < nvec) {
#pragma unroll
          for (int e = 0; e < P; ++e) lane_state.see(Logit<T>::get(buf[u], e), static_cast<uint32_t>(v * P + e));
        }
      }
    }
    // The tail past the last whole vector, by the first lanes.
    const int64_t tail = nvec * P + tid;
    if (tail < a.cols) lane_state.see(Logit<T>::get1(base + tail * a.esize), static_cast<uint32_t>(tail));
  } else {
    for (int64_t c = tid; c < a.cols; c += kArgmaxThreads)
      lane_state.see(Logit<T>::get1(base + c * a.esize), static_cast<uint32_t>(c));
  }
  uint64_t k = lane_state.key();
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) k = max_u64(k, __shfl_xor(k, m, 64));
  __shared__ uint64_t wave_best[kArgmaxThreads / 64];
  if ((tid & 63) == 0) wave_best[tid >> 6] = k;
  __syncthreads();
  if (tid == 0) {
    uint64_t best = 0;
#pragma unroll
    for (int w = 0; w < kArgmaxThreads / 64; ++w) best = max_u64(best, wave_best[w]);
    const int64_t idx = static_cast<int64_t>(0xFFFFFFFFu - static_cast<uint32_t>(best & 0xFFFFFFFFu));
    a.out[row] = idx;
    if (a.out_copy) a.out_copy[row] = idx;
  }
}

bool half_dtype(int32_t d) { return d == MVLLM_DTYPE_BF16 || d == MVLLM_DTYPE_F16; }

bool aligned4(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 3u) == 0; }

bool mult8(int64_t v) { return (v & 7) == 0; }

template <typename T, bool GATHER = false>
int launch_add_rms_norm_rows(const NormArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>((a.rows + 3) / 4));
  const int chunks = (a.dim + 511) / 512;
  if (chunks <= 1) hipLaunchKernelGGL((add_rms_norm_rows_kernel<T, 1, GATHER>), grid, dim3(256), 0, s, a);
  else if (chunks <= 2) hipLaunchKernelGGL((add_rms_norm_rows_kernel<T, 2, GATHER>), grid, dim3(256), 0, s, a);
  else if (chunks <= 4) hipLaunchKernelGGL((add_rms_norm_rows_kernel<T, 4, GATHER>), grid, dim3(256), 0, s, a);
  else if (chunks <= 8) hipLaunchKernelGGL((add_rms_norm_rows_kernel<T, 8, GATHER>), grid, dim3(256), 0, s, a);
  else hipLaunchKernelGGL((add_rms_norm_rows_kernel<T, 16, GATHER>), grid, dim3(256), 0, s, a);
  MVLLM_LAUNCH_CHECK("add_rms_norm_rows_kernel");
  return MVLLM_OK;
}

}  // namespace
}  // namespace mvllm

using namespace mvllm;

extern "C" int mvllm_add_rms_norm(const void* x, int64_t x_stride, void* residual, int64_t residual_stride,
                                  const void* weight, void* out, int64_t out_stride, int64_t rows,
                                  int64_t dim, float eps, int32_t dtype, void* stream) {
  clear_error();
  if (!half_dtype(dtype)) return fail(MVLLM_ERR_UNSUPPORTED, "add_rms_norm needs bf16 or fp16");
  if (rows < 0 || dim <= 0 || dim > kNormThreads * kNormMaxPerThread)
    return fail(MVLLM_ERR_INVALID, "add_rms_norm: rows %lld / dim %lld out of range", (long long)rows,
                (long long)dim);
  if (rows == 0) return MVLLM_OK;
  if (!x || !weight || !out) return fail(MVLLM_ERR_INVALID, "add_rms_norm: null pointer");
  if (rows > INT32_MAX) return fail(MVLLM_ERR_INVALID, "add_rms_norm: too many rows");
  NormArgs a{};
  a.x = static_cast<const uint16_t*>(x);
  a.residual = static_cast<uint16_t*>(residual);
  a.weight = static_cast<const uint16_t*>(weight);
  a.out = static_cast<uint16_t*>(out);
  a.x_stride = x_stride;
  a.res_stride = residual_stride;
  a.out_stride = out_stride;
  a.rows = rows;
  a.dim = static_cast<int32_t>(dim);
  a.eps = eps;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = mult8(dim) && mult8(x_stride) && mult8(out_stride) && aligned16(x) && aligned16(weight) &&
                   aligned16(out) && (!residual || (mult8(residual_stride) && aligned16(residual)));
  if (vec && dtype == MVLLM_DTYPE_BF16) return launch_add_rms_norm_rows<bf16_t>(a, s);
  if (vec) return launch_add_rms_norm_rows<f16_t>(a, s);
  if (dtype == MVLLM_DTYPE_BF16)
    hipLaunchKernelGGL(add_rms_norm_kernel<bf16_t>, dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0, s, a);
  else
    hipLaunchKernelGGL(add_rms_norm_kernel<f16_t>, dim3(static_cast<unsigned>(rows)), dim3(kNormThreads), 0, s, a);
  MVLLM_LAUNCH_CHECK("add_rms_norm_kernel");
  return MVLLM_OK;
}

extern "C" int mvllm_qk_norm_rope_kv_write(const mvllm_tensor3* query, const mvllm_tensor3* key,
                                           const mvllm_tensor3* value, const void* q_weight,
                                           const void* k_weight, const float* cos_table,
                                           const float* sin_table, const int64_t* positions,
                                           int64_t table_rows, float eps, void* q_out,
                                           const mvllm_kv_cache* cache, const int64_t* slot_mapping,
                                           void* stream) {
  clear_error();
  if (!query || !key || !value || !cache) return fail(MVLLM_ERR_INVALID, "qk_norm_rope: null descriptor");
  const int32_t dtype = query->dtype;
  if (!half_dtype(dtype) || key->dtype != dtype || value->dtype != dtype || cache->dtype != dtype)
    return fail(MVLLM_ERR_UNSUPPORTED, "qk_norm_rope needs bf16 or fp16 throughout");
  const int64_t N = query->size[0];
  if (query->size[2] != 128 || key->size[2] != 128 || value->size[2] != 128 || cache->head_dim != 128)
    return fail(MVLLM_ERR_UNSUPPORTED, "qk_norm_rope needs head_dim 128");
  if (key->size[0] != N || value->size[0] != N || key->size[1] != value->size[1] ||
      key->size[1] != cache->num_kv_heads)
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: query/key/value/cache shapes disagree");
  if (query->stride[2] != 1 || key->stride[2] != 1 || value->stride[2] != 1 || cache->stride[4] != 1 ||
      (query->stride[0] | query->stride[1] | key->stride[0] | key->stride[1] | value->stride[0] |
       value->stride[1] | cache->stride[0] | cache->stride[1] | cache->stride[2] | cache->stride[3]) & 1)
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: rows must be contiguous with even strides");
  if ((cos_table == nullptr) != (sin_table == nullptr) || (q_weight == nullptr) != (k_weight == nullptr))
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: cos/sin and q/k weights come in pairs");
  if (positions && (!cos_table || table_rows <= 0))
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: positions need cos/sin tables of table_rows > 0 rows");
  if (N == 0) return MVLLM_OK;
  if (!slot_mapping || !q_out || !cache->data || !aligned4(query->data) || !aligned4(key->data) ||
      !aligned4(value->data) || !aligned4(q_out) || !aligned4(cache->data))
    return fail(MVLLM_ERR_INVALID, "qk_norm_rope: null or misaligned pointer");
  QkArgs a = {};
  a.q = static_cast<const uint16_t*>(query->data);
  a.k = static_cast<const uint16_t*>(key->data);
  a.v = static_cast<const uint16_t*>(value->data);
  a.q_s0 = query->stride[0]; a.q_s1 = query->stride[1];
  a.k_s0 = key->stride[0]; a.k_s1 = key->stride[1];
  a.v_s0 = value->stride[0]; a.v_s1 = value->stride[1];
  a.q_weight = static_cast<const uint16_t*>(q_weight);
  a.k_weight = static_cast<const uint16_t*>(k_weight);
  a.cos = cos_table;
  a.sin = sin_table;
  a.pos = positions;
  a.table_rows = positions ? table_rows : N;
  a.q_out = static_cast<uint16_t*>(q_out);
  a.cache = static_cast<uint16_t*>(cache->data);
  for (int i = 0; i < 5; ++i) a.c_s[i] = cache->stride[i];
  a.slots = slot_mapping;
  a.num_tokens = N;
  a.num_slots = cache->num_blocks * cache->block_size;
  a.block_size = cache->block_size;
  a.num_q_heads = static_cast<int32_t>(query->size[1]);
  a.num_kv_heads = static_cast<int32_t>(key->size[1]);
  a.eps = eps;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const bool vec = aligned16(query->data) && aligned16(key->data) && aligned16(value->data) && aligned16(q_out) &&
                   aligned16(cache->data) && mult8(a.q_s0) && mult8(a.q_s1) && mult8(a.k_s0) && mult8(a.k_s1) &&
                   mult8(a.v_s0) && mult8(a.v_s1) && mult8(a.c_s[0]) && mult8(a.c_s[1]) && mult8(a.c_s[2]) &&
                   mult8(a.c_s[3]) && (!q_weight || (aligned16(q_weight) && aligned16(k_weight))) &&
                   (!cos_table || (aligned16(cos_table) && aligned16(sin_table)));
  if (vec) {
    // Whole tokens per wave once the batch alone fills the GPU (>= 8 waves
    // per CU at 256 CUs); one pass of four rows per wave below that.
    const bool whole = N >= 2048;
    const int64_t passes = (query->size[1] + 2 * key->size[1] + 3) / 4;
    const int64_t blocks = ((whole ? N : N * passes) + 3) / 4;
    if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "qk_norm_rope: grid too large");
    if (dtype == MVLLM_DTYPE_BF16) {
      if (whole) hipLaunchKernelGGL((qk_norm_rope_token_kernel<bf16_t, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((qk_norm_rope_token_kernel<bf16_t, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
    } else {
      if (whole) hipLaunchKernelGGL((qk_norm_rope_token_kernel<f16_t, true>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
      else hipLaunchKernelGGL((qk_norm_rope_token_kernel<f16_t, false>), dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
    }
    MVLLM_LAUNCH_CHECK("qk_norm_rope_token_kernel");
    return MVLLM_OK;
  }
  const int64_t items = N * (query->size[1] + 2 * key->size[1]);
  const int64_t blocks = (items + 3) / 4;
  if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "qk_norm_rope: grid too large");
  if (dtype == MVLLM_DTYPE_BF16)
    hipLaunchKernelGGL(qk_norm_rope_kernel<bf16_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(qk_norm_rope_kernel<f16_t>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, s, a);
  MVLLM_LAUNCH_CHECK("qk_norm_rope_kernel");
  return MVLLM_OK;
}

extern "C" int mvllm_silu_mul(const void* gate_up, int64_t in_stride, void* out, int64_t out_stride,
                              int64_t rows, int64_t intermediate, int32_t dtype, void* stream) {
  clear_error();
  if (!half_dtype(dtype)) return fail(MVLLM_ERR_UNSUPPORTED, "silu_mul needs bf16 or fp16");
  if (rows < 0 || intermediate <= 0 || (intermediate & 1) || (in_stride & 1) || (out_stride & 1))
    return fail(MVLLM_ERR_INVALID, "silu_mul: sizes and strides must be even");
  if (rows == 0) return MVLLM_OK;
  if (!gate_up || !out || !aligned4(gate_up) || !aligned4(out))
    return fail(MVLLM_ERR_INVALID, "silu_mul: null or misaligned pointer");
  if (rows > 65535) return fail(MVLLM_ERR_INVALID, "silu_mul: more than 65535 rows");
  SiluArgs a{static_cast<const uint16_t*>(gate_up), static_cast<uint16_t*>(out), in_stride, out_stride, rows,
             static_cast<int32_t>(intermediate)};
  const dim3 grid(static_cast<unsigned>((intermediate / 2 + 255) / 256), static_cast<unsigned>(rows));
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == MVLLM_DTYPE_BF16)
    hipLaunchKernelGGL(silu_mul_kernel<bf16_t>, grid, dim3(256), 0, s, a);
  else
    hipLaunchKernelGGL(silu_mul_kernel<f16_t>, grid, dim3(256), 0, s, a);
  MVLLM_LAUNCH_CHECK("silu_mul_kernel");
  return MVLLM_OK;
}

extern "C" int mvllm_embed_rms_norm(const int64_t* ids, int64_t num_tokens, const int64_t* last_tokens,
                                    int64_t last_count, const void* embedding, int64_t vocab,
                                    int64_t embedding_stride, const void* weight, void* residual_out,
                                    int64_t residual_stride, void* out, int64_t out_stride, int64_t dim,
                                    float eps, int32_t dtype, void* stream) {
  clear_error();
  if (!half_dtype(dtype)) return fail(MVLLM_ERR_UNSUPPORTED, "embed_rms_norm needs bf16 or fp16");
  if (num_tokens < 0 || vocab <= 0 || last_count < 0 || dim <= 0 || dim > 8192)
    return fail(MVLLM_ERR_INVALID, "embed_rms_norm: sizes out of range");
  if (num_tokens == 0) return MVLLM_OK;
  if (!ids || !embedding || !weight || !residual_out || !out || (last_count > 0 && !last_tokens))
    return fail(MVLLM_ERR_INVALID, "embed_rms_norm: null pointer");
  if (num_tokens > INT32_MAX) return fail(MVLLM_ERR_INVALID, "embed_rms_norm: too many tokens");
  if (!mult8(dim) || !mult8(embedding_stride) || !mult8(residual_stride) || !mult8(out_stride) ||
      !aligned16(embedding) || !aligned16(weight) || !aligned16(residual_out) || !aligned16(out))
    return fail(MVLLM_ERR_UNSUPPORTED, "embed_rms_norm needs dim and row strides in multiples of 8 elements "
                                       "and 16-byte aligned rows");
  NormArgs a{};
  a.x = static_cast<const uint16_t*>(embedding);
  a.weight = static_cast<const uint16_t*>(weight);
  a.out = static_cast<uint16_t*>(out);
  a.x_stride = embedding_stride;
  a.out_stride = out_stride;
  a.rows = num_tokens;
  a.dim = static_cast<int32_t>(dim);
  a.eps = eps;
  a.ids = ids;
  a.last = last_count > 0 ? last_tokens : nullptr;
  a.last_count = last_count;
  a.vocab = vocab;
  a.copy_out = static_cast<uint16_t*>(residual_out);
  a.copy_stride = residual_stride;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  if (dtype == MVLLM_DTYPE_BF16) return launch_add_rms_norm_rows<bf16_t, true>(a, s);
  return launch_add_rms_norm_rows<f16_t, true>(a, s);
}

extern "C" int mvllm_argmax_rows(const void* logits, int64_t rows, int64_t cols, int64_t row_stride,
                                 int32_t dtype, int64_t* out, int64_t* out_copy, void* stream) {
  clear_error();
  const int32_t esize = dtype == MVLLM_DTYPE_F32 ? 4 : half_dtype(dtype) ? 2 : 0;
  if (!esize) return fail(MVLLM_ERR_UNSUPPORTED, "argmax_rows needs bf16, fp16 or fp32 logits");
  if (rows < 0 || cols <= 0 || cols > INT32_MAX || row_stride < cols)
    return fail(MVLLM_ERR_INVALID, "argmax_rows: rows %lld / cols %lld / row stride %lld out of range",
                (long long)rows, (long long)cols, (long long)row_stride);
  if (rows == 0) return MVLLM_OK;
  if (!logits || !out) return fail(MVLLM_ERR_INVALID, "argmax_rows: null pointer");
  if (rows > INT32_MAX) return fail(MVLLM_ERR_INVALID, "argmax_rows: too many rows");
  if ((reinterpret_cast<uintptr_t>(logits) & (esize - 1)) != 0)
    return fail(MVLLM_ERR_INVALID, "argmax_rows: misaligned logits");
  ArgmaxArgs a{};
  a.logits = static_cast<const uint8_t*>(logits);
  a.rows = rows;
  a.cols = cols;
  a.row_stride = row_stride;
  a.out = out;
  a.out_copy = out_copy;
  a.esize = esize;
  a.vec = aligned16(logits) && (row_stride * esize) % 16 == 0;
  hipStream_t s = reinterpret_cast<hipStream_t>(stream);
  const dim3 grid(static_cast<unsigned>(rows));
  if (dtype == MVLLM_DTYPE_BF16)
    hipLaunchKernelGGL(argmax_rows_kernel<bf16_t>, grid, dim3(kArgmaxThreads), 0, s, a);
  else if (dtype == MVLLM_DTYPE_F16)
    hipLaunchKernelGGL(argmax_rows_kernel<f16_t>, grid, dim3(kArgmaxThreads), 0, s, a);
  else
    hipLaunchKernelGGL(argmax_rows_kernel<float>, grid, dim3(kArgmaxThreads), 0, s, a);
  MVLLM_LAUNCH_CHECK("argmax_rows_kernel");
  return MVLLM_OK;
}
