// Split-KV ragged decode on gfx950 matrix cores (head_dim 128, bf16/fp16).
//
// Work item: (KV head, split of the visible context, request). One wavefront
// owns one KV head; a workgroup holds up to 8 waves = 8 consecutive KV heads
// of the same (request, split), so together they stream whole token rows
// (all heads of a token are contiguous in the cache) with 16-byte loads.
// A one-workgroup kernel lists the (request, split) items on the GPU, full
// splits first and partial last splits from the largest down, so that the
// grid's in-order dispatch ends on its shortest items (decode_items_kernel).
// Each record carries the request's query token, visible range and the
// split's key range, so a workgroup needs no metadata loads of its own.
//
// Per 16-token tile a wave computes S^T = K . Q^T with four
// v_mfma_f32_16x16x32 (M = 16 tokens, N = the G query heads of the KV head,
// padded to 16, K = 128 dims), so K is consumed straight from its natural
// row layout. The softmax runs on the accumulator layout (each lane holds 4
// tokens of one head: max/sum need only two cross-lane steps). P^T is
// already the B operand of O^T += V^T . P^T (v_mfma_f32_16x16x16), which
// keeps alpha rescaling in-lane; V^T comes from a transposed read of the V
// tile through a per-wave LDS slab. P is fed as a bf16 hi/lo pair so the
// P.V product keeps ~16 mantissa bits (the kernel is HBM-bound; the extra
// MFMAs are free).
//
// Each split writes (max, sum, unnormalised acc) partials; a request whose
// context fits one split writes its output directly. The combine kernel
// merges partials with the standard log-sum-exp rescaling (FlashAttention-2,
// Dao 2023; flash-decoding, Dao et al. 2023) and zero-fills tokens that
// belong to no request. It learns each request's query token and split count
// from a table that the work-list kernel writes, one load per workgroup.
#include <cmath>
#include <cstdlib>
#include <cstring>

#include <hip/hip_ext.h>

#include "decode_split.h"

namespace mvllm {
namespace {

using namespace dec;

constexpr int kRow = 144;  // LDS row stride (elements): 288 B keeps both LDS access patterns conflict-free
constexpr int kMaxWaves = 8;

// One 16-token tile of one KV head as MFMA A operands: lane (col, grp)
// holds token `col`, dims 32i + 8grp .. +8 of K and of V.
struct Tile {
  short8_t k[4];
  short8_t v[4];
  bool ok;
};

template <bool NT>
__device__ __forceinline__ short8_t load16(const uint16_t* p) {
  if constexpr (NT) {
    return __builtin_nontemporal_load(reinterpret_cast<const short8_t*>(p));
  } else {
    return *reinterpret_cast<const short8_t*>(p);
  }
}

template <bool NT>
__device__ __forceinline__ void load_tile(const AttnArgs& a, const uint16_t* cache, int64_t r,
                                          int64_t base, int64_t lo, int64_t end, int col,
                                          int64_t head_off, Tile& t) {
  const int64_t tk = base + col;
  bool ok = tk >= lo && tk <= end;
  int64_t off = 0;
  if (ok) {
    const int64_t b = block_of(a, r, tk);
    ok = b >= 0;
    off = b * a.c_s[1] + (tk % a.block_size) * a.c_s[2] + head_off;
  }
  const short8_t zero = {0, 0, 0, 0, 0, 0, 0, 0};
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    t.k[i] = ok ? load16<NT>(cache + off + 32 * i) : zero;
    t.v[i] = ok ? load16<NT>(cache + a.c_s[0] + off + 32 * i) : zero;
  }
  t.ok = ok;
}

template <typename T, bool PREFETCH, bool NT>
__global__ __launch_bounds__(512) void decode_split_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[kMaxWaves][16 * kRow];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int waves = blockDim.x >> 6;
  // 1-D grid: workgroup b takes head group b % groups of work-list slot b / groups.
  const int groups = (a.num_kv_heads + waves - 1) / waves;
  const int h = static_cast<int>(blockIdx.x % groups) * waves + wave;
  const DecodeItem item = a.decode_items[blockIdx.x / groups];
  if (item.r < 0 || item.r >= a.num_requests) return;
  const int split = item.split;
  const int64_t r = item.r;
  if (h >= a.num_kv_heads) return;
  const int64_t qs = item.qs;
  const int64_t lo = item.lo;
  const int64_t begin = item.begin;
  const int64_t end = item.end;
  // Records index the query, the table and the partials: out-of-range
  // fields (never written by the work-list kernel) end the workgroup.
  if (begin < 0 || begin > end || end - begin >= a.split_tokens || end >= a.width * a.block_size ||
      qs < 0 || qs >= a.num_tokens || split < 0 || split >= a.max_splits)
    return;

  // Q^T as the B operand: lane (col, grp) holds head col, dims 32i + 8grp .. +8.
  const int G = a.group;
  const int hq = h * G + col;
  short8_t qv[4];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qs * a.q_s0 +
                         static_cast<int64_t>(col < G ? hq : 0) * a.q_s1 + 8 * grp;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      qv[i] = (col < G) ? *reinterpret_cast<const short8_t*>(qp + 32 * i) : short8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
  }

  float4_t acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[j][c] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;
  uint16_t* slab = lds[wave];
  const uint16_t* cache = static_cast<const uint16_t*>(a.cache);
  const int64_t head_off = static_cast<int64_t>(h) * kDim + 8 * grp;

  Tile cur;
  load_tile<NT>(a, cache, r, begin, lo, end, col, head_off, cur);
  for (int64_t base = begin; base <= end; base += 16) {
    Tile nxt;
    if constexpr (PREFETCH) {
      if (base + 16 <= end) load_tile<NT>(a, cache, r, base + 16, lo, end, col, head_off, nxt);
    }
    const uint64_t okmask = __ballot(cur.ok);  // bit j (j < 16): token j of the tile is visible

    float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) sc = Mfma<T>::k32(cur.k[i], qv[i], sc);

    float s[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      s[e] = ((okmask >> (4 * grp + e)) & 1u) ? sc[e] * a.scale_log2 : -INFINITY;
    float bm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    bm = max_xor32_f(max_xor16_f(bm));
    const float mn = fmaxf(m, bm);
    const float alpha = (mn == -INFINITY) ? 1.f : exp2f(m - mn);
    float p[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) p[e] = (s[e] == -INFINITY) ? 0.f : exp2f(s[e] - mn);
    l = l * alpha + ((p[0] + p[1]) + (p[2] + p[3]));
    if (__ballot(alpha != 1.f)) {
#pragma unroll
      for (int j = 0; j < 2; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) acc[j][c] *= alpha;
    }
    m = mn;

    // P^T as the B operand (tokens 4grp .. +4 of head col), as a hi/lo pair.
    uint32_t ph[4], pl[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split_hi_lo<T>(p[e], ph[e], pl[e]);
    const short4_t pb_hi = __builtin_bit_cast(short4_t, uint2{ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16)});
    const short4_t pb_lo = __builtin_bit_cast(short4_t, uint2{pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16)});

    // V tile -> LDS (row = token, natural layout), then read V^T.
    wave_lds_sync();
#pragma unroll
    for (int i = 0; i < 4; ++i)
      *reinterpret_cast<short8_t*>(slab + col * kRow + 32 * i + 8 * grp) = cur.v[i];
    wave_lds_sync();
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint2 rv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e)
        rv[e] = *reinterpret_cast<const uint2*>(slab + (4 * grp + e) * kRow + 64 * j + 4 * col);
      // A operand c: row col <-> dim 64j + 4col + c; k = tokens 4grp + e.
      short4_t av[4];
      av[0] = __builtin_bit_cast(short4_t, uint2{pack_lo16(rv[0].x, rv[1].x), pack_lo16(rv[2].x, rv[3].x)});
      av[1] = __builtin_bit_cast(short4_t, uint2{pack_hi16(rv[0].x, rv[1].x), pack_hi16(rv[2].x, rv[3].x)});
      av[2] = __builtin_bit_cast(short4_t, uint2{pack_lo16(rv[0].y, rv[1].y), pack_lo16(rv[2].y, rv[3].y)});
      av[3] = __builtin_bit_cast(short4_t, uint2{pack_hi16(rv[0].y, rv[1].y), pack_hi16(rv[2].y, rv[3].y)});
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[j][c] = Mfma<T>::k16(av[c], pb_hi, acc[j][c]);
        acc[j][c] = Mfma<T>::k16(av[c], pb_lo, acc[j][c]);
      }
    }
    if constexpr (PREFETCH) {
      cur = nxt;
    } else {
      if (base + 16 <= end) load_tile<NT>(a, cache, r, base + 16, lo, end, col, head_off, cur);
    }
  }

  const float lt = sum_xor32_f(sum_xor16_f(l));
  if (col >= G) return;
  write_decode_result<T>(a, r, qs, hq, split, item.ns, m, lt, acc, grp);
}

// The pipelined kernel (decode_split_lds_body) for block sizes that are
// multiples of 16: K and V tiles go straight from HBM to LDS.
template <typename T, int STAGES>
__global__ __launch_bounds__(256) void decode_split_lds_kernel(AttnArgs a) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  decode_split_lds_body<T, STAGES>(a, smem, blockIdx.x, blockDim.x >> 6);
}


// Blocks [0, R * head_groups): merge split partials of multi-split
// decode requests, kCombineHeads query heads per block, 32 lanes per head
// (4 dims each). Up to CAP splits are merged from one round of loads (the
// launch picks CAP >= the layout's split count when it is at most 32).
// Blocks after that: zero tokens outside every request, kZeroTokens each.
constexpr int kZeroTokens = 16;
constexpr int kCombineHeads = 8;

template <typename T, int CAP>
__global__ __launch_bounds__(256) void decode_combine_kernel(AttnArgs a, int32_t head_groups) {
  const int64_t R = a.num_requests;
  const int64_t combine_blocks = R * head_groups;
  if (static_cast<int64_t>(blockIdx.x) >= combine_blocks) {
    const int64_t first = a.qsl[0], last = a.qsl[R];
    const int64_t t0 = (blockIdx.x - combine_blocks) * kZeroTokens;
    const int64_t row = static_cast<int64_t>(a.num_q_heads) * a.head_dim;
    // Contiguous, 16-byte aligned token rows (the usual output): 16-byte
    // stores of zero bits (+0 in every dtype); otherwise element stores.
    const bool vec = a.o_s2 == 1 && a.o_s1 == a.head_dim && (row * static_cast<int64_t>(sizeof(T))) % 16 == 0 &&
                     (a.o_s0 * static_cast<int64_t>(sizeof(T))) % 16 == 0 &&
                     (reinterpret_cast<uintptr_t>(a.out) & 15u) == 0;
    for (int64_t t = t0; t < t0 + kZeroTokens && t < a.num_tokens; ++t) {
      if (t >= first && t < last) continue;
      T* op = static_cast<T*>(a.out) + t * a.o_s0;
      if (vec) {
        const int64_t chunks = row * static_cast<int64_t>(sizeof(T)) / 16;
        for (int64_t i = threadIdx.x; i < chunks; i += blockDim.x)
          reinterpret_cast<uint4*>(op)[i] = uint4{0u, 0u, 0u, 0u};
      } else {
        for (int64_t i = threadIdx.x; i < row; i += blockDim.x) {
          const int64_t hq = i / a.head_dim, d = i - hq * a.head_dim;
          Elem<T>::store(op + hq * a.o_s1 + d * a.o_s2, 0.f);
        }
      }
    }
    return;
  }
  const int64_t r = blockIdx.x / head_groups;
  const int hq = static_cast<int>(blockIdx.x % head_groups) * kCombineHeads + (threadIdx.x >> 5);
  if (hq >= a.num_q_heads) return;
  // (query token, splits) from the work-list kernel: -1 is not a decode
  // request, and a single split has written its output itself.
  const int2 req = a.decode_req[r];
  const int64_t qs = req.x, ns = req.y;
  const int d0 = (threadIdx.x & 31) * 4;
  if (ns < 0 && a.decode_only) {
    // A request with another query count in a batch whose hint promised
    // single-query requests only: no kernel computes its rows, so they are
    // made NaN rather than left holding whatever the output memory held.
    const int64_t q0 = a.qsl[r], q1 = a.qsl[r + 1];
    if (q0 < 0 || q1 > a.num_tokens) return;
    const uint32_t nan_bits = Elem<T>::to_bits(NAN);
    const uint32_t nan2 = nan_bits | (nan_bits << 16);
    for (int64_t t = q0; t < q1; ++t) {
      uint16_t* op = static_cast<uint16_t*>(a.out) + t * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1;
      *reinterpret_cast<uint2*>(op + d0) = uint2{nan2, nan2};
    }
    return;
  }
  if (ns < 0 || ns == 1 || ns > a.max_splits || qs < 0 || qs >= a.num_tokens) return;
  uint32_t w[2];
  if (ns == 0) {
    // Nothing visible: softmax over no keys is NaN in the reference.
    const uint32_t nan_bits = Elem<T>::to_bits(NAN);
    w[0] = w[1] = nan_bits | (nan_bits << 16);
  } else if (ns <= CAP) {
    // Up to CAP splits (the common case): every split's (max, sum) and
    // accumulator slice are loaded at once, one round trip after the table.
    const int sub = threadIdx.x & 31;
    const int64_t first_item = r * a.max_splits * a.num_q_heads + hq;
    const int cnt = static_cast<int>(ns);
    float2 ml = make_float2(-INFINITY, 0.f);
    if (sub < cnt) ml = a.ws_ml[first_item + sub * a.num_q_heads];
    const float* accp = a.ws_acc + first_item * kDim + d0;
    float4_t v[CAP];
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      const int k = j < cnt ? j : cnt - 1;  // indices past the last split re-read it, unused
      v[j] = *reinterpret_cast<const float4_t*>(accp + static_cast<int64_t>(k) * a.num_q_heads * kDim);
    }
    float mx = ml.x;  // lanes past the last split hold -inf and a zero sum
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 32));
    // A split with no visible key (m = -inf) weighs 0; so does every split
    // when none has one, and the output is then NaN (0 / 0).
    const float wgt = ml.x == -INFINITY ? 0.f : exp2f(ml.x - mx);
    float sum = wgt * ml.y;
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 32);
    float4_t o = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int j = 0; j < CAP; ++j) {
      const float wj = __shfl(wgt, j, 32);
      if (j < cnt) o += v[j] * wj;
    }
    const float inv = 1.f / sum;
    w[0] = Elem<T>::to_bits(o[0] * inv) | (Elem<T>::to_bits(o[1] * inv) << 16);
    w[1] = Elem<T>::to_bits(o[2] * inv) | (Elem<T>::to_bits(o[3] * inv) << 16);
  } else {
    // Two passes over the head's splits, 32 lanes wide: the maximum first,
    // then every split's weight exp2(m_s - max) from its own lane, so the
    // accumulator loads do not wait on a running maximum.
    const int sub = threadIdx.x & 31;
    const int64_t first_item = r * a.max_splits * a.num_q_heads + hq;
    float mx = -INFINITY;
    for (int64_t s0 = 0; s0 < ns; s0 += 32)
      if (s0 + sub < ns) mx = fmaxf(mx, a.ws_ml[first_item + (s0 + sub) * a.num_q_heads].x);
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) mx = fmaxf(mx, __shfl_xor(mx, m, 32));
    float sum = 0.f;
    float4_t o = {0.f, 0.f, 0.f, 0.f};
    for (int64_t s0 = 0; s0 < ns; s0 += 32) {
      float w = 0.f;
      if (s0 + sub < ns) {
        const float2 ml = a.ws_ml[first_item + (s0 + sub) * a.num_q_heads];
        // A split with no visible key (m = -inf) weighs 0; so does every
        // split when none has one, and the output is then NaN (0 / 0).
        w = ml.x == -INFINITY ? 0.f : exp2f(ml.x - mx);
        sum += w * ml.y;
      }
      const int cnt = ns - s0 < 32 ? static_cast<int>(ns - s0) : 32;
      const float* accp = a.ws_acc + (first_item + s0 * a.num_q_heads) * kDim + d0;
      // Eight splits per pass, their loads issued together (indices past
      // the last split re-read it and are not added).
      for (int k0 = 0; k0 < cnt; k0 += 8) {
        float4_t v[8];
        float wk[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) {
          const int k = k0 + j < cnt ? k0 + j : cnt - 1;
          wk[j] = __shfl(w, k, 32);
          v[j] = *reinterpret_cast<const float4_t*>(accp + static_cast<int64_t>(k) * a.num_q_heads * kDim);
        }
#pragma unroll
        for (int j = 0; j < 8; ++j)
          if (k0 + j < cnt) o += v[j] * wk[j];
      }
    }
#pragma unroll
    for (int m = 16; m >= 1; m >>= 1) sum += __shfl_xor(sum, m, 32);
    const float inv = 1.f / sum;
    w[0] = Elem<T>::to_bits(o[0] * inv) | (Elem<T>::to_bits(o[1] * inv) << 16);
    w[1] = Elem<T>::to_bits(o[2] * inv) | (Elem<T>::to_bits(o[3] * inv) << 16);
  }
  uint16_t* op = static_cast<uint16_t*>(a.out) + qs * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1;
  *reinterpret_cast<uint2*>(op + d0) = uint2{w[0], w[1]};
}


__global__ __launch_bounds__(kDecodeListThreads) void decode_items_kernel(AttnArgs a) { build_decode_list(a); }

struct DecodeTuning {
  bool lds_pipeline;  // the global->LDS pipelined kernel (block_size % 16 == 0)
  int waves;          // waves (KV heads) per workgroup
  int stages;         // tiles in flight per wave (pipelined kernel)
  bool prefetch;      // register prefetch (general kernel)
  bool nontemporal;   // non-temporal loads (general kernel)
};

DecodeTuning decode_tuning(const AttnArgs& a) {
  DecodeTuning t;
  t.lds_pipeline = a.block_size % 16 == 0 && a.split_tokens <= 2048;
  t.waves = 4;
  t.stages = 2;
  t.prefetch = false;
  t.nontemporal = false;
  if (const char* env = std::getenv("MVLLM_DECODE_KERNEL")) {
    if (std::strcmp(env, "general") == 0) t.lds_pipeline = false;
  }
  if (const char* env = std::getenv("MVLLM_DECODE_WAVES")) {
    const int v = std::atoi(env);
    if (v >= 1 && v <= kMaxWaves) t.waves = v;
  }
  if (const char* env = std::getenv("MVLLM_DECODE_STAGES")) {
    const int v = std::atoi(env);
    if (v >= 2 && v <= 4) t.stages = v;
  }
  if (const char* env = std::getenv("MVLLM_DECODE_PREFETCH")) t.prefetch = std::atoi(env) != 0;
  if (const char* env = std::getenv("MVLLM_DECODE_NT")) t.nontemporal = std::atoi(env) != 0;
  if (t.lds_pipeline && t.waves > 4) t.waves = 4;
  if (t.waves > a.num_kv_heads) t.waves = a.num_kv_heads;
  return t;
}

template <typename T, int STAGES>
int launch_lds_kernel(const AttnArgs& a, dim3 grid, int waves, hipStream_t s, hipEvent_t start,
                      hipEvent_t stop) {
  const size_t lds = static_cast<size_t>(waves) * STAGES * 2 * kTileBytes;
  if (lds > 64 * 1024) {
    static bool raised = false;  // per instantiation; the attribute is process-wide
    if (!raised) {
      MVLLM_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(decode_split_lds_kernel<T, STAGES>),
                                        hipFuncAttributeMaxDynamicSharedMemorySize,
                                        static_cast<int>(lds)));
      raised = true;
    }
  }
  hipExtLaunchKernelGGL(decode_split_lds_kernel<T, STAGES>, grid, dim3(64 * waves), lds, s, start, stop,
                        0, a);
  MVLLM_LAUNCH_CHECK("decode_split_lds_kernel");
  return MVLLM_OK;
}

template <typename T>
int launch_combine_t(const AttnArgs& a, hipStream_t s) {
  const int32_t head_groups = (a.num_q_heads + kCombineHeads - 1) / kCombineHeads;
  const int64_t blocks = a.num_requests * head_groups + (a.num_tokens + kZeroTokens - 1) / kZeroTokens;
  if (blocks > 0) {
    if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "combine grid too large");
    // Short splits on small batches give requests up to ~20 splits; they
    // still merge in one round of loads.
    const dim3 grid(static_cast<unsigned>(blocks)), block(32 * kCombineHeads);
    if (a.max_splits <= 8) hipLaunchKernelGGL((decode_combine_kernel<T, 8>), grid, block, 0, s, a, head_groups);
    else if (a.max_splits <= 16) hipLaunchKernelGGL((decode_combine_kernel<T, 16>), grid, block, 0, s, a, head_groups);
    else hipLaunchKernelGGL((decode_combine_kernel<T, 32>), grid, block, 0, s, a, head_groups);
    MVLLM_LAUNCH_CHECK("decode_combine_kernel");
  }
  return MVLLM_OK;
}

template <typename T>
int launch_decode_t(const AttnArgs& a, hipStream_t s, hipEvent_t start, hipEvent_t stop) {
  const DecodeTuning tune = decode_tuning(a);
  const int waves = tune.waves;
  const int groups = (a.num_kv_heads + waves - 1) / waves;

  if (a.num_requests > 0) {
    const int64_t blocks = a.num_requests * a.max_splits * groups;
    if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "decode grid too large (%lld workgroups)", (long long)blocks);
    if (!a.lists_ready) {
      if (int rc = launch_decode_lists(a, s)) return rc;
    } else if (a.width * a.block_size > INT32_MAX || a.num_tokens > INT32_MAX) {
      return fail(MVLLM_ERR_UNSUPPORTED, "decode positions beyond 2^31 are not supported");
    }
    const dim3 grid(static_cast<unsigned>(blocks));
    const dim3 block(64 * waves);
    if (tune.lds_pipeline) {
      int rc = MVLLM_OK;
      if (tune.stages == 2) rc = launch_lds_kernel<T, 2>(a, grid, waves, s, start, stop);
      else if (tune.stages == 3) rc = launch_lds_kernel<T, 3>(a, grid, waves, s, start, stop);
      else rc = launch_lds_kernel<T, 4>(a, grid, waves, s, start, stop);
      if (rc) return rc;
    } else {
      if (tune.prefetch && tune.nontemporal)
        hipExtLaunchKernelGGL(decode_split_kernel<T, true, true>, grid, block, 0, s, start, stop, 0, a);
      else if (tune.prefetch)
        hipExtLaunchKernelGGL(decode_split_kernel<T, true, false>, grid, block, 0, s, start, stop, 0, a);
      else if (tune.nontemporal)
        hipExtLaunchKernelGGL(decode_split_kernel<T, false, true>, grid, block, 0, s, start, stop, 0, a);
      else
        hipExtLaunchKernelGGL(decode_split_kernel<T, false, false>, grid, block, 0, s, start, stop, 0, a);
      MVLLM_LAUNCH_CHECK("decode_split_kernel");
    }
  }
  return launch_combine_t<T>(a, s);
}

}  // namespace

int launch_decode_lists(const AttnArgs& a, hipStream_t s) {
  if (a.num_requests <= 0) return MVLLM_OK;
  if (!a.decode_items || !a.decode_req) return fail(MVLLM_ERR_INVALID, "decode work list is missing");
  // Work-list records carry positions and token indices as int32.
  if (a.width * a.block_size > INT32_MAX || a.num_tokens > INT32_MAX)
    return fail(MVLLM_ERR_UNSUPPORTED, "decode positions beyond 2^31 are not supported");
  hipLaunchKernelGGL(decode_items_kernel, dim3(1), dim3(kDecodeListThreads), 0, s, a);
  MVLLM_LAUNCH_CHECK("decode_items_kernel");
  return MVLLM_OK;
}

int launch_decode(const AttnArgs& a, int32_t dtype, hipStream_t s, hipEvent_t start,
                  hipEvent_t stop) {
  if (a.head_dim != kDim) return fail(MVLLM_ERR_UNSUPPORTED, "decode kernel needs head_dim 128");
  if (dtype == MVLLM_DTYPE_BF16) return launch_decode_t<bf16_t>(a, s, start, stop);
  if (dtype == MVLLM_DTYPE_F16) return launch_decode_t<f16_t>(a, s, start, stop);
  return fail(MVLLM_ERR_UNSUPPORTED, "decode kernel needs bf16 or fp16");
}

bool decode_step_eligible(const AttnArgs& a) {
  if (a.head_dim != kDim || a.num_requests <= 0) return false;
  // The default shape only (fewer KV heads than waves: the spare waves of
  // the step's workgroups end at once, as the pipelined kernel's do).
  const DecodeTuning tune = decode_tuning(a);
  const int waves = a.num_kv_heads < kStepDecodeWaves ? a.num_kv_heads : kStepDecodeWaves;
  return tune.lds_pipeline && tune.waves == waves && tune.stages == 2;
}

int64_t decode_step_blocks(const AttnArgs& a) {
  return a.num_requests * a.max_splits * ((a.num_kv_heads + kStepDecodeWaves - 1) / kStepDecodeWaves);
}

int launch_decode_combine(const AttnArgs& a, int32_t dtype, hipStream_t s) {
  if (dtype == MVLLM_DTYPE_BF16) return launch_combine_t<bf16_t>(a, s);
  if (dtype == MVLLM_DTYPE_F16) return launch_combine_t<f16_t>(a, s);
  return fail(MVLLM_ERR_UNSUPPORTED, "decode kernel needs bf16 or fp16");
}

}  // namespace mvllm
