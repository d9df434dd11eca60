// Split-KV ragged decode on gfx950 matrix cores (head_dim 128, bf16/fp16).
//
// Work item: (KV head, split of the visible context, request). One wavefront
// owns one KV head; a workgroup holds up to 8 waves = 8 consecutive KV heads
// of the same (request, split), so together they stream whole token rows
// (all heads of a token are contiguous in the cache) with 16-byte loads.
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
// belong to no request.
#include <cmath>

#include "attention.h"

namespace mvllm {
namespace {

constexpr int kDim = 128;
constexpr int kRow = 144;  // LDS row stride (elements): 288 B keeps both LDS access patterns conflict-free
constexpr int kMaxWaves = 8;

template <typename T>
__device__ __forceinline__ void split_hi_lo(float p, uint32_t& hi, uint32_t& lo) {
  hi = Elem<T>::to_bits(p);
  lo = Elem<T>::to_bits(p - Elem<T>::from_bits(hi));
}

template <typename T>
__global__ __launch_bounds__(512) void decode_split_kernel(AttnArgs a) {
  __shared__ __attribute__((aligned(16))) uint16_t lds[kMaxWaves][16 * kRow];
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  const int waves = blockDim.x >> 6;
  const int h = blockIdx.x * waves + wave;
  const int split = blockIdx.y;
  const int64_t r = blockIdx.z;
  if (h >= a.num_kv_heads) return;
  const int64_t qs = a.qsl[r];
  if (qs < 0 || qs >= a.num_tokens || a.qsl[r + 1] - qs != 1) return;
  int64_t lo, hi;
  visible_range(a, r, qs, qs, lo, hi);
  if (hi < lo) return;
  const int64_t base0 = lo & ~int64_t(15);
  const int64_t begin = base0 + static_cast<int64_t>(split) * a.split_tokens;
  if (begin > hi) return;
  const int64_t end = (begin + a.split_tokens - 1 < hi) ? begin + a.split_tokens - 1 : hi;

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

  for (int64_t base = begin; base <= end; base += 16) {
    // This lane loads token `col` of the tile (A operand row), dims 32i + 8grp.
    const int64_t tk = base + col;
    bool ok = tk >= lo && tk <= end;
    int64_t off = 0;
    if (ok) {
      const int64_t b = block_of(a, r, tk);
      ok = b >= 0;
      off = b * a.c_s[1] + (tk % a.block_size) * a.c_s[2] + head_off;
    }
    short8_t kv[4], vv[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      kv[i] = ok ? *reinterpret_cast<const short8_t*>(cache + off + 32 * i) : short8_t{0, 0, 0, 0, 0, 0, 0, 0};
      vv[i] = ok ? *reinterpret_cast<const short8_t*>(cache + a.c_s[0] + off + 32 * i) : short8_t{0, 0, 0, 0, 0, 0, 0, 0};
    }
    const uint64_t okmask = __ballot(ok);  // bit j (j < 16): token j of the tile is visible

    float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) sc = Mfma<T>::k32(kv[i], qv[i], sc);

    float s[4];
#pragma unroll
    for (int e = 0; e < 4; ++e)
      s[e] = ((okmask >> (4 * grp + e)) & 1u) ? sc[e] * a.scale_log2 : -INFINITY;
    float bm = fmaxf(fmaxf(s[0], s[1]), fmaxf(s[2], s[3]));
    bm = fmaxf(bm, shfl_xor_f(bm, 16));
    bm = fmaxf(bm, shfl_xor_f(bm, 32));
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
      *reinterpret_cast<short8_t*>(slab + col * kRow + 32 * i + 8 * grp) = vv[i];
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
  }

  // acc[j][c][e] is O[head col][dim 64j + 16grp + 4e + c] (unnormalised).
  const float l2 = l + shfl_xor_f(l, 16);
  const float lt = l2 + shfl_xor_f(l2, 32);
  if (col >= G) return;
  const int64_t ns = decode_num_splits(lo, hi, a.split_tokens);
  if (ns == 1) {
    const float inv = 1.f / lt;
    uint16_t* op = static_cast<uint16_t*>(a.out) + qs * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1;
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint32_t w[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) {
        const int i0 = 2 * i, i1 = 2 * i + 1;
        w[i] = Elem<T>::to_bits(acc[j][i0 & 3][i0 >> 2] * inv) |
               (Elem<T>::to_bits(acc[j][i1 & 3][i1 >> 2] * inv) << 16);
      }
      uint4* dst = reinterpret_cast<uint4*>(op + 64 * j + 16 * grp);
      dst[0] = uint4{w[0], w[1], w[2], w[3]};
      dst[1] = uint4{w[4], w[5], w[6], w[7]};
    }
    return;
  }
  const int64_t item = (r * a.max_splits + split) * a.num_q_heads + hq;
  float* wp = a.ws_acc + item * kDim;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    float4_t* dst = reinterpret_cast<float4_t*>(wp + 64 * j + 16 * grp);
#pragma unroll
    for (int e = 0; e < 4; ++e)
      dst[e] = float4_t{acc[j][0][e], acc[j][1][e], acc[j][2][e], acc[j][3][e]};
  }
  if (grp == 0) a.ws_ml[item] = float2{m, lt};
}

// Blocks [0, R): merge split partials of multi-split decode requests.
// Blocks [R, R + ceil(N / kZeroTokens)): zero tokens outside every request.
constexpr int kZeroTokens = 16;

template <typename T>
__global__ __launch_bounds__(256) void decode_combine_kernel(AttnArgs a) {
  const int64_t R = a.num_requests;
  if (blockIdx.x >= R) {
    const int64_t first = a.qsl[0], last = a.qsl[R];
    const int64_t t0 = (blockIdx.x - R) * kZeroTokens;
    const int64_t row = static_cast<int64_t>(a.num_q_heads) * a.head_dim;
    for (int64_t t = t0; t < t0 + kZeroTokens && t < a.num_tokens; ++t) {
      if (t >= first && t < last) continue;
      T* op = static_cast<T*>(a.out) + t * a.o_s0;
      for (int64_t i = threadIdx.x; i < row; i += blockDim.x) {
        const int64_t hq = i / a.head_dim, d = i - hq * a.head_dim;
        Elem<T>::store(op + hq * a.o_s1 + d * a.o_s2, 0.f);
      }
    }
    return;
  }
  const int64_t r = blockIdx.x;
  const int64_t qs = a.qsl[r];
  if (qs < 0 || qs >= a.num_tokens || a.qsl[r + 1] - qs != 1) return;
  int64_t lo, hi;
  visible_range(a, r, qs, qs, lo, hi);
  const int64_t ns = decode_num_splits(lo, hi, a.split_tokens);
  if (ns == 1) return;
  uint16_t* op = static_cast<uint16_t*>(a.out) + qs * a.o_s0;
  for (int idx = threadIdx.x; idx < a.num_q_heads * 16; idx += blockDim.x) {
    const int hq = idx >> 4;
    const int d0 = (idx & 15) * 8;
    uint32_t w[4];
    if (ns == 0) {
      // Nothing visible: softmax over no keys is NaN in the reference.
      const uint32_t nan_bits = Elem<T>::to_bits(NAN);
#pragma unroll
      for (int i = 0; i < 4; ++i) w[i] = nan_bits | (nan_bits << 16);
    } else {
      float mx = -INFINITY;
      for (int64_t s = 0; s < ns; ++s)
        mx = fmaxf(mx, a.ws_ml[(r * a.max_splits + s) * a.num_q_heads + hq].x);
      float sum = 0.f;
      float o[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
      for (int64_t s = 0; s < ns; ++s) {
        const int64_t item = (r * a.max_splits + s) * a.num_q_heads + hq;
        const float2 ml = a.ws_ml[item];
        const float wgt = (ml.x == -INFINITY) ? 0.f : exp2f(ml.x - mx);
        sum += wgt * ml.y;
        const float4_t* src = reinterpret_cast<const float4_t*>(a.ws_acc + item * kDim + d0);
        const float4_t v0 = src[0], v1 = src[1];
        o[0] += wgt * v0[0]; o[1] += wgt * v0[1]; o[2] += wgt * v0[2]; o[3] += wgt * v0[3];
        o[4] += wgt * v1[0]; o[5] += wgt * v1[1]; o[6] += wgt * v1[2]; o[7] += wgt * v1[3];
      }
      const float inv = 1.f / sum;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        w[i] = Elem<T>::to_bits(o[2 * i] * inv) | (Elem<T>::to_bits(o[2 * i + 1] * inv) << 16);
    }
    *reinterpret_cast<uint4*>(op + static_cast<int64_t>(hq) * a.o_s1 + d0) = uint4{w[0], w[1], w[2], w[3]};
  }
}

template <typename T>
int launch_decode_t(const AttnArgs& a, hipStream_t s) {
  const int waves = a.num_kv_heads < kMaxWaves ? a.num_kv_heads : kMaxWaves;
  const int groups = (a.num_kv_heads + waves - 1) / waves;
  if (a.max_splits > 65535 || a.num_requests > 65535)
    return fail(MVLLM_ERR_INVALID, "decode grid too large (%d splits, %lld requests)",
                a.max_splits, (long long)a.num_requests);
  if (a.num_requests > 0) {
    hipLaunchKernelGGL(decode_split_kernel<T>,
                       dim3(groups, a.max_splits, static_cast<unsigned>(a.num_requests)),
                       dim3(64 * waves), 0, s, a);
    MVLLM_LAUNCH_CHECK("decode_split_kernel");
  }
  const int64_t blocks = a.num_requests + (a.num_tokens + kZeroTokens - 1) / kZeroTokens;
  if (blocks > 0) {
    if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "combine grid too large");
    hipLaunchKernelGGL(decode_combine_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(256),
                       0, s, a);
    MVLLM_LAUNCH_CHECK("decode_combine_kernel");
  }
  return MVLLM_OK;
}

}  // namespace

int launch_decode(const AttnArgs& a, int32_t dtype, hipStream_t s) {
  if (a.head_dim != kDim) return fail(MVLLM_ERR_UNSUPPORTED, "decode kernel needs head_dim 128");
  if (dtype == MVLLM_DTYPE_BF16) return launch_decode_t<bf16_t>(a, s);
  if (dtype == MVLLM_DTYPE_F16) return launch_decode_t<f16_t>(a, s);
  return fail(MVLLM_ERR_UNSUPPORTED, "decode kernel needs bf16 or fp16");
}

}  // namespace mvllm
