// Any-shape ragged paged attention: one wavefront per (token, query head).
//
// This kernel carries the shapes the specialised kernels do not (fp32,
// head_dim other than 128, query-head groups above 16, non-contiguous
// rows): lanes walk 64 keys at a time, each lane scoring one key, then
// accumulate P.V with lanes spread over head_dim. Online softmax in fp32
// (exp2 domain) in the manner of FlashAttention-2 (Dao, 2023).
#include <cmath>

#include "attention.h"

namespace mvllm {
namespace {

constexpr int kMaxDimPerLane = 8;  // head_dim <= 512

__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = fmaxf(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v += __shfl_xor(v, m, 64);
  return v;
}

// Largest i in [0, R] with qsl[i] <= t (qsl is non-decreasing).
__device__ __forceinline__ int64_t request_of(const AttnArgs& a, int64_t t) {
  int64_t lo = 0, hi = a.num_requests;
  while (lo < hi) {
    const int64_t mid = (lo + hi + 1) >> 1;
    if (a.qsl[mid] <= t) lo = mid; else hi = mid - 1;
  }
  return lo;
}

template <typename T>
__global__ __launch_bounds__(64) void attention_generic_kernel(AttnArgs a) {
  const int64_t t = blockIdx.x;
  const int hq = blockIdx.y;
  const int lane = threadIdx.x;
  const int D = a.head_dim;
  T* out = static_cast<T*>(a.out) + t * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1;

  const int64_t r = request_of(a, t);
  const bool covered = r < a.num_requests && a.qsl[r] <= t && t < a.qsl[r + 1];
  if (!covered) {
    if (a.mode == 0)
      for (int d = lane; d < D; d += 64) Elem<T>::store(out + d * a.o_s2, 0.f);
    return;
  }
  const int64_t qs = a.qsl[r];
  if (a.mode == 1 && a.qsl[r + 1] - qs == 1) return;

  __shared__ float qsh[64 * kMaxDimPerLane];
  const T* q = static_cast<const T*>(a.q) + t * a.q_s0 + static_cast<int64_t>(hq) * a.q_s1;
  for (int d = lane; d < D; d += 64) qsh[d] = Elem<T>::load(q + d * a.q_s2) * a.scale_log2;
  __syncthreads();

  int64_t lo, hi;
  visible_range(a, r, qs, t, lo, hi);
  const int kvh = hq / a.group;
  const T* cache = static_cast<const T*>(a.cache);
  float acc[kMaxDimPerLane];
#pragma unroll
  for (int j = 0; j < kMaxDimPerLane; ++j) acc[j] = 0.f;
  float m = -INFINITY, l = 0.f;

  for (int64_t base = lo; base <= hi; base += 64) {
    const int64_t p = base + lane;
    int64_t row = -1;  // element offset of this lane's key row
    if (p <= hi) {
      const int64_t b = block_of(a, r, p);
      if (b >= 0)
        row = b * a.c_s[1] + (p % a.block_size) * a.c_s[2] + static_cast<int64_t>(kvh) * a.c_s[3];
    }
    float s = -INFINITY;
    if (row >= 0) {
      float dot = 0.f;
      for (int d = 0; d < D; ++d) dot += qsh[d] * Elem<T>::load(cache + row + d * a.c_s[4]);
      s = dot;
    }
    const float mn = fmaxf(m, wave_max(s));
    const float alpha = (mn == -INFINITY) ? 1.f : exp2f(m - mn);
    const float pr = (s == -INFINITY) ? 0.f : exp2f(s - mn);
    l = l * alpha + wave_sum(pr);
#pragma unroll
    for (int j = 0; j < kMaxDimPerLane; ++j) acc[j] *= alpha;
    const int count = static_cast<int>(hi - base + 1 < 64 ? hi - base + 1 : 64);
    for (int k = 0; k < count; ++k) {
      const int64_t vrow = __shfl(row, k, 64);
      const float pk = __shfl(pr, k, 64);
      if (vrow < 0) continue;
#pragma unroll
      for (int j = 0; j < kMaxDimPerLane; ++j) {
        const int d = lane + 64 * j;
        if (d < D) acc[j] += pk * Elem<T>::load(cache + a.c_s[0] + vrow + d * a.c_s[4]);
      }
    }
    m = mn;
  }
  const float inv = 1.f / l;  // an empty visible range gives 0/0 = NaN, as the reference's softmax does
#pragma unroll
  for (int j = 0; j < kMaxDimPerLane; ++j) {
    const int d = lane + 64 * j;
    if (d < D) Elem<T>::store(out + d * a.o_s2, acc[j] * inv);
  }
}

}  // namespace

int launch_generic(const AttnArgs& a, int32_t dtype, hipStream_t s) {
  if (a.head_dim > 64 * kMaxDimPerLane)
    return fail(MVLLM_ERR_UNSUPPORTED, "head_dim %d exceeds %d", a.head_dim, 64 * kMaxDimPerLane);
  if (a.num_tokens == 0 || a.num_q_heads == 0) return MVLLM_OK;
  if (a.num_tokens > INT32_MAX || a.num_q_heads > 65535)
    return fail(MVLLM_ERR_INVALID, "generic attention grid too large");
  const dim3 grid(static_cast<unsigned>(a.num_tokens), static_cast<unsigned>(a.num_q_heads));
  switch (dtype) {
    case MVLLM_DTYPE_F32:
      hipLaunchKernelGGL(attention_generic_kernel<float>, grid, dim3(64), 0, s, a);
      break;
    case MVLLM_DTYPE_F16:
      hipLaunchKernelGGL(attention_generic_kernel<f16_t>, grid, dim3(64), 0, s, a);
      break;
    case MVLLM_DTYPE_BF16:
      hipLaunchKernelGGL(attention_generic_kernel<bf16_t>, grid, dim3(64), 0, s, a);
      break;
    default:
      return fail(MVLLM_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  }
  MVLLM_LAUNCH_CHECK("attention_generic_kernel");
  return MVLLM_OK;
}

}  // namespace mvllm
