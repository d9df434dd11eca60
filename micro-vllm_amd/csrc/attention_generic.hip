// Any-shape ragged paged attention: one workgroup of W waves per (token,
// query head).
//
// This kernel carries the shapes the specialised kernels do not (fp32,
// head_dim other than 128, query-head groups above 16, non-contiguous
// rows): each wave walks every W-th block of 64 keys, each lane scoring
// one key, then accumulates P.V with lanes spread over head_dim (one
// instantiation per bound of 64, 128, 256 and 512 elements, so the loops
// over a lane's elements and over a block's keys unroll without guards on
// elements past head_dim's bound). Online softmax in fp32 (exp2 domain) in
// the manner of FlashAttention-2 (Dao, 2023); the waves' partial states are
// merged through LDS at the end, so a long visible range costs 1/W of the
// dependent memory round trips of one wave walking it alone. W is 4 when
// the block table reaches at most 1,024 keys (more waves would find no
// block to walk) and 16 beyond (8 for head_dim above 128, whose
// accumulators do not fit the register share of 16 waves).
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

// The 16 bytes at p (16-byte aligned) as 16 / sizeof(T) floats.
template <typename T>
__device__ __forceinline__ void load16(const T* p, float (&f)[16 / sizeof(T)]) {
  const uint4 w = *reinterpret_cast<const uint4*>(p);
  const uint32_t ws[4] = {w.x, w.y, w.z, w.w};
  if constexpr (sizeof(T) == 4) {
#pragma unroll
    for (int i = 0; i < 4; ++i) f[i] = __uint_as_float(ws[i]);
  } else {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      f[2 * i] = Elem<T>::from_bits(ws[i] & 0xFFFFu);
      f[2 * i + 1] = Elem<T>::from_bits(ws[i] >> 16);
    }
  }
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

// DPL: head_dim elements per lane in the P.V accumulation (head_dim <= 64 * DPL);
// WAVES: waves per workgroup, each walking every WAVES-th block of 64 keys.
template <typename T, int DPL, int WAVES>
__global__ __launch_bounds__(64 * WAVES) void attention_generic_kernel(AttnArgs a) {
  const int64_t t = blockIdx.x;
  const int hq = blockIdx.y;
  const int lane = threadIdx.x & 63;
  const int wave = threadIdx.x >> 6;
  const int D = a.head_dim;
  T* out = static_cast<T*>(a.out) + t * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1;

  const int64_t r = request_of(a, t);
  const bool covered = r < a.num_requests && a.qsl[r] <= t && t < a.qsl[r + 1];
  if (!covered) {
    if (a.mode == 0)
      for (int d = threadIdx.x; d < D; d += 64 * WAVES) Elem<T>::store(out + d * a.o_s2, 0.f);
    return;
  }
  const int64_t qs = a.qsl[r];
  if (a.mode == 1 && a.qsl[r + 1] - qs == 1) return;

  __shared__ float qsh[64 * DPL];
  const T* q = static_cast<const T*>(a.q) + t * a.q_s0 + static_cast<int64_t>(hq) * a.q_s1;
  for (int d = threadIdx.x; d < D; d += 64 * WAVES) qsh[d] = Elem<T>::load(q + d * a.q_s2) * a.scale_log2;
  __syncthreads();

  int64_t lo, hi;
  visible_range(a, r, qs, t, lo, hi);
  const int kvh = hq / a.group;
  const T* cache = static_cast<const T*>(a.cache);
  float acc[DPL];
#pragma unroll
  for (int j = 0; j < DPL; ++j) acc[j] = 0.f;
  float m = -INFINITY, l = 0.f;
  // Key rows contiguous and 16-byte aligned: each lane reads its row in
  // 16-byte pieces (a quarter or an eighth of the load instructions, each
  // of which touches one cache line per lane).
  constexpr int kVec = 16 / static_cast<int>(sizeof(T));
  const bool vec_rows = a.c_s[4] == 1 && D % kVec == 0 && a.c_s[1] % kVec == 0 && a.c_s[2] % kVec == 0 &&
                        a.c_s[3] % kVec == 0 && (reinterpret_cast<uintptr_t>(a.cache) & 15u) == 0;

  for (int64_t base = lo + 64 * wave; base <= hi; base += 64 * WAVES) {
    const int64_t p = base + lane;
    int64_t row = -1;  // element offset of this lane's key row
    if (p <= hi) {
      const int64_t b = block_of(a, r, p);
      if (b >= 0)
        row = b * a.c_s[1] + (p % a.block_size) * a.c_s[2] + static_cast<int64_t>(kvh) * a.c_s[3];
    }
    // Four independent partial sums, so a lane keeps several loads of its
    // key row in flight instead of one chain of dependent ones.
    float s = -INFINITY;
    if (row >= 0) {
      const T* kp = cache + row;
      const int64_t ks = a.c_s[4];
      float d0 = 0.f, d1 = 0.f, d2 = 0.f, d3 = 0.f;
      int d = 0;
      if (vec_rows) {
#pragma unroll 16
        for (; d < D; d += kVec) {
          float f[kVec];
          load16(kp + d, f);
#pragma unroll
          for (int e = 0; e < kVec; e += 4) {
            d0 = __builtin_fmaf(qsh[d + e], f[e], d0);
            d1 = __builtin_fmaf(qsh[d + e + 1], f[e + 1], d1);
            d2 = __builtin_fmaf(qsh[d + e + 2], f[e + 2], d2);
            d3 = __builtin_fmaf(qsh[d + e + 3], f[e + 3], d3);
          }
        }
      } else {
#pragma unroll 8
        for (; d + 4 <= D; d += 4) {
          d0 = __builtin_fmaf(qsh[d], Elem<T>::load(kp + d * ks), d0);
          d1 = __builtin_fmaf(qsh[d + 1], Elem<T>::load(kp + (d + 1) * ks), d1);
          d2 = __builtin_fmaf(qsh[d + 2], Elem<T>::load(kp + (d + 2) * ks), d2);
          d3 = __builtin_fmaf(qsh[d + 3], Elem<T>::load(kp + (d + 3) * ks), d3);
        }
        for (; d < D; ++d) d0 = __builtin_fmaf(qsh[d], Elem<T>::load(kp + d * ks), d0);
      }
      s = (d0 + d1) + (d2 + d3);
    }
    const float mn = fmaxf(m, wave_max(s));
    const float alpha = (mn == -INFINITY) ? 1.f : exp2f(m - mn);
    const float pr = (s == -INFINITY) ? 0.f : exp2f(s - mn);
    l = l * alpha + wave_sum(pr);
#pragma unroll
    for (int j = 0; j < DPL; ++j) acc[j] *= alpha;
    // P.V without a branch per key, so the loads of several keys overlap:
    // a key with no row reads row 0 of the V plane and adds nothing (a
    // select, not a product with 0, so a non-finite stale value stays out).
    const int count = static_cast<int>(hi - base + 1 < 64 ? hi - base + 1 : 64);
#pragma unroll 32
    for (int k = 0; k < count; ++k) {
      const int64_t vrow = __shfl(row, k, 64);
      const float pk = __shfl(pr, k, 64);
      const bool has = vrow >= 0;
      const T* vp = cache + a.c_s[0] + (has ? vrow : 0);
#pragma unroll
      for (int j = 0; j < DPL; ++j) {
        const int d = lane + 64 * j;
        if (d < D) {
          const float pv = pk * Elem<T>::load(vp + d * a.c_s[4]);
          acc[j] += has ? pv : 0.f;
        }
      }
    }
    m = mn;
  }
  // Merge the waves' (offset, sum, accumulator) states; a wave that saw no
  // key holds (-inf, 0, 0) and weighs nothing.
  __shared__ float msh[WAVES], lsh[WAVES];
  __shared__ float accsh[WAVES][64 * DPL];
  if (lane == 0) {
    msh[wave] = m;
    lsh[wave] = l;
  }
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) accsh[wave][d] = acc[j];
  }
  __syncthreads();
  if (wave != 0) return;
  float mx = -INFINITY;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) mx = fmaxf(mx, msh[w]);
  float weight[WAVES];
  float total = 0.f;
#pragma unroll
  for (int w = 0; w < WAVES; ++w) {
    weight[w] = msh[w] == -INFINITY ? 0.f : exp2f(msh[w] - mx);
    total += weight[w] * lsh[w];
  }
  const float inv = 1.f / total;  // an empty visible range gives 0/0 = NaN, as the reference's softmax does
#pragma unroll
  for (int j = 0; j < DPL; ++j) {
    const int d = lane + 64 * j;
    if (d < D) {
      float o = 0.f;
#pragma unroll
      for (int w = 0; w < WAVES; ++w) o += weight[w] * accsh[w][d];
      Elem<T>::store(out + d * a.o_s2, o * inv);
    }
  }
}

template <typename T, int DPL, int WAVES>
void launch_generic_w(const AttnArgs& a, hipStream_t s) {
  const dim3 grid(static_cast<unsigned>(a.num_tokens), static_cast<unsigned>(a.num_q_heads));
  hipLaunchKernelGGL((attention_generic_kernel<T, DPL, WAVES>), grid, dim3(64 * WAVES), 0, s, a);
}

template <typename T>
int launch_generic_t(const AttnArgs& a, int dpl, hipStream_t s) {
  const bool long_reach = a.width * a.block_size > 1024;
  switch (dpl) {
    case 1: long_reach ? launch_generic_w<T, 1, 16>(a, s) : launch_generic_w<T, 1, 4>(a, s); break;
    case 2: long_reach ? launch_generic_w<T, 2, 16>(a, s) : launch_generic_w<T, 2, 4>(a, s); break;
    case 4: long_reach ? launch_generic_w<T, 4, 8>(a, s) : launch_generic_w<T, 4, 4>(a, s); break;
    default: long_reach ? launch_generic_w<T, 8, 8>(a, s) : launch_generic_w<T, 8, 4>(a, s); break;
  }
  return MVLLM_OK;
}

}  // namespace

int launch_generic(const AttnArgs& a, int32_t dtype, hipStream_t s) {
  if (a.head_dim > 64 * kMaxDimPerLane)
    return fail(MVLLM_ERR_UNSUPPORTED, "head_dim %d exceeds %d", a.head_dim, 64 * kMaxDimPerLane);
  if (a.num_tokens == 0 || a.num_q_heads == 0) return MVLLM_OK;
  if (a.num_tokens > INT32_MAX || a.num_q_heads > 65535)
    return fail(MVLLM_ERR_INVALID, "generic attention grid too large");
  const int dpl = a.head_dim <= 64 ? 1 : a.head_dim <= 128 ? 2 : a.head_dim <= 256 ? 4 : 8;
  int rc = MVLLM_OK;
  switch (dtype) {
    case MVLLM_DTYPE_F32: rc = launch_generic_t<float>(a, dpl, s); break;
    case MVLLM_DTYPE_F16: rc = launch_generic_t<f16_t>(a, dpl, s); break;
    case MVLLM_DTYPE_BF16: rc = launch_generic_t<bf16_t>(a, dpl, s); break;
    default: return fail(MVLLM_ERR_UNSUPPORTED, "unsupported dtype code %d", dtype);
  }
  if (rc) return rc;
  MVLLM_LAUNCH_CHECK("attention_generic_kernel");
  return MVLLM_OK;
}

}  // namespace mvllm
