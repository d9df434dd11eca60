// Shared host/device helpers of the gfx950 paged-attention library.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <cstdarg>
#include <cstdio>

#include "mvllm_amd.h"

namespace mvllm {

// ---------------------------------------------------------------- errors ----

// Records the failure text for mvllm_last_error() and returns `code`.
int fail(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));
void clear_error();

#define MVLLM_HIP_TRY(expr)                                                   \
  do {                                                                        \
    hipError_t mvllm_status_ = (expr);                                        \
    if (mvllm_status_ != hipSuccess)                                          \
      return ::mvllm::fail(MVLLM_ERR_HIP, "%s failed: %s", #expr,             \
                           hipGetErrorString(mvllm_status_));                 \
  } while (0)

// After a kernel launch: report a launch failure (bad configuration etc.).
#define MVLLM_LAUNCH_CHECK(name)                                              \
  do {                                                                        \
    hipError_t mvllm_status_ = hipGetLastError();                             \
    if (mvllm_status_ != hipSuccess)                                          \
      return ::mvllm::fail(MVLLM_ERR_HIP, "launch of %s failed: %s", name,    \
                           hipGetErrorString(mvllm_status_));                 \
  } while (0)

inline int64_t dtype_bytes(int32_t dtype) {
  switch (dtype) {
    case MVLLM_DTYPE_F32: return 4;
    case MVLLM_DTYPE_F16: return 2;
    case MVLLM_DTYPE_BF16: return 2;
    default: return 0;
  }
}

inline const char* dtype_name(int32_t dtype) {
  switch (dtype) {
    case MVLLM_DTYPE_F32: return "float32";
    case MVLLM_DTYPE_F16: return "float16";
    case MVLLM_DTYPE_BF16: return "bfloat16";
    default: return "unknown";
  }
}

inline bool aligned16(const void* p) {
  return (reinterpret_cast<uintptr_t>(p) & 15u) == 0;
}

inline int64_t ceil_div(int64_t a, int64_t b) { return (a + b - 1) / b; }

// -------------------------------------------------------- element types ----

// 16-bit storage types are carried as raw bits; arithmetic is always fp32.
struct bf16_t { uint16_t bits; };
struct f16_t { uint16_t bits; };

typedef short short4_t __attribute__((ext_vector_type(4)));
typedef short short8_t __attribute__((ext_vector_type(8)));
typedef _Float16 half4_t __attribute__((ext_vector_type(4)));
typedef _Float16 half8_t __attribute__((ext_vector_type(8)));
typedef float float4_t __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float bf16_bits_to_float(uint32_t bits16) {
  return __uint_as_float(bits16 << 16);
}

// fp32 -> bf16 bits, round to nearest even (the IEEE conversion the
// hardware implements on gfx950); NaN stays NaN.
__device__ __forceinline__ uint32_t float_to_bf16_bits(float f) {
  const __bf16 b = static_cast<__bf16>(f);
  return __builtin_bit_cast(uint16_t, b);
}

__device__ __forceinline__ float f16_bits_to_float(uint32_t bits16) {
  _Float16 h;
  uint16_t b = static_cast<uint16_t>(bits16);
  __builtin_memcpy(&h, &b, 2);
  return static_cast<float>(h);
}

__device__ __forceinline__ uint32_t float_to_f16_bits(float f) {
  _Float16 h = static_cast<_Float16>(f);  // v_cvt_f16_f32: round to nearest even
  uint16_t b;
  __builtin_memcpy(&b, &h, 2);
  return b;
}

template <typename T> struct Elem;

template <> struct Elem<float> {
  static constexpr int32_t code = MVLLM_DTYPE_F32;
  __device__ static float load(const float* p) { return *p; }
  __device__ static void store(float* p, float v) { *p = v; }
};

template <> struct Elem<bf16_t> {
  static constexpr int32_t code = MVLLM_DTYPE_BF16;
  __device__ static float load(const bf16_t* p) { return bf16_bits_to_float(p->bits); }
  __device__ static void store(bf16_t* p, float v) {
    p->bits = static_cast<uint16_t>(float_to_bf16_bits(v));
  }
  __device__ static float from_bits(uint32_t b) { return bf16_bits_to_float(b); }
  __device__ static uint32_t to_bits(float v) { return float_to_bf16_bits(v); }
};

template <> struct Elem<f16_t> {
  static constexpr int32_t code = MVLLM_DTYPE_F16;
  __device__ static float load(const f16_t* p) { return f16_bits_to_float(p->bits); }
  __device__ static void store(f16_t* p, float v) {
    p->bits = static_cast<uint16_t>(float_to_f16_bits(v));
  }
  __device__ static float from_bits(uint32_t b) { return f16_bits_to_float(b); }
  __device__ static uint32_t to_bits(float v) { return float_to_f16_bits(v); }
};

// ------------------------------------------------------- wave utilities ----

// Lane exchanges across 16- and 32-lane halves in one VALU instruction each
// (gfx950 v_permlane16_swap / v_permlane32_swap with both operands x): the
// two results hold x of this lane and of lane ^ 16 (^ 32), in an order that
// depends on the lane, so they feed only order-free combinations (max, sum).
__device__ __forceinline__ float max_xor16_f(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32_f(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16_f(float x) {
  const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32_f(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Orders this wave's LDS writes before its later LDS reads (and vice versa)
// without a workgroup barrier: the waves of one workgroup never share LDS
// rows in the decode kernel.
__device__ __forceinline__ void wave_lds_sync() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
}

// Direct HBM -> LDS load of 16 bytes per lane (global_load_lds_dwordx4):
// lane l's 16 bytes land at LDS byte address lds_base + 16 * l (lds_base is
// wave-uniform). Issued through inline assembly so that the compiler does not
// track the LDS write; callers order it with explicit s_waitcnt vmcnt counts.
// The assembly sets M0, which the compiler treats as reserved (it warns about
// the clobber): the kernels that use these loads contain no compiler-generated
// M0 use, which their assembly shows.
__device__ __forceinline__ void lds_dma_load16(const void* global_ptr, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off"
      :
      : "v"(global_ptr), "s"(__builtin_amdgcn_readfirstlane(lds_base))
      : "memory", "m0");
}

// lds_dma_load16 for data read exactly once (the decode kernel's K/V
// stream): the non-temporal hint lets the lines leave the caches first
// instead of displacing data that is reused.
__device__ __forceinline__ void lds_dma_load16_stream(const void* global_ptr, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, off nt"
      :
      : "v"(global_ptr), "s"(__builtin_amdgcn_readfirstlane(lds_base))
      : "memory", "m0");
}

// lds_dma_load16 with a wave-uniform 64-bit base in SGPRs and a per-lane
// 32-bit byte offset, which saves the 64-bit vector address arithmetic.
__device__ __forceinline__ void lds_dma_load16_sbase(const void* base, uint32_t offset, uint32_t lds_base) {
  asm volatile(
      "s_mov_b32 m0, %1\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %2"
      :
      : "v"(offset), "s"(__builtin_amdgcn_readfirstlane(lds_base)), "s"(base)
      : "memory", "m0");
}

// s_waitcnt with vmcnt <= N (N < 64), other counters unconstrained (gfx9 encoding).
template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 0xF) | ((N >> 4) << 14) | (0x7 << 4) | (0xF << 8));
}

// Byte address of an LDS location, for lds_dma_load16.
__device__ __forceinline__ uint32_t lds_address(const void* p) {
  return static_cast<uint32_t>(
      reinterpret_cast<uintptr_t>((const __attribute__((address_space(3))) void*)p));
}

// Compiler-level fence: no memory access moves across it.
__device__ __forceinline__ void compiler_fence() { asm volatile("" ::: "memory"); }

// ---------------------------------------------------------------- MFMA ----
//
// gfx950 matrix cores, wave64. Operand layouts used throughout (lane l,
// col = l % 16, grp = l / 16):
//   16x16x32: A[m][k] lane holds m = col, k = 8*grp .. 8*grp+7
//             B[k][n] lane holds n = col, k = 8*grp .. 8*grp+7
//   16x16x16: A lane holds m = col, k = 4*grp .. 4*grp+3 (B likewise)
//   C/D (16x16 fp32): lane holds n = col, m = 4*grp .. 4*grp+3
// The kernels only rely on these layouts; they are checked on the device by
// the MFMA layout test.

template <typename T> struct Mfma;

template <> struct Mfma<bf16_t> {
  __device__ static float4_t k32(short8_t a, short8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(
        __builtin_bit_cast(__attribute__((ext_vector_type(8))) __bf16, a),
        __builtin_bit_cast(__attribute__((ext_vector_type(8))) __bf16, b), c,
        0, 0, 0);
  }
  __device__ static float4_t k16(short4_t a, short4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(a, b, c, 0, 0, 0);
  }
};

template <> struct Mfma<f16_t> {
  __device__ static float4_t k32(short8_t a, short8_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_f16(
        __builtin_bit_cast(half8_t, a), __builtin_bit_cast(half8_t, b), c, 0,
        0, 0);
  }
  __device__ static float4_t k16(short4_t a, short4_t b, float4_t c) {
    return __builtin_amdgcn_mfma_f32_16x16x16f16(
        __builtin_bit_cast(half4_t, a), __builtin_bit_cast(half4_t, b), c, 0,
        0, 0);
  }
};

// Byte permute (v_perm_b32): result byte i = byte sel_i of {hi:lo}.
__device__ __forceinline__ uint32_t perm_b32(uint32_t hi, uint32_t lo, uint32_t sel) {
  return __builtin_amdgcn_perm(hi, lo, sel);
}
// Low 16 bits of a and b -> (a.lo | b.lo << 16).
__device__ __forceinline__ uint32_t pack_lo16(uint32_t a, uint32_t b) {
  return perm_b32(b, a, 0x05040100u);
}
// High 16 bits of a and b -> (a.hi | b.hi << 16).
__device__ __forceinline__ uint32_t pack_hi16(uint32_t a, uint32_t b) {
  return perm_b32(b, a, 0x07060302u);
}

}  // namespace mvllm
