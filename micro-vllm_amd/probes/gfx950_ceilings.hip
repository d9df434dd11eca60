// Microbenchmarks of the gfx950 limits that the attention kernels are
// designed against. Every number that bounds a kernel (MFMA rate, how MFMA
// and vector work share a SIMD, the issue cost of vector instructions and of
// HBM loads, LDS read rates, the achievable streaming-read rate) is measured
// here.
//
//   python micro-vllm_amd/build.py   (builds micro-vllm_amd/probes/gfx950_ceilings)
//   micro-vllm_amd/probes/gfx950_ceilings
//
// Per-wave cycle counts come from s_memtime (the shader clock counter); the
// whole-chip rates from HIP events. Every probe indexes its buffers with
// masks or bounds that keep each access inside them, and every loop runs a
// fixed number of iterations.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cstdint>
#include <cstdio>
#include <cstdlib>
#include <vector>

#define CHECK(x)                                                                     \
  do {                                                                               \
    hipError_t e_ = (x);                                                             \
    if (e_ != hipSuccess) {                                                          \
      std::printf("HIP error %s at line %d\n", hipGetErrorString(e_), __LINE__);     \
      std::exit(1);                                                                  \
    }                                                                                \
  } while (0)

namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float float16v __attribute__((ext_vector_type(16)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) void lds_void;

constexpr double kMfmaFlops = 32.0 * 32 * 16 * 2;  // one v_mfma_f32_32x32x16_bf16

__device__ __forceinline__ void operands(bf16x8& a, bf16x8& b) {
  const int lane = threadIdx.x & 63;
  for (int i = 0; i < 8; ++i) {
    a[i] = static_cast<__bf16>(0.001f * (lane + i));
    b[i] = static_cast<__bf16>(0.002f * i);
  }
}

// Keeps a value alive without writing it (the condition never holds).
__device__ __forceinline__ void sink(float v, float* out) {
  if (v == 1234567.f) out[blockIdx.x * blockDim.x + threadIdx.x] = v;
}

double median(std::vector<double> v) {
  std::sort(v.begin(), v.end());
  return v.empty() ? 0.0 : v[v.size() / 2];
}

struct Timer {
  hipEvent_t a, b;
  Timer() {
    CHECK(hipEventCreate(&a));
    CHECK(hipEventCreate(&b));
  }
  ~Timer() {
    (void)hipEventDestroy(a);
    (void)hipEventDestroy(b);
  }
  // Milliseconds per launch, averaged over `reps` launches after a warm-up.
  template <typename F>
  float ms(F launch, int reps = 1) {
    launch();
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipEventRecord(a, 0));
    for (int i = 0; i < reps; ++i) launch();
    CHECK(hipEventRecord(b, 0));
    CHECK(hipEventSynchronize(b));
    float t = 0.f;
    CHECK(hipEventElapsedTime(&t, a, b));
    return t / reps;
  }
};

// s_waitcnt immediate that waits for vmcnt <= v and leaves the other counters
// at their maxima (vmcnt bits 3:0 and 15:14, expcnt 6:4, lgkmcnt 11:8).
constexpr int vmcnt_only(int v) { return (v & 15) | ((v >> 4) << 14) | (7 << 4) | (15 << 8); }

// LDS reserved so that one 256-thread workgroup runs per CU (one wave per
// SIMD), or two with `per_cu` = 2.
template <typename K>
size_t reserve_cu(K kernel, int per_cu) {
  const size_t lds = per_cu == 1 ? 96 * 1024 : 64 * 1024;
  CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)));
  return lds;
}

// ---------------------------------------------------------------- MFMA rate
// Each wave runs `iters` x 32 MFMAs over C independent accumulators.
template <int C>
__global__ __launch_bounds__(256) void mfma_chains(float* out, unsigned long long* ticks, int iters) {
  bf16x8 a, b;
  operands(a, b);
  float16v c[C];
  for (int j = 0; j < C; ++j) c[j] = float16v{};
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int k = 0; k < 32 / C; ++k)
#pragma unroll
      for (int j = 0; j < C; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
  for (int j = 0; j < C; ++j) s += c[j][0] + c[j][15];
  sink(s, out);
  if ((threadIdx.x & 63) == 0) ticks[blockIdx.x * 4 + (threadIdx.x >> 6)] = t1 - t0;
}

template <int C>
void mfma_rate(float* out, unsigned long long* ticks, int cus, int per_simd, double* ticks_per_us) {
  const int blocks = cus * per_simd;  // 4 waves per workgroup: one per SIMD
  const int iters = 2000;
  const size_t lds = reserve_cu(mfma_chains<C>, per_simd);
  Timer t;
  const float ms =
      t.ms([&] { hipLaunchKernelGGL(mfma_chains<C>, dim3(blocks), dim3(256), lds, 0, out, ticks, iters); });
  std::vector<unsigned long long> h(blocks * 4);
  CHECK(hipMemcpy(h.data(), ticks, h.size() * 8, hipMemcpyDeviceToHost));
  std::vector<double> d(h.begin(), h.end());
  const double med = median(d);
  const double flops = double(blocks) * 4 * iters * 32 * kMfmaFlops;
  if (ticks_per_us) *ticks_per_us = med / (ms * 1e3);
  std::printf("mfma 32x32x16 bf16, %d chain(s) per wave, %d wave(s) per SIMD: %7.1f TFLOP/s, %6.2f ticks per MFMA per wave\n",
              C, per_simd, flops / (ms * 1e9), med / (iters * 32.0));
}

// ------------------------------------------------ MFMA and VALU on one SIMD
// 512-thread workgroups, one per CU: waves w and w + 4 share a SIMD. Waves
// 0-3 run MFMAs (four chains), waves 4-7 run FMAs or exponentials (eight
// chains). mode bit 0: MFMA waves run; bit 1: VALU waves run; bit 2: the
// VALU waves run v_exp_f32 instead of v_fma_f32.
__global__ __launch_bounds__(512) void cross_wave(float* out, unsigned long long* ticks, unsigned* simd, int mode,
                                                  int iters) {
  const int wave = threadIdx.x >> 6;
  const bool mfma_wave = wave < 4;
  const bool active = mfma_wave ? (mode & 1) : (mode & 2);
  // HW_ID bits 5:4 hold the SIMD of the wave.
  const unsigned id = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
  if (active && mfma_wave) {
    bf16x8 a, b;
    operands(a, b);
    float16v c[4];
    for (int j = 0; j < 4; ++j) c[j] = float16v{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
    }
    for (int j = 0; j < 4; ++j) s += c[j][0];
  } else if (active) {
    float x[8];
    for (int j = 0; j < 8; ++j) x[j] = 0.001f * ((threadIdx.x & 63) + j);
    if (mode & 4) {
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) asm volatile("v_exp_f32_e64 %0, -%0" : "+v"(x[j]));
      }
    } else {
      for (int it = 0; it < iters; ++it) {
#pragma unroll
        for (int j = 0; j < 8; ++j) x[j] = __builtin_fmaf(x[j], 0.999f, 0.0001f);
      }
    }
    for (int j = 0; j < 8; ++j) s += x[j];
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  sink(s, out);
  if ((threadIdx.x & 63) == 0) {
    ticks[blockIdx.x * 8 + wave] = t1 - t0;
    simd[blockIdx.x * 8 + wave] = (id >> 4) & 3;
  }
}

void cross_wave_rates(float* out, unsigned long long* ticks, unsigned* simd, int cus) {
  const int iters = 4000;
  const size_t lds = 96 * 1024;  // one workgroup per CU
  CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(cross_wave), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)));
  struct Mode {
    int mode;
    const char* name;
  } modes[] = {{1, "mfma alone"}, {2, "fma alone"}, {3, "mfma + fma"}, {6, "exp alone"}, {7, "mfma + exp"}};
  std::vector<unsigned long long> h(cus * 8);
  std::vector<unsigned> hs(cus * 8);
  bool paired = true;
  for (const Mode& m : modes) {
    hipLaunchKernelGGL(cross_wave, dim3(cus), dim3(512), lds, 0, out, ticks, simd, m.mode, iters);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(h.data(), ticks, h.size() * 8, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(hs.data(), simd, hs.size() * 4, hipMemcpyDeviceToHost));
    std::vector<double> mf, va;
    for (int b = 0; b < cus; ++b)
      for (int w = 0; w < 4; ++w) {
        mf.push_back(double(h[b * 8 + w]));
        va.push_back(double(h[b * 8 + 4 + w]));
        paired = paired && hs[b * 8 + w] == hs[b * 8 + 4 + w];
      }
    // Per iteration: 4 MFMAs (MFMA waves), 8 VALU instructions (VALU waves).
    std::printf("one SIMD, %-11s: MFMA wave %6.2f ticks per MFMA, VALU wave %6.2f ticks per instruction\n", m.name,
                (m.mode & 1) ? median(mf) / (iters * 4.0) : 0.0, (m.mode & 2) ? median(va) / (iters * 8.0) : 0.0);
  }
  std::printf("waves w and w + 4 on the same SIMD in every workgroup: %s\n", paired ? "yes" : "no");
}

// ------------------------------------- MFMA beside two vector ALU waves
// Twelve waves per workgroup, one workgroup per CU: waves w, w + 4 and w + 8
// share a SIMD. Waves 0-3 run back-to-back MFMAs (4 chains), waves 4-11 run
// 16 independent chains of FMAs (or exponentials), each wave the same count.
__global__ __launch_bounds__(768) void cross_wave3(float* out, unsigned long long* ticks, unsigned* simd, int mode,
                                                  int iters) {
  const int wave = threadIdx.x >> 6;
  const int grp = wave >> 2;  // 0 MFMA, 1 and 2 vector ALU
  const bool active = grp == 0 ? (mode & 1) : (mode & 2);
  const unsigned id = __builtin_amdgcn_s_getreg((31 << 11) | (0 << 6) | 4);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
  if (active && grp == 0) {
    bf16x8 a, b;
    operands(a, b);
    float16v c[4];
    for (int j = 0; j < 4; ++j) c[j] = float16v{};
    for (int it = 0; it < iters; ++it) {
#pragma unroll
      for (int j = 0; j < 4; ++j) c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
    }
    for (int j = 0; j < 4; ++j) s += c[j][0];
  } else if (active) {
    float x[16];
    for (int j = 0; j < 16; ++j) x[j] = 0.001f * ((threadIdx.x & 63) + j);
    if (mode & 4) {
      for (int it = 0; it < iters / 2; ++it) {
#pragma unroll
        for (int j = 0; j < 16; ++j) asm volatile("v_exp_f32_e64 %0, -%0" : "+v"(x[j]));
      }
    } else {
      for (int it = 0; it < iters / 2; ++it) {
#pragma unroll
        for (int j = 0; j < 16; ++j) x[j] = __builtin_fmaf(x[j], 0.999f, 0.0001f);
      }
    }
    for (int j = 0; j < 16; ++j) s += x[j];
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  sink(s, out);
  if ((threadIdx.x & 63) == 0) {
    ticks[blockIdx.x * 12 + wave] = t1 - t0;
    simd[blockIdx.x * 12 + wave] = (id >> 4) & 3;
  }
}

void cross_wave3_rates(float* out, unsigned long long* ticks, unsigned* simd, int cus) {
  const int iters = 4000;
  const size_t lds = 96 * 1024;  // one workgroup per CU
  CHECK(hipFuncSetAttribute(reinterpret_cast<const void*>(cross_wave3), hipFuncAttributeMaxDynamicSharedMemorySize,
                            static_cast<int>(lds)));
  struct Mode {
    int mode;
    const char* name;
  } modes[] = {{2, "fma"}, {3, "fma"}, {6, "exp"}, {7, "exp"}};
  std::vector<unsigned long long> h(cus * 12);
  std::vector<unsigned> hs(cus * 12);
  bool paired = true;
  for (const Mode& m : modes) {
    hipLaunchKernelGGL(cross_wave3, dim3(cus), dim3(768), lds, 0, out, ticks, simd, m.mode, iters);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
    CHECK(hipMemcpy(h.data(), ticks, h.size() * 8, hipMemcpyDeviceToHost));
    CHECK(hipMemcpy(hs.data(), simd, hs.size() * 4, hipMemcpyDeviceToHost));
    std::vector<double> mf, span;
    for (int b = 0; b < cus; ++b)
      for (int w = 0; w < 4; ++w) {
        mf.push_back(double(h[b * 12 + w]));
        span.push_back(double(std::max(h[b * 12 + 4 + w], h[b * 12 + 8 + w])));
        paired = paired && hs[b * 12 + w] == hs[b * 12 + 4 + w] && hs[b * 12 + w] == hs[b * 12 + 8 + w];
      }
    // Each vector wave issues 8 * iters instructions; both finish within the
    // MFMA waves' run, so the later one's span bounds the pair's rate.
    std::printf("one SIMD, two %s waves%-7s: %5.2f ticks per vector instruction between them%s", m.name,
                (m.mode & 1) ? " + mfma" : "", median(span) / (2.0 * 8.0 * iters), (m.mode & 1) ? "" : "\n");
    if (m.mode & 1) std::printf(", MFMA wave %6.2f ticks per MFMA\n", median(mf) / (iters * 4.0));
  }
  std::printf("waves w, w + 4 and w + 8 on the same SIMD in every workgroup: %s\n", paired ? "yes" : "no");
}

// ------------------------------------------ MFMA and VALU in the same wave
// Each iteration: one MFMA (four chains in rotation) then K independent FMAs.
template <int K>
__global__ __launch_bounds__(256) void in_wave(float* out, unsigned long long* ticks, int iters) {
  bf16x8 a, b;
  operands(a, b);
  float16v c[4];
  for (int j = 0; j < 4; ++j) c[j] = float16v{};
  float x[16];
  for (int j = 0; j < 16; ++j) x[j] = 0.001f * ((threadIdx.x & 63) + j);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      c[j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c[j], 0, 0, 0);
#pragma unroll
      for (int k = 0; k < K; ++k) x[k] = __builtin_fmaf(x[k], 0.999f, 0.0001f);
      __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
      if constexpr (K > 0) __builtin_amdgcn_sched_group_barrier(0x002, K, 0);
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
  for (int j = 0; j < 4; ++j) s += c[j][0];
  for (int k = 0; k < 16; ++k) s += x[k];
  sink(s, out);
  if ((threadIdx.x & 63) == 0) ticks[blockIdx.x * 4 + (threadIdx.x >> 6)] = t1 - t0;
}

template <int K>
void in_wave_rate(float* out, unsigned long long* ticks, int cus) {
  const int iters = 2000;
  const size_t lds = reserve_cu(in_wave<K>, 1);
  hipLaunchKernelGGL(in_wave<K>, dim3(cus), dim3(256), lds, 0, out, ticks, iters);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  std::vector<unsigned long long> h(cus * 4);
  CHECK(hipMemcpy(h.data(), ticks, h.size() * 8, hipMemcpyDeviceToHost));
  std::vector<double> d(h.begin(), h.end());
  std::printf("one wave per SIMD, 1 MFMA + %2d independent FMAs: %6.2f ticks per MFMA\n", K,
              median(d) / (iters * 4.0));
}

// ------------------------------------------------------ VALU issue costs
// CH independent chains of one instruction per wave.
template <int OP, int CH>
__global__ __launch_bounds__(256) void valu_cost(float* out, unsigned long long* ticks, int iters) {
  float x[CH];
  uint32_t u[CH];
  for (int j = 0; j < CH; ++j) {
    x[j] = 0.001f * ((threadIdx.x & 63) + j);
    u[j] = 0x3f803f80u + j;
  }
  const float y = 0.5f, z = 0.25f;
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < CH; ++j) {
      if constexpr (OP == 0) asm volatile("v_exp_f32_e64 %0, -%0" : "+v"(x[j]));
      if constexpr (OP == 1) asm volatile("v_fma_f32 %0, %0, %1, %2" : "+v"(x[j]) : "v"(y), "v"(z));
      if constexpr (OP == 2) asm volatile("v_max3_f32 %0, %0, %1, %2" : "+v"(x[j]) : "v"(y), "v"(z));
      if constexpr (OP == 3) asm volatile("v_cvt_pk_bf16_f32 %0, %1, %2" : "=v"(u[j]) : "v"(x[j]), "v"(y));
      if constexpr (OP == 4) asm volatile("v_dot2c_f32_bf16 %0, %1, %2" : "+v"(x[j]) : "v"(u[j]), "v"(u[j]));
    }
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  float s = 0.f;
  for (int j = 0; j < CH; ++j) s += x[j] + __uint_as_float(u[j]);
  sink(s, out);
  if ((threadIdx.x & 63) == 0) ticks[blockIdx.x * 4 + (threadIdx.x >> 6)] = t1 - t0;
}

template <int OP, int CH = 8>
void valu_rate(const char* name, float* out, unsigned long long* ticks, int cus, int per_simd = 1) {
  const int iters = 320000 / CH;
  const size_t lds = reserve_cu(valu_cost<OP, CH>, per_simd);
  Timer t;
  const float ms = t.ms(
      [&] { hipLaunchKernelGGL((valu_cost<OP, CH>), dim3(cus * per_simd), dim3(256), lds, 0, out, ticks, iters); });
  std::vector<unsigned long long> h(cus * per_simd * 4);
  CHECK(hipMemcpy(h.data(), ticks, h.size() * 8, hipMemcpyDeviceToHost));
  std::vector<double> d(h.begin(), h.end());
  std::printf("%d wave(s) per SIMD, %2d chains, %-18s: %5.2f ticks per instruction per wave (%.0f ticks per us)\n",
              per_simd, CH, name, median(d) / (double(iters) * CH), median(d) / (ms * 1e3));
}

// ------------------------------------------------------ load issue costs
// Each wave stamps, issues kLoads loads of 1 KiB (16 bytes per lane), stamps,
// drains and stamps again. KIND 0: global_load_lds_dwordx4 (HBM -> LDS);
// 1: buffer_load_dwordx4 ... lds; 2: global_load_dwordx4 into VGPRs;
// 3: MFMA chain only; 4: one MFMA then one global_load_lds per step.
constexpr int kLoads = 8;
constexpr size_t kLoadBuf = size_t(256) << 20;

template <int KIND>
__global__ __launch_bounds__(256) void load_issue(const char* g, unsigned long long* ticks, float* out) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  const unsigned gw = blockIdx.x * (blockDim.x >> 6) + wv;
  char* const dst = lds + wv * 1024;  // each wave's own 1 KiB of LDS
  const __amdgpu_buffer_rsrc_t rsrc =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<char*>(g), 0, static_cast<int>(kLoadBuf), 0x00020000);
  bf16x8 a, b;
  operands(a, b);
  float16v acc = {};
  u32x4 got[kLoads];  // VGPR loads land here and are consumed after the issue stamp
  __syncthreads();
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int i = 0; i < kLoads; ++i) {
    // Masked into the buffer: the highest byte read is kLoadBuf - 1.
    const size_t off = ((size_t(gw) * kLoads + i) * 1024 + lane * 16) & (kLoadBuf - 1);
    if constexpr (KIND == 0) {
      __builtin_amdgcn_global_load_lds(g + off, (lds_void*)(dst), 16, 0, 0);
    } else if constexpr (KIND == 1) {
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rsrc, (lds_void*)(dst), 16, static_cast<uint32_t>(off),
                                               0, 0, 0);
    } else if constexpr (KIND == 2) {
      got[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(g + off));
    } else if constexpr (KIND == 3) {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
    } else {
      acc = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, acc, 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);
      __builtin_amdgcn_global_load_lds(g + off, (lds_void*)(dst), 16, 0, 0);
    }
    __builtin_amdgcn_sched_barrier(0);
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_waitcnt(0);
  __builtin_amdgcn_sched_barrier(0);
  const unsigned long long t2 = __builtin_amdgcn_s_memtime();
  __syncthreads();
  u32x4 keep = {0, 0, 0, 0};
  if constexpr (KIND == 2)
    for (int i = 0; i < kLoads; ++i) keep ^= got[i];
  float s = acc[0] + acc[15] + __uint_as_float(keep.x ^ keep.y ^ keep.z ^ keep.w);
  s += reinterpret_cast<const float*>(dst)[lane];
  sink(s, out);
  if (lane == 0) {
    ticks[2 * gw] = t1 - t0;
    ticks[2 * gw + 1] = t2 - t0;
  }
}

template <int KIND>
void load_rate(const char* name, const char* g, int blocks, int threads, unsigned long long* ticks, float* out) {
  const int waves = blocks * threads / 64;
  for (int rep = 0; rep < 3; ++rep) {
    hipLaunchKernelGGL(load_issue<KIND>, dim3(blocks), dim3(threads), 4096, 0, g, ticks, out);
    CHECK(hipGetLastError());
    CHECK(hipDeviceSynchronize());
  }
  std::vector<unsigned long long> h(2 * waves);
  CHECK(hipMemcpy(h.data(), ticks, h.size() * 8, hipMemcpyDeviceToHost));
  std::vector<double> issue, drain;
  for (int w = 0; w < waves; ++w) {
    issue.push_back(double(h[2 * w]));
    drain.push_back(double(h[2 * w + 1]));
  }
  std::printf("%-28s %5d x %3d threads: issue %6.1f ticks per step (median), drained after %7.1f\n", name, blocks,
              threads, median(issue) / kLoads, median(drain));
}

// ------------------------------------------------------ LDS read rate
// One workgroup of 256 threads per CU reads a 16 KiB tile of 64 rows of 256
// bytes laid out as the prefill kernel's K/V tiles are: 16-byte chunk c of
// row r sits at chunk c ^ s(r), s(r) = r' ^ ((r' & 2) << 2), r' = r % 16.
// KIND 0 reads it with ds_read_b128 as the score MFMAs' K operands (lane l:
// row l % 32, chunks 2 st + l / 32, st = 0..7); KIND 1 with the transposing
// ds_read_b64_tr_b16 as the P.V MFMAs' V operands (lane (g, j) = (l / 16,
// l % 16): row 8 u + 4 (g / 2) + j / 4, dims 32 c + 16 (g % 2) + 4 (j % 4)).
// Eight reads are in flight per wave.
__host__ __device__ constexpr int tile_chunk_off(int row, int chunk) {
  return row * 256 + ((chunk ^ ((row & 15) ^ (((row & 15) & 2) << 2))) << 4);
}

template <int KIND>
__global__ __launch_bounds__(256) void lds_read(float* out, unsigned long long* ticks, int iters) {
  extern __shared__ __attribute__((aligned(16))) char lds[];
  constexpr uint32_t kBytes = 64 * 1024;
  for (uint32_t i = threadIdx.x; i < kBytes / 4; i += blockDim.x) reinterpret_cast<uint32_t*>(lds)[i] = i;
  __syncthreads();
  const int lane = threadIdx.x & 63;
  const int wv = threadIdx.x >> 6;
  // Eight LDS byte addresses per lane, one per read in flight, inside the
  // wave's own 16 KiB tile (four tiles: 64 KiB).
  const uint32_t base = static_cast<uint32_t>(reinterpret_cast<uintptr_t>((lds_void*)lds)) + wv * 16384;
  uint32_t addr[8];
  for (int x = 0; x < 8; ++x) {
    if constexpr (KIND == 0) {
      addr[x] = base + tile_chunk_off(lane & 31, 2 * x + (lane >> 5));
    } else {
      const int g = lane >> 4, jj = lane & 15, u = x >> 2, c = x & 3;
      const int row = 8 * u + 4 * (g >> 1) + (jj >> 2);
      const int dim = 32 * c + 16 * (g & 1) + 4 * (jj & 3);
      addr[x] = base + tile_chunk_off(row, dim >> 3) + 2 * (dim & 7);
    }
  }
  u32x4 r[8];
  const unsigned long long t0 = __builtin_amdgcn_s_memtime();
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j) {
      if constexpr (KIND == 0)
        asm volatile("ds_read_b128 %0, %1" : "=v"(r[j]) : "v"(addr[j]));
      else
        asm volatile("ds_read_b64_tr_b16 %0, %1" : "=v"(reinterpret_cast<uint64_t&>(r[j])) : "v"(addr[j]));
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
  }
  const unsigned long long t1 = __builtin_amdgcn_s_memtime();
  u32x4 acc = {0, 0, 0, 0};
  for (int j = 0; j < 8; ++j) acc ^= r[j];
  sink(__uint_as_float(acc.x ^ acc.y ^ acc.z ^ acc.w), out);
  if (lane == 0) ticks[blockIdx.x * 4 + wv] = t1 - t0;
}

template <int KIND>
void lds_rate(const char* name, float* out, unsigned long long* ticks, int cus) {
  const int iters = 4000;
  const size_t lds = reserve_cu(lds_read<KIND>, 1);
  hipLaunchKernelGGL(lds_read<KIND>, dim3(cus), dim3(256), lds, 0, out, ticks, iters);
  CHECK(hipGetLastError());
  CHECK(hipDeviceSynchronize());
  std::vector<unsigned long long> h(cus * 4);
  CHECK(hipMemcpy(h.data(), ticks, h.size() * 8, hipMemcpyDeviceToHost));
  std::vector<double> d(h.begin(), h.end());
  const double bytes_per_wave = double(iters) * 8 * 64 * (KIND == 0 ? 16 : 8);
  std::printf("%-34s: %6.1f bytes per cycle per CU (four waves)\n", name, 4 * bytes_per_wave / median(d));
}

// --------------------------------------------------- HBM streaming reads
// Plain 16-byte non-temporal loads, UNROLL in flight per thread.
template <int UNROLL>
__global__ __launch_bounds__(256) void stream_vgpr(const u32x4* __restrict__ p, size_t n, u32x4* out) {
  u32x4 acc = {0, 0, 0, 0};
  const size_t stride = size_t(gridDim.x) * 256 * UNROLL;
  for (size_t i = size_t(blockIdx.x) * 256 * UNROLL + threadIdx.x; i < n; i += stride) {
#pragma unroll
    for (int u = 0; u < UNROLL; ++u) {
      const size_t j = i + size_t(u) * 256;
      if (j < n) acc ^= __builtin_nontemporal_load(p + j);
    }
  }
  if (acc.x == 0x12345678u) out[threadIdx.x] = acc;
}

// HBM -> LDS streaming: each wave moves 1 KiB chunks into its own ring of
// DEPTH slots with global_load_lds_dwordx4, DEPTH - 1 loads in flight.
template <int DEPTH>
__global__ __launch_bounds__(256) void stream_lds(const char* __restrict__ p, size_t bytes, u32x4* out) {
  __shared__ __attribute__((aligned(16))) char ring[4][DEPTH][1024];
  const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int lane = threadIdx.x & 63;
  const size_t chunks = bytes / 1024;
  const size_t stride = size_t(gridDim.x) * 4;
  int slot = 0;
  for (size_t c = size_t(blockIdx.x) * 4 + wave; c < chunks; c += stride) {
    __builtin_amdgcn_global_load_lds(p + c * 1024 + lane * 16, (lds_void*)(&ring[wave][slot][0]), 16,
                                     0, 0);
    slot = slot + 1 == DEPTH ? 0 : slot + 1;
    __builtin_amdgcn_s_waitcnt(vmcnt_only(DEPTH - 1));
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  if (ring[wave][0][lane] == 0x7f && lane == 999) out[0] = u32x4{1, 1, 1, 1};
}

}  // namespace

int main() {
  int cus = 0;
  CHECK(hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, 0));
  int clk_khz = 0;
  CHECK(hipDeviceGetAttribute(&clk_khz, hipDeviceAttributeClockRate, 0));
  std::printf("device: %d CUs, reported peak clock %.0f MHz\n", cus, clk_khz / 1e3);

  const int max_waves = 1024 * 8;
  float* out;
  unsigned long long* ticks;
  unsigned* simd;
  CHECK(hipMalloc(&out, size_t(max_waves) * 64 * sizeof(float)));
  CHECK(hipMalloc(&ticks, size_t(max_waves) * 2 * sizeof(unsigned long long)));
  CHECK(hipMalloc(&simd, size_t(max_waves) * sizeof(unsigned)));

  std::printf("\n== MFMA rate (all CUs)\n");
  double tpu = 0.0;
  mfma_rate<1>(out, ticks, cus, 1, nullptr);
  mfma_rate<2>(out, ticks, cus, 1, nullptr);
  mfma_rate<4>(out, ticks, cus, 1, &tpu);
  mfma_rate<8>(out, ticks, cus, 1, nullptr);
  mfma_rate<4>(out, ticks, cus, 2, nullptr);
  std::printf("s_memtime ticks per microsecond under MFMA load: %.0f\n", tpu);

  std::printf("\n== MFMA and vector ALU work of two waves on one SIMD\n");
  cross_wave_rates(out, ticks, simd, cus);

  std::printf("\n== MFMA beside two vector ALU waves on one SIMD\n");
  cross_wave3_rates(out, ticks, simd, cus);

  std::printf("\n== MFMA and independent vector ALU work in one wave\n");
  in_wave_rate<0>(out, ticks, cus);
  in_wave_rate<4>(out, ticks, cus);
  in_wave_rate<8>(out, ticks, cus);
  in_wave_rate<16>(out, ticks, cus);

  std::printf("\n== vector ALU issue cost\n");
  valu_rate<0>("v_exp_f32", out, ticks, cus);
  valu_rate<1>("v_fma_f32", out, ticks, cus);
  valu_rate<2>("v_max3_f32", out, ticks, cus);
  valu_rate<3>("v_cvt_pk_bf16_f32", out, ticks, cus);
  valu_rate<4>("v_dot2c_f32_bf16", out, ticks, cus);
  valu_rate<0, 16>("v_exp_f32", out, ticks, cus);
  valu_rate<1, 16>("v_fma_f32", out, ticks, cus);
  valu_rate<0>("v_exp_f32", out, ticks, cus, 2);
  valu_rate<1>("v_fma_f32", out, ticks, cus, 2);
  valu_rate<0, 16>("v_exp_f32", out, ticks, cus, 2);
  valu_rate<1, 16>("v_fma_f32", out, ticks, cus, 2);

  std::printf("\n== LDS reads\n");
  lds_rate<0>("ds_read_b128, K operand pattern", out, ticks, cus);
  lds_rate<1>("ds_read_b64_tr_b16, V operand pattern", out, ticks, cus);

  std::printf("\n== load issue cost (8 steps of 1 KiB per wave)\n");
  char* g;
  CHECK(hipMalloc(&g, kLoadBuf));
  CHECK(hipMemset(g, 1, kLoadBuf));
  const int shapes[3][2] = {{1, 64}, {1, 256}, {4 * cus, 256}};
  for (const auto& s : shapes) {
    load_rate<0>("global_load_lds_dwordx4", g, s[0], s[1], ticks, out);
    load_rate<1>("buffer_load_dwordx4 lds", g, s[0], s[1], ticks, out);
    load_rate<2>("global_load_dwordx4 (VGPR)", g, s[0], s[1], ticks, out);
    load_rate<3>("MFMA chain only", g, s[0], s[1], ticks, out);
    load_rate<4>("MFMA + global_load_lds", g, s[0], s[1], ticks, out);
  }
  CHECK(hipFree(g));

  std::printf("\n== HBM streaming read, 4 GiB\n");
  const size_t bytes = size_t(4) << 30;
  char* p;
  u32x4* o;
  CHECK(hipMalloc(&p, bytes));
  CHECK(hipMalloc(&o, 4096));
  CHECK(hipMemset(p, 1, bytes));
  Timer t;
  for (int grid : {8 * cus, 16 * cus, 32 * cus, 64 * cus}) {
    const float a = t.ms([&] {
      hipLaunchKernelGGL(stream_vgpr<8>, dim3(grid), dim3(256), 0, 0, reinterpret_cast<const u32x4*>(p), bytes / 16, o);
    }, 5);
    const float b = t.ms([&] { hipLaunchKernelGGL(stream_lds<16>, dim3(grid), dim3(256), 0, 0, p, bytes, o); }, 5);
    const float c = t.ms([&] { hipLaunchKernelGGL(stream_lds<8>, dim3(grid), dim3(256), 0, 0, p, bytes, o); }, 5);
    std::printf("grid %6d: 16-byte nt loads %6.0f GB/s, global_load_lds ring of 16 KiB per wave %6.0f GB/s, of 8 KiB %6.0f GB/s\n",
                grid, bytes / (a * 1e6), bytes / (b * 1e6), bytes / (c * 1e6));
  }
  CHECK(hipFree(p));
  CHECK(hipFree(o));
  CHECK(hipFree(out));
  CHECK(hipFree(ticks));
  CHECK(hipFree(simd));
  std::printf("\ndone\n");
  return 0;
}
