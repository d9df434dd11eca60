// MFMA prefill / chunked-prefill kernel (requests with more than one query),
// head_dim 128, bf16/fp16, block sizes that are multiples of 16.
//
// Work item: (request, block of T query tokens, KV head), one workgroup of
// four waves. The workgroup's 128 rows are (query head of the KV head's
// group, token) pairs: row f -> head f / T, token f % T with T = 128 / G, so
// all G query heads that share a KV head (GQA) read each K/V tile once.
// Each wave owns 32 rows.
//
// Keys are processed in tiles of 64 (four 16-token pages). Every wave stages
// one page of K and of V through registers into a double-buffered LDS tile
// (one barrier per tile; the next page is in flight while the current tile
// is computed). Per tile a wave computes
//   S^T = K . Q^T      two v_mfma_f32_32x32x16 blocks (32 keys x 32 rows)
// so each lane holds the scores of ONE row (lane % 32) for 16 keys per
// block: the row max and sum are in-lane, plus one exchange with lane ^ 32.
// P^T, as produced by the accumulator layout, is already the B operand of
//   O^T += V^T . P^T   four 32x32x16 blocks per 16 keys (dims permuted)
// and V^T comes from 8-byte LDS reads repacked with v_perm. The online
// softmax (FlashAttention-2, Dao 2023) runs in the exp2 domain and rescales
// the accumulators only when a row's maximum grows by more than 2^8
// (lazy rescaling as in FlashAttention-3, Shah et al. 2024): the final
// normalisation divides by a sum taken with the same offsets, so the result
// is unchanged.
//
// Masking is applied only on tiles that cross a row's visible range or hold
// an unmapped page; there, keys outside every row's range of the wave are
// also zeroed in V so that stale or non-finite cache rows cannot leak
// through 0 * NaN.
#include <climits>
#include <cmath>

#include <hip/hip_ext.h>

#include "attention.h"

namespace mvllm {
namespace {

constexpr int kDim = 128;
constexpr int kTileKeys = 64;
constexpr int kWaves = 4;
constexpr int kRows = kWaves * 32;                   // rows per workgroup
constexpr int kTileBytes = kTileKeys * kDim * 2;     // one K (or V) tile: 16 KiB
constexpr int kStageBytes = 2 * kTileBytes;          // K + V
constexpr int kTablePages = 2048;                    // block ids held in LDS at a time
constexpr int kChunkTiles = kTablePages / 4;
constexpr size_t kLdsBytes = 2 * kStageBytes + kTablePages * 4 + 16 * 4;

typedef float float16v __attribute__((ext_vector_type(16)));
typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef _Float16 f16x2_t __attribute__((ext_vector_type(2)));
typedef float float2v __attribute__((ext_vector_type(2)));

template <typename T> struct Mma32;

template <> struct Mma32<bf16_t> {
  __device__ static float16v mma(short8_t a, short8_t b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8_t, a),
                                                   __builtin_bit_cast(bf16x8_t, b), c, 0, 0, 0);
  }
  // Two fp32 values -> packed 16-bit pair (round to nearest even).
  __device__ static uint32_t pack2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{x, y}, bf16x2_t));
  }
  __device__ static float2v unpack2(uint32_t w) {
    return float2v{__uint_as_float(w << 16), __uint_as_float(w & 0xFFFF0000u)};
  }
};

template <> struct Mma32<f16_t> {
  __device__ static float16v mma(short8_t a, short8_t b, float16v c) {
    return __builtin_amdgcn_mfma_f32_32x32x16_f16(__builtin_bit_cast(half8_t, a),
                                                  __builtin_bit_cast(half8_t, b), c, 0, 0, 0);
  }
  __device__ static uint32_t pack2(float x, float y) {
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(float2v{x, y}, f16x2_t));
  }
  __device__ static float2v unpack2(uint32_t w) {
    return __builtin_convertvector(__builtin_bit_cast(f16x2_t, w), float2v);
  }
};

__device__ __forceinline__ int32_t wave_min_i(int32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = min(v, __shfl_xor(v, m, 64));
  return v;
}

__device__ __forceinline__ int32_t wave_max_i(int32_t v) {
#pragma unroll
  for (int m = 32; m >= 1; m >>= 1) v = max(v, __shfl_xor(v, m, 64));
  return v;
}

// LDS byte offset of 16-byte chunk `chunk` of tile row `row` (256-byte rows).
// XOR-swizzling the chunk with the row keeps both the 16-byte K reads (32
// rows, one chunk) and the 8-byte V reads (one row, all chunks) free of bank
// conflicts.
__device__ __forceinline__ int tile_off(int row, int chunk) {
  return row * 256 + ((chunk ^ (row & 15)) << 4);
}

template <typename T, bool PSPLIT>
__global__ __launch_bounds__(256, 2) void prefill_kernel(AttnArgs a, int32_t lg_tok) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const kv_lds = smem;
  int32_t* const page_tbl = reinterpret_cast<int32_t*>(smem + 2 * kStageBytes);
  int32_t* const red = page_tbl + kTablePages;

  const int tid = threadIdx.x;
  const int lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int n = lane & 31;
  const int hh = lane >> 5;
  const int Hkv = a.num_kv_heads;
  const int G = a.group;
  const int tpb = 1 << lg_tok;  // tokens per workgroup
  const int64_t R = a.num_requests;
  const int64_t nblk = a.num_tokens / tpb + R;
  const int h = static_cast<int>(blockIdx.x % Hkv);
  // Late blocks of late requests first: they see the most keys.
  const int64_t j = nblk - 1 - static_cast<int64_t>(blockIdx.x / Hkv);

  // Request owning block slot j. Request r's blocks occupy slots
  // [qsl[r] / T + r, qsl[r] / T + r + ceil(n_r / T)), which never overlap.
  int64_t rl = 0, rh = R - 1;
  while (rl < rh) {
    const int64_t mid = (rl + rh + 1) >> 1;
    if (a.qsl[mid] / tpb + mid <= j) rl = mid; else rh = mid - 1;
  }
  const int64_t r = rl;
  const int64_t qs = a.qsl[r], qe = a.qsl[r + 1];
  if (qs < 0 || qe > a.num_tokens || qe - qs <= 1) return;
  const int64_t b = j - (qs / tpb + r);
  const int64_t t0 = qs + b * tpb;
  if (b < 0 || t0 >= qe) return;
  const int64_t t1 = t0 + tpb < qe ? t0 + tpb : qe;

  // ---- rows of this lane: (head hg of the group, token tok)
  const int f = wave * 32 + n;
  const int hg = f >> lg_tok;
  const int64_t tok = t0 + (f & (tpb - 1));
  const bool row_ok = tok < t1;
  const int hq = h * G + hg;
  int32_t lo_n = 1, hi_n = 0;
  if (row_ok) {
    int64_t lo, hi;
    visible_range(a, r, qs, tok, lo, hi);
    if (hi >= lo) {
      lo_n = static_cast<int32_t>(lo);
      hi_n = static_cast<int32_t>(hi);
    }
  }
  const bool nonempty = hi_n >= lo_n;
  // Wave-uniform bounds of the wave's rows' visible ranges.
  const int32_t w_lo_min = __builtin_amdgcn_readfirstlane(wave_min_i(nonempty ? lo_n : INT_MAX));
  const int32_t w_lo_max = __builtin_amdgcn_readfirstlane(wave_max_i(nonempty ? lo_n : INT_MIN));
  const int32_t w_hi_min = __builtin_amdgcn_readfirstlane(wave_min_i(nonempty ? hi_n : INT_MAX));
  const int32_t w_hi_max = __builtin_amdgcn_readfirstlane(wave_max_i(nonempty ? hi_n : -1));
  if (lane == 0) {
    red[2 * wave] = w_lo_min;
    red[2 * wave + 1] = w_hi_max;
  }

  // Q^T as B operands: lane (n, hh) holds row n, dims 16 st + 8 hh .. +8.
  short8_t qv[8];
  {
    const short8_t zero = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + (row_ok ? tok : t0) * a.q_s0 +
                         static_cast<int64_t>(hq) * a.q_s1 + 8 * hh;
#pragma unroll
    for (int st = 0; st < 8; ++st)
      qv[st] = row_ok ? *reinterpret_cast<const short8_t*>(qp + 16 * st) : zero;
  }
  __syncthreads();
  int32_t kmin = INT_MAX, kmax = -1;
#pragma unroll
  for (int w = 0; w < kWaves; ++w) {
    kmin = min(kmin, red[2 * w]);
    kmax = max(kmax, red[2 * w + 1]);
  }
  kmin = __builtin_amdgcn_readfirstlane(kmin);
  kmax = __builtin_amdgcn_readfirstlane(kmax);

  float16v oacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) oacc[c] = float16v{};
  float m_c = -INFINITY;  // running offset of this row (exp2 domain)
  float l = 0.f;          // this lane's share of the row's softmax sum
  const float cs = a.scale_log2;

  const uint16_t* cache = static_cast<const uint16_t*>(a.cache);
  const int64_t head_elems = static_cast<int64_t>(h) * kDim;
  const int32_t base = kmax >= kmin ? (kmin & ~15) : 0;
  const int32_t ntiles = kmax >= kmin ? (kmax - base) / kTileKeys + 1 : 0;

  const uint32_t kv_addr = lds_address(kv_lds);
  const uint32_t bs32 = static_cast<uint32_t>(a.block_size);
  for (int32_t c0 = 0; c0 < ntiles; c0 += kChunkTiles) {
    const int32_t nt = ntiles - c0 < kChunkTiles ? ntiles - c0 : kChunkTiles;
    // Block ids of the chunk's pages; pages past the last visible key are
    // never looked up (their table entries may be anything).
    for (int i = tid; i < nt * 4; i += 256) {
      const int32_t pos = base + kTileKeys * c0 + 16 * i;
      page_tbl[i] = pos <= kmax ? static_cast<int32_t>(block_of(a, r, pos)) : -1;
    }
    __syncthreads();

    // Wave w moves page w of tile tl (16 keys, K and V) straight into LDS
    // stage `stage`: instruction i covers tile rows 16 w + 4 i .. +3; lane l
    // lands at row 16 w + 4 i + l / 16, physical chunk l % 16, so it fetches
    // the logical chunk that the swizzle puts there. An unmapped page is not
    // loaded (its keys are masked and its V rows zeroed).
    auto issue_page = [&](int32_t tl, int stage) {
      const int32_t id = __builtin_amdgcn_readfirstlane(page_tbl[4 * tl + wave]);
      if (id < 0) return;
      const uint32_t pos = static_cast<uint32_t>(base + kTileKeys * (c0 + tl) + 16 * wave);
      const int64_t row0 = pos % bs32;
      const uint16_t* page = cache + static_cast<int64_t>(id) * a.c_s[1] + row0 * a.c_s[2] + head_elems;
      const uint32_t kdst = kv_addr + stage * kStageBytes + wave * 4096;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rip = 4 * i + (lane >> 4);     // row in the page (its swizzle is rip)
        const int chunk = (lane & 15) ^ rip;     // logical 16-byte chunk stored at lane's slot
        const uint16_t* src = page + rip * a.c_s[2] + 8 * chunk;
        lds_dma_load16(src, kdst + i * 1024);
        lds_dma_load16(src + a.c_s[0], kdst + kTileBytes + i * 1024);
      }
    };

    issue_page(0, 0);
    wait_vmcnt<0>();
    __syncthreads();

    for (int32_t tl = 0; tl < nt; ++tl) {
      const int stage = tl & 1;
      // The other stage was last read before the previous barrier.
      if (tl + 1 < nt) issue_page(tl + 1, stage ^ 1);
      const int32_t k0 = base + kTileKeys * (c0 + tl);
      if (k0 <= w_hi_max && k0 + kTileKeys - 1 >= w_lo_min) {
        uint32_t pv = 0;
#pragma unroll
        for (int p = 0; p < 4; ++p) pv |= (page_tbl[4 * tl + p] >= 0 ? 1u : 0u) << p;
        pv = __builtin_amdgcn_readfirstlane(pv);
        const bool edge = k0 < w_lo_max || k0 + kTileKeys - 1 > w_hi_min || pv != 0xFu;
        const uint8_t* kt = kv_lds + stage * kStageBytes;
        const uint8_t* vt = kt + kTileBytes;

        float16v s[2];
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
          s[bb] = float16v{};
          const int row = 32 * bb + n;
#pragma unroll
          for (int st = 0; st < 8; ++st) {
            const short8_t kk = *reinterpret_cast<const short8_t*>(kt + tile_off(row, 2 * st + hh));
            s[bb] = Mma32<T>::mma(kk, qv[st], s[bb]);
          }
        }
        // s[bb][i] = score of key 32 bb + 8 (i / 4) + 4 hh + i % 4 for row n.
        if (edge) {
          const int32_t rlo = lo_n - k0, rhi = hi_n - k0;
#pragma unroll
          for (int bb = 0; bb < 2; ++bb)
#pragma unroll
            for (int i = 0; i < 16; ++i) {
              const int kk = 32 * bb + 8 * (i >> 2) + 4 * hh + (i & 3);
              const bool page_ok = (pv >> (2 * bb + (i >> 3))) & 1u;
              const bool vis = page_ok && kk >= rlo && kk <= rhi;
              s[bb][i] = vis ? s[bb][i] : -INFINITY;
            }
        }
        float mx = -INFINITY;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[bb][i]);
        mx = fmaxf(mx, __shfl_xor(mx, 32, 64));
        const float mx_c = mx * cs;
        const bool grow = mx_c > m_c + 8.f;
        if (__ballot(grow)) {
          const float m_new = grow ? mx_c : m_c;
          const float alpha = grow ? __builtin_amdgcn_exp2f(m_c - m_new) : 1.f;
          l *= alpha;
#pragma unroll
          for (int c = 0; c < 4; ++c) oacc[c] *= alpha;
          m_c = m_new;
        }
        const float m_use = m_c == -INFINITY ? 0.f : m_c;

        // Keys of the tile that no row of this wave may see (edge tiles only).
        const int32_t vlo = w_lo_min - k0, vhi = w_hi_max - k0;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb) {
          float p[16];
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s[bb][i], cs, -m_use));
            l += p[i];
          }
#pragma unroll
          for (int s2 = 0; s2 < 2; ++s2) {
            // P^T B operand: keys 32 bb + 16 s2 + 8 u + 4 hh + e  <->  k = 8 hh + 4 u + e.
            uint32_t ph[4], pl[4];
#pragma unroll
            for (int w = 0; w < 4; ++w) {
              ph[w] = Mma32<T>::pack2(p[8 * s2 + 2 * w], p[8 * s2 + 2 * w + 1]);
              if constexpr (PSPLIT) {
                const float2v back = Mma32<T>::unpack2(ph[w]);
                pl[w] = Mma32<T>::pack2(p[8 * s2 + 2 * w] - back[0], p[8 * s2 + 2 * w + 1] - back[1]);
              }
            }
            const short8_t pb_hi = __builtin_bit_cast(short8_t, uint4{ph[0], ph[1], ph[2], ph[3]});
            short8_t pb_lo = {};
            if constexpr (PSPLIT) pb_lo = __builtin_bit_cast(short8_t, uint4{pl[0], pl[1], pl[2], pl[3]});

            // V rows of those keys, dims 4 n .. 4 n + 3.
            uint2 rv[2][4];
#pragma unroll
            for (int u = 0; u < 2; ++u)
#pragma unroll
              for (int e = 0; e < 4; ++e) {
                const int key = 32 * bb + 16 * s2 + 8 * u + 4 * hh + e;
                rv[u][e] = *reinterpret_cast<const uint2*>(vt + tile_off(key, n >> 1) + 8 * (n & 1));
              }
            if (edge) {
              const bool page_ok = (pv >> (2 * bb + s2)) & 1u;
#pragma unroll
              for (int u = 0; u < 2; ++u)
#pragma unroll
                for (int e = 0; e < 4; ++e) {
                  const int key = 32 * bb + 16 * s2 + 8 * u + 4 * hh + e;
                  const bool keep = page_ok && key >= vlo && key <= vhi;
                  rv[u][e].x = keep ? rv[u][e].x : 0u;
                  rv[u][e].y = keep ? rv[u][e].y : 0u;
                }
            }
            // A operand of dim block c: row m <-> dim 4 m + c.
            short8_t av[4];
            {
              uint32_t w0[4], w1[4], w2[4], w3[4];
#pragma unroll
              for (int w = 0; w < 4; ++w) {
                const uint2 x0 = rv[w >> 1][2 * (w & 1)];
                const uint2 x1 = rv[w >> 1][2 * (w & 1) + 1];
                w0[w] = pack_lo16(x0.x, x1.x);
                w1[w] = pack_hi16(x0.x, x1.x);
                w2[w] = pack_lo16(x0.y, x1.y);
                w3[w] = pack_hi16(x0.y, x1.y);
              }
              av[0] = __builtin_bit_cast(short8_t, uint4{w0[0], w0[1], w0[2], w0[3]});
              av[1] = __builtin_bit_cast(short8_t, uint4{w1[0], w1[1], w1[2], w1[3]});
              av[2] = __builtin_bit_cast(short8_t, uint4{w2[0], w2[1], w2[2], w2[3]});
              av[3] = __builtin_bit_cast(short8_t, uint4{w3[0], w3[1], w3[2], w3[3]});
            }
#pragma unroll
            for (int c = 0; c < 4; ++c) {
              oacc[c] = Mma32<T>::mma(av[c], pb_hi, oacc[c]);
              if constexpr (PSPLIT) oacc[c] = Mma32<T>::mma(av[c], pb_lo, oacc[c]);
            }
          }
        }
      }
      wait_vmcnt<0>();
      __syncthreads();
    }
  }

  const float lt = l + __shfl_xor(l, 32, 64);
  if (!row_ok) return;
  // O^T block c, register 4 q + e of lane (n, hh): dim 32 q + 16 hh + 4 e + c.
  const float inv = nonempty ? 1.f / lt : NAN;  // an empty visible range is NaN, as in the reference
  uint16_t* op = static_cast<uint16_t*>(a.out) + tok * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1 + 16 * hh;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    uint32_t w[8];
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      w[2 * e] = Mma32<T>::pack2(oacc[0][4 * q + e] * inv, oacc[1][4 * q + e] * inv);
      w[2 * e + 1] = Mma32<T>::pack2(oacc[2][4 * q + e] * inv, oacc[3][4 * q + e] * inv);
    }
    uint4* dst = reinterpret_cast<uint4*>(op + 32 * q);
    dst[0] = uint4{w[0], w[1], w[2], w[3]};
    dst[1] = uint4{w[4], w[5], w[6], w[7]};
  }
}

template <typename T, bool PSPLIT>
int launch_prefill_t(const AttnArgs& a, hipStream_t s, hipEvent_t start, hipEvent_t stop) {
  int lg_tok = 0;
  while ((kRows >> lg_tok) > a.group) ++lg_tok;  // T = kRows / G
  const int64_t nblk = a.num_tokens / (int64_t{1} << lg_tok) + a.num_requests;
  const int64_t blocks = nblk * a.num_kv_heads;
  if (blocks <= 0) return MVLLM_OK;
  if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "prefill grid too large");
  static bool raised = false;  // per instantiation; the attribute is process-wide
  if (!raised) {
    MVLLM_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_kernel<T, PSPLIT>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kLdsBytes)));
    raised = true;
  }
  hipExtLaunchKernelGGL(prefill_kernel<T, PSPLIT>, dim3(static_cast<unsigned>(blocks)), dim3(256),
                        kLdsBytes, s, start, stop, 0, a, lg_tok);
  MVLLM_LAUNCH_CHECK("prefill_kernel");
  return MVLLM_OK;
}

}  // namespace

bool prefill_supported(const AttnArgs& a, int32_t dtype) {
  if (dtype != MVLLM_DTYPE_BF16 && dtype != MVLLM_DTYPE_F16) return false;
  if (a.head_dim != kDim || a.block_size % 16 != 0) return false;
  const int g = a.group;
  if (g != 1 && g != 2 && g != 4 && g != 8 && g != 16) return false;
  // Key positions and block ids are carried as int32 inside the kernel.
  if (a.width * a.block_size >= (int64_t{1} << 30) || a.num_blocks >= INT32_MAX) return false;
  return true;
}

int launch_prefill(const AttnArgs& a, int32_t dtype, hipStream_t s, hipEvent_t start,
                   hipEvent_t stop) {
  if (!prefill_supported(a, dtype))
    return fail(MVLLM_ERR_UNSUPPORTED, "prefill kernel does not support this geometry");
  // bf16 keeps P in bf16 (as the reference's Triton kernel keeps it in its
  // input type); fp16 carries P as a hi/lo pair to meet fp16 tolerances.
  if (dtype == MVLLM_DTYPE_BF16) return launch_prefill_t<bf16_t, false>(a, s, start, stop);
  return launch_prefill_t<f16_t, true>(a, s, start, stop);
}

}  // namespace mvllm
