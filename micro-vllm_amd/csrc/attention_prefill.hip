// MFMA prefill / chunked-prefill kernel (requests with more than one query),
// head_dim 128, bf16/fp16, block sizes that are multiples of 16.
//
// Work item: (request, block of T query tokens, KV head), one workgroup of
// four waves. The workgroup's 128 rows are (query head of the KV head's
// group, token) pairs: row f -> head f / T, token f % T with T = 128 / G, so
// all G query heads that share a KV head (GQA) read each K/V tile once.
// Each wave owns 32 rows.
//
// Keys are processed in tiles of 64 (four 16-token pages). Each wave moves
// one page of K and of V per tile straight from HBM into LDS
// (global_load_lds_dwordx4) into double-buffered K and V tiles: the loads of
// tile k+1 are in flight while tile k is computed, with one barrier per tile.
// The block ids of a tile's four pages are read from an LDS copy of the
// block-table row one iteration ahead, so no table lookup sits on the
// critical path. The K fragments of a tile are read in batches ahead of their
// MFMAs, and the V operands of the first two 16-key steps are in flight
// during the softmax.
//
// Scores: S^T = K . Q^T as two v_mfma_f32_32x32x16 blocks (32 keys x 32
// rows): each lane holds the scores of ONE row (lane % 32) for 16 keys per
// block, so the row max and sum are in-lane plus one v_permlane32_swap.
// P^T, as produced by the accumulator layout, is already the B operand of
// O^T += V^T . P^T; the V^T A operand comes straight from transposing LDS
// reads (ds_read_b64_tr_b16: in each 16-lane group, lane i receives element
// i % 4 of the addresses given by lanes 4k + i / 4, k = 0..3).
//
// The online softmax (FlashAttention-2, Dao 2023) runs in the exp2 domain and
// rescales the accumulators only when a row's maximum grows by more than 2^8
// (lazy rescaling as in FlashAttention-3, Shah et al. 2024); the final
// normalisation divides by a sum taken with the same offsets.
//
// Masking: scores are masked only on tiles that cross a row's visible range
// or hold an unmapped page. V rows outside the workgroup's visible key range
// (the tile overhang) and rows of unmapped pages are zeroed in LDS once per
// tile, so stale or non-finite cache rows cannot leak through 0 * NaN and the
// P.V path never branches.
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
constexpr int kTablePages = 2048;                    // block ids held in LDS at a time
constexpr int kChunkTiles = kTablePages / 4;
constexpr size_t kLdsBytes = 4 * kTileBytes + kTablePages * 4 + 16 * 4;  // K, V double buffers

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
// The chunk is XOR-swizzled with r ^ ((r & 2) << 2), r = row % 16. Both read
// patterns are then free of bank conflicts: the K reads (32 rows, one chunk:
// the swizzle is a bijection of r) and the transposing V reads (8 rows 8u ..
// 8u + 7, chunks 4c .. 4c + 3: every physical chunk is hit exactly twice).
__device__ __forceinline__ int tile_swizzle(int row) {
  const int r = row & 15;
  return r ^ ((r & 2) << 2);
}

__device__ __forceinline__ int tile_off(int row, int chunk) {
  return row * 256 + ((chunk ^ tile_swizzle(row)) << 4);
}

__device__ __forceinline__ float max_with_partner(float x) {
  // v_permlane32_swap(x, x): lanes 0-31 get x[l + 32] in the second result,
  // lanes 32-63 get x[l - 32] in the first; the other result is x itself.
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

__device__ __forceinline__ float sum_with_partner(float x) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(x), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

typedef short short4v __attribute__((ext_vector_type(4)));
typedef __attribute__((address_space(3))) short4v lds_short4v;

// Transposing LDS read (see the file comment for its lane layout).
__device__ __forceinline__ short4v lds_read_tr16(const uint8_t* p) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16((lds_short4v*)(p));
}

template <typename T, bool PSPLIT>
__global__ __launch_bounds__(256, 2) void prefill_kernel(AttnArgs a, int32_t lg_tok) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  uint8_t* const kbuf = smem;                   // K stages 0, 1 (16 KiB each)
  uint8_t* const vbuf = smem + 2 * kTileBytes;  // V stages 0, 1
  int32_t* const page_tbl = reinterpret_cast<int32_t*>(smem + 4 * kTileBytes);
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

  // Per-lane LDS byte offsets within a tile.
  // K, A operand of S^T: row n (+ 32 bb), chunk 2 st + hh.
  int koff[8];
#pragma unroll
  for (int st = 0; st < 8; ++st) koff[st] = tile_off(n, 2 * st + hh);
  // V, transposing reads for the A operand of O^T (dim block c, keys
  // 8 hh + 4 u .. +4): lane (g = lane / 16, j = lane % 16) points at row
  // 8 u + 4 (g / 2) + j / 4 (+ 32 bb + 16 s2), dims 32 c + 16 (g % 2) + 4 (j % 4).
  int voff[8];
  {
    const int g = lane >> 4, jj = lane & 15;
#pragma unroll
    for (int u = 0; u < 2; ++u)
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const int row = 8 * u + 4 * (g >> 1) + (jj >> 2);
        const int dim = 32 * c + 16 * (g & 1) + 4 * (jj & 3);
        voff[4 * u + c] = tile_off(row, dim >> 3) + 2 * (dim & 7);
      }
  }
  const uint32_t kaddr = lds_address(kbuf);
  const uint32_t vaddr = lds_address(vbuf);
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

    // Wave w moves page w of tile tl into LDS: instruction i covers page rows
    // 4 i .. 4 i + 3; lane l lands at row 4 i + l / 16, physical chunk l % 16,
    // so it fetches the logical chunk that the swizzle puts there.
    auto page_src = [&](int32_t tl, int32_t id) {
      const uint32_t pos = static_cast<uint32_t>(base + kTileKeys * (c0 + tl) + 16 * wave);
      const int64_t row0 = pos % bs32;
      return cache + static_cast<int64_t>(id) * a.c_s[1] + row0 * a.c_s[2] + head_elems;
    };
    auto issue_k = [&](int32_t tl, int stage, int32_t id) {
      if (id < 0) return;  // an unmapped page's keys are masked
      const uint16_t* page = page_src(tl, id);
      const uint32_t dst = kaddr + stage * kTileBytes + wave * 4096;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rip = 4 * i + (lane >> 4);
        lds_dma_load16(page + rip * a.c_s[2] + 8 * ((lane & 15) ^ tile_swizzle(rip)), dst + i * 1024);
      }
    };
    auto issue_v = [&](int32_t tl, int stage, int32_t id) {
      uint8_t* slot = vbuf + stage * kTileBytes + wave * 4096;
      if (id < 0) {
        // Unmapped (or beyond the last visible key): zero rows.
#pragma unroll
        for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(slot + i * 1024 + 16 * lane) = uint4{0, 0, 0, 0};
        return;
      }
      const uint16_t* page = page_src(tl, id) + a.c_s[0];
      const uint32_t dst = vaddr + stage * kTileBytes + wave * 4096;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int rip = 4 * i + (lane >> 4);
        lds_dma_load16(page + rip * a.c_s[2] + 8 * ((lane & 15) ^ tile_swizzle(rip)), dst + i * 1024);
      }
    };
    // After the loads landed: zero the V rows of this wave's page that lie
    // outside [kmin, kmax] (they may hold stale or non-finite data).
    auto fix_v = [&](int32_t tl, int stage) {
      const int32_t pos0 = base + kTileKeys * (c0 + tl) + 16 * wave;
      if (pos0 >= kmin && pos0 + 15 <= kmax) return;
      uint8_t* slot = vbuf + stage * kTileBytes + wave * 4096;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int32_t p = pos0 + 4 * i + (lane >> 4);
        if (p < kmin || p > kmax) *reinterpret_cast<uint4*>(slot + i * 1024 + 16 * lane) = uint4{0, 0, 0, 0};
      }
    };
    // One tile: S = K . Q^T, softmax, O^T += V^T . P^T. LDS reads are issued
    // in batches ahead of the MFMAs that consume them (sched_barrier keeps
    // the compiler from sinking them next to their uses).
    // The four block ids of a tile (one LDS read; tiles past the chunk read
    // the last valid entry and are never used).
    auto tile_ids = [&](int32_t tl) {
      const int32_t t = tl < nt ? tl : nt - 1;
      return *reinterpret_cast<const int4*>(page_tbl + 4 * t);
    };
    auto page_mask = [&](int4 ids) {
      return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(
          (ids.x >= 0 ? 1 : 0) | (ids.y >= 0 ? 2 : 0) | (ids.z >= 0 ? 4 : 0) | (ids.w >= 0 ? 8 : 0)));
    };
    auto own_id = [&](int4 ids) {
      const int32_t v = wave == 0 ? ids.x : wave == 1 ? ids.y : wave == 2 ? ids.z : ids.w;
      return __builtin_amdgcn_readfirstlane(v);
    };
    // cur_ids: tile tl; nxt_ids: tile tl + 1 (read one iteration ahead).
    int4 cur_ids = tile_ids(0), nxt_ids = tile_ids(1);
    auto step = [&](int32_t tl) {
      const int stage = tl & 1;
      if (tl + 1 < nt) {
        const int32_t id = own_id(nxt_ids);
        issue_k(tl + 1, stage ^ 1, id);
        issue_v(tl + 1, stage ^ 1, id);
      }
      const int4 fut_ids = tile_ids(tl + 2);
      const int32_t k0 = base + kTileKeys * (c0 + tl);
      const uint32_t pv = page_mask(cur_ids);
      const bool edge = k0 < w_lo_max || k0 + kTileKeys - 1 > w_hi_min || pv != 0xFu;
      const uint8_t* kt = kbuf + stage * kTileBytes;
      const uint8_t* vt = vbuf + stage * kTileBytes;

      short8_t kf[2][8];
#pragma unroll
      for (int st = 0; st < 8; ++st) kf[0][st] = *reinterpret_cast<const short8_t*>(kt + koff[st]);
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int st = 0; st < 8; ++st) kf[1][st] = *reinterpret_cast<const short8_t*>(kt + 8192 + koff[st]);
      float16v s_cur[2];
      s_cur[0] = float16v{};
      s_cur[1] = float16v{};
#pragma unroll
      for (int st = 0; st < 8; ++st) s_cur[0] = Mma32<T>::mma(kf[0][st], qv[st], s_cur[0]);
#pragma unroll
      for (int st = 0; st < 8; ++st) s_cur[1] = Mma32<T>::mma(kf[1][st], qv[st], s_cur[1]);
      __builtin_amdgcn_sched_barrier(0);
      // V operands of the first two 16-key steps, in flight during the softmax.
      short4v vf[4][8];
#pragma unroll
      for (int q = 0; q < 2; ++q)
#pragma unroll
        for (int x = 0; x < 8; ++x) vf[q][x] = lds_read_tr16(vt + 256 * (16 * q) + voff[x]);
      __builtin_amdgcn_sched_barrier(0);

      // s_cur[bb][i] = score of key 32 bb + 8 (i / 4) + 4 hh + i % 4, row n.
      if (edge) {
        // The empty asm keeps the compiler from if-converting the masking
        // into every tile: interior tiles skip it entirely.
        asm volatile("");
        const int32_t rlo = lo_n - k0, rhi = hi_n - k0;
#pragma unroll
        for (int bb = 0; bb < 2; ++bb)
#pragma unroll
          for (int i = 0; i < 16; ++i) {
            const int kk = 32 * bb + 8 * (i >> 2) + 4 * hh + (i & 3);
            const bool page_ok = (pv >> (2 * bb + (i >> 3))) & 1u;
            const bool vis = page_ok && kk >= rlo && kk <= rhi;
            s_cur[bb][i] = vis ? s_cur[bb][i] : -INFINITY;
          }
      }
      float mx = -INFINITY;
#pragma unroll
      for (int bb = 0; bb < 2; ++bb)
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s_cur[bb][i]);
      mx = max_with_partner(mx);
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

      short8_t pb[4], pbl[4];
#pragma unroll
      for (int bb = 0; bb < 2; ++bb) {
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          p[i] = __builtin_amdgcn_exp2f(__builtin_fmaf(s_cur[bb][i], cs, -m_use));
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
          pb[2 * bb + s2] = __builtin_bit_cast(short8_t, uint4{ph[0], ph[1], ph[2], ph[3]});
          if constexpr (PSPLIT) pbl[2 * bb + s2] = __builtin_bit_cast(short8_t, uint4{pl[0], pl[1], pl[2], pl[3]});
        }
      }
      __builtin_amdgcn_sched_barrier(0);
      // O^T += V^T . P^T over the four 16-key steps q; the V operands of
      // step q + 2 are read while step q multiplies.
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        if (q + 2 < 4) {
#pragma unroll
          for (int x = 0; x < 8; ++x) vf[q + 2][x] = lds_read_tr16(vt + 256 * (16 * (q + 2)) + voff[x]);
        }
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const short4v lo4 = vf[q][c], hi4 = vf[q][4 + c];
          const short8_t av = short8_t{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          oacc[c] = Mma32<T>::mma(av, pb[q], oacc[c]);
          if constexpr (PSPLIT) oacc[c] = Mma32<T>::mma(av, pbl[q], oacc[c]);
        }
        __builtin_amdgcn_sched_barrier(0);
      }
      wait_vmcnt<0>();
      if (tl + 1 < nt) fix_v(tl + 1, stage ^ 1);
      __syncthreads();
      cur_ids = nxt_ids;
      nxt_ids = fut_ids;
    };

    {
      const int32_t id = own_id(cur_ids);
      issue_k(0, 0, id);
      issue_v(0, 0, id);
    }
    wait_vmcnt<0>();
    fix_v(0, 0);
    __syncthreads();
    for (int32_t tl = 0; tl < nt; ++tl) step(tl);
  }

  const float lt = sum_with_partner(l);
  if (!row_ok) return;
  // O^T block c, register 4 q + e of lane (n, hh): dim 32 c + 8 q + 4 hh + e.
  const float inv = nonempty ? 1.f / lt : NAN;  // an empty visible range is NaN, as in the reference
  uint16_t* op = static_cast<uint16_t*>(a.out) + tok * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1 + 4 * hh;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const uint32_t w0 = Mma32<T>::pack2(oacc[c][4 * q] * inv, oacc[c][4 * q + 1] * inv);
      const uint32_t w1 = Mma32<T>::pack2(oacc[c][4 * q + 2] * inv, oacc[c][4 * q + 3] * inv);
      *reinterpret_cast<uint2*>(op + 32 * c + 8 * q) = uint2{w0, w1};
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
