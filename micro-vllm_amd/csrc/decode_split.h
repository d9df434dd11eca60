// The split-KV decode tile loop of the pipelined decode kernel, as a device
// function: the decode kernel (attention_decode.hip) and the one-launch
// attention step (attention_prefill.hip), which runs decode and prefill
// workgroups in one grid, both call it.
//
// Work item: (KV head, split of the visible context, request). One wavefront
// owns one KV head; a workgroup holds `waves` consecutive KV heads of the
// same (request, split), so together they stream whole token rows (all heads
// of a token are contiguous in the cache). Per 16-token tile a wave computes
// S^T = K . Q^T with four v_mfma_f32_16x16x32 (M = 16 tokens, N = the G query
// heads of the KV head, padded to 16, K = 128 dims); the softmax runs on the
// accumulator layout, and P^T is the B operand of O^T += V^T . P^T
// (v_mfma_f32_16x16x16), fed as a hi/lo pair so the product keeps ~16
// mantissa bits.
#pragma once

#include <cmath>

#include "worklists.h"

namespace mvllm {
namespace {
namespace dec {
constexpr int kDim = 128;

template <typename T>
__device__ __forceinline__ void split_hi_lo(float p, uint32_t& hi, uint32_t& lo) {
  hi = Elem<T>::to_bits(p);
  lo = Elem<T>::to_bits(p - Elem<T>::from_bits(hi));
}

// Epilogue shared by the decode kernels. acc[j][c][e] is
// O[head hq][dim 64j + 16grp + 4e + c] (unnormalised), m / lt the running
// max (exp2 domain) and the complete softmax denominator of this split. A
// request with one split gets its output directly; otherwise the partial goes
// to the workspace for the combine kernel.
template <typename T>
__device__ __forceinline__ void write_decode_result(const AttnArgs& a, int64_t r, int64_t qs, int hq,
                                                    int split, int64_t ns, float m, float lt,
                                                    const float4_t (&acc)[2][4], int grp) {
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

// ---------------------------------------------------------------------------
// Pipelined variant for block sizes that are multiples of 16 (every 16-token
// tile then lies in one block). K and V tiles go straight from HBM to LDS
// (global_load_lds_dwordx4): each load instruction covers 4 tokens x 256 B,
// i.e. whole 128-byte lines. Tile slot (token t, 16-byte chunk q) lives at
// LDS chunk 16t + (q ^ swz(t)) with swz(t) = t ^ ((t & 4) << 1), which keeps
// 8 consecutive lanes inside one line on the global side and makes both LDS
// read patterns (K rows as MFMA A operands, V columns for V^T) free of bank
// conflicts. STAGES tiles per wave are in flight; waits are explicit vmcnt
// counts because the only vector-memory instructions in the loop are these
// tile loads (the split's block ids are fetched once, up front). The loads
// carry the non-temporal hint: every K/V byte is read exactly once, and
// keeping the stream from displacing other cached lines raised the measured
// bandwidth from 5.5 to 6.0 TB/s on the Qwen3 decode batch.

constexpr int kTileBytes = 16 * 256;  // one 16-token tile of one head, K or V

__device__ __forceinline__ int tile_swizzle(int t) { return t ^ ((t & 4) << 1); }

__device__ __forceinline__ void wait_vmcnt_dyn(int n) {
  // n is wave-uniform; 8 loads per tile in flight, at most 3 tiles ahead.
  if (n >= 24) wait_vmcnt<24>();
  else if (n >= 16) wait_vmcnt<16>();
  else if (n >= 8) wait_vmcnt<8>();
  else wait_vmcnt<0>();
}

template <typename T, int STAGES>
__device__ __forceinline__ void decode_split_lds_body(const AttnArgs& a, uint8_t* smem, uint32_t wg, int waves) {
  const int wave = threadIdx.x >> 6;
  const int lane = threadIdx.x & 63;
  const int col = lane & 15;
  const int grp = lane >> 4;
  // 1-D grid: workgroup b takes head group b % groups of work-list slot b / groups.
  const int groups = (a.num_kv_heads + waves - 1) / waves;
  const int h = static_cast<int>(wg % groups) * waves + wave;
  // The work-list record carries the request's query token, visible range
  // and this split's key range, so the first tile loads wait on two
  // dependent loads (the record, then the block ids) rather than four.
  const DecodeItem item = a.decode_items[wg / groups];
  if (item.r < 0 || item.r >= a.num_requests) return;
  if (h >= a.num_kv_heads) return;
  const int split = item.split;
  const int64_t r = item.r;
  const int64_t qs = item.qs;
  const int64_t lo = item.lo;
  const int64_t begin = item.begin;
  const int64_t end = item.end;
  // Records index the query, the table and the partials: out-of-range
  // fields (never written by the work-list kernel) end the workgroup.
  if (begin < 0 || begin > end || end - begin >= a.split_tokens || end >= a.width * a.block_size ||
      qs < 0 || qs >= a.num_tokens || split < 0 || split >= a.max_splits)
    return;
  const int ntiles = static_cast<int>((end - begin) / 16 + 1);  // <= 128 (split <= 2048)

  // Block id and in-block row of tiles `lane` and `lane + 64` of this split,
  // fetched once (block ids are < 2^31; a 16-aligned tile never straddles a
  // block).
  int32_t my_block[2] = {-1, -1}, my_row[2] = {0, 0};
#pragma unroll
  for (int x = 0; x < 2; ++x) {
    if (lane + 64 * x < ntiles) {
      const int64_t p = begin + 16 * (lane + 64 * x);
      my_block[x] = static_cast<int32_t>(block_of(a, r, p));
      my_row[x] = static_cast<int32_t>(p % a.block_size);
    }
  }
  // Tile t's block id and row (t wave-uniform).
  auto tile_block = [&](int t) {
    return t < 64 ? __builtin_amdgcn_readlane(my_block[0], t) : __builtin_amdgcn_readlane(my_block[1], t - 64);
  };
  auto tile_row = [&](int t) {
    return t < 64 ? __builtin_amdgcn_readlane(my_row[0], t) : __builtin_amdgcn_readlane(my_row[1], t - 64);
  };

  const int G = a.group;
  const int hq = h * G + col;
  short8_t qv[4];
  {
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + qs * a.q_s0 +
                         static_cast<int64_t>(col < G ? hq : 0) * a.q_s1 + 8 * grp;
#pragma unroll
    for (int i = 0; i < 4; ++i)
      qv[i] = (col < G) ? *reinterpret_cast<const short8_t*>(qp + 32 * i) : short8_t{0, 0, 0, 0, 0, 0, 0, 0};
  }

  uint8_t* wave_lds = smem + static_cast<size_t>(wave) * STAGES * 2 * kTileBytes;
  const uint32_t wave_lds_addr = lds_address(wave_lds);
  const uint16_t* cache = static_cast<const uint16_t*>(a.cache);
  const int64_t head_elems = static_cast<int64_t>(h) * kDim;

  // Load-side mapping: instruction i, this lane -> token 4i + lane/16 of the
  // tile, 16-byte chunk q (element offset from the tile's first row).
  int64_t lane_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int t = 4 * i + (lane >> 4);
    const int q = (lane & 15) ^ tile_swizzle(t);
    lane_off[i] = t * a.c_s[2] + 8 * q;
  }

  auto issue = [&](int tile, int stage) {
    const int32_t blk = tile_block(tile);
    const int32_t row = tile_row(tile);
    const uint32_t kdst = wave_lds_addr + stage * 2 * kTileBytes;
    const uint32_t vdst = kdst + kTileBytes;
    // An invalid block id masks the whole tile: read a valid dummy line instead.
    const uint16_t* tile_k = blk >= 0 ? cache + static_cast<int64_t>(blk) * a.c_s[1] +
                                            static_cast<int64_t>(row) * a.c_s[2] + head_elems
                                      : cache;
    const int64_t plane = blk >= 0 ? a.c_s[0] : 0;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint16_t* src = blk >= 0 ? tile_k + lane_off[i] : cache;
      lds_dma_load16_stream(src, kdst + i * 1024);
      lds_dma_load16_stream(src + plane, vdst + i * 1024);
    }
  };

  float4_t acc[2][4];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int c = 0; c < 4; ++c) acc[j][c] = float4_t{0.f, 0.f, 0.f, 0.f};
  float m = -INFINITY, l = 0.f;

  // The block ids and Q must be in registers before the first tile address.
  __builtin_amdgcn_s_waitcnt(0);
#pragma unroll
  for (int s = 0; s < STAGES - 1; ++s)
    if (s < ntiles) issue(s, s);

  for (int k = 0; k < ntiles; ++k) {
    const int stage = k % STAGES;
    const int ahead = k + STAGES - 1;
    if (ahead < ntiles) {
      // The stage being refilled, (k - 1) % STAGES, was read in the previous
      // iteration. Its LDS reads have retired only because that iteration
      // ended with an lgkmcnt(0) wait; that wait is what makes the refill safe.
      issue(ahead, ahead % STAGES);
    }
    const int later = (ntiles - 1 - k) < (STAGES - 1) ? (ntiles - 1 - k) : (STAGES - 1);
    wait_vmcnt_dyn(8 * later);
    __builtin_amdgcn_wave_barrier();
    compiler_fence();

    const int64_t tb = begin + 16 * static_cast<int64_t>(k);
    const int64_t blk = tile_block(k);
    // Token j of the tile is visible iff its position is in [lo, end] and the block is valid.
    uint32_t okmask = 0;
    if (blk >= 0) {
      const int64_t first_ok = lo > tb ? lo - tb : 0;
      const int64_t last_ok = end - tb < 15 ? end - tb : 15;
      okmask = (last_ok >= first_ok) ? ((0xFFFFu >> (15 - last_ok)) & (0xFFFFu << first_ok)) : 0u;
    }
    const uint8_t* kt = wave_lds + stage * 2 * kTileBytes;
    const uint8_t* vt = kt + kTileBytes;

    float4_t sc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const short8_t kk = *reinterpret_cast<const short8_t*>(
          kt + 16 * (16 * col + ((4 * i + grp) ^ tile_swizzle(col))));
      sc = Mfma<T>::k32(kk, qv[i], sc);
    }
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

    uint32_t ph[4], pl[4];
#pragma unroll
    for (int e = 0; e < 4; ++e) split_hi_lo<T>(p[e], ph[e], pl[e]);
    const short4_t pb_hi = __builtin_bit_cast(short4_t, uint2{ph[0] | (ph[1] << 16), ph[2] | (ph[3] << 16)});
    const short4_t pb_lo = __builtin_bit_cast(short4_t, uint2{pl[0] | (pl[1] << 16), pl[2] | (pl[3] << 16)});
    // Rows of masked tokens may hold stale or non-finite data: zero them in V.
    const uint32_t mlo = ((okmask >> (4 * grp)) & 1u ? 0xFFFFu : 0u) | ((okmask >> (4 * grp + 1)) & 1u ? 0xFFFF0000u : 0u);
    const uint32_t mhi = ((okmask >> (4 * grp + 2)) & 1u ? 0xFFFFu : 0u) | ((okmask >> (4 * grp + 3)) & 1u ? 0xFFFF0000u : 0u);
#pragma unroll
    for (int j = 0; j < 2; ++j) {
      uint2 rv[4];
#pragma unroll
      for (int e = 0; e < 4; ++e) {
        const int t = 4 * grp + e;
        const int q = 8 * j + (col >> 1);
        rv[e] = *reinterpret_cast<const uint2*>(vt + 16 * (16 * t + (q ^ tile_swizzle(t))) + 8 * (col & 1));
      }
      short4_t av[4];
      av[0] = __builtin_bit_cast(short4_t, uint2{pack_lo16(rv[0].x, rv[1].x) & mlo, pack_lo16(rv[2].x, rv[3].x) & mhi});
      av[1] = __builtin_bit_cast(short4_t, uint2{pack_hi16(rv[0].x, rv[1].x) & mlo, pack_hi16(rv[2].x, rv[3].x) & mhi});
      av[2] = __builtin_bit_cast(short4_t, uint2{pack_lo16(rv[0].y, rv[1].y) & mlo, pack_lo16(rv[2].y, rv[3].y) & mhi});
      av[3] = __builtin_bit_cast(short4_t, uint2{pack_hi16(rv[0].y, rv[1].y) & mlo, pack_hi16(rv[2].y, rv[3].y) & mhi});
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        acc[j][c] = Mfma<T>::k16(av[c], pb_hi, acc[j][c]);
        acc[j][c] = Mfma<T>::k16(av[c], pb_lo, acc[j][c]);
      }
    }
    // All LDS reads of this stage must retire before a later issue refills it.
    __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0)
    compiler_fence();
  }

  const float lt = sum_xor32_f(sum_xor16_f(l));
  if (col >= G) return;
  write_decode_result<T>(a, r, qs, hq, split, item.ns, m, lt, acc, grp);
}

}  // namespace dec
}  // namespace
}  // namespace mvllm
