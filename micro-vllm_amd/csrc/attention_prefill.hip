// MFMA prefill / chunked-prefill kernel (requests with more than one query),
// head_dim 128, bf16/fp16, block sizes that are multiples of 16.
//
// Work item: (request, block of T query tokens, KV head), one workgroup of
// four waves. The workgroup's 128 rows are (query head of the KV head's
// group, token) pairs: row f -> head f / T, token f % T with T = 128 / G, so
// all G query heads that share a KV head (GQA) read each K/V tile once.
// Each wave owns 32 rows. A small kernel lists the items on the GPU, sorted
// by their number of key tiles, heaviest first (prefill_items_kernel).
//
// Keys are processed in tiles of 64 (four 16-token pages). Each wave moves
// one page of K and of V per tile straight from HBM into LDS
// (global_load_lds_dwordx4) into double-buffered K and V tiles: the loads of
// tile k+1 are issued between the MFMAs of tile k (a burst of loads would
// stall the issuing wave) and land before the tile's one barrier. Each wave
// reads its page of a tile from an LDS table of per-tile records (the page's
// packed block id and 16-row group, and the tile's valid-page mask), filled
// from the block table per chunk of 256 tiles, one iteration ahead, so no
// table lookup and little scalar arithmetic sits in the tile loop. Each
// tile is computed as two halves of 32 keys, each a full online-softmax
// update; that keeps the live registers under the 256 of two waves per SIMD.
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
// normalisation divides by a sum taken with the same offsets. Q is multiplied
// once per item by the softmax scale in the exp2 domain (log2(e) / sqrt(D))
// and rounded back to the input type, and the S MFMA chain starts from the
// row's running offset negated, so the MFMAs produce scaled, offset scores
// and an unmasked half takes exp2 of them directly. Halves that need no
// masking first skip the row maximum: their probabilities are taken
// against the current offset, and the half is redone from its maximum only
// if some lane's sum exceeds 2^12 (or is not finite).
//
// Order inside a tile: S(0); softmax(0); S(1); softmax(1) and P.V(0) in one
// basic block, which the compiler interleaves (the vector work of one half
// beside the other half's MFMAs); P.V(1); the tile's barrier.
//
// Masking: scores are masked only on tiles that cross a row's visible range
// or hold an unmapped page. V rows outside the workgroup's visible key range
// (the tile overhang) and rows of unmapped pages are zeroed in LDS once per
// tile, so stale or non-finite cache rows cannot leak through 0 * NaN and the
// P.V path never branches.
#include <climits>
#include <cmath>
#include <type_traits>

#include <hip/hip_ext.h>

#include "decode_split.h"

namespace mvllm {
namespace {

constexpr int kDim = 128;
constexpr int kTileKeys = 64;
constexpr int kWaves = 4;
static_assert(kRows == kWaves * 32, "rows per workgroup");
constexpr int kTileBytes = kTileKeys * kDim * 2;     // one K (or V) tile: 16 KiB
constexpr int kChunkTiles = 256;                     // key tiles whose pages are held in LDS at a time
constexpr int kTableInts = kChunkTiles * 8;          // per tile and wave: (page entry, tile's valid-page mask)
constexpr int kDummyBytes = 4096;                    // target of V page loads that are switched off
constexpr size_t kLdsBytes = 4 * kTileBytes + kTableInts * 4 + 16 * 4 + kDummyBytes;  // K, V double buffers

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
  // acc + the two bf16 values of w.
  __device__ static float dot2_ones(uint32_t w, float acc) {
    const bf16x2_t one = {static_cast<__bf16>(1.0f), static_cast<__bf16>(1.0f)};
    return __builtin_amdgcn_fdot2_f32_bf16(__builtin_bit_cast(bf16x2_t, w), one, acc, false);
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
  // acc + the two fp16 values of w.
  __device__ static float dot2_ones(uint32_t w, float acc) {
    const f16x2_t one = {static_cast<_Float16>(1.0f), static_cast<_Float16>(1.0f)};
    return __builtin_amdgcn_fdot2(__builtin_bit_cast(f16x2_t, w), one, acc, false);
  }
};

// Minimum / maximum over the wave, in every lane, with no LDS round trip:
// DPP quad permutes [1,0,3,2] and [2,3,0,1], then the 8- and 16-lane mirrors,
// then the 16- and 32-lane swaps.
template <typename Op>
__device__ __forceinline__ int32_t wave_reduce_i(int32_t v, Op op) {
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0xB1, 0xF, 0xF, false));
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x4E, 0xF, 0xF, false));
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x141, 0xF, 0xF, false));
  v = op(v, __builtin_amdgcn_update_dpp(v, v, 0x140, 0xF, 0xF, false));
  const auto r16 = __builtin_amdgcn_permlane16_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
  v = op(static_cast<int32_t>(r16[0]), static_cast<int32_t>(r16[1]));
  const auto r32 = __builtin_amdgcn_permlane32_swap(static_cast<uint32_t>(v), static_cast<uint32_t>(v), false, false);
  return op(static_cast<int32_t>(r32[0]), static_cast<int32_t>(r32[1]));
}

__device__ __forceinline__ int32_t wave_min_i(int32_t v) {
  return wave_reduce_i(v, [](int32_t x, int32_t y) { return x < y ? x : y; });
}

__device__ __forceinline__ int32_t wave_max_i(int32_t v) {
  return wave_reduce_i(v, [](int32_t x, int32_t y) { return x > y ? x : y; });
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

// lds_dma_load16_sbase with the LDS destination given as a wave-uniform
// base plus an immediate, added straight into M0 (s_add_u32 also writes SCC,
// which the clobber list declares).
template <int OFF>
__device__ __forceinline__ void lds_dma_load16_m0(const void* base, uint32_t offset, uint32_t lds_base) {
  asm volatile(
      "s_add_u32 m0, %1, %3\n\t"
      "s_nop 0\n\t"
      "global_load_lds_dwordx4 %0, %2"
      :
      : "v"(offset), "s"(lds_base), "s"(base), "i"(OFF)
      : "memory", "m0", "scc");
}

// Load i (of four) of a 16-row page: rows 4 i .. 4 i + 3, 1 KiB further into
// the page's LDS slot per load.
__device__ __forceinline__ void page_load(const void* src, int i, uint32_t lane_offset, uint32_t lds_slot) {
  if (i == 0) lds_dma_load16_m0<0>(src, lane_offset, lds_slot);
  else if (i == 1) lds_dma_load16_m0<1024>(src, lane_offset, lds_slot);
  else if (i == 2) lds_dma_load16_m0<2048>(src, lane_offset, lds_slot);
  else lds_dma_load16_m0<3072>(src, lane_offset, lds_slot);
}

typedef __attribute__((address_space(3))) const short8_t lds_short8c;
// LDS reads from a 32-bit LDS byte address (the constant part of the
// address goes into the instruction's offset field).
__device__ __forceinline__ short8_t lds_read_b128_at(uint32_t addr) {
  return *reinterpret_cast<lds_short8c*>(static_cast<uintptr_t>(addr));
}
__device__ __forceinline__ short4v lds_read_tr16_at(uint32_t addr) {
  return __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_short4v*>(static_cast<uintptr_t>(addr)));
}

// Page-table entry of the 16-key page at position pos: (block id << 4) |
// (the page's 16-row group inside its block), or -1 for an unmapped page.
// `row` is the request's block-table row. With a power-of-two number of
// pages per block the block and group come from shifts of pos / 16 (32-bit:
// positions stay below 2^30); otherwise from 64-bit division.
__device__ __forceinline__ int32_t page_entry(const AttnArgs& a, const int64_t* row, int64_t r, int32_t pos) {
  if (a.page_shift >= 0) {
    const uint32_t p16 = static_cast<uint32_t>(pos) >> 4;
    const int64_t b = row[static_cast<int64_t>(p16 >> a.page_shift) * a.t_s1];
    return (b >= 0 && b < a.num_blocks) ? static_cast<int32_t>((b << 4) | (p16 & ((1u << a.page_shift) - 1u))) : -1;
  }
  const int64_t b = block_of(a, r, pos);
  return b >= 0 ? static_cast<int32_t>((b << 4) | ((pos % a.block_size) >> 4)) : -1;
}

// The records of key tile i of a page-table chunk, starting at key position
// tpos: for each of its four 16-key pages (one per wave), the page entry
// (-1 past `last` or unmapped) and the tile's valid-page mask.
__device__ __forceinline__ void fill_tile_record(int32_t* tbl, const AttnArgs& a, int64_t r, int i, int32_t tpos,
                                                 int32_t last) {
  const int64_t* row = a.table + r * a.t_s0;
  int32_t e[4];
  uint32_t mask = 0;
#pragma unroll
  for (int w = 0; w < 4; ++w) {
    const int32_t pos = tpos + 16 * w;
    e[w] = pos <= last ? page_entry(a, row, r, pos) : -1;
    mask |= e[w] >= 0 ? 1u << w : 0u;
  }
  int4* rec = reinterpret_cast<int4*>(tbl + 8 * i);
  rec[0] = int4{e[0], static_cast<int32_t>(mask), e[1], static_cast<int32_t>(mask)};
  rec[1] = int4{e[2], static_cast<int32_t>(mask), e[3], static_cast<int32_t>(mask)};
}

template <typename T>
__device__ __forceinline__ void prefill_body(const AttnArgs& a, int32_t lg_tok, uint8_t* smem, uint32_t wg) {
  uint8_t* const kbuf = smem;                   // K stages 0, 1 (16 KiB each)
  uint8_t* const vbuf = smem + 2 * kTileBytes;  // V stages 0, 1
  int32_t* const page_tbl = reinterpret_cast<int32_t*>(smem + 4 * kTileBytes);
  int32_t* const red = page_tbl + kTableInts;
  uint8_t* const dummy = reinterpret_cast<uint8_t*>(red + 16);

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
  // Consecutive workgroups take the KV heads of one work item (so each XCD
  // keeps reading the same head); items come heaviest first.
  const int h = static_cast<int>(wg % Hkv);
  const int64_t slot = static_cast<int64_t>(wg / Hkv);
  if (slot >= nblk) return;
  // The record carries the rows' tokens and the hull [first row's first
  // key, last row's last key], so the page table of that range is fetched
  // while the rows' own ranges load; one barrier then publishes both.
  const PrefillItem item = a.items[slot];
  if (item.r < 0 || item.r >= R) return;
  const int64_t r = item.r;
  const int64_t qs = item.qs;
  const int64_t t0 = item.t0;
  const int64_t t1 = item.t1;
  if (qs < 0 || t0 < qs || t0 >= t1 || t1 > a.num_tokens) return;
  const int32_t hull_lo = item.lo, hull_hi = item.hi;
  // The hull bounds the page-table fill below: keep it inside the table.
  const bool hull_ok = hull_hi >= hull_lo && hull_lo >= 0 && hull_hi < a.width * a.block_size;
  const int32_t hull_base = hull_ok ? (hull_lo & ~15) : 0;
  const int32_t hull_tiles = hull_ok ? (hull_hi - hull_base) / kTileKeys + 1 : 0;

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
  // Block ids of the hull's first chunk of pages (pages past its last key
  // are never looked up: their table entries may be anything).
  {
    const int32_t nt = hull_tiles < kChunkTiles ? hull_tiles : kChunkTiles;
    for (int i = tid; i < nt; i += 256) fill_tile_record(page_tbl, a, r, i, hull_base + kTileKeys * i, hull_hi);
  }
  // Wave-uniform bounds of the wave's rows' visible ranges.
  const int32_t w_lo_min = __builtin_amdgcn_readfirstlane(wave_min_i(nonempty ? lo_n : INT_MAX));
  const int32_t w_lo_max = __builtin_amdgcn_readfirstlane(wave_max_i(nonempty ? lo_n : INT_MIN));
  const int32_t w_hi_min = __builtin_amdgcn_readfirstlane(wave_min_i(nonempty ? hi_n : INT_MAX));
  const int32_t w_hi_max = __builtin_amdgcn_readfirstlane(wave_max_i(nonempty ? hi_n : -1));
  if (lane == 0) {
    red[2 * wave] = w_lo_min;
    red[2 * wave + 1] = w_hi_max;
  }

  // Q^T as B operands: lane (n, hh) holds row n, dims 16 st + 8 hh .. +8,
  // each multiplied by the softmax scale in the exp2 domain (log2(e) /
  // sqrt(D)) and rounded back to the input type, so the MFMAs produce
  // scaled scores and the softmax needs no multiply.
  short8_t qv[8];
  {
    const short8_t zero = {0, 0, 0, 0, 0, 0, 0, 0};
    const uint16_t* qp = static_cast<const uint16_t*>(a.q) + (row_ok ? tok : t0) * a.q_s0 +
                         static_cast<int64_t>(hq) * a.q_s1 + 8 * hh;
#pragma unroll
    for (int st = 0; st < 8; ++st) {
      const short8_t raw = row_ok ? *reinterpret_cast<const short8_t*>(qp + 16 * st) : zero;
      const uint4 w = __builtin_bit_cast(uint4, raw);
      uint32_t sw[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float2v f = Mma32<T>::unpack2(sw[j]);
        sw[j] = Mma32<T>::pack2(f[0] * a.scale_log2, f[1] * a.scale_log2);
      }
      qv[st] = __builtin_bit_cast(short8_t, uint4{sw[0], sw[1], sw[2], sw[3]});
    }
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
  // Rows inside the hull (always, when ranges grow with the token): keys
  // [hull_lo, hull_hi], whose first chunk of block ids is already in LDS.
  // Otherwise the rows' own bounds, and the table is fetched again.
  const bool hull_table = hull_ok && kmax >= kmin && kmin >= hull_lo && kmax <= hull_hi;
  if (hull_table) {
    kmin = hull_lo;
    kmax = hull_hi;
  }

  float16v oacc[4];
#pragma unroll
  for (int c = 0; c < 4; ++c) oacc[c] = float16v{};
  // Softmax state of this lane's row, in the exp2 domain. m_c is the
  // running offset (-inf until the row has seen a visible key); the S MFMAs
  // start from the accumulator value -c_in, so they produce scores already
  // shifted by c_in = (m_c finite ? m_c : 0), and halves whose offset does
  // not change take exp2 of the MFMA results directly.
  float m_c = -INFINITY;
  float c_in = 0.f;
  float16v neg_c = float16v{};
  float l = 0.f;          // this lane's share of the row's softmax sum

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
  // LDS byte addresses from the start of dynamic LDS (the static size): as
  // plain integers they stay constants, where addresses derived from the
  // shared array's symbol are recomputed next to each use.
  const uint32_t lds0 = __builtin_amdgcn_groupstaticsize();
  const uint32_t kaddr = lds0;
  const uint32_t vaddr = lds0 + 2 * kTileBytes;
  const uint32_t daddr = lds0 + static_cast<uint32_t>(dummy - smem);
  uint32_t klane[8], vlane[8];
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    klane[x] = lds0 + koff[x];
    vlane[x] = lds0 + 2 * kTileBytes + voff[x];
    // Opaque to the compiler, so the sums stay in registers instead of
    // being recomputed next to every read.
    asm volatile("" : "+v"(klane[x]), "+v"(vlane[x]));
  }
  // Byte offsets within a 16-row page segment of the page loads: instruction
  // i covers rows 4 i .. 4 i + 3; lane l lands at row 4 i + l / 16, physical
  // chunk l % 16, so it fetches the logical chunk that the swizzle puts there.
  uint32_t dma_off[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int rip = 4 * i + (lane >> 4);
    dma_off[i] = static_cast<uint32_t>(2 * (rip * a.c_s[2] + 8 * ((lane & 15) ^ tile_swizzle(rip))));
  }
  const char* const cache_bytes = static_cast<const char*>(a.cache);
  // Byte strides of a block and of a 16-row group (32-bit: see prefill_supported).
  const char* const cache_head = cache_bytes + 2 * head_elems;
  const uint32_t blk_bytes = static_cast<uint32_t>(2 * a.c_s[1]);
  const uint32_t grp_bytes = static_cast<uint32_t>(32 * a.c_s[2]);

  for (int32_t c0 = 0; c0 < ntiles; c0 += kChunkTiles) {
    const int32_t nt = ntiles - c0 < kChunkTiles ? ntiles - c0 : kChunkTiles;
    // Block ids of the chunk's pages; pages past the last visible key are
    // never looked up (their table entries may be anything).
    if (c0 > 0 || !hull_table) {
      for (int i = tid; i < nt; i += 256) fill_tile_record(page_tbl, a, r, i, base + kTileKeys * (c0 + i), kmax);
      __syncthreads();
    }

    // Wave w moves page w of each tile into LDS (K and V), four 1 KiB
    // instructions each. Byte address of the K page segment with entry id:
    auto page_base = [&](int32_t id) {
      const uint32_t u = static_cast<uint32_t>(id);
      return cache_head + static_cast<uint64_t>(u >> 4) * blk_bytes + (u & 15u) * grp_bytes;
    };
    // Unmapped page (or beyond the last visible key): its V rows are zeroed.
    auto zero_v = [&](int stage) {
      uint8_t* slot = vbuf + stage * kTileBytes + wave * 4096;
#pragma unroll
      for (int i = 0; i < 4; ++i) *reinterpret_cast<uint4*>(slot + i * 1024 + 16 * lane) = uint4{0, 0, 0, 0};
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
    // This wave's record of a tile: its page's entry and the tile's
    // valid-page mask (one LDS read; tiles past the chunk read the last
    // valid record and are never used).
    auto tile_rec = [&](int32_t tl) {
      const int32_t t = tl < nt ? tl : nt - 1;
      return *reinterpret_cast<const int2*>(page_tbl + 8 * t + 2 * wave);
    };
    auto own_id = [&](int2 rec) { return __builtin_amdgcn_readfirstlane(rec.x); };
    auto page_mask = [&](int2 rec) { return static_cast<uint32_t>(__builtin_amdgcn_readfirstlane(rec.y)); };
    // Wave-uniform page facts of tile tl (valid-page mask) and tile tl + 1
    // (this wave's page entry, mask), read from LDS one iteration ahead.
    uint32_t cur_mask = page_mask(tile_rec(0));
    int32_t nxt_own;
    uint32_t nxt_mask;
    {
      const int2 rec = tile_rec(1);
      nxt_own = own_id(rec);
      nxt_mask = page_mask(rec);
    }
    // The stage is a compile-time constant (the loop below is unrolled by
    // two), so LDS offsets fold into the instructions' offset fields.
    auto step = [&](int32_t tl, auto stage_c) {
      constexpr int stage = decltype(stage_c)::value;
      // Loads of tile tl + 1 into the other stage, issued between the S
      // MFMAs below so that the address unit drains while the matrix cores
      // work (a burst of loads stalls the issuing wave).
      const int32_t nid = nxt_own;
      // The loads have no branches. An unmapped page still reads a mapped
      // one: its K rows land in the other stage (its scores are masked), its
      // V rows in the dummy region, as the stage's rows are being zeroed.
      // With no next tile, nothing reads the other stage before the next
      // chunk's first loads, which wait for these.
      if (tl + 1 < nt && nid < 0) zero_v(stage ^ 1);
      const char* const kp = page_base(nid >= 0 ? nid : 0);
      const char* const vp = kp + 2 * a.c_s[0];
      const uint32_t kdst = kaddr + (stage ^ 1) * kTileBytes + wave * 4096;
      const uint32_t vdst = nid >= 0 ? vaddr + (stage ^ 1) * kTileBytes + wave * 4096 : daddr;
      const int2 fut_rec = tile_rec(tl + 2);

      // The tile as two halves of 32 keys, each a full online-softmax
      // update, ordered so that each half's softmax runs beside MFMAs of the
      // same wave: S(0); softmax(0) beside S(1); softmax(1) beside P.V(0);
      // P.V(1). Each pairing is one basic block on the common path, so the
      // compiler interleaves the vector and matrix instructions.
      auto half_k0 = [&](int bb) { return base + kTileKeys * (c0 + tl) + 32 * bb; };
      auto half_pages = [&](int bb) { return (cur_mask >> (2 * bb)) & 3u; };
      auto half_edge = [&](int bb) {
        const int32_t k0 = half_k0(bb);
        return k0 < w_lo_max || k0 + 31 > w_hi_min || half_pages(bb) != 3u;
      };
      auto read_k = [&](int bb, short8_t (&kf)[8]) {
#pragma unroll
        for (int st = 0; st < 8; ++st) kf[st] = lds_read_b128_at(klane[st] + stage * kTileBytes + 8192 * bb);
      };
      // V operands of both 16-key steps of half bb (transposing reads).
      auto read_v = [&](int bb, short4v (&vf)[2][8]) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int x = 0; x < 8; ++x) vf[q][x] = lds_read_tr16_at(vlane[x] + stage * kTileBytes + 8192 * bb + 4096 * q);
      };
      // S^T of half bb from the K fragments, starting at `init` (-c_in), with
      // the loads of tile tl + 1 between the MFMAs: K pages with half 0, V
      // pages with half 1. PIN places each load after its MFMA pair.
      auto s_chain = [&](int bb, const short8_t (&kf)[8], float16v init, auto pin_c) {
        constexpr bool PIN = decltype(pin_c)::value;
        float16v s = init;
#pragma unroll
        for (int st = 0; st < 8; ++st) {
          s = Mma32<T>::mma(kf[st], qv[st], s);
          if (st & 1) {
            const int i = st >> 1;
            if constexpr (PIN) __builtin_amdgcn_sched_barrier(0);
            page_load(bb == 0 ? kp : vp, i, dma_off[i], bb == 0 ? kdst : vdst);
            if constexpr (PIN) __builtin_amdgcn_sched_barrier(0);
          }
        }
        return s;
      };
      // s[i] = scaled score of key k0 + 8 (i / 4) + 4 hh + i % 4, row n,
      // minus c_in: -inf outside the row's visible range or on an unmapped
      // page.
      auto mask = [&](int bb, float16v& s) {
        const int32_t k0 = half_k0(bb);
        const uint32_t pv = half_pages(bb);
        // kk = 8 (i / 4) + 4 hh + i % 4: the lane's 4 hh goes into the
        // bounds, so each compare takes an immediate.
        const int32_t rlo = lo_n - k0 - 4 * hh, rhi = hi_n - k0 - 4 * hh;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          constexpr int kk_base[16] = {0, 1, 2, 3, 8, 9, 10, 11, 16, 17, 18, 19, 24, 25, 26, 27};
          const bool page_ok = (pv >> (i >> 3)) & 1u;
          const bool vis = page_ok && kk_base[i] >= rlo && kk_base[i] <= rhi;
          s[i] = vis ? s[i] : -INFINITY;
        }
      };
      // O^T += V^T . P^T over a half's two 16-key steps.
      auto pv_mma = [&](const short4v (&vf)[2][8], const short8_t (&pb)[2]) {
#pragma unroll
        for (int q = 0; q < 2; ++q)
#pragma unroll
          for (int c = 0; c < 4; ++c) {
            const short4v lo4 = vf[q][c], hi4 = vf[q][4 + c];
            const short8_t av = short8_t{lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
            oacc[c] = Mma32<T>::mma(av, pb[q], oacc[c]);
          }
      };
      // Probabilities exp2(s + shift) (P^T B operands in pb), the add
      // skipped for SHIFTED false; returns this lane's share of their row
      // sum, taken over the rounded values the P.V product uses.
      auto make_p = [&](const float16v& s, float shift, auto shifted_c, short8_t (&pb)[2]) {
        constexpr bool SHIFTED = decltype(shifted_c)::value;
        float inc = 0.f;
        float p[16];
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          p[i] = __builtin_amdgcn_exp2f(SHIFTED ? s[i] + shift : s[i]);
        }
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          // P^T B operand: keys 16 s2 + 8 u + 4 hh + e  <->  k = 8 hh + 4 u + e.
          uint32_t ph[4];
#pragma unroll
          for (int w = 0; w < 4; ++w) {
            ph[w] = Mma32<T>::pack2(p[8 * s2 + 2 * w], p[8 * s2 + 2 * w + 1]);
            inc = Mma32<T>::dot2_ones(ph[w], inc);
          }
          pb[s2] = __builtin_bit_cast(short8_t, uint4{ph[0], ph[1], ph[2], ph[3]});
        }
        return inc;
      };
      // From the half's row maximum: a new offset when the maximum grew by
      // more than 2^8 over the current one (the accumulators and the sum
      // rescaled), then the probabilities against it; c_in follows.
      auto softmax_slow = [&](float16v& s, short8_t (&pb)[2]) {
        float mx = -INFINITY;
#pragma unroll
        for (int i = 0; i < 16; ++i) mx = fmaxf(mx, s[i]);
        mx = max_with_partner(mx);
        const float mx_c = mx + c_in;
        const bool grow = mx_c > m_c + 8.f;
        if (__ballot(grow)) {
          const float m_new = grow ? mx_c : m_c;
          const float alpha = grow ? __builtin_amdgcn_exp2f(m_c - m_new) : 1.f;
          l *= alpha;
#pragma unroll
          for (int c = 0; c < 4; ++c) oacc[c] *= alpha;
          m_c = m_new;
        }
        const float m_eff = m_c == -INFINITY ? 0.f : m_c;
        const float inc = make_p(s, c_in - m_eff, std::true_type{}, pb);
        c_in = m_eff;
        neg_c = float16v{} - m_eff;
        return inc;
      };
      // A half's softmax with `work` (MFMAs of this wave that do not depend
      // on it) in the same block. A half first tries the current offset with
      // no row maximum (the scores already carry it): a lane's 16
      // probabilities summing to at most 2^12 keep each below 2^12, which
      // bf16 and fp16 P and the accumulators hold; otherwise (a maximum that
      // grew, an unset offset, NaN) the half is redone from its maximum.
      auto softmax_with = [&](float16v& s, short8_t (&pb)[2], auto&& work) {
        work();
        // Speculative: the probabilities are formed in the same block as
        // `work`, and kept only when every lane has an offset.
        float inc = make_p(s, 0.f, std::false_type{}, pb);
        const bool done = !__ballot(m_c == -INFINITY || !(inc <= 4096.f));
        if (!done) inc = softmax_slow(s, pb);
        return inc;
      };

      // V operands of one 16-key step of half bb.
      auto read_v1 = [&](int bb, int q, short4v (&vq)[8]) {
#pragma unroll
        for (int x = 0; x < 8; ++x) vq[x] = lds_read_tr16_at(vlane[x] + stage * kTileBytes + 8192 * bb + 4096 * q);
      };
      short4v vf[2][8];
      float16v s0, s1;
      {
        short8_t kf[8];
        read_k(0, kf);
        __builtin_amdgcn_sched_barrier(0);
        s0 = s_chain(0, kf, neg_c, std::true_type{});
      }
      read_v1(0, 0, vf[0]);
      __builtin_amdgcn_sched_barrier(0);
      if (half_edge(0)) {
        // The empty asm keeps the compiler from if-converting the masking
        // into every tile: interior halves skip it entirely.
        asm volatile("");
        mask(0, s0);
      }
      short8_t pb0[2];
      l += softmax_with(s0, pb0, [] {});
      __builtin_amdgcn_sched_barrier(0);
      {
        short8_t kf[8];
        read_k(1, kf);
        __builtin_amdgcn_sched_barrier(0);
        s1 = s_chain(1, kf, neg_c, std::true_type{});
      }
      read_v1(0, 1, vf[1]);
      __builtin_amdgcn_sched_barrier(0);
      if (half_edge(1)) {
        asm volatile("");
        mask(1, s1);
      }
      // softmax(1) beside P.V(0).
      short8_t pb1[2];
      l += softmax_with(s1, pb1, [&] { pv_mma(vf, pb0); });
      __builtin_amdgcn_sched_barrier(0);
      read_v1(1, 0, vf[0]);
      read_v1(1, 1, vf[1]);
      __builtin_amdgcn_sched_barrier(0);
      pv_mma(vf, pb1);
      __builtin_amdgcn_sched_barrier(0);
      wait_vmcnt<0>();
      if (tl + 1 < nt) fix_v(tl + 1, stage ^ 1);
      __syncthreads();
      cur_mask = nxt_mask;
      nxt_own = own_id(fut_rec);
      nxt_mask = page_mask(fut_rec);
    };

    {
      const int32_t id = own_id(tile_rec(0));
      const char* kp = page_base(id >= 0 ? id : 0);
      if (id < 0) {
        zero_v(0);
      } else {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          lds_dma_load16_sbase(kp, dma_off[i], kaddr + wave * 4096 + i * 1024);
          lds_dma_load16_sbase(kp + 2 * a.c_s[0], dma_off[i], vaddr + wave * 4096 + i * 1024);
        }
      }
    }
    wait_vmcnt<0>();
    fix_v(0, 0);
    __syncthreads();
    int32_t tl = 0;
    for (; tl + 1 < nt; tl += 2) {
      step(tl, std::integral_constant<int, 0>{});
      step(tl + 1, std::integral_constant<int, 1>{});
    }
    if (tl < nt) step(tl, std::integral_constant<int, 0>{});
  }

  const float lt = sum_with_partner(l);
  // O^T block c, register 4 q + e of lane (n, hh): dim 32 c + 8 q + 4 hh + e.
  // Lanes n and n + 32 hold the two halves of each 8-dim group 8 q; one
  // v_permlane32_swap per word gives lane hh the whole group q = 2 p + hh,
  // so every lane writes 16-byte pieces.
  const float inv = nonempty ? 1.f / lt : NAN;  // an empty visible range is NaN, as in the reference
  uint16_t* op = static_cast<uint16_t*>(a.out) + tok * a.o_s0 + static_cast<int64_t>(hq) * a.o_s1;
#pragma unroll
  for (int c = 0; c < 4; ++c)
#pragma unroll
    for (int p = 0; p < 2; ++p) {
      uint32_t w[2][2];  // [q - 2 p][word]
#pragma unroll
      for (int u = 0; u < 2; ++u) {
        const int q = 2 * p + u;
        w[u][0] = Mma32<T>::pack2(oacc[c][4 * q] * inv, oacc[c][4 * q + 1] * inv);
        w[u][1] = Mma32<T>::pack2(oacc[c][4 * q + 2] * inv, oacc[c][4 * q + 3] * inv);
      }
      // Lane hh keeps its half of group 2 p + hh and sends its half of the
      // other group to its partner.
      uint32_t got[2];
#pragma unroll
      for (int k = 0; k < 2; ++k) {
        const uint32_t send = hh ? w[0][k] : w[1][k];
        const auto r2 = __builtin_amdgcn_permlane32_swap(send, send, false, false);
        got[k] = hh ? r2[0] : r2[1];
      }
      const uint4 piece = hh ? uint4{got[0], got[1], w[1][0], w[1][1]} : uint4{w[0][0], w[0][1], got[0], got[1]};
      if (row_ok) *reinterpret_cast<uint4*>(op + 32 * c + 8 * (2 * p + hh)) = piece;
    }
}

template <typename T>
__global__ __launch_bounds__(256, 2) void prefill_kernel(AttnArgs a, int32_t lg_tok) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  prefill_body<T>(a, lg_tok, smem, blockIdx.x);
}

// The one-launch attention step: the decode and prefill workgroups of a
// forward in one grid. The first `first` workgroups run one kind (the
// prefill ones when `prefill_first`), the rest the other, each indexing its
// own work list exactly as in its own kernel. A CU holds two workgroups of
// either kind (the launch reserves the prefill kernel's LDS, which covers
// the decode kernel's four waves of two K/V stages), so the grid needs no
// second stream to run prefill beside decode, and a batch without prefill
// work pays only for the prefill workgroups that find an empty record.
static_assert(kStepDecodeWaves * 2 * 2 * dec::kTileBytes <= kLdsBytes,
              "the step kernel's LDS must hold the decode kernel's tiles");

template <typename T>
__global__ __launch_bounds__(256, 2) void attention_step_kernel(AttnArgs a, int32_t lg_tok, uint32_t first,
                                                               int32_t prefill_first) {
  extern __shared__ __attribute__((aligned(16))) uint8_t smem[];
  const uint32_t b = blockIdx.x;
  const bool lead = b < first;
  const uint32_t wg = lead ? b : b - first;
  if (lead == (prefill_first != 0)) prefill_body<T>(a, lg_tok, smem, wg);
  else dec::decode_split_lds_body<T, 2>(a, smem, wg, kStepDecodeWaves);
}

__global__ __launch_bounds__(kItemThreads) void prefill_items_kernel(AttnArgs a, int32_t lg_tok) {
  build_prefill_list(a, lg_tok);
}


template <typename T>
int launch_prefill_t(const AttnArgs& a, hipStream_t s, hipEvent_t start, hipEvent_t stop) {
  const int lg_tok = prefill_lg_tok(a);
  const int64_t nblk = a.num_tokens / (int64_t{1} << lg_tok) + a.num_requests;
  const int64_t blocks = nblk * a.num_kv_heads;
  if (blocks <= 0) return MVLLM_OK;
  if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "prefill grid too large");
  if (!a.items) return fail(MVLLM_ERR_INVALID, "prefill work list is missing");
  if (!a.lists_ready) {
    prefill_items_kernel<<<1, kItemThreads, 0, s>>>(a, lg_tok);
    MVLLM_LAUNCH_CHECK("prefill_items_kernel");
  }
  static bool raised = false;  // per instantiation; the attribute is process-wide
  if (!raised) {
    MVLLM_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(prefill_kernel<T>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kLdsBytes)));
    raised = true;
  }
  hipExtLaunchKernelGGL(prefill_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(256),
                        kLdsBytes, s, start, stop, 0, a, lg_tok);
  MVLLM_LAUNCH_CHECK("prefill_kernel");
  return MVLLM_OK;
}

template <typename T>
int launch_step_t(const AttnArgs& a, bool prefill_first, hipStream_t s, hipEvent_t start, hipEvent_t stop) {
  const int lg_tok = prefill_lg_tok(a);
  const int64_t prefill_blocks = (a.num_tokens / (int64_t{1} << lg_tok) + a.num_requests) * a.num_kv_heads;
  const int64_t decode_blocks = decode_step_blocks(a);
  const int64_t first = prefill_first ? prefill_blocks : decode_blocks;
  const int64_t blocks = prefill_blocks + decode_blocks;
  if (blocks <= 0) return MVLLM_OK;
  if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "attention step grid too large");
  if (!a.items || !a.decode_items || !a.decode_req) return fail(MVLLM_ERR_INVALID, "work lists are missing");
  if (!a.lists_ready) {
    if (int rc = launch_decode_lists(a, s)) return rc;
    prefill_items_kernel<<<1, kItemThreads, 0, s>>>(a, lg_tok);
    MVLLM_LAUNCH_CHECK("prefill_items_kernel");
  }
  static bool raised = false;  // per instantiation; the attribute is process-wide
  if (!raised) {
    MVLLM_HIP_TRY(hipFuncSetAttribute(reinterpret_cast<const void*>(attention_step_kernel<T>),
                                      hipFuncAttributeMaxDynamicSharedMemorySize,
                                      static_cast<int>(kLdsBytes)));
    raised = true;
  }
  hipExtLaunchKernelGGL(attention_step_kernel<T>, dim3(static_cast<unsigned>(blocks)), dim3(256),
                        kLdsBytes, s, start, stop, 0, a, lg_tok, static_cast<uint32_t>(first),
                        prefill_first ? 1 : 0);
  MVLLM_LAUNCH_CHECK("attention_step_kernel");
  return MVLLM_OK;
}

}  // namespace

int launch_prefill_lists(const AttnArgs& a, hipStream_t s) {
  const int lg_tok = prefill_lg_tok(a);
  const int64_t blocks = (a.num_tokens / (int64_t{1} << lg_tok) + a.num_requests) * a.num_kv_heads;
  if (blocks <= 0) return MVLLM_OK;
  if (blocks > INT32_MAX) return fail(MVLLM_ERR_INVALID, "prefill grid too large");
  if (!a.items) return fail(MVLLM_ERR_INVALID, "prefill work list is missing");
  prefill_items_kernel<<<1, kItemThreads, 0, s>>>(a, lg_tok);
  MVLLM_LAUNCH_CHECK("prefill_items_kernel");
  return MVLLM_OK;
}

bool prefill_supported(const AttnArgs& a, int32_t dtype) {
  if (dtype != MVLLM_DTYPE_BF16 && dtype != MVLLM_DTYPE_F16) return false;
  if (a.head_dim != kDim || a.block_size % 16 != 0) return false;
  const int g = a.group;
  if (g != 1 && g != 2 && g != 4 && g != 8 && g != 16) return false;
  // Key positions and block ids are carried as int32 inside the kernel.
  if (a.width * a.block_size >= (int64_t{1} << 30) || a.num_blocks >= INT32_MAX) return false;
  // Page-table entries pack (block id, 16-row group): 2^27 blocks of at most
  // 256 rows; block and group strides fit 32-bit byte offsets.
  if (a.num_blocks >= (int64_t{1} << 27) || a.block_size > 256) return false;
  if (2 * a.c_s[1] >= (int64_t{1} << 32) || 32 * a.c_s[2] >= (int64_t{1} << 32)) return false;
  return true;
}

int launch_prefill(const AttnArgs& a, int32_t dtype, hipStream_t s, hipEvent_t start,
                   hipEvent_t stop) {
  if (!prefill_supported(a, dtype))
    return fail(MVLLM_ERR_UNSUPPORTED, "prefill kernel does not support this geometry");
  // P is kept in the input type, as the reference's Triton kernel keeps it
  // (triton_paged.py:271-277).
  if (dtype == MVLLM_DTYPE_BF16) return launch_prefill_t<bf16_t>(a, s, start, stop);
  return launch_prefill_t<f16_t>(a, s, start, stop);
}

int launch_step(const AttnArgs& a, int32_t dtype, bool prefill_first, hipStream_t s, hipEvent_t start,
                hipEvent_t stop) {
  if (!prefill_supported(a, dtype) || !decode_step_eligible(a))
    return fail(MVLLM_ERR_UNSUPPORTED, "the attention step kernel does not support this geometry");
  if (a.width * a.block_size > INT32_MAX || a.num_tokens > INT32_MAX)
    return fail(MVLLM_ERR_UNSUPPORTED, "decode positions beyond 2^31 are not supported");
  int rc = dtype == MVLLM_DTYPE_BF16 ? launch_step_t<bf16_t>(a, prefill_first, s, start, stop)
                                     : launch_step_t<f16_t>(a, prefill_first, s, start, stop);
  if (rc) return rc;
  return launch_decode_combine(a, dtype, s);
}

}  // namespace mvllm
