// attention.hip: softmax attention over fp32 rows in one pass for gfx950,
// on the fp32 matrix cores (v_mfma_f32_32x32x2f32): for every slice s
// (a head, or a head of one window) and query row t
//   out[s, t] = softmax_k(scale * q[s, t] . k[s, k] + bias[t, k]) . v[s, k]
// with bias none, a mask [rows, keys] shared by the slices (the decoder's
// prefill: the routed key mask, -inf where a key is not attended), or SAM's
// decomposed relative-position bias dh[t, ky] + dw[t, kx] (key = ky * w +
// kx). It replaces the reference's scores product, bias, row softmax and
// values product (src/model/cuda/cuda_vision.cpp:159-170,251-254,
// src/model/cuda/cuda_decoder.cpp:88-105): the scores never reach memory.
//
// A workgroup of 4 waves (2 with the relative-position bias over a grid of
// whole tiles) takes 128 (64) query rows of one slice; each wave owns 32 of
// them and walks the keys 32 at a time, the key tiles and transposed value
// tiles staged in LDS for the workgroup (the next tile's loads in flight in
// registers while the current one is used; without the relative-position
// bias two LDS stages, the next tile written while the current one is
// read); a wave past the last row only helps stage the tiles. Per tile a
// wave forms S^T = K Q^T (32 keys x 32
// queries, hd / 2 products, each summing 2 of the head's columns: lane half
// h supplies column h * hd / 2 + i to product i, so a lane keeps its query's
// half row in registers and reads its key's half row from LDS), which leaves
// lane l holding query l % 32's scores for 16 of the 32 keys (8 (r / 4) + 4 h
// + r % 4 in register r) and the other 16 in lane l ^ 32. The running max,
// rescale and sum are per lane plus one exchange with the partner lane. The
// values' product O^T += V^T P^T takes the probabilities straight from those
// registers: product i sums keys 8 (i / 4) + r % 4 + 4 h, exactly the keys
// register i holds, so P needs no movement, and a lane's V^T values for four
// consecutive products are one 16-byte read; each 32 columns of the head are
// 16 products into 16 accumulators.
//
// With a mask, a wave reads its 32 x 32 block of the mask before a tile's
// products and skips the tile where every entry is -inf: a causal mask's
// upper tiles, and all but the selected blocks (32 keys each) of the
// decoder's routed mask, cost only their share of the K/V staging.
//
// Arithmetic: fp32 products and sums on the matrix cores; the scores are
// scaled, then the bias added (the reference's order); e = exp(s - running
// max) with the running sum and the output rescaled when the max grows;
// out = O * (1 / sum); a row with no finite score gives zeros, as the
// reference's softmax does. The sums run in another order than the
// reference's row softmax and products, so results agree to fp32 rounding.

#include "common.hpp"

namespace uocr_rocm {
namespace {

typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr float kLog2e = 1.4426950408889634f;

// kRelPosRows: the relative-position bias where the grid's width is a
// multiple of the 32-key tile, so a tile's keys are 32 consecutive columns
// of one grid row: one height term per tile and the width terms as 4-wide
// vector reads, where kRelPos looks both up per key.
// kRelPosTable: kRelPosRows with the per-query dot products read from the
// table rel_dots_k formed in memory rather than copied into LDS (4 waves a
// workgroup: no LDS for them).
enum class Bias { kNone, kMask, kRelPos, kRelPosRows, kRelPosTable };
template <Bias kBias>
constexpr bool rel_pos() {
  return kBias == Bias::kRelPos || kBias == Bias::kRelPosRows || kBias == Bias::kRelPosTable;
}
// the per-query dot products held in LDS
template <Bias kBias>
constexpr bool dots_in_lds() {
  return kBias == Bias::kRelPos || kBias == Bias::kRelPosRows;
}
constexpr int kQueriesPerWave = 32;
constexpr int kKeyTile = 32;
// Waves per workgroup: 4 (128 query rows share each key/value tile), or 2
// with the relative-position bias over a grid of whole tiles (SAM's global
// layer: the per-query dot products, h + w of them, take LDS, and 2 waves
// keep three workgroups on a CU instead of one).
template <Bias kBias>
constexpr int waves_of() {
  return kBias == Bias::kRelPosRows ? 2 : 4;
}
constexpr int kMaxRelSpan = 256;  // h + w of the relative-position bias

struct AttnArgs {
  const float* q;
  const float* k;
  const float* v;
  float* out;
  int64_t ldq, sq, ldk, sk, ldv, sv, ldo, so;  // row and slice strides (elements)
  int rows, keys;
  float scale;
  const float* mask;  // [rows, mask_ld] (kMask)
  int64_t mask_ld;
  const float* rh;  // [h, h, hd] (kRelPos, kRelPosRows)
  const float* rw;  // [w, w, hd]
  int h, w;
  int dots_ld;  // floats between two query rows' dot products in LDS
  int dw_off;   // where a row's width terms start (its height terms at 0)
  // The dot products of every (slice, query row) formed beforehand by
  // rel_dots_k, [slices][rows][dots_ld] in the LDS layout; null: each
  // workgroup forms its own.
  const float* table;
  float* table_out;  // rel_dots_k's output (the same table)
  // Slices in two levels: slice s is (s / inner, s % inner), its operands at
  // (s / inner) * s_ + (s % inner) * i_ (inner 1: the single level)
  int inner;
  int64_t iq, ik, iv, io;
  // non-null: the output in bf16 (nearest even, the rounding a projection
  // reading it applies) at the same element offsets; out unused
  uint16_t* out16;
  // rel_dots_k's products are stored times this (1: the dots themselves)
  float table_mul = 1.0f;
  // non-null: the split-operand kernel's key and value tiles, formed by the
  // dot-table launch (kv_tiles_of), for key tiles of x3_rows grid rows
  uint16_t* kvx = nullptr;
  int x3_rows = -1;
  // non-null (attention_k with a mask): the mask's live-tile map (a bit per
  // 128 query rows and 32-key tile, map_words words per row block); a row
  // block's walk is cut into `runs` runs of run_tiles live tiles, and where
  // a block takes more than one, each run leaves per row (m, l) in part_ml
  // and its unnormalised output in part_o ([slices][row blocks][runs][128
  // rows]) for the merge launch
  const uint32_t* map = nullptr;
  int map_words = 0, run_tiles = 0, runs = 1;
  float* part_o = nullptr;
  float* part_ml = nullptr;
};

// Four output values at element offset off: fp32, or bf16 into out16.
__device__ __forceinline__ void store4(const AttnArgs& a, int64_t off, float v0, float v1, float v2, float v3) {
  if (a.out16 != nullptr) {
    *reinterpret_cast<u32x2*>(a.out16 + off) = u32x2{pack_bf16(v0, v1), pack_bf16(v2, v3)};
  } else {
    *reinterpret_cast<float4*>(a.out + off) = make_float4(v0, v1, v2, v3);
  }
}

template <int HD, int kThreads>
struct Tile {
  static constexpr int kChunks = kKeyTile * HD / 4;           // float4 chunks of one operand tile
  static constexpr int kPerThread = kChunks / kThreads;       // 2 to 8
  static constexpr int kKStride = HD + 4;                     // padded K rows: 16-lane reads conflict-free
  static constexpr int kVTStride = kKeyTile + 4;              // V^T rows (a dimension's 32 keys): 9 16-byte groups
};

template <int HD, int kThreads>
__device__ __forceinline__ void load_tile(const AttnArgs& a, const float* kb, const float* vb, int key0,
                                          float4 (&kr)[Tile<HD, kThreads>::kPerThread],
                                          float4 (&vr)[Tile<HD, kThreads>::kPerThread]) {
#pragma unroll
  for (int j = 0; j < Tile<HD, kThreads>::kPerThread; ++j) {
    const int idx = static_cast<int>(threadIdx.x) + kThreads * j;
    const int row = idx / (HD / 4), c4 = idx % (HD / 4);
    const int key = key0 + row;
    kr[j] = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    vr[j] = kr[j];
    if (key < a.keys) {
      kr[j] = *reinterpret_cast<const float4*>(kb + key * a.ldk + 4 * c4);
      vr[j] = *reinterpret_cast<const float4*>(vb + key * a.ldv + 4 * c4);
    }
  }
}

template <int HD, int kThreads>
__device__ __forceinline__ void store_tile(float* ks, float* vs, const float4 (&kr)[Tile<HD, kThreads>::kPerThread],
                                           const float4 (&vr)[Tile<HD, kThreads>::kPerThread]) {
#pragma unroll
  for (int j = 0; j < Tile<HD, kThreads>::kPerThread; ++j) {
    const int idx = static_cast<int>(threadIdx.x) + kThreads * j;
    const int row = idx / (HD / 4), c4 = idx % (HD / 4);
    *reinterpret_cast<float4*>(ks + row * Tile<HD, kThreads>::kKStride + 4 * c4) = kr[j];
    // V transposed: the values' product reads 4 keys of a dimension at once
    float* vt = vs + 4 * c4 * Tile<HD, kThreads>::kVTStride + row;
    vt[0] = vr[j].x;
    vt[Tile<HD, kThreads>::kVTStride] = vr[j].y;
    vt[2 * Tile<HD, kThreads>::kVTStride] = vr[j].z;
    vt[3 * Tile<HD, kThreads>::kVTStride] = vr[j].w;
  }
}

__device__ __forceinline__ float partner(float v) { return __shfl_xor(v, 32); }

// The offset of slice s of an operand with outer stride so and inner stride si.
__device__ __forceinline__ int64_t slice_at(const AttnArgs& a, int64_t s, int64_t so, int64_t si) {
  return a.inner == 1 ? s * so : (s / a.inner) * so + (s % a.inner) * si;
}

// Four mask entries from key4 (a multiple of 4) of a row: one 16-byte read
// where rows are whole 16-byte chunks apart (mask_ld % 4 == 0 and the mask
// 16-byte aligned; mask_ld >= keys, so a read that starts below keys stays
// in its row), else element by element; -inf from key `keys` on.
__device__ __forceinline__ float4 mask4(const float* row, int key4, int keys, bool vec) {
  float4 m = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
  if (vec) {
    m = *reinterpret_cast<const float4*>(row + key4);
  } else {
    m.x = row[key4];
    if (key4 + 1 < keys) m.y = row[key4 + 1];
    if (key4 + 2 < keys) m.z = row[key4 + 2];
    if (key4 + 3 < keys) m.w = row[key4 + 3];
  }
  if (key4 + 1 >= keys) m.y = -INFINITY;
  if (key4 + 2 >= keys) m.z = -INFINITY;
  if (key4 + 3 >= keys) m.w = -INFINITY;
  return m;
}

__device__ __forceinline__ bool mask_vec(const float* mask, int64_t mask_ld) {
  return (mask_ld & 3) == 0 && (reinterpret_cast<uintptr_t>(mask) & 15) == 0;
}

// The live tiles of a row block (the bits of its map words).
__device__ __forceinline__ int live_tiles(const uint32_t* tmap, int words) {
  int n = 0;
  for (int w = 0; w < words; ++w) n += __builtin_popcount(tmap[w]);
  return n;
}

// A walk over a row block's map: the word last read is kept, so a walk
// reads each word once (a scalar load per 32 tiles, not per tile).
struct MapCursor {
  const uint32_t* words;
  int idx;
  uint32_t w;
};

// The first live tile after t (tiles: none).
__device__ __forceinline__ int next_live_tile(MapCursor& m, int tiles, int t) {
  int u = t + 1;
  while (u < tiles) {
    if ((u >> 5) != m.idx) {
      m.idx = u >> 5;
      m.w = m.words[m.idx];
    }
    const uint32_t w = m.w >> (u & 31);
    if (w != 0) return u + __builtin_ctz(w);
    u = (u | 31) + 1;
  }
  return tiles;
}

template <int HD, Bias kBias>
__global__ __launch_bounds__(64 * waves_of<kBias>()) void attention_k(const AttnArgs a) {
  constexpr int kThreads = 64 * waves_of<kBias>();
  constexpr int kQueriesPerBlock = waves_of<kBias>() * kQueriesPerWave;
  using T = Tile<HD, kThreads>;
  constexpr int kHalf = HD / 2;  // columns per lane half in the scores' products
  constexpr int kDBlocks = HD / 32;
  // Two LDS stages of K and V^T without the relative-position bias (tile t
  // + 1 is written into one while tile t is read from the other: one barrier
  // a tile); one with it, whose per-query dot products take the LDS.
  constexpr int kStages = rel_pos<kBias>() ? 1 : 2;
  constexpr int kKElems = kKeyTile * T::kKStride, kVElems = HD * T::kVTStride;
  __shared__ __attribute__((aligned(16))) float ks[kStages * kKElems];
  __shared__ __attribute__((aligned(16))) float vs[kStages * kVElems];  // V^T
  // The relative-position bias: per query row its h height terms at 0 and
  // w width terms at dw_off, rows dots_ld apart: h + w + 1 (odd) for
  // kRelPos, so that the 32 queries of a wave read 32 different banks; for
  // kRelPosRows 4 times an odd number with dw_off a multiple of 4, so that
  // 16 queries' 16-byte reads at one offset cover 16 bank groups.
  extern __shared__ __attribute__((aligned(16))) float dots[];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, c = lane & 31;
  const int64_t slice = blockIdx.y;
  // with a mask, the last row blocks first (under a causal mask the longest
  // walks); with a map, workgroup x is (row block, run)
  const int run = kBias == Bias::kMask ? static_cast<int>(blockIdx.x) % a.runs : 0;
  const int rblk = kBias == Bias::kMask ? static_cast<int>(gridDim.x / a.runs - 1 - blockIdx.x / a.runs)
                                        : static_cast<int>(blockIdx.x);
  const int q0 = rblk * kQueriesPerBlock + wave * kQueriesPerWave;
  const int qrow = q0 + c;
  const bool qin = qrow < a.rows;
  const float* qb = a.q + slice_at(a, slice, a.sq, a.iq);
  const float* kb = a.k + slice_at(a, slice, a.sk, a.ik);
  const float* vb = a.v + slice_at(a, slice, a.sv, a.iv);

  // the tiles this workgroup walks: every one, or with a map the live tiles
  // of its run (uniform: scalar reads)
  const int tiles = (a.keys + kKeyTile - 1) / kKeyTile;
  const bool mapped = kBias == Bias::kMask && a.map != nullptr;
  const uint32_t* tmap = mapped ? a.map + static_cast<int64_t>(rblk) * a.map_words : nullptr;
  MapCursor cursor{tmap, -1, 0u};
  const int64_t orow = slice_at(a, slice, a.so, a.io) + static_cast<int64_t>(qrow) * a.ldo;
  int first = 0, block_runs = 1;
  if (mapped) {
    const int live = live_tiles(tmap, a.map_words);
    block_runs = (live + a.run_tiles - 1) / a.run_tiles;
    if (live == 0) {  // no key attended by any row of the block: zeros
      if (run == 0 && qin) {
#pragma unroll
        for (int e = 0; e < HD / 8; ++e) store4(a, orow + 8 * e + 4 * hl, 0.0f, 0.0f, 0.0f, 0.0f);
      }
      return;
    }
    if (run >= block_runs) return;  // uniform, before any barrier
    first = -1;
    for (int skip = run * a.run_tiles; skip >= 0; --skip) first = next_live_tile(cursor, tiles, first);
  }
  // the tile after t (i: t's place in the run), or tiles
  auto after = [&](int t, int i) {
    return mapped ? (i + 1 < a.run_tiles ? next_live_tile(cursor, tiles, t) : tiles) : t + 1;
  };

  // the first tile's loads go out first
  float4 kr[T::kPerThread], vr[T::kPerThread];
  load_tile<HD, kThreads>(a, kb, vb, first * kKeyTile, kr, vr);

  // this lane's half of its query row
  float qv[kHalf];
#pragma unroll
  for (int i = 0; i < kHalf; i += 4) {
    float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (qin) t = *reinterpret_cast<const float4*>(qb + qrow * a.ldq + hl * kHalf + i);
    qv[i] = t.x;
    qv[i + 1] = t.y;
    qv[i + 2] = t.z;
    qv[i + 3] = t.w;
  }

  float* my_dots = dots + (wave * kQueriesPerWave + c) * a.dots_ld;
  if constexpr (dots_in_lds<kBias>()) {
    if (a.table != nullptr) {
      // the workgroup's rows of the table lie contiguous in memory with the
      // LDS row stride: one coalesced copy by every thread
      const int first = rblk * kQueriesPerBlock;
      const int here = a.rows - first < kQueriesPerBlock ? a.rows - first : kQueriesPerBlock;
      const float* src = a.table + (slice * a.rows + first) * static_cast<int64_t>(a.dots_ld);
      const int count = here * a.dots_ld;
      if constexpr (kBias == Bias::kRelPosRows) {  // dots_ld a multiple of 4
        for (int i = 4 * static_cast<int>(threadIdx.x); i < count; i += 4 * kThreads) {
          *reinterpret_cast<float4*>(dots + i) = *reinterpret_cast<const float4*>(src + i);
        }
      } else {
        for (int i = static_cast<int>(threadIdx.x); i < count; i += kThreads) dots[i] = src[i];
      }
    }
  }
  if constexpr (dots_in_lds<kBias>()) {
    if (a.table == nullptr) {
    // dh[ky] = q . rh[qy, ky] and dw[kx] = q . rw[qx, kx]: each lane forms
    // the partial dot over the half of the columns it holds in qv (fp32 in
    // column order, the table rows as 16-byte loads), and the two halves'
    // partials are added, half 0's first, so that both lanes of a query
    // hold the same sum; half 0 stores the height terms, half 1 the width
    // terms.
    const int qy = qin ? qrow / a.w : 0, qx = qin ? qrow - qy * a.w : 0;
    const float* th = a.rh + static_cast<int64_t>(qy) * a.h * HD + hl * kHalf;
    const float* tw = a.rw + static_cast<int64_t>(qx) * a.w * HD + hl * kHalf;
    const int n_dots = a.h + a.w;
#pragma unroll 2
    for (int j = 0; j < n_dots; ++j) {
      const float* row = j < a.h ? th + j * HD : tw + (j - a.h) * HD;
      float p = 0.0f;
#pragma unroll
      for (int i = 0; i < kHalf; i += 4) {
        const float4 t = *reinterpret_cast<const float4*>(row + i);
        p = fmaf(qv[i], t.x, p);
        p = fmaf(qv[i + 1], t.y, p);
        p = fmaf(qv[i + 2], t.z, p);
        p = fmaf(qv[i + 3], t.w, p);
      }
      const float other = partner(p);
      const float dot = hl == 0 ? p + other : other + p;
      if ((j < a.h) == (hl == 0)) my_dots[j < a.h ? j : a.dw_off + (j - a.h)] = dot;
    }
    }
  }

  store_tile<HD, kThreads>(ks, vs, kr, vr);
  int nxt = after(first, 0);  // the tile after the current one
  if constexpr (kStages == 2) {
    if (nxt < tiles) load_tile<HD, kThreads>(a, kb, vb, nxt * kKeyTile, kr, vr);
  }
  __syncthreads();

  f32x16 o[kDBlocks];
#pragma unroll
  for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[b][r] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  // With a mask, this wave's 32 x 32 block of it (register r: key 8 (r / 4)
  // + 4 h + r % 4 of the tile; -inf past the keys or the rows), read a tile
  // ahead: where every entry is -inf (a causal or routed mask's dead tiles)
  // the wave skips the tile's products and softmax; the tile's K and V
  // still reach LDS for the other waves.
  constexpr int kMk = kBias == Bias::kMask ? 16 : 1;
  float mk[kMk], mn[kMk];
  const bool vec = kBias == Bias::kMask && mask_vec(a.mask, a.mask_ld);
  const float* mrow = a.mask + static_cast<int64_t>(qin ? qrow : 0) * a.mask_ld;
  auto load_mask = [&](int tt, float (&dst)[kMk]) {
    if constexpr (kBias == Bias::kMask) {
      const bool whole = vec && (tt + 1) * kKeyTile <= a.keys;  // uniform
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int key4 = tt * kKeyTile + 8 * g + 4 * hl;
        float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
        if (whole) {
          if (qin) v = *reinterpret_cast<const float4*>(mrow + key4);
        } else if (qin && key4 < a.keys) {
          v = mask4(mrow, key4, a.keys, vec);
        }
        dst[4 * g] = v.x;
        dst[4 * g + 1] = v.y;
        dst[4 * g + 2] = v.z;
        dst[4 * g + 3] = v.w;
      }
    }
  };
  load_mask(first, mk);
  int st = 0;  // the LDS stage holding the current tile
  for (int t = first, i = 0; t < tiles; ++i) {
    const int key0 = t * kKeyTile;
    const bool more = nxt < tiles;
    int nxt2 = tiles;  // (two stages) the tile after nxt, requested now
    if constexpr (kStages == 2) {
      if (more) store_tile<HD, kThreads>(ks + (st ^ 1) * kKElems, vs + (st ^ 1) * kVElems, kr, vr);
      nxt2 = more ? after(nxt, i + 1) : tiles;
      if (nxt2 < tiles) load_tile<HD, kThreads>(a, kb, vb, nxt2 * kKeyTile, kr, vr);
    } else {
      if (more) load_tile<HD, kThreads>(a, kb, vb, nxt * kKeyTile, kr, vr);
    }
    load_mask(more ? nxt : t, mn);
    const float* kcur = ks + st * kKElems;
    const float* vcur = vs + st * kVElems;

    // A wave whose rows all lie past the last query row (the tail workgroup
    // of a slice) only helps stage the tiles.
    bool live = q0 < a.rows;
    if constexpr (kBias == Bias::kMask) {
      bool any = false;
#pragma unroll
      for (int r = 0; r < 16; ++r) any = any || mk[r] != -INFINITY;
      live = live && __ballot(any) != 0;
    }
    if (live) {
      // S^T = K Q^T: 32 keys x 32 queries
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
      const float* krow = kcur + c * T::kKStride + hl * kHalf;
#pragma unroll
      for (int i = 0; i < kHalf; i += 4) {
        const float4 kk = *reinterpret_cast<const float4*>(krow + i);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.x, qv[i], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.y, qv[i + 1], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.z, qv[i + 2], s, 0, 0, 0);
        s = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.w, qv[i + 3], s, 0, 0, 0);
      }

      // scale, bias, running max
      float tmax = -INFINITY;
      int ky0 = 0, kx0 = 0;
      if constexpr (rel_pos<kBias>()) {
        ky0 = key0 / a.w;  // once per tile; the lane's keys step from here
        kx0 = key0 - ky0 * a.w;
      }
      // kRelPos: the grid position of the first key of each of this lane's
      // four groups of 4 consecutive keys (8 g + 4 h), each key then at most
      // one row further once the grid is at least 4 wide
      int gky[kBias == Bias::kRelPos ? 4 : 1], gkx[kBias == Bias::kRelPos ? 4 : 1];
      if constexpr (kBias == Bias::kRelPos) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          int ky = ky0, kx = kx0 + 8 * g + 4 * hl;
          while (kx >= a.w) {
            kx -= a.w;
            ++ky;
          }
          gky[g] = ky;
          gkx[g] = kx;
        }
      }
      // kRelPosRows: the tile's height term, and the width terms of this
      // lane's keys kx0 + 8 g + 4 h + (0..3)
      constexpr bool kRowTerms = kBias == Bias::kRelPosRows || kBias == Bias::kRelPosTable;
      float dh = 0.0f, dwv[kRowTerms ? 16 : 1];
      if constexpr (kRowTerms) {
        // kRelPosTable: the query's row of the table in memory
        const float* trow = kBias == Bias::kRelPosTable
                                ? a.table + (slice * a.rows + (qin ? qrow : 0)) * static_cast<int64_t>(a.dots_ld)
                                : my_dots;
        dh = trow[ky0];
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 t = *reinterpret_cast<const float4*>(trow + a.dw_off + kx0 + 8 * g + 4 * hl);
          dwv[4 * g] = t.x;
          dwv[4 * g + 1] = t.y;
          dwv[4 * g + 2] = t.z;
          dwv[4 * g + 3] = t.w;
        }
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int off = 8 * (r / 4) + 4 * hl + (r % 4), key = key0 + off;
        float x = s[r] * a.scale;
        if constexpr (kBias == Bias::kMask) {
          x = x + mk[r];
        } else if constexpr (kBias == Bias::kRelPos) {
          int ky = gky[r / 4], kx = gkx[r / 4] + r % 4;
          while (kx >= a.w) {  // at most once for a grid 4 or more wide
            kx -= a.w;
            ++ky;
          }
          if (key < a.keys) x = x + (my_dots[ky] + my_dots[a.dw_off + kx]);
        } else if constexpr (kRowTerms) {
          x = x + (dh + dwv[r]);
        }
        x = key < a.keys ? x : -INFINITY;
        s[r] = x;
        tmax = fmaxf(tmax, x);
      }
      tmax = fmaxf(tmax, partner(tmax));
      const float m_new = fmaxf(m, tmax);
      const bool dead = m_new == -INFINITY;  // nothing finite yet
      const float corr = dead ? 1.0f : __builtin_amdgcn_exp2f((m - m_new) * kLog2e);
      float psum = 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = dead ? 0.0f : __builtin_amdgcn_exp2f((s[r] - m_new) * kLog2e);
        psum += s[r];
      }
      psum += partner(psum);
      l = l * corr + psum;
      m = m_new;
      // the accumulators are rescaled only when some row's max moved (a
      // factor of exactly 1 elsewhere): most tiles skip the 16 hd / 32
      // multiplies
      if (__ballot(corr != 1.0f) != 0) {
#pragma unroll
        for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
          for (int r = 0; r < 16; ++r) o[b][r] *= corr;
        }
      }

      // O^T += V^T P^T: product i = 4 g + e sums keys 8 g + 4 h + e, held
      // in s[i]; the lane's four values of dimension 32 b + c for keys 8 g
      // + 4 h .. + 3 are one 16-byte read of its V^T row
#pragma unroll
      for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
        for (int g = 0; g < 4; ++g) {
          const float4 vt = *reinterpret_cast<const float4*>(vcur + (32 * b + c) * T::kVTStride + 8 * g + 4 * hl);
          o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt.x, s[4 * g], o[b], 0, 0, 0);
          o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt.y, s[4 * g + 1], o[b], 0, 0, 0);
          o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt.z, s[4 * g + 2], o[b], 0, 0, 0);
          o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vt.w, s[4 * g + 3], o[b], 0, 0, 0);
        }
      }
    }

    __syncthreads();  // every wave is done with this tile
    if constexpr (kStages == 1) {
      if (more) {
        store_tile<HD, kThreads>(ks, vs, kr, vr);
        __syncthreads();
      }
    }
    if constexpr (kBias == Bias::kMask) {
#pragma unroll
      for (int r = 0; r < 16; ++r) mk[r] = mn[r];
    }
    t = nxt;
    if constexpr (kStages == 2) {
      nxt = nxt2;
      st ^= 1;
    } else {
      nxt = more ? after(t, i + 1) : tiles;
    }
  }

  if (!qin) return;
  if (mapped && block_runs > 1) {
    // the run's partial record: (m, l) (lane half 0) and O unnormalised
    const int row_blocks = static_cast<int>(gridDim.x) / a.runs;
    const int64_t rec = ((slice * row_blocks + rblk) * a.runs + run) * kQueriesPerBlock + (qrow - rblk * kQueriesPerBlock);
    if (hl == 0) *reinterpret_cast<float2*>(a.part_ml + 2 * rec) = make_float2(m, l);
#pragma unroll
    for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * b + 8 * g + 4 * hl;
        *reinterpret_cast<float4*>(a.part_o + rec * HD + d) =
            make_float4(o[b][4 * g], o[b][4 * g + 1], o[b][4 * g + 2], o[b][4 * g + 3]);
      }
    }
    return;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * b + 8 * g + 4 * hl;
      store4(a, orow + d, o[b][4 * g] * inv, o[b][4 * g + 1] * inv, o[b][4 * g + 2] * inv, o[b][4 * g + 3] * inv);
    }
  }
}

// ---- split-bf16 products for a bf16 output ----------------------------------
//
// With the output rounded to bf16 (2^-9 relative) the fp32 products carry
// more precision than survives. attention_x3_k forms them on the bf16
// matrix cores (v_mfma_f32_32x32x16_bf16, 8 times the fp32 rate per
// instruction) with each fp32 operand split into bf16 parts, x = hi + lo
// (hi = bf16(x), lo = bf16(x - hi)), and a . b = lo_a hi_b + hi_a lo_b +
// hi_a hi_b accumulated in fp32: about 2^-16 of each product is dropped,
// three orders below the output's rounding. Head dim 64, the
// relative-position bias from the dot table, 4 waves of 32 query rows. The
// key and value tiles come split from the dot-table launch (x3_split_tiles):
// K rows as hi and lo bf16 rows, V transposed (a dimension's 32 keys
// contiguous, so one 16-byte read gives a lane its 8 keys) and its key
// order permuted so that the
// probabilities' registers feed the values' product without movement: the
// scores' register r of lane half h holds key 8 (r / 4) + 4 h + r % 4, and
// the product's k index 16 j + 8 h + t reads register 8 j + t, key
// 16 j + 8 (t / 4) + 4 h + t % 4 (bits 2 and 3 of the key swapped). The
// scores are kept in log2 units (the queries times scale log2(e) before the
// split, the dot table formed times log2(e)), and the online softmax moves
// a row's reference point only when a tile passes it by more than
// kX3Slack, so that most tiles rescale nothing.
constexpr int kX3KStride = 64 + 8;        // K rows in bf16: 144 bytes, 16 lanes' reads on 16 bank groups
constexpr int kX3VStride = kKeyTile + 8;  // V^T rows: 80 bytes, likewise

constexpr float kX3Slack = 8.0f;           // log2 of the largest probability before a rescale

// The maximum and the sum of lane l's and lane l ^ 32's values, in both
// lanes (v_permlane32_swap: r[0] holds the low half's values in both halves,
// r[1] the high half's).
__device__ __forceinline__ float max_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_halves(float v) {
  const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

__device__ __forceinline__ int x3_key_slot(int key) {  // bits 2 and 3 swapped (an involution)
  return (key & ~12) | ((key & 4) << 1) | ((key & 8) >> 1);
}

// The hi and lo bf16 parts of two floats, each pair packed (x0 low).
__device__ __forceinline__ void split2(float x0, float x1, uint32_t* hi, uint32_t* lo) {
  *hi = pack_bf16(x0, x1);
  *lo = pack_bf16(x0 - bf16_lo(*hi), x1 - bf16_hi(*hi));
}

// Eight floats' parts as 8 bf16 each (a matrix-core operand).
__device__ __forceinline__ void split8(const float (&x)[8], u32x4& hi, u32x4& lo) {
  uint32_t h[4], l[4];
#pragma unroll
  for (int i = 0; i < 4; ++i) split2(x[2 * i], x[2 * i + 1], &h[i], &l[i]);
  hi = u32x4{h[0], h[1], h[2], h[3]};
  lo = u32x4{l[0], l[1], l[2], l[3]};
}

// A tile's fp32 K and V rows (32 slots, 16-byte chunks spread over 256
// threads) split into LDS: K rows as hi and lo bf16 rows, V^T rows in the
// permuted slot order.
__device__ __forceinline__ void store_tile_x3(uint16_t* khi, uint16_t* klo, uint16_t* vhi, uint16_t* vlo,
                                              const float4 (&kr)[Tile<64, 256>::kPerThread],
                                              const float4 (&vr)[Tile<64, 256>::kPerThread]) {
#pragma unroll
  for (int j = 0; j < Tile<64, 256>::kPerThread; ++j) {
    const int idx = static_cast<int>(threadIdx.x) + 256 * j;
    const int row = idx / 16, c4 = idx % 16;
    uint32_t h[2], l[2];
    split2(kr[j].x, kr[j].y, &h[0], &l[0]);
    split2(kr[j].z, kr[j].w, &h[1], &l[1]);
    *reinterpret_cast<u32x2*>(khi + row * kX3KStride + 4 * c4) = u32x2{h[0], h[1]};
    *reinterpret_cast<u32x2*>(klo + row * kX3KStride + 4 * c4) = u32x2{l[0], l[1]};
    split2(vr[j].x, vr[j].y, &h[0], &l[0]);
    split2(vr[j].z, vr[j].w, &h[1], &l[1]);
    const int slot = x3_key_slot(row);
    const uint16_t hv[4] = {static_cast<uint16_t>(h[0]), static_cast<uint16_t>(h[0] >> 16),
                            static_cast<uint16_t>(h[1]), static_cast<uint16_t>(h[1] >> 16)};
    const uint16_t lv[4] = {static_cast<uint16_t>(l[0]), static_cast<uint16_t>(l[0] >> 16),
                            static_cast<uint16_t>(l[1]), static_cast<uint16_t>(l[1] >> 16)};
#pragma unroll
    for (int e = 0; e < 4; ++e) {
      vhi[(4 * c4 + e) * kX3VStride + slot] = hv[e];
      vlo[(4 * c4 + e) * kX3VStride + slot] = lv[e];
    }
  }
}

// ---- key and value tiles in bf16 parts, formed once per slice ---------------
//
// On a grid of whole tiles (SAM's global layers) the split-operand kernel
// reads each key tile once per workgroup of query rows (32 of them per head
// at 4096 rows); splitting its fp32 K and V rows there cost every workgroup
// the same VALU work. The dot-table launch forms them once instead, per
// tile 4 parts of 2048 bf16 (16 KB, the fp32 rows' size): K hi and lo
// [32 slots][64], V^T hi and lo [64 dims][32 slots] in the permuted slot
// order (x3_key_slot), unpadded; the attention copies them into its padded
// LDS rows with 16-byte writes (measured: 333 to 290 us for 12 heads of
// 4096 rows, table launch included). A window's tile is read by two or
// three workgroups, where the extra pass cost more than it saved (51 to 58
// us over 25 windows of 196): windows split their tiles in the attention.
constexpr int kX3PartElems = kKeyTile * 64;       // one part of one tile
constexpr int kX3TileFloats = 4 * kX3PartElems / 2;  // a tile's four parts, in floats

// Key tiles of a slice, and the key of a tile's slot (a dead slot: the
// nearest key, whose score the attention sets to -inf).
__device__ __forceinline__ int x3_tiles(const AttnArgs& a) {
  return a.x3_rows == 0 ? a.keys / kKeyTile : (a.h + a.x3_rows - 1) / a.x3_rows;
}
__device__ __forceinline__ int x3_key(const AttnArgs& a, int t, int slot) {
  if (a.x3_rows == 0) return t * kKeyTile + slot;
  const int per_row = kKeyTile / a.x3_rows;
  return min(t * a.x3_rows + slot / per_row, a.h - 1) * a.w + min(slot % per_row, a.w - 1);
}

// Tiles first, first + stride, ... of `slice` into a.kvx; 16-byte chunks
// spread over the block's threads.
__device__ void x3_split_tiles(const AttnArgs& a, int64_t slice, int first, int stride) {
  const float* kb = a.k + slice_at(a, slice, a.sk, a.ik);
  const float* vb = a.v + slice_at(a, slice, a.sv, a.iv);
  const int tiles = x3_tiles(a);
  for (int t = first; t < tiles; t += stride) {
    uint16_t* base = a.kvx + (slice * tiles + t) * static_cast<int64_t>(4 * kX3PartElems);
    for (int c = static_cast<int>(threadIdx.x); c < kX3PartElems / 8; c += static_cast<int>(blockDim.x)) {
      // K: slot c / 8, dims 8 (c % 8) .. + 7
      const int slot = c / 8, d0 = 8 * (c % 8);
      const float* kr = kb + static_cast<int64_t>(x3_key(a, t, slot)) * a.ldk + d0;
      const float4 k0 = *reinterpret_cast<const float4*>(kr), k1 = *reinterpret_cast<const float4*>(kr + 4);
      const float kx[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
      u32x4 hi, lo;
      split8(kx, hi, lo);
      *reinterpret_cast<u32x4*>(base + slot * 64 + d0) = hi;
      *reinterpret_cast<u32x4*>(base + kX3PartElems + slot * 64 + d0) = lo;
      // V^T: dim c / 4, slot positions 8 (c % 4) .. + 7
      const int dim = c / 4, p0 = 8 * (c % 4);
      float vx[8];
#pragma unroll
      for (int e = 0; e < 8; ++e) {
        vx[e] = vb[static_cast<int64_t>(x3_key(a, t, x3_key_slot(p0 + e))) * a.ldv + dim];
      }
      split8(vx, hi, lo);
      *reinterpret_cast<u32x4*>(base + 2 * kX3PartElems + dim * kKeyTile + p0) = hi;
      *reinterpret_cast<u32x4*>(base + 3 * kX3PartElems + dim * kKeyTile + p0) = lo;
    }
  }
}

// kRows 0: a grid of whole tiles, each key tile 32 keys of one grid row
// (the global layers); kRows 1, 2 or 4: each key tile kRows grid rows of at
// most 32 / kRows keys (the windows: 14 x 14 takes 2 rows of 14 per tile),
// a row's keys in the 32 / kRows slots from slot row * 32 / kRows, the
// slots past the row's width dead. Register r of lane half h holds slot
// 8 (r / 4) + 4 h + r % 4, which lies in row (r / 4) kRows / 4 of the tile
// whatever h: the height term is a register chosen at compile time, the
// width terms (dead slots -inf) the same in every tile.
template <int kRows>
__global__ __launch_bounds__(256) void attention_x3_k(const AttnArgs a) {
  constexpr int HD = 64, kQueriesPerBlock = 4 * kQueriesPerWave;
  constexpr int kSlotsPerRow = kKeyTile / (kRows == 0 ? 1 : kRows);
  constexpr int kDh = kRows == 0 ? 1 : kRows;  // height terms per tile
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  // two stages: tile t + 1 is written into one while tile t is read from the other
  constexpr int kKElems = kKeyTile * kX3KStride, kVElems = HD * kX3VStride;
  __shared__ __attribute__((aligned(16))) uint16_t khi_s[2 * kKElems];
  __shared__ __attribute__((aligned(16))) uint16_t klo_s[2 * kKElems];
  __shared__ __attribute__((aligned(16))) uint16_t vhi_s[2 * kVElems];
  __shared__ __attribute__((aligned(16))) uint16_t vlo_s[2 * kVElems];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, c = lane & 31;
  const int64_t slice = blockIdx.y;
  const int q0 = blockIdx.x * kQueriesPerBlock + wave * kQueriesPerWave;
  const int qrow = q0 + c;
  const bool qin = qrow < a.rows;
  const float* qb = a.q + slice_at(a, slice, a.sq, a.iq);
  auto mfma = [](u32x4 x, u32x4 y, f32x16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x), __builtin_bit_cast(bf16x8, y),
                                                   acc, 0, 0, 0);
  };
  const int tiles = x3_tiles(a);

  // kRows 0: this thread's 16-byte chunk of each of a tile's four parts
  // (formed by the dot-table launch): K slot tid / 8, dims 8 (tid % 8) ..
  // + 7; V^T dim tid / 4, slot positions 8 (tid % 4) .. + 7. Otherwise its
  // two 16-byte chunks of the fp32 K and V rows, split as they reach LDS: a
  // slot's key is its tile row's grid row (the last grid row past the last)
  // and its column (the last column for a dead slot; its score is -inf, its
  // probability 0). Every address in range and no branch, so that a tile's
  // use waits only for its own loads.
  const int tid = static_cast<int>(threadIdx.x);
  const int kslot = tid / 8, kd0 = 8 * (tid % 8), vdim = tid / 4, vp0 = 8 * (tid % 4);
  const uint16_t* kvs = a.kvx + slice * tiles * static_cast<int64_t>(4 * kX3PartElems);
  const float* kb = a.k + slice_at(a, slice, a.sk, a.ik);
  const float* vb = a.v + slice_at(a, slice, a.sv, a.iv);
  u32x4 kv[4];
  float4 kr[2], vr[2];
  int srow[2], scol[2], sc4[2];
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int idx = tid + 256 * j;
    const int slot = idx / (HD / 4), c4 = idx % (HD / 4);
    srow[j] = slot / kSlotsPerRow;
    scol[j] = min(slot % kSlotsPerRow, a.w - 1);
    sc4[j] = 4 * c4;
  }
  auto load_kv = [&](int t) {
    if constexpr (kRows == 0) {
      const uint16_t* base = kvs + static_cast<int64_t>(t) * (4 * kX3PartElems);
      kv[0] = *reinterpret_cast<const u32x4*>(base + kslot * 64 + kd0);
      kv[1] = *reinterpret_cast<const u32x4*>(base + kX3PartElems + kslot * 64 + kd0);
      kv[2] = *reinterpret_cast<const u32x4*>(base + 2 * kX3PartElems + vdim * kKeyTile + vp0);
      kv[3] = *reinterpret_cast<const u32x4*>(base + 3 * kX3PartElems + vdim * kKeyTile + vp0);
    } else {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const int key = min(t * kRows + srow[j], a.h - 1) * a.w + scol[j];
        kr[j] = *reinterpret_cast<const float4*>(kb + key * a.ldk + sc4[j]);
        vr[j] = *reinterpret_cast<const float4*>(vb + key * a.ldv + sc4[j]);
      }
    }
  };
  // the tile into LDS stage `stage`, K rows and V^T rows padded
  auto store_kv = [&](int stage) {
    uint16_t* khi = khi_s + stage * kKElems;
    uint16_t* klo = klo_s + stage * kKElems;
    uint16_t* vhi = vhi_s + stage * kVElems;
    uint16_t* vlo = vlo_s + stage * kVElems;
    if constexpr (kRows == 0) {
      *reinterpret_cast<u32x4*>(khi + kslot * kX3KStride + kd0) = kv[0];
      *reinterpret_cast<u32x4*>(klo + kslot * kX3KStride + kd0) = kv[1];
      *reinterpret_cast<u32x4*>(vhi + vdim * kX3VStride + vp0) = kv[2];
      *reinterpret_cast<u32x4*>(vlo + vdim * kX3VStride + vp0) = kv[3];
    } else {
      store_tile_x3(khi, klo, vhi, vlo, kr, vr);
    }
  };
  load_kv(0);

  // this lane's query columns 16 b + 8 h + (0..7), b < 4, times the scale
  // and log2(e) (the scores in log2 units, for exp2), split
  const float qmul = a.scale * kLog2e;
  u32x4 qh[4], ql[4];
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    float4 t0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), t1 = t0;
    if (qin) {
      const float* qr = qb + qrow * a.ldq + 16 * b + 8 * hl;
      t0 = *reinterpret_cast<const float4*>(qr);
      t1 = *reinterpret_cast<const float4*>(qr + 4);
    }
    const float x[8] = {t0.x * qmul, t0.y * qmul, t0.z * qmul, t0.w * qmul,
                        t1.x * qmul, t1.y * qmul, t1.z * qmul, t1.w * qmul};
    split8(x, qh[b], ql[b]);
  }

  store_kv(0);
  load_kv(tiles > 1 ? 1 : 0);  // tile 1 (tile 0 again when there is no tile 1)
  __syncthreads();

  f32x16 o[2];
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[b][r] = 0.0f;
  }
  // m: the row's reference point in log2 units, the running maximum or at
  // most kX3Slack below it, so that a probability is at most 2^kX3Slack
  // (exact enough in fp32 and in its bf16 parts; the output divides by a
  // total over the same reference). It moves, and the sums are rescaled,
  // only when a tile's maximum passes it by more than that. lh: the total
  // of this lane half's probabilities (the halves added at the end).
  float m = -INFINITY, lh = 0.0f;
  const bool live = q0 < a.rows;
  const float* trow = a.table + (slice * a.rows + (qin ? qrow : 0)) * static_cast<int64_t>(a.dots_ld);
  // The bias terms, in log2 units (the table was formed times log2(e)).
  // kRows 0: a tile's height term and the lane's 16 width terms (keys
  // kx0 + 8 g + 4 h + (0..3)). Otherwise the width terms of the lane's
  // slots, once, and a tile's kRows height terms (-inf past the grid).
  float dwc[16];
  if constexpr (kRows != 0) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int col = (8 * (r / 4) + 4 * hl + r % 4) % kSlotsPerRow;
      const float t = trow[a.dw_off + min(col, a.w - 1)];
      dwc[r] = col < a.w ? t : -INFINITY;
    }
  }
  struct Bias {
    float dh[kDh];
    float dw[kRows == 0 ? 16 : 1];
  };
  auto load_bias = [&](int t, Bias& bias) {
    if constexpr (kRows == 0) {
      const int key0 = t * kKeyTile, ky0 = key0 / a.w, kx0 = key0 - ky0 * a.w;
      bias.dh[0] = trow[ky0];
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const float4 tw = *reinterpret_cast<const float4*>(trow + a.dw_off + kx0 + 8 * g + 4 * hl);
        bias.dw[4 * g] = tw.x;
        bias.dw[4 * g + 1] = tw.y;
        bias.dw[4 * g + 2] = tw.z;
        bias.dw[4 * g + 3] = tw.w;
      }
    } else {
#pragma unroll
      for (int i = 0; i < kRows; ++i) {
        const int row = t * kRows + i;
        const float d = trow[min(row, a.h - 1)];
        bias.dh[i] = row < a.h ? d : -INFINITY;
      }
    }
  };
  // One key tile, read from LDS stage `stage`, its bias terms in `bias`.
  // First tile t + 1 (in kv since tile t - 1) is written into the other
  // stage and tile t + 2 requested; the next tile's bias terms are requested
  // into `next` (two register sets used in turn: no copies). One barrier
  // per tile: after it, stage t + 1 is whole and no wave still reads stage
  // t, which tile t + 1 then refills with tile t + 2.
  auto tile = [&](int t, int stage, const Bias& bias, Bias& next) {
    const bool more = t + 1 < tiles;
    if (more) store_kv(1 - stage);
    load_kv(t + 2 < tiles ? t + 2 : t);  // the current tile again past the end
    load_bias(more ? t + 1 : t, next);
    const uint16_t* khi = khi_s + stage * kKElems;
    const uint16_t* klo = klo_s + stage * kKElems;
    const uint16_t* vhi = vhi_s + stage * kVElems;
    const uint16_t* vlo = vlo_s + stage * kVElems;
    if (live) {
      // every K operand of the tile read from LDS before the first product,
      // then the V operands before the softmax (their latency behind it)
      u32x4 kh[4], kl[4], vh[2][2], vl[2][2];
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const int at = c * kX3KStride + 16 * b + 8 * hl;
        kh[b] = *reinterpret_cast<const u32x4*>(khi + at);
        kl[b] = *reinterpret_cast<const u32x4*>(klo + at);
      }
      __builtin_amdgcn_sched_barrier(0);  // the reads stay ahead of the products
      // S^T = K Q^T: 32 keys x 32 queries, the small products first
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = 0.0f;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        s = mfma(kl[b], qh[b], s);
        s = mfma(kh[b], ql[b], s);
        s = mfma(kh[b], qh[b], s);
      }
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int at = (32 * b + c) * kX3VStride + 16 * j + 8 * hl;
          vh[b][j] = *reinterpret_cast<const u32x4*>(vhi + at);
          vl[b][j] = *reinterpret_cast<const u32x4*>(vlo + at);
        }
      }
      // the bias terms, the tile's row maximum
      float tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if constexpr (kRows == 0) {
          s[r] = s[r] + (bias.dh[0] + bias.dw[r]);
        } else {
          s[r] = s[r] + (bias.dh[(r / 4) * kRows / 4] + dwc[r]);
        }
        tmax = fmaxf(tmax, s[r]);
      }
      tmax = max_halves(tmax);
      const bool grow = tmax > m + kX3Slack;
      if (__ballot(grow) != 0) {
        const float m_new = grow ? tmax : m;
        const float corr = grow ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
        lh *= corr;
#pragma unroll
        for (int b = 0; b < 2; ++b) {
#pragma unroll
          for (int r = 0; r < 16; ++r) o[b][r] *= corr;
        }
        m = m_new;
      }
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - m);
        lh += s[r];
      }
      // P split: product j takes registers 8 j .. 8 j + 7
      u32x4 ph[2], pl[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float x[8] = {s[8 * j],     s[8 * j + 1], s[8 * j + 2], s[8 * j + 3],
                            s[8 * j + 4], s[8 * j + 5], s[8 * j + 6], s[8 * j + 7]};
        split8(x, ph[j], pl[j]);
      }
      // O^T += V^T P^T over the permuted key slots
#pragma unroll
      for (int b = 0; b < 2; ++b) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          o[b] = mfma(vl[b][j], ph[j], o[b]);
          o[b] = mfma(vh[b][j], pl[j], o[b]);
          o[b] = mfma(vh[b][j], ph[j], o[b]);
        }
      }
    }
    __syncthreads();
  };
  Bias bias_a, bias_b;
  load_bias(0, bias_a);
  for (int t = 0; t < tiles; t += 2) {
    tile(t, 0, bias_a, bias_b);
    if (t + 1 < tiles) tile(t + 1, 1, bias_b, bias_a);
  }

  const float l = sum_halves(lh);
  if (!qin) return;
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
  const int64_t orow = slice_at(a, slice, a.so, a.io) + qrow * a.ldo;
#pragma unroll
  for (int b = 0; b < 2; ++b) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * b + 8 * g + 4 * hl;
      store4(a, orow + d, o[b][4 * g] * inv, o[b][4 * g + 1] * inv, o[b][4 * g + 2] * inv, o[b][4 * g + 3] * inv);
    }
  }
}

// ---- a mask on split operands --------------------------------------------------
//
// The decoder prefill's attention (a mask [rows, keys] shared by the heads,
// -inf where a key is not attended: past the query's position, and off the
// router's selected blocks and window) into bf16 on the bf16 matrix cores
// with split operands, as attention_x3_k does for SAM, for head dim 64 or
// 128. A first launch (mask_tiles_k) sets a bit per (128 query rows, 32-key
// tile) where some entry of that mask block is finite; a workgroup then walks
// only its live tiles, staging each (the fp32 K and V rows split into hi and
// lo parts as they reach LDS, V transposed and permuted as in
// attention_x3_k) and reading its rows' 32 x 32 mask block one tile ahead;
// a wave whose block is all -inf skips the tile's products. Workgroups go
// out last row block first (under a causal mask the longest walks first).
constexpr int kMaskRowBlock = 4 * kQueriesPerWave;  // query rows per workgroup
constexpr int kMaskMapKeys = 32 * kKeyTile;         // keys per map word (a bit per tile)

// Map byte (row block blockIdx.y, byte blockIdx.x of the row block's words):
// bit j set where some entry of rows [128 rb, 128 rb + 128) x keys of tile
// 8 blockIdx.x + j is not -inf (NaN counts as live; tiles past the keys
// clear). Wave w: rows 32 w .. 32 w + 31 of the block; lane: keys 4 lane ..
// 4 lane + 3 of the byte's 256; the four waves' votes OR'ed in LDS.
__global__ __launch_bounds__(256) void mask_tiles_k(const float* __restrict__ mask, int64_t mask_ld, int rows,
                                                    int keys, uint32_t* __restrict__ map, int words) {
  __shared__ uint32_t part[4];
  const int rb = blockIdx.y, byte = blockIdx.x;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int key4 = 8 * kKeyTile * byte + 4 * lane;
  const bool vec = mask_vec(mask, mask_ld);
  bool any = false;
  if (key4 < keys) {
    const int r0 = rb * kMaskRowBlock + wave * kQueriesPerWave;
    const int r1 = min(r0 + kQueriesPerWave, rows);
#pragma unroll 8
    for (int r = r0; r < r1; ++r) {
      const float4 m = mask4(mask + r * mask_ld, key4, keys, vec);
      any = any || m.x != -INFINITY || m.y != -INFINITY || m.z != -INFINITY || m.w != -INFINITY;
    }
  }
  // lanes 8 j .. 8 j + 7: tile j of the byte
  const uint64_t b = __ballot(any);
  uint32_t bits = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) bits |= ((b >> (8 * j)) & 0xffu) != 0 ? (1u << j) : 0u;
  if (lane == 0) part[wave] = bits;
  __syncthreads();
  if (threadIdx.x == 0) {
    reinterpret_cast<uint8_t*>(map + static_cast<int64_t>(rb) * words)[byte] =
        static_cast<uint8_t>(part[0] | part[1] | part[2] | part[3]);
  }
}

// Key tile t of slice s (blockIdx (t, s)) split once for every workgroup
// that reads it, 4 parts of 32 x HD bf16 (8 HD bytes per key): K hi and lo
// [32 slots][HD], V^T hi and lo [HD][32 slots] in the permuted slot order
// (x3_key_slot); a slot past the last key holds the last key (its mask
// entry is -inf). 16-byte chunks spread over the block's threads.
template <int HD>
__global__ __launch_bounds__(256) void x3m_split_k(const AttnArgs a, int tiles) {
  constexpr int kPart = kKeyTile * HD;
  const int t = blockIdx.x;
  const int64_t slice = blockIdx.y;
  const float* kb = a.k + slice_at(a, slice, a.sk, a.ik);
  const float* vb = a.v + slice_at(a, slice, a.sv, a.iv);
  uint16_t* base = a.kvx + (slice * tiles + t) * static_cast<int64_t>(4 * kPart);
  for (int c = static_cast<int>(threadIdx.x); c < kPart / 8; c += 256) {
    // K: slot c / (HD / 8), dims 8 (c % (HD / 8)) .. + 7
    const int slot = c / (HD / 8), d0 = 8 * (c % (HD / 8));
    const float* kr = kb + static_cast<int64_t>(min(t * kKeyTile + slot, a.keys - 1)) * a.ldk + d0;
    const float4 k0 = *reinterpret_cast<const float4*>(kr), k1 = *reinterpret_cast<const float4*>(kr + 4);
    const float kx[8] = {k0.x, k0.y, k0.z, k0.w, k1.x, k1.y, k1.z, k1.w};
    u32x4 hi, lo;
    split8(kx, hi, lo);
    *reinterpret_cast<u32x4*>(base + slot * HD + d0) = hi;
    *reinterpret_cast<u32x4*>(base + kPart + slot * HD + d0) = lo;
    // V^T: dim c / 4, slot positions 8 (c % 4) .. + 7
    const int dim = c / 4, p0 = 8 * (c % 4);
    float vx[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const int key = min(t * kKeyTile + x3_key_slot(p0 + e), a.keys - 1);
      vx[e] = vb[static_cast<int64_t>(key) * a.ldv + dim];
    }
    split8(vx, hi, lo);
    *reinterpret_cast<u32x4*>(base + 2 * kPart + dim * kKeyTile + p0) = hi;
    *reinterpret_cast<u32x4*>(base + 3 * kPart + dim * kKeyTile + p0) = lo;
  }
}

// Where a row block's live tiles are many, workgroup (row block, j) walks
// the j-th run of `chunk` of them and leaves per row the partial record
// (m, l, unnormalised O: X3Partials) that x3m_merge_k combines; a row block
// with one run writes its output itself.
struct X3Partials {
  int chunk;     // live tiles per workgroup
  int chunks;    // runs per row block (workgroups per row block and slice)
  float* o;      // [slices][row blocks][chunks][128 rows][hd]
  float* ml;     // [slices][row blocks][chunks][128 rows][2]: m, l
};

template <int HD>
__global__ __launch_bounds__(256) void attention_x3m_k(const AttnArgs a, const uint32_t* __restrict__ map, int words,
                                                       int row_blocks, int slices, X3Partials part) {
  constexpr int kNB = HD / 16;           // 16-column blocks of a query or key row
  constexpr int kDB = HD / 32;           // 32-dimension blocks of the output
  constexpr int kKS = HD + 8;            // K rows in bf16: an odd number of 16-byte groups apart
  constexpr int kVS = kX3VStride;        // V^T rows
  constexpr int kKElems = kKeyTile * kKS, kVElems = HD * kVS;
  constexpr int kPer = kKeyTile * HD / 8 / 256;  // 16-byte chunks of one split part per thread: 1 or 2
  typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
  __shared__ __attribute__((aligned(16))) uint16_t khi_s[2 * kKElems];
  __shared__ __attribute__((aligned(16))) uint16_t klo_s[2 * kKElems];
  __shared__ __attribute__((aligned(16))) uint16_t vhi_s[2 * kVElems];
  __shared__ __attribute__((aligned(16))) uint16_t vlo_s[2 * kVElems];

  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, c = lane & 31;
  const int tid = static_cast<int>(threadIdx.x);
  // workgroup: (row block, run, slice), every slice's last row block first
  const int run = static_cast<int>(blockIdx.x) / slices % part.chunks;
  const int rb = row_blocks - 1 - static_cast<int>(blockIdx.x) / slices / part.chunks;
  const int64_t slice = static_cast<int>(blockIdx.x) % slices;
  const int q0 = rb * kMaskRowBlock + wave * kQueriesPerWave;
  const int qrow = q0 + c;
  const bool qin = qrow < a.rows;
  const float* qb = a.q + slice_at(a, slice, a.sq, a.iq);
  const int64_t orow = slice_at(a, slice, a.so, a.io) + static_cast<int64_t>(qrow) * a.ldo;
  auto mfma = [](u32x4 x, u32x4 y, f32x16 acc) {
    return __builtin_amdgcn_mfma_f32_32x32x16_bf16(__builtin_bit_cast(bf16x8, x), __builtin_bit_cast(bf16x8, y),
                                                   acc, 0, 0, 0);
  };

  // the live tiles of this row block, in order (uniform: scalar reads)
  const uint32_t* tmap = map + static_cast<int64_t>(rb) * words;
  const int tiles = (a.keys + kKeyTile - 1) / kKeyTile;
  MapCursor cursor{tmap, -1, 0u};
  auto next_live = [&](int t) { return next_live_tile(cursor, tiles, t); };  // the first live tile after t, or tiles
  const int live = live_tiles(tmap, words);
  const int runs = (live + part.chunk - 1) / part.chunk;
  if (live == 0) {  // no key attended by any row of the block: zeros
    if (run == 0 && qin) {
#pragma unroll
      for (int e = 0; e < HD / 8; ++e) store4(a, orow + 8 * e + 4 * hl, 0.0f, 0.0f, 0.0f, 0.0f);
    }
    return;
  }
  if (run >= runs) return;  // uniform over the workgroup, before any barrier
  // the first live tile of this run: skip run * chunk of them
  int t = -1;
  for (int skip = run * part.chunk; skip >= 0; --skip) t = next_live(t);
  // the run's live tiles i = 0 .. chunk - 1 (past the run: tiles)
  auto after = [&](int tt, int i) { return i + 1 < part.chunk && tt < tiles ? next_live(tt) : tiles; };

  // this thread's 16-byte chunks of each of a tile's four split parts
  // (formed by x3m_split_k), copied into the padded LDS rows
  constexpr int kPart = kKeyTile * HD;
  const uint16_t* kvs = a.kvx + slice * tiles * static_cast<int64_t>(4 * kPart);
  u32x4 kv[4][kPer];
  auto load_kv = [&](int tt) {
    const uint16_t* base = kvs + static_cast<int64_t>(tt) * (4 * kPart);
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int c = tid + 256 * j;
#pragma unroll
      for (int part = 0; part < 4; ++part) {
        kv[part][j] = *reinterpret_cast<const u32x4*>(base + part * kPart + 8 * c);
      }
    }
  };
  // into LDS stage `stage`: K rows [32][HD] and V^T rows [HD][32], padded
  auto store_kv = [&](int stage) {
#pragma unroll
    for (int j = 0; j < kPer; ++j) {
      const int c = tid + 256 * j;
      const int slot = c / (HD / 8), d0 = 8 * (c % (HD / 8)), dim = c / 4, p0 = 8 * (c % 4);
      *reinterpret_cast<u32x4*>(khi_s + stage * kKElems + slot * kKS + d0) = kv[0][j];
      *reinterpret_cast<u32x4*>(klo_s + stage * kKElems + slot * kKS + d0) = kv[1][j];
      *reinterpret_cast<u32x4*>(vhi_s + stage * kVElems + dim * kVS + p0) = kv[2][j];
      *reinterpret_cast<u32x4*>(vlo_s + stage * kVElems + dim * kVS + p0) = kv[3][j];
    }
  };
  // this lane's 16 mask entries of a tile (register r: key 8 (r / 4) + 4 h +
  // r % 4 of the tile), -inf past the keys or the rows
  struct Block {
    float m[16];
  };
  const bool vec = mask_vec(a.mask, a.mask_ld);
  const float* mrow = a.mask + static_cast<int64_t>(qin ? qrow : 0) * a.mask_ld;
  auto load_mask = [&](int tt, Block& blk) {
    const bool whole = vec && (tt + 1) * kKeyTile <= a.keys;  // uniform: every key of the tile exists
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int key4 = tt * kKeyTile + 8 * g + 4 * hl;
      float4 v = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
      if (whole) {
        if (qin) v = *reinterpret_cast<const float4*>(mrow + key4);
      } else if (qin && key4 < a.keys) {
        v = mask4(mrow, key4, a.keys, vec);
      }
      blk.m[4 * g] = v.x;
      blk.m[4 * g + 1] = v.y;
      blk.m[4 * g + 2] = v.z;
      blk.m[4 * g + 3] = v.w;
    }
  };

  load_kv(t);
  // the lane's query columns 16 b + 8 h + (0..7) times scale log2(e), split
  const float qmul = a.scale * kLog2e;
  u32x4 qh[kNB], ql[kNB];
#pragma unroll
  for (int b = 0; b < kNB; ++b) {
    float4 t0 = make_float4(0.0f, 0.0f, 0.0f, 0.0f), t1 = t0;
    if (qin) {
      const float* qr = qb + static_cast<int64_t>(qrow) * a.ldq + 16 * b + 8 * hl;
      t0 = *reinterpret_cast<const float4*>(qr);
      t1 = *reinterpret_cast<const float4*>(qr + 4);
    }
    const float x[8] = {t0.x * qmul, t0.y * qmul, t0.z * qmul, t0.w * qmul,
                        t1.x * qmul, t1.y * qmul, t1.z * qmul, t1.w * qmul};
    split8(x, qh[b], ql[b]);
  }
  Block blk_a, blk_b;
  load_mask(t, blk_a);
  store_kv(0);
  int i = 0;  // t's place in the run
  int n1 = after(t, i);
  load_kv(n1 < tiles ? n1 : t);
  __syncthreads();

  f32x16 o[kDB];
#pragma unroll
  for (int b = 0; b < kDB; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[b][r] = 0.0f;
  }
  // m: the row's reference point in log2 units, as in attention_x3_k (-inf
  // until a finite score is seen); lh: this lane half's total
  float m = -INFINITY, lh = 0.0f;
  const bool rows_live = q0 < a.rows;
  // Live tile t from LDS stage `stage`, its mask block in `cur`; the next
  // live tile n1 (in kr, vr) goes to the other stage, the one after (n2) is
  // requested, and n1's mask block into `next`. One barrier per tile.
  auto tile = [&](int tt, int nx1, int nx2, int stage, const Block& cur, Block& next) {
    if (nx1 < tiles) store_kv(1 - stage);
    load_kv(nx2 < tiles ? nx2 : tt);  // in range; not stored past the last tile
    load_mask(nx1 < tiles ? nx1 : tt, next);
    bool any = false;
#pragma unroll
    for (int r = 0; r < 16; ++r) any = any || cur.m[r] != -INFINITY;
    if (rows_live && __ballot(any) != 0) {
      const uint16_t* khi = khi_s + stage * kKElems;
      const uint16_t* klo = klo_s + stage * kKElems;
      const uint16_t* vhi = vhi_s + stage * kVElems;
      const uint16_t* vlo = vlo_s + stage * kVElems;
      // S^T = K Q^T + the mask in log2 units (32 keys x 32 queries): the
      // products accumulate onto the mask block, the small ones first
      f32x16 s;
#pragma unroll
      for (int r = 0; r < 16; ++r) s[r] = cur.m[r] * kLog2e;
#pragma unroll
      for (int b = 0; b < kNB; ++b) {
        const int at = c * kKS + 16 * b + 8 * hl;
        const u32x4 kh = *reinterpret_cast<const u32x4*>(khi + at);
        const u32x4 kl = *reinterpret_cast<const u32x4*>(klo + at);
        s = mfma(kl, qh[b], s);
        s = mfma(kh, ql[b], s);
        s = mfma(kh, qh[b], s);
      }
      // the tile's row maximum
      float tmax = -INFINITY;
#pragma unroll
      for (int r = 0; r < 16; ++r) tmax = fmaxf(tmax, s[r]);
      tmax = max_halves(tmax);
      const bool grow = tmax > m + kX3Slack;
      if (__ballot(grow) != 0) {
        const float m_new = grow ? tmax : m;
        const float corr = grow ? __builtin_amdgcn_exp2f(m - m_new) : 1.0f;
        lh *= corr;
#pragma unroll
        for (int b = 0; b < kDB; ++b) {
#pragma unroll
          for (int r = 0; r < 16; ++r) o[b][r] *= corr;
        }
        m = m_new;
      }
      // a row with no finite score yet: its probabilities are 0
      const float ref = m == -INFINITY ? INFINITY : m;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        s[r] = __builtin_amdgcn_exp2f(s[r] - ref);
        lh += s[r];
      }
      u32x4 ph[2], pl[2];
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        const float x[8] = {s[8 * j],     s[8 * j + 1], s[8 * j + 2], s[8 * j + 3],
                            s[8 * j + 4], s[8 * j + 5], s[8 * j + 6], s[8 * j + 7]};
        split8(x, ph[j], pl[j]);
      }
      // O^T += V^T P^T over the permuted key slots
#pragma unroll
      for (int b = 0; b < kDB; ++b) {
#pragma unroll
        for (int j = 0; j < 2; ++j) {
          const int at = (32 * b + c) * kVS + 16 * j + 8 * hl;
          const u32x4 vh = *reinterpret_cast<const u32x4*>(vhi + at);
          const u32x4 vl = *reinterpret_cast<const u32x4*>(vlo + at);
          o[b] = mfma(vl, ph[j], o[b]);
          o[b] = mfma(vh, pl[j], o[b]);
          o[b] = mfma(vh, ph[j], o[b]);
        }
      }
    }
    __syncthreads();
  };
  // two mask blocks used in turn (no copies): tiles alternate stages 0, 1
  while (true) {
    int n2 = after(n1, i + 1);
    tile(t, n1, n2, 0, blk_a, blk_b);
    t = n1;
    ++i;
    if (t >= tiles) break;
    n1 = n2;
    n2 = after(n1, i + 1);
    tile(t, n1, n2, 1, blk_b, blk_a);
    t = n1;
    ++i;
    if (t >= tiles) break;
    n1 = n2;
  }

  const float l = sum_halves(lh);
  if (!qin) return;
  if (runs > 1) {
    // the partial record: m and l (lane half 0), O unnormalised
    const int64_t rec = ((slice * row_blocks + rb) * part.chunks + run) * kMaskRowBlock + (qrow - rb * kMaskRowBlock);
    if (hl == 0) *reinterpret_cast<float2*>(part.ml + 2 * rec) = make_float2(m, l);
#pragma unroll
    for (int b = 0; b < kDB; ++b) {
#pragma unroll
      for (int g = 0; g < 4; ++g) {
        const int d = 32 * b + 8 * g + 4 * hl;
        *reinterpret_cast<float4*>(part.o + rec * HD + d) =
            make_float4(o[b][4 * g], o[b][4 * g + 1], o[b][4 * g + 2], o[b][4 * g + 3]);
      }
    }
    return;
  }
  const float inv = l > 0.0f ? 1.0f / l : 0.0f;
#pragma unroll
  for (int b = 0; b < kDB; ++b) {
#pragma unroll
    for (int g = 0; g < 4; ++g) {
      const int d = 32 * b + 8 * g + 4 * hl;
      store4(a, orow + d, o[b][4 * g] * inv, o[b][4 * g + 1] * inv, o[b][4 * g + 2] * inv, o[b][4 * g + 3] * inv);
    }
  }
}

// The rows of row blocks walked in several runs: out = sum_j 2^(u (m_j - M))
// O_j / sum_j 2^(u (m_j - M)) l_j with M the largest m_j and u the records'
// unit (1: m in log2 units; log2(e): natural units) (a run where the row saw
// no finite score holds m = -inf, l = 0, O = 0 and weighs 0; no finite
// score at all: zeros), into bf16. Workgroup (row block, slice); thread:
// row tid / 2, dimensions (tid % 2) hd / 2 .. + hd / 2 - 1.
template <int HD>
__global__ __launch_bounds__(256) void x3m_merge_k(const AttnArgs a, const uint32_t* __restrict__ map, int words,
                                                   int row_blocks, X3Partials part, float unit) {
  constexpr int kHalf = HD / 2;
  const int rb = blockIdx.x;
  const int64_t slice = blockIdx.y;
  const int live = live_tiles(map + static_cast<int64_t>(rb) * words, words);
  const int runs = (live + part.chunk - 1) / part.chunk;
  if (runs <= 1) return;
  const int r = static_cast<int>(threadIdx.x) / 2, d0 = kHalf * (static_cast<int>(threadIdx.x) % 2);
  const int qrow = rb * kMaskRowBlock + r;
  if (qrow >= a.rows) return;
  const int64_t rec0 = (slice * row_blocks + rb) * part.chunks * kMaskRowBlock + r;
  float big = -INFINITY;
  for (int j = 0; j < runs; ++j) big = fmaxf(big, part.ml[2 * (rec0 + j * kMaskRowBlock)]);
  const float ref = big == -INFINITY ? 0.0f : big;
  float acc[kHalf];
#pragma unroll
  for (int e = 0; e < kHalf; ++e) acc[e] = 0.0f;
  float total = 0.0f;
  for (int j = 0; j < runs; ++j) {
    const int64_t rec = rec0 + j * kMaskRowBlock;
    const float2 ml = *reinterpret_cast<const float2*>(part.ml + 2 * rec);
    const float wgt = __builtin_amdgcn_exp2f((ml.x - ref) * unit);  // 0 for m = -inf
    total += wgt * ml.y;
    const float* src = part.o + rec * HD + d0;
#pragma unroll
    for (int e = 0; e < kHalf; e += 4) {
      const float4 v = *reinterpret_cast<const float4*>(src + e);
      acc[e] += wgt * v.x;
      acc[e + 1] += wgt * v.y;
      acc[e + 2] += wgt * v.z;
      acc[e + 3] += wgt * v.w;
    }
  }
  const float inv = total > 0.0f ? 1.0f / total : 0.0f;
  const int64_t orow = slice_at(a, slice, a.so, a.io) + static_cast<int64_t>(qrow) * a.ldo + d0;
#pragma unroll
  for (int e = 0; e < kHalf; e += 4) store4(a, orow + e, acc[e] * inv, acc[e + 1] * inv, acc[e + 2] * inv, acc[e + 3] * inv);
}

// ---- few query rows: the keys split over the waves ---------------------------
//
// With few query rows (CLIP: 16 heads x 257 rows are 48 workgroups of 128
// rows for 256 CUs) one wave's walk over every key tile is the whole call's
// critical path. Here the 4 waves of a workgroup take the same 32 query rows
// and every fourth key tile each: its own K and V tiles, straight from
// memory into its own LDS region (two stages; K rows' 16-byte chunks
// swizzled by the row so that the S^T reads of 16 rows cover 16 bank
// groups), the same products and online softmax as attention_k, and at the
// end the four (max, total, values) records of each row are combined
// through LDS in wave order. No bias; head dim 64.
constexpr int kSplitWaves = 4;
constexpr int kSplitHd = 64;
constexpr int kSplitTileFloats = kKeyTile * kSplitHd;                     // one operand tile, unpadded
constexpr size_t kSplitLds = sizeof(float) * kSplitWaves * 2 * 2 * kSplitTileFloats;  // 128 KB

__global__ __launch_bounds__(64 * kSplitWaves) void attention_keysplit_k(const AttnArgs a) {
  constexpr int HD = kSplitHd, kHalf = HD / 2, kDBlocks = HD / 32;
  constexpr int kRowChunks = HD / 4;                                  // 16-byte chunks per K or V row
  constexpr int kLoads = kSplitTileFloats / 4 / kWave;                // memory-to-LDS loads per operand tile
  extern __shared__ __attribute__((aligned(16))) float lds[];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hl = lane >> 5, c = lane & 31;
  const int64_t slice = blockIdx.y;
  const int qrow = blockIdx.x * kQueriesPerWave + c;
  const bool qin = qrow < a.rows;
  const float* qb = a.q + slice_at(a, slice, a.sq, a.iq);
  const float* kb = a.k + slice_at(a, slice, a.sk, a.ik);
  const float* vb = a.v + slice_at(a, slice, a.sv, a.iv);
  float* const mine = lds + wave * 2 * 2 * kSplitTileFloats;  // [stage][K | V]
  const int tiles = (a.keys + kKeyTile - 1) / kKeyTile;

  // tile t into stage st: lane l of load i writes LDS chunk i * 64 + l
  auto stage_tile = [&](int t, int st) {
    float* ks = mine + st * 2 * kSplitTileFloats;
    float* vs = ks + kSplitTileFloats;
#pragma unroll
    for (int i = 0; i < kLoads; ++i) {
      const int sl = i * kWave + lane, row = sl / kRowChunks, cj = sl % kRowChunks;
      const int key = t * kKeyTile + row < a.keys ? t * kKeyTile + row : a.keys - 1;  // past the end: a valid row
      __builtin_amdgcn_global_load_lds(kb + static_cast<int64_t>(key) * a.ldk + 4 * (cj ^ (row & 15)),
                                       ks + i * kWave * 4, 16, 0, 0);
      __builtin_amdgcn_global_load_lds(vb + static_cast<int64_t>(key) * a.ldv + 4 * cj, vs + i * kWave * 4, 16, 0,
                                       0);
    }
  };

  float qv[kHalf];
#pragma unroll
  for (int i = 0; i < kHalf; i += 4) {
    float4 t = make_float4(0.0f, 0.0f, 0.0f, 0.0f);
    if (qin) t = *reinterpret_cast<const float4*>(qb + qrow * a.ldq + hl * kHalf + i);
    qv[i] = t.x;
    qv[i + 1] = t.y;
    qv[i + 2] = t.z;
    qv[i + 3] = t.w;
  }
  f32x16 o[kDBlocks];
#pragma unroll
  for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) o[b][r] = 0.0f;
  }
  float m = -INFINITY, l = 0.0f;
  if (wave < tiles) stage_tile(wave, 0);
  for (int t = wave, n = 0; t < tiles; t += kSplitWaves, ++n) {
    const int st = n & 1;
    const bool more = t + kSplitWaves < tiles;
    if (more) {
      __builtin_amdgcn_s_waitcnt(0xC07F);  // lgkmcnt(0): this wave's reads of the other stage are done
      stage_tile(t + kSplitWaves, st ^ 1);
      __builtin_amdgcn_s_waitcnt(((2 * kLoads) & 0xF) | ((((2 * kLoads) >> 4) & 3) << 14) | (7 << 4) | (0xF << 8));
    } else {
      __builtin_amdgcn_s_waitcnt((7 << 4) | (0xF << 8));  // vmcnt(0)
    }
    const float* ks = mine + st * 2 * kSplitTileFloats;
    const float* vs = ks + kSplitTileFloats;
    const int key0 = t * kKeyTile;
    f32x16 sacc;
#pragma unroll
    for (int r = 0; r < 16; ++r) sacc[r] = 0.0f;
#pragma unroll
    for (int i = 0; i < kHalf; i += 4) {
      const float4 kk = *reinterpret_cast<const float4*>(ks + c * HD + 4 * ((hl * (kHalf / 4) + i / 4) ^ (c & 15)));
      sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.x, qv[i], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.y, qv[i + 1], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.z, qv[i + 2], sacc, 0, 0, 0);
      sacc = __builtin_amdgcn_mfma_f32_32x32x2f32(kk.w, qv[i + 3], sacc, 0, 0, 0);
    }
    float tmax = -INFINITY;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int key = key0 + 8 * (r / 4) + 4 * hl + (r % 4);
      const float x = key < a.keys ? sacc[r] * a.scale : -INFINITY;
      sacc[r] = x;
      tmax = fmaxf(tmax, x);
    }
    tmax = fmaxf(tmax, partner(tmax));
    const float m_new = fmaxf(m, tmax);
    const bool dead = m_new == -INFINITY;
    const float corr = dead ? 1.0f : __builtin_amdgcn_exp2f((m - m_new) * kLog2e);
    float psum = 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      sacc[r] = dead ? 0.0f : __builtin_amdgcn_exp2f((sacc[r] - m_new) * kLog2e);
      psum += sacc[r];
    }
    psum += partner(psum);
    l = l * corr + psum;
    m = m_new;
    if (__ballot(corr != 1.0f) != 0) {
#pragma unroll
      for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
        for (int r = 0; r < 16; ++r) o[b][r] *= corr;
      }
    }
#pragma unroll
    for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
      for (int i = 0; i < 16; ++i) {
        const int key = 8 * (i / 4) + 4 * hl + (i % 4);
        o[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vs[key * HD + 32 * b + c], sacc[i], o[b], 0, 0, 0);
      }
    }
  }

  // the four records of each row through LDS: values [wave][row][HD], then
  // max and total [wave][row]
  __syncthreads();
  float* vals = lds;
  float* mx = lds + kSplitWaves * kQueriesPerWave * HD;
  float* tot = mx + kSplitWaves * kQueriesPerWave;
#pragma unroll
  for (int b = 0; b < kDBlocks; ++b) {
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      vals[(wave * kQueriesPerWave + c) * HD + 32 * b + 8 * (r / 4) + 4 * hl + (r % 4)] = o[b][r];
    }
  }
  if (hl == 0) {
    mx[wave * kQueriesPerWave + c] = m;
    tot[wave * kQueriesPerWave + c] = l;
  }
  __syncthreads();
  // thread: row threadIdx.x / 8, columns 8 (threadIdx.x % 8) .. + 7
  const int row = static_cast<int>(threadIdx.x) / 8, d0 = 8 * (static_cast<int>(threadIdx.x) % 8);
  const int orow = blockIdx.x * kQueriesPerWave + row;
  if (orow >= a.rows) return;
  float big = -INFINITY;
#pragma unroll
  for (int w = 0; w < kSplitWaves; ++w) big = fmaxf(big, mx[w * kQueriesPerWave + row]);
  float e[kSplitWaves], total = 0.0f;
#pragma unroll
  for (int w = 0; w < kSplitWaves; ++w) {
    const float mw = mx[w * kQueriesPerWave + row];
    e[w] = mw == -INFINITY ? 0.0f : __builtin_amdgcn_exp2f((mw - big) * kLog2e);
    total += e[w] * tot[w * kQueriesPerWave + row];
  }
  const float inv = total > 0.0f ? 1.0f / total : 0.0f;
  float acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
#pragma unroll
  for (int w = 0; w < kSplitWaves; ++w) {
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] += e[w] * vals[(w * kQueriesPerWave + row) * HD + d0 + j];
  }
  const int64_t op = slice_at(a, slice, a.so, a.io) + static_cast<int64_t>(orow) * a.ldo + d0;
  store4(a, op, acc[0] * inv, acc[1] * inv, acc[2] * inv, acc[3] * inv);
  store4(a, op + 4, acc[4] * inv, acc[5] * inv, acc[6] * inv, acc[7] * inv);
}

// The relative-position dot products of every (slice, query row) into
// table [slices][rows][dots_ld] (height terms at 0, width terms at dw_off),
// on the fp32 matrix cores: block (j, s) takes table slice j of slice s
// (rh[qy = j] for j < h, else rw[qx = j - h]) and the h or w query rows that
// use it, a product Q_j [queries, hd] . T_j^T [hd, table rows] in 32 x 32
// tiles, one tile per wave at a time. Lane l of a tile holds query row
// l % 32 and table row l % 32 (past the last: the last), columns
// 32 (l / 32) + (0..31) of each 64-column chunk straight from memory; step
// i of the chunk's 32 v_mfma_f32_32x32x2f32 takes columns i and 32 + i.
// Each table slice is read once per slice here, where a workgroup of the
// attention forming its own dots reads a width slice per query.
template <int HD>
__global__ __launch_bounds__(256) void rel_dots_k(const AttnArgs a) {
  const int j = static_cast<int>(blockIdx.x);
  const int64_t slice = blockIdx.y;
  if (HD == 64 && a.kvx != nullptr) x3_split_tiles(a, slice, j, static_cast<int>(gridDim.x));
  const bool height = j < a.h;
  const int nq = height ? a.w : a.h;  // the query rows that use this table slice
  const int nr = height ? a.h : a.w;  // its rows: dots per query
  const float* tab = height ? a.rh + static_cast<int64_t>(j) * a.h * HD : a.rw + static_cast<int64_t>(j - a.h) * a.w * HD;
  auto query = [&](int i) { return height ? j * a.w + i : i * a.w + (j - a.h); };
  const float* qb = a.q + slice_at(a, slice, a.sq, a.iq);
  float* out = a.table_out + slice * a.rows * static_cast<int64_t>(a.dots_ld);
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int hh = lane >> 5, l32 = lane & 31;
  const int tq = (nq + 31) / 32, tr = (nr + 31) / 32;
  const int waves = static_cast<int>(blockDim.x) / 64;
  for (int tile = wave; tile < tq * tr; tile += waves) {
    const int iq = tile / tr, ir = tile - iq * tr;
    const int qi = min(iq * 32 + l32, nq - 1), ti = min(ir * 32 + l32, nr - 1);
    const float* qrow = qb + static_cast<int64_t>(query(qi)) * a.ldq + 32 * hh;
    const float* trow = tab + static_cast<int64_t>(ti) * HD + 32 * hh;
    f32x16 acc;
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[r] = 0.0f;
#pragma unroll
    for (int k0 = 0; k0 < HD; k0 += 64) {
      float qv[32], tv[32];
#pragma unroll
      for (int i = 0; i < 32; i += 4) {
        const float4 x = *reinterpret_cast<const float4*>(qrow + k0 + i);
        const float4 y = *reinterpret_cast<const float4*>(trow + k0 + i);
        qv[i] = x.x;
        qv[i + 1] = x.y;
        qv[i + 2] = x.z;
        qv[i + 3] = x.w;
        tv[i] = y.x;
        tv[i + 1] = y.y;
        tv[i + 2] = y.z;
        tv[i + 3] = y.w;
      }
#pragma unroll
      for (int i = 0; i < 32; ++i) acc = __builtin_amdgcn_mfma_f32_32x32x2f32(qv[i], tv[i], acc, 0, 0, 0);
    }
    // D[query][table row]: register r of lane l holds query 8 (r / 4) +
    // 4 (l / 32) + r % 4 of the tile, table row l % 32
    const int t = ir * 32 + l32;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      const int q = iq * 32 + 8 * (r / 4) + 4 * hh + r % 4;
      if (q < nq && t < nr) {
        out[static_cast<int64_t>(query(q)) * a.dots_ld + (height ? t : a.dw_off + t)] = acc[r] * a.table_mul;
      }
    }
  }
}

// rel_dots_k for grids at most 16 by 16 (SAM's 14 x 14 windows): a table
// slice's product is one 16 x 16 tile of v_mfma_f32_16x16x4f32, a wave per
// table slice, four table slices per workgroup. Lane l holds query row and
// table row l % 16 (past the last: the last), columns 16 (l / 16) + (0..15)
// of each 64-column chunk; step i of the chunk takes columns i, 16 + i,
// 32 + i and 48 + i. Register r of lane l then holds query 4 (l / 16) + r,
// table row l % 16.
template <int HD>
__global__ __launch_bounds__(256) void rel_dots16_k(const AttnArgs a) {
  typedef float f32x4 __attribute__((ext_vector_type(4)));
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int64_t slice = blockIdx.y;
  const int j = static_cast<int>(blockIdx.x) * 4 + wave;
  if (j >= a.h + a.w) return;  // the whole wave (no barrier follows)
  const bool height = j < a.h;
  const int nq = height ? a.w : a.h;
  const int nr = height ? a.h : a.w;
  const float* tab = height ? a.rh + static_cast<int64_t>(j) * a.h * HD : a.rw + static_cast<int64_t>(j - a.h) * a.w * HD;
  auto query = [&](int i) { return height ? j * a.w + i : i * a.w + (j - a.h); };
  const float* qb = a.q + slice_at(a, slice, a.sq, a.iq);
  float* out = a.table_out + slice * a.rows * static_cast<int64_t>(a.dots_ld);
  const int g = lane >> 4, l16 = lane & 15;
  const float* qrow = qb + static_cast<int64_t>(query(min(l16, nq - 1))) * a.ldq + 16 * g;
  const float* trow = tab + static_cast<int64_t>(min(l16, nr - 1)) * HD + 16 * g;
  f32x4 acc = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
  for (int k0 = 0; k0 < HD; k0 += 64) {
    float qv[16], tv[16];
#pragma unroll
    for (int i = 0; i < 16; i += 4) {
      const float4 x = *reinterpret_cast<const float4*>(qrow + k0 + i);
      const float4 y = *reinterpret_cast<const float4*>(trow + k0 + i);
      qv[i] = x.x;
      qv[i + 1] = x.y;
      qv[i + 2] = x.z;
      qv[i + 3] = x.w;
      tv[i] = y.x;
      tv[i + 1] = y.y;
      tv[i + 2] = y.z;
      tv[i + 3] = y.w;
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) acc = __builtin_amdgcn_mfma_f32_16x16x4f32(qv[i], tv[i], acc, 0, 0, 0);
  }
#pragma unroll
  for (int r = 0; r < 4; ++r) {
    const int q = 4 * g + r;
    if (q < nq && l16 < nr) {
      out[static_cast<int64_t>(query(q)) * a.dots_ld + (height ? l16 : a.dw_off + l16)] = acc[r] * a.table_mul;
    }
  }
}

// Dynamic LDS above 64 KB has to be allowed per kernel first.
template <class Kernel>
void allow_lds(Kernel kernel, size_t bytes) {
  if (bytes > 65536) {
    (void)hipFuncSetAttribute(reinterpret_cast<const void*>(kernel), hipFuncAttributeMaxDynamicSharedMemorySize,
                              static_cast<int>(bytes));
  }
}

template <Bias kBias>
int launch(const char* what, void* stream, int64_t hd, int64_t slices, const AttnArgs& a) {
  constexpr int kThreads = 64 * waves_of<kBias>(), kQueriesPerBlock = waves_of<kBias>() * kQueriesPerWave;
  const dim3 grid(static_cast<unsigned>((a.rows + kQueriesPerBlock - 1) / kQueriesPerBlock),
                  static_cast<unsigned>(slices));
  const size_t dyn = dots_in_lds<kBias>() ? sizeof(float) * kQueriesPerBlock * static_cast<size_t>(a.dots_ld) : 0;
  clear_launch_error();
  if (hd == 64) {
    allow_lds(attention_k<64, kBias>, dyn);
    attention_k<64, kBias><<<grid, kThreads, dyn, as_stream(stream)>>>(a);
  } else {
    allow_lds(attention_k<128, kBias>, dyn);
    attention_k<128, kBias><<<grid, kThreads, dyn, as_stream(stream)>>>(a);
  }
  return check_launch(what);
}

int check_common(const char* what, const float* q, int64_t ldq, int64_t sq, const float* k, int64_t ldk, int64_t sk,
                 const float* v, int64_t ldv, int64_t sv, const float* out, int64_t ldo, int64_t so, int64_t slices,
                 int64_t rows, int64_t keys, int64_t hd) {
  UOCR_REQUIRE(hd == 64 || hd == 128, what, "head dim must be 64 or 128");
  UOCR_REQUIRE(slices >= 1 && slices < 65536 && rows >= 1 && rows < (int64_t{1} << 31) && keys >= 1 &&
                   keys < (int64_t{1} << 31),
               what, "need 1 <= slices < 65536 and rows, keys in [1, 2^31)");
  UOCR_REQUIRE(q != nullptr && k != nullptr && v != nullptr && out != nullptr, what, "null pointer");
  UOCR_REQUIRE(ldq >= hd && ldk >= hd && ldv >= hd && ldo >= hd && sq >= 0 && sk >= 0 && sv >= 0 && so >= 0, what,
               "row strides must be >= hd and slice strides >= 0");
  UOCR_REQUIRE(aligned16(q) && aligned16(k) && aligned16(v) && aligned16(out) && ldq % 4 == 0 && ldk % 4 == 0 &&
                   ldv % 4 == 0 && ldo % 4 == 0 && sq % 4 == 0 && sk % 4 == 0 && sv % 4 == 0 && so % 4 == 0,
               what, "operands must be 16-byte aligned with strides of whole 16-byte chunks");
  return UOCR_ROCM_OK;
}

// The LDS layout of the per-query dot products: a grid width of whole
// tiles takes the per-tile bias terms with the width terms 16-byte aligned
// and rows 4 times an odd number of floats apart; otherwise rows h + w + 1
// apart.
struct DotsLayout {
  bool tile_rows;
  int64_t ld, dw_off;
};

DotsLayout dots_layout(int64_t h, int64_t w) {
  const bool tile_rows = w % kKeyTile == 0;
  const int64_t dw_off = tile_rows ? (h + 3) / 4 * 4 : h;
  int64_t quads = (dw_off + w) / 4;
  quads += quads % 2 == 0 ? 1 : 0;
  return {tile_rows, tile_rows ? 4 * quads : h + w + 1, dw_off};
}

// Grid rows per key tile of the split-operand kernel: 0 for a grid of
// whole 32-key tiles, 4, 2 or 1 for grids at most 8, 16 or 31 wide, -1
// otherwise.
int x3_rows_for(int64_t h, int64_t w) {
  if (w % kKeyTile == 0) return 0;
  return w <= 8 ? 4 : w <= 16 ? 2 : w < kKeyTile ? 1 : -1;
}

// Where the split key and value tiles start in the workspace (after the dot
// table, at a 256-byte boundary), and their floats (grids of whole tiles).
int64_t x3_tiles_offset(int64_t slices, int64_t h, int64_t w) {
  return (slices * h * w * dots_layout(h, w).ld + 63) / 64 * 64;
}
int64_t x3_tiles_floats(int64_t slices, int64_t h, int64_t w, int rows) {
  return rows == 0 ? slices * (h * w / kKeyTile) * kX3TileFloats : 0;  // grids of whole tiles only
}

// inner > 1: slice s = (s / inner, s % inner) with inner strides iq .. io.
int rel_pos_entry(const char* what, void* stream, const float* q, int64_t ldq, int64_t sq, const float* k, int64_t ldk,
                  int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out, int64_t ldo, int64_t so,
                  int64_t slices, int64_t h, int64_t w, int64_t hd, float scale, const float* rh, const float* rw,
                  float* workspace, int64_t workspace_floats, int64_t inner = 1, int64_t iq = 0, int64_t ik = 0,
                  int64_t iv = 0, int64_t io = 0, uint16_t* out16 = nullptr) {
  UOCR_REQUIRE(h >= 1 && w >= 1 && h + w <= kMaxRelSpan, what, "need h, w >= 1 and h + w <= 256");
  const int64_t n = h * w;
  if (const int st = check_common(what, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, slices, n, n, hd)) {
    return st;
  }
  UOCR_REQUIRE(rh != nullptr && rw != nullptr, what, "null relative-position table");
  UOCR_REQUIRE(aligned16(rh) && aligned16(rw), what, "relative-position tables must be 16-byte aligned");
  const DotsLayout lay = dots_layout(h, w);
  // the dot table goes to the workspace when it holds it (16-byte aligned)
  const bool table = workspace != nullptr && aligned16(workspace) && workspace_floats >= slices * n * lay.ld;
  // a bf16 output from the dot table with head dim 64: the split-operand
  // kernel, whose tiles are 32 keys of one grid row (whole tiles) or 4, 2
  // or 1 grid rows of at most 8, 16 or 31 keys, when the workspace also
  // holds the split key and value tiles
  int x3_rows = table && out16 != nullptr && hd == 64 ? x3_rows_for(h, w) : -1;
  if (x3_rows == 0 && workspace_floats < x3_tiles_offset(slices, h, w) + x3_tiles_floats(slices, h, w, 0)) {
    x3_rows = -1;  // no room for the split tiles of a whole-tile grid: the fp32 products
  }
  UOCR_REQUIRE(inner >= 1 && slices % inner == 0 && iq >= 0 && ik >= 0 && iv >= 0 && io >= 0 && iq % 4 == 0 &&
                   ik % 4 == 0 && iv % 4 == 0 && io % 4 == 0,
               what, "windows must divide the slices, window strides >= 0 in whole 16-byte chunks");
  AttnArgs a{q, k, v, out, ldq, sq, ldk, sk, ldv, sv, ldo, so, static_cast<int>(n), static_cast<int>(n),
             scale, nullptr, 0, rh, rw, static_cast<int>(h), static_cast<int>(w), static_cast<int>(lay.ld),
             static_cast<int>(lay.dw_off), table ? workspace : nullptr, table ? workspace : nullptr,
             static_cast<int>(inner), iq, ik, iv, io, out16};
  if (out16 != nullptr) a.out = nullptr;
  const bool x3 = x3_rows >= 0;
  if (x3) {
    a.table_mul = kLog2e;  // the split-operand kernel takes the bias in log2 units
    if (x3_rows == 0) a.kvx = reinterpret_cast<uint16_t*>(workspace + x3_tiles_offset(slices, h, w));
    a.x3_rows = x3_rows;
  }
  if (table) {
    clear_launch_error();
    if (h <= 16 && w <= 16) {
      // a 16 x 16 tile per table slice, four slices per workgroup
      const dim3 grid(static_cast<unsigned>((h + w + 3) / 4), static_cast<unsigned>(slices));
      if (hd == 64) {
        rel_dots16_k<64><<<grid, 256, 0, as_stream(stream)>>>(a);
      } else {
        rel_dots16_k<128><<<grid, 256, 0, as_stream(stream)>>>(a);
      }
    } else {
      // one wave per 32 x 32 tile of a block's product, up to 4 waves
      const int64_t tiles = ((h + 31) / 32) * ((w + 31) / 32);
      const unsigned threads = static_cast<unsigned>(64 * (tiles < 4 ? tiles : 4));
      const dim3 grid(static_cast<unsigned>(h + w), static_cast<unsigned>(slices));
      if (hd == 64) {
        rel_dots_k<64><<<grid, threads, 0, as_stream(stream)>>>(a);
      } else {
        rel_dots_k<128><<<grid, threads, 0, as_stream(stream)>>>(a);
      }
    }
    if (const int st = check_launch(what)) return st;
  }
  if (x3) {
    // a bf16 output: the products on the bf16 matrix cores, operands split
    const dim3 grid(static_cast<unsigned>((n + 4 * kQueriesPerWave - 1) / (4 * kQueriesPerWave)),
                    static_cast<unsigned>(slices));
    clear_launch_error();
    switch (x3_rows) {
      case 0: attention_x3_k<0><<<grid, 256, 0, as_stream(stream)>>>(a); break;
      case 1: attention_x3_k<1><<<grid, 256, 0, as_stream(stream)>>>(a); break;
      case 2: attention_x3_k<2><<<grid, 256, 0, as_stream(stream)>>>(a); break;
      default: attention_x3_k<4><<<grid, 256, 0, as_stream(stream)>>>(a); break;
    }
    return check_launch(what);
  }
  if (lay.tile_rows && table) return launch<Bias::kRelPosTable>(what, stream, hd, slices, a);
  return lay.tile_rows ? launch<Bias::kRelPosRows>(what, stream, hd, slices, a)
                       : launch<Bias::kRelPos>(what, stream, hd, slices, a);
}

// out: the fp32 output, or out16 reinterpreted (for the pointer checks) when
// out16 is non-null.
int attention_entry(const char* what, void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                    int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out, int64_t ldo,
                    int64_t so, int64_t slices, int64_t rows, int64_t keys, int64_t hd, float scale,
                    const float* mask, int64_t mask_ld, uint16_t* out16) {
  if (const int st = check_common(what, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, slices, rows, keys, hd)) {
    return st;
  }
  UOCR_REQUIRE(mask == nullptr || mask_ld >= keys, what, "mask rows must hold every key");
  AttnArgs a{q, k, v, out, ldq, sq, ldk, sk, ldv, sv, ldo, so, static_cast<int>(rows), static_cast<int>(keys),
             scale, mask, mask_ld, nullptr, nullptr, 0, 0, 0, 0, nullptr, nullptr, 1, 0, 0, 0, 0, out16};
  if (out16 != nullptr) a.out = nullptr;
  if (mask == nullptr && hd == kSplitHd && slices * ((rows + 127) / 128) < 256) {
    // few query rows: the keys split over a workgroup's waves
    const dim3 grid(static_cast<unsigned>((rows + kQueriesPerWave - 1) / kQueriesPerWave),
                    static_cast<unsigned>(slices));
    clear_launch_error();
    allow_lds(attention_keysplit_k, kSplitLds);
    attention_keysplit_k<<<grid, 64 * kSplitWaves, kSplitLds, as_stream(stream)>>>(a);
    return check_launch(what);
  }
  return mask != nullptr ? launch<Bias::kMask>(what, stream, hd, slices, a)
                         : launch<Bias::kNone>(what, stream, hd, slices, a);
}

// The masked split-operand attention's workspace: the mask's tile map
// (words per row block), then at a 256-byte boundary the split key and
// value tiles (64 hd floats per tile of 32 keys).
int64_t mask_map_words(int64_t keys) { return (keys + kMaskMapKeys - 1) / kMaskMapKeys; }
int64_t mask_map_floats(int64_t rows, int64_t keys) {
  return (rows + kMaskRowBlock - 1) / kMaskRowBlock * mask_map_words(keys);
}
int64_t masked_tiles_offset(int64_t rows, int64_t keys) { return (mask_map_floats(rows, keys) + 63) / 64 * 64; }
// Live tiles per workgroup: at most the tiles one of the slots (512: two
// workgroups on each of 256 CUs) would get if every tile of every row block
// were live, and at least 32; a row block with more live tiles has its walk
// cut into runs, so that the longest walks of a causal mask no longer set
// the time (row blocks enough to fill the slots: no cut). Then the runs per
// row block, and the partial records (O, then m and l) after the split tiles.
constexpr int64_t kSlots = 2 * 256;
constexpr int64_t kMinRunTiles = 32;
int64_t masked_run_tiles(int64_t slices, int64_t rows, int64_t keys, int64_t slots = kSlots) {
  const int64_t tiles = (keys + kKeyTile - 1) / kKeyTile;
  const int64_t blocks = slices * ((rows + kMaskRowBlock - 1) / kMaskRowBlock);
  const int64_t share = (tiles * blocks + slots - 1) / slots;  // >= tiles: no run is cut
  return share > kMinRunTiles ? share : kMinRunTiles;
}
int64_t masked_runs(int64_t slices, int64_t rows, int64_t keys, int64_t slots = kSlots) {
  const int64_t per = masked_run_tiles(slices, rows, keys, slots);
  return ((keys + kKeyTile - 1) / kKeyTile + per - 1) / per;
}
int64_t masked_partials_offset(int64_t slices, int64_t rows, int64_t keys, int64_t hd) {
  return masked_tiles_offset(rows, keys) + slices * ((keys + kKeyTile - 1) / kKeyTile) * 64 * hd;
}
int64_t masked_partial_rows(int64_t slices, int64_t rows, int64_t keys) {
  const int64_t runs = masked_runs(slices, rows, keys);
  return runs > 1 ? slices * ((rows + kMaskRowBlock - 1) / kMaskRowBlock) * runs * kMaskRowBlock : 0;
}
int64_t masked_workspace_floats(int64_t slices, int64_t rows, int64_t keys, int64_t hd) {
  return masked_partials_offset(slices, rows, keys, hd) + masked_partial_rows(slices, rows, keys) * (hd + 2);
}

// The fp32 masked attention with a workspace: the tile map, then the runs'
// partial records. Its head dim 128 holds one 4-wave workgroup per CU (the
// registers), so 256 slots there; 64 holds two.
int64_t fp32_slots(int64_t hd) { return hd == 128 ? kSlots / 2 : kSlots; }
int64_t fp32_partial_rows(int64_t slices, int64_t rows, int64_t keys, int64_t hd) {
  const int64_t runs = masked_runs(slices, rows, keys, fp32_slots(hd));
  return runs > 1 ? slices * ((rows + kMaskRowBlock - 1) / kMaskRowBlock) * runs * kMaskRowBlock : 0;
}
int64_t fp32_workspace_floats(int64_t slices, int64_t rows, int64_t keys, int64_t hd) {
  return masked_tiles_offset(rows, keys) + fp32_partial_rows(slices, rows, keys, hd) * (hd + 2);
}

int masked_fp32_entry(const char* what, void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                      int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out, int64_t ldo,
                      int64_t so, int64_t slices, int64_t rows, int64_t keys, int64_t hd, float scale,
                      const float* mask, int64_t mask_ld, float* workspace, int64_t workspace_floats,
                      uint16_t* out16) {
  if (mask == nullptr) {
    return attention_entry(what, stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, slices, rows, keys, hd,
                           scale, mask, mask_ld, out16);
  }
  if (const int st = check_common(what, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, slices, rows, keys, hd)) {
    return st;
  }
  UOCR_REQUIRE(mask_ld >= keys, what, "mask rows must hold every key");
  const int64_t row_blocks = (rows + kMaskRowBlock - 1) / kMaskRowBlock, words = mask_map_words(keys);
  UOCR_REQUIRE(row_blocks < 65536 && slices < 65536, what, "need rows < 2^23");
  UOCR_REQUIRE(workspace != nullptr && aligned16(workspace) &&
                   workspace_floats >= fp32_workspace_floats(slices, rows, keys, hd),
               what, "workspace: 16-byte aligned, uocr_rocm_attention_workspace_floats floats");
  AttnArgs a{q, k, v, out, ldq, sq, ldk, sk, ldv, sv, ldo, so, static_cast<int>(rows), static_cast<int>(keys),
             scale, mask, mask_ld, nullptr, nullptr, 0, 0, 0, 0, nullptr, nullptr, 1, 0, 0, 0, 0, out16};
  if (out16 != nullptr) a.out = nullptr;
  const int64_t runs = masked_runs(slices, rows, keys, fp32_slots(hd));
  uint32_t* map = reinterpret_cast<uint32_t*>(workspace);
  a.map = map;
  a.map_words = static_cast<int>(words);
  a.run_tiles = static_cast<int>(masked_run_tiles(slices, rows, keys, fp32_slots(hd)));
  a.runs = static_cast<int>(runs);
  float* po = workspace + masked_tiles_offset(rows, keys);
  a.part_o = runs > 1 ? po : nullptr;
  a.part_ml = runs > 1 ? po + fp32_partial_rows(slices, rows, keys, hd) * hd : nullptr;
  UOCR_REQUIRE(row_blocks * runs < (int64_t{1} << 31), what, "too many workgroups");
  clear_launch_error();
  mask_tiles_k<<<dim3(static_cast<unsigned>(4 * words), static_cast<unsigned>(row_blocks)), 256, 0,
                 as_stream(stream)>>>(
      mask, mask_ld, static_cast<int>(rows), static_cast<int>(keys), map, static_cast<int>(words));
  if (const int st = check_launch(what)) return st;
  const dim3 grid(static_cast<unsigned>(row_blocks * runs), static_cast<unsigned>(slices));
  clear_launch_error();
  if (hd == 64) {
    attention_k<64, Bias::kMask><<<grid, 256, 0, as_stream(stream)>>>(a);
  } else {
    attention_k<128, Bias::kMask><<<grid, 256, 0, as_stream(stream)>>>(a);
  }
  if (runs == 1) return check_launch(what);
  if (const int st = check_launch(what)) return st;
  X3Partials part{a.run_tiles, a.runs, a.part_o, a.part_ml};
  const dim3 merge_grid(static_cast<unsigned>(row_blocks), static_cast<unsigned>(slices));
  clear_launch_error();
  if (hd == 64) {
    x3m_merge_k<64><<<merge_grid, 256, 0, as_stream(stream)>>>(a, map, static_cast<int>(words),
                                                               static_cast<int>(row_blocks), part, kLog2e);
  } else {
    x3m_merge_k<128><<<merge_grid, 256, 0, as_stream(stream)>>>(a, map, static_cast<int>(words),
                                                                static_cast<int>(row_blocks), part, kLog2e);
  }
  return check_launch(what);
}

int masked_split_entry(const char* what, void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                       int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv, uint16_t* out, int64_t ldo,
                       int64_t so, int64_t slices, int64_t rows, int64_t keys, int64_t hd, float scale,
                       const float* mask, int64_t mask_ld, float* workspace, int64_t workspace_floats) {
  if (const int st = check_common(what, q, ldq, sq, k, ldk, sk, v, ldv, sv, reinterpret_cast<const float*>(out), ldo,
                                  so, slices, rows, keys, hd)) {
    return st;
  }
  UOCR_REQUIRE(mask != nullptr && mask_ld >= keys, what, "mask [rows, mask_ld] with mask_ld >= keys");
  const int64_t row_blocks = (rows + kMaskRowBlock - 1) / kMaskRowBlock, words = mask_map_words(keys);
  UOCR_REQUIRE(row_blocks < 65536 && row_blocks * slices < (int64_t{1} << 31), what,
               "need rows < 2^23 and row blocks x slices < 2^31");
  UOCR_REQUIRE(workspace != nullptr && aligned16(workspace) &&
                   workspace_floats >= masked_workspace_floats(slices, rows, keys, hd),
               what, "workspace: 16-byte aligned, uocr_rocm_attention_masked_workspace_floats floats");
  AttnArgs a{q, k, v, nullptr, ldq, sq, ldk, sk, ldv, sv, ldo, so, static_cast<int>(rows), static_cast<int>(keys),
             scale, mask, mask_ld, nullptr, nullptr, 0, 0, 0, 0, nullptr, nullptr, 1, 0, 0, 0, 0, out};
  a.kvx = reinterpret_cast<uint16_t*>(workspace + masked_tiles_offset(rows, keys));
  uint32_t* map = reinterpret_cast<uint32_t*>(workspace);
  const int64_t tiles = (keys + kKeyTile - 1) / kKeyTile;
  clear_launch_error();
  mask_tiles_k<<<dim3(static_cast<unsigned>(4 * words), static_cast<unsigned>(row_blocks)), 256, 0,
                 as_stream(stream)>>>(
      mask, mask_ld, static_cast<int>(rows), static_cast<int>(keys), map, static_cast<int>(words));
  if (const int st = check_launch(what)) return st;
  const dim3 split_grid(static_cast<unsigned>(tiles), static_cast<unsigned>(slices));
  clear_launch_error();
  if (hd == 64) {
    x3m_split_k<64><<<split_grid, 256, 0, as_stream(stream)>>>(a, static_cast<int>(tiles));
  } else {
    x3m_split_k<128><<<split_grid, 256, 0, as_stream(stream)>>>(a, static_cast<int>(tiles));
  }
  if (const int st = check_launch(what)) return st;
  const int64_t runs = masked_runs(slices, rows, keys);
  float* po = workspace + masked_partials_offset(slices, rows, keys, hd);
  X3Partials part{static_cast<int>(masked_run_tiles(slices, rows, keys)), static_cast<int>(runs), runs > 1 ? po : nullptr,
                  runs > 1 ? po + masked_partial_rows(slices, rows, keys) * hd : nullptr};
  UOCR_REQUIRE(row_blocks * runs * slices < (int64_t{1} << 31), what, "too many workgroups");
  const unsigned grid = static_cast<unsigned>(row_blocks * runs * slices);
  const int w = static_cast<int>(words), rbs = static_cast<int>(row_blocks), sl = static_cast<int>(slices);
  clear_launch_error();
  if (hd == 64) {
    attention_x3m_k<64><<<grid, 256, 0, as_stream(stream)>>>(a, map, w, rbs, sl, part);
  } else {
    attention_x3m_k<128><<<grid, 256, 0, as_stream(stream)>>>(a, map, w, rbs, sl, part);
  }
  if (runs == 1) return check_launch(what);
  if (const int st = check_launch(what)) return st;
  const dim3 merge_grid(static_cast<unsigned>(row_blocks), static_cast<unsigned>(slices));
  clear_launch_error();
  if (hd == 64) {
    x3m_merge_k<64><<<merge_grid, 256, 0, as_stream(stream)>>>(a, map, w, rbs, part, 1.0f);
  } else {
    x3m_merge_k<128><<<merge_grid, 256, 0, as_stream(stream)>>>(a, map, w, rbs, part, 1.0f);
  }
  return check_launch(what);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_attention(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k, int64_t ldk,
                        int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out, int64_t ldo, int64_t so,
                        int64_t slices, int64_t rows, int64_t keys, int64_t hd, float scale, const float* mask,
                        int64_t mask_ld) {
  return attention_entry("uocr_rocm_attention", stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, slices,
                         rows, keys, hd, scale, mask, mask_ld, nullptr);
}

int uocr_rocm_attention_bf16(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k, int64_t ldk,
                             int64_t sk, const float* v, int64_t ldv, int64_t sv, uint16_t* out, int64_t ldo,
                             int64_t so, int64_t slices, int64_t rows, int64_t keys, int64_t hd, float scale,
                             const float* mask, int64_t mask_ld) {
  return attention_entry("uocr_rocm_attention_bf16", stream, q, ldq, sq, k, ldk, sk, v, ldv, sv,
                         reinterpret_cast<float*>(out), ldo, so, slices, rows, keys, hd, scale, mask, mask_ld, out);
}

int64_t uocr_rocm_attention_workspace_floats(int64_t slices, int64_t rows, int64_t keys, int64_t hd) {
  if (slices < 1 || rows < 1 || keys < 1 || (hd != 64 && hd != 128)) return 0;
  return fp32_workspace_floats(slices, rows, keys, hd);
}

int uocr_rocm_attention_ws(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k, int64_t ldk,
                           int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out, int64_t ldo, int64_t so,
                           int64_t slices, int64_t rows, int64_t keys, int64_t hd, float scale, const float* mask,
                           int64_t mask_ld, float* workspace, int64_t workspace_floats) {
  return masked_fp32_entry("uocr_rocm_attention_ws", stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, slices,
                           rows, keys, hd, scale, mask, mask_ld, workspace, workspace_floats, nullptr);
}

int uocr_rocm_attention_bf16_ws(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k, int64_t ldk,
                                int64_t sk, const float* v, int64_t ldv, int64_t sv, uint16_t* out, int64_t ldo,
                                int64_t so, int64_t slices, int64_t rows, int64_t keys, int64_t hd, float scale,
                                const float* mask, int64_t mask_ld, float* workspace, int64_t workspace_floats) {
  return masked_fp32_entry("uocr_rocm_attention_bf16_ws", stream, q, ldq, sq, k, ldk, sk, v, ldv, sv,
                           reinterpret_cast<float*>(out), ldo, so, slices, rows, keys, hd, scale, mask, mask_ld,
                           workspace, workspace_floats, out);
}

int64_t uocr_rocm_attention_masked_workspace_floats(int64_t slices, int64_t rows, int64_t keys, int64_t hd) {
  if (slices < 1 || rows < 1 || keys < 1 || (hd != 64 && hd != 128)) return 0;
  return masked_workspace_floats(slices, rows, keys, hd);
}

int uocr_rocm_attention_masked_bf16_ws(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                                       int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv,
                                       uint16_t* out, int64_t ldo, int64_t so, int64_t slices, int64_t rows,
                                       int64_t keys, int64_t hd, float scale, const float* mask, int64_t mask_ld,
                                       float* workspace, int64_t workspace_floats) {
  return masked_split_entry("uocr_rocm_attention_masked_bf16_ws", stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo,
                            so, slices, rows, keys, hd, scale, mask, mask_ld, workspace, workspace_floats);
}

int uocr_rocm_attention_rel_pos(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k, int64_t ldk,
                                int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out, int64_t ldo,
                                int64_t so, int64_t slices, int64_t h, int64_t w, int64_t hd, float scale,
                                const float* rh, const float* rw) {
  return rel_pos_entry("uocr_rocm_attention_rel_pos", stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, slices,
                       h, w, hd, scale, rh, rw, nullptr, 0);
}

int64_t uocr_rocm_attention_rel_pos_workspace_floats(int64_t slices, int64_t h, int64_t w) {
  if (slices < 1 || h < 1 || w < 1 || h + w > kMaxRelSpan) return 0;
  const int rows = x3_rows_for(h, w);
  if (rows != 0) return slices * h * w * dots_layout(h, w).ld;
  return x3_tiles_offset(slices, h, w) + x3_tiles_floats(slices, h, w, 0);
}

int uocr_rocm_attention_rel_pos_ws(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                                   int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out,
                                   int64_t ldo, int64_t so, int64_t slices, int64_t h, int64_t w, int64_t hd,
                                   float scale, const float* rh, const float* rw, float* workspace,
                                   int64_t workspace_floats) {
  return rel_pos_entry("uocr_rocm_attention_rel_pos_ws", stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so,
                       slices, h, w, hd, scale, rh, rw, workspace, workspace_floats);
}

int uocr_rocm_attention_rel_pos_windows_ws(void* stream, const float* q, int64_t ldq, int64_t sq, int64_t wq,
                                           const float* k, int64_t ldk, int64_t sk, int64_t wk, const float* v,
                                           int64_t ldv, int64_t sv, int64_t wv, float* out, int64_t ldo, int64_t so,
                                           int64_t wo, int64_t heads, int64_t windows, int64_t h, int64_t w,
                                           int64_t hd, float scale, const float* rh, const float* rw, float* workspace,
                                           int64_t workspace_floats) {
  constexpr const char* kWhat = "uocr_rocm_attention_rel_pos_windows_ws";
  UOCR_REQUIRE(heads >= 1 && windows >= 1 && heads * windows < 65536, kWhat, "need heads, windows >= 1");
  return rel_pos_entry(kWhat, stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, out, ldo, so, heads * windows, h, w, hd,
                       scale, rh, rw, workspace, workspace_floats, windows, wq, wk, wv, wo);
}

int uocr_rocm_attention_rel_pos_windows_bf16_ws(void* stream, const float* q, int64_t ldq, int64_t sq, int64_t wq,
                                                const float* k, int64_t ldk, int64_t sk, int64_t wk, const float* v,
                                                int64_t ldv, int64_t sv, int64_t wv, uint16_t* out, int64_t ldo,
                                                int64_t so, int64_t wo, int64_t heads, int64_t windows, int64_t h,
                                                int64_t w, int64_t hd, float scale, const float* rh, const float* rw,
                                                float* workspace, int64_t workspace_floats) {
  constexpr const char* kWhat = "uocr_rocm_attention_rel_pos_windows_bf16_ws";
  UOCR_REQUIRE(heads >= 1 && windows >= 1 && heads * windows < 65536, kWhat, "need heads, windows >= 1");
  return rel_pos_entry(kWhat, stream, q, ldq, sq, k, ldk, sk, v, ldv, sv, reinterpret_cast<float*>(out), ldo, so,
                       heads * windows, h, w, hd, scale, rh, rw, workspace, workspace_floats, windows, wq, wk, wv, wo,
                       out);
}

}  // extern "C"
