// gemm.hip: the prefill projection y[m, n] = bf16(x)[m, k] . w[n, k]^T
// (+ bias[n]) on gfx950's bf16 matrix cores, fp32 accumulation and output:
// the reference's cuda::linear for m > 1 (src/backend/cuda/ops.h:14-17,
// ops.cu:268-287, which rounds x to bf16 in its own pass and calls a bf16
// cuBLAS GEMM with fp32 compute, then adds the bias).
//
// Both operands are k-contiguous (x rows, w rows), so one tile layout serves
// both. A workgroup of 4 waves computes a 128 x 128 tile of y; wave (wm, wn)
// owns a 64 x 64 quarter as 2 x 2 v_mfma_f32_32x32x16_bf16 tiles. The k
// loop steps 64 at a time through two LDS buffers. Tile rows are 8 chunks of
// 8 bf16 (16 bytes); a chunk's slot is XOR-swizzled by the row so that the
// rows one operand read spans fall on different banks (slot() below). Two kernels:
//   * x already bf16 and k a multiple of 64: both tiles go from memory
//     straight into LDS (16-byte global_load_lds, each lane's chunk picked so
//     that it lands in its swizzled slot), the next step's loads in flight
//     while the current step's 16 matrix products run;
//   * otherwise (fp32 x, or k not a multiple of 64): chunks staged through
//     registers, x rounded to bf16 with the hardware's nearest-even
//     conversion on the way, chunks past k zero-filled; a k that is not a
//     multiple of 8 (or unaligned rows) loads element by element.
// Workgroups are dealt to the 8 XCDs round-robin; each XCD takes a
// contiguous run of tiles, ordered in groups of 8 tile-rows sweeping the
// columns, so the tiles resident on one XCD share x rows and w rows in its
// L2. The bias is added to each finished sum (one fp32 rounding, as the
// reference's separate bias pass). A product with few tiles and a long k
// (the vision encoder's convolutions, CLIP's 257-row projections) may split
// k over a caller's workspace: each split writes its partial products and one
// more launch sums them in split order, then adds the bias. Products of bf16
// rows with no epilogue beyond the bias and the add into y, at least 128
// rows, go to hipBLASLt instead (gemm_library.hip); the tiles take the
// activation epilogues, the row scatter, fp32 rows and few rows.

#include "act_math.hpp"
#include "common.hpp"

namespace uocr_rocm {
namespace {

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x16 __attribute__((ext_vector_type(16)));

constexpr int kTileM = 128;
constexpr int kTileN = 128;
constexpr int kTileK = 64;
constexpr int kGemmThreads = 256;
constexpr int kRowChunks = kTileK / 8;                                     // 16-byte chunks per tile row
constexpr int kTileChunks = kTileM * kRowChunks;                           // per operand tile
constexpr int kChunksPerThread = kTileChunks / kGemmThreads;               // 4
static_assert(kTileM == kTileN, "one staging pattern for both operands");

// The LDS slot of 16-byte chunk `chunk` of tile row `row`. A 128-bit LDS
// read serves 16 lanes a pass from 64 four-byte banks (16 chunk-wide bank
// groups, 256 bytes); the products' reads take one chunk column of 16
// consecutive rows per pass, whose row bases fall on 2 bank groups (rows are
// 128 bytes). XOR-ing the chunk with (row / 2) mod 8 spreads the 8 rows of
// each parity over the 8 groups of its half: the 16 reads land on 16
// different groups. (With row mod 8, rows r and r + 8 met in one group:
// measured 4 conflict cycles per LDS instruction on MI355X.)
__device__ __forceinline__ int swz(int row) { return (row >> 1) & 7; }
__device__ __forceinline__ int slot(int row, int chunk) { return row * kRowChunks + (chunk ^ swz(row)); }

constexpr int kXcds = 8;
constexpr int kGroupRows = 8;

// The tile (tm, tn) of workgroup bid: a contiguous run of tiles per XCD
// (workgroups go to the XCDs in turn, bid mod 8; XCD x holds total / 8
// tiles, one more for the first total mod 8), groups of kGroupRows
// tile-rows sweeping the columns inside a run.
__device__ __forceinline__ void tile_of(int bid, int tiles_m, int tiles_n, int& tm, int& tn) {
  const int total = tiles_m * tiles_n;
  const int per_xcd = total / kXcds, extra = total % kXcds, xcd = bid % kXcds;
  const int t = xcd * per_xcd + (xcd < extra ? xcd : extra) + bid / kXcds;
  const int per = kGroupRows * tiles_n, group = t / per, first = group * kGroupRows;
  const int rows = tiles_m - first < kGroupRows ? tiles_m - first : kGroupRows;
  const int in = t - group * per;
  tm = first + in % rows;
  tn = in / rows;
}

struct LinearArgs {
  const void* x;  // float or bf16 rows
  const uint16_t* w;
  const float* bias;
  float* y;
  int64_t m, n;
  int k;
  int tiles_m, tiles_n;
  // Split k: workgroup b takes tile b % tiles of split b / tiles, columns
  // [split * k_len, min(k, (split + 1) * k_len)) of the sums, into part +
  // split * m * n (no bias); part null: one split, into y with the bias.
  int k_len;
  float* part;
  // y += the product (+ bias): each element y + (sum + bias), as the
  // product followed by an in-place add
  bool accumulate;
  // Non-null: product row r goes to y row row_map[r], dropped when that is
  // y_rows or more (a scatter of window slots back into a grid); the
  // TM x 128 kernels only, no split.
  const int64_t* row_map;
  int64_t y_rows;
  // the activation epilogues' output: y16 = bf16(act(sum + bias)), no split,
  // no accumulate
  uint16_t* y16;
};

// What the epilogue writes: the fp32 sums, or an MLP's activation of them
// rounded to bf16, bitwise the fp32 product followed by the elementwise
// activation into bf16 (the same arithmetic, from act_math.hpp).
enum class Epi { kPlain, kGeluBf16, kQuickGeluBf16 };

template <Epi kEpi>
__device__ __forceinline__ void store_act(const LinearArgs& a, int64_t row, int64_t col, float v) {
  v = kEpi == Epi::kGeluBf16 ? gelu_f<10>(v) : quick_gelu_f(v);
  a.y16[row * a.n + col] = f32_to_bf16(v);
}

// 16 elements of one output column, product rows row0 + 8 (r / 4) + r % 4
// (r < 16), into y through the row map.
__device__ __forceinline__ void store_mapped(const LinearArgs& a, int64_t row0, int64_t col, float bv, bool add,
                                             const float (&val)[16]) {
  int64_t at[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    const int64_t row = row0 + 8 * (r / 4) + (r % 4);
    const int64_t to = row < a.m ? a.row_map[row] : a.y_rows;
    at[r] = to < a.y_rows ? to * a.n + col : -1;
  }
  float base[16];
#pragma unroll
  for (int r = 0; r < 16; ++r) base[r] = a.accumulate && at[r] >= 0 ? a.y[at[r]] : 0.0f;
#pragma unroll
  for (int r = 0; r < 16; ++r) {
    if (at[r] >= 0) {
      const float v = add ? val[r] + bv : val[r];
      a.y[at[r]] = a.accumulate ? base[r] + v : v;
    }
  }
}

// The tile, split and k range of this workgroup.
struct Work {
  int64_t m0, n0;
  int split, k_begin, k_end;
};

template <int kTileRows = kTileM>
__device__ __forceinline__ Work work_of(const LinearArgs& a) {
  const int tiles = a.tiles_m * a.tiles_n;
  const int split = static_cast<int>(blockIdx.x) / tiles;
  int tm, tn;
  tile_of(static_cast<int>(blockIdx.x) - split * tiles, a.tiles_m, a.tiles_n, tm, tn);
  const int kb = split * a.k_len;
  return {static_cast<int64_t>(tm) * kTileRows, static_cast<int64_t>(tn) * kTileN, split, kb,
          a.k - kb < a.k_len ? a.k : kb + a.k_len};
}

// The registers one k step stages: per thread kChunksPerThread chunks of the
// x tile (8 elements each: fp32, rounded on the way to LDS, or bf16) and of
// the w tile.
template <bool kF32X>
struct Staged {
  u32x4 xa[kChunksPerThread][kF32X ? 2 : 1];
  u32x4 wb[kChunksPerThread];
};

template <bool kF32X>
__device__ __forceinline__ void load_step(const LinearArgs& a, int64_t m0, int64_t n0, int k0, int k_end,
                                          Staged<kF32X>& s) {
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int id = static_cast<int>(threadIdx.x) + kGemmThreads * i;
    const int row = id / kRowChunks, c = id % kRowChunks;
    const int kc = k0 + 8 * c;
    const bool kin = kc < k_end;
    const int64_t xr = m0 + row, wr = n0 + row;
#pragma unroll
    for (int h = 0; h < (kF32X ? 2 : 1); ++h) s.xa[i][h] = u32x4{0u, 0u, 0u, 0u};
    s.wb[i] = u32x4{0u, 0u, 0u, 0u};
    if (kin && xr < a.m) {
      if constexpr (kF32X) {
        const u32x4* p = reinterpret_cast<const u32x4*>(static_cast<const float*>(a.x) + xr * a.k + kc);
        s.xa[i][0] = p[0];
        s.xa[i][1] = p[1];
      } else {
        s.xa[i][0] = *reinterpret_cast<const u32x4*>(static_cast<const uint16_t*>(a.x) + xr * a.k + kc);
      }
    }
    if (kin && wr < a.n) s.wb[i] = *reinterpret_cast<const u32x4*>(a.w + wr * a.k + kc);
  }
}

// A k that is not a multiple of 8 (rows not 16-byte aligned): each chunk's
// 8 elements are loaded one by one, those at or past k read as zero.
template <bool kF32X>
__device__ __forceinline__ void load_step_ragged(const LinearArgs& a, int64_t m0, int64_t n0, int k0, int k_end,
                                                 Staged<kF32X>& s) {
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int id = static_cast<int>(threadIdx.x) + kGemmThreads * i;
    const int row = id / kRowChunks, c = id % kRowChunks;
    const int kc = k0 + 8 * c;
    const int64_t xr = m0 + row, wr = n0 + row;
    uint32_t xv[8], wv[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const bool in = kc + e < k_end;
      xv[e] = 0u;
      wv[e] = 0u;
      if (in && xr < a.m) {
        if constexpr (kF32X) {
          xv[e] = __float_as_uint(static_cast<const float*>(a.x)[xr * a.k + kc + e]);
        } else {
          xv[e] = static_cast<const uint16_t*>(a.x)[xr * a.k + kc + e];
        }
      }
      if (in && wr < a.n) wv[e] = a.w[wr * a.k + kc + e];
    }
    if constexpr (kF32X) {
      s.xa[i][0] = u32x4{xv[0], xv[1], xv[2], xv[3]};
      s.xa[i][1] = u32x4{xv[4], xv[5], xv[6], xv[7]};
    } else {
      s.xa[i][0] = u32x4{xv[0] | (xv[1] << 16), xv[2] | (xv[3] << 16), xv[4] | (xv[5] << 16), xv[6] | (xv[7] << 16)};
    }
    s.wb[i] = u32x4{wv[0] | (wv[1] << 16), wv[2] | (wv[3] << 16), wv[4] | (wv[5] << 16), wv[6] | (wv[7] << 16)};
  }
}

template <bool kF32X>
__device__ __forceinline__ void store_step(const Staged<kF32X>& s, u32x4* xs, u32x4* ws) {
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int id = static_cast<int>(threadIdx.x) + kGemmThreads * i;
    const int row = id / kRowChunks, c = id % kRowChunks;
    if constexpr (kF32X) {
      const u32x4 lo = s.xa[i][0], hi = s.xa[i][1];
      xs[slot(row, c)] = u32x4{pack_bf16(__uint_as_float(lo.x), __uint_as_float(lo.y)),
                               pack_bf16(__uint_as_float(lo.z), __uint_as_float(lo.w)),
                               pack_bf16(__uint_as_float(hi.x), __uint_as_float(hi.y)),
                               pack_bf16(__uint_as_float(hi.z), __uint_as_float(hi.w))};
    } else {
      xs[slot(row, c)] = s.xa[i][0];
    }
    ws[slot(row, c)] = s.wb[i];
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

// The 16 matrix products of one 64-wide k step of a wave's 64 x 64 quarter
// from the tiles in LDS. The operand reads of slice kk + 1 go out one
// between each two products of slice kk, and `issue` (the next step's
// memory-to-LDS loads, kIssued instructions, or nothing) among the first
// slice's products: a wave never waits on LDS with products it could have
// issued (the group barriers pin that order; left to itself the scheduler
// bunches the reads and waits for them before the products).
template <int kIssued, class Issue>
__device__ __forceinline__ void mfma_step(const u32x4* xs, const u32x4* ws, int wm, int wn, int half, int r32,
                                          f32x16 (&acc)[2][2], Issue issue) {
  constexpr int kMfma = 0x008, kDsRead = 0x100, kVmemRead = 0x020;
  bf16x8 fa[2][2], fb[2][2];
  auto read = [&](int kk, int b) {
    const int c = 2 * kk + half;
#pragma unroll
    for (int i = 0; i < 2; ++i) fa[b][i] = as_bf16x8(xs[slot(64 * wm + 32 * i + r32, c)]);
#pragma unroll
    for (int j = 0; j < 2; ++j) fb[b][j] = as_bf16x8(ws[slot(64 * wn + 32 * j + r32, c)]);
  };
  read(0, 0);
  __builtin_amdgcn_sched_barrier(0);
#pragma unroll
  for (int kk = 0; kk < kTileK / 16; ++kk) {
    if (kk + 1 < kTileK / 16) read(kk + 1, (kk + 1) & 1);
    if (kk == 0) issue();
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int j = 0; j < 2; ++j) {
        acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk & 1][i], fb[kk & 1][j], acc[i][j], 0, 0, 0);
      }
    }
    if (kk + 1 < kTileK / 16) {
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        __builtin_amdgcn_sched_group_barrier(kMfma, 1, 0);
        __builtin_amdgcn_sched_group_barrier(kDsRead, 1, 0);
        if (kk == 0 && kIssued > 0) __builtin_amdgcn_sched_group_barrier(kVmemRead, (kIssued + 3) / 4, 0);
      }
    }
    __builtin_amdgcn_sched_barrier(0);
  }
}

// acc[i][j][r] is y row 8 (r / 4) + 4 half + r % 4 of the 32 x 32 tile,
// column r32.
template <Epi kEpi = Epi::kPlain>
__device__ __forceinline__ void store_tile(const LinearArgs& a, const Work& wk, int wm, int wn, int half, int r32,
                                           const f32x16 (&acc)[2][2]) {
  const bool split = a.part != nullptr;
  float* out = split ? a.part + static_cast<int64_t>(wk.split) * a.m * a.n : a.y;
  const bool add = !split && a.bias != nullptr;
  const bool accumulate = !split && a.accumulate;
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = wk.n0 + 64 * wn + 32 * j + r32;
    if (col >= a.n) continue;
    const float bv = add ? a.bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
      const int64_t row0 = wk.m0 + 64 * wm + 32 * i + 4 * half;
      if constexpr (kEpi != Epi::kPlain) {
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          const int64_t row = row0 + 8 * (r / 4) + (r % 4);
          if (row < a.m) store_act<kEpi>(a, row, col, add ? acc[i][j][r] + bv : acc[i][j][r]);
        }
        continue;
      }
      float* const o = out + row0 * a.n + col;  // element r: row row0 + 8 (r / 4) + r % 4
      auto live = [&](int r) { return row0 + 8 * (r / 4) + (r % 4) < a.m; };
      auto off = [&](int r) { return static_cast<int64_t>(8 * (r / 4) + (r % 4)) * a.n; };
      // accumulate: the 16 y values are requested before the first store (a
      // load issued after a store could alias it and would wait for it)
      float base[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) base[r] = accumulate && live(r) ? o[off(r)] : 0.0f;
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        if (live(r)) {
          const float v = add ? acc[i][j][r] + bv : acc[i][j][r];
          o[off(r)] = accumulate ? base[r] + v : v;
        }
      }
    }
  }
}

// y = the sum of the splits' partial products in split order (+ bias);
// accumulate: y += that.
__global__ __launch_bounds__(kBlock) void split_sum_k(const float* __restrict__ part, int splits, int64_t m, int64_t n,
                                                       const float* __restrict__ bias, float* __restrict__ y,
                                                       bool accumulate) {
  const int64_t total = m * n;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    float v = part[i];
    for (int sp = 1; sp < splits; ++sp) v += part[sp * total + i];
    v = bias != nullptr ? v + bias[i % n] : v;
    y[i] = accumulate ? y[i] + v : v;
  }
}

__device__ __forceinline__ void zero(f32x16 (&acc)[2][2]) {
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    }
  }
}

// Chunks staged through registers (fp32 x, or a k that is not a multiple of
// 64; kRagged: not a multiple of 8).
template <bool kF32X, bool kRagged>
__global__ __launch_bounds__(kGemmThreads) void linear_staged_k(const LinearArgs a) {
  __shared__ u32x4 xs[2][kTileChunks];
  __shared__ u32x4 ws[2][kTileChunks];
  const Work wk = work_of(a);
  const int lane = threadIdx.x & (kWave - 1), wave = wave_in_block();
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, r32 = lane & 31;
  f32x16 acc[2][2];
  zero(acc);
  const int steps = (wk.k_end - wk.k_begin + kTileK - 1) / kTileK;
  Staged<kF32X> s;
  auto load = [&](int k0) {
    if constexpr (kRagged) {
      load_step_ragged(a, wk.m0, wk.n0, k0, wk.k_end, s);
    } else {
      load_step(a, wk.m0, wk.n0, k0, wk.k_end, s);
    }
  };
  load(wk.k_begin);
  store_step(s, xs[0], ws[0]);
  lds_barrier();
  for (int t = 0; t < steps; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < steps;
    if (more) load(wk.k_begin + (t + 1) * kTileK);
    mfma_step<0>(xs[buf], ws[buf], wm, wn, half, r32, acc, [] {});
    if (more) store_step(s, xs[buf ^ 1], ws[buf ^ 1]);
    lds_barrier();
  }
  store_tile(a, wk, wm, wn, half, r32, acc);
}

// bf16 x and k a multiple of 64: tiles go straight from memory into LDS.
// Each wave issues 4 + 4 16-byte global_load_lds per step, each writing 64
// consecutive chunk slots (lane l to slot base + l) with the chunk that
// belongs there under the swizzle. Rows past m or n read a valid row (their
// sums are never stored). The step's loads are waited for with the wave's
// own vmcnt before the barrier (a fence there would also wait for the next
// step's loads); the barrier is an s_barrier with a compiler memory clobber.
__device__ __forceinline__ void dma_step(const LinearArgs& a, int64_t m0, int64_t n0, int k0, u32x4* xs, u32x4* ws,
                                         int wave, int lane) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
#pragma unroll
  for (int i = 0; i < kTileChunks / kGemmThreads; ++i) {
    const int s0 = (wave * (kTileChunks / kGemmThreads) + i) * kWave;  // wave-uniform
    const int sl = s0 + lane, row = sl / kRowChunks, c = (sl % kRowChunks) ^ swz(row);
    const int64_t xr = m0 + row < a.m ? m0 + row : a.m - 1;
    const int64_t wr = n0 + row < a.n ? n0 + row : a.n - 1;
    __builtin_amdgcn_global_load_lds(x + xr * a.k + k0 + 8 * c, xs + s0, 16, 0, 0);
    __builtin_amdgcn_global_load_lds(a.w + wr * a.k + k0 + 8 * c, ws + s0, 16, 0, 0);
  }
}

template <int kPending>
__device__ __forceinline__ void wait_loads_and_barrier() {
  // s_waitcnt vmcnt(kPending) with the other counters left alone, then the
  // barrier; the asm's memory clobber keeps LDS accesses on their side.
  __builtin_amdgcn_s_waitcnt((kPending & 0xF) | (((kPending >> 4) & 3) << 14) | (7 << 4) | (0xF << 8));
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

template <Epi kEpi>
__global__ __launch_bounds__(kGemmThreads) void linear_dma_k(const LinearArgs a) {
  __shared__ u32x4 xs[2][kTileChunks];
  __shared__ u32x4 ws[2][kTileChunks];
  const Work wk = work_of(a);
  const int lane = threadIdx.x & (kWave - 1), wave = wave_in_block();
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, r32 = lane & 31;
  f32x16 acc[2][2];
  zero(acc);
  const int steps = (wk.k_end - wk.k_begin) / kTileK;
  dma_step(a, wk.m0, wk.n0, wk.k_begin, xs[0], ws[0], wave, lane);
  for (int t = 0; t < steps; ++t) {
    const int buf = t & 1;
    wait_loads_and_barrier<0>();  // this step's tiles are in LDS; every wave is done with the other buffer
    const bool more = t + 1 < steps;
    mfma_step<2 * kTileChunks / kGemmThreads>(xs[buf], ws[buf], wm, wn, half, r32, acc, [&] {
      if (more) dma_step(a, wk.m0, wk.n0, wk.k_begin + (t + 1) * kTileK, xs[buf ^ 1], ws[buf ^ 1], wave, lane);
    });
  }
  store_tile<kEpi>(a, wk, wm, wn, half, r32, acc);
}

// Products of few rows (CLIP's 257, a short prompt), or of too few 128-row
// tiles to give every CU two: TM x 128 tiles with TM 32 or 64, so that a
// 257-row product has 9 row tiles instead of 3 (the last of them holding
// one row), and a [4096, 768] output 384 tiles instead of 192. Wave w of 4
// owns columns 32 w .. 32 w + 31 of the tile, TM / 32
// v_mfma_f32_32x32x16_bf16 tiles, its operands read from the same swizzled
// LDS layout as the 128 x 128 tiles; bf16 x and k a multiple of 64, tiles
// straight from memory into LDS.
constexpr int kNarrowM = 32;

template <int TM>
__device__ __forceinline__ void dma_step_narrow(const LinearArgs& a, int64_t m0, int64_t n0, int k0, u32x4* xs,
                                                u32x4* ws, int wave, int lane) {
  const uint16_t* x = static_cast<const uint16_t*>(a.x);
  constexpr int kXPerWave = TM * kRowChunks / kGemmThreads;  // x tile loads per wave: 1 or 2
#pragma unroll
  for (int i = 0; i < kXPerWave; ++i) {
    const int s0 = (wave * kXPerWave + i) * kWave;
    const int sl = s0 + lane, row = sl / kRowChunks, c = (sl % kRowChunks) ^ swz(row);
    const int64_t xr = m0 + row < a.m ? m0 + row : a.m - 1;
    __builtin_amdgcn_global_load_lds(x + xr * a.k + k0 + 8 * c, xs + s0, 16, 0, 0);
  }
#pragma unroll
  for (int i = 0; i < kTileChunks / kGemmThreads; ++i) {
    const int s0 = (wave * (kTileChunks / kGemmThreads) + i) * kWave;
    const int sl = s0 + lane, row = sl / kRowChunks, c = (sl % kRowChunks) ^ swz(row);
    const int64_t wr = n0 + row < a.n ? n0 + row : a.n - 1;
    __builtin_amdgcn_global_load_lds(a.w + wr * a.k + k0 + 8 * c, ws + s0, 16, 0, 0);
  }
}

template <int TM, Epi kEpi>
__global__ __launch_bounds__(kGemmThreads) void linear_narrow_k(const LinearArgs a) {
  constexpr int FI = TM / 32;
  __shared__ u32x4 xs[2][TM * kRowChunks];
  __shared__ u32x4 ws[2][kTileChunks];
  const Work wk = work_of<TM>(a);
  const int lane = threadIdx.x & (kWave - 1), wave = wave_in_block();
  const int half = lane >> 5, r32 = lane & 31;
  f32x16 acc[FI];
#pragma unroll
  for (int i = 0; i < FI; ++i) {
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[i][r] = 0.0f;
  }
  const int steps = (wk.k_end - wk.k_begin) / kTileK;
  dma_step_narrow<TM>(a, wk.m0, wk.n0, wk.k_begin, xs[0], ws[0], wave, lane);
  for (int t = 0; t < steps; ++t) {
    const int buf = t & 1;
    wait_loads_and_barrier<0>();  // this step's tiles are in LDS; every wave is done with the other buffer
    if (t + 1 < steps) {
      dma_step_narrow<TM>(a, wk.m0, wk.n0, wk.k_begin + (t + 1) * kTileK, xs[buf ^ 1], ws[buf ^ 1], wave, lane);
    }
    bf16x8 fa[4][FI], fb[4];
#pragma unroll
    for (int kk = 0; kk < kTileK / 16; ++kk) {
#pragma unroll
      for (int i = 0; i < FI; ++i) fa[kk][i] = as_bf16x8(xs[buf][slot(32 * i + r32, 2 * kk + half)]);
      fb[kk] = as_bf16x8(ws[buf][slot(32 * wave + r32, 2 * kk + half)]);
    }
#pragma unroll
    for (int kk = 0; kk < kTileK / 16; ++kk) {
#pragma unroll
      for (int i = 0; i < FI; ++i) acc[i] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[kk][i], fb[kk], acc[i], 0, 0, 0);
    }
  }
  // acc[i][r]: row 32 i + 8 (r / 4) + 4 half + r % 4 of the tile, column
  // 32 wave + r32
  const bool split = a.part != nullptr;
  float* out = split ? a.part + static_cast<int64_t>(wk.split) * a.m * a.n : a.y;
  const int64_t col = wk.n0 + 32 * wave + r32;
  if (col >= a.n) return;
  const bool add = !split && a.bias != nullptr;
  const bool accumulate = !split && a.accumulate;
  const float bv = add ? a.bias[col] : 0.0f;
#pragma unroll
  for (int i = 0; i < FI; ++i) {
    const int64_t row0 = wk.m0 + 32 * i + 4 * half;
    if constexpr (kEpi != Epi::kPlain) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = row0 + 8 * (r / 4) + (r % 4);
        if (row < a.m) store_act<kEpi>(a, row, col, add ? acc[i][r] + bv : acc[i][r]);
      }
      continue;
    }
    if (a.row_map != nullptr) {
      float val[16];
#pragma unroll
      for (int r = 0; r < 16; ++r) val[r] = acc[i][r];
      store_mapped(a, row0, col, bv, add, val);
      continue;
    }
    float* const o = out + row0 * a.n + col;
    auto live = [&](int r) { return row0 + 8 * (r / 4) + (r % 4) < a.m; };
    auto off = [&](int r) { return static_cast<int64_t>(8 * (r / 4) + (r % 4)) * a.n; };
    float base[16];
#pragma unroll
    for (int r = 0; r < 16; ++r) base[r] = accumulate && live(r) ? o[off(r)] : 0.0f;
#pragma unroll
    for (int r = 0; r < 16; ++r) {
      if (live(r)) {
        const float v = add ? acc[i][r] + bv : acc[i][r];
        o[off(r)] = accumulate ? base[r] + v : v;
      }
    }
  }
}

__global__ __launch_bounds__(kBlock) void round_bf16_k(const float* __restrict__ src, int64_t n,
                                                        uint16_t* __restrict__ dst) {
  const int64_t i = (static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x) * 8;
  if (i + 8 <= n) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(src + i), hi = *reinterpret_cast<const u32x4*>(src + i + 4);
    *reinterpret_cast<u32x4*>(dst + i) = u32x4{pack_bf16(__uint_as_float(lo.x), __uint_as_float(lo.y)),
                                               pack_bf16(__uint_as_float(lo.z), __uint_as_float(lo.w)),
                                               pack_bf16(__uint_as_float(hi.x), __uint_as_float(hi.y)),
                                               pack_bf16(__uint_as_float(hi.z), __uint_as_float(hi.w))};
  } else {
    for (int64_t j = i; j < n; ++j) dst[j] = f32_to_bf16(src[j]);
  }
}

// Products of at most this many rows take the 32-row tiles (bf16 x, k a
// multiple of 64), splitting k below this many of those tiles when k is at
// least 2048 (measured at 257 rows: k 4096 runs 2.5x faster split 16 ways,
// k 1024 loses 20-30% split 3-4 ways).
constexpr int64_t kNarrowRows = 512;
constexpr int64_t kNarrowSplitBelow = 256;
// Products of more rows whose 128 x 128 tiles are fewer than this (two
// workgroups per CU), and that would not split k, take 64 x 128 tiles:
// twice the workgroups, a shorter tail (the decoder's [4096 <- 1280] -> 1280,
// 320 tiles: 35.7 -> 32.2 us).
constexpr int64_t kMediumTilesBelow = 512;

}  // namespace

// The splits of k worth taking for an m x n x k product: a product of
// fewer than 64 tiles with k >= 1024 (of 32-row tiles: fewer than 256 with
// k >= 2048) gets enough workgroups to cover the 256 CUs twice, each split
// at least 4 steps of 64 columns; any other runs unsplit. (Measured at the
// vision encoder's shapes: 16-24 tiles with k of 2304-4608 run 1.3-1.9x
// faster split; 72-234 tiles, or k of 768-1024, lose 5-100% to the partial
// sums' traffic and the extra launch.)
int64_t splits_for(int64_t m, int64_t k, int64_t n, bool narrow = false) {
  const int64_t tile_rows = narrow ? kNarrowM : kTileM;
  const int64_t tiles = ((m + tile_rows - 1) / tile_rows) * ((n + kTileN - 1) / kTileN);
  if (tiles >= (narrow ? kNarrowSplitBelow : 64) || k < (narrow ? 32 : 16) * kTileK) return 1;
  int64_t s = (512 + tiles - 1) / tiles;
  s = s < k / (4 * kTileK) ? s : k / (4 * kTileK);
  return s < 32 ? s : 32;
}

// The bf16-x kernels that read their tiles straight into LDS (k a multiple
// of 64, x and w 16-byte aligned).
template <Epi kEpi>
void launch_tiles(const LinearArgs& a, unsigned grid, hipStream_t st, bool narrow, bool medium) {
  if (narrow) {
    linear_narrow_k<kNarrowM, kEpi><<<grid, kGemmThreads, 0, st>>>(a);
  } else if (medium) {
    linear_narrow_k<2 * kNarrowM, kEpi><<<grid, kGemmThreads, 0, st>>>(a);
  } else {
    linear_dma_k<kEpi><<<grid, kGemmThreads, 0, st>>>(a);
  }
}

int linear_entry(const char* what, void* stream, const void* x, bool f32x, int64_t m, int64_t k, const uint16_t* w,
                 int64_t n, const float* bias, float* y, float* workspace = nullptr, int64_t workspace_floats = 0,
                 bool accumulate = false, const int64_t* row_map = nullptr, int64_t y_rows = 0,
                 Epi epi = Epi::kPlain, uint16_t* y16 = nullptr) {
  UOCR_REQUIRE(m >= 0 && n >= 0 && k >= 0, what, "m, n and k must be >= 0");
  if (m == 0 || n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(k >= 1 && k < (int64_t{1} << 30), what, "k must be in [1, 2^30)");
  UOCR_REQUIRE(x != nullptr && w != nullptr && (epi == Epi::kPlain ? y != nullptr : y16 != nullptr), what,
               "null x, w or y");
  // products of bf16 rows with no epilogue beyond the bias (and the add
  // into y) go to the BLAS library when it takes them
  if (!f32x && epi == Epi::kPlain && row_map == nullptr) {
    const int st =
        library_linear_bf16(what, as_stream(stream), static_cast<const uint16_t*>(x), m, k, w, n, bias, y, accumulate);
    if (st != kLibraryDeclined) return st;
  }
  const bool ragged = k % 8 != 0 || !aligned16(x) || !aligned16(w);
  const bool dma = !ragged && !f32x && k % kTileK == 0;
  const int64_t tiles128 = ((m + kTileM - 1) / kTileM) * ((n + kTileN - 1) / kTileN);
  const bool narrow = dma && m <= kNarrowRows;
  // 64-row tiles where the 128-row ones are too few and would not be split
  // (and always with a row map)
  const bool medium = dma && !narrow &&
                      (row_map != nullptr ||
                       (tiles128 < kMediumTilesBelow && (workspace == nullptr || splits_for(m, k, n) == 1)));
  const int64_t tile_rows = narrow ? kNarrowM : medium ? 2 * kNarrowM : kTileM;
  const int64_t tiles_m = (m + tile_rows - 1) / tile_rows, tiles_n = (n + kTileN - 1) / kTileN;
  UOCR_REQUIRE(tiles_m * tiles_n < (int64_t{1} << 31), what, "too many tiles");
  // split k into the workspace when it holds the partial products
  int64_t splits =
      workspace != nullptr && !medium && row_map == nullptr && epi == Epi::kPlain ? splits_for(m, k, n, narrow) : 1;
  if (splits > 1 && workspace_floats < splits * m * n) splits = 1;
  const int64_t k_len = splits > 1 ? (k / splits + kTileK - 1) / kTileK * kTileK : k;
  splits = (k + k_len - 1) / k_len;
  UOCR_REQUIRE(tiles_m * tiles_n * splits < (int64_t{1} << 31), what, "too many tiles");
  LinearArgs a{x,
               w,
               bias,
               y,
               m,
               n,
               static_cast<int>(k),
               static_cast<int>(tiles_m),
               static_cast<int>(tiles_n),
               static_cast<int>(k_len),
               splits > 1 ? workspace : nullptr,
               accumulate,
               row_map,
               y_rows,
               y16};
  const unsigned grid = static_cast<unsigned>(tiles_m * tiles_n * splits);
  clear_launch_error();
  const hipStream_t st = as_stream(stream);
  if (ragged) {
    if (f32x) {
      linear_staged_k<true, true><<<grid, kGemmThreads, 0, st>>>(a);
    } else {
      linear_staged_k<false, true><<<grid, kGemmThreads, 0, st>>>(a);
    }
  } else if (f32x) {
    linear_staged_k<true, false><<<grid, kGemmThreads, 0, st>>>(a);
  } else if (epi == Epi::kGeluBf16) {
    launch_tiles<Epi::kGeluBf16>(a, grid, st, narrow, medium);
  } else if (epi == Epi::kQuickGeluBf16) {
    launch_tiles<Epi::kQuickGeluBf16>(a, grid, st, narrow, medium);
  } else if (k % kTileK == 0) {
    launch_tiles<Epi::kPlain>(a, grid, st, narrow, medium);
  } else {
    linear_staged_k<false, false><<<grid, kGemmThreads, 0, st>>>(a);
  }
  if (splits > 1) {
    const int64_t blocks = (m * n + kBlock - 1) / kBlock;
    split_sum_k<<<static_cast<unsigned>(blocks < 65536 ? blocks : 65536), kBlock, 0, st>>>(
        workspace, static_cast<int>(splits), m, n, bias, y, accumulate);
  }
  return check_launch(what);
}

}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_linear(void* stream, const float* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                     const float* bias, float* y) {
  // One row streams the weights once through the GEMV (the reference's
  // m == 1 path, ops.cu:271-274).
  if (m == 1 && k % 8 == 0 && k <= 12288 && aligned16(x) && aligned16(w)) {
    return uocr_rocm_gemv_bf16(stream, x, k, w, n, bias, y);
  }
  return linear_entry("uocr_rocm_linear", stream, x, true, m, k, w, n, bias, y);
}

int uocr_rocm_linear_bf16x(void* stream, const uint16_t* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                           const float* bias, float* y) {
  return linear_entry("uocr_rocm_linear_bf16x", stream, x, false, m, k, w, n, bias, y);
}

int64_t uocr_rocm_linear_workspace_floats(int64_t m, int64_t k, int64_t n) {
  if (m <= 1 || n <= 0 || k <= 0) return 0;
  // enough for either tiling a product of few rows may take
  int64_t s = splits_for(m, k, n);
  if (m <= kNarrowRows) {
    const int64_t sn = splits_for(m, k, n, true);
    s = sn > s ? sn : s;
  }
  return s > 1 ? s * m * n : 0;
}

int uocr_rocm_linear_ws(void* stream, const float* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                        const float* bias, float* y, float* workspace, int64_t workspace_floats) {
  if (m == 1 && k % 8 == 0 && k <= 12288 && aligned16(x) && aligned16(w)) {
    return uocr_rocm_gemv_bf16(stream, x, k, w, n, bias, y);
  }
  return linear_entry("uocr_rocm_linear_ws", stream, x, true, m, k, w, n, bias, y, workspace, workspace_floats);
}

int uocr_rocm_linear_bf16x_ws(void* stream, const uint16_t* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                              const float* bias, float* y, float* workspace, int64_t workspace_floats) {
  return linear_entry("uocr_rocm_linear_bf16x_ws", stream, x, false, m, k, w, n, bias, y, workspace,
                      workspace_floats);
}

int uocr_rocm_linear_bf16x_add_ws(void* stream, const uint16_t* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                                  const float* bias, float* y, float* workspace, int64_t workspace_floats) {
  return linear_entry("uocr_rocm_linear_bf16x_add_ws", stream, x, false, m, k, w, n, bias, y, workspace,
                      workspace_floats, true);
}

int uocr_rocm_linear_bf16x_add_rows(void* stream, const uint16_t* x, int64_t m, int64_t k, const uint16_t* w,
                                    int64_t n, const float* bias, float* y, const int64_t* y_row, int64_t y_rows) {
  constexpr const char* kWhat = "uocr_rocm_linear_bf16x_add_rows";
  UOCR_REQUIRE(y_row != nullptr || m == 0, kWhat, "null row map");
  UOCR_REQUIRE(y_rows >= 0, kWhat, "y_rows must be >= 0");
  UOCR_REQUIRE(k % kTileK == 0 && aligned16(x) && aligned16(w), kWhat,
               "k must be a multiple of 64 and x, w 16-byte aligned");
  return linear_entry(kWhat, stream, x, false, m, k, w, n, bias, y, nullptr, 0, true, y_row, y_rows);
}

int uocr_rocm_linear_bf16x_gelu_erf_bf16(void* stream, const uint16_t* x, int64_t m, int64_t k, const uint16_t* w,
                                         int64_t n, const float* bias, uint16_t* y) {
  constexpr const char* kWhat = "uocr_rocm_linear_bf16x_gelu_erf_bf16";
  UOCR_REQUIRE(k % kTileK == 0 && aligned16(x) && aligned16(w), kWhat,
               "k must be a multiple of 64 and x, w 16-byte aligned");
  return linear_entry(kWhat, stream, x, false, m, k, w, n, bias, nullptr, nullptr, 0, false, nullptr, 0,
                      Epi::kGeluBf16, y);
}

int uocr_rocm_linear_bf16x_quick_gelu_bf16(void* stream, const uint16_t* x, int64_t m, int64_t k,
                                           const uint16_t* w, int64_t n, const float* bias, uint16_t* y) {
  constexpr const char* kWhat = "uocr_rocm_linear_bf16x_quick_gelu_bf16";
  UOCR_REQUIRE(k % kTileK == 0 && aligned16(x) && aligned16(w), kWhat,
               "k must be a multiple of 64 and x, w 16-byte aligned");
  return linear_entry(kWhat, stream, x, false, m, k, w, n, bias, nullptr, nullptr, 0, false, nullptr, 0,
                      Epi::kQuickGeluBf16, y);
}

int uocr_rocm_round_bf16(void* stream, const float* src, int64_t n, uint16_t* dst) {
  constexpr const char* kWhat = "uocr_rocm_round_bf16";
  UOCR_REQUIRE(n >= 0, kWhat, "n must be >= 0");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(src != nullptr && dst != nullptr, kWhat, "null pointer");
  UOCR_REQUIRE(aligned16(src) && aligned16(dst), kWhat, "src and dst must be 16-byte aligned");
  const int64_t blocks = (n + 8 * kBlock - 1) / (8 * kBlock);
  UOCR_REQUIRE(blocks < (int64_t{1} << 31), kWhat, "n too large");
  clear_launch_error();
  round_bf16_k<<<static_cast<unsigned>(blocks), kBlock, 0, as_stream(stream)>>>(src, n, dst);
  return check_launch(kWhat);
}

}  // extern "C"
