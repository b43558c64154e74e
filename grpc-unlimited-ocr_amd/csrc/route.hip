// route.hip: the block router of sparse decode attention for gfx950, fp32.
//
// Keys are grouped into blocks of block_size router keys (rk rows of d
// floats). A block's summary is the softmax(clamp(rk . head_cls / sqrt d))-
// weighted mean of its keys. A query (router query rq, position pos) scores
// the blocks that end before its local window (b <= pos / block_size -
// local_blocks), z_b = rq . S_b / sqrt d, clamped; restricted to the blocks
// that hold image tokens of the query's page when the prompt's block pages
// say so, the best top_m scores (times idx_scale) go through 1.5-entmax and
// the first top_k are read with a log-prior bias. The query's key mask is 0
// on its local window, the bias on the keys of a selected block and -inf on
// every other key (references: src/model/block_router.cpp:20-154,
// src/model/attention_plan.cpp:34-56, src/model/decoder.cpp:42-56, and the
// device forms src/backend/cuda/decode_ops.cu:57-110, ops.cu:419-561).
//
// Entry points: block_summaries (every block of a prompt), summary_step /
// scores_step / route_step (one decode query, lengths from the StepState),
// route_blocks (prompt rows), and route_decode_step, the whole router half of
// a decode step in one launch: the router norm of rq and rk, rope at the
// step's coordinate, the append of rk, the summary of the block holding pos,
// the scores and the route into the mask.
//
// Arithmetic: every product and sum here is rounded on its own (no FMA
// contraction), and the stage functions below are the same code in every
// entry point, so the one-launch route_decode_step gives bitwise what the
// separate steps give. The selection order is the reference's: descending
// score, the lower block first on a tie. Exponentials and logarithms are the
// device library's expf and logf; sqrtf and division are correctly rounded,
// as in the reference, so 1.5-entmax reproduces its fp32 steps exactly.

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int kRouteBlock = 1024;  // 16 waves
constexpr int kMaxBlockKeys = 64;  // block_size
constexpr int kMaxIndexDim = 256;  // d
constexpr int kStageFloats = 8192;  // block_size * d: one block's keys staged in LDS
constexpr int kMaxTop = 32;        // top_m
constexpr int64_t kMaxRouteBlocks = 4096;  // blocks per query row
constexpr float kEntmaxMasked = -1.0e4f;
constexpr float kActClamp = 1.0e4f;

__device__ __forceinline__ float clamp_act(float v) { return fminf(fmaxf(v, -kActClamp), kActClamp); }

struct RouteArgs {
  int block_size;
  int local_blocks;
  int top_m;
  int top_k;
  float idx_scale;
  float floor;
  float sigma;
};

// ---- stages shared by every entry point ----------------------------------------------------

__device__ __forceinline__ float readlane_f32(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Inclusive sums over lanes 0..lane in lane order: lane j gets the fp32 sum
// ((v_0 + v_1) + ...) + v_j, for lanes j <= kSteps. kSteps unrolled steps of
// s = v + (s of the lane below, through a one-lane DPP shift; lane 0 reads
// 0); after step t the first t + 1 lanes hold their final sums, and as fp32
// addition commutes, v_j + s_(j-1) equals s_(j-1) + v_j bit for bit. Every
// lane of the wave must be active.
template <int kSteps>
__device__ __forceinline__ float prefix_in_order(float v) {
#pragma clang fp contract(off)
  float s = v;
#pragma unroll
  for (int t = 0; t < kSteps; ++t) s = v + dpp_f32<0x138>(s);  // wave_shr:1
  return s;
}


// head_cls as summarize takes it: lane l holds features l, l + 64, l + 128,
// l + 192 (zero past d).
__device__ __forceinline__ void load_cls(const float* __restrict__ cls, int d, float (&c)[4]) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int i = 0; i < 4; ++i) c[i] = lane + kWave * i < d ? cls[lane + kWave * i] : 0.0f;
}

// The summary of one block whose n keys (1 <= n <= kMaxBlockKeys) sit in
// LDS, row-major with row stride d: out[e] = sum_t (w_t / total) key_t[e],
// w_t = exp(a_t - max a), a_t = clamp(key_t . cls / sqrt d), total =
// max(sum_t w_t, 1e-6). Wave w forms the logits of keys w, w + waves, ...
// (lane e takes features e, e + 64, ...); wave 0 then holds a_t in lane t,
// and total and the feature sums run over t in order. `p` is kMaxBlockKeys
// floats of LDS. Every thread of the block must call it.
__device__ void summarize(const float* keys, int n, int d, const float (&cls)[4], float inv_sqrt_d, float* p,
                          float* __restrict__ out) {
#pragma clang fp contract(off)
  const int wave = wave_in_block(), lane = threadIdx.x & (kWave - 1);
  const int waves = static_cast<int>(blockDim.x) / kWave;
  for (int t = wave; t < n; t += waves) {
    float part = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      if (lane + kWave * i < d) part += keys[t * d + lane + kWave * i] * cls[i];
    }
    const float a = wave_sum(part);
    if (lane == 0) p[t] = clamp_act(a * inv_sqrt_d);
  }
  lds_barrier();
  if (wave == 0) {
    const float a = lane < n ? p[lane] : -3.402823466e+38f;
    const float peak = wave_max(a);
    const float w = lane < n ? expf(a - peak) : 0.0f;
    // the sum over t in order (lanes past n hold +0, which adds nothing)
    float total = n <= 32 ? readlane_f32(prefix_in_order<31>(w), 31) : readlane_f32(prefix_in_order<kWave - 1>(w), kWave - 1);
    total = fmaxf(total, 1e-6f);
    if (lane < n) p[lane] = w / total;
  }
  lds_barrier();
  for (int e = threadIdx.x; e < d; e += blockDim.x) {
    float acc = 0.0f;
#pragma unroll 8
    for (int t = 0; t < n; ++t) acc += p[t] * keys[t * d + e];
    out[e] = acc;
  }
}

// Block scores. Each lane takes eight 16-byte chunks of a summary row (32
// features, past d zero), so a row spans L = d / 32 lanes (rounded up to 1,
// 2, 4 or 8) and a wave reads 64 / L rows per pass. Lane c of a row takes
// chunks c, c + L, c + 2 L, ..., so each load instruction reads L adjacent
// chunks of every row; the lane sums its products in that order and the
// row's L lanes add by DPP butterfly. All of a pass's loads are in flight
// together. (Four features per lane over 32 lanes spent most of the time in
// per-row butterflies and readlanes.)
constexpr int kScoreChunks = 8;  // 16-byte chunks per lane

struct ScoreRows {
  u32x4 row[kScoreChunks];
};

__device__ __forceinline__ int score_lanes(int d) { return d <= 32 ? 1 : (d <= 64 ? 2 : (d <= 128 ? 4 : 8)); }

// Rows per pass: waves * (64 / L).
__device__ __forceinline__ int score_pass_rows(int d) {
  return static_cast<int>(blockDim.x) / kWave * (kWave / score_lanes(d));
}

// Issues the loads of the pass starting at row `base` (rows < n).
__device__ __forceinline__ void score_load(const float* __restrict__ summaries, int d, int n, int base,
                                           ScoreRows& s) {
  const int wave = wave_in_block(), lane = threadIdx.x & (kWave - 1);
  const int L = score_lanes(d), R = kWave / L, sub = lane / L, c = lane & (L - 1);
  const int b = base + wave * R + sub;
  const float* row = summaries + static_cast<int64_t>(b) * d;
#pragma unroll
  for (int i = 0; i < kScoreChunks; ++i) {
    const int f = 4 * (c + L * i);  // the chunk's first feature
    s.row[i] = u32x4{0u, 0u, 0u, 0u};
    if (b < n && f < d) s.row[i] = *reinterpret_cast<const u32x4*>(row + f);
  }
}

// z[b] = (rq . summaries[b]) / sqrt d for the pass's rows b < n (unclamped),
// rq [d] in LDS. Each dot is summed as a lane's products in its chunks'
// order, then over the row's lanes in a fixed order, the same for every
// entry point.
__device__ __forceinline__ void score_reduce(const float* rq, int d, int n, int base, float inv_sqrt_d,
                                             const ScoreRows& s, float* z) {
#pragma clang fp contract(off)
  const int wave = wave_in_block(), lane = threadIdx.x & (kWave - 1);
  const int L = score_lanes(d), R = kWave / L, sub = lane / L, c = lane & (L - 1);
  const int b0 = base + wave * R;  // wave-uniform
  if (b0 >= n) return;
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < kScoreChunks; ++i) {
    const int f = 4 * (c + L * i);
    if (f < d) {
      const float* q = rq + f;
      part += q[0] * __uint_as_float(s.row[i].x);
      part += q[1] * __uint_as_float(s.row[i].y);
      part += q[2] * __uint_as_float(s.row[i].z);
      part += q[3] * __uint_as_float(s.row[i].w);
    }
  }
  if (L >= 2) part += dpp_f32<0xB1>(part);   // lane ^ 1
  if (L >= 4) part += dpp_f32<0x4E>(part);   // lane ^ 2
  if (L >= 8) part += dpp_f32<0x141>(part);  // the two quads of each 8 lanes
  const int b = b0 + sub;
  if (c == 0 && b < n) z[b] = part * inv_sqrt_d;
}

// z[b] for b < n, pass by pass. Every thread of the block must call it.
__device__ void score_blocks(const float* rq, const float* __restrict__ summaries, int d, int n, float inv_sqrt_d,
                             float* z) {
  const int step = score_pass_rows(d);
  for (int base = 0; base < n; base += step) {
    ScoreRows s;
    score_load(summaries, d, n, base, s);
    score_reduce(rq, d, n, base, inv_sqrt_d, s, z);
  }
}

// Block-order key of a candidate score for the top-m: larger scores first,
// then the lower block index (all scores are finite here; 0 is below every
// key and marks an empty slot).
__device__ __forceinline__ uint64_t order_key(float v, int b) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<uint64_t>(u) << 32) | (0xffffffffu - static_cast<uint32_t>(b));
}

__device__ __forceinline__ float key_value(uint64_t key) {
  const uint32_t u = static_cast<uint32_t>(key >> 32);
  return __uint_as_float((u & 0x80000000u) ? (u & 0x7fffffffu) : ~u);
}

__device__ __forceinline__ int key_block(uint64_t key) {
  return static_cast<int>(0xffffffffu - static_cast<uint32_t>(key));
}

template <int kCtrl>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {
  const uint32_t lo = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v)), kCtrl, 0xF, 0xF, false));
  const uint32_t hi = static_cast<uint32_t>(
      __builtin_amdgcn_update_dpp(0, static_cast<int>(static_cast<uint32_t>(v >> 32)), kCtrl, 0xF, 0xF, false));
  return (static_cast<uint64_t>(hi) << 32) | lo;
}

template <int kCtrl>
__device__ __forceinline__ uint32_t dpp_u32(uint32_t v) {
  return static_cast<uint32_t>(__builtin_amdgcn_update_dpp(0, static_cast<int>(v), kCtrl, 0xF, 0xF, false));
}

// The wave's largest of v (unsigned), in every lane: a DPP butterfly inside
// each 16-lane row, then the four row maxima. Every lane must be active.
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
  auto umax = [](uint32_t x, uint32_t y) { return x > y ? x : y; };
  v = umax(v, dpp_u32<0xB1>(v));   // lane ^ 1
  v = umax(v, dpp_u32<0x4E>(v));   // lane ^ 2
  v = umax(v, dpp_u32<0x141>(v));  // row_half_mirror
  v = umax(v, dpp_u32<0x140>(v));  // row_mirror
  const uint32_t r0 = __builtin_amdgcn_readlane(static_cast<int>(v), 0);
  const uint32_t r1 = __builtin_amdgcn_readlane(static_cast<int>(v), 16);
  const uint32_t r2 = __builtin_amdgcn_readlane(static_cast<int>(v), 32);
  const uint32_t r3 = __builtin_amdgcn_readlane(static_cast<int>(v), 48);
  return umax(umax(r0, r1), umax(r2, r3));
}

// The m largest of the wave's keys (S per lane, m <= 64): lane j returns the
// j-th largest (0 past the wave's keys). Each lane sorts its S keys, then m
// rounds take the largest head and the winning lane drops it. A round finds
// the largest high word (the score); the low word (the block) decides only
// between lanes whose heads share it, the common single holder taking a
// readlane instead. Keys are distinct apart from empty slots (0), so the
// winner is the lane holding the wave's largest key.
template <int S>
__device__ __forceinline__ uint64_t wave_top(uint64_t (&key)[S], int m, int lane) {
#pragma unroll
  for (int i = 0; i < S; ++i) {
#pragma unroll
    for (int j = 0; j + 1 < S - i; ++j) {
      const uint64_t a = key[j], b = key[j + 1];
      key[j] = a > b ? a : b;
      key[j + 1] = a > b ? b : a;
    }
  }
  uint32_t hi[S], lo[S];
#pragma unroll
  for (int i = 0; i < S; ++i) {
    hi[i] = static_cast<uint32_t>(key[i] >> 32);
    lo[i] = static_cast<uint32_t>(key[i]);
  }
  uint64_t mine = 0;
  for (int j = 0; j < m; ++j) {
    const uint32_t top = wave_max_u32(hi[0]);
    const uint64_t tied = __ballot(hi[0] == top);
    uint32_t top_lo;
    int winner;
    if ((tied & (tied - 1)) == 0) {
      winner = __builtin_ctzll(tied);
      top_lo = __builtin_amdgcn_readlane(static_cast<int>(lo[0]), winner);
    } else {
      top_lo = wave_max_u32(hi[0] == top ? lo[0] : 0u);
      winner = __builtin_ctzll(__ballot(hi[0] == top && lo[0] == top_lo));
    }
    if (lane == j) mine = (static_cast<uint64_t>(top) << 32) | top_lo;
    if (lane == winner) {
#pragma unroll
      for (int i = 0; i + 1 < S; ++i) {
        hi[i] = hi[i + 1];
        lo[i] = lo[i + 1];
      }
      hi[S - 1] = 0;
      lo[S - 1] = 0;
    }
  }
  return mine;
}

// LDS working set of the route of one query row: x the blocks' entmax
// inputs (it may be the z array itself: each thread reads z[b] before it
// writes x[b]), cand the candidate flags, block_bias the mask value of a
// block's keys outside the window, and list the per-wave top-m keys (16
// waves x kMaxTop).
struct RouteLds {
  float* x;             // [nblk]
  unsigned char* cand;  // [nblk]
  float* block_bias;    // [nblk]
  uint64_t* list;       // [16 * kMaxTop]
  int* any;             // [16]
};

// The prompt blocks' page ranges of the blocks this thread owns (b =
// threadIdx.x + kRouteBlock i, i < 4; -1 where a block has no range or the
// query no page).
constexpr int kBlocksPerThread = static_cast<int>(kMaxRouteBlocks) / kRouteBlock;

struct PageRanges {
  int64_t lo[kBlocksPerThread], hi[kBlocksPerThread];
};

__device__ __forceinline__ void load_pages(const int64_t* __restrict__ block_min,
                                           const int64_t* __restrict__ block_max, int64_t prompt_blocks, int nblk,
                                           int64_t page, PageRanges& r) {
#pragma unroll
  for (int i = 0; i < kBlocksPerThread; ++i) {
    const int b = static_cast<int>(threadIdx.x) + kRouteBlock * i;
    r.lo[i] = -1;
    r.hi[i] = -1;
    if (page >= 0 && b < nblk && b < prompt_blocks) {
      r.lo[i] = block_min[b];
      r.hi[i] = block_max[b];
    }
  }
}

// cand[b], b < nblk: remote (b <= last_remote) and, for a query on a page,
// one of the page's prompt blocks; a query whose page has no remote block
// routes over every remote block (decoder.cpp:42-56). In two halves around
// a workgroup LDS barrier the caller places: the first writes the flags of
// this thread's blocks and its wave's vote into slots (kRouteBlock / 64
// ints); the second reads the votes and, with none, applies the fallback to
// this thread's blocks. Every thread of a kRouteBlock block must call both.
__device__ __forceinline__ void route_candidates_begin(const PageRanges& r, int nblk, int64_t last_remote,
                                                       int64_t page, unsigned char* cand, int* slots) {
  int any_local = 0;
#pragma unroll
  for (int i = 0; i < kBlocksPerThread; ++i) {
    const int b = static_cast<int>(threadIdx.x) + kRouteBlock * i;
    if (b < nblk) {
      const bool remote = b <= last_remote;
      const bool allowed = page >= 0 && r.lo[i] >= 0 && r.lo[i] <= page && page <= r.hi[i];
      cand[b] = remote && allowed;
      any_local |= remote && allowed;
    }
  }
  const uint64_t lanes = __ballot(any_local != 0);
  if ((threadIdx.x & (kWave - 1)) == 0) slots[wave_in_block()] = lanes != 0;
}

__device__ __forceinline__ void route_candidates_end(int nblk, int64_t last_remote, unsigned char* cand,
                                                     const int* slots) {
  int any = 0;
#pragma unroll
  for (int w = 0; w < kRouteBlock / kWave; ++w) any |= slots[w];
  if (any == 0) {
#pragma unroll
    for (int i = 0; i < kBlocksPerThread; ++i) {
      const int b = static_cast<int>(threadIdx.x) + kRouteBlock * i;
      if (b < nblk) cand[b] = b <= last_remote;
    }
  }
}

__device__ __forceinline__ void route_candidates(const PageRanges& r, int nblk, int64_t last_remote, int64_t page,
                                                 unsigned char* cand, int* slots) {
  route_candidates_begin(r, nblk, last_remote, page, cand, slots);
  lds_barrier();
  route_candidates_end(nblk, last_remote, cand, slots);
}

// The selection and the key mask of one query at position pos over nblk
// blocks (z[b], raw scores of the blocks b <= last_remote; other entries are
// not read), given cand: x = clamp(z) * idx_scale on candidates and -1e4
// elsewhere; the top m = clamp(top_m, 1, nblk) by (x desc, block asc)
// through 1.5-entmax (block_router.cpp:68-91: the running sums in order,
// each tau and the support in its own lane); the first k = clamp(top_k, 1,
// m) with their log-prior bias (logp - mean over the valid ones) / sigma
// (block_router.cpp:131-151); then mask[0..keys): 0 on the local window,
// the bias on the keys of a valid selected block, -inf elsewhere and past
// pos (attention_plan.cpp:34-56). Every thread of a kRouteBlock block must
// call it.
// segs (decode only; null: none) receives the keys the mask keeps as
// segments in ascending key order (the key segments of uocr_rocm.h); with
// segs, mask may be null (not written).
// words 0 and 1 the segment count and the live key count, then per segment
// {first key, keys, bias bits, 0}: the valid selections by block, each
// clipped at the local window and at pos, then the window itself.
__device__ void route_select(const float* z, int nblk, int64_t pos, int64_t keys, const RouteArgs p, RouteLds sh,
                             float* __restrict__ mask, int* __restrict__ segs = nullptr) {
#pragma clang fp contract(off)
  constexpr int kSlice = 4 * kWave;  // blocks per wave
  // With nblk <= kSlice the top m goes by rank (below), whose keys, counts
  // and result slots are set here, before the same barrier.
  static_assert(kRouteBlock == 4 * kSlice, "four quarters of the blocks");
  uint64_t* key_of = sh.list;                            // [kSlice]
  int* rank = reinterpret_cast<int*>(sh.list + kSlice);  // [kSlice]
  uint64_t* top = sh.list + kSlice + kSlice / 2;         // [kMaxTop]
  const int t = static_cast<int>(threadIdx.x);
#pragma unroll
  for (int i = 0; i < kBlocksPerThread; ++i) {
    const int b = t + kRouteBlock * i;
    if (b < nblk) {
      const float xb = sh.cand[b] ? clamp_act(z[b]) * p.idx_scale : kEntmaxMasked;
      sh.x[b] = xb;
      sh.block_bias[b] = -INFINITY;
      if (i == 0 && nblk <= kSlice) key_of[b] = order_key(xb, b);
    }
  }
  if (nblk <= kSlice && t < kSlice) {
    if (t >= nblk) key_of[t] = 0;
    rank[t] = 0;
    if (t < kMaxTop) top[t] = 0;
  }
  lds_barrier();

  const int m = p.top_m < nblk ? (p.top_m > 1 ? p.top_m : 1) : (nblk > 1 ? nblk : 1);
  const int k = p.top_k < m ? (p.top_k > 1 ? p.top_k : 1) : m;
  const int wave = wave_in_block(), lane = threadIdx.x & (kWave - 1);
  uint64_t mine = 0;
  if (nblk <= kSlice) {
    // By rank: the keys are distinct, so a block's place in the order is
    // the count of keys above it. Thread (q, b) counts the keys of quarter q
    // above block b's; the quarters' counts add in LDS, and each block with
    // a rank below m puts its key at that rank.
    // the slots past nblk hold 0, below every key, so every thread counts
    // its quarter's 64 slots with the same unrolled loop (LDS broadcasts)
    const int b = t & (kSlice - 1);
    const int q = __builtin_amdgcn_readfirstlane(t / kSlice);
    const uint64_t own = key_of[b];
    const uint64_t* quarter = key_of + q * (kSlice / 4);
    int above = 0;
#pragma unroll
    for (int j = 0; j < kSlice / 4; j += 2) {
      const u32x4 two = *reinterpret_cast<const u32x4*>(quarter + j);
      const uint64_t k0 = (static_cast<uint64_t>(two.y) << 32) | two.x;
      const uint64_t k1 = (static_cast<uint64_t>(two.w) << 32) | two.z;
      above += (k0 > own ? 1 : 0) + (k1 > own ? 1 : 0);
    }
    if (b < nblk) atomicAdd(&rank[b], above);
    lds_barrier();
    if (t < nblk && rank[t] < m) top[rank[t]] = key_of[t];
    lds_barrier();
    if (wave == 0 && lane < m) mine = top[lane];
  } else {
    // each wave's top m of its slice, then wave 0 takes the top m of those
    uint64_t key[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int b = wave * kSlice + lane + kWave * i;
      key[i] = b < nblk ? order_key(sh.x[b], b) : 0;
    }
    const uint64_t best = wave_top<4>(key, m, lane);
    if (lane < m) sh.list[wave * m + lane] = best;
    lds_barrier();
    if (wave == 0) {
      const int listed = static_cast<int>(blockDim.x) / kWave * m;
      uint64_t key8[8];
#pragma unroll
      for (int i = 0; i < 8; ++i) key8[i] = lane + kWave * i < listed ? sh.list[lane + kWave * i] : 0;
      mine = wave_top<8>(key8, m, lane);
    }
  }
  if (wave == 0) {
    // lane j < m holds the j-th selection
    const bool have = lane < m;
    const int blk = have ? key_block(mine) : 0;
    const float val = have ? key_value(mine) : 0.0f;
    const float peak = readlane_f32(val, 0);
    const float v = have ? (val - peak) / 2.0f : 0.0f;
    // running sums in lane order over the first m lanes (the later lanes'
    // sums are never read)
    auto prefix = [m](float x) { return m <= 16 ? prefix_in_order<15>(x) : prefix_in_order<kMaxTop - 1>(x); };
    const float sum = prefix(v), sum_sq = prefix(v * v);
    const float rho = static_cast<float>(lane + 1);
    const float mean = sum / rho, mean_sq = sum_sq / rho;
    const float ss = rho * (mean_sq - mean * mean);
    const float delta = fmaxf((1.0f - ss) / rho, 0.0f);
    const float tau = mean - sqrtf(delta);
    const int support = __popcll(__ballot(have && tau <= v));
    const float tau_star = readlane_f32(tau, (support > 1 ? support : 1) - 1);
    const float t = fmaxf(v - tau_star, 0.0f);
    const float prob = t * t;
    const bool valid = lane < k && sh.cand[blk] != 0;
    const float logp = logf(fmaxf(prob, p.floor));
    const float logp_sum = readlane_f32(prefix(valid ? logp : 0.0f), k - 1);
    const uint64_t vmask = __ballot(valid);
    const int count = __popcll(vmask);
    const float mu = logp_sum / static_cast<float>(count > 1 ? count : 1);
    const float bias = (logp - mu) / p.sigma;
    if (valid) sh.block_bias[blk] = bias;
    if (segs != nullptr) {
      const int64_t wkeys = static_cast<int64_t>(p.local_blocks) * p.block_size;
      const int64_t wfirst = pos - wkeys + 1 > 0 ? pos - wkeys + 1 : 0;  // first key of the window
      const int64_t wlen = wkeys > 0 ? pos - wfirst + 1 : 0;
      // this lane's rank among the valid selections, by block
      int rank = 0;
      for (int j = 0; j < k; ++j) {  // the valid lanes are among the first k
        const int bj = __builtin_amdgcn_readlane(blk, j);
        rank += ((vmask >> j) & 1) != 0 && bj < blk ? 1 : 0;
      }
      const int64_t first = static_cast<int64_t>(blk) * p.block_size;
      int64_t end = first + p.block_size;
      const int64_t stop = wkeys > 0 ? wfirst : pos + 1;  // remote keys end at the window (or at pos)
      end = end < stop ? end : stop;
      const int len = valid && end > first ? static_cast<int>(end - first) : 0;
      const int live = static_cast<int>(wave_sum(static_cast<float>(len))) + static_cast<int>(wlen);
      if (valid) {
        int* sg = segs + 4 * (1 + rank);
        sg[0] = static_cast<int>(first);
        sg[1] = len;
        sg[2] = __float_as_int(bias);
        sg[3] = 0;
      }
      if (lane == 0) {
        if (wlen > 0) {
          int* sg = segs + 4 * (1 + count);
          sg[0] = static_cast<int>(wfirst);
          sg[1] = static_cast<int>(wlen);
          sg[2] = __float_as_int(0.0f);
          sg[3] = 0;
        }
        segs[0] = count + (wlen > 0 ? 1 : 0);
        segs[1] = live;
      }
    }
  }
  lds_barrier();
  if (mask == nullptr) return;  // the segments alone (uniform)

  const int64_t window = static_cast<int64_t>(p.local_blocks) * p.block_size;
  const uint32_t bs = static_cast<uint32_t>(p.block_size);
  auto value = [&](int64_t j) {
    float v = -INFINITY;
    if (j <= pos) v = j > pos - window ? 0.0f : sh.block_bias[static_cast<uint32_t>(j) / bs];
    return v;
  };
  int64_t j0 = 0;
  if ((reinterpret_cast<uintptr_t>(mask) & 15u) == 0) {  // 16-byte stores
    const int64_t quads = keys / 4;
    for (int64_t c = threadIdx.x; c < quads; c += blockDim.x) {
      const u32x4 q{__float_as_uint(value(4 * c)), __float_as_uint(value(4 * c + 1)),
                    __float_as_uint(value(4 * c + 2)), __float_as_uint(value(4 * c + 3))};
      *reinterpret_cast<u32x4*>(mask + 4 * c) = q;
    }
    j0 = 4 * quads;
  }
  for (int64_t j = j0 + threadIdx.x; j < keys; j += blockDim.x) mask[j] = value(j);
}

// Routes one query row: its candidates, then route_select.
__device__ void route_row(const float* z, int nblk, int64_t pos, int64_t keys, int64_t page,
                          const int64_t* __restrict__ block_min, const int64_t* __restrict__ block_max,
                          int64_t prompt_blocks, const RouteArgs p, RouteLds sh, float* __restrict__ mask) {
  PageRanges r;
  load_pages(block_min, block_max, prompt_blocks, nblk, page, r);
  route_candidates(r, nblk, pos / p.block_size - p.local_blocks, page, sh.cand, sh.any);
  route_select(z, nblk, pos, keys, p, sh, mask);
}

// LDS for route_row in a kernel that routes one row and needs nothing else.
struct RouteShared {
  float x[kMaxRouteBlocks];
  unsigned char cand[kMaxRouteBlocks];
  float block_bias[kMaxRouteBlocks];
  uint64_t list[kRouteBlock / kWave * kMaxTop];
  int any[kRouteBlock / kWave];
  __device__ RouteLds lds() { return RouteLds{x, cand, block_bias, list, any}; }
};

// Stages rows [first, first + n) of router keys [*, d] into LDS (16-byte
// chunks; d % 4 == 0). Every thread of the block must call it.
__device__ void stage_keys(const float* __restrict__ rk, int64_t first, int n, int d, float* lds) {
  const int chunks = n * d / 4;
  const float* src = rk + first * d;
  for (int c = threadIdx.x; c < chunks; c += blockDim.x) {
    *reinterpret_cast<u32x4*>(lds + 4 * c) = *reinterpret_cast<const u32x4*>(src + 4 * c);
  }
}

// The same rows loaded into registers by a kRouteBlock block (n * d <=
// kStageFloats: at most two chunks per thread), stored to LDS later.
constexpr int kStageChunks = kStageFloats / 4 / kRouteBlock;

struct StagedKeys {
  u32x4 chunk[kStageChunks];
};

__device__ __forceinline__ void load_keys(const float* __restrict__ rk, int64_t first, int n, int d, StagedKeys& s) {
  const int chunks = n * d / 4;
  const float* src = rk + first * d;
#pragma unroll
  for (int i = 0; i < kStageChunks; ++i) {
    const int c = static_cast<int>(threadIdx.x) + kRouteBlock * i;
    s.chunk[i] = u32x4{0u, 0u, 0u, 0u};
    if (c < chunks) s.chunk[i] = *reinterpret_cast<const u32x4*>(src + 4 * c);
  }
}

__device__ __forceinline__ void store_keys(const StagedKeys& s, int n, int d, float* lds) {
  const int chunks = n * d / 4;
#pragma unroll
  for (int i = 0; i < kStageChunks; ++i) {
    const int c = static_cast<int>(threadIdx.x) + kRouteBlock * i;
    if (c < chunks) *reinterpret_cast<u32x4*>(lds + 4 * c) = s.chunk[i];
  }
}

// ---- kernels -------------------------------------------------------------------------------

// Every block of s keys: one workgroup per block.
__global__ __launch_bounds__(256) void block_summaries_k(const float* __restrict__ rk, int64_t s, int d,
                                                         const float* __restrict__ cls, int block_size,
                                                         float inv_sqrt_d, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float keys[kStageFloats];
  __shared__ float p[kMaxBlockKeys];
  const int64_t first = static_cast<int64_t>(blockIdx.x) * block_size;
  const int n = static_cast<int>(s - first < block_size ? s - first : block_size);
  float c[4];
  load_cls(cls, d, c);
  stage_keys(rk, first, n, d, keys);
  lds_barrier();
  summarize(keys, n, d, c, inv_sqrt_d, p, out + static_cast<int64_t>(blockIdx.x) * d);
}

// The summary of the block holding state->pos (keys first..pos).
__global__ __launch_bounds__(256) void summary_step_k(const float* __restrict__ rk, int d,
                                                      const float* __restrict__ cls, int block_size,
                                                      float inv_sqrt_d, const uocr_rocm_step_state* __restrict__ state,
                                                      int64_t max_blocks, float* __restrict__ summaries) {
  __shared__ __attribute__((aligned(16))) float keys[kStageFloats];
  __shared__ float p[kMaxBlockKeys];
  const int64_t pos = state->pos;
  const int64_t blk = pos / block_size;
  if (pos < 0 || blk >= max_blocks) return;  // uniform over the block
  const int64_t first = blk * block_size;
  const int n = static_cast<int>(pos - first + 1);
  float c[4];
  load_cls(cls, d, c);
  stage_keys(rk, first, n, d, keys);
  lds_barrier();
  summarize(keys, n, d, c, inv_sqrt_d, p, summaries + blk * d);
}

// z[b] for every block up to the one holding pos.
__global__ __launch_bounds__(kRouteBlock) void scores_step_k(const float* __restrict__ rq,
                                                             const float* __restrict__ summaries, int d,
                                                             int block_size, float inv_sqrt_d,
                                                             const uocr_rocm_step_state* __restrict__ state,
                                                             int64_t max_blocks, float* __restrict__ z) {
  __shared__ float q[kMaxIndexDim];
  __shared__ float zs[kMaxRouteBlocks];
  const int64_t pos = state->pos;
  const int64_t nb = pos < 0 ? 0 : pos / block_size + 1;
  const int n = static_cast<int>(nb < max_blocks ? nb : max_blocks);
  for (int e = threadIdx.x; e < d; e += blockDim.x) q[e] = rq[e];
  lds_barrier();
  score_blocks(q, summaries, d, n, inv_sqrt_d, zs);
  lds_barrier();
  for (int b = threadIdx.x; b < n; b += blockDim.x) z[b] = zs[b];
}

// Prompt rows: one workgroup per query row (position first_pos + row, page
// query_page[row] or one_page); z [rows, nblk], mask [rows, keys].
__global__ __launch_bounds__(kRouteBlock) void route_rows_k(const float* __restrict__ z, int nblk, int64_t first_pos,
                                                            int64_t keys, const int64_t* __restrict__ block_min,
                                                            const int64_t* __restrict__ block_max,
                                                            int64_t prompt_blocks,
                                                            const int64_t* __restrict__ query_page, int64_t one_page,
                                                            RouteArgs p, float* __restrict__ mask) {
  __shared__ RouteShared sh;
  const int64_t row = blockIdx.x;
  const int64_t page = query_page != nullptr ? query_page[row] : one_page;
  route_row(z + row * nblk, nblk, first_pos + row, keys, page, block_min, block_max, prompt_blocks, p, sh.lds(),
            mask + row * keys);
}

// One decode query, lengths from the StepState: mask [pos + 1].
__global__ __launch_bounds__(kRouteBlock) void route_step_k(const float* __restrict__ z, int64_t max_blocks,
                                                            const int64_t* __restrict__ block_min,
                                                            const int64_t* __restrict__ block_max,
                                                            int64_t prompt_blocks,
                                                            const uocr_rocm_step_state* __restrict__ state,
                                                            RouteArgs p, float* __restrict__ mask) {
  __shared__ RouteShared sh;
  const int64_t pos = state->pos;
  if (pos < 0 || pos / p.block_size >= max_blocks) return;  // uniform over the block
  const int nblk = static_cast<int>(pos / p.block_size + 1);
  route_row(z, nblk, pos, pos + 1, state->query_page, block_min, block_max, prompt_blocks, p, sh.lds(), mask);
}

struct DecodeRouteArgs {
  const float* rq;       // [d] router query, before its norm
  const float* rk;       // [d] router key, before its norm
  const float* q_norm;   // [d]
  const float* k_norm;   // [d]
  float eps;
  const float* inv_tok;  // [n_tok]
  int n_tok;
  const float* inv_page;  // [d / 2 - n_tok]
  int64_t page_mod;
  const float* cls;      // [d]
  float* router_keys;    // [capacity, d]
  float* summaries;      // [capacity / block_size rounded up, d]
  int d;
  float inv_sqrt_d;
  const int64_t* block_min;
  const int64_t* block_max;
  int64_t prompt_blocks;
  const uocr_rocm_step_state* state;
  int64_t capacity;
  RouteArgs p;
  float* mask;           // [capacity]; keys 0..pos written
  float* z_out;          // null, or [capacity blocks]: the scores the route read
  float* rqk_out;        // null, or [2 d]: rq and rk after norm and rope
  int* segs;             // null, or the live keys as segments (route_select)
};

// The router's RMSNorm of one row of d floats held four per lane (lanes with
// 4 lane >= d hold zeros), with its weights w held the same way: non-finite
// values count as 0, y = clamp(clamp(v inv) (1 + w)) with inv = 1 / sqrt(ss
// / d + eps) formed in fp64 from the fp32 sum of squares
// (src/model/decoder.cpp:20-34).
__device__ __forceinline__ void router_norm_lane(float (&v)[4], const float (&w)[4], int d, float eps, int lane) {
#pragma clang fp contract(off)
  float part = 0.0f;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[i] = __builtin_isfinite(v[i]) ? v[i] : 0.0f;
    part += v[i] * v[i];
  }
  const float ss = wave_sum(part);
  const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(ss) / static_cast<double>(d) +
                                                  static_cast<double>(eps)));
  if (4 * lane < d) {
#pragma unroll
    for (int i = 0; i < 4; ++i) v[i] = clamp_act(clamp_act(v[i] * inv) * (1.0f + w[i]));
  }
}

__global__ __launch_bounds__(kRouteBlock) void route_decode_k(DecodeRouteArgs a) {
#pragma clang fp contract(off)
  // keys holds the staged block of router keys until its summary is formed,
  // then the blocks' mask values and the per-wave top-m lists; zs holds the
  // scores, then (in place) the entmax inputs.
  __shared__ __attribute__((aligned(16))) float keys[kStageFloats];
  __shared__ float rqk[2][kMaxIndexDim];  // normed, then rotated rq and rk
  __shared__ float rope_sc[2][kMaxIndexDim / 2];  // the rope's sines and cosines
  __shared__ float zs[kMaxRouteBlocks];
  __shared__ unsigned char cand[kMaxRouteBlocks];
  __shared__ float p_lds[kMaxBlockKeys];
  __shared__ int any_slots[kRouteBlock / kWave];
  static_assert(kStageFloats >= kMaxRouteBlocks + 2 * (kRouteBlock / kWave) * kMaxTop,
                "the staged keys' space holds the blocks' mask values and the top-m lists");
  const int d = a.d, half = d / 2;
  const int lane = threadIdx.x & (kWave - 1), wave = wave_in_block();

  // 1. every load that does not wait for another: first those that need no
  // position (the router rows and their weights, head_cls, the rope
  // frequency of this thread's pair, the page ranges), then the step state,
  // then the block's earlier keys and the first pass of summaries
  float v[4] = {0.0f, 0.0f, 0.0f, 0.0f}, w[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (wave < 2 && 4 * lane < d) {
    const float* src = wave == 0 ? a.rq : a.rk;
    const float* wn = wave == 0 ? a.q_norm : a.k_norm;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      v[i] = src[4 * lane + i];
      w[i] = wn[4 * lane + i];
    }
  }
  float cls[4];
  load_cls(a.cls, d, cls);
  const int pr = threadIdx.x;
  const int sc = pr - 2 * kWave;  // waves 2 and 3 form the rope's sines and cosines, pair sc
  float freq = 0.0f;
  if (sc >= 0 && sc < half) freq = sc < a.n_tok ? a.inv_tok[sc] : a.inv_page[sc - a.n_tok];

  // the prompt blocks' page ranges (route_candidates checks the query's
  // page and the block count)
  PageRanges ranges;
  load_pages(a.block_min, a.block_max, a.prompt_blocks, kMaxRouteBlocks, 0, ranges);

  const int64_t pos64 = a.state->pos;
  if (pos64 < 0 || pos64 >= a.capacity) return;  // uniform over the block
  // capacity / block_size <= 4096 blocks of at most 64 keys: 32-bit from here
  const int pos = static_cast<int>(pos64), bs = a.p.block_size;
  const int blk = pos / bs, first = blk * bs;
  const int n = pos - first + 1;
  const int last_remote = blk - a.p.local_blocks;
  const int nrem = last_remote < 0 ? 0 : last_remote + 1;
  const int nblk = blk + 1;
  const int64_t query_page = a.state->query_page;
  StagedKeys staged;
  load_keys(a.router_keys, first, n - 1, d, staged);
  // with a local window the remote blocks are whole, none of them the
  // block summarized here: the first pass of their summaries goes out now
  // (issued after the keys, which are waited for first)
  const bool early = a.p.local_blocks > 0;
  ScoreRows rows;
  if (early) score_load(a.summaries, d, nrem, 0, rows);

  // 2. router norm of rq (wave 0) and rk (wave 1) while waves 2-3 form the
  // sines and cosines of (tok, page) and every thread its blocks' candidate
  // flags; then the rope
  if (wave < 2) {
    router_norm_lane(v, w, d, a.eps, lane);
    if (4 * lane < d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) rqk[wave][4 * lane + i] = v[i];
    }
  }
  if (sc >= 0 && sc < half) {
    int64_t pg = a.state->page;
    if (a.page_mod > 0) pg = ((pg % a.page_mod) + a.page_mod) % a.page_mod;
    const float angle = (sc < a.n_tok ? static_cast<float>(a.state->tok) : static_cast<float>(pg)) * freq;
    sincosf(angle, &rope_sc[0][sc], &rope_sc[1][sc]);
  }
  store_keys(staged, n - 1, d, keys);
  route_candidates_begin(ranges, nblk, last_remote, query_page, cand, any_slots);
  lds_barrier();
  route_candidates_end(nblk, last_remote, cand, any_slots);
  if (pr < half) {
    const float sn = rope_sc[0][pr], cs = rope_sc[1][pr];
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float x0 = rqk[r][pr], x1 = rqk[r][pr + half];
      rqk[r][pr] = x0 * cs - x1 * sn;
      rqk[r][pr + half] = x1 * cs + x0 * sn;
    }
  }
  lds_barrier();

  // 3. append rk at pos and refresh the summary of the block holding pos
  for (int e = threadIdx.x; e < d; e += blockDim.x) {
    a.router_keys[pos * d + e] = rqk[1][e];
    keys[(n - 1) * d + e] = rqk[1][e];
    if (a.rqk_out != nullptr) {
      a.rqk_out[e] = rqk[0][e];
      a.rqk_out[d + e] = rqk[1][e];
    }
  }
  lds_barrier();
  summarize(keys, n, d, cls, a.inv_sqrt_d, p_lds, a.summaries + blk * d);

  // 4. the scores of the blocks before the window
  if (!early) {
    __syncthreads();  // the summary just written is one of the rows scored
    score_load(a.summaries, d, nrem, 0, rows);
  }
  score_reduce(rqk[0], d, nrem, 0, a.inv_sqrt_d, rows, zs);
  const int pass = score_pass_rows(d);
  for (int base = pass; base < nrem; base += pass) {
    score_load(a.summaries, d, nrem, base, rows);
    score_reduce(rqk[0], d, nrem, base, a.inv_sqrt_d, rows, zs);
  }
  lds_barrier();
  if (a.z_out != nullptr) {
    for (int b = threadIdx.x; b < nrem; b += blockDim.x) a.z_out[b] = zs[b];
  }

  // 5. the selection and the key mask over keys 0..pos
  route_select(zs, nblk, pos, pos + 1, a.p,
               RouteLds{zs, cand, keys, reinterpret_cast<uint64_t*>(keys + kMaxRouteBlocks), any_slots}, a.mask,
               a.segs);
}

// ---- host side -----------------------------------------------------------------------------

int check_params(const char* what, const uocr_rocm_route_params* params, RouteArgs* out) {
  UOCR_REQUIRE(params != nullptr, what, "null params");
  const auto& q = *params;
  UOCR_REQUIRE(q.block_size >= 1 && q.block_size <= kMaxBlockKeys, what, "block_size must be in [1, 64]");
  UOCR_REQUIRE(q.local_blocks >= 0 && q.local_blocks < (int64_t{1} << 24), what, "local_blocks out of range");
  UOCR_REQUIRE(q.top_m <= kMaxTop, what, "top_m above 32");
  UOCR_REQUIRE(q.top_k < (int64_t{1} << 24) && q.top_m > -(int64_t{1} << 24) && q.top_k > -(int64_t{1} << 24),
               what, "top_k out of range");
  UOCR_REQUIRE(q.sigma != 0.0f, what, "sigma must not be 0");
  *out = RouteArgs{static_cast<int>(q.block_size), static_cast<int>(q.local_blocks), static_cast<int>(q.top_m),
                   static_cast<int>(q.top_k), q.idx_scale, q.floor, q.sigma};
  return UOCR_ROCM_OK;
}

int check_dim(const char* what, int64_t d, int64_t block_size) {
  UOCR_REQUIRE(d >= 4 && d <= kMaxIndexDim && d % 4 == 0, what, "d must be a multiple of 4 in [4, 256]");
  UOCR_REQUIRE(block_size >= 1 && block_size <= kMaxBlockKeys, what, "block_size must be in [1, 64]");
  UOCR_REQUIRE(block_size * d <= kStageFloats, what, "block_size * d above 8192");
  return UOCR_ROCM_OK;
}

float inv_sqrt(int64_t d) { return 1.0f / sqrtf(static_cast<float>(d)); }

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_block_summaries(void* stream, const float* keys, int64_t s, int64_t d, const float* head_cls,
                              int64_t block_size, float* out) {
  constexpr const char* kWhat = "uocr_rocm_block_summaries";
  if (const int st = check_dim(kWhat, d, block_size)) return st;
  UOCR_REQUIRE(s >= 0 && s < (int64_t{1} << 40), kWhat, "s out of range");
  if (s == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(keys != nullptr && head_cls != nullptr && out != nullptr, kWhat, "null pointer");
  UOCR_REQUIRE(aligned16(keys), kWhat, "keys must be 16-byte aligned");
  const int64_t nblk = (s + block_size - 1) / block_size;
  UOCR_REQUIRE(nblk < (int64_t{1} << 31), kWhat, "too many blocks");
  clear_launch_error();
  block_summaries_k<<<static_cast<unsigned>(nblk), 256, 0, as_stream(stream)>>>(
      keys, s, static_cast<int>(d), head_cls, static_cast<int>(block_size), inv_sqrt(d), out);
  return check_launch(kWhat);
}

int uocr_rocm_summary_step(void* stream, const float* router_keys, int64_t d, const float* head_cls,
                           int64_t block_size, const uocr_rocm_step_state* state, int64_t max_blocks,
                           float* summaries) {
  constexpr const char* kWhat = "uocr_rocm_summary_step";
  if (const int st = check_dim(kWhat, d, block_size)) return st;
  UOCR_REQUIRE(max_blocks >= 1, kWhat, "max_blocks must be >= 1");
  UOCR_REQUIRE(router_keys != nullptr && head_cls != nullptr && state != nullptr && summaries != nullptr, kWhat,
               "null pointer");
  UOCR_REQUIRE(aligned16(router_keys), kWhat, "router_keys must be 16-byte aligned");
  clear_launch_error();
  summary_step_k<<<1, 256, 0, as_stream(stream)>>>(router_keys, static_cast<int>(d), head_cls,
                                                   static_cast<int>(block_size), inv_sqrt(d), state, max_blocks,
                                                   summaries);
  return check_launch(kWhat);
}

int uocr_rocm_scores_step(void* stream, const float* rq, const float* summaries, int64_t d, int64_t block_size,
                          const uocr_rocm_step_state* state, int64_t max_blocks, float* z) {
  constexpr const char* kWhat = "uocr_rocm_scores_step";
  if (const int st = check_dim(kWhat, d, block_size)) return st;
  UOCR_REQUIRE(max_blocks >= 1 && max_blocks <= kMaxRouteBlocks, kWhat, "max_blocks must be in [1, 4096]");
  UOCR_REQUIRE(rq != nullptr && summaries != nullptr && state != nullptr && z != nullptr, kWhat, "null pointer");
  UOCR_REQUIRE(aligned16(summaries), kWhat, "summaries must be 16-byte aligned");
  clear_launch_error();
  scores_step_k<<<1, kRouteBlock, 0, as_stream(stream)>>>(rq, summaries, static_cast<int>(d),
                                                          static_cast<int>(block_size), inv_sqrt(d), state,
                                                          max_blocks, z);
  return check_launch(kWhat);
}

int uocr_rocm_route_blocks(void* stream, const float* z, int64_t rows, int64_t nblk, int64_t first_pos, int64_t keys,
                           const int64_t* block_min, const int64_t* block_max, int64_t prompt_blocks,
                           const int64_t* query_page, int64_t one_page, const uocr_rocm_route_params* params,
                           float* mask) {
  constexpr const char* kWhat = "uocr_rocm_route_blocks";
  RouteArgs p;
  if (const int st = check_params(kWhat, params, &p)) return st;
  UOCR_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), kWhat, "rows out of range");
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(nblk >= 1 && nblk <= kMaxRouteBlocks, kWhat, "nblk must be in [1, 4096]");
  UOCR_REQUIRE(first_pos >= 0 && keys >= 1, kWhat, "first_pos must be >= 0 and keys >= 1");
  UOCR_REQUIRE((first_pos + rows - 1) / p.block_size < nblk, kWhat, "nblk does not cover the last query");
  UOCR_REQUIRE(prompt_blocks >= 0 && (prompt_blocks == 0 || (block_min != nullptr && block_max != nullptr)),
               kWhat, "prompt blocks without their pages");
  UOCR_REQUIRE(z != nullptr && mask != nullptr, kWhat, "null pointer");
  clear_launch_error();
  route_rows_k<<<static_cast<unsigned>(rows), kRouteBlock, 0, as_stream(stream)>>>(
      z, static_cast<int>(nblk), first_pos, keys, block_min, block_max, prompt_blocks, query_page, one_page, p, mask);
  return check_launch(kWhat);
}

int uocr_rocm_route_step(void* stream, const float* z, int64_t max_blocks, const int64_t* block_min,
                         const int64_t* block_max, int64_t prompt_blocks, const uocr_rocm_step_state* state,
                         const uocr_rocm_route_params* params, float* mask) {
  constexpr const char* kWhat = "uocr_rocm_route_step";
  RouteArgs p;
  if (const int st = check_params(kWhat, params, &p)) return st;
  UOCR_REQUIRE(max_blocks >= 1 && max_blocks <= kMaxRouteBlocks, kWhat, "max_blocks must be in [1, 4096]");
  UOCR_REQUIRE(prompt_blocks >= 0 && (prompt_blocks == 0 || (block_min != nullptr && block_max != nullptr)),
               kWhat, "prompt blocks without their pages");
  UOCR_REQUIRE(z != nullptr && state != nullptr && mask != nullptr, kWhat, "null pointer");
  clear_launch_error();
  route_step_k<<<1, kRouteBlock, 0, as_stream(stream)>>>(z, max_blocks, block_min, block_max, prompt_blocks, state,
                                                         p, mask);
  return check_launch(kWhat);
}

int uocr_rocm_route_decode_step(void* stream, const float* rq, const float* rk, const float* q_norm,
                                const float* k_norm, float eps, const float* inv_tok, int64_t n_tok,
                                const float* inv_page, int64_t page_mod, const float* head_cls, float* router_keys,
                                float* summaries, int64_t d, const int64_t* block_min, const int64_t* block_max,
                                int64_t prompt_blocks, const uocr_rocm_step_state* state,
                                const uocr_rocm_route_params* params, int64_t capacity, float* mask, float* z_out,
                                float* rqk_out) {
  return uocr_rocm_route_decode_step_segments(stream, rq, rk, q_norm, k_norm, eps, inv_tok, n_tok, inv_page, page_mod,
                                              head_cls, router_keys, summaries, d, block_min, block_max,
                                              prompt_blocks, state, params, capacity, mask, z_out, rqk_out, nullptr);
}

int uocr_rocm_route_decode_step_segments(void* stream, const float* rq, const float* rk, const float* q_norm,
                                         const float* k_norm, float eps, const float* inv_tok, int64_t n_tok,
                                         const float* inv_page, int64_t page_mod, const float* head_cls,
                                         float* router_keys, float* summaries, int64_t d, const int64_t* block_min,
                                         const int64_t* block_max, int64_t prompt_blocks,
                                         const uocr_rocm_step_state* state, const uocr_rocm_route_params* params,
                                         int64_t capacity, float* mask, float* z_out, float* rqk_out,
                                         int32_t* segments) {
  constexpr const char* kWhat = "uocr_rocm_route_decode_step";
  RouteArgs p;
  if (const int st = check_params(kWhat, params, &p)) return st;
  if (const int st = check_dim(kWhat, d, p.block_size)) return st;
  UOCR_REQUIRE(capacity >= 1 && (capacity + p.block_size - 1) / p.block_size <= kMaxRouteBlocks, kWhat,
               "capacity / block_size must be in [1, 4096]");
  UOCR_REQUIRE(n_tok >= 0 && n_tok <= d / 2, kWhat, "n_tok must be in [0, d / 2]");
  UOCR_REQUIRE(n_tok == 0 || inv_tok != nullptr, kWhat, "null inv_tok");
  UOCR_REQUIRE(n_tok == d / 2 || inv_page != nullptr, kWhat, "null inv_page");
  UOCR_REQUIRE(prompt_blocks >= 0 && (prompt_blocks == 0 || (block_min != nullptr && block_max != nullptr)),
               kWhat, "prompt blocks without their pages");
  UOCR_REQUIRE(rq != nullptr && rk != nullptr && q_norm != nullptr && k_norm != nullptr && head_cls != nullptr &&
                   router_keys != nullptr && summaries != nullptr && state != nullptr &&
                   (mask != nullptr || segments != nullptr),
               kWhat, "null pointer");
  UOCR_REQUIRE(aligned16(router_keys) && aligned16(summaries), kWhat,
               "router_keys and summaries must be 16-byte aligned");
  DecodeRouteArgs a{rq, rk, q_norm, k_norm, eps, inv_tok, static_cast<int>(n_tok), inv_page, page_mod, head_cls,
                    router_keys, summaries, static_cast<int>(d), inv_sqrt(d), block_min, block_max, prompt_blocks,
                    state, capacity, p, mask, z_out, rqk_out, segments};
  clear_launch_error();
  route_decode_k<<<1, kRouteBlock, 0, as_stream(stream)>>>(a);
  return check_launch(kWhat);
}

}  // extern "C"
