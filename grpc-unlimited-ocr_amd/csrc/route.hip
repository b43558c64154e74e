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

// The summary of one block whose n keys (n <= kMaxBlockKeys) sit in LDS,
// row-major with row stride d: out[e] = sum_t (w_t / total) key_t[e], w_t =
// exp(a_t - max a), a_t = clamp(key_t . cls / sqrt d), total = max(sum_t
// w_t, 1e-6). Wave w forms the logits of keys w, w + waves, ... (lane e
// takes features e, e + 64, ...); total and the feature sums run over t in
// order. Every thread of the block must call it.
__device__ void summarize(const float* keys, int n, int d, const float* __restrict__ cls, float inv_sqrt_d,
                          float* logit, float* total_slot, float* __restrict__ out) {
#pragma clang fp contract(off)
  const int wave = wave_in_block(), lane = threadIdx.x & (kWave - 1);
  const int waves = static_cast<int>(blockDim.x) / kWave;
  for (int t = wave; t < n; t += waves) {
    float part = 0.0f;
    for (int e = lane; e < d; e += kWave) part += keys[t * d + e] * cls[e];
    const float a = wave_sum(part);
    if (lane == 0) logit[t] = clamp_act(a * inv_sqrt_d);
  }
  __syncthreads();
  if (threadIdx.x == 0) {
    float peak = -3.402823466e+38f;
    for (int t = 0; t < n; ++t) peak = fmaxf(peak, logit[t]);
    float total = 0.0f;
    for (int t = 0; t < n; ++t) {
      logit[t] = expf(logit[t] - peak);
      total += logit[t];
    }
    *total_slot = fmaxf(total, 1e-6f);
  }
  __syncthreads();
  const float total = *total_slot;
  for (int e = threadIdx.x; e < d; e += blockDim.x) {
    float acc = 0.0f;
    for (int t = 0; t < n; ++t) acc += (logit[t] / total) * keys[t * d + e];
    out[e] = acc;
  }
}

// z[b] = (rq . summaries[b]) / sqrt d for b < n (unclamped), rq [d] in LDS.
// Wave w scores blocks w, w + waves, ... eight at a time, every lane
// holding four features (d <= 256, d % 4 == 0): the eight rows' loads go out
// together. Every thread of the block must call it.
__device__ void score_blocks(const float* rq, const float* __restrict__ summaries, int d, int n, float inv_sqrt_d,
                             float* z) {
#pragma clang fp contract(off)
  const int wave = wave_in_block(), lane = threadIdx.x & (kWave - 1);
  const int waves = static_cast<int>(blockDim.x) / kWave;
  const bool on = 4 * lane < d;
  float q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
  if (on) {
#pragma unroll
    for (int i = 0; i < 4; ++i) q[i] = rq[4 * lane + i];
  }
  constexpr int kBatch = 8;
  for (int b0 = wave; b0 < n; b0 += waves * kBatch) {
    u32x4 row[kBatch];
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int b = b0 + i * waves;
      row[i] = u32x4{0u, 0u, 0u, 0u};
      if (on && b < n) row[i] = *reinterpret_cast<const u32x4*>(summaries + static_cast<int64_t>(b) * d + 4 * lane);
    }
#pragma unroll
    for (int i = 0; i < kBatch; ++i) {
      const int b = b0 + i * waves;  // wave-uniform
      if (b < n) {
        float part = 0.0f;
        part += q[0] * __uint_as_float(row[i].x);
        part += q[1] * __uint_as_float(row[i].y);
        part += q[2] * __uint_as_float(row[i].z);
        part += q[3] * __uint_as_float(row[i].w);
        const float s = wave_sum(part);
        if (lane == 0) z[b] = s * inv_sqrt_d;
      }
    }
  }
}

// Block-order key of a candidate score for the top-m: larger scores first,
// then the lower block index (all scores are finite here).
__device__ __forceinline__ uint64_t order_key(float v, int b) {
  uint32_t u = __float_as_uint(v);
  u = (u & 0x80000000u) ? ~u : (u | 0x80000000u);
  return (static_cast<uint64_t>(u) << 32) | (0xffffffffu - static_cast<uint32_t>(b));
}

__device__ __forceinline__ uint64_t wave_max_u64(uint64_t v) {
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) {
    const uint64_t o = __shfl_xor(v, off, kWave);
    v = o > v ? o : v;
  }
  return v;
}

// LDS working set of route_row for one query row: x the blocks' entmax
// inputs (it may be the z array itself, which is read before x is written at
// the same index), cand the candidate flags, block_bias the mask value of a
// block's keys outside the window, and the top-m values, blocks and logs.
struct RouteLds {
  float* x;                 // [nblk]
  unsigned char* cand;      // [nblk]
  float* block_bias;        // [nblk]
  float* top_val;           // [kMaxTop]
  int* top_idx;             // [kMaxTop]
  float* top_logp;          // [kMaxTop]
};

// 1.5-entmax of the m values v[0..m) (in descending order), in place, with
// block_router.cpp:68-91's fp32 steps: v = (v - v0) / 2, running mean and
// mean square give tau_i = mean - sqrt(max((1 - rho (msq - mean^2)) / rho,
// 0)), the support is the count of tau_i <= v_i, and v = max(v - tau*, 0)^2
// with tau* = tau at support - 1 (recomputed by a second pass, so no array
// is indexed by a run-time value).
__device__ void entmax15_sorted(float* v, int m) {
#pragma clang fp contract(off)
  const float peak = v[0];
  for (int i = 0; i < m; ++i) v[i] = (v[i] - peak) / 2.0f;
  int support = 0;
  {
    float sum = 0.0f, sum_sq = 0.0f;
    for (int i = 0; i < m; ++i) {
      sum += v[i];
      sum_sq += v[i] * v[i];
      const float rho = static_cast<float>(i + 1);
      const float mean = sum / rho, mean_sq = sum_sq / rho;
      const float ss = rho * (mean_sq - mean * mean);
      const float delta = fmaxf((1.0f - ss) / rho, 0.0f);
      if (mean - sqrtf(delta) <= v[i]) ++support;
    }
  }
  const int at = (support > 1 ? support : 1) - 1;
  float tau_star = 0.0f;
  {
    float sum = 0.0f, sum_sq = 0.0f;
    for (int i = 0; i <= at; ++i) {
      sum += v[i];
      sum_sq += v[i] * v[i];
      const float rho = static_cast<float>(i + 1);
      const float mean = sum / rho, mean_sq = sum_sq / rho;
      const float ss = rho * (mean_sq - mean * mean);
      const float delta = fmaxf((1.0f - ss) / rho, 0.0f);
      tau_star = mean - sqrtf(delta);
    }
  }
  for (int i = 0; i < m; ++i) {
    const float t = fmaxf(v[i] - tau_star, 0.0f);
    v[i] = t * t;
  }
}

// Routes one query at position pos over nblk blocks (z[b], raw scores of the
// blocks b <= last_remote; other entries are not read) and writes its key
// mask mask[0..keys) (keys past pos get -inf). page < 0: no page
// restriction. Every thread of the block must call it.
__device__ void route_row(const float* z, int nblk, int64_t pos, int64_t keys, int64_t page,
                          const int64_t* __restrict__ block_min, const int64_t* __restrict__ block_max,
                          int64_t prompt_blocks, const RouteArgs p, RouteLds sh, float* __restrict__ mask) {
#pragma clang fp contract(off)
  const int64_t last_remote = pos / p.block_size - p.local_blocks;
  int any_local = 0;
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    const bool remote = b <= last_remote;
    const bool allowed = page >= 0 && b < prompt_blocks && block_min[b] >= 0 && block_min[b] <= page &&
                         page <= block_max[b];
    sh.cand[b] = remote && allowed;
    any_local |= remote && allowed;
  }
  // A page with no remote block of its own routes over every remote block.
  const int any = __syncthreads_or(any_local);
  for (int b = threadIdx.x; b < nblk; b += blockDim.x) {
    const bool remote = b <= last_remote;
    if (!any) sh.cand[b] = remote;
    const float xb = sh.cand[b] ? clamp_act(z[b]) * p.idx_scale : kEntmaxMasked;
    sh.x[b] = xb;
    sh.block_bias[b] = -INFINITY;
  }
  __syncthreads();

  const int m = p.top_m < nblk ? (p.top_m > 1 ? p.top_m : 1) : (nblk > 1 ? nblk : 1);
  const int k = p.top_k < m ? (p.top_k > 1 ? p.top_k : 1) : m;
  if (wave_in_block() == 0) {
    // The top m by m rounds of a wave-wide max over each lane's best block
    // not yet taken (lane l owns blocks l, l + 64, ...; up to 64 each).
    const int lane = threadIdx.x & (kWave - 1);
    uint64_t taken = 0;
    for (int j = 0; j < m; ++j) {
      uint64_t best = 0;
      for (int i = 0, b = lane; b < nblk; ++i, b += kWave) {
        if ((taken >> i) & 1u) continue;
        const uint64_t key = order_key(sh.x[b], b);
        best = key > best ? key : best;
      }
      const uint64_t win = wave_max_u64(best);
      const int wb = static_cast<int>(0xffffffffu - static_cast<uint32_t>(win));
      if ((wb & (kWave - 1)) == lane) taken |= uint64_t{1} << (wb / kWave);
      if (lane == 0) {
        sh.top_idx[j] = wb;
        sh.top_val[j] = sh.x[wb];
      }
    }
    if (lane == 0) {
      // the log-prior bias of the first k (block_router.cpp:131-151)
      entmax15_sorted(sh.top_val, m);
      float logp_sum = 0.0f;
      int count = 0;
      for (int i = 0; i < k; ++i) {
        sh.top_logp[i] = logf(fmaxf(sh.top_val[i], p.floor));
        if (sh.cand[sh.top_idx[i]]) {
          logp_sum += sh.top_logp[i];
          ++count;
        }
      }
      const float mu = logp_sum / static_cast<float>(count > 1 ? count : 1);
      for (int i = 0; i < k; ++i) {
        if (sh.cand[sh.top_idx[i]]) sh.block_bias[sh.top_idx[i]] = (sh.top_logp[i] - mu) / p.sigma;
      }
    }
  }
  __syncthreads();

  const int64_t window = static_cast<int64_t>(p.local_blocks) * p.block_size;
  for (int64_t j = threadIdx.x; j < keys; j += blockDim.x) {
    float v = -INFINITY;
    if (j <= pos) v = j > pos - window ? 0.0f : sh.block_bias[j / p.block_size];
    mask[j] = v;
  }
}

// LDS for route_row in a kernel that routes one row and needs nothing else.
struct RouteShared {
  float x[kMaxRouteBlocks];
  unsigned char cand[kMaxRouteBlocks];
  float block_bias[kMaxRouteBlocks];
  float top_val[kMaxTop];
  int top_idx[kMaxTop];
  float top_logp[kMaxTop];
  __device__ RouteLds lds() { return RouteLds{x, cand, block_bias, top_val, top_idx, top_logp}; }
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

// ---- kernels -------------------------------------------------------------------------------

// Every block of s keys: one workgroup per block.
__global__ __launch_bounds__(256) void block_summaries_k(const float* __restrict__ rk, int64_t s, int d,
                                                         const float* __restrict__ cls, int block_size,
                                                         float inv_sqrt_d, float* __restrict__ out) {
  __shared__ __attribute__((aligned(16))) float keys[kStageFloats];
  __shared__ float logit[kMaxBlockKeys];
  __shared__ float total;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * block_size;
  const int n = static_cast<int>(s - first < block_size ? s - first : block_size);
  stage_keys(rk, first, n, d, keys);
  __syncthreads();
  summarize(keys, n, d, cls, inv_sqrt_d, logit, &total, out + static_cast<int64_t>(blockIdx.x) * d);
}

// The summary of the block holding state->pos (keys first..pos).
__global__ __launch_bounds__(256) void summary_step_k(const float* __restrict__ rk, int d,
                                                      const float* __restrict__ cls, int block_size,
                                                      float inv_sqrt_d, const uocr_rocm_step_state* __restrict__ state,
                                                      int64_t max_blocks, float* __restrict__ summaries) {
  __shared__ __attribute__((aligned(16))) float keys[kStageFloats];
  __shared__ float logit[kMaxBlockKeys];
  __shared__ float total;
  const int64_t pos = state->pos;
  const int64_t blk = pos / block_size;
  if (pos < 0 || blk >= max_blocks) return;  // uniform over the block
  const int64_t first = blk * block_size;
  const int n = static_cast<int>(pos - first + 1);
  stage_keys(rk, first, n, d, keys);
  __syncthreads();
  summarize(keys, n, d, cls, inv_sqrt_d, logit, &total, summaries + blk * d);
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
  __syncthreads();
  score_blocks(q, summaries, d, n, inv_sqrt_d, zs);
  __syncthreads();
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
};

// The router's RMSNorm of one row of d floats held four per lane (lanes with
// 4 lane >= d hold zeros): non-finite values count as 0, y = clamp(clamp(v
// inv) (1 + w)) with inv = 1 / sqrt(ss / d + eps) formed in fp64 from the
// fp32 sum of squares (src/model/decoder.cpp:20-34).
__device__ __forceinline__ void router_norm_lane(float (&v)[4], const float* __restrict__ w, int d, float eps,
                                                 int lane) {
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
    for (int i = 0; i < 4; ++i) v[i] = clamp_act(clamp_act(v[i] * inv) * (1.0f + w[4 * lane + i]));
  }
}

__global__ __launch_bounds__(kRouteBlock) void route_decode_k(DecodeRouteArgs a) {
#pragma clang fp contract(off)
  // keys holds the staged block of router keys until its summary is formed,
  // then the blocks' mask values; zs holds the scores, then (in place) the
  // entmax inputs.
  __shared__ __attribute__((aligned(16))) float keys[kStageFloats];
  __shared__ float rqk[2][kMaxIndexDim];  // normed, then rotated rq and rk
  __shared__ float zs[kMaxRouteBlocks];
  __shared__ unsigned char cand[kMaxRouteBlocks];
  __shared__ float logit[kMaxBlockKeys];
  __shared__ float top_val[kMaxTop], top_logp[kMaxTop];
  __shared__ int top_idx[kMaxTop];
  __shared__ float total;
  static_assert(kStageFloats >= kMaxRouteBlocks, "the staged keys' space holds the blocks' mask values");
  const int64_t pos = a.state->pos;
  const int bs = a.p.block_size;
  if (pos < 0 || pos >= a.capacity) return;  // uniform over the block
  const int d = a.d, half = d / 2;
  const int lane = threadIdx.x & (kWave - 1), wave = wave_in_block();

  // 1. router norm of rq (wave 0) and rk (wave 1), then rope at (tok, page)
  if (wave < 2) {
    const float* src = wave == 0 ? a.rq : a.rk;
    float v[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    if (4 * lane < d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) v[i] = src[4 * lane + i];
    }
    router_norm_lane(v, wave == 0 ? a.q_norm : a.k_norm, d, a.eps, lane);
    if (4 * lane < d) {
#pragma unroll
      for (int i = 0; i < 4; ++i) rqk[wave][4 * lane + i] = v[i];
    }
  }
  __syncthreads();
  if (static_cast<int>(threadIdx.x) < half) {
    const int pr = threadIdx.x;
    int64_t pg = a.state->page;
    if (a.page_mod > 0) pg = ((pg % a.page_mod) + a.page_mod) % a.page_mod;
    const float angle = pr < a.n_tok ? static_cast<float>(a.state->tok) * a.inv_tok[pr]
                                     : static_cast<float>(pg) * a.inv_page[pr - a.n_tok];
    float sn, cs;
    sincosf(angle, &sn, &cs);
#pragma unroll
    for (int r = 0; r < 2; ++r) {
      const float x0 = rqk[r][pr], x1 = rqk[r][pr + half];
      rqk[r][pr] = x0 * cs - x1 * sn;
      rqk[r][pr + half] = x1 * cs + x0 * sn;
    }
  }
  __syncthreads();

  // 2. append rk at pos; stage the keys of the block holding pos (the new
  // one from LDS) and refresh that block's summary
  const int64_t blk = pos / bs, first = blk * bs;
  const int n = static_cast<int>(pos - first + 1);
  for (int e = threadIdx.x; e < d; e += blockDim.x) {
    a.router_keys[pos * d + e] = rqk[1][e];
    keys[(n - 1) * d + e] = rqk[1][e];
    if (a.rqk_out != nullptr) {
      a.rqk_out[e] = rqk[0][e];
      a.rqk_out[d + e] = rqk[1][e];
    }
  }
  stage_keys(a.router_keys, first, n - 1, d, keys);
  __syncthreads();
  summarize(keys, n, d, a.cls, a.inv_sqrt_d, logit, &total, a.summaries + blk * d);

  // 3. scores of the blocks before the window (whole, so unchanged here)
  const int64_t last_remote = blk - a.p.local_blocks;
  const int nrem = last_remote < 0 ? 0 : static_cast<int>(last_remote + 1);
  score_blocks(rqk[0], a.summaries, d, nrem, a.inv_sqrt_d, zs);
  __syncthreads();
  if (a.z_out != nullptr) {
    for (int b = threadIdx.x; b < nrem; b += blockDim.x) a.z_out[b] = zs[b];
  }

  // 4. the route and the key mask over keys 0..pos
  route_row(zs, static_cast<int>(blk + 1), pos, pos + 1, a.state->query_page, a.block_min, a.block_max,
            a.prompt_blocks, a.p, RouteLds{zs, cand, keys, top_val, top_idx, top_logp}, a.mask);
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
                   router_keys != nullptr && summaries != nullptr && state != nullptr && mask != nullptr,
               kWhat, "null pointer");
  UOCR_REQUIRE(aligned16(router_keys) && aligned16(summaries), kWhat,
               "router_keys and summaries must be 16-byte aligned");
  DecodeRouteArgs a{rq, rk, q_norm, k_norm, eps, inv_tok, static_cast<int>(n_tok), inv_page, page_mod, head_cls,
                    router_keys, summaries, static_cast<int>(d), inv_sqrt(d), block_min, block_max, prompt_blocks,
                    state, capacity, p, mask, z_out, rqk_out};
  clear_launch_error();
  route_decode_k<<<1, kRouteBlock, 0, as_stream(stream)>>>(a);
  return check_launch(kWhat);
}

}  // extern "C"
