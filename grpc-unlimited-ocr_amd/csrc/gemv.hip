// gemv.hip: the bf16 weight-streaming GEMV of the decode step for gfx950,
//   y[n] = bf16(x) . w[n, :] (+ bias[n]),  x fp32 [k], w bf16 [n, k],
// with the input rounded to bf16 first and fp32 accumulation, as the
// reference's gemv_bf16 (src/backend/cuda/gemv_ops.h:25-26, gemv_ops.cu:
// 132-141,199-203) and linear (ops.h:14-17) define it. The time is the time
// to read w once: 2 n k bytes.
//
// Layout: a weight row is a run of 16-byte chunks (8 bf16); lane l of a wave
// takes chunks l, l + 64, l + 128, ... of every row the wave owns. Each wave
// keeps its share of bf16(x) in registers (CPL chunks per lane, k <= 2048),
// reused for every row; waves walk the rows grid-stride, RPW rows at a time,
// so RPW * CPL weight loads per lane are in flight together. Weight rows
// stream with nontemporal loads. The row total is a wave64 DPP butterfly.
// Workgroups are 8 waves: the first rows' weights are requested, then the
// workgroup stages bf16(x) in LDS with one 16-byte load per thread and each
// wave takes its registers from there. Every wave reading x from L2 itself
// put hundreds of waves per XCD on the same few lines at once: 8-wave
// groups staging x ran the decode projections 2-12% faster (the fused
// QKV projection 5.55 -> 4.86 us). Inputs wider than the registers hold (k
// up to kGemvMaxK) keep x in LDS; widths that are not a multiple of 8 or not
// 16-byte aligned take the element-wise kernel.

#include <type_traits>

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int64_t kGemvMaxK = 12288;        // the reference's bound (gemv_ops.h:16)
constexpr int kGemvRegChunks = 4;           // register-resident x: k <= 64 * 4 * 8
// Large matrices: 2 rows per wave and at most 6144 workgroups, walking the
// rows grid-stride. Measured on the 129280 x 1280 LM head: 49.3 us against
// 54.3 us for 4 rows and 2048 workgroups, and against 51-65 us for the other
// combinations of 1, 2, 4 rows and 512 .. unbounded workgroups.
constexpr unsigned kGemvMaxBlocks = 6144;
constexpr int kBigRows = 16384;  // from here on, 2 rows per wave
// The register-resident kernels (gemv_reg, gemv_fused): 8-wave workgroups,
// at most half as many (the same wave count).
constexpr int kGemvBlock = 512;
constexpr int kGemvWaves = kGemvBlock / kWave;
constexpr unsigned kGemvRegMaxBlocks = kGemvMaxBlocks * kWavesPerBlock / kGemvWaves;

// Eight bf16 weights (one chunk) against eight fp32 inputs, in order.
__device__ __forceinline__ float dot8(const u32x4 w, const float (&x)[8], float acc) {
  acc = fmaf(bf16_lo(w.x), x[0], acc);
  acc = fmaf(bf16_hi(w.x), x[1], acc);
  acc = fmaf(bf16_lo(w.y), x[2], acc);
  acc = fmaf(bf16_hi(w.y), x[3], acc);
  acc = fmaf(bf16_lo(w.z), x[4], acc);
  acc = fmaf(bf16_hi(w.z), x[5], acc);
  acc = fmaf(bf16_lo(w.w), x[6], acc);
  acc = fmaf(bf16_hi(w.w), x[7], acc);
  return acc;
}

__device__ __forceinline__ float round_bf16(float v) { return bf16_to_f32(f32_to_bf16(v)); }

// bf16(x[8c .. 8c + 7]) for chunk c.
__device__ __forceinline__ void load_x8(const float* x, int c, float (&v)[8]) {
  float raw[8];
  load_f32<8>(x + 8 * static_cast<int64_t>(c), raw);
#pragma unroll
  for (int e = 0; e < 8; ++e) v[e] = round_bf16(raw[e]);
}

__device__ __forceinline__ void store_rows(float* y, const float* bias, int64_t row0, int64_t n, const float* acc,
                                           int count) {
  const int lane = threadIdx.x & (kWave - 1);
  for (int r = 0; r < count; ++r) {
    if (lane == r && row0 + r < n) y[row0 + r] = acc[r] + (bias != nullptr ? bias[row0 + r] : 0.0f);
  }
}

// bf16(x[0 .. 8 nchunks)) into xs, one 16-byte load per thread per pass of
// the workgroup; every thread of the workgroup calls it.
__device__ __forceinline__ void stage_x(const float* __restrict__ x, int nchunks, float* xs) {
  for (int t = threadIdx.x; t < 2 * nchunks; t += kGemvBlock) {
    float v[4];
    load_f32<4>(x + 4 * static_cast<int64_t>(t), v);
#pragma unroll
    for (int e = 0; e < 4; ++e) xs[4 * t + e] = round_bf16(v[e]);
  }
  __syncthreads();
}

// The input of the attention's output projection as the split records of
// its split-K attention (decode.hip's attend_partial): per head, `splits`
// records of hd + 2 floats (the running max m, the exp-sum l, the weighted
// value sums). x_out (optional) receives the merged row in fp32.
struct MergedX {
  const float* part;
  int heads, hd, splits;
  float* x_out;
};

// bf16(merge(records)) into xs[0 .. heads hd), one wave per (head, 64-element
// slice), with attend_merge's arithmetic for splits <= 64: the weights
// w_s = exp(m_s - max m) (0 for an empty split), the total as the wave sum
// of w_s l_s over the splits in lanes, the value sum as four partials over
// the splits s = p, p + 4, ... (fma in split order) added as (p0 + p1) +
// (p2 + p3), and the row as sum / total (0 without a total). Each lane's
// first 16 value loads go out before the weights are formed. Every thread of
// the workgroup calls it.
__device__ __forceinline__ void stage_merged_x(const MergedX& mx, float* xs) {
  __shared__ float sw[kGemvWaves][kWave];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int slices = (mx.hd + kWave - 1) / kWave;
  const int64_t rec_len = mx.hd + 2;
  constexpr int kBatch = 16;
  for (int u = wave; u < mx.heads * slices; u += kGemvWaves) {
    const int h = u / slices;
    const int e = (u - h * slices) * kWave + lane;
    const int ec = e < mx.hd ? e : mx.hd - 1;
    const float* recs = mx.part + static_cast<int64_t>(h) * mx.splits * rec_len;
    const int sc = lane < mx.splits ? lane : mx.splits - 1;
    float m = recs[sc * rec_len];
    const float l = recs[sc * rec_len + 1];
    float val[kBatch];
#pragma unroll
    for (int j = 0; j < kBatch; ++j) val[j] = recs[(j < mx.splits ? j : mx.splits - 1) * rec_len + 2 + ec];
    m = lane < mx.splits ? m : -INFINITY;
    const float big = wave_max(m);
    const float wgt = (m == -INFINITY || big == -INFINITY) ? 0.0f : exp_shift(m, big);
    const float total = wave_sum(wgt * l);
    sw[wave][lane] = wgt;
    __builtin_amdgcn_wave_barrier();
    float acc[4] = {0.0f, 0.0f, 0.0f, 0.0f};
    for (int s0 = 0; s0 < mx.splits; s0 += kBatch) {
      if (s0 > 0) {
#pragma unroll
        for (int j = 0; j < kBatch; ++j) {
          const int sp = s0 + j;
          val[j] = recs[(sp < mx.splits ? sp : mx.splits - 1) * rec_len + 2 + ec];
        }
      }
#pragma unroll
      for (int j = 0; j < kBatch; ++j) {
        const int sp = s0 + j;
        if (sp < mx.splits) acc[j & 3] = fmaf(sw[wave][sp], val[j], acc[j & 3]);
      }
    }
    __builtin_amdgcn_wave_barrier();
    const float sum = (acc[0] + acc[1]) + (acc[2] + acc[3]);
    const float out = total > 0.0f ? sum / total : 0.0f;
    if (e < mx.hd) {
      xs[h * mx.hd + e] = round_bf16(out);
      if (mx.x_out != nullptr && blockIdx.x == 0) mx.x_out[h * mx.hd + e] = out;
    }
  }
  __syncthreads();
}

// x in registers: CPL chunks per lane; RPW rows per wave per pass. kMerged:
// x is the merge of split attention records (mx), formed in the prologue.
template <int CPL, int RPW, bool kMerged = false>
__global__ __launch_bounds__(kGemvBlock) void gemv_reg(const float* __restrict__ x, int nchunks,
                                                       const uint16_t* __restrict__ w, int64_t n,
                                                       const float* __restrict__ bias, float* __restrict__ y,
                                                       const MergedX mx = {}) {
  __shared__ __align__(16) float xs[kWave * kGemvRegChunks * 8];
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t k = static_cast<int64_t>(nchunks) * 8;
  const int64_t groups = (n + RPW - 1) / RPW;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kGemvWaves;
  const int64_t g0 = static_cast<int64_t>(blockIdx.x) * kGemvWaves + threadIdx.x / kWave;
  u32x4 wc[RPW][CPL];
  auto load_w = [&](int64_t g) {
    const int64_t row0 = g * RPW;
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int c = lane + kWave * i;
        wc[r][i] = u32x4{0u, 0u, 0u, 0u};
        if (row0 + r < n && c < nchunks) {
          wc[r][i] = stream_load(reinterpret_cast<const u32x4*>(w + (row0 + r) * k) + c);
        }
      }
    }
  };
  // Few rows (RPW = 1, one pass): the first rows' weights go out before x is
  // staged, so both are in flight together. Many rows (RPW = 2, the LM
  // head's grid-stride walk): x is staged first and every pass stores the
  // workgroup's rows as one contiguous run from LDS (49.6 -> 48.5 us on the
  // 129280 x 1280 LM head, 100 launches back to back; the same order was 2%
  // slower on the decode projections).
  constexpr bool kManyRows = RPW > 1;
  static_assert(!(kMerged && kManyRows), "the merged input serves the few-rows kernel");
  if constexpr (kManyRows) {
    stage_x(x, nchunks, xs);
  } else {
    if (g0 < groups) load_w(g0);
    if constexpr (kMerged) {
      stage_merged_x(mx, xs);
    } else {
      stage_x(x, nchunks, xs);
    }
  }
  float xv[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + kWave * i;
    if (c < nchunks) {
      load_f32<8>(xs + 8 * c, xv[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[i][e] = 0.0f;
    }
  }
  if constexpr (kManyRows) {
    // Passes are uniform over the workgroup (wave w takes group gb + w), so
    // every wave reaches the barriers around the LDS row store.
    __shared__ float ys[kGemvWaves * RPW];
    const int wave = threadIdx.x / kWave;
    for (int64_t gb = static_cast<int64_t>(blockIdx.x) * kGemvWaves; gb < groups; gb += step) {
      const int64_t g = gb + wave;
      if (g < groups) {
        load_w(g);
        float acc[RPW];
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          float a = 0.0f;
#pragma unroll
          for (int i = 0; i < CPL; ++i) a = dot8(wc[r][i], xv[i], a);
          acc[r] = wave_sum(a);
        }
#pragma unroll
        for (int r = 0; r < RPW; ++r) {
          if (lane == r) ys[wave * RPW + r] = acc[r];
        }
      }
      __syncthreads();
      const int64_t r0 = gb * RPW;
      const int t = static_cast<int>(threadIdx.x);
      if (t < kGemvWaves * RPW && r0 + t < n) y[r0 + t] = ys[t] + (bias != nullptr ? bias[r0 + t] : 0.0f);
      __syncthreads();
    }
  } else {
    for (int64_t g = g0; g < groups; g += step) {
      if (g != g0) load_w(g);
      const int64_t row0 = g * RPW;
      float acc[RPW];
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        float a = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) a = dot8(wc[r][i], xv[i], a);
        acc[r] = wave_sum(a);
      }
      store_rows(y, bias, row0, n, acc, RPW);
    }
  }
}

// x staged in LDS as bf16-rounded fp32 (k <= kGemvMaxK): one row per wave,
// four chunks per lane in flight.
__global__ __launch_bounds__(kBlock) void gemv_lds(const float* __restrict__ x, int nchunks,
                                                   const uint16_t* __restrict__ w, int64_t n,
                                                   const float* __restrict__ bias, float* __restrict__ y) {
  extern __shared__ float xs[];
  for (int c = threadIdx.x; c < nchunks; c += kBlock) {
    float v[8];
    load_x8(x, c, v);
#pragma unroll
    for (int e = 0; e < 8; ++e) xs[8 * c + e] = v[e];
  }
  __syncthreads();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t k = static_cast<int64_t>(nchunks) * 8;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave; row < n; row += step) {
    const u32x4* wr = reinterpret_cast<const u32x4*>(w + row * k);
    float a = 0.0f;
    for (int base = 0; base < nchunks; base += 4 * kWave) {
      u32x4 wc[4];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = base + lane + kWave * i;
        wc[i] = c < nchunks ? stream_load(wr + c) : u32x4{0u, 0u, 0u, 0u};
      }
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const int c = base + lane + kWave * i;
        if (c < nchunks) {
          float xv[8];
          load_f32<8>(xs + 8 * c, xv);
          a = dot8(wc[i], xv, a);
        }
      }
    }
    a = wave_sum(a);
    if (lane == 0) y[row] = a + (bias != nullptr ? bias[row] : 0.0f);
  }
}

// Any k and alignment: element-wise, one row per wave.
__global__ __launch_bounds__(kBlock) void gemv_any(const float* __restrict__ x, int64_t k,
                                                   const uint16_t* __restrict__ w, int64_t n,
                                                   const float* __restrict__ bias, float* __restrict__ y) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave; row < n; row += step) {
    const uint16_t* wr = w + row * k;
    float a = 0.0f;
    for (int64_t i = lane; i < k; i += kWave) a = fmaf(bf16_to_f32(wr[i]), round_bf16(x[i]), a);
    a = wave_sum(a);
    if (lane == 0) y[row] = a + (bias != nullptr ? bias[row] : 0.0f);
  }
}

unsigned gemv_blocks(int64_t waves) {
  const int64_t b = (waves + kWavesPerBlock - 1) / kWavesPerBlock;
  return static_cast<unsigned>(b < kGemvMaxBlocks ? b : kGemvMaxBlocks);
}

unsigned gemv_reg_blocks(int64_t waves) {
  const int64_t b = (waves + kGemvWaves - 1) / kGemvWaves;
  return static_cast<unsigned>(b < kGemvRegMaxBlocks ? b : kGemvRegMaxBlocks);
}

template <int CPL>
void launch_reg(hipStream_t s, const float* x, int nchunks, const uint16_t* w, int64_t n, const float* bias,
                float* y) {
  if (n >= kBigRows) {
    gemv_reg<CPL, 2><<<gemv_reg_blocks((n + 1) / 2), kGemvBlock, 0, s>>>(x, nchunks, w, n, bias, y);
  } else {
    gemv_reg<CPL, 1><<<gemv_reg_blocks(n), kGemvBlock, 0, s>>>(x, nchunks, w, n, bias, y);
  }
}

// ---- expert routing (used by the fused GEMVs and the expert kernels) ----------------

constexpr int kMaxExperts = 2 * kWave;
constexpr int kMaxExpertSlots = 8;
constexpr int kExpertActFloats = 8192;  // k * ffn staged in LDS by the down kernel

__device__ __forceinline__ bool topk_better(float v, int e, float bv, int be) { return v > bv || (v == bv && e < be); }

// One wave: the softmax and top k of one row of logits lr (global or LDS),
// ids and scores to ids[0..k) and wts[0..k); sv is kMaxExperts floats of
// LDS for this wave. The top k are the experts whose rank is below k, the
// rank of e being the number of experts ahead of it under topk_better (a
// strict total order, so the ranks are 0..experts-1 and equal the rounds in
// which k successive argmaxes would pick them). Each lane ranks its own
// experts against all of them read back from LDS: no dependent shuffles,
// where k wave argmaxes were 12 dependent permutes each. A NaN score ranks
// below every number.
struct TopkLane {
  float v[2];     // the scores of experts lane and lane + 64
  int rank[2];    // their ranks (meaningful below experts)
};

__device__ __forceinline__ TopkLane topk_rank(const float* lr, int experts, float* sv) {
  const int lane = threadIdx.x & (kWave - 1);
  TopkLane t;
  float (&v)[2] = t.v;
  float peak = -INFINITY;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const int e = lane + kWave * i;
    v[i] = e < experts ? lr[e] : -INFINITY;
    peak = fmaxf(peak, v[i]);
  }
  peak = wave_max(peak);
  // A row of -inf logits scores every expert 0, as softmax_rows leaves a
  // fully masked row (src/backend/reference/ops.cpp:175-178).
  const bool dead = peak == -INFINITY;
  double total = 0.0;
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (lane + kWave * i < experts) {
      v[i] = dead ? 0.0f : expf(v[i] - peak);
      total += static_cast<double>(v[i]);
    }
  }
#pragma unroll
  for (int off = kWave / 2; off > 0; off >>= 1) total += __shfl_xor(total, off);
  const float inv = dead ? 0.0f : static_cast<float>(1.0 / total);
#pragma unroll
  for (int i = 0; i < 2; ++i) v[i] = lane + kWave * i < experts ? v[i] * inv : -INFINITY;
  float key[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const bool valid = lane + kWave * i < experts;
    key[i] = valid ? (v[i] == v[i] ? v[i] : -1.0f) : -INFINITY;
    sv[lane + kWave * i] = key[i];
  }
  // A wave's LDS accesses complete in order; the fences keep the compiler
  // from moving the reads above the writes.
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
  __builtin_amdgcn_wave_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  const bool two = experts > kWave;
  const int quads = ((two ? experts : kWave) + 3) / 4;
  int (&rank)[2] = t.rank;
  rank[0] = rank[1] = 0;
  if (two) {
    for (int q = 0; q < quads; ++q) {
      const float4 o = reinterpret_cast<const float4*>(sv)[q];
      const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        rank[0] += topk_better(ov[t], 4 * q + t, key[0], lane) ? 1 : 0;
        rank[1] += topk_better(ov[t], 4 * q + t, key[1], lane + kWave) ? 1 : 0;
      }
    }
  } else {
    for (int q = 0; q < quads; ++q) {
      const float4 o = reinterpret_cast<const float4*>(sv)[q];
      const float ov[4] = {o.x, o.y, o.z, o.w};
#pragma unroll
      for (int t = 0; t < 4; ++t) rank[0] += topk_better(ov[t], 4 * q + t, key[0], lane) ? 1 : 0;
    }
  }
  return t;
}

// The top k of a wave's ranks to ids[0..k) and wts[0..k).
__device__ __forceinline__ void topk_store(const TopkLane& t, int experts, int k, int64_t* ids, float* wts) {
  const int lane = threadIdx.x & (kWave - 1);
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    if (lane + kWave * i < experts && t.rank[i] < k) {
      ids[t.rank[i]] = lane + kWave * i;
      wts[t.rank[i]] = t.v[i];
    }
  }
}

__device__ __forceinline__ void topk_row(const float* lr, int experts, int k, int64_t* ids, float* wts, float* sv) {
  topk_store(topk_rank(lr, experts, sv), experts, k, ids, wts);
}

// ---- fused decode GEMVs ----------------------------------------------------------
//
// The decode step's projections take the residual stream's add + RMSNorm as
// a prologue: every workgroup reduces the one input row itself (k <= 2048,
// a few KB from L2), so the normalised row never round-trips through HBM and
// the norm's launch disappears. The reduction is the row kernel's own
// (norm.hip): 4-float chunks, 64-chunk groups, one wave butterfly per group,
// group sums folded in order, inv formed in fp64; h = w * (s * inv) with no
// contraction. h is therefore bitwise the h that add_rms_norm writes, and y
// bitwise what gemv_bf16 gives on it. With two weight matrices the rows pair
// up (gate row r, up row r) and the epilogue is SwiGLU, so
// y[r] = silu(gate_r . h) (up_r . h), bitwise the swiglu of the two GEMVs.

constexpr int kFusedMaxK = kWave * kGemvRegChunks * 8;  // 2048: bf16(h) stays in VGPRs

struct FusedGemv {
  const float* x;       // residual row [k]
  const float* delta;   // added to x first, or null
  float* x_out;         // x + delta written here by workgroup 0, or null
  const float* w_norm;  // RMSNorm weight [k], or null for h = x (+ delta)
  float* h_out;         // the fp32 h written here by workgroup 0, or null
  const uint16_t* w1;   // [n, k] bf16 (the gate rows when w2 is set)
  const uint16_t* w2;   // [n, k] bf16 up rows, or null
  const float* bias;    // [n] or null (single matrix only)
  float* y;             // [n]
  int64_t n;
  int k;
  float eps;
  // Expert rows (mixture of experts): with ids set, row r of the call is row
  // r mod slot_rows of expert ids[r / slot_rows] in stacks of `experts`
  // experts (an id outside the stack reads expert 0; its rows are not used).
  const int64_t* ids = nullptr;
  int64_t slot_rows = 0;
  int64_t experts = 0;
  // With logits set (the router's [experts] logits), every workgroup takes
  // the top_k itself (expert_topk's rule) and uses those ids; workgroup 0
  // also writes them and their scores to ids_out / wts_out.
  const float* logits = nullptr;
  int top_k = 0;
  int64_t* ids_out = nullptr;
  float* wts_out = nullptr;
  // fp32 rows against the unrounded h (the router's gate, no bias), formed
  // by the workgroups from main_blocks on, one row per wave, exactly as
  // gemv_f32 forms them; main_blocks is set at launch.
  const float* w_f32 = nullptr;
  int64_t n_f32 = 0;
  float* y_f32 = nullptr;
  unsigned main_blocks = 0;
};

// The weight row that output row r of a fused GEMV reads with the ids given.
__device__ __forceinline__ int64_t fused_weight_row(const FusedGemv& a, const int64_t* ids, int64_t r) {
  if (ids == nullptr) return r;
  const int64_t slot = r / a.slot_rows;
  int64_t id = ids[slot];
  id = id >= 0 && id < a.experts ? id : 0;
  return id * a.slot_rows + (r - slot * a.slot_rows);
}

// The prologue: the workgroup holds the row once, in the row kernel's layout
// (4-float chunks v = (wave + 8 g) 64 + lane), reduces it in that kernel's
// order, and writes bf16(h) to LDS, from which every wave reads its 8-float
// GEMV chunks. x, delta and w_norm are read once per workgroup.
template <bool kNorm, class IssueW>
__device__ __forceinline__ void fused_prologue(const FusedGemv& a, float* h_lds, int wave, int lane, IssueW issue_w,
                                               bool round_h = true) {
  __shared__ float red[kMaxGroups];
  constexpr int kG = kFusedMaxK / 4 / kWave / kGemvWaves;  // 1 group per wave
  const int nvec = a.k / 4;
  const int groups = (nvec + kWave - 1) / kWave;
  float s[kG][4], d[kG][4], wn[kG][4];
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const int v = (wave + kGemvWaves * g) * kWave + lane;
    const int vc = v < nvec ? v : nvec - 1;
    load_f32<4>(a.x + 4 * vc, s[g]);
    if (a.delta != nullptr) load_f32<4>(a.delta + 4 * vc, d[g]);
    if constexpr (kNorm) load_f32<4>(a.w_norm + 4 * vc, wn[g]);
  }
  issue_w();
  if (a.delta != nullptr) {
#pragma unroll
    for (int g = 0; g < kG; ++g)
#pragma unroll
      for (int e = 0; e < 4; ++e) s[g][e] += d[g][e];
  }
  float part[kG];
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const int v = (wave + kGemvWaves * g) * kWave + lane;
    part[g] = 0.0f;
    if (v < nvec) {
      if (blockIdx.x == 0 && a.x_out != nullptr) {
        *reinterpret_cast<u32x4*>(a.x_out + 4 * v) = u32x4{__float_as_uint(s[g][0]), __float_as_uint(s[g][1]),
                                                          __float_as_uint(s[g][2]), __float_as_uint(s[g][3])};
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) part[g] += s[g][e] * s[g][e];
    }
  }
  float inv = 0.0f;
  if constexpr (kNorm) {
    const float ss = fold_groups<kGemvWaves, kG>(part, wave, groups, red);
    inv = static_cast<float>(1.0 / sqrt(static_cast<double>(ss) / static_cast<double>(a.k) +
                                        static_cast<double>(a.eps)));
  }
#pragma unroll
  for (int g = 0; g < kG; ++g) {
    const int v = (wave + kGemvWaves * g) * kWave + lane;
    if (v < nvec) {
      float h[4];
      if constexpr (kNorm) {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = wn[g][e] * (s[g][e] * inv);
      } else {
#pragma unroll
        for (int e = 0; e < 4; ++e) h[e] = s[g][e];
      }
      if (blockIdx.x == 0 && a.h_out != nullptr) {
        *reinterpret_cast<u32x4*>(a.h_out + 4 * v) =
            u32x4{__float_as_uint(h[0]), __float_as_uint(h[1]), __float_as_uint(h[2]), __float_as_uint(h[3])};
      }
#pragma unroll
      for (int e = 0; e < 4; ++e) h_lds[4 * v + e] = round_h ? round_bf16(h[e]) : h[e];
    }
  }
  __syncthreads();
}

template <int CPL, int RPW, bool kNorm, bool kPair>
__global__ __launch_bounds__(kGemvBlock) void gemv_fused(const FusedGemv a) {
  constexpr int kMats = kPair ? 2 : 1;
  __shared__ __align__(16) float h_lds[kFusedMaxK];
  const int lane = threadIdx.x & (kWave - 1), wave = threadIdx.x / kWave;
  const int nchunks = a.k / 8;
  const int64_t k = a.k;
  const int64_t groups = (a.n + RPW - 1) / RPW;
  const int64_t step = static_cast<int64_t>(a.main_blocks) * kGemvWaves;
  const int64_t g0 = static_cast<int64_t>(blockIdx.x) * kGemvWaves + wave;

  if (blockIdx.x >= a.main_blocks) {
    // An fp32 row per wave against h unrounded in LDS: chunk c = lane + 64 i
    // in order, fmaf per element, wave butterfly, + 0, as gemv_f32 forms it.
    // The row's chunks are requested before the prologue's arithmetic.
    constexpr int kF32Chunks = kFusedMaxK / 4 / kWave;
    const int nv = a.k / 4;
    const int64_t row = static_cast<int64_t>(blockIdx.x - a.main_blocks) * kGemvWaves + wave;
    const float* wr = a.w_f32 + (row < a.n_f32 ? row : a.n_f32 - 1) * k;
    u32x4 wf[kF32Chunks];
    fused_prologue<kNorm>(
        a, h_lds, wave, lane,
        [&] {
#pragma unroll
          for (int i = 0; i < kF32Chunks; ++i) {
            const int c = lane + kWave * i;
            wf[i] = stream_load(reinterpret_cast<const u32x4*>(wr) + (c < nv ? c : nv - 1));
          }
        },
        false);
    float acc = 0.0f;
#pragma unroll
    for (int i = 0; i < kF32Chunks; ++i) {
      const int c = lane + kWave * i;
      if (c < nv) {
        const float wv[4] = {__uint_as_float(wf[i].x), __uint_as_float(wf[i].y), __uint_as_float(wf[i].z),
                             __uint_as_float(wf[i].w)};
#pragma unroll
        for (int e = 0; e < 4; ++e) acc = fmaf(h_lds[4 * c + e], wv[e], acc);
      }
    }
    acc = wave_sum(acc);
    if (lane == 0 && row < a.n_f32) a.y_f32[row] = acc + 0.0f;
    return;
  }

  // The routed experts' rows: the workgroup's own top k of the router's
  // logits (bitwise expert_topk's), formed by wave 0 once the prologue's row
  // loads are in flight, or the ids given.
  __shared__ __align__(16) float s_scores[kMaxExperts];
  __shared__ int64_t s_ids[kMaxExpertSlots];
  __shared__ float s_wts[kMaxExpertSlots];
  const bool routed = a.logits != nullptr;
  auto weight_row = [&](int64_t r) -> int64_t {
    if (!routed) return fused_weight_row(a, a.ids, r);
    const int64_t slot = r / a.slot_rows;
    int64_t id = s_ids[slot];
    id = id >= 0 && id < a.experts ? id : 0;
    return id * a.slot_rows + (r - slot * a.slot_rows);
  };
  u32x4 wc[kMats][RPW][CPL];
  auto load_w = [&](int64_t g) {
    const int64_t row0 = g * RPW;
#pragma unroll
    for (int m = 0; m < kMats; ++m) {
      const uint16_t* w = m == 0 ? a.w1 : a.w2;
#pragma unroll
      for (int r = 0; r < RPW; ++r) {
        // formed by the whole wave (the expert lookup is a ballot), for a
        // row clamped into [0, n) (the ids path reads ids[row / slot_rows])
        const uint16_t* wrow = w + weight_row(row0 + r < a.n ? row0 + r : a.n - 1) * k;
#pragma unroll
        for (int i = 0; i < CPL; ++i) {
          const int c = lane + kWave * i;
          wc[m][r][i] = u32x4{0u, 0u, 0u, 0u};
          if (row0 + r < a.n && c < nchunks) {
            wc[m][r][i] = stream_load(reinterpret_cast<const u32x4*>(wrow) + c);
          }
        }
      }
    }
  };
  // The prologue's row loads go out first, then the first rows' weights, so
  // both are in flight together and the row's arithmetic waits only for the
  // row (fused QKV 5.03 -> 4.88 us, with x written by the kernel before).
  fused_prologue<kNorm>(a, h_lds, wave, lane, [&] {
    if (routed) {
      if (wave == 0) topk_row(a.logits, static_cast<int>(a.experts), a.top_k, s_ids, s_wts, s_scores);
      __syncthreads();
      if (blockIdx.x == 0 && static_cast<int>(threadIdx.x) < a.top_k) {
        a.ids_out[threadIdx.x] = s_ids[threadIdx.x];
        a.wts_out[threadIdx.x] = s_wts[threadIdx.x];
      }
    }
    if (g0 < groups) load_w(g0);
  });
  float xv[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + kWave * i;
    if (c < nchunks) {
      load_f32<8>(h_lds + 8 * c, xv[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[i][e] = 0.0f;
    }
  }
  for (int64_t g = g0; g < groups; g += step) {
    if (g != g0) load_w(g);
    const int64_t row0 = g * RPW;
    float acc[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) {
      float d1 = 0.0f;
#pragma unroll
      for (int i = 0; i < CPL; ++i) d1 = dot8(wc[0][r][i], xv[i], d1);
      d1 = wave_sum(d1);
      if constexpr (kPair) {
        float d2 = 0.0f;
#pragma unroll
        for (int i = 0; i < CPL; ++i) d2 = dot8(wc[kMats - 1][r][i], xv[i], d2);
        d2 = wave_sum(d2);
        // + 0.0f as the single-matrix store forms its outputs (a -0 sum
        // becomes +0), so the pair matches two GEMVs then silu_mul bitwise.
        acc[r] = silu_mul_f(d1 + 0.0f, d2 + 0.0f);
      } else {
        acc[r] = d1 + (a.bias != nullptr && row0 + r < a.n ? a.bias[row0 + r] : 0.0f);
      }
    }
    for (int r = 0; r < RPW; ++r) {
      if (lane == r && row0 + r < a.n) a.y[row0 + r] = acc[r];
    }
  }
}

template <int CPL, bool kNorm, bool kPair>
void launch_fused_rows(hipStream_t s, const FusedGemv& a) {
  FusedGemv b = a;
  const unsigned f32_blocks = a.w_f32 != nullptr ? static_cast<unsigned>((a.n_f32 + kGemvWaves - 1) / kGemvWaves) : 0u;
  if (a.n >= kBigRows) {
    b.main_blocks = gemv_reg_blocks((a.n + 1) / 2);
    gemv_fused<CPL, 2, kNorm, kPair><<<b.main_blocks + f32_blocks, kGemvBlock, 0, s>>>(b);
  } else {
    b.main_blocks = gemv_reg_blocks(a.n);
    gemv_fused<CPL, 1, kNorm, kPair><<<b.main_blocks + f32_blocks, kGemvBlock, 0, s>>>(b);
  }
}

template <bool kNorm, bool kPair>
void launch_fused(hipStream_t s, const FusedGemv& a) {
  switch ((a.k / 8 + kWave - 1) / kWave) {
    case 1: launch_fused_rows<1, kNorm, kPair>(s, a); break;
    case 2: launch_fused_rows<2, kNorm, kPair>(s, a); break;
    case 3: launch_fused_rows<3, kNorm, kPair>(s, a); break;
    default: launch_fused_rows<kGemvRegChunks, kNorm, kPair>(s, a); break;
  }
}

int fused_entry(const char* what, void* stream, FusedGemv a) {
  UOCR_REQUIRE(a.k >= 0 && a.n >= 0, what, "k and n must be >= 0");
  if (a.n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(a.k % 8 == 0 && a.k >= 8 && a.k <= kFusedMaxK, what, "k must be a multiple of 8 in [8, 2048]");
  UOCR_REQUIRE(a.x != nullptr && a.w1 != nullptr && a.y != nullptr, what, "null x, w or y");
  UOCR_REQUIRE(a.n < (int64_t{1} << 40), what, "n too large");
  UOCR_REQUIRE(aligned16(a.x) && aligned16(a.w1) && (a.w2 == nullptr || aligned16(a.w2)) &&
                   (a.delta == nullptr || aligned16(a.delta)) && (a.x_out == nullptr || aligned16(a.x_out)) &&
                   (a.w_norm == nullptr || aligned16(a.w_norm)) && (a.h_out == nullptr || aligned16(a.h_out)),
               what, "x, delta, x_out, w_norm, h_out and the weights must be 16-byte aligned");
  // Every workgroup reads x and delta while workgroup 0 writes x_out and
  // h_out, so those must not overlap the inputs.
  auto overlaps = [&](const float* out, const float* in) {
    return out != nullptr && in != nullptr && out < in + a.k && in < out + a.k;
  };
  UOCR_REQUIRE(!overlaps(a.x_out, a.x) && !overlaps(a.x_out, a.delta) && !overlaps(a.h_out, a.x) &&
                   !overlaps(a.h_out, a.delta) && !overlaps(a.x_out, a.h_out),
               what, "x_out and h_out must not overlap x, delta or each other");
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  const bool norm = a.w_norm != nullptr, pair = a.w2 != nullptr;
  if (norm && pair) launch_fused<true, true>(s, a);
  else if (norm) launch_fused<true, false>(s, a);
  else if (pair) launch_fused<false, true>(s, a);
  else launch_fused<false, false>(s, a);
  return check_launch(what);
}

// ---- mixture of experts at decode (src/backend/cuda/ops.h:77-90) ------------------
//
// expert_topk: the gate's softmax over each row of logits [rows, experts],
// then the k highest scores (the lower index first on a tie) as expert ids
// and their (unnormalised) scores, the rule of MixtureOfExperts::forward
// (src/model/feed_forward.cpp:36-53): peak = max, total = sum of
// float(exp(v - peak)) in fp64, score = float(exp(v - peak)) * float(1 /
// total). One wave per row, two experts per lane (experts <= 128); an
// expert is picked when fewer than k experts are ahead of it.
//
// expert_ffn_one: the routed experts of one decode row, weights stacked by
// expert (gate/up [experts * ffn, hidden], down [experts * hidden, ffn]):
//   act_j = silu(gate_j . bf16(x)) * (up_j . bf16(x))      (the fused pair
//           GEMV over k * ffn rows, expert rows picked through the ids)
//   out[c] = sum_j w_j (down_j[c] . bf16(act_j))           (in j order)
// with each down product formed exactly as gemv_bf16 forms it, so the call
// is bitwise k pair GEMVs, k GEMVs and the weighted sum (mul then add).

__global__ __launch_bounds__(kBlock) void expert_topk_k(const float* __restrict__ logits, int64_t rows, int experts,
                                                        int k, int64_t* __restrict__ ids, float* __restrict__ wts) {
  __shared__ __align__(16) float sv[kWavesPerBlock][kMaxExperts];
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  topk_row(logits + row * experts, experts, k, ids + row * k, wts + row * k, sv[threadIdx.x / kWave]);
}

// out[c] = sum_j w_j (down[ids[j] * hidden + c] . bf16(act_j)): bf16(act) of
// every slot in LDS; a wave per output row requests the row of every slot,
// then forms each product as gemv_reg does (chunk c = lane + 64 i, dot8 in
// order, wave butterfly, + 0) and adds w_j d_j in slot order. With CPLS > 0
// the shared experts' down row (shared_down [hidden, shared_ffn] against
// bf16(shared_act)) is formed the same way and the sum is added to it: out =
// (shared . act_s + 0) + sum, bitwise their GEMV followed by add_inplace.
// Otherwise out = base + sum (base may be out), or the sum.
template <int CPL, int CPLS>
__global__ __launch_bounds__(kGemvBlock) void expert_down_k(const float* __restrict__ act, int nchunks,
                                                            const uint16_t* __restrict__ down, int64_t hidden,
                                                            const int64_t* __restrict__ ids,
                                                            const float* __restrict__ wts, int k, int64_t experts,
                                                            const float* __restrict__ shared_act, int shared_nchunks,
                                                            const uint16_t* __restrict__ shared_down,
                                                            const float* base, float* out) {
  __shared__ __align__(16) float xs[kExpertActFloats];
  const int lane = threadIdx.x & (kWave - 1);
  const int ffn = nchunks * 8, sffn = shared_nchunks * 8;
  float* xsh = xs + k * ffn;  // bf16(shared_act) after the routed slots
  const int64_t step = static_cast<int64_t>(gridDim.x) * kGemvWaves;
  const int64_t c0 = static_cast<int64_t>(blockIdx.x) * kGemvWaves + threadIdx.x / kWave;
  u32x4 wc[kMaxExpertSlots][CPL];
  u32x4 ws[CPLS > 0 ? CPLS : 1];
  auto load_rows = [&](int64_t c) {
#pragma unroll
    for (int i = 0; i < CPLS; ++i) {
      const int ci = lane + kWave * i;
      ws[i] = u32x4{0u, 0u, 0u, 0u};
      if (ci < shared_nchunks) ws[i] = stream_load(reinterpret_cast<const u32x4*>(shared_down + c * sffn) + ci);
    }
#pragma unroll
    for (int j = 0; j < kMaxExpertSlots; ++j) {
      const int64_t id = j < k ? ids[j] : 0;
      const bool live = j < k && id >= 0 && id < experts;
#pragma unroll
      for (int i = 0; i < CPL; ++i) {
        const int ci = lane + kWave * i;
        wc[j][i] = u32x4{0u, 0u, 0u, 0u};
        if (live && ci < nchunks) wc[j][i] = stream_load(reinterpret_cast<const u32x4*>(down + (id * hidden + c) * ffn) + ci);
      }
    }
  };
  // The first rows' weights go out before the activations are staged (they
  // depend only on the ids), so both are in flight together, as in gemv_reg.
  if (c0 < hidden) load_rows(c0);
  for (int t = threadIdx.x; t < 2 * nchunks * k; t += kGemvBlock) {
    float v[4];
    load_f32<4>(act + 4 * static_cast<int64_t>(t), v);
#pragma unroll
    for (int e = 0; e < 4; ++e) xs[4 * t + e] = round_bf16(v[e]);
  }
  if constexpr (CPLS > 0) {
    for (int t = threadIdx.x; t < 2 * shared_nchunks; t += kGemvBlock) {
      float v[4];
      load_f32<4>(shared_act + 4 * static_cast<int64_t>(t), v);
#pragma unroll
      for (int e = 0; e < 4; ++e) xsh[4 * t + e] = round_bf16(v[e]);
    }
  }
  __syncthreads();
  auto dot_lds = [&](const u32x4* wrow, const float* xrow, int n_chunks, auto cpl) {
    constexpr int kC = decltype(cpl)::value;
    float a = 0.0f;
#pragma unroll
    for (int i = 0; i < kC; ++i) {
      const int ci = lane + kWave * i;
      float xv[8];
      if (ci < n_chunks) {
        load_f32<8>(xrow + 8 * ci, xv);
      } else {
#pragma unroll
        for (int e = 0; e < 8; ++e) xv[e] = 0.0f;
      }
      a = dot8(wrow[i], xv, a);
    }
    return wave_sum(a) + 0.0f;
  };
  for (int64_t c = c0; c < hidden; c += step) {
    if (c != c0) load_rows(c);
    float total = 0.0f;
#pragma unroll
    for (int j = 0; j < kMaxExpertSlots; ++j) {
      if (j < k && ids[j] >= 0 && ids[j] < experts) {
        const float d = dot_lds(wc[j], xs + j * ffn, nchunks, std::integral_constant<int, CPL>{});
        {
#pragma clang fp contract(off)
          total = total + wts[j] * d;
        }
      }
    }
    float r;
    if constexpr (CPLS > 0) {
      r = dot_lds(ws, xsh, shared_nchunks, std::integral_constant<int, CPLS>{}) + total;
    } else {
      r = base != nullptr ? base[c] + total : total;
    }
    if (lane == 0) out[c] = r;
  }
}

template <int CPL>
void launch_expert_down(hipStream_t s, unsigned blocks, int cpls, const float* act, int nchunks, const uint16_t* down,
                        int64_t hidden, const int64_t* ids, const float* wts, int k, int64_t experts,
                        const float* shared_act, int shared_nchunks, const uint16_t* shared_down, const float* base,
                        float* out) {
#define UOCR_EXPERT_DOWN(S)                                                                                   \
  expert_down_k<CPL, S><<<blocks, kGemvBlock, 0, s>>>(act, nchunks, down, hidden, ids, wts, k, experts,      \
                                                     shared_act, shared_nchunks, shared_down, base, out)
  switch (cpls) {
    case 0: UOCR_EXPERT_DOWN(0); break;
    case 1: UOCR_EXPERT_DOWN(1); break;
    case 2: UOCR_EXPERT_DOWN(2); break;
    case 3: UOCR_EXPERT_DOWN(3); break;
    default: UOCR_EXPERT_DOWN(kGemvRegChunks); break;
  }
#undef UOCR_EXPERT_DOWN
}

// y[n] = x . w[n, :] (+ bias[n]) with fp32 weights and no rounding of x: the
// mixture-of-experts gate, which the reference keeps in fp32 for routing
// (moe_gate_f32, src/model/cuda/cuda_decoder.cpp:141-142). One wave per row,
// 16-byte chunks when k and the pointers allow, a wave butterfly.
// One wave: x . wr over k fp32 elements (chunk c = lane + 64 i in order).
template <bool kVec>
__device__ __forceinline__ float dot_f32_row(const float* x, const float* wr, int64_t k) {
  const int lane = threadIdx.x & (kWave - 1);
  float a = 0.0f;
  if constexpr (kVec) {
    for (int64_t c = lane; c < k / 4; c += kWave) {
      float xv[4], wv[4];
      load_f32<4>(x + 4 * c, xv);
      const u32x4 q = stream_load(reinterpret_cast<const u32x4*>(wr) + c);
      wv[0] = __uint_as_float(q.x);
      wv[1] = __uint_as_float(q.y);
      wv[2] = __uint_as_float(q.z);
      wv[3] = __uint_as_float(q.w);
#pragma unroll
      for (int e = 0; e < 4; ++e) a = fmaf(xv[e], wv[e], a);
    }
  } else {
    for (int64_t c = lane; c < k; c += kWave) a = fmaf(x[c], wr[c], a);
  }
  return wave_sum(a);
}

template <bool kVec>
__global__ __launch_bounds__(kBlock) void gemv_f32_k(const float* __restrict__ x, int64_t k,
                                                     const float* __restrict__ w, int64_t n,
                                                     const float* __restrict__ bias, float* __restrict__ y) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave; row < n; row += step) {
    const float a = dot_f32_row<kVec>(x, w + row * k, k);
    if (lane == 0) y[row] = a + (bias != nullptr ? bias[row] : 0.0f);
  }
}


}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_gemv_bf16(void* stream, const float* x, int64_t k, const uint16_t* w, int64_t n, const float* bias,
                        float* y) {
  const char* what = "uocr_rocm_gemv_bf16";
  UOCR_REQUIRE(k >= 0 && n >= 0, what, "k and n must be >= 0");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(y != nullptr, what, "null y");
  UOCR_REQUIRE(k <= kGemvMaxK, what, "k above 12288");
  UOCR_REQUIRE(k == 0 || (x != nullptr && w != nullptr), what, "null x or w");
  UOCR_REQUIRE(n < (int64_t{1} << 40), what, "n too large");
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  const bool vec = k > 0 && k % 8 == 0 && aligned16(x) && aligned16(w);
  if (!vec) {
    gemv_any<<<gemv_blocks(n), kBlock, 0, s>>>(x, k, w, n, bias, y);
    return check_launch(what);
  }
  const int nchunks = static_cast<int>(k / 8);
  const int cpl = (nchunks + kWave - 1) / kWave;
  switch (cpl) {
    case 1: launch_reg<1>(s, x, nchunks, w, n, bias, y); break;
    case 2: launch_reg<2>(s, x, nchunks, w, n, bias, y); break;
    case 3: launch_reg<3>(s, x, nchunks, w, n, bias, y); break;
    case kGemvRegChunks: launch_reg<kGemvRegChunks>(s, x, nchunks, w, n, bias, y); break;
    default:
      gemv_lds<<<gemv_blocks(n), kBlock, static_cast<size_t>(k) * sizeof(float), s>>>(x, nchunks, w, n, bias, y);
      break;
  }
  return check_launch(what);
}

int uocr_rocm_attend_merge_gemv_bf16(void* stream, const float* scratch, int64_t heads, int64_t hd,
                                     int64_t max_live, const uint16_t* w, int64_t n, const float* bias, float* y,
                                     float* x_out) {
  const char* what = "uocr_rocm_attend_merge_gemv_bf16";
  UOCR_REQUIRE(heads >= 1 && hd >= 1 && n >= 0, what, "heads and hd must be >= 1, n >= 0");
  const int64_t k = heads * hd;
  UOCR_REQUIRE(k % 8 == 0 && k <= int64_t{kWave} * kGemvRegChunks * 8, what,
               "heads * hd must be a multiple of 8 and at most 2048");
  UOCR_REQUIRE(max_live >= 1, what, "max_live must be >= 1");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(scratch != nullptr && w != nullptr && y != nullptr, what, "null pointer");
  UOCR_REQUIRE(aligned16(w), what, "w must be 16-byte aligned");
  UOCR_REQUIRE(n < (int64_t{1} << 40), what, "n too large");
  const MergedX mx{scratch, static_cast<int>(heads), static_cast<int>(hd), segment_splits(max_live), x_out};
  const int nchunks = static_cast<int>(k / 8);
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  const unsigned blocks = gemv_reg_blocks(n);
  switch ((nchunks + kWave - 1) / kWave) {
    case 1: gemv_reg<1, 1, true><<<blocks, kGemvBlock, 0, s>>>(nullptr, nchunks, w, n, bias, y, mx); break;
    case 2: gemv_reg<2, 1, true><<<blocks, kGemvBlock, 0, s>>>(nullptr, nchunks, w, n, bias, y, mx); break;
    case 3: gemv_reg<3, 1, true><<<blocks, kGemvBlock, 0, s>>>(nullptr, nchunks, w, n, bias, y, mx); break;
    default:
      gemv_reg<kGemvRegChunks, 1, true><<<blocks, kGemvBlock, 0, s>>>(nullptr, nchunks, w, n, bias, y, mx);
      break;
  }
  return check_launch(what);
}

int uocr_rocm_add_rms_norm_gemv_bf16(void* stream, const float* x, const float* delta, float* x_out,
                                     const float* w_norm, float eps, float* h_out, int64_t k, const uint16_t* w,
                                     int64_t n, const float* bias, float* y) {
  if (k < 0 || k > kFusedMaxK) return fail(UOCR_ROCM_INVALID_ARGUMENT, "uocr_rocm_add_rms_norm_gemv_bf16",
                                           "k must be a multiple of 8 in [8, 2048]");
  return fused_entry("uocr_rocm_add_rms_norm_gemv_bf16", stream,
                     FusedGemv{x, delta, x_out, w_norm, h_out, w, nullptr, bias, y, n, static_cast<int>(k), eps});
}

int uocr_rocm_add_rms_norm_swiglu_gemv_bf16(void* stream, const float* x, const float* delta, float* x_out,
                                            const float* w_norm, float eps, float* h_out, int64_t k,
                                            const uint16_t* w_gate, const uint16_t* w_up, int64_t ffn, float* act) {
  const char* what = "uocr_rocm_add_rms_norm_swiglu_gemv_bf16";
  if (k < 0 || k > kFusedMaxK) return fail(UOCR_ROCM_INVALID_ARGUMENT, what, "k must be a multiple of 8 in [8, 2048]");
  UOCR_REQUIRE(ffn == 0 || w_up != nullptr, what, "null up weights");
  return fused_entry(what, stream,
                     FusedGemv{x, delta, x_out, w_norm, h_out, w_gate, w_up, nullptr, act, ffn, static_cast<int>(k),
                               eps});
}

int uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16(void* stream, const float* x, const float* delta, float* x_out,
                                                   const float* w_norm, float eps, float* h_out, int64_t k,
                                                   const uint16_t* w_gate, const uint16_t* w_up, int64_t ffn,
                                                   float* act, const float* router, int64_t experts, float* logits) {
  const char* what = "uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16";
  if (k < 0 || k > kFusedMaxK) return fail(UOCR_ROCM_INVALID_ARGUMENT, what, "k must be a multiple of 8 in [8, 2048]");
  UOCR_REQUIRE(ffn >= 1 && experts >= 1 && experts <= (int64_t{1} << 20), what,
               "ffn must be >= 1 and experts in [1, 2^20]");
  UOCR_REQUIRE(w_up != nullptr && router != nullptr && logits != nullptr, what, "null up, router or logits");
  UOCR_REQUIRE(aligned16(router), what, "the router weights must be 16-byte aligned");
  auto overlaps = [&](const float* in) { return in != nullptr && logits < in + k && in < logits + experts; };
  UOCR_REQUIRE(!overlaps(x) && !overlaps(delta) && !overlaps(x_out) && !overlaps(h_out), what,
               "logits must not overlap x, delta, x_out or h_out");
  FusedGemv a{x, delta, x_out, w_norm, h_out, w_gate, w_up, nullptr, act, ffn, static_cast<int>(k), eps};
  a.w_f32 = router;
  a.n_f32 = experts;
  a.y_f32 = logits;
  return fused_entry(what, stream, a);
}

int uocr_rocm_gemv_f32(void* stream, const float* x, int64_t k, const float* w, int64_t n, const float* bias,
                       float* y) {
  const char* what = "uocr_rocm_gemv_f32";
  UOCR_REQUIRE(k >= 0 && n >= 0, what, "k and n must be >= 0");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(y != nullptr && (k == 0 || (x != nullptr && w != nullptr)), what, "null pointer");
  UOCR_REQUIRE(n < (int64_t{1} << 40) && k < (int64_t{1} << 40), what, "n or k too large");
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  if (k % 4 == 0 && aligned16(x) && aligned16(w)) {
    gemv_f32_k<true><<<gemv_blocks(n), kBlock, 0, s>>>(x, k, w, n, bias, y);
  } else {
    gemv_f32_k<false><<<gemv_blocks(n), kBlock, 0, s>>>(x, k, w, n, bias, y);
  }
  return check_launch(what);
}

int uocr_rocm_expert_topk(void* stream, const float* logits, int64_t rows, int64_t experts, int64_t k, int64_t* ids,
                          float* weights) {
  const char* what = "uocr_rocm_expert_topk";
  UOCR_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), what, "rows must be in [0, 2^31)");
  UOCR_REQUIRE(experts >= 1 && experts <= kMaxExperts, what, "experts must be in [1, 128]");
  UOCR_REQUIRE(k >= 1 && k <= experts, what, "k must be in [1, experts]");
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(logits != nullptr && ids != nullptr && weights != nullptr, what, "null pointer");
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  expert_topk_k<<<blocks_for_rows(rows), kBlock, 0, s>>>(logits, rows, static_cast<int>(experts), static_cast<int>(k),
                                                          ids, weights);
  return check_launch(what);
}

int64_t uocr_rocm_expert_scratch_floats(int64_t k, int64_t ffn) { return k > 0 && ffn > 0 ? k * ffn : 0; }

namespace {

int expert_ffn_entry(const char* what, void* stream, const float* x, int64_t hidden, int64_t ffn,
                     const uint16_t* gate, const uint16_t* up, const uint16_t* down, int64_t experts,
                     const float* logits, int64_t* ids, float* weights, int64_t k, const float* shared_act,
                     const uint16_t* shared_down, int64_t shared_ffn, const float* base, float* scratch, float* out) {
  UOCR_REQUIRE(hidden % 8 == 0 && hidden >= 8 && hidden <= kFusedMaxK, what,
               "hidden must be a multiple of 8 in [8, 2048]");
  UOCR_REQUIRE(ffn % 8 == 0 && ffn >= 8 && ffn / 8 <= kWave * kGemvRegChunks, what,
               "ffn must be a multiple of 8 in [8, 2048]");
  UOCR_REQUIRE(k >= 1 && k <= kMaxExpertSlots && k * ffn + shared_ffn <= kExpertActFloats, what,
               "k must be in [1, 8] with k * ffn (+ shared_ffn) <= 8192");
  UOCR_REQUIRE(shared_ffn == 0 || (shared_ffn % 8 == 0 && shared_ffn / 8 <= kWave * kGemvRegChunks &&
                                   shared_act != nullptr && shared_down != nullptr && aligned16(shared_act) &&
                                   aligned16(shared_down) && base == nullptr),
               what, "shared_ffn must be a multiple of 8 in [8, 2048] with shared_act and shared_down 16-byte "
                     "aligned, and no base");
  UOCR_REQUIRE(experts >= 1, what, "experts must be >= 1");
  UOCR_REQUIRE(x != nullptr && gate != nullptr && up != nullptr && down != nullptr && ids != nullptr &&
                   weights != nullptr && scratch != nullptr && out != nullptr,
               what, "null pointer");
  UOCR_REQUIRE(aligned16(x) && aligned16(gate) && aligned16(up) && aligned16(down) && aligned16(scratch), what,
               "x, the weights and scratch must be 16-byte aligned");
  auto overlaps = [](const float* a, int64_t na, const float* b, int64_t nb) { return a < b + nb && b < a + na; };
  UOCR_REQUIRE(!overlaps(scratch, k * ffn, x, hidden) && !overlaps(scratch, k * ffn, out, hidden) &&
                   !overlaps(out, hidden, x, hidden) && (base == nullptr || !overlaps(scratch, k * ffn, base, hidden)),
               what, "x, base, scratch and out must not overlap (base may be out itself)");
  FusedGemv a{x, nullptr, nullptr, nullptr, nullptr, gate, up, nullptr, scratch, k * ffn, static_cast<int>(hidden),
              0.0f};
  a.slot_rows = ffn;
  a.experts = experts;
  if (logits != nullptr) {
    UOCR_REQUIRE(experts <= kMaxExperts && k <= experts, what,
                 "experts must be in [1, 128] and k <= experts with router logits");
    a.logits = logits;
    a.top_k = static_cast<int>(k);
    a.ids_out = ids;
    a.wts_out = weights;
  } else {
    a.ids = ids;
  }
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  launch_fused<false, true>(s, a);
  const int nchunks = static_cast<int>(ffn / 8), snchunks = static_cast<int>(shared_ffn / 8);
  const unsigned blocks = gemv_reg_blocks(hidden);
  const int kk = static_cast<int>(k), cpls = (snchunks + kWave - 1) / kWave;
  switch ((nchunks + kWave - 1) / kWave) {
    case 1: launch_expert_down<1>(s, blocks, cpls, scratch, nchunks, down, hidden, ids, weights, kk, experts, shared_act, snchunks, shared_down, base, out); break;
    case 2: launch_expert_down<2>(s, blocks, cpls, scratch, nchunks, down, hidden, ids, weights, kk, experts, shared_act, snchunks, shared_down, base, out); break;
    case 3: launch_expert_down<3>(s, blocks, cpls, scratch, nchunks, down, hidden, ids, weights, kk, experts, shared_act, snchunks, shared_down, base, out); break;
    default: launch_expert_down<kGemvRegChunks>(s, blocks, cpls, scratch, nchunks, down, hidden, ids, weights, kk, experts, shared_act, snchunks, shared_down, base, out); break;
  }
  return check_launch(what);
}

}  // namespace

int uocr_rocm_expert_ffn_one(void* stream, const float* x, int64_t hidden, int64_t ffn, const uint16_t* gate,
                             const uint16_t* up, const uint16_t* down, int64_t experts, const int64_t* ids,
                             const float* weights, int64_t k, const float* base, float* scratch, float* out) {
  return expert_ffn_entry("uocr_rocm_expert_ffn_one", stream, x, hidden, ffn, gate, up, down, experts, nullptr,
                          const_cast<int64_t*>(ids), const_cast<float*>(weights), k, nullptr, nullptr, 0, base,
                          scratch, out);
}

int uocr_rocm_moe_ffn_one(void* stream, const float* x, int64_t hidden, int64_t ffn, const uint16_t* gate,
                          const uint16_t* up, const uint16_t* down, int64_t experts, const float* logits, int64_t k,
                          int64_t* ids, float* weights, const float* shared_act, const uint16_t* shared_down,
                          int64_t shared_ffn, float* scratch, float* out) {
  const char* what = "uocr_rocm_moe_ffn_one";
  UOCR_REQUIRE(shared_ffn >= 8, what, "shared_ffn must be a multiple of 8 in [8, 2048]");
  UOCR_REQUIRE(logits != nullptr, what, "null logits");
  return expert_ffn_entry(what, stream, x, hidden, ffn, gate, up, down, experts, logits, ids, weights, k, shared_act,
                          shared_down, shared_ffn, nullptr, scratch, out);
}

}  // extern "C"
