// norm.hip: RMSNorm, residual add fused with RMSNorm, and LayerNorm for
// gfx950, fp32 and bf16 activations, fp32 arithmetic, fp32 norm weights.
//
// Layout: x [rows, cols] row-major, cut into 128-bit chunks (VW elements)
// and the chunks into groups of 64 (one chunk per lane). A row is held in
// registers by WPR waves (1, or 4 when there are too few rows to fill the
// GPU with one wave per row): wave w owns groups w, w + WPR, w + 2 WPR, ...
// (workgroups of 4 waves, or of one wave for one-wave rows below 8192 rows),
// so the row is read from HBM once and written once. Rows wider than 64
// groups take the *_wide kernels: one workgroup per row and a second read of
// the row.
//
// Reduction order: each group's sum is a lane sum over its VW elements in
// order, then a DPP butterfly over the 64 lanes (wave_sum); the row's sum
// folds the group sums left to right in group order (through LDS when
// WPR > 1). The order depends only on cols, so a row's result is bitwise
// the same whatever the number of rows in the call and whatever WPR.
//
// Arithmetic (reference: src/backend/reference/ops.cpp:111-141):
//   rms_norm:    ss = sum x^2 (fp32), inv = float(1 / sqrt(ss / cols + eps))
//                evaluated in fp64 as the reference does, y = w * (x * inv).
//   layer_norm:  mean = sum x / cols, var = sum (x - mean)^2 / cols (two
//                passes over the registers, fp32), inv as above in fp64 from
//                var, y = ((x - mean) * inv) * w + b.
//   add_rms_norm: s = x + delta (fp32), x <- s, h <- w * (s * inv(s)).
//   router_norm: non-finite x count as 0; y = clamp(clamp(x inv) (1 + w))
//                with clamp to [-1e4, 1e4] (src/model/decoder.cpp:20-34).
// The output expressions are evaluated without FMA contraction so that each
// product and sum is rounded where the reference rounds it. Norm weights are
// shared by every row (cache resident): they are requested in batches between
// the reductions (kWeightEarlyQ, kWeightMidQ), or staged once per workgroup
// through LDS for calls of kOneRowGroupsBelow rows or more. Loads and stores
// are issued without branches (clamped chunks, dropped stores) so that the
// compiler's waits on the row loads stay exact.

#include <type_traits>

#include "common.hpp"

namespace uocr_rocm {
namespace {

// kRouter: the router's RMSNorm (non-finite inputs count as 0, output
// clamp(clamp(x inv, +-1e4) (1 + w), +-1e4); src/model/decoder.cpp:20-34).
// kLayerToBf16: layer_norm out of place, x read only and y = bf16 of the
// normed row (nearest even) into h: the arithmetic of kLayer with the
// rounding a following projection applies to its input.
enum class Norm { kRms, kAddRms, kLayer, kRouter, kEmbedRms, kLayerToBf16 };

// kEmbedRms's row source: the bf16 table row of state->token (a zero row for
// a token outside [0, table_rows) when table_rows >= 0).
struct EmbedSrc {
  const uint16_t* table;
  int64_t table_rows;
  const uocr_rocm_step_state* state;
};

constexpr float kActClamp = 1.0e4f;

__device__ __forceinline__ float clamp_act(float v) { return fminf(fmaxf(v, -kActClamp), kActClamp); }

// TB threads per workgroup: kBlock, or one wave (one row per workgroup) for
// one-wave rows in calls of fewer than kOneRowGroupsBelow rows. At 2048-4096
// rows of 1024-2048 columns the one-wave groups ran LayerNorm and RMSNorm 2-8%
// faster (add + RMSNorm -6% to +3%), also against 4- and 8-wave groups that
// share the weights through LDS (LayerNorm [4096, 1024] 4.46 against 4.66
// and 4.76 us); at 8192 rows the 4-wave groups with shared weights are
// faster (add+RMSNorm [8192, 2048] 1.5%).
constexpr int64_t kOneRowGroupsBelow = 8192;
// Workgroup size for one-wave rows below kOneRowGroupsBelow rows (no weight
// sharing), and the row count below which a row of 4 or more 64-chunk groups
// is spread over 4 waves (fp32 RMSNorm [1024, 2048]: one-wave rows and
// spread rows ran alike; at 512 rows spreading is faster).
constexpr int kSmallRowsBlock = kWave;
constexpr int64_t kSpreadRowsBelow = 1024;
// When a wave that does not share its weights through LDS requests them, in
// quarters of its chunks: kWeightEarlyQ right after its row loads,
// kWeightMidQ after the first fold, the rest after the last fold. The
// weights are 4 (RMSNorm) or 8 (LayerNorm) bytes per element against the
// row's 2 (bf16) or 4, and they pass through the same per-CU load path as
// the row: requested with the row they delay the row loads of the waves
// dispatched next (LayerNorm [4096, 1024] bf16 5.4 us against 4.5 us), and
// requested one chunk at a time just before its store they wait a round trip
// each. Swept over 19 norm shapes against the earlier per-chunk loads:
// 0 / 1 was the best or within 2% on 16 of them (LayerNorm [4096, 1024]
// bf16 4.70 -> 4.53 us, add+RMSNorm [2048, 2048] bf16 7.47 -> 6.34 us).
constexpr int kWeightEarlyQ = 0;
constexpr int kWeightMidQ = 1;

template <class T, int VW, int WPR, int VPL, Norm kMode, int TB, bool kShareW>
__global__ __launch_bounds__(TB) void norm_rows(T* __restrict__ x, const T* __restrict__ delta,
                                                const float* __restrict__ w, const float* __restrict__ b,
                                                T* __restrict__ h, int64_t rows, int cols, float eps,
                                                EmbedSrc src) {
  constexpr bool kEmbed = kMode == Norm::kEmbedRms;
  constexpr bool kTwoOut = kMode == Norm::kAddRms || kEmbed;  // writes x' and h
  constexpr bool kLn = kMode == Norm::kLayer || kMode == Norm::kLayerToBf16;
  constexpr bool kToBf16 = kMode == Norm::kLayerToBf16;  // h holds the bf16 output rows
  using OutT = typename std::conditional<kToBf16, uint16_t, T>::type;
  constexpr int kRowsPerBlock = TB / kWave / WPR;
  __shared__ float red[kRowsPerBlock][kMaxGroups];
  // One-wave rows in multi-wave workgroups share the norm weights through
  // LDS: the block's waves each request a slice of w (and b) right after
  // their row loads, write it to LDS after the fold, and every row reads its
  // weights back from LDS. One request per block instead of one per row.
  constexpr int kWavesPerGroup = TB / kWave;
  constexpr bool kStage = kShareW && WPR == 1 && kWavesPerGroup > 1 && VPL <= 8;
  constexpr int kStageSlices = kStage ? (VPL + kWavesPerGroup - 1) / kWavesPerGroup : 1;
  constexpr bool kStageB = kStage && kLn;
  // Without staging, every wave requests its own weights in three batches
  // of chunks: kE right after its row loads, kM after the first fold and the
  // rest after the last fold (kWeightEarlyQ / kWeightMidQ quarters of VPL).
  constexpr int kE = kStage ? 0 : (VPL * kWeightEarlyQ + 3) / 4;
  constexpr int kM = kStage ? 0 : ((VPL * kWeightMidQ + 3) / 4 < VPL - kE ? (VPL * kWeightMidQ + 3) / 4 : VPL - kE);
  __shared__ __attribute__((aligned(16))) float wst[kStage ? VPL * kWave * VW : 1];
  __shared__ __attribute__((aligned(16))) float bst[kStageB ? VPL * kWave * VW : 1];
  const int wave = wave_in_block();
  const int lane = threadIdx.x & (kWave - 1);
  const int rloc = wave / WPR, wr = wave % WPR;
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kRowsPerBlock + rloc;
  // Waves past the last row still take part in the block's barriers; their
  // stores go to a zero-size resource and are dropped.
  const bool active = row < rows;
  const int nvec = cols / VW;
  const int groups = (nvec + kWave - 1) / kWave;
  const int64_t off = (active ? row : 0) * cols;

  // Every lane issues its row loads unconditionally: a chunk past the row
  // (v >= nvec) or a wave past the last row reads a valid chunk instead and
  // its values are dropped below. With no branch around them, the compiler
  // waits for each chunk's own loads only (vmcnt counts down in order), so
  // chunk k is formed, folded into its partial and its x' stored while
  // chunks k + 1, ... are still in flight.
  Chunk<T, VW> cx[VPL];
  Chunk<T, VW> cd[VPL];
  Chunk<uint16_t, VW> ce[kEmbed ? VPL : 1];
  bool live[VPL];
  const uint16_t* erow = nullptr;
  bool erow_valid = false;
  if constexpr (kEmbed) {
    const int64_t id = src.state->token;
    erow_valid = src.table_rows < 0 || (id >= 0 && id < src.table_rows);
    erow = src.table + (erow_valid ? id : 0) * cols;
  }
  // Row bases are wave-uniform; a lane adds a 32-bit element offset.
  T* const xrow = x + off;
  const T* const drow = delta != nullptr ? delta + off : nullptr;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = (wr + WPR * k) * kWave + lane;
    live[k] = active && v < nvec;
    const uint32_t at = static_cast<uint32_t>(v < nvec ? v : nvec - 1) * VW;
    if constexpr (kEmbed) {
      ce[k].load(erow + at);
      if (delta != nullptr) cd[k].load(drow + at);
    } else {
      cx[k].load(xrow + at);
      if constexpr (kMode == Norm::kAddRms) cd[k].load(drow + at);
    }
  }

  // The weights, requested behind the row (clamped chunks, no branch): they
  // arrive while the row is reduced.
  float wsl[kStageSlices][VW], bsl[kStageB ? kStageSlices : 1][VW];
  float wv[kStage ? 1 : VPL][VW], bv[!kStage && kLn ? VPL : 1][VW];
  // Chunks [k0, k1)'s weights; the scheduling barriers keep each batch where
  // it is written.
  auto load_weights = [&](auto k0, auto k1) {
    if constexpr (!kStage && decltype(k0)::value < decltype(k1)::value) {
      __builtin_amdgcn_sched_barrier(0);
#pragma unroll
      for (int k = decltype(k0)::value; k < decltype(k1)::value; ++k) {
        const int v = (wr + WPR * k) * kWave + lane;
        const int vc = v < nvec ? v : nvec - 1;
        load_f32<VW>(w + vc * VW, wv[k]);
        if constexpr (kLn) load_f32<VW>(b + vc * VW, bv[k]);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  };
  using C0 = std::integral_constant<int, 0>;
  using CE = std::integral_constant<int, kE>;
  using CM = std::integral_constant<int, kE + kM>;
  using CV = std::integral_constant<int, VPL>;
  if constexpr (kStage) {
#pragma unroll
    for (int j = 0; j < kStageSlices; ++j) {
      const int g = wave + kWavesPerGroup * j;
      const int v = (g < groups ? g : groups - 1) * kWave + lane;
      const int vc = v < nvec ? v : nvec - 1;
      load_f32<VW>(w + vc * VW, wsl[j]);
      if constexpr (kStageB) load_f32<VW>(b + vc * VW, bsl[j]);
    }
  } else {
    load_weights(C0{}, CE{});
  }

  // x' leaves through a resource over this row (nothing for an idle wave).
  const __amdgpu_buffer_rsrc_t xres = buffer_rsrc(xrow, active ? static_cast<uint32_t>(cols) * sizeof(T) : 0u);
  float s[VPL][VW];
  float part[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = (wr + WPR * k) * kWave + lane;
    if constexpr (kEmbed) {
      ce[k].widen(s[k]);
#pragma unroll
      for (int e = 0; e < VW; ++e) s[k][e] = erow_valid ? s[k][e] : 0.0f;
      if (delta != nullptr) {
        float d[VW];
        cd[k].widen(d);
#pragma unroll
        for (int e = 0; e < VW; ++e) s[k][e] += d[e];
      }
    } else {
      cx[k].widen(s[k]);
    }
    if constexpr (kMode == Norm::kAddRms) {
      float d[VW];
      cd[k].widen(d);
#pragma unroll
      for (int e = 0; e < VW; ++e) s[k][e] += d[e];
    }
    if constexpr (kMode == Norm::kRouter) {
#pragma unroll
      for (int e = 0; e < VW; ++e) s[k][e] = __builtin_isfinite(s[k][e]) ? s[k][e] : 0.0f;
    }
    part[k] = 0.0f;
#pragma unroll
    for (int e = 0; e < VW; ++e) part[k] += kLn ? s[k][e] : s[k][e] * s[k][e];
    part[k] = live[k] ? part[k] : 0.0f;  // a dropped chunk adds nothing
    // x' = x + delta does not depend on the reduction: it leaves as soon as
    // its chunk is formed, so half of the kernel's writes overlap the row
    // loads still in flight.
    if constexpr (kTwoOut) {
      Chunk<T, VW> xs;
      xs.narrow(s[k]);
      store_chunk(xres, v < nvec ? static_cast<uint32_t>(v) * VW * sizeof(T) : kDropOffset, xs);
    }
  }

  float inv;
  if constexpr (kLn) {
    const float mean = fold_groups<WPR, VPL>(part, wr, groups, red[rloc]) / static_cast<float>(cols);
    load_weights(CE{}, CM{});
#pragma unroll
    for (int k = 0; k < VPL; ++k) {
      const int v = (wr + WPR * k) * kWave + lane;
      part[k] = 0.0f;
      if (active && v < nvec) {
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          s[k][e] -= mean;
          part[k] += s[k][e] * s[k][e];
        }
      }
    }
    const float var = fold_groups<WPR, VPL>(part, wr, groups, red[rloc]) / static_cast<float>(cols);
    inv = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + static_cast<double>(eps)));
  } else {
    const float ss = fold_groups<WPR, VPL>(part, wr, groups, red[rloc]);
    load_weights(CE{}, CM{});
    inv = static_cast<float>(1.0 / sqrt(static_cast<double>(ss) / static_cast<double>(cols) +
                                        static_cast<double>(eps)));
  }
  if constexpr (kStage) {
#pragma unroll
    for (int j = 0; j < kStageSlices; ++j) {
      const int g = wave + kWavesPerGroup * j;
      if (g < groups) {
#pragma unroll
        for (int e = 0; e < VW; ++e) {
          wst[(g * kWave + lane) * VW + e] = wsl[j][e];
          if constexpr (kStageB) bst[(g * kWave + lane) * VW + e] = bsl[j][e];
        }
      }
    }
    lds_barrier();
  } else {
    load_weights(CM{}, CV{});
  }

  OutT* const orow = kToBf16 ? reinterpret_cast<OutT*>(reinterpret_cast<uint16_t*>(h) + off)
                             : reinterpret_cast<OutT*>((kTwoOut ? h : x) + off);
  const __amdgpu_buffer_rsrc_t ores = buffer_rsrc(orow, active ? static_cast<uint32_t>(cols) * sizeof(OutT) : 0u);
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = (wr + WPR * k) * kWave + lane;
    float wk[VW], bk[VW], y[VW];
    if constexpr (kStage) {
      const int vc = v < nvec ? v : nvec - 1;
      load_f32<VW>(wst + vc * VW, wk);
      if constexpr (kLn) load_f32<VW>(bst + vc * VW, bk);
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        wk[e] = wv[k][e];
        if constexpr (kLn) bk[e] = bv[k][e];
      }
    }
    {
#pragma clang fp contract(off)
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        if constexpr (kLn) {
          y[e] = (s[k][e] * inv) * wk[e] + bk[e];
        } else if constexpr (kMode == Norm::kRouter) {
          y[e] = clamp_act(clamp_act(s[k][e] * inv) * (1.0f + wk[e]));
        } else {
          y[e] = wk[e] * (s[k][e] * inv);
        }
      }
    }
    Chunk<OutT, VW> o;
    o.narrow(y);
    store_chunk(ores, v < nvec ? static_cast<uint32_t>(v) * VW * sizeof(OutT) : kDropOffset, o);
  }
}

// ---- wide rows: one workgroup per row, row read twice (or three times) -----

template <class T>
__device__ __forceinline__ float ld1(const T* p) {
  Chunk<T, 1> c;
  c.load(p);
  float v[1];
  c.widen(v);
  return v[0];
}

template <class T>
__device__ __forceinline__ void st1(T* p, float f) {
  Chunk<T, 1> c;
  const float v[1] = {f};
  c.narrow(v);
  c.store(p);
}

template <class T, bool kAdd, bool kRouter = false>
__global__ __launch_bounds__(kBlock) void rms_rows_wide(T* x, const T* delta, const float* w, T* h, int64_t cols,
                                                        float eps) {
  __shared__ float red[kWavesPerBlock];
  const int64_t off = static_cast<int64_t>(blockIdx.x) * cols;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    float s = ld1(x + off + i);
    if constexpr (kAdd) s += ld1(delta + off + i);
    if constexpr (kRouter) s = __builtin_isfinite(s) ? s : 0.0f;
    ss += s * s;
  }
  ss = block_sum(ss, red);
  const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(ss) / static_cast<double>(cols) +
                                                  static_cast<double>(eps)));
  T* out = kAdd ? h : x;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    float s = ld1(x + off + i);
    if constexpr (kAdd) {
      s += ld1(delta + off + i);
      st1(x + off + i, s);
    }
    if constexpr (kRouter) s = __builtin_isfinite(s) ? s : 0.0f;
    float y;
    {
#pragma clang fp contract(off)
      y = kRouter ? clamp_act(clamp_act(s * inv) * (1.0f + w[i])) : w[i] * (s * inv);
    }
    st1(out + off + i, y);
  }
}

template <class T>
__global__ __launch_bounds__(kBlock) void ln_rows_wide(T* x, const float* w, const float* b, int64_t cols,
                                                       float eps) {
  __shared__ float red[kWavesPerBlock];
  const int64_t off = static_cast<int64_t>(blockIdx.x) * cols;
  float sum = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) sum += ld1(x + off + i);
  const float mean = block_sum(sum, red) / static_cast<float>(cols);
  float q = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    const float d = ld1(x + off + i) - mean;
    q += d * d;
  }
  const float var = block_sum(q, red) / static_cast<float>(cols);
  const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + static_cast<double>(eps)));
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    const float d = ld1(x + off + i) - mean;
    float y;
    {
#pragma clang fp contract(off)
      y = (d * inv) * w[i] + b[i];
    }
    st1(x + off + i, y);
  }
}

// ---- host dispatch -----------------------------------------------------------

int check_rows(const char* what, int64_t rows, int64_t cols) {
  UOCR_REQUIRE(rows >= 0, what, "rows must be >= 0");
  UOCR_REQUIRE(rows == 0 || cols > 0, what, "cols must be > 0");
  UOCR_REQUIRE(rows < (int64_t{1} << 31), what, "rows must be < 2^31");
  UOCR_REQUIRE(cols < (int64_t{1} << 31), what, "cols must be < 2^31");
  return UOCR_ROCM_OK;
}

template <class T, int VW, int WPR, Norm kMode, int TB, bool kShareW, int VPL>
void launch_vpl(hipStream_t s, T* x, const T* delta, const float* w, const float* b, T* h, int64_t rows, int cols,
                float eps, const EmbedSrc& e) {
  constexpr int kRowsPerBlock = TB / kWave / WPR;
  const unsigned blocks = static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  norm_rows<T, VW, WPR, VPL, kMode, TB, kShareW><<<blocks, TB, 0, s>>>(x, delta, w, b, h, rows, cols, eps, e);
}

// vpl: chunks per lane. One-wave rows (WPR 1) take exactly their group count
// up to 8, so no chunk of a row is past its end for every lane (such a chunk
// would still be requested, and its weights and its dropped store with it);
// rows spread over waves take the next of 1, 2, 4, 8, 16.
template <class T, int VW, int WPR, Norm kMode, int TB, bool kShareW>
void launch_norm_tb(int vpl, hipStream_t s, T* x, const T* delta, const float* w, const float* b, T* h,
                    int64_t rows, int cols, float eps, const EmbedSrc& e) {
#define UOCR_NORM_VPL(n) launch_vpl<T, VW, WPR, kMode, TB, kShareW, n>(s, x, delta, w, b, h, rows, cols, eps, e)
  if constexpr (WPR == 1) {
    switch (vpl) {
      case 1: UOCR_NORM_VPL(1); return;
      case 2: UOCR_NORM_VPL(2); return;
      case 3: UOCR_NORM_VPL(3); return;
      case 4: UOCR_NORM_VPL(4); return;
      case 5: UOCR_NORM_VPL(5); return;
      case 6: UOCR_NORM_VPL(6); return;
      case 7: UOCR_NORM_VPL(7); return;
      case 8: UOCR_NORM_VPL(8); return;
      default: UOCR_NORM_VPL(16); return;
    }
  } else {
    switch (vpl_bucket(vpl)) {
      case 1: UOCR_NORM_VPL(1); return;
      case 2: UOCR_NORM_VPL(2); return;
      case 4: UOCR_NORM_VPL(4); return;
      case 8: UOCR_NORM_VPL(8); return;
      default: UOCR_NORM_VPL(16); return;
    }
  }
#undef UOCR_NORM_VPL
}

template <class T, int VW, int WPR, Norm kMode>
void launch_norm_rows(int vpl, hipStream_t s, T* x, const T* delta, const float* w, const float* b, T* h,
                      int64_t rows, int cols, float eps, const EmbedSrc& e) {
  if constexpr (WPR == 1) {
    if (rows < kOneRowGroupsBelow) {
      launch_norm_tb<T, VW, WPR, kMode, kSmallRowsBlock, false>(vpl, s, x, delta, w, b, h, rows, cols, eps, e);
      return;
    }
    launch_norm_tb<T, VW, WPR, kMode, kBlock, true>(vpl, s, x, delta, w, b, h, rows, cols, eps, e);
    return;
  }
  launch_norm_tb<T, VW, WPR, kMode, kBlock, false>(vpl, s, x, delta, w, b, h, rows, cols, eps, e);
}

template <class T, Norm kMode>
int launch_norm(const char* what, void* stream, T* x, const T* delta, const float* w, const float* b, T* h,
                int64_t rows, int64_t cols, float eps, EmbedSrc e = {}) {
  if (int st = check_rows(what, rows, cols)) return st;
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && w != nullptr, what, "null x or w");
  if constexpr (kMode == Norm::kEmbedRms) {
    UOCR_REQUIRE(e.table != nullptr && e.state != nullptr && h != nullptr, what, "null table, state or h");
    UOCR_REQUIRE(h != x && (delta == nullptr || (delta != x && delta != h)), what,
                 "x, delta and h must be distinct buffers");
    UOCR_REQUIRE((cols + kVec<T> - 1) / kVec<T> <= kWave * kMaxGroups, what, "cols too large for one row kernel");
  }
  if constexpr (kMode == Norm::kLayer || kMode == Norm::kLayerToBf16) UOCR_REQUIRE(b != nullptr, what, "null b");
  if constexpr (kMode == Norm::kLayerToBf16) {
    UOCR_REQUIRE(h != nullptr, what, "null y");
    UOCR_REQUIRE((cols + kVec<T> - 1) / kVec<T> <= kWave * kMaxGroups, what, "cols too large for one row kernel");
  }
  if constexpr (kMode == Norm::kAddRms) {
    UOCR_REQUIRE(delta != nullptr && h != nullptr, what, "null delta or h");
    UOCR_REQUIRE(h != x && delta != x && h != delta, what, "x, delta and h must be distinct buffers");
  }
  constexpr int kV = kVec<T>;
  const bool vec = cols % kV == 0 && aligned16(x) && aligned16(w) &&
                   ((kMode != Norm::kLayer && kMode != Norm::kLayerToBf16) || aligned16(b)) &&
                   (kMode != Norm::kLayerToBf16 || aligned16(h)) &&
                   (kMode != Norm::kAddRms || (aligned16(delta) && aligned16(h))) &&
                   (kMode != Norm::kEmbedRms || (aligned16(e.table) && aligned16(h) && (delta == nullptr ||
                                                                                       aligned16(delta))));
  const int64_t nvec = vec ? cols / kV : cols;
  const int64_t groups = (nvec + kWave - 1) / kWave;
  if constexpr (kMode == Norm::kEmbedRms || kMode == Norm::kLayerToBf16) {
    UOCR_REQUIRE(groups <= kMaxGroups, what, "cols too large for one row kernel");
  }
  const hipStream_t s = as_stream(stream);
  const int c32 = static_cast<int>(cols);
  clear_launch_error();
  // Row pieces of kPieceRows (one piece below a million rows). A row's result
  // does not depend on its piece: the reduction order is fixed by cols.
  for_each_piece(rows, kPieceRows, [&](int64_t r0, int64_t rn) {
    const int64_t o = r0 * cols;
    T* xp = x + o;
    const T* dp = delta != nullptr ? delta + o : nullptr;
    T* hp = h == nullptr ? nullptr
            : kMode == Norm::kLayerToBf16 ? reinterpret_cast<T*>(reinterpret_cast<uint16_t*>(h) + o)  // bf16 rows
                                          : h + o;
    if (groups > kMaxGroups) {
      if constexpr (kMode == Norm::kLayer) {
        ln_rows_wide<T><<<static_cast<unsigned>(rn), kBlock, 0, s>>>(xp, w, b, cols, eps);
      } else if constexpr (kMode != Norm::kEmbedRms && kMode != Norm::kLayerToBf16) {
        rms_rows_wide<T, kMode == Norm::kAddRms, kMode == Norm::kRouter>
            <<<static_cast<unsigned>(rn), kBlock, 0, s>>>(xp, dp, w, hp, cols, eps);
      }
      return;
    }
    const bool spread = groups > 16 || (rn < kSpreadRowsBelow && groups >= 4);
    const int vpl = static_cast<int>(spread ? (groups + 3) / 4 : groups);
    if (vec) {
      if (spread) launch_norm_rows<T, kV, 4, kMode>(vpl, s, xp, dp, w, b, hp, rn, c32, eps, e);
      else launch_norm_rows<T, kV, 1, kMode>(vpl, s, xp, dp, w, b, hp, rn, c32, eps, e);
    } else {
      if (spread) launch_norm_rows<T, 1, 4, kMode>(vpl, s, xp, dp, w, b, hp, rn, c32, eps, e);
      else launch_norm_rows<T, 1, 1, kMode>(vpl, s, xp, dp, w, b, hp, rn, c32, eps, e);
    }
  });
  return check_launch(what);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_rms_norm(void* stream, float* x, const float* w, int64_t rows, int64_t cols, float eps) {
  return launch_norm<float, Norm::kRms>("uocr_rocm_rms_norm", stream, x, nullptr, w, nullptr, nullptr, rows, cols,
                                        eps);
}

int uocr_rocm_rms_norm_bf16(void* stream, uint16_t* x, const float* w, int64_t rows, int64_t cols, float eps) {
  return launch_norm<uint16_t, Norm::kRms>("uocr_rocm_rms_norm_bf16", stream, x, nullptr, w, nullptr, nullptr, rows,
                                           cols, eps);
}

int uocr_rocm_add_rms_norm(void* stream, float* x, const float* delta, const float* w, float* h, int64_t rows,
                           int64_t cols, float eps) {
  return launch_norm<float, Norm::kAddRms>("uocr_rocm_add_rms_norm", stream, x, delta, w, nullptr, h, rows, cols,
                                           eps);
}

int uocr_rocm_add_rms_norm_bf16(void* stream, uint16_t* x, const uint16_t* delta, const float* w, uint16_t* h,
                                int64_t rows, int64_t cols, float eps) {
  return launch_norm<uint16_t, Norm::kAddRms>("uocr_rocm_add_rms_norm_bf16", stream, x, delta, w, nullptr, h, rows,
                                              cols, eps);
}

int uocr_rocm_layer_norm(void* stream, float* x, const float* w, const float* b, int64_t rows, int64_t cols,
                         float eps) {
  return launch_norm<float, Norm::kLayer>("uocr_rocm_layer_norm", stream, x, nullptr, w, b, nullptr, rows, cols, eps);
}

int uocr_rocm_layer_norm_to_bf16(void* stream, const float* x, const float* w, const float* b, uint16_t* y,
                                 int64_t rows, int64_t cols, float eps) {
  // x is only read in this mode; y travels in the kernel's h slot
  return launch_norm<float, Norm::kLayerToBf16>("uocr_rocm_layer_norm_to_bf16", stream, const_cast<float*>(x), nullptr,
                                                w, b, reinterpret_cast<float*>(y), rows, cols, eps);
}

int uocr_rocm_layer_norm_bf16(void* stream, uint16_t* x, const float* w, const float* b, int64_t rows, int64_t cols,
                              float eps) {
  return launch_norm<uint16_t, Norm::kLayer>("uocr_rocm_layer_norm_bf16", stream, x, nullptr, w, b, nullptr, rows,
                                             cols, eps);
}

int uocr_rocm_router_norm(void* stream, float* x, const float* w, int64_t rows, int64_t cols, float eps) {
  return launch_norm<float, Norm::kRouter>("uocr_rocm_router_norm", stream, x, nullptr, w, nullptr, nullptr, rows,
                                           cols, eps);
}

int uocr_rocm_router_norm_bf16(void* stream, uint16_t* x, const float* w, int64_t rows, int64_t cols, float eps) {
  return launch_norm<uint16_t, Norm::kRouter>("uocr_rocm_router_norm_bf16", stream, x, nullptr, w, nullptr, nullptr,
                                              rows, cols, eps);
}

int uocr_rocm_embed_add_rms_norm_step(void* stream, const uint16_t* table, int64_t table_rows,
                                      const uocr_rocm_step_state* state, const float* delta, const float* w, float* x,
                                      float* h, int64_t cols, float eps) {
  return launch_norm<float, Norm::kEmbedRms>("uocr_rocm_embed_add_rms_norm_step", stream, x, delta, w, nullptr, h, 1,
                                             cols, eps, EmbedSrc{table, table_rows, state});
}

int uocr_rocm_embed_add_rms_norm_step_bf16(void* stream, const uint16_t* table, int64_t table_rows,
                                           const uocr_rocm_step_state* state, const uint16_t* delta, const float* w,
                                           uint16_t* x, uint16_t* h, int64_t cols, float eps) {
  return launch_norm<uint16_t, Norm::kEmbedRms>("uocr_rocm_embed_add_rms_norm_step_bf16", stream, x, delta, w,
                                                nullptr, h, 1, cols, eps, EmbedSrc{table, table_rows, state});
}

}  // extern "C"
