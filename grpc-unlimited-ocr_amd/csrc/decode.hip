// decode.hip: the key/value-cache ops of one decode step for gfx950, with
// every length-dependent value read from the device StepState so that a
// captured step replays for every token (the reference's append_step and
// attend_step, src/backend/cuda/decode_ops.h:28-47, decode_ops.cu:49-52,
// 112-195).
//
// append_step: cache[pos, :] = row, one 16-byte chunk per thread.
//
// attend_step: out[h] = softmax(q_h . K_h^T * scale + mask) V_h over the keys
// 0..pos of a cache [capacity, heads * hd], one query row. Split-K in two
// launches of fixed shape:
//   partial  grid heads x splits, 4 waves each. A split owns a contiguous
//            run of keys (its length follows pos). Inside a wave, G lanes
//            share a key (each holds VW * VPL elements of the head), so
//            64 / G keys are scored at once; a lane group walks its keys U
//            at a time with an online softmax (running max m, total l and
//            weighted sum of value rows), so no score array is kept. Masked
//            keys (-inf) are neither scored nor read. The 4 * 64 / G lane
//            groups then fold through LDS into one (m, l, acc[hd]) record
//            per split.
//   merge    one workgroup per head folds the splits' records and writes
//            out = acc / l (zeros when every key is masked).
// Scores are s = (q . k) * scale + mask (two roundings, as the reference's
// CPU attention forms them, src/backend/reference/ops.cpp:219-251); every
// exponential is 2^((s - m) log2 e) on v_exp_f32.

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int64_t kMaxHeadDim = 256;
constexpr int kMaxSplits = 64;
constexpr int kAttendUnroll = 4;

// ---- append ---------------------------------------------------------------------

template <int VW>
__global__ __launch_bounds__(kBlock) void append_k(float* __restrict__ cache, const float* __restrict__ row,
                                                   int64_t width, const uocr_rocm_step_state* __restrict__ state,
                                                   int64_t capacity) {
  const int64_t pos = state->pos;
  if (pos < 0 || (capacity >= 0 && pos >= capacity)) return;
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (c * VW >= width) return;
  Chunk<float, VW> v;
  v.load(row + c * VW);
  v.store(cache + pos * width + c * VW);
}

// ---- attention ------------------------------------------------------------------

// Sum over aligned groups of G lanes; every lane of a group ends with the
// same bits (each step adds the same two operands in either lane).
template <int G>
__device__ __forceinline__ float group_sum(float v) {
  if constexpr (G >= 2) v += dpp_f32<0xB1>(v);   // lane ^ 1
  if constexpr (G >= 4) v += dpp_f32<0x4E>(v);   // lane ^ 2
  if constexpr (G >= 8) v += dpp_f32<0x141>(v);  // the two quads of 8 lanes
  if constexpr (G >= 16) v += dpp_f32<0x140>(v); // the two halves of 16 lanes
  if constexpr (G >= 32) {
    // ds_swizzle bit mode: and 0x1f, xor 0x10 -> lane ^ 16 within 32 lanes.
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  }
  if constexpr (G >= 64) v += __shfl_xor(v, 32);
  return v;
}

struct AttendArgs {
  const float* q;
  const float* k;
  const float* v;
  const float* mask;
  float* part;  // [heads, splits, hd + 2]: m, l, acc[hd]
  const uocr_rocm_step_state* state;
  int64_t width;
  int64_t capacity;
  float scale;
  int hd;
  int splits;
};

__device__ __forceinline__ float exp_shift(float s, float m) { return __builtin_amdgcn_exp2f((s - m) * kLog2e); }

template <int VW, int G, int VPL>
__global__ __launch_bounds__(kBlock) void attend_partial(const AttendArgs a) {
  constexpr int kSlotsPerWave = kWave / G;
  constexpr int kSlots = kWavesPerBlock * kSlotsPerWave;
  constexpr int kPerLane = VW * VPL;
  constexpr int U = kAttendUnroll;
  __shared__ float s_m[kSlots];
  __shared__ float s_l[kSlots];
  __shared__ float s_acc[kSlots * G * kPerLane];

  const int h = blockIdx.x / a.splits, split = blockIdx.x % a.splits;
  const int lane = threadIdx.x & (kWave - 1);
  const int slot = (threadIdx.x / kWave) * kSlotsPerWave + lane / G;
  const int gl = lane % G;
  int64_t keys = a.state->pos + 1;
  keys = keys < 0 ? 0 : (keys > a.capacity ? a.capacity : keys);
  const int64_t chunk = (keys + a.splits - 1) / a.splits;
  const int64_t first = split * chunk;
  const int64_t last = first + chunk < keys ? first + chunk : keys;
  const int nvec = a.hd / VW;
  const int64_t head_off = static_cast<int64_t>(h) * a.hd;

  float qv[VPL][VW];
#pragma unroll
  for (int i = 0; i < VPL; ++i) {
    const int c = gl + G * i;
#pragma unroll
    for (int e = 0; e < VW; ++e) qv[i][e] = c < nvec ? a.q[head_off + c * VW + e] : 0.0f;
  }

  float m = -INFINITY, l = 0.0f;
  float acc[VPL][VW];
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int e = 0; e < VW; ++e) acc[i][e] = 0.0f;

  for (int64_t j0 = first + slot; j0 < last; j0 += static_cast<int64_t>(kSlots) * U) {
    float mk[U];
    bool live[U];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + static_cast<int64_t>(kSlots) * u;
      live[u] = j < last;
      mk[u] = live[u] ? (a.mask != nullptr ? a.mask[j] : 0.0f) : -INFINITY;
      live[u] = live[u] && mk[u] != -INFINITY;
    }
    Chunk<float, VW> kc[U][VPL], vc[U][VPL];
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const int64_t j = j0 + static_cast<int64_t>(kSlots) * u;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        const int c = gl + G * i;
        kc[u][i].clear();
        vc[u][i].clear();
        if (live[u] && c < nvec) {
          const int64_t off = j * a.width + head_off + c * VW;
          kc[u][i].load(a.k + off);
          vc[u][i].load(a.v + off);
        }
      }
    }
    float s[U];
    float peak = m;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      float d = 0.0f;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float kv[VW];
        kc[u][i].widen(kv);
#pragma unroll
        for (int e = 0; e < VW; ++e) d = fmaf(qv[i][e], kv[e], d);
      }
      d = group_sum<G>(d);
      {
#pragma clang fp contract(off)
        s[u] = live[u] ? d * a.scale + mk[u] : -INFINITY;
      }
      peak = fmaxf(peak, s[u]);
    }
    if (peak == -INFINITY) continue;  // uniform over the lane group
    const float alpha = exp_shift(m, peak);
    l *= alpha;
#pragma unroll
    for (int i = 0; i < VPL; ++i)
#pragma unroll
      for (int e = 0; e < VW; ++e) acc[i][e] *= alpha;
#pragma unroll
    for (int u = 0; u < U; ++u) {
      const float p = exp_shift(s[u], peak);
      l += p;
#pragma unroll
      for (int i = 0; i < VPL; ++i) {
        float vv[VW];
        vc[u][i].widen(vv);
#pragma unroll
        for (int e = 0; e < VW; ++e) acc[i][e] = fmaf(p, vv[e], acc[i][e]);
      }
    }
    m = peak;
  }

  if (gl == 0) {
    s_m[slot] = m;
    s_l[slot] = l;
  }
#pragma unroll
  for (int i = 0; i < VPL; ++i)
#pragma unroll
    for (int e = 0; e < VW; ++e) s_acc[slot * G * kPerLane + (gl + G * i) * VW + e] = acc[i][e];
  __syncthreads();

  float* rec = a.part + (static_cast<int64_t>(h) * a.splits + split) * (a.hd + 2);
  float big = -INFINITY;
  for (int t = 0; t < kSlots; ++t) big = fmaxf(big, s_m[t]);
  for (int e = threadIdx.x; e < a.hd; e += kBlock) {
    float total = 0.0f, sum = 0.0f;
    if (big != -INFINITY) {
      for (int t = 0; t < kSlots; ++t) {
        if (s_m[t] == -INFINITY) continue;
        const float wgt = exp_shift(s_m[t], big);
        total += s_l[t] * wgt;
        sum += s_acc[t * G * kPerLane + e] * wgt;
      }
    }
    rec[2 + e] = sum;
    if (e == 0) {
      rec[0] = big;
      rec[1] = total;
    }
  }
}

__global__ __launch_bounds__(kBlock) void attend_merge(const float* __restrict__ part, int hd, int splits,
                                                       float* __restrict__ out) {
  const int h = blockIdx.x;
  const float* recs = part + static_cast<int64_t>(h) * splits * (hd + 2);
  float big = -INFINITY;
  for (int i = 0; i < splits; ++i) big = fmaxf(big, recs[i * (hd + 2)]);
  for (int e = threadIdx.x; e < hd; e += kBlock) {
    float total = 0.0f, sum = 0.0f;
    if (big != -INFINITY) {
      for (int i = 0; i < splits; ++i) {
        const float* r = recs + i * (hd + 2);
        if (r[0] == -INFINITY) continue;
        const float wgt = exp_shift(r[0], big);
        total += r[1] * wgt;
        sum += r[2 + e] * wgt;
      }
    }
    out[static_cast<int64_t>(h) * hd + e] = total > 0.0f ? sum / total : 0.0f;
  }
}

// Splits per head: enough workgroups for the 256 CUs at every head count,
// but no split shorter than 32 keys of capacity.
int attend_splits(int64_t heads, int64_t capacity) {
  int64_t s = (1024 + heads - 1) / heads;
  const int64_t by_keys = (capacity + 31) / 32;
  if (s > by_keys) s = by_keys;
  if (s > kMaxSplits) s = kMaxSplits;
  return static_cast<int>(s < 1 ? 1 : s);
}

template <int VW, int G, int VPL>
void launch_partial(hipStream_t s, const AttendArgs& a, int64_t heads) {
  attend_partial<VW, G, VPL><<<static_cast<unsigned>(heads * a.splits), kBlock, 0, s>>>(a);
}

void launch_attend_vec(hipStream_t s, const AttendArgs& a, int64_t heads) {
  const int nvec = a.hd / 4;
  if (nvec <= 1) launch_partial<4, 1, 1>(s, a, heads);
  else if (nvec <= 2) launch_partial<4, 2, 1>(s, a, heads);
  else if (nvec <= 4) launch_partial<4, 4, 1>(s, a, heads);
  else if (nvec <= 8) launch_partial<4, 8, 1>(s, a, heads);
  else if (nvec <= 16) launch_partial<4, 16, 1>(s, a, heads);
  else if (nvec <= 32) launch_partial<4, 32, 1>(s, a, heads);
  else launch_partial<4, 64, 1>(s, a, heads);
}

void launch_attend_any(hipStream_t s, const AttendArgs& a, int64_t heads) {
  if (a.hd <= 64) launch_partial<1, 64, 1>(s, a, heads);
  else if (a.hd <= 128) launch_partial<1, 64, 2>(s, a, heads);
  else launch_partial<1, 64, 4>(s, a, heads);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_append_step(void* stream, float* cache, const float* row, int64_t width,
                          const uocr_rocm_step_state* state, int64_t capacity) {
  const char* what = "uocr_rocm_append_step";
  UOCR_REQUIRE(width >= 0, what, "width must be >= 0");
  if (width == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(cache != nullptr && row != nullptr && state != nullptr, what, "null pointer");
  UOCR_REQUIRE(width < (int64_t{1} << 36), what, "width too large");
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  if (width % 4 == 0 && aligned16(cache) && aligned16(row)) {
    const unsigned blocks = static_cast<unsigned>((width / 4 + kBlock - 1) / kBlock);
    append_k<4><<<blocks, kBlock, 0, s>>>(cache, row, width, state, capacity);
  } else {
    const unsigned blocks = static_cast<unsigned>((width + kBlock - 1) / kBlock);
    append_k<1><<<blocks, kBlock, 0, s>>>(cache, row, width, state, capacity);
  }
  return check_launch(what);
}

int64_t uocr_rocm_attend_scratch_floats(int64_t heads, int64_t hd, int64_t capacity) {
  if (heads <= 0 || hd <= 0 || capacity <= 0) return 0;
  return heads * attend_splits(heads, capacity) * (hd + 2);
}

int uocr_rocm_attend_step(void* stream, const float* q, const float* k_cache, const float* v_cache, int64_t heads,
                          int64_t hd, const float* mask, float scale, const uocr_rocm_step_state* state,
                          float* scratch, int64_t capacity, float* out) {
  const char* what = "uocr_rocm_attend_step";
  UOCR_REQUIRE(heads >= 0 && hd >= 0, what, "heads and hd must be >= 0");
  if (heads == 0 || hd == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(hd <= kMaxHeadDim, what, "head dim above 256");
  UOCR_REQUIRE(heads < (int64_t{1} << 24), what, "too many heads");
  UOCR_REQUIRE(capacity >= 1, what, "capacity must be >= 1");
  UOCR_REQUIRE(q != nullptr && k_cache != nullptr && v_cache != nullptr && state != nullptr && scratch != nullptr &&
                   out != nullptr,
               what, "null pointer");
  AttendArgs a{q, k_cache, v_cache, mask, scratch, state, heads * hd, capacity, scale, static_cast<int>(hd),
               attend_splits(heads, capacity)};
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  if (hd % 4 == 0 && aligned16(q) && aligned16(k_cache) && aligned16(v_cache)) {
    launch_attend_vec(s, a, heads);
  } else {
    launch_attend_any(s, a, heads);
  }
  if (const int st = check_launch(what); st != UOCR_ROCM_OK) return st;
  attend_merge<<<static_cast<unsigned>(heads), kBlock, 0, s>>>(scratch, a.hd, a.splits, out);
  return check_launch(what);
}

}  // extern "C"
