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
// loaded once and reused for every row; waves walk the rows grid-stride, RPW
// rows at a time, so RPW * CPL weight loads per lane are in flight together.
// Weight rows stream with nontemporal loads. The row total is a wave64 DPP
// butterfly. Inputs wider than the registers hold (k up to kGemvMaxK) stage
// bf16(x) in LDS instead; widths that are not a multiple of 8 or not 16-byte
// aligned take the element-wise kernel.

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int64_t kGemvMaxK = 12288;        // the reference's bound (gemv_ops.h:16)
constexpr int kGemvRegChunks = 4;           // register-resident x: k <= 64 * 4 * 8
constexpr unsigned kGemvMaxBlocks = 2048;   // grid-stride beyond 8192 waves

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

// x in registers: CPL chunks per lane; RPW rows per wave per pass.
template <int CPL, int RPW>
__global__ __launch_bounds__(kBlock) void gemv_reg(const float* __restrict__ x, int nchunks,
                                                   const uint16_t* __restrict__ w, int64_t n,
                                                   const float* __restrict__ bias, float* __restrict__ y) {
  const int lane = threadIdx.x & (kWave - 1);
  float xv[CPL][8];
#pragma unroll
  for (int i = 0; i < CPL; ++i) {
    const int c = lane + kWave * i;
    if (c < nchunks) {
      load_x8(x, c, xv[i]);
    } else {
#pragma unroll
      for (int e = 0; e < 8; ++e) xv[i][e] = 0.0f;
    }
  }
  const int64_t k = static_cast<int64_t>(nchunks) * 8;
  const int64_t groups = (n + RPW - 1) / RPW;
  const int64_t step = static_cast<int64_t>(gridDim.x) * kWavesPerBlock;
  for (int64_t g = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave; g < groups; g += step) {
    const int64_t row0 = g * RPW;
    u32x4 wc[RPW][CPL];
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

template <int CPL>
void launch_reg(hipStream_t s, const float* x, int nchunks, const uint16_t* w, int64_t n, const float* bias,
                float* y) {
  // Four rows per wave once there are enough rows to fill the GPU with them.
  if (n >= 16384) {
    gemv_reg<CPL, 4><<<gemv_blocks((n + 3) / 4), kBlock, 0, s>>>(x, nchunks, w, n, bias, y);
  } else {
    gemv_reg<CPL, 1><<<gemv_blocks(n), kBlock, 0, s>>>(x, nchunks, w, n, bias, y);
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

}  // extern "C"
