// norm.hip: RMSNorm, residual add fused with RMSNorm, and LayerNorm for
// gfx950, fp32 and bf16 activations, fp32 arithmetic, fp32 norm weights.
//
// Layout: x [rows, cols] row-major. One wave64 owns one row: each lane holds
// VPL 128-bit chunks of the row (chunk v = lane + 64 k) in registers, so the
// row is read from HBM once and written once; the row statistics reduce
// across the wave with DPP (wave_sum) and never touch LDS. Rows wider than
// 16 chunks per lane take the *_wide kernels: one workgroup per row, a second
// read of the row, and a 4-float LDS exchange between the four waves.
//
// Arithmetic (reference: src/backend/reference/ops.cpp:111-141):
//   rms_norm:    ss = sum x^2 (fp32), inv = float(1 / sqrt(ss / cols + eps))
//                evaluated in fp64 as the reference does, y = w * (x * inv).
//   layer_norm:  mean = sum x / cols, var = sum (x - mean)^2 / cols (two
//                passes over the registers, fp32), inv as above in fp64 from
//                var, y = ((x - mean) * inv) * w + b.
//   add_rms_norm: s = x + delta (fp32), x <- s, h <- w * (s * inv(s)).
// The output expressions are evaluated without FMA contraction so that each
// product and sum is rounded where the reference rounds it.

#include "common.hpp"

namespace uocr_rocm {
namespace {


// ---- register-resident rows ------------------------------------------------

template <class T, int VW, int VPL, bool kAdd>
__global__ __launch_bounds__(kBlock) void rms_rows(T* __restrict__ x, const T* __restrict__ delta,
                                                   const float* __restrict__ w, T* __restrict__ h, int64_t rows,
                                                   int cols, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;  // uniform across the wave
  const int nvec = cols / VW;
  const int64_t off = row * cols;

  Chunk<T, VW> cx[VPL];
  Chunk<T, VW> cd[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) {
      cx[k].load(x + off + static_cast<int64_t>(v) * VW);
      if constexpr (kAdd) cd[k].load(delta + off + static_cast<int64_t>(v) * VW);
    }
  }

  float s[VPL][VW];
  float ss = 0.0f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) {
      cx[k].widen(s[k]);
      if constexpr (kAdd) {
        float d[VW];
        cd[k].widen(d);
#pragma unroll
        for (int e = 0; e < VW; ++e) s[k][e] += d[e];
      }
#pragma unroll
      for (int e = 0; e < VW; ++e) ss += s[k][e] * s[k][e];
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) s[k][e] = 0.0f;
    }
  }
  ss = wave_sum(ss);
  const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(ss) / static_cast<double>(cols) +
                                                  static_cast<double>(eps)));

  T* out = kAdd ? h : x;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) {
      const int64_t at = off + static_cast<int64_t>(v) * VW;
      if constexpr (kAdd) {
        Chunk<T, VW> xs;
        xs.narrow(s[k]);
        xs.store(x + at);
      }
      // w is read after the reduction: it is shared by every row (cache
      // resident), and loading it late keeps the wave's register count low.
      float wv[VW];
      load_f32<VW>(w + v * VW, wv);
      float y[VW];
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < VW; ++e) y[e] = wv[e] * (s[k][e] * inv);
      }
      Chunk<T, VW> o;
      o.narrow(y);
      o.store(out + at);
    }
  }
}

template <class T, int VW, int VPL>
__global__ __launch_bounds__(kBlock) void ln_rows(T* __restrict__ x, const float* __restrict__ w,
                                                  const float* __restrict__ b, int64_t rows, int cols, float eps) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const int nvec = cols / VW;
  const int64_t off = row * cols;

  Chunk<T, VW> cx[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) cx[k].load(x + off + static_cast<int64_t>(v) * VW);
  }

  float s[VPL][VW];
  float sum = 0.0f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) {
      cx[k].widen(s[k]);
#pragma unroll
      for (int e = 0; e < VW; ++e) sum += s[k][e];
    }
  }
  const float mean = wave_sum(sum) / static_cast<float>(cols);

  float q = 0.0f;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) {
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        s[k][e] -= mean;
        q += s[k][e] * s[k][e];
      }
    }
  }
  const float var = wave_sum(q) / static_cast<float>(cols);
  const float inv = static_cast<float>(1.0 / sqrt(static_cast<double>(var) + static_cast<double>(eps)));

#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int v = lane + k * kWave;
    if (v < nvec) {
      float wv[VW], bv[VW];
      load_f32<VW>(w + v * VW, wv);
      load_f32<VW>(b + v * VW, bv);
      float y[VW];
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < VW; ++e) y[e] = (s[k][e] * inv) * wv[e] + bv[e];
      }
      Chunk<T, VW> o;
      o.narrow(y);
      o.store(x + off + static_cast<int64_t>(v) * VW);
    }
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

template <class T, bool kAdd>
__global__ __launch_bounds__(kBlock) void rms_rows_wide(T* x, const T* delta, const float* w, T* h, int64_t cols,
                                                        float eps) {
  __shared__ float red[kWavesPerBlock];
  const int64_t off = static_cast<int64_t>(blockIdx.x) * cols;
  float ss = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    float s = ld1(x + off + i);
    if constexpr (kAdd) s += ld1(delta + off + i);
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
    float y;
    {
#pragma clang fp contract(off)
      y = w[i] * (s * inv);
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

// Chunks per lane rounded up to the instantiated set.
inline int vpl_bucket(int64_t nvec) {
  const int64_t need = (nvec + kWave - 1) / kWave;
  if (need <= 1) return 1;
  if (need <= 2) return 2;
  if (need <= 4) return 4;
  if (need <= 8) return 8;
  if (need <= 16) return 16;
  return 0;  // wider than the registers hold
}

#define UOCR_VPL_SWITCH(VPL_VALUE, ...)            \
  switch (VPL_VALUE) {                             \
    case 1: { constexpr int VPL = 1; __VA_ARGS__; } break;   \
    case 2: { constexpr int VPL = 2; __VA_ARGS__; } break;   \
    case 4: { constexpr int VPL = 4; __VA_ARGS__; } break;   \
    case 8: { constexpr int VPL = 8; __VA_ARGS__; } break;   \
    default: { constexpr int VPL = 16; __VA_ARGS__; } break; \
  }

int check_rows(const char* what, int64_t rows, int64_t cols) {
  UOCR_REQUIRE(rows >= 0, what, "rows must be >= 0");
  UOCR_REQUIRE(rows == 0 || cols > 0, what, "cols must be > 0");
  UOCR_REQUIRE(rows < (int64_t{1} << 31), what, "rows must be < 2^31");
  UOCR_REQUIRE(cols < (int64_t{1} << 31), what, "cols must be < 2^31");
  return UOCR_ROCM_OK;
}

template <class T, bool kAdd>
int launch_rms(const char* what, void* stream, T* x, const T* delta, const float* w, T* h, int64_t rows,
               int64_t cols, float eps) {
  if (int st = check_rows(what, rows, cols)) return st;
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && w != nullptr, what, "null x or w");
  if constexpr (kAdd) {
    UOCR_REQUIRE(delta != nullptr && h != nullptr, what, "null delta or h");
    UOCR_REQUIRE(h != x && delta != x && h != delta, what, "x, delta and h must be distinct buffers");
  }
  constexpr int kV = kVec<T>;
  const bool vec = cols % kV == 0 && aligned16(x) && aligned16(w) && (!kAdd || (aligned16(delta) && aligned16(h)));
  const int64_t nvec = vec ? cols / kV : cols;
  const int bucket = vpl_bucket(nvec);
  const hipStream_t s = as_stream(stream);
  const int c32 = static_cast<int>(cols);
  clear_launch_error();
  if (bucket == 0) {
    rms_rows_wide<T, kAdd><<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, delta, w, h, cols, eps);
  } else if (vec) {
    UOCR_VPL_SWITCH(bucket, (rms_rows<T, kV, VPL, kAdd><<<blocks_for_rows(rows), kBlock, 0, s>>>(
                                x, delta, w, h, rows, c32, eps)))
  } else {
    UOCR_VPL_SWITCH(bucket, (rms_rows<T, 1, VPL, kAdd><<<blocks_for_rows(rows), kBlock, 0, s>>>(
                                x, delta, w, h, rows, c32, eps)))
  }
  return check_launch(what);
}

template <class T>
int launch_ln(const char* what, void* stream, T* x, const float* w, const float* b, int64_t rows, int64_t cols,
              float eps) {
  if (int st = check_rows(what, rows, cols)) return st;
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && w != nullptr && b != nullptr, what, "null x, w or b");
  constexpr int kV = kVec<T>;
  const bool vec = cols % kV == 0 && aligned16(x) && aligned16(w) && aligned16(b);
  const int64_t nvec = vec ? cols / kV : cols;
  const int bucket = vpl_bucket(nvec);
  const hipStream_t s = as_stream(stream);
  const int c32 = static_cast<int>(cols);
  clear_launch_error();
  if (bucket == 0) {
    ln_rows_wide<T><<<static_cast<unsigned>(rows), kBlock, 0, s>>>(x, w, b, cols, eps);
  } else if (vec) {
    UOCR_VPL_SWITCH(bucket, (ln_rows<T, kV, VPL><<<blocks_for_rows(rows), kBlock, 0, s>>>(x, w, b, rows, c32, eps)))
  } else {
    UOCR_VPL_SWITCH(bucket, (ln_rows<T, 1, VPL><<<blocks_for_rows(rows), kBlock, 0, s>>>(x, w, b, rows, c32, eps)))
  }
  return check_launch(what);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_rms_norm(void* stream, float* x, const float* w, int64_t rows, int64_t cols, float eps) {
  return launch_rms<float, false>("uocr_rocm_rms_norm", stream, x, nullptr, w, nullptr, rows, cols, eps);
}

int uocr_rocm_rms_norm_bf16(void* stream, uint16_t* x, const float* w, int64_t rows, int64_t cols, float eps) {
  return launch_rms<uint16_t, false>("uocr_rocm_rms_norm_bf16", stream, x, nullptr, w, nullptr, rows, cols, eps);
}

int uocr_rocm_add_rms_norm(void* stream, float* x, const float* delta, const float* w, float* h, int64_t rows,
                           int64_t cols, float eps) {
  return launch_rms<float, true>("uocr_rocm_add_rms_norm", stream, x, delta, w, h, rows, cols, eps);
}

int uocr_rocm_add_rms_norm_bf16(void* stream, uint16_t* x, const uint16_t* delta, const float* w, uint16_t* h,
                                int64_t rows, int64_t cols, float eps) {
  return launch_rms<uint16_t, true>("uocr_rocm_add_rms_norm_bf16", stream, x, delta, w, h, rows, cols, eps);
}

int uocr_rocm_layer_norm(void* stream, float* x, const float* w, const float* b, int64_t rows, int64_t cols,
                         float eps) {
  return launch_ln<float>("uocr_rocm_layer_norm", stream, x, w, b, rows, cols, eps);
}

int uocr_rocm_layer_norm_bf16(void* stream, uint16_t* x, const float* w, const float* b, int64_t rows, int64_t cols,
                              float eps) {
  return launch_ln<uint16_t>("uocr_rocm_layer_norm_bf16", stream, x, w, b, rows, cols, eps);
}

}  // extern "C"
