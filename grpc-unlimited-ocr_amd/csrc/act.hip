// act.hip: elementwise ops for gfx950: exact-erf GELU, SiLU-and-multiply,
// SwiGLU over a concatenated [gate | up] row, and the fp32 residual add.
// fp32 and bf16 activations, fp32 arithmetic.
//
// Flat ops (gelu_erf, silu_mul, add_inplace) stream 128-bit chunks: each
// thread owns kUnroll chunks spaced one workgroup apart, issues all of their
// loads before any math, then stores. A ragged tail shorter than one chunk,
// or any buffer not 16-byte aligned, takes the scalar path.
//
// SwiGLU is row-shaped: one wave64 per row reads the row's gate half and up
// half (chunks c = lane + 64 k) and writes one output row, so the gate/up
// pair never round-trips through HBM between the activation and the product.
//
// Arithmetic (reference: src/backend/reference/ops.cpp:40,151-167 and
// src/model/feed_forward.cpp:18-24), each rounded where the reference
// rounds (no FMA contraction):
//   gelu_erf:  y = (0.5 v) (1 + erf(v * 0.70710678f))
//   silu:      y = v (1 / (1 + exp(-v)));   silu_mul / swiglu: y = silu(g) u

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int kUnroll = 4;

__device__ __forceinline__ float gelu_f(float v) {
#pragma clang fp contract(off)
  return 0.5f * v * (1.0f + erff(v * 0.70710678118654752440f));
}

__device__ __forceinline__ float silu_mul_f(float g, float u) {
#pragma clang fp contract(off)
  const float sig = 1.0f / (1.0f + expf(-g));
  return (g * sig) * u;
}

// ---- flat ops ------------------------------------------------------------------

enum class Flat { kGelu, kSiluMul, kAdd };

// x (in place) op= y over n elements; y is unused by kGelu.
template <Flat kOp, class T, int VW>
__global__ __launch_bounds__(kBlock) void flat_kernel(T* __restrict__ x, const T* __restrict__ y, int64_t n) {
  const int64_t nvec = n / VW;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * (kBlock * kUnroll) + threadIdx.x;
  Chunk<T, VW> cx[kUnroll], cy[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = first + static_cast<int64_t>(u) * kBlock;
    if (i < nvec) {
      cx[u].load(x + i * VW);
      if constexpr (kOp != Flat::kGelu) cy[u].load(y + i * VW);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = first + static_cast<int64_t>(u) * kBlock;
    if (i < nvec) {
      float a[VW], b[VW];
      cx[u].widen(a);
      if constexpr (kOp != Flat::kGelu) cy[u].widen(b);
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        if constexpr (kOp == Flat::kGelu) a[e] = gelu_f(a[e]);
        if constexpr (kOp == Flat::kSiluMul) a[e] = silu_mul_f(a[e], b[e]);
        if constexpr (kOp == Flat::kAdd) a[e] = a[e] + b[e];
      }
      cx[u].narrow(a);
      cx[u].store(x + i * VW);
    }
  }
  // The last n % VW elements (VW > 1 only): one thread each in block 0.
  if constexpr (VW > 1) {
    const int64_t rest = n - nvec * VW;
    if (blockIdx.x == 0 && threadIdx.x < rest) {
      const int64_t i = nvec * VW + threadIdx.x;
      Chunk<T, 1> c, d;
      c.load(x + i);
      float a[1], b[1];
      c.widen(a);
      if constexpr (kOp != Flat::kGelu) {
        d.load(y + i);
        d.widen(b);
      }
      if constexpr (kOp == Flat::kGelu) a[0] = gelu_f(a[0]);
      if constexpr (kOp == Flat::kSiluMul) a[0] = silu_mul_f(a[0], b[0]);
      if constexpr (kOp == Flat::kAdd) a[0] = a[0] + b[0];
      c.narrow(a);
      c.store(x + i);
    }
  }
}

template <Flat kOp, class T>
int launch_flat(const char* what, void* stream, T* x, const T* y, int64_t n) {
  UOCR_REQUIRE(n >= 0, what, "n must be >= 0");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && (kOp == Flat::kGelu || y != nullptr), what, "null pointer");
  constexpr int kV = kVec<T>;
  const bool vec = aligned16(x) && (kOp == Flat::kGelu || aligned16(y));
  const int64_t nvec = vec ? n / kV : n;
  int64_t blocks = (nvec + kBlock * kUnroll - 1) / (kBlock * kUnroll);
  if (blocks < 1) blocks = 1;
  UOCR_REQUIRE(blocks < (int64_t{1} << 31), what, "n too large");
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  if (vec) {
    flat_kernel<kOp, T, kV><<<static_cast<unsigned>(blocks), kBlock, 0, s>>>(x, y, n);
  } else {
    flat_kernel<kOp, T, 1><<<static_cast<unsigned>(blocks), kBlock, 0, s>>>(x, y, n);
  }
  return check_launch(what);
}

// ---- SwiGLU on [rows, 2 ffn] -> [rows, ffn] -------------------------------------

template <class T, int VW, int ITERS>
__global__ __launch_bounds__(kBlock) void swiglu_rows(const T* __restrict__ in, T* __restrict__ out, int64_t rows,
                                                      int ffn) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const int nvec = ffn / VW;
  const T* gate = in + row * 2 * ffn;
  const T* up = gate + ffn;
  T* dst = out + row * ffn;
  for (int base = 0; base < nvec; base += kWave * ITERS) {
    Chunk<T, VW> cg[ITERS], cu[ITERS];
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int v = base + lane + it * kWave;
      if (v < nvec) {
        cg[it].load(gate + v * VW);
        cu[it].load(up + v * VW);
      }
    }
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      const int v = base + lane + it * kWave;
      if (v < nvec) {
        float g[VW], u[VW];
        cg[it].widen(g);
        cu[it].widen(u);
#pragma unroll
        for (int e = 0; e < VW; ++e) g[e] = silu_mul_f(g[e], u[e]);
        Chunk<T, VW> o;
        o.narrow(g);
        o.store(dst + v * VW);
      }
    }
  }
}

template <class T>
int launch_swiglu(const char* what, void* stream, const T* in, T* out, int64_t rows, int64_t ffn) {
  UOCR_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), what, "rows must be in [0, 2^31)");
  UOCR_REQUIRE(rows == 0 || (ffn > 0 && ffn < (int64_t{1} << 29)), what, "ffn must be in [1, 2^29)");
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(in != nullptr && out != nullptr, what, "null pointer");
  {
    const auto in_lo = reinterpret_cast<uintptr_t>(in), out_lo = reinterpret_cast<uintptr_t>(out);
    const auto in_hi = in_lo + static_cast<uintptr_t>(rows * 2 * ffn) * sizeof(T);
    const auto out_hi = out_lo + static_cast<uintptr_t>(rows * ffn) * sizeof(T);
    UOCR_REQUIRE(out_hi <= in_lo || in_hi <= out_lo, what, "in and out must not overlap");
  }
  constexpr int kV = kVec<T>;
  const bool vec = ffn % kV == 0 && aligned16(in) && aligned16(out);
  const int64_t nvec = vec ? ffn / kV : ffn;
  int64_t iters = (nvec + kWave - 1) / kWave;
  if (iters > 4) iters = 4;
  const hipStream_t s = as_stream(stream);
  const unsigned blocks = blocks_for_rows(rows);
  const int f = static_cast<int>(ffn);
  clear_launch_error();
#define UOCR_SWIGLU_LAUNCH(VW)                                                          \
  switch (iters) {                                                                      \
    case 1: swiglu_rows<T, VW, 1><<<blocks, kBlock, 0, s>>>(in, out, rows, f); break;   \
    case 2: swiglu_rows<T, VW, 2><<<blocks, kBlock, 0, s>>>(in, out, rows, f); break;   \
    case 3: swiglu_rows<T, VW, 3><<<blocks, kBlock, 0, s>>>(in, out, rows, f); break;   \
    default: swiglu_rows<T, VW, 4><<<blocks, kBlock, 0, s>>>(in, out, rows, f); break;  \
  }
  if (vec) {
    UOCR_SWIGLU_LAUNCH(kV)
  } else {
    UOCR_SWIGLU_LAUNCH(1)
  }
#undef UOCR_SWIGLU_LAUNCH
  return check_launch(what);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_add_inplace(void* stream, float* y, const float* x, int64_t n) {
  UOCR_REQUIRE(n == 0 || y != x, "uocr_rocm_add_inplace", "y and x must be distinct buffers");
  return launch_flat<Flat::kAdd, float>("uocr_rocm_add_inplace", stream, y, x, n);
}

int uocr_rocm_copy(void* stream, float* dst, const float* src, int64_t n) {
  UOCR_REQUIRE(n >= 0, "uocr_rocm_copy", "n must be >= 0");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(dst != nullptr && src != nullptr, "uocr_rocm_copy", "null pointer");
  return check_hip(hipMemcpyAsync(dst, src, static_cast<size_t>(n) * sizeof(float), hipMemcpyDeviceToDevice,
                                  as_stream(stream)),
                   "uocr_rocm_copy");
}

int uocr_rocm_gelu_erf(void* stream, float* x, int64_t n) {
  return launch_flat<Flat::kGelu, float>("uocr_rocm_gelu_erf", stream, x, nullptr, n);
}

int uocr_rocm_gelu_erf_bf16(void* stream, uint16_t* x, int64_t n) {
  return launch_flat<Flat::kGelu, uint16_t>("uocr_rocm_gelu_erf_bf16", stream, x, nullptr, n);
}

int uocr_rocm_silu_mul(void* stream, float* g, const float* u, int64_t n) {
  UOCR_REQUIRE(n == 0 || g != u, "uocr_rocm_silu_mul", "g and u must be distinct buffers");
  return launch_flat<Flat::kSiluMul, float>("uocr_rocm_silu_mul", stream, g, u, n);
}

int uocr_rocm_swiglu(void* stream, const float* in, float* out, int64_t rows, int64_t ffn) {
  return launch_swiglu<float>("uocr_rocm_swiglu", stream, in, out, rows, ffn);
}

int uocr_rocm_swiglu_bf16(void* stream, const uint16_t* in, uint16_t* out, int64_t rows, int64_t ffn) {
  return launch_swiglu<uint16_t>("uocr_rocm_swiglu_bf16", stream, in, out, rows, ffn);
}

}  // extern "C"
