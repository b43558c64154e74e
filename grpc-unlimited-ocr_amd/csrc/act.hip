// act.hip: elementwise ops for gfx950: exact-erf GELU, SiLU-and-multiply,
// SwiGLU over a concatenated [gate | up] row, the fp32 residual add and the
// fp32 device copy.
// fp32 and bf16 activations, fp32 arithmetic.
//
// Flat ops (gelu_erf, silu_mul, add_inplace, copy) stream 128-bit chunks,
// one per thread, over a grid that covers the whole tensor in one pass (one
// launch per 2^28 chunks, for tensors past the work-items of a dispatch). A
// ragged tail shorter than one chunk, or any buffer not 16-byte aligned,
// takes the scalar path.
//
// SwiGLU maps one thread to one 128-bit output chunk (row r, chunk j): it
// reads chunk j of the row's gate half and of its up half and writes chunk
// j of output row r, so the gate/up pair never round-trips through HBM
// between the activation and the product. r and j come from the flat thread
// index by a multiply-high with a host-computed reciprocal (no division in
// the kernel).
//
// Arithmetic (reference: src/backend/reference/ops.cpp:40,151-167 and
// src/model/feed_forward.cpp:18-24) in fp32:
//   gelu_erf:  y = v Phi(v), Phi the standard normal CDF (= the reference's
//              0.5 v (1 + erf(v / sqrt 2)))
//   silu:      y = v / (1 + exp(-v));   silu_mul / swiglu: y = silu(g) u
// The transcendentals run on the hardware's exp2 and reciprocal so that the
// ops stay bound by HBM rather than by the fp32 ALUs.
//
// copy (dst = src) streams the same 128-bit chunks with nontemporal loads and
// stores: at 256 MiB it moved 6.4 TB/s where the runtime's memcpy kernel
// moved 5.4 TB/s.

#include "act_math.hpp"
#include "common.hpp"

namespace uocr_rocm {
namespace {

// One 128-bit chunk per thread: measured faster on MI355X than several
// chunks per thread for these streaming shapes (more waves in flight).
constexpr int kUnroll = 1;

// Workgroup size by grid size. A grid of more than 1.25 resident rounds of
// waves (8 per SIMD on 1024 SIMDs) runs as one-wave workgroups, which refill
// a SIMD as soon as any wave retires: 3-5% faster from 23 to 134 MB. A grid
// that fits in about one round keeps four-wave workgroups, which dispatch
// faster: one-wave groups were 14% slower at 17 MB (one round exactly, and
// a copy of one round plus 256 threads).
constexpr int64_t kResidentThreads = int64_t{256} * 4 * 8 * kWave;

inline bool one_wave_groups(int64_t threads) { return threads > kResidentThreads + kResidentThreads / 4; }

// Element counts of the flat ops stay below 2^56, so byte offsets and the
// overlap checks never overflow (any tensor that fits in memory passes).
constexpr int64_t kMaxElems = int64_t{1} << 56;

// ---- flat ops ------------------------------------------------------------------

enum class Flat { kGelu, kSiluMul, kAdd, kQuickGelu };

constexpr bool unary(Flat op) { return op == Flat::kGelu || op == Flat::kQuickGelu; }

// x (in place) op= y over n elements; y is unused by kGelu.
template <Flat kOp, class T, int VW, int TB>
__global__ __launch_bounds__(TB) void flat_kernel(T* __restrict__ x, const T* __restrict__ y, int64_t n) {
  const int64_t nvec = n / VW;
  const int64_t first = static_cast<int64_t>(blockIdx.x) * (TB * kUnroll) + threadIdx.x;
  Chunk<T, VW> cx[kUnroll], cy[kUnroll];
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = first + static_cast<int64_t>(u) * TB;
    if (i < nvec) {
      cx[u].load(x + i * VW);
      if constexpr (!unary(kOp)) cy[u].load(y + i * VW);
    }
  }
#pragma unroll
  for (int u = 0; u < kUnroll; ++u) {
    const int64_t i = first + static_cast<int64_t>(u) * TB;
    if (i < nvec) {
      float a[VW], b[VW];
      cx[u].widen(a);
      if constexpr (!unary(kOp)) cy[u].widen(b);
#pragma unroll
      for (int e = 0; e < VW; ++e) {
        if constexpr (kOp == Flat::kGelu) a[e] = gelu_of<T>(a[e]);
        if constexpr (kOp == Flat::kQuickGelu) a[e] = quick_gelu_f(a[e]);
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
      if constexpr (!unary(kOp)) {
        d.load(y + i);
        d.widen(b);
      }
      if constexpr (kOp == Flat::kGelu) a[0] = gelu_of<T>(a[0]);
      if constexpr (kOp == Flat::kQuickGelu) a[0] = quick_gelu_f(a[0]);
      if constexpr (kOp == Flat::kSiluMul) a[0] = silu_mul_f(a[0], b[0]);
      if constexpr (kOp == Flat::kAdd) a[0] = a[0] + b[0];
      c.narrow(a);
      c.store(x + i);
    }
  }
}

template <Flat kOp, class T, int VW>
void launch_flat_tb(hipStream_t s, T* x, const T* y, int64_t n, int64_t nvec) {
  auto blocks = [nvec](int64_t tb) {
    const int64_t b = (nvec + tb * kUnroll - 1) / (tb * kUnroll);
    return static_cast<unsigned>(b < 1 ? 1 : b);
  };
  if (one_wave_groups(nvec)) {
    flat_kernel<kOp, T, VW, kWave><<<blocks(kWave), kWave, 0, s>>>(x, y, n);
  } else {
    flat_kernel<kOp, T, VW, kBlock><<<blocks(kBlock), kBlock, 0, s>>>(x, y, n);
  }
}

template <Flat kOp, class T>
int launch_flat(const char* what, void* stream, T* x, const T* y, int64_t n) {
  UOCR_REQUIRE(n >= 0, what, "n must be >= 0");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && (unary(kOp) || y != nullptr), what, "null pointer");
  UOCR_REQUIRE(n < kMaxElems, what, "n too large");
  constexpr int kV = kVec<T>;
  const bool vec = aligned16(x) && (unary(kOp) || aligned16(y));
  const int vw = vec ? kV : 1;
  const int64_t nvec = n / vw;
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  // Pieces of kPieceChunks chunks; the last piece takes the ragged tail.
  for_each_piece(nvec, kPieceChunks, [&](int64_t c0, int64_t cn) {
    const int64_t e0 = c0 * vw, en = c0 + cn == nvec ? n - e0 : cn * vw;
    const T* yp = unary(kOp) ? y : y + e0;
    if (vec) {
      launch_flat_tb<kOp, T, kV>(s, x + e0, yp, en, cn);
    } else {
      launch_flat_tb<kOp, T, 1>(s, x + e0, yp, en, cn);
    }
  });
  return check_launch(what);
}

// ---- activation into bf16 ----------------------------------------------------------

// y = bf16(act(x)): fp32 x in, the activation in fp32 (the same function as
// the in-place fp32 op), rounded to nearest even on the way out. The MLPs'
// second projection rounds its input to bf16 anyway, so this is the
// activation and that rounding in one pass (half the output bytes, and the
// projection takes its memory-to-LDS path). 8 elements per thread; the last
// n % 8 (or every element where a pointer is not 16-byte aligned) one per
// thread.
template <Flat kOp>
__global__ __launch_bounds__(kBlock) void act_to_bf16_k(const float* __restrict__ x, uint16_t* __restrict__ y,
                                                          int64_t n, bool vec) {
  auto act = [](float v) {
    if constexpr (kOp == Flat::kGelu) return gelu_of<float>(v);
    return quick_gelu_f(v);
  };
  const int64_t t = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (vec && 8 * t + 8 <= n) {
    const u32x4 lo = *reinterpret_cast<const u32x4*>(x + 8 * t), hi = *reinterpret_cast<const u32x4*>(x + 8 * t + 4);
    *reinterpret_cast<u32x4*>(y + 8 * t) =
        u32x4{pack_bf16(act(__uint_as_float(lo.x)), act(__uint_as_float(lo.y))),
              pack_bf16(act(__uint_as_float(lo.z)), act(__uint_as_float(lo.w))),
              pack_bf16(act(__uint_as_float(hi.x)), act(__uint_as_float(hi.y))),
              pack_bf16(act(__uint_as_float(hi.z)), act(__uint_as_float(hi.w)))};
    return;
  }
  for (int64_t i = vec ? 8 * t : t; i < n && (vec ? i < 8 * t + 8 : i == t); ++i) y[i] = f32_to_bf16(act(x[i]));
}

template <Flat kOp>
int launch_act_to_bf16(const char* what, void* stream, const float* x, uint16_t* y, int64_t n) {
  UOCR_REQUIRE(n >= 0, what, "n must be >= 0");
  if (n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && y != nullptr, what, "null pointer");
  UOCR_REQUIRE(n < kMaxElems, what, "n too large");
  const bool vec = aligned16(x) && aligned16(y);
  const int64_t threads = vec ? (n + 7) / 8 : n;
  const int64_t blocks = (threads + kBlock - 1) / kBlock;
  UOCR_REQUIRE(blocks < (int64_t{1} << 31), what, "n too large");
  clear_launch_error();
  act_to_bf16_k<kOp><<<static_cast<unsigned>(blocks), kBlock, 0, as_stream(stream)>>>(x, y, n, vec);
  return check_launch(what);
}

// ---- copy -----------------------------------------------------------------------

// dst = src over n elements, VW per chunk, UNROLL chunks per thread (chunk
// i and i + the grid's thread count); the last n % VW elements (VW > 1
// only) by the first threads of block 0.
template <int VW, int TB, int UNROLL>
__global__ __launch_bounds__(TB) void copy_flat(float* __restrict__ dst, const float* __restrict__ src, int64_t n) {
  const int64_t nvec = n / VW;
  const int64_t threads = static_cast<int64_t>(gridDim.x) * TB;
  const int64_t i0 = static_cast<int64_t>(blockIdx.x) * TB + threadIdx.x;
  Chunk<float, VW> c[UNROLL];
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = i0 + u * threads;
    if (i < nvec) c[u].load(src + i * VW);
  }
#pragma unroll
  for (int u = 0; u < UNROLL; ++u) {
    const int64_t i = i0 + u * threads;
    if (i < nvec) c[u].store(dst + i * VW);
  }
  if constexpr (VW > 1) {
    const int64_t rest = n - nvec * VW;
    if (blockIdx.x == 0 && threadIdx.x < rest) {
      Chunk<float, 1> t;
      t.load(src + nvec * VW + threadIdx.x);
      t.store(dst + nvec * VW + threadIdx.x);
    }
  }
}

// A grid just over one resident round would run its last workgroups as a
// second round of their own (a 16.8 MB copy of 524,544 chunks took 4.48 us
// against 3.84 us for 524,288), so from one to 1.25 rounds each thread takes
// two chunks and the grid fits in one round.
template <int VW>
void launch_copy_tb(hipStream_t s, float* dst, const float* src, int64_t n) {
  const int64_t nvec = n / VW > 0 ? n / VW : 1;
  auto blocks = [](int64_t threads, int64_t tb) { return static_cast<unsigned>((threads + tb - 1) / tb); };
  if (one_wave_groups(nvec)) {
    copy_flat<VW, kWave, 1><<<blocks(nvec, kWave), kWave, 0, s>>>(dst, src, n);
  } else if (nvec > kResidentThreads) {
    copy_flat<VW, kBlock, 2><<<blocks((nvec + 1) / 2, kBlock), kBlock, 0, s>>>(dst, src, n);
  } else {
    copy_flat<VW, kBlock, 1><<<blocks(nvec, kBlock), kBlock, 0, s>>>(dst, src, n);
  }
}

// ---- SwiGLU on [rows, 2 ffn] -> [rows, ffn] -------------------------------------

// The 128-bit output chunks are stored with the sc1 policy bit (through a
// buffer resource over the launch's output, at most 1 GiB): at [8192,
// 2 x 1408] bf16 that measured 1.5-2.5% faster than nontemporal stores.
template <class T, int VW, int TB>
__global__ __launch_bounds__(TB) void swiglu_flat(const T* __restrict__ in, T* __restrict__ out, uint32_t total,
                                                  uint32_t cpr, uint64_t magic, int ffn) {
  const uint32_t t = blockIdx.x * TB + threadIdx.x;
  if (t >= total) return;
  const uint32_t row = div_by_magic(t, magic);
  const uint32_t j = t - row * cpr;
  const T* gate = in + static_cast<uint64_t>(row) * 2 * ffn + static_cast<uint64_t>(j) * VW;
  Chunk<T, VW> cg, cu;
  cg.load(gate);
  cu.load(gate + ffn);
  float g[VW], u[VW];
  cg.widen(g);
  cu.widen(u);
#pragma unroll
  for (int e = 0; e < VW; ++e) g[e] = silu_mul_f(g[e], u[e]);
  Chunk<T, VW> o;
  o.narrow(g);
  if constexpr (VW * sizeof(T) == 16) {
    const uint32_t bytes = total * 16u;  // total <= 2^26 chunks
    buffer_store16<kPolicySc1>(buffer_rsrc(out, bytes), t * 16u, o.raw);
  } else {
    o.store(out + static_cast<uint64_t>(row) * ffn + static_cast<uint64_t>(j) * VW);
  }
}

template <class T, int VW>
void launch_swiglu_tb(hipStream_t s, const T* in, T* out, uint32_t total, uint32_t cpr, uint64_t magic, int ffn) {
  const int64_t t = total;
  if (one_wave_groups(t)) {
    swiglu_flat<T, VW, kWave><<<static_cast<unsigned>((t + kWave - 1) / kWave), kWave, 0, s>>>(in, out, total, cpr,
                                                                                              magic, ffn);
  } else {
    swiglu_flat<T, VW, kBlock><<<static_cast<unsigned>((t + kBlock - 1) / kBlock), kBlock, 0, s>>>(in, out, total, cpr,
                                                                                                 magic, ffn);
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
  const int64_t cpr = vec ? ffn / kV : ffn;
  const uint32_t c32 = static_cast<uint32_t>(cpr);
  const uint64_t magic = reciprocal_magic(c32);
  const hipStream_t s = as_stream(stream);
  const int f = static_cast<int>(ffn);
  clear_launch_error();
  // Row pieces of about kPieceChunks / 4 chunks (at least one row, under
  // 2^29 chunks), so the flat chunk index of a launch stays in 32 bits.
  const int64_t piece = cpr < kPieceChunks / 4 ? kPieceChunks / 4 / cpr : 1;
  for_each_piece(rows, piece, [&](int64_t r0, int64_t rn) {
    const uint32_t t32 = static_cast<uint32_t>(rn * cpr);
    if (vec) {
      launch_swiglu_tb<T, kV>(s, in + r0 * 2 * ffn, out + r0 * ffn, t32, c32, magic, f);
    } else {
      launch_swiglu_tb<T, 1>(s, in + r0 * 2 * ffn, out + r0 * ffn, t32, c32, magic, f);
    }
  });
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
  if (n == 0 || dst == src) return UOCR_ROCM_OK;
  UOCR_REQUIRE(dst != nullptr && src != nullptr, "uocr_rocm_copy", "null pointer");
  UOCR_REQUIRE(n < kMaxElems, "uocr_rocm_copy", "n too large");
  {
    const auto d = reinterpret_cast<uintptr_t>(dst), r = reinterpret_cast<uintptr_t>(src);
    const auto bytes = static_cast<uintptr_t>(n) * sizeof(float);
    UOCR_REQUIRE(d + bytes <= r || r + bytes <= d, "uocr_rocm_copy", "dst and src must not overlap");
  }
  const hipStream_t s = as_stream(stream);
  const bool vec = aligned16(dst) && aligned16(src);
  const int vw = vec ? 4 : 1;
  const int64_t nvec = n / vw;
  clear_launch_error();
  for_each_piece(nvec, kPieceChunks, [&](int64_t c0, int64_t cn) {
    const int64_t e0 = c0 * vw, en = c0 + cn == nvec ? n - e0 : cn * vw;
    if (vec) {
      launch_copy_tb<4>(s, dst + e0, src + e0, en);
    } else {
      launch_copy_tb<1>(s, dst + e0, src + e0, en);
    }
  });
  return check_launch("uocr_rocm_copy");
}

int uocr_rocm_gelu_erf(void* stream, float* x, int64_t n) {
  return launch_flat<Flat::kGelu, float>("uocr_rocm_gelu_erf", stream, x, nullptr, n);
}

int uocr_rocm_gelu_erf_bf16(void* stream, uint16_t* x, int64_t n) {
  return launch_flat<Flat::kGelu, uint16_t>("uocr_rocm_gelu_erf_bf16", stream, x, nullptr, n);
}

int uocr_rocm_gelu_erf_to_bf16(void* stream, const float* x, uint16_t* y, int64_t n) {
  return launch_act_to_bf16<Flat::kGelu>("uocr_rocm_gelu_erf_to_bf16", stream, x, y, n);
}

int uocr_rocm_quick_gelu_to_bf16(void* stream, const float* x, uint16_t* y, int64_t n) {
  return launch_act_to_bf16<Flat::kQuickGelu>("uocr_rocm_quick_gelu_to_bf16", stream, x, y, n);
}

int uocr_rocm_quick_gelu(void* stream, float* x, int64_t n) {
  return launch_flat<Flat::kQuickGelu, float>("uocr_rocm_quick_gelu", stream, x, nullptr, n);
}

int uocr_rocm_quick_gelu_bf16(void* stream, uint16_t* x, int64_t n) {
  return launch_flat<Flat::kQuickGelu, uint16_t>("uocr_rocm_quick_gelu_bf16", stream, x, nullptr, n);
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
