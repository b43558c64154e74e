// gemm.hip: the prefill projection y[m, n] = bf16(x)[m, k] . w[n, k]^T
// (+ bias[n]) on gfx950's bf16 matrix cores, fp32 accumulation and output:
// the reference's cuda::linear for m > 1 (src/backend/cuda/ops.h:14-17,
// ops.cu:268-287, which rounds x to bf16 in its own pass and calls a bf16
// cuBLAS GEMM with fp32 compute, then adds the bias).
//
// Both operands are k-contiguous (x rows, w rows), so one tile layout serves
// both. A workgroup of 4 waves computes a 128 x 128 tile of y; wave (wm, wn)
// owns a 64 x 64 quarter as 2 x 2 v_mfma_f32_32x32x16_bf16 tiles. The k
// loop steps 64 at a time through LDS, double-buffered: the next step's
// x (fp32, rounded to bf16 with the hardware's nearest-even conversion as
// it is staged) and w chunks are loaded into registers while the current
// step's 16 matrix products run, then written to the other buffer. Tile rows
// are 8 chunks of 8 bf16 (16 bytes); a chunk's slot is XOR-swizzled by the
// row so that the 32 rows one operand read spans fall on different banks.
// The bias is added to each finished sum (one fp32 rounding, as the
// reference's separate bias pass).

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

__device__ __forceinline__ int slot(int row, int chunk) { return row * kRowChunks + (chunk ^ (row & 7)); }

struct LinearArgs {
  const float* x;
  const uint16_t* w;
  const float* bias;
  float* y;
  int64_t m, n;
  int k;
  int tiles_n;
};

// The registers one k step stages: per thread kChunksPerThread chunks of the
// x tile (8 floats each, rounded on the way to LDS) and of the w tile.
struct Staged {
  u32x4 xa[kChunksPerThread][2];
  u32x4 wb[kChunksPerThread];
};

__device__ __forceinline__ void load_step(const LinearArgs& a, int64_t m0, int64_t n0, int k0, Staged& s) {
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int id = static_cast<int>(threadIdx.x) + kGemmThreads * i;
    const int row = id / kRowChunks, c = id % kRowChunks;
    const int kc = k0 + 8 * c;
    const bool kin = kc < a.k;
    const int64_t xr = m0 + row, wr = n0 + row;
    s.xa[i][0] = s.xa[i][1] = u32x4{0u, 0u, 0u, 0u};
    s.wb[i] = u32x4{0u, 0u, 0u, 0u};
    if (kin && xr < a.m) {
      const u32x4* p = reinterpret_cast<const u32x4*>(a.x + xr * a.k + kc);
      s.xa[i][0] = p[0];
      s.xa[i][1] = p[1];
    }
    if (kin && wr < a.n) s.wb[i] = *reinterpret_cast<const u32x4*>(a.w + wr * a.k + kc);
  }
}

__device__ __forceinline__ void store_step(const Staged& s, u32x4* xs, u32x4* ws) {
#pragma unroll
  for (int i = 0; i < kChunksPerThread; ++i) {
    const int id = static_cast<int>(threadIdx.x) + kGemmThreads * i;
    const int row = id / kRowChunks, c = id % kRowChunks;
    const u32x4 lo = s.xa[i][0], hi = s.xa[i][1];
    xs[slot(row, c)] = u32x4{pack_bf16(__uint_as_float(lo.x), __uint_as_float(lo.y)),
                             pack_bf16(__uint_as_float(lo.z), __uint_as_float(lo.w)),
                             pack_bf16(__uint_as_float(hi.x), __uint_as_float(hi.y)),
                             pack_bf16(__uint_as_float(hi.z), __uint_as_float(hi.w))};
    ws[slot(row, c)] = s.wb[i];
  }
}

__device__ __forceinline__ bf16x8 as_bf16x8(u32x4 v) { return __builtin_bit_cast(bf16x8, v); }

__global__ __launch_bounds__(kGemmThreads) void linear_bf16_k(const LinearArgs a) {
  __shared__ u32x4 xs[2][kTileChunks];
  __shared__ u32x4 ws[2][kTileChunks];
  const int tile = blockIdx.x;
  const int64_t m0 = static_cast<int64_t>(tile / a.tiles_n) * kTileM;
  const int64_t n0 = static_cast<int64_t>(tile % a.tiles_n) * kTileN;
  const int lane = threadIdx.x & (kWave - 1), wave = wave_in_block();
  const int wm = wave >> 1, wn = wave & 1;
  const int half = lane >> 5, r32 = lane & 31;

  f32x16 acc[2][2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    }
  }

  const int steps = (a.k + kTileK - 1) / kTileK;
  Staged s;
  load_step(a, m0, n0, 0, s);
  store_step(s, xs[0], ws[0]);
  lds_barrier();
  for (int t = 0; t < steps; ++t) {
    const int buf = t & 1;
    const bool more = t + 1 < steps;
    if (more) load_step(a, m0, n0, (t + 1) * kTileK, s);
#pragma unroll
    for (int kk = 0; kk < kTileK / 16; ++kk) {
      const int c = 2 * kk + half;
      bf16x8 fa[2], fb[2];
#pragma unroll
      for (int i = 0; i < 2; ++i) fa[i] = as_bf16x8(xs[buf][slot(64 * wm + 32 * i + r32, c)]);
#pragma unroll
      for (int j = 0; j < 2; ++j) fb[j] = as_bf16x8(ws[buf][slot(64 * wn + 32 * j + r32, c)]);
#pragma unroll
      for (int i = 0; i < 2; ++i) {
#pragma unroll
        for (int j = 0; j < 2; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(fa[i], fb[j], acc[i][j], 0, 0, 0);
      }
    }
    if (more) store_step(s, xs[buf ^ 1], ws[buf ^ 1]);
    lds_barrier();
  }

  // acc[i][j][r] is y row 8 (r / 4) + 4 half + r % 4 of the 32 x 32 tile, column r32
#pragma unroll
  for (int j = 0; j < 2; ++j) {
    const int64_t col = n0 + 64 * wn + 32 * j + r32;
    if (col >= a.n) continue;
    const float bv = a.bias != nullptr ? a.bias[col] : 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i) {
#pragma unroll
      for (int r = 0; r < 16; ++r) {
        const int64_t row = m0 + 64 * wm + 32 * i + 8 * (r / 4) + 4 * half + (r % 4);
        if (row < a.m) a.y[row * a.n + col] = a.bias != nullptr ? acc[i][j][r] + bv : acc[i][j][r];
      }
    }
  }
}

}  // namespace

int linear_entry(const char* what, void* stream, const float* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                 const float* bias, float* y) {
  UOCR_REQUIRE(m >= 0 && n >= 0 && k >= 0, what, "m, n and k must be >= 0");
  if (m == 0 || n == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(k % 8 == 0 && k >= 8 && k < (int64_t{1} << 30), what, "k must be a multiple of 8 in [8, 2^30)");
  UOCR_REQUIRE(x != nullptr && w != nullptr && y != nullptr, what, "null x, w or y");
  UOCR_REQUIRE(aligned16(x) && aligned16(w), what, "x and w must be 16-byte aligned");
  const int64_t tiles_m = (m + kTileM - 1) / kTileM, tiles_n = (n + kTileN - 1) / kTileN;
  UOCR_REQUIRE(tiles_m * tiles_n < (int64_t{1} << 31), what, "too many tiles");
  LinearArgs a{x, w, bias, y, m, n, static_cast<int>(k), static_cast<int>(tiles_n)};
  clear_launch_error();
  linear_bf16_k<<<static_cast<unsigned>(tiles_m * tiles_n), kGemmThreads, 0, as_stream(stream)>>>(a);
  return check_launch(what);
}

}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_linear(void* stream, const float* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                     const float* bias, float* y) {
  // One row streams the weights once through the GEMV (the reference's
  // m == 1 path, ops.cu:271-274).
  if (m == 1 && k <= 12288) return uocr_rocm_gemv_bf16(stream, x, k, w, n, bias, y);
  return linear_entry("uocr_rocm_linear", stream, x, m, k, w, n, bias, y);
}

}  // extern "C"
