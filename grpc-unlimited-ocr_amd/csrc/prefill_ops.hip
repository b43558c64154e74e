// prefill_ops.hip: the fp32 products and row moves of a prefill pass for
// gfx950 (the reference's gemm_nt, gemm_nn, gather_rows and
// scatter_add_rows, src/backend/cuda/ops.h:19-27,56-60, ops.cu:185-190,
// 289-309, 377-391).
//
// gemm_nt / gemm_nn: c[b] = alpha a[b] . b[b]^T (b rows k-contiguous) or
// a[b] . b[b] (b rows n-contiguous), batched over slices `stride_*` elements
// apart, leading dimensions given. A workgroup of 256 threads computes a
// 64 x 64 tile of one slice; each thread a 4 x 4 block. k advances 16 at a
// time through LDS, both operands held k-major there so that a thread reads
// its 4 a values and 4 b values as two 16-byte loads per k. Sums are fp32
// (fused multiply-adds), alpha applied to the finished sum. Any m, n, k.
//
// gather_rows: dst[i] = src[index[i]]; scatter_add_rows: dst[index[i]] +=
// weight[i] * src[i] for i in order (each column walks the rows in order, so
// an index that repeats accumulates deterministically, as in the reference).

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int kGM = 64, kGN = 64, kGK = 16;
constexpr int kGemmBlock = 256;

struct GemmArgs {
  const float* a;
  const float* b;
  float* c;
  int64_t m, n, k;
  int64_t lda, ldb, ldc;
  int64_t sa, sb, sc;
  float alpha;
};

template <bool kNT>
__global__ __launch_bounds__(kGemmBlock) void gemm_f32_k(const GemmArgs g) {
  __shared__ __attribute__((aligned(16))) float as[kGK][kGM + 4];
  __shared__ __attribute__((aligned(16))) float bs[kGK][kGN + 4];
  const int64_t slice = blockIdx.z;
  const float* A = g.a + slice * g.sa;
  const float* B = g.b + slice * g.sb;
  float* C = g.c + slice * g.sc;
  const int64_t m0 = static_cast<int64_t>(blockIdx.y) * kGM, n0 = static_cast<int64_t>(blockIdx.x) * kGN;
  const int tx = threadIdx.x % 16, ty = threadIdx.x / 16;
  float acc[4][4];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
#pragma unroll
    for (int j = 0; j < 4; ++j) acc[i][j] = 0.0f;
  }
  for (int64_t k0 = 0; k0 < g.k; k0 += kGK) {
#pragma unroll
    for (int i = 0; i < kGM * kGK / kGemmBlock; ++i) {
      const int id = static_cast<int>(threadIdx.x) + kGemmBlock * i;
      const int r = id / kGK, kk = id % kGK;
      const int64_t row = m0 + r, kc = k0 + kk;
      as[kk][r] = row < g.m && kc < g.k ? A[row * g.lda + kc] : 0.0f;
    }
    if constexpr (kNT) {
#pragma unroll
      for (int i = 0; i < kGN * kGK / kGemmBlock; ++i) {
        const int id = static_cast<int>(threadIdx.x) + kGemmBlock * i;
        const int r = id / kGK, kk = id % kGK;
        const int64_t col = n0 + r, kc = k0 + kk;
        bs[kk][r] = col < g.n && kc < g.k ? B[col * g.ldb + kc] : 0.0f;
      }
    } else {
#pragma unroll
      for (int i = 0; i < kGN * kGK / kGemmBlock; ++i) {
        const int id = static_cast<int>(threadIdx.x) + kGemmBlock * i;
        const int kk = id / kGN, cc = id % kGN;
        const int64_t col = n0 + cc, kc = k0 + kk;
        bs[kk][cc] = col < g.n && kc < g.k ? B[kc * g.ldb + col] : 0.0f;
      }
    }
    __syncthreads();
#pragma unroll
    for (int kk = 0; kk < kGK; ++kk) {
      const u32x4 av = *reinterpret_cast<const u32x4*>(&as[kk][4 * ty]);
      const u32x4 bv = *reinterpret_cast<const u32x4*>(&bs[kk][4 * tx]);
      const float a4[4] = {__uint_as_float(av.x), __uint_as_float(av.y), __uint_as_float(av.z), __uint_as_float(av.w)};
      const float b4[4] = {__uint_as_float(bv.x), __uint_as_float(bv.y), __uint_as_float(bv.z), __uint_as_float(bv.w)};
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = __builtin_fmaf(a4[i], b4[j], acc[i][j]);
      }
    }
    __syncthreads();
  }
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int64_t row = m0 + 4 * ty + i;
    if (row >= g.m) continue;
#pragma unroll
    for (int j = 0; j < 4; ++j) {
      const int64_t col = n0 + 4 * tx + j;
      if (col < g.n) C[row * g.ldc + col] = g.alpha * acc[i][j];
    }
  }
}

__global__ __launch_bounds__(kBlock) void gather_rows_f32_k(const float* __restrict__ src,
                                                            const int64_t* __restrict__ index, int64_t rows,
                                                            int64_t cols, float* __restrict__ dst) {
  const int64_t total = rows * cols;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t r = i / cols, c = i - r * cols;
    dst[i] = src[index[r] * cols + c];
  }
}

__global__ __launch_bounds__(kBlock) void scatter_add_rows_k(float* __restrict__ dst, const int64_t* __restrict__ index,
                                                             const float* __restrict__ weight,
                                                             const float* __restrict__ src, int64_t rows,
                                                             int64_t cols) {
#pragma clang fp contract(off)
  const int64_t c = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x;
  if (c >= cols) return;
  for (int64_t r = 0; r < rows; ++r) {
    float* d = dst + index[r] * cols + c;
    *d = *d + weight[r] * src[r * cols + c];
  }
}

int gemm_entry(const char* what, bool nt, void* stream, int64_t m, int64_t n, int64_t k, float alpha, const float* a,
               int64_t lda, int64_t stride_a, const float* b, int64_t ldb, int64_t stride_b, float* c, int64_t ldc,
               int64_t stride_c, int64_t batch) {
  UOCR_REQUIRE(m >= 0 && n >= 0 && k >= 0 && batch >= 0, what, "m, n, k and batch must be >= 0");
  if (m == 0 || n == 0 || batch == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(a != nullptr && b != nullptr && c != nullptr, what, "null pointer");
  UOCR_REQUIRE(lda >= k && ldc >= n && ldb >= (nt ? k : n), what, "a leading dimension is below the row width");
  UOCR_REQUIRE(stride_a >= 0 && stride_b >= 0 && stride_c >= 0, what, "strides must be >= 0");
  const int64_t gx = (n + kGN - 1) / kGN, gy = (m + kGM - 1) / kGM;
  UOCR_REQUIRE(gx < (int64_t{1} << 31) && gy < 65536 && batch < 65536, what, "grid too large");
  GemmArgs g{a, b, c, m, n, k, lda, ldb, ldc, stride_a, stride_b, stride_c, alpha};
  const dim3 grid(static_cast<unsigned>(gx), static_cast<unsigned>(gy), static_cast<unsigned>(batch));
  clear_launch_error();
  if (nt) {
    gemm_f32_k<true><<<grid, kGemmBlock, 0, as_stream(stream)>>>(g);
  } else {
    gemm_f32_k<false><<<grid, kGemmBlock, 0, as_stream(stream)>>>(g);
  }
  return check_launch(what);
}

unsigned flat_blocks(int64_t total) {
  const int64_t b = (total + kBlock - 1) / kBlock;
  return static_cast<unsigned>(b < 65536 ? (b > 0 ? b : 1) : 65536);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_gemm_nt(void* stream, int64_t m, int64_t n, int64_t k, float alpha, const float* a, int64_t lda,
                      int64_t stride_a, const float* b, int64_t ldb, int64_t stride_b, float* c, int64_t ldc,
                      int64_t stride_c, int64_t batch) {
  return gemm_entry("uocr_rocm_gemm_nt", true, stream, m, n, k, alpha, a, lda, stride_a, b, ldb, stride_b, c, ldc,
                    stride_c, batch);
}

int uocr_rocm_gemm_nn(void* stream, int64_t m, int64_t n, int64_t k, const float* a, int64_t lda, int64_t stride_a,
                      const float* b, int64_t ldb, int64_t stride_b, float* c, int64_t ldc, int64_t stride_c,
                      int64_t batch) {
  return gemm_entry("uocr_rocm_gemm_nn", false, stream, m, n, k, 1.0f, a, lda, stride_a, b, ldb, stride_b, c, ldc,
                    stride_c, batch);
}

int uocr_rocm_gather_rows(void* stream, const float* src, const int64_t* index, int64_t rows, int64_t cols,
                          float* dst) {
  constexpr const char* kWhat = "uocr_rocm_gather_rows";
  UOCR_REQUIRE(rows >= 0 && cols >= 0, kWhat, "rows and cols must be >= 0");
  if (rows == 0 || cols == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(src != nullptr && index != nullptr && dst != nullptr, kWhat, "null pointer");
  clear_launch_error();
  gather_rows_f32_k<<<flat_blocks(rows * cols), kBlock, 0, as_stream(stream)>>>(src, index, rows, cols, dst);
  return check_launch(kWhat);
}

int uocr_rocm_scatter_add_rows(void* stream, float* dst, const int64_t* index, const float* weight, const float* src,
                               int64_t rows, int64_t cols) {
  constexpr const char* kWhat = "uocr_rocm_scatter_add_rows";
  UOCR_REQUIRE(rows >= 0 && cols >= 0, kWhat, "rows and cols must be >= 0");
  if (rows == 0 || cols == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(dst != nullptr && index != nullptr && weight != nullptr && src != nullptr, kWhat, "null pointer");
  UOCR_REQUIRE(cols < (int64_t{1} << 40), kWhat, "cols too large");
  clear_launch_error();
  scatter_add_rows_k<<<static_cast<unsigned>((cols + kBlock - 1) / kBlock), kBlock, 0, as_stream(stream)>>>(
      dst, index, weight, src, rows, cols);
  return check_launch(kWhat);
}

}  // extern "C"
