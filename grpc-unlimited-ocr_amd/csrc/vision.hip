// vision.hip: the vision encoder's layout ops and SAM's relative-position
// attention bias for gfx950 (the reference's im2col, chw_to_hwc,
// hwc_to_chw, concat_cols and rel_pos_bias, src/backend/cuda/ops.h:54-58,
// 65-67,91-95, ops.cu:153-168,219-250,259-262,362-378,393-403).
//
// im2col: x [c, h, w] -> patches [oh * ow, c * kh * kw] in the weight's
// [c, kh, kw] order, zeros outside the image. One workgroup per output row
// (position), its threads over the row's columns: the row's (oy, ox) is
// computed once and consecutive threads write consecutive columns.
//
// chw_to_hwc / hwc_to_chw: a transpose of [a, b] rows through a 64 x 65
// LDS tile, both the reads and the writes row-contiguous.
//
// concat_cols: out[r] = a[r] | b[r], one workgroup per row.
//
// rel_pos_bias (one window, one head, as the reference's op): bias[t, ky *
// w + kx] = q_t . rh[qy, ky] + q_t . rw[qx, kx] for query t = qy * w + qx.
// One workgroup per query row: the q row is staged in LDS, the h + w dot
// products (fp32, in e order) are formed once into LDS, then the n biases
// are written as sums of two of them. The reference's two kernels through a
// scratch buffer become one launch that allocates nothing.
//
// split_heads / merge_heads: the attention's operands between the rows the
// projections write, x [rows, parts * heads * hd] (parts = 3 for q | k | v),
// and a head-major layout y [parts, heads, rows, hd], and the heads' outputs
// back: with every head's (and every window's) rows contiguous, one batched
// product covers all heads and windows (batch index head * windows + window,
// one stride) instead of one launch per head. 16-byte chunks, both sides
// row-contiguous; exact.
//
// rel_pos_softmax_rows: the SAM attention's scores of every window of one
// head, s [windows * n, n], replaced by softmax(s + bias) row by row with
// the bias formed as above inside the row's workgroup: the reference's
// rel_pos_bias + add_inplace + softmax_rows (src/model/cuda/cuda_vision.cpp:
// 161-166) as one read and one write of the scores. The softmax is the
// rows' own (fp32 max, exp, fp32 sum, inv = float(1 / sum) in fp64, a row
// whose max is -inf becomes zeros) with v = s + (by + bx) as the reference
// forms it.

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr float kLog2e = 1.4426950408889634f;
constexpr int kMaxRelDots = 2048;  // h + w
constexpr int kMaxRelDim = 256;    // head dim

// T float, or uint16_t: the patches rounded to bf16 (nearest even), the
// rounding the convolution's product applies to them.
template <class T>
__global__ __launch_bounds__(kBlock) void im2col_k(const float* __restrict__ x, int c, int h, int w, int kh, int kw,
                                                    int stride, int pad, int ow, int64_t rows, T* __restrict__ cols) {
  const int patch = c * kh * kw, khw = kh * kw;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    const int oy = static_cast<int>(r / ow), ox = static_cast<int>(r - static_cast<int64_t>(oy) * ow);
    const int y0 = oy * stride - pad, x0 = ox * stride - pad;
    T* out = cols + r * patch;
    for (int e = threadIdx.x; e < patch; e += kBlock) {
      const int ci = e / khw, rem = e - ci * khw, ky = rem / kw, kx = rem - ky * kw;
      const int iy = y0 + ky, ix = x0 + kx;
      const float v = (iy >= 0 && iy < h && ix >= 0 && ix < w) ? x[(static_cast<int64_t>(ci) * h + iy) * w + ix] : 0.0f;
      if constexpr (sizeof(T) == 2) {
        out[e] = f32_to_bf16(v);
      } else {
        out[e] = v;
      }
    }
  }
}

constexpr int kTile = 64;

// y [b, a] = x [a, b] transposed.
__global__ __launch_bounds__(kBlock) void transpose_k(const float* __restrict__ x, int64_t a, int64_t b,
                                                       float* __restrict__ y) {
  __shared__ float tile[kTile][kTile + 1];
  const int64_t a0 = static_cast<int64_t>(blockIdx.y) * kTile, b0 = static_cast<int64_t>(blockIdx.x) * kTile;
  const int tc = threadIdx.x % kTile, tr = threadIdx.x / kTile;
#pragma unroll
  for (int i = 0; i < kTile / (kBlock / kTile); ++i) {
    const int r = tr + (kBlock / kTile) * i;
    if (a0 + r < a && b0 + tc < b) tile[r][tc] = x[(a0 + r) * b + b0 + tc];
  }
  __syncthreads();
#pragma unroll
  for (int i = 0; i < kTile / (kBlock / kTile); ++i) {
    const int r = tr + (kBlock / kTile) * i;
    if (b0 + r < b && a0 + tc < a) y[(b0 + r) * a + a0 + tc] = tile[tc][r];
  }
}

__global__ __launch_bounds__(kBlock) void concat_cols_k(const float* __restrict__ a, int64_t ca,
                                                         const float* __restrict__ b, int64_t cb, int64_t rows,
                                                         float* __restrict__ out) {
  const int64_t width = ca + cb;
  for (int64_t r = blockIdx.x; r < rows; r += gridDim.x) {
    for (int64_t c = threadIdx.x; c < width; c += kBlock) {
      out[r * width + c] = c < ca ? a[r * ca + c] : b[r * cb + (c - ca)];
    }
  }
}

// The h + w dot products of query row q (d values) into dots: dots[j] =
// q . rh[qy, j] for j < h, q . rw[qx, j - h] after; fp32 in e order.
__device__ __forceinline__ void rel_dots(const float* __restrict__ q, int t, int h, int w, int d,
                                         const float* __restrict__ rh, const float* __restrict__ rw, float* qs,
                                         float* dots) {
  for (int e = threadIdx.x; e < d; e += kBlock) qs[e] = q[e];
  __syncthreads();
  const int qy = t / w, qx = t - qy * w;
  for (int j = threadIdx.x; j < h + w; j += kBlock) {
    const float* r = j < h ? rh + (static_cast<int64_t>(qy) * h + j) * d : rw + (static_cast<int64_t>(qx) * w + (j - h)) * d;
    float s = 0.0f;
    for (int e = 0; e < d; ++e) s += qs[e] * r[e];
    dots[j] = s;
  }
  __syncthreads();
}

__global__ __launch_bounds__(kBlock) void rel_pos_bias_k(const float* __restrict__ q, int64_t ldq, int h, int w,
                                                          int d, const float* __restrict__ rh,
                                                          const float* __restrict__ rw, float* __restrict__ bias) {
  __shared__ float qs[kMaxRelDim];
  __shared__ float dots[kMaxRelDots];
  const int n = h * w, t = blockIdx.x;
  rel_dots(q + t * ldq, t, h, w, d, rh, rw, qs, dots);
  float* row = bias + static_cast<int64_t>(t) * n;
  for (int key = threadIdx.x; key < n; key += kBlock) {
    const int ky = key / w;
    row[key] = dots[ky] + dots[h + (key - ky * w)];
  }
}

// Row R = window * n + t of s [windows * n, n]; q row R at q + R * ldq.
// kPer values per thread in registers (n <= kPer * kBlock).
template <int kPer>
__global__ __launch_bounds__(kBlock) void rel_pos_softmax_k(float* __restrict__ s, const float* __restrict__ q,
                                                             int64_t ldq, int h, int w, int d,
                                                             const float* __restrict__ rh,
                                                             const float* __restrict__ rw) {
  __shared__ float qs[kMaxRelDim];
  __shared__ float dots[kMaxRelDots];
  __shared__ float red[kWavesPerBlock];
  const int n = h * w;
  const int64_t row_id = blockIdx.x;
  const int t = static_cast<int>(row_id % n);
  float* row = s + row_id * n;
  // the scores' loads go out before the dot products
  float v[kPer];
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int key = threadIdx.x + kBlock * i;
    v[i] = key < n ? row[key] : 0.0f;
  }
  rel_dots(q + row_id * ldq, t, h, w, d, rh, rw, qs, dots);
  float m = -INFINITY;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int key = threadIdx.x + kBlock * i;
    if (key < n) {
      const int ky = key / w;
      v[i] = v[i] + (dots[ky] + dots[h + (key - ky * w)]);
      m = fmaxf(m, v[i]);
    } else {
      v[i] = -INFINITY;
    }
  }
  const float peak = block_max(m, red);
  const bool masked = peak == -INFINITY;
  float sum = 0.0f;
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    v[i] = masked ? 0.0f : __builtin_amdgcn_exp2f((v[i] - peak) * kLog2e);
    sum += v[i];
  }
  const float total = block_sum(sum, red);
  const float inv = masked ? 0.0f : static_cast<float>(1.0 / static_cast<double>(total));
#pragma unroll
  for (int i = 0; i < kPer; ++i) {
    const int key = threadIdx.x + kBlock * i;
    if (key < n) row[key] = v[i] * inv;
  }
}

// Rows wider than the registers hold: three passes over the row (bias
// added in place first).
__global__ __launch_bounds__(kBlock) void rel_pos_softmax_wide_k(float* __restrict__ s, const float* __restrict__ q,
                                                                  int64_t ldq, int h, int w, int d,
                                                                  const float* __restrict__ rh,
                                                                  const float* __restrict__ rw) {
  __shared__ float qs[kMaxRelDim];
  __shared__ float dots[kMaxRelDots];
  __shared__ float red[kWavesPerBlock];
  const int n = h * w;
  const int64_t row_id = blockIdx.x;
  const int t = static_cast<int>(row_id % n);
  float* row = s + row_id * n;
  rel_dots(q + row_id * ldq, t, h, w, d, rh, rw, qs, dots);
  float m = -INFINITY;
  for (int key = threadIdx.x; key < n; key += kBlock) {
    const int ky = key / w;
    const float v = row[key] + (dots[ky] + dots[h + (key - ky * w)]);
    row[key] = v;
    m = fmaxf(m, v);
  }
  const float peak = block_max(m, red);
  const bool masked = peak == -INFINITY;
  float sum = 0.0f;
  for (int key = threadIdx.x; key < n; key += kBlock) {
    sum += masked ? 0.0f : __builtin_amdgcn_exp2f((row[key] - peak) * kLog2e);
  }
  const float total = block_sum(sum, red);
  const float inv = masked ? 0.0f : static_cast<float>(1.0 / static_cast<double>(total));
  for (int key = threadIdx.x; key < n; key += kBlock) {
    row[key] = masked ? 0.0f : __builtin_amdgcn_exp2f((row[key] - peak) * kLog2e) * inv;
  }
}

// y [parts, heads, rows, hd] = x [rows, parts, heads, hd]; hd % 4 == 0.
__global__ __launch_bounds__(kBlock) void split_heads_k(const float* __restrict__ x, int64_t rows, int parts_heads,
                                                         int hd4, float* __restrict__ y) {
  const int64_t row_chunks = static_cast<int64_t>(parts_heads) * hd4, total = rows * row_chunks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t r = i / row_chunks;
    const int rem = static_cast<int>(i - r * row_chunks), ph = rem / hd4, e = rem - ph * hd4;
    const u32x4 v = reinterpret_cast<const u32x4*>(x)[i];
    reinterpret_cast<u32x4*>(y)[(static_cast<int64_t>(ph) * rows + r) * hd4 + e] = v;
  }
}

// y [rows, heads, hd] = x [heads, rows, hd]; hd % 4 == 0.
__global__ __launch_bounds__(kBlock) void merge_heads_k(const float* __restrict__ x, int heads, int64_t rows, int hd4,
                                                         float* __restrict__ y) {
  const int64_t row_chunks = static_cast<int64_t>(heads) * hd4, total = rows * row_chunks;
  for (int64_t i = static_cast<int64_t>(blockIdx.x) * kBlock + threadIdx.x; i < total;
       i += static_cast<int64_t>(gridDim.x) * kBlock) {
    const int64_t r = i / row_chunks;
    const int rem = static_cast<int>(i - r * row_chunks), h = rem / hd4, e = rem - h * hd4;
    reinterpret_cast<u32x4*>(y)[i] = reinterpret_cast<const u32x4*>(x)[(static_cast<int64_t>(h) * rows + r) * hd4 + e];
  }
}

unsigned flat_grid(int64_t chunks) {
  const int64_t b = (chunks + kBlock - 1) / kBlock;
  return static_cast<unsigned>(b < (int64_t{1} << 20) ? (b > 0 ? b : 1) : (int64_t{1} << 20));
}

unsigned row_grid(int64_t rows) { return static_cast<unsigned>(rows < (int64_t{1} << 20) ? rows : (int64_t{1} << 20)); }

int transpose_entry(const char* what, void* stream, const float* x, int64_t a, int64_t b, float* y) {
  UOCR_REQUIRE(a >= 0 && b >= 0, what, "dimensions must be >= 0");
  if (a == 0 || b == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && y != nullptr, what, "null pointer");
  const int64_t gx = (b + kTile - 1) / kTile, gy = (a + kTile - 1) / kTile;
  UOCR_REQUIRE(gx < (int64_t{1} << 31) && gy < 65536, what, "tensor too large");
  clear_launch_error();
  transpose_k<<<dim3(static_cast<unsigned>(gx), static_cast<unsigned>(gy)), kBlock, 0, as_stream(stream)>>>(x, a, b, y);
  return check_launch(what);
}

int rel_shape_ok(int64_t ldq, int64_t h, int64_t w, int64_t d) {
  return h >= 1 && w >= 1 && d >= 1 && d <= kMaxRelDim && h + w <= kMaxRelDots && ldq >= d && h * w < (1 << 24);
}

}  // namespace
}  // namespace uocr_rocm

namespace uocr_rocm {
namespace {

template <class T>
int im2col_entry(const char* kWhat, void* stream, const float* x, int64_t c, int64_t h, int64_t w, int64_t kh,
                 int64_t kw, int64_t stride, int64_t pad, T* cols) {
  UOCR_REQUIRE(c >= 1 && h >= 1 && w >= 1 && kh >= 1 && kw >= 1 && stride >= 1 && pad >= 0, kWhat,
               "c, h, w, kh, kw and stride must be >= 1 and pad >= 0");
  UOCR_REQUIRE(h < (1 << 24) && w < (1 << 24) && c * kh * kw < (int64_t{1} << 30) && pad < (1 << 20) &&
                   stride < (1 << 20),
               kWhat, "shape too large");
  const int64_t oh = (h + 2 * pad - kh) / stride + 1, ow = (w + 2 * pad - kw) / stride + 1;
  UOCR_REQUIRE(h + 2 * pad >= kh && w + 2 * pad >= kw, kWhat, "kernel larger than the padded image");
  UOCR_REQUIRE(x != nullptr && cols != nullptr, kWhat, "null pointer");
  clear_launch_error();
  im2col_k<<<row_grid(oh * ow), kBlock, 0, as_stream(stream)>>>(
      x, static_cast<int>(c), static_cast<int>(h), static_cast<int>(w), static_cast<int>(kh), static_cast<int>(kw),
      static_cast<int>(stride), static_cast<int>(pad), static_cast<int>(ow), oh * ow, cols);
  return check_launch(kWhat);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {


int uocr_rocm_im2col(void* stream, const float* x, int64_t c, int64_t h, int64_t w, int64_t kh, int64_t kw,
                     int64_t stride, int64_t pad, float* cols) {
  return im2col_entry("uocr_rocm_im2col", stream, x, c, h, w, kh, kw, stride, pad, cols);
}

int uocr_rocm_im2col_bf16(void* stream, const float* x, int64_t c, int64_t h, int64_t w, int64_t kh, int64_t kw,
                          int64_t stride, int64_t pad, uint16_t* cols) {
  return im2col_entry("uocr_rocm_im2col_bf16", stream, x, c, h, w, kh, kw, stride, pad, cols);
}

int uocr_rocm_chw_to_hwc(void* stream, const float* x, int64_t c, int64_t h, int64_t w, float* y) {
  UOCR_REQUIRE(h >= 0 && w >= 0 && (h == 0 || w < (int64_t{1} << 62) / h), "uocr_rocm_chw_to_hwc", "bad h, w");
  return transpose_entry("uocr_rocm_chw_to_hwc", stream, x, c, h * w, y);
}

int uocr_rocm_hwc_to_chw(void* stream, const float* x, int64_t h, int64_t w, int64_t c, float* y) {
  UOCR_REQUIRE(h >= 0 && w >= 0 && (h == 0 || w < (int64_t{1} << 62) / h), "uocr_rocm_hwc_to_chw", "bad h, w");
  return transpose_entry("uocr_rocm_hwc_to_chw", stream, x, h * w, c, y);
}

int uocr_rocm_concat_cols(void* stream, const float* a, int64_t ca, const float* b, int64_t cb, int64_t rows,
                          float* out) {
  constexpr const char* kWhat = "uocr_rocm_concat_cols";
  UOCR_REQUIRE(ca >= 0 && cb >= 0 && rows >= 0, kWhat, "ca, cb and rows must be >= 0");
  if (rows == 0 || ca + cb == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(out != nullptr && (ca == 0 || a != nullptr) && (cb == 0 || b != nullptr), kWhat, "null pointer");
  clear_launch_error();
  concat_cols_k<<<row_grid(rows), kBlock, 0, as_stream(stream)>>>(a, ca, b, cb, rows, out);
  return check_launch(kWhat);
}

int uocr_rocm_split_heads(void* stream, const float* x, int64_t rows, int64_t parts, int64_t heads, int64_t hd,
                          float* y) {
  constexpr const char* kWhat = "uocr_rocm_split_heads";
  UOCR_REQUIRE(rows >= 0 && parts >= 1 && heads >= 1 && hd >= 4 && hd % 4 == 0, kWhat,
               "need rows >= 0, parts and heads >= 1, hd a multiple of 4");
  UOCR_REQUIRE(parts * heads < (1 << 20) && hd < (1 << 20), kWhat, "too many heads or too wide");
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && y != nullptr, kWhat, "null pointer");
  UOCR_REQUIRE(aligned16(x) && aligned16(y), kWhat, "x and y must be 16-byte aligned");
  clear_launch_error();
  split_heads_k<<<flat_grid(rows * parts * heads * hd / 4), kBlock, 0, as_stream(stream)>>>(
      x, rows, static_cast<int>(parts * heads), static_cast<int>(hd / 4), y);
  return check_launch(kWhat);
}

int uocr_rocm_merge_heads(void* stream, const float* x, int64_t heads, int64_t rows, int64_t hd, float* y) {
  constexpr const char* kWhat = "uocr_rocm_merge_heads";
  UOCR_REQUIRE(rows >= 0 && heads >= 1 && hd >= 4 && hd % 4 == 0, kWhat,
               "need rows >= 0, heads >= 1, hd a multiple of 4");
  UOCR_REQUIRE(heads < (1 << 20) && hd < (1 << 20), kWhat, "too many heads or too wide");
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr && y != nullptr, kWhat, "null pointer");
  UOCR_REQUIRE(aligned16(x) && aligned16(y), kWhat, "x and y must be 16-byte aligned");
  clear_launch_error();
  merge_heads_k<<<flat_grid(rows * heads * hd / 4), kBlock, 0, as_stream(stream)>>>(
      x, static_cast<int>(heads), rows, static_cast<int>(hd / 4), y);
  return check_launch(kWhat);
}

int uocr_rocm_rel_pos_bias(void* stream, const float* q, int64_t ldq, int64_t h, int64_t w, int64_t d,
                           const float* rh, const float* rw, float* bias) {
  constexpr const char* kWhat = "uocr_rocm_rel_pos_bias";
  UOCR_REQUIRE(rel_shape_ok(ldq, h, w, d), kWhat,
               "need h, w, d >= 1, d <= 256, h + w <= 2048, h * w < 2^24 and ldq >= d");
  UOCR_REQUIRE(q != nullptr && rh != nullptr && rw != nullptr && bias != nullptr, kWhat, "null pointer");
  clear_launch_error();
  rel_pos_bias_k<<<static_cast<unsigned>(h * w), kBlock, 0, as_stream(stream)>>>(
      q, ldq, static_cast<int>(h), static_cast<int>(w), static_cast<int>(d), rh, rw, bias);
  return check_launch(kWhat);
}

int uocr_rocm_rel_pos_softmax_rows(void* stream, float* scores, int64_t windows, const float* q, int64_t ldq,
                                   int64_t h, int64_t w, int64_t d, const float* rh, const float* rw) {
  constexpr const char* kWhat = "uocr_rocm_rel_pos_softmax_rows";
  UOCR_REQUIRE(windows >= 0, kWhat, "windows must be >= 0");
  if (windows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(rel_shape_ok(ldq, h, w, d), kWhat,
               "need h, w, d >= 1, d <= 256, h + w <= 2048, h * w < 2^24 and ldq >= d");
  const int64_t n = h * w;
  UOCR_REQUIRE(windows * n < (int64_t{1} << 31), kWhat, "windows * h * w must be below 2^31");
  UOCR_REQUIRE(scores != nullptr && q != nullptr && rh != nullptr && rw != nullptr, kWhat, "null pointer");
  const unsigned grid = static_cast<unsigned>(windows * n);
  const hipStream_t st = as_stream(stream);
  const int hi = static_cast<int>(h), wi = static_cast<int>(w), di = static_cast<int>(d);
  clear_launch_error();
  if (n <= kBlock) {
    rel_pos_softmax_k<1><<<grid, kBlock, 0, st>>>(scores, q, ldq, hi, wi, di, rh, rw);
  } else if (n <= 2 * kBlock) {
    rel_pos_softmax_k<2><<<grid, kBlock, 0, st>>>(scores, q, ldq, hi, wi, di, rh, rw);
  } else if (n <= 4 * kBlock) {
    rel_pos_softmax_k<4><<<grid, kBlock, 0, st>>>(scores, q, ldq, hi, wi, di, rh, rw);
  } else if (n <= 8 * kBlock) {
    rel_pos_softmax_k<8><<<grid, kBlock, 0, st>>>(scores, q, ldq, hi, wi, di, rh, rw);
  } else if (n <= 16 * kBlock) {
    rel_pos_softmax_k<16><<<grid, kBlock, 0, st>>>(scores, q, ldq, hi, wi, di, rh, rw);
  } else {
    rel_pos_softmax_wide_k<<<grid, kBlock, 0, st>>>(scores, q, ldq, hi, wi, di, rh, rw);
  }
  return check_launch(kWhat);
}

}  // extern "C"
