// softmax.hip: row softmax and the attention scores' scale-and-mask for
// gfx950, fp32. These are the row ops on either side of the attention
// products in prefill and in the vision encoder (the reference's
// softmax_rows and scale_add_mask, src/backend/cuda/ops.h:41-46).
//
// scale_mask_softmax_rows fuses the two: the scores are scaled and masked in
// registers on the softmax's read, so they cross HBM once instead of twice.
//
// softmax_rows, layout as the norms (norm.hip): the row in registers, 64-
// chunk groups, WPR waves per row (about two groups per wave). Three steps
// over the registers: the row max (an exact fold), e = exp(v - max) and its sum
// (folded in group order, so the result is bitwise independent of WPR and of
// the row count), then v = e / sum. Rows wider than the registers hold take
// softmax_rows_wide (one workgroup per row, three reads of the row).
//
// Arithmetic (reference: src/backend/reference/ops.cpp:169-187): fp32 max;
// exp(v - max) in fp32 (here 2^((v - max) log2 e) on v_exp_f32); sum in fp32
// over the groups, inv = float(1 / sum) in fp64 as the reference forms it
// from its fp64 total; a row whose max is -inf (fully masked) becomes zeros.
//
// scale_add_mask (src/backend/cuda/ops.cu:129-132): x[b, r, c] =
// x[b, r, c] * scale + mask[r, c] over `batch` slices. A thread owns one
// 128-bit mask chunk and up to 4 slices of it, so the mask is read once per
// 4 slices rather than once per slice.

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr float kLog2e = 1.4426950408889634f;

// With kMask the row is first scaled and masked in registers, v = x * scale
// + mask[row mod mask_rows] (no contraction), exactly as scale_add_mask forms
// it: scale_mask_softmax_rows is then bitwise scale_add_mask + softmax_rows
// with one read and one write of the scores instead of two of each.
// Rows are visited mask-row-major: logical row R is slice R mod batch of mask
// row R / batch, and the blocks run in XCD-aware order (xcd_block), so the
// `batch` rows that share a mask row run side by side on one XCD and the
// mask row is read once into its L2 (258 -> 240 us on [10 x 4096, 4096]).
// A launch may cover mask rows first .. of the call (row pieces): its logical
// row r is slice r mod batch of mask row first + r / batch.
struct RowMask {
  const float* mask;  // [mask_rows, cols], or null (+ 0)
  float scale;
  int64_t mask_rows;
  int64_t batch;
  int64_t first;
  __device__ __forceinline__ int64_t mask_row(int64_t r) const { return first + r / batch; }
  __device__ __forceinline__ int64_t data_row(int64_t r) const {
    return (r % batch) * mask_rows + first + r / batch;
  }
};

// Waves per row (WPR) and workgroup size: one wave per row in 4-wave
// workgroups for rows of 1-3 chunk groups, else about two groups per wave
// (WPR = 2, 4, 8) with one row per workgroup. Measured on [10 x rows, cols]
// fp32 scores (640 MB) against one wave per row (4 waves at a mask): 1024
// columns 1-3% faster, 2048 6% (unmasked), 4096 13% (unmasked) and 4% (the
// one-pass masked kernel), 8192 masked 10% faster and unmasked 5% slower.
template <int WPR>
constexpr int softmax_block() {
  return WPR == 1 ? kBlock : WPR * kWave;
}

template <int VW, int WPR, int VPL, bool kMask>
__global__ __launch_bounds__(softmax_block<WPR>()) void softmax_rows_k(float* __restrict__ x, int64_t rows, int cols,
                                                                      RowMask rm) {
  constexpr int kRowsPerBlock = softmax_block<WPR>() / kWave / WPR;
  __shared__ float red[kRowsPerBlock][kMaxGroups];
  const int wave = threadIdx.x / kWave;
  const int lane = threadIdx.x & (kWave - 1);
  const int rloc = wave / WPR, wr = wave % WPR;
  // With a mask, XCD-aware order: the rows of one mask row run on one XCD.
  const unsigned blk = kMask ? xcd_block(blockIdx.x, gridDim.x) : blockIdx.x;
  const int64_t row = static_cast<int64_t>(blk) * kRowsPerBlock + rloc;
  const bool active = row < rows;
  const int nvec = cols / VW;
  const int groups = (nvec + kWave - 1) / kWave;
  const int64_t off = (active ? (kMask ? rm.data_row(row) : row) : 0) * cols;

  Chunk<float, VW> cx[VPL];
  float v[VPL][VW];
  float part[VPL];
  // The mask chunks load together with the scores: a mask load issued after
  // the scores' loads and waited on alone would drain the whole queue.
  float m[kMask ? VPL : 1][VW];
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = (wr + WPR * k) * kWave + lane;
    if (active && c < nvec) {
      cx[k].load(x + off + static_cast<int64_t>(c) * VW);
      if constexpr (kMask) {
        if (rm.mask != nullptr) {
          load_f32<VW>(rm.mask + rm.mask_row(row) * cols + static_cast<int64_t>(c) * VW, m[k]);
        } else {
#pragma unroll
          for (int e = 0; e < VW; ++e) m[k][e] = 0.0f;
        }
      }
    }
  }
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = (wr + WPR * k) * kWave + lane;
    part[k] = -INFINITY;
    if (active && c < nvec) {
      cx[k].widen(v[k]);
      if constexpr (kMask) {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < VW; ++e) v[k][e] = v[k][e] * rm.scale + m[k][e];
      }
#pragma unroll
      for (int e = 0; e < VW; ++e) part[k] = fmaxf(part[k], v[k][e]);
    } else {
#pragma unroll
      for (int e = 0; e < VW; ++e) v[k][e] = -INFINITY;
    }
  }
  const float peak = fold_groups<WPR, VPL, true>(part, wr, groups, red[rloc]);
  const bool masked = peak == -INFINITY;
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    part[k] = 0.0f;
#pragma unroll
    for (int e = 0; e < VW; ++e) {
      v[k][e] = masked ? 0.0f : __builtin_amdgcn_exp2f((v[k][e] - peak) * kLog2e);
      part[k] += v[k][e];
    }
  }
  const float total = fold_groups<WPR, VPL>(part, wr, groups, red[rloc]);
  if (!active) return;
  const float inv = masked ? 0.0f : static_cast<float>(1.0 / static_cast<double>(total));
#pragma unroll
  for (int k = 0; k < VPL; ++k) {
    const int c = (wr + WPR * k) * kWave + lane;
    if (c < nvec) {
      float y[VW];
#pragma unroll
      for (int e = 0; e < VW; ++e) y[e] = v[k][e] * inv;
      Chunk<float, VW> o;
      o.narrow(y);
      o.store(x + off + static_cast<int64_t>(c) * VW);
    }
  }
}

template <bool kMask>
__global__ __launch_bounds__(kBlock) void softmax_rows_wide(float* x, int64_t cols, RowMask rm) {
  __shared__ float red[kWavesPerBlock];
  float* row = x + (kMask ? rm.data_row(blockIdx.x) : static_cast<int64_t>(blockIdx.x)) * cols;
  if constexpr (kMask) {
    // Scale and mask in place first (this workgroup owns the row).
    const float* mrow = rm.mask != nullptr ? rm.mask + rm.mask_row(blockIdx.x) * cols : nullptr;
    for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
      const float mv = mrow != nullptr ? mrow[i] : 0.0f;
      {
#pragma clang fp contract(off)
        row[i] = row[i] * rm.scale + mv;
      }
    }
    __syncthreads();
  }
  float m = -INFINITY;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) m = fmaxf(m, row[i]);
  const float peak = block_max(m, red);
  const bool masked = peak == -INFINITY;
  float sum = 0.0f;
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    sum += masked ? 0.0f : __builtin_amdgcn_exp2f((row[i] - peak) * kLog2e);
  }
  const float total = block_sum(sum, red);
  const float inv = masked ? 0.0f : static_cast<float>(1.0 / static_cast<double>(total));
  for (int64_t i = threadIdx.x; i < cols; i += kBlock) {
    row[i] = masked ? 0.0f : __builtin_amdgcn_exp2f((row[i] - peak) * kLog2e) * inv;
  }
}

template <int VW, int WPR, bool kMask>
void launch_softmax_rows(int vpl, hipStream_t s, float* x, int64_t rows, int cols, const RowMask& rm) {
  constexpr int kThreads = softmax_block<WPR>();
  constexpr int kRowsPerBlock = kThreads / kWave / WPR;
  const unsigned blocks = static_cast<unsigned>((rows + kRowsPerBlock - 1) / kRowsPerBlock);
  switch (vpl) {
    case 1: softmax_rows_k<VW, WPR, 1, kMask><<<blocks, kThreads, 0, s>>>(x, rows, cols, rm); break;
    case 2: softmax_rows_k<VW, WPR, 2, kMask><<<blocks, kThreads, 0, s>>>(x, rows, cols, rm); break;
    case 4: softmax_rows_k<VW, WPR, 4, kMask><<<blocks, kThreads, 0, s>>>(x, rows, cols, rm); break;
    case 8: softmax_rows_k<VW, WPR, 8, kMask><<<blocks, kThreads, 0, s>>>(x, rows, cols, rm); break;
    default: softmax_rows_k<VW, WPR, 16, kMask><<<blocks, kThreads, 0, s>>>(x, rows, cols, rm); break;
  }
}

template <int VW, bool kMask>
void launch_softmax_wpr(int64_t groups, hipStream_t s, float* x, int64_t rows, int cols, const RowMask& rm) {
  if (groups < 4) {
    launch_softmax_rows<VW, 1, kMask>(vpl_bucket(groups), s, x, rows, cols, rm);
  } else if (groups < 8) {
    launch_softmax_rows<VW, 2, kMask>(vpl_bucket((groups + 1) / 2), s, x, rows, cols, rm);
  } else if (groups < 16) {
    launch_softmax_rows<VW, 4, kMask>(vpl_bucket((groups + 3) / 4), s, x, rows, cols, rm);
  } else {
    launch_softmax_rows<VW, 8, kMask>(vpl_bucket((groups + 7) / 8), s, x, rows, cols, rm);
  }
}

// Row softmax, optionally scaled and masked first; x [rows, cols], the mask
// repeating every rm.mask_rows rows.
template <bool kMask>
int softmax_entry(const char* what, void* stream, float* x, int64_t rows, int64_t cols, const RowMask& rm) {
  const bool vec = cols % 4 == 0 && aligned16(x) && (!kMask || rm.mask == nullptr || aligned16(rm.mask));
  const int64_t nvec = vec ? cols / 4 : cols;
  const int64_t groups = (nvec + kWave - 1) / kWave;
  const hipStream_t s = as_stream(stream);
  const int c32 = static_cast<int>(cols);
  clear_launch_error();
  // Pieces of about kPieceRows rows (one piece below a million rows): whole
  // mask rows (all batch slices of each) when masked, else plain row ranges.
  const int64_t unit = kMask ? rm.batch : 1;
  const int64_t piece = kPieceRows / unit > 0 ? kPieceRows / unit : 1;
  for_each_piece(rows / unit, piece, [&](int64_t u0, int64_t un) {
    RowMask p = rm;
    float* xp = x;
    if constexpr (kMask) {
      p.first = u0;
    } else {
      xp = x + u0 * cols;
    }
    const int64_t rn = un * unit;
    if (groups > kMaxGroups) {
      softmax_rows_wide<kMask><<<static_cast<unsigned>(rn), kBlock, 0, s>>>(xp, cols, p);
    } else if (vec) {
      launch_softmax_wpr<4, kMask>(groups, s, xp, rn, c32, p);
    } else {
      launch_softmax_wpr<1, kMask>(groups, s, xp, rn, c32, p);
    }
  });
  return check_launch(what);
}

// ---- scale and mask -------------------------------------------------------------

// One thread per mask chunk and group of SB slices: the mask chunk is read
// once into registers, then the SB slices' chunks are loaded together,
// scaled, masked and stored. blockIdx.x = group * blocks_per_slice + block.
// (An XCD-aware, chunk-major order measured no faster: the Infinity Cache
// already serves the other groups' re-reads of a mask chunk.)
template <int VW, int SB>
__global__ __launch_bounds__(kBlock) void scale_mask_k(float* __restrict__ x, float scale,
                                                        const float* __restrict__ mask, uint32_t per_chunks,
                                                        uint32_t batch, uint32_t blocks_per_slice) {
  const uint32_t group = blockIdx.x / blocks_per_slice;
  const uint32_t c = (blockIdx.x - group * blocks_per_slice) * kBlock + threadIdx.x;
  if (c >= per_chunks) return;
  const uint32_t b0 = group * SB;
  float m[VW];
  if (mask != nullptr) {
    load_f32<VW>(mask + static_cast<uint64_t>(c) * VW, m);
  } else {
#pragma unroll
    for (int e = 0; e < VW; ++e) m[e] = 0.0f;
  }
  Chunk<float, VW> cx[SB];
#pragma unroll
  for (int s = 0; s < SB; ++s) {
    if (b0 + s < batch) cx[s].load(x + (static_cast<uint64_t>(b0 + s) * per_chunks + c) * VW);
  }
#pragma unroll
  for (int s = 0; s < SB; ++s) {
    if (b0 + s < batch) {
      float v[VW];
      cx[s].widen(v);
      {
#pragma clang fp contract(off)
#pragma unroll
        for (int e = 0; e < VW; ++e) v[e] = v[e] * scale + m[e];
      }
      cx[s].narrow(v);
      cx[s].store(x + (static_cast<uint64_t>(b0 + s) * per_chunks + c) * VW);
    }
  }
}

template <int VW>
void launch_scale_mask(hipStream_t s, float* x, float scale, const float* mask, uint32_t per_chunks,
                       uint32_t batch) {
  const uint32_t bps = (per_chunks + kBlock - 1) / kBlock;
  auto grid = [&](uint32_t sb) { return static_cast<unsigned>(bps * ((batch + sb - 1) / sb)); };
  // Four slices per thread: measured on [10 x 4096, 4096] fp32 scores, 2 or
  // 4 slices run 10% faster than 1 (a mask read per slice) or 16 (fewer
  // waves, each holding 16 chunks), and 4 reads the mask a third as often.
  if (batch <= 1) scale_mask_k<VW, 1><<<grid(1), kBlock, 0, s>>>(x, scale, mask, per_chunks, batch, bps);
  else if (batch <= 2) scale_mask_k<VW, 2><<<grid(2), kBlock, 0, s>>>(x, scale, mask, per_chunks, batch, bps);
  else scale_mask_k<VW, 4><<<grid(4), kBlock, 0, s>>>(x, scale, mask, per_chunks, batch, bps);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_softmax_rows(void* stream, float* x, int64_t rows, int64_t cols) {
  const char* what = "uocr_rocm_softmax_rows";
  UOCR_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), what, "rows must be in [0, 2^31)");
  UOCR_REQUIRE(rows == 0 || (cols > 0 && cols < (int64_t{1} << 31)), what, "cols must be in [1, 2^31)");
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr, what, "null x");
  return softmax_entry<false>(what, stream, x, rows, cols, RowMask{nullptr, 1.0f, 1, 1, 0});
}

int uocr_rocm_scale_mask_softmax_rows(void* stream, float* x, float scale, const float* mask, int64_t batch,
                                      int64_t rows, int64_t cols) {
  const char* what = "uocr_rocm_scale_mask_softmax_rows";
  UOCR_REQUIRE(batch >= 0 && rows >= 0, what, "batch and rows must be >= 0");
  UOCR_REQUIRE(batch == 0 || rows < (int64_t{1} << 31) / batch, what, "batch * rows must be below 2^31");
  const int64_t all = batch * rows;
  UOCR_REQUIRE(all == 0 || (cols > 0 && cols < (int64_t{1} << 31)), what, "cols must be in [1, 2^31)");
  if (all == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr, what, "null x");
  return softmax_entry<true>(what, stream, x, all, cols, RowMask{mask, scale, rows, batch, 0});
}

int uocr_rocm_scale_add_mask(void* stream, float* x, float scale, const float* mask, int64_t batch, int64_t rows,
                             int64_t cols) {
  const char* what = "uocr_rocm_scale_add_mask";
  UOCR_REQUIRE(batch >= 0 && rows >= 0 && cols >= 0, what, "shape must be >= 0");
  const int64_t per = rows * cols;
  const int64_t total = batch * per;
  if (total == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(x != nullptr, what, "null x");
  UOCR_REQUIRE(total < (int64_t{1} << 32) - kBlock, what, "batch * rows * cols too large");
  // 16-byte chunks when no chunk straddles two slices.
  const bool vec = per % 4 == 0 && aligned16(x) && (mask == nullptr || aligned16(mask));
  const hipStream_t s = as_stream(stream);
  clear_launch_error();
  if (vec) {
    launch_scale_mask<4>(s, x, scale, mask, static_cast<uint32_t>(per / 4), static_cast<uint32_t>(batch));
  } else {
    launch_scale_mask<1>(s, x, scale, mask, static_cast<uint32_t>(per), static_cast<uint32_t>(batch));
  }
  return check_launch(what);
}

}  // extern "C"
