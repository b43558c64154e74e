// gather.hip: token-embedding gather from a bf16 table [table_rows, cols] for
// gfx950, by a device index array, a host index, or the decode step's
// StepState::token. The output is fp32 (bf16 -> fp32 is a 16-bit shift, so
// the result is bit-exact) or bf16 (a bit copy).
//
// Layout: one wave64 per output row; the lanes move the row in 128-bit
// chunks (8 bf16), up to 4 chunks per lane loaded before any is stored.
// Reference: Decoder::embed (src/model/decoder.cpp:85-92) and
// gather_bf16_kernel / gather_one_bf16_kernel / embed_kernel
// (src/backend/cuda/ops.cu:177-181,589-592, decode_ops.cu:26-29).

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int kGatherIters = 4;

// One chunk of VW table elements, widened or copied into the output type.
template <class TO, int VW>
struct OutChunk;

template <int VW>
struct OutChunk<uint16_t, VW> {
  static __device__ __forceinline__ void put(uint16_t* dst, const Chunk<uint16_t, VW>& c) { c.store(dst); }
};

template <>
struct OutChunk<float, 8> {
  static __device__ __forceinline__ void put(float* dst, const Chunk<uint16_t, 8>& c) {
    // The pair (lo, hi) of each 32-bit word widens to two fp32 words.
    const u32x4 a{c.raw.x << 16, c.raw.x & 0xffff0000u, c.raw.y << 16, c.raw.y & 0xffff0000u};
    const u32x4 b{c.raw.z << 16, c.raw.z & 0xffff0000u, c.raw.w << 16, c.raw.w & 0xffff0000u};
    *reinterpret_cast<u32x4*>(dst) = a;
    *reinterpret_cast<u32x4*>(dst + 4) = b;
  }
};

template <>
struct OutChunk<float, 1> {
  static __device__ __forceinline__ void put(float* dst, const Chunk<uint16_t, 1>& c) {
    *dst = __uint_as_float(static_cast<uint32_t>(c.raw) << 16);
  }
};

// Index source: state->token when state is set, else index[row] when index
// is set, else one_index. With table_rows >= 0 an index outside
// [0, table_rows) produces a zero row and the table is not read.
template <class TO, int VW>
__global__ __launch_bounds__(kBlock) void gather_rows_kernel(const uint16_t* __restrict__ table, int64_t table_rows,
                                                             const int64_t* __restrict__ index, int64_t one_index,
                                                             const uocr_rocm_step_state* __restrict__ state,
                                                             int64_t rows, int cols, TO* __restrict__ dst) {
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row = static_cast<int64_t>(blockIdx.x) * kWavesPerBlock + threadIdx.x / kWave;
  if (row >= rows) return;
  const int64_t id = state != nullptr ? state->token : (index != nullptr ? index[row] : one_index);
  const bool valid = table_rows < 0 || (id >= 0 && id < table_rows);
  const uint16_t* src = table + (valid ? id : 0) * static_cast<int64_t>(cols);
  TO* out = dst + row * cols;
  const int nvec = cols / VW;
  for (int base = 0; base < nvec; base += kWave * kGatherIters) {
    Chunk<uint16_t, VW> c[kGatherIters];
#pragma unroll
    for (int it = 0; it < kGatherIters; ++it) {
      const int v = base + lane + it * kWave;
      c[it].clear();
      if (valid && v < nvec) c[it].load(src + v * VW);
    }
#pragma unroll
    for (int it = 0; it < kGatherIters; ++it) {
      const int v = base + lane + it * kWave;
      if (v < nvec) OutChunk<TO, VW>::put(out + v * VW, c[it]);
    }
  }
}

template <class TO>
int launch_gather(const char* what, void* stream, const uint16_t* table, int64_t table_rows, const int64_t* index,
                  int64_t one_index, const uocr_rocm_step_state* state, int64_t rows, int64_t cols, TO* dst) {
  UOCR_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), what, "rows must be in [0, 2^31)");
  UOCR_REQUIRE(rows == 0 || (cols > 0 && cols < (int64_t{1} << 30)), what, "cols must be in [1, 2^30)");
  if (rows == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(table != nullptr && dst != nullptr, what, "null table or dst");
  UOCR_REQUIRE(table_rows < 0 || state != nullptr || index != nullptr ||
                   (one_index >= 0 && one_index < table_rows),
               what, "index outside the table");
  const bool vec = cols % 8 == 0 && aligned16(table) && aligned16(dst);
  const hipStream_t s = as_stream(stream);
  const int c32 = static_cast<int>(cols);
  clear_launch_error();
  // Row pieces of kPieceRows (one piece below a million rows).
  for_each_piece(rows, kPieceRows, [&](int64_t r0, int64_t rn) {
    const unsigned blocks = blocks_for_rows(rn);
    const int64_t* ip = index != nullptr ? index + r0 : nullptr;
    TO* dp = dst + r0 * cols;
    if (vec) {
      gather_rows_kernel<TO, 8><<<blocks, kBlock, 0, s>>>(table, table_rows, ip, one_index, state, rn, c32, dp);
    } else {
      gather_rows_kernel<TO, 1><<<blocks, kBlock, 0, s>>>(table, table_rows, ip, one_index, state, rn, c32, dp);
    }
  });
  return check_launch(what);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_gather_rows_bf16(void* stream, const uint16_t* table, int64_t table_rows, const int64_t* index,
                               int64_t rows, int64_t cols, float* dst) {
  UOCR_REQUIRE(rows == 0 || index != nullptr, "uocr_rocm_gather_rows_bf16", "null index");
  return launch_gather<float>("uocr_rocm_gather_rows_bf16", stream, table, table_rows, index, 0, nullptr, rows, cols,
                              dst);
}

int uocr_rocm_gather_rows_bf16_bf16(void* stream, const uint16_t* table, int64_t table_rows, const int64_t* index,
                                    int64_t rows, int64_t cols, uint16_t* dst) {
  UOCR_REQUIRE(rows == 0 || index != nullptr, "uocr_rocm_gather_rows_bf16_bf16", "null index");
  return launch_gather<uint16_t>("uocr_rocm_gather_rows_bf16_bf16", stream, table, table_rows, index, 0, nullptr,
                                 rows, cols, dst);
}

int uocr_rocm_gather_row_bf16(void* stream, const uint16_t* table, int64_t table_rows, int64_t one_index,
                              int64_t cols, float* dst) {
  return launch_gather<float>("uocr_rocm_gather_row_bf16", stream, table, table_rows, nullptr, one_index, nullptr, 1,
                              cols, dst);
}

int uocr_rocm_embed_step(void* stream, const uint16_t* table, int64_t table_rows, const uocr_rocm_step_state* state,
                         int64_t cols, float* dst) {
  UOCR_REQUIRE(state != nullptr, "uocr_rocm_embed_step", "null state");
  return launch_gather<float>("uocr_rocm_embed_step", stream, table, table_rows, nullptr, 0, state, 1, cols, dst);
}

int uocr_rocm_embed_step_bf16(void* stream, const uint16_t* table, int64_t table_rows,
                              const uocr_rocm_step_state* state, int64_t cols, uint16_t* dst) {
  UOCR_REQUIRE(state != nullptr, "uocr_rocm_embed_step_bf16", "null state");
  return launch_gather<uint16_t>("uocr_rocm_embed_step_bf16", stream, table, table_rows, nullptr, 0, state, 1, cols,
                                 dst);
}

}  // extern "C"
