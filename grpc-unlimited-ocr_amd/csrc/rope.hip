// rope.hip: rotate-half rotary position embedding, in place, for gfx950;
// fp32 and bf16 activations, fp32 arithmetic.
//
// Layout: X0 [rows, heads0 * dim] and X1 [rows, heads1 * dim] row-major (Q
// and K of one attention layer; X1 may be absent). One wave64 owns one row
// (token), or two rows when the batch is long:
//   1. The lanes compute each row's dim/2 (cos, sin) pairs, one sincosf per
//      pair per row rather than per (row, head), into the wave's slice of
//      LDS.
//   2. The row's (heads0 + heads1) * dim / (2 VW) chunk pairs are spread
//      over the lanes: chunk pair (head h, j) is elements [j VW, (j+1) VW) of
//      the first half of head h and the same span of its second half. A lane
//      loads both 128-bit chunks, reads its VW cos/sin values from LDS,
//      rotates, and stores both chunks back, so Q/K make one HBM round trip.
//      Up to ITERS chunk pairs per lane are loaded before any is rotated, and
//      the first ITERS are in flight while step 1 runs.
//
// Arithmetic (reference: src/model/page_rope.cpp:26-56 and the
// uocr::cuda::rope coordinate rule, src/backend/cuda/ops.cu:134-151):
//   angle = float(tok) * inv_tok[p]              for p <  n_tok
//   angle = float(page mod page_mod) * inv_page[p - n_tok]   otherwise
//   c, s = cos(angle), sin(angle) in fp32 (device sincosf)
//   v[p] = a c - b s,  v[p + half] = b c + a s     (no FMA contraction)

#include "common.hpp"

namespace uocr_rocm {
namespace {

constexpr int kMaxHalf = 256;  // dim <= 512
// Two waves per workgroup: at Q/K [8192, 16+4, 128] bf16 this measured 1.5%
// faster than four waves (and than one or eight).
constexpr int kRopeBlock = 128;
constexpr int kRopeWaves = kRopeBlock / kWave;

template <class T>
struct RopeArgs {
  T* x0;
  T* x1;
  int heads0;
  int heads1;
  int64_t rows;
  int dim;
  int half;
  const int64_t* tok;
  const int64_t* page;
  const float* inv_tok;
  int n_tok;
  const float* inv_page;
  int64_t page_mod;
  int64_t one_tok;
  int64_t one_page;
  const uocr_rocm_step_state* state;
  int cpp_shift;  // log2(chunk pairs per head) when that is a power of two
};

// Chunk pair c of a row -> (head h, chunk j): a shift and a mask when the
// chunk pairs per head are a power of two (kPow2), else a division.
template <bool kPow2>
__device__ __forceinline__ void split_chunk(int c, int cpp, int shift, int& h, int& j) {
  if constexpr (kPow2) {
    h = c >> shift;
    j = c & (cpp - 1);
  } else {
    h = c / cpp;
    j = c - h * cpp;
  }
}

// Loads chunk pairs base + lane + 64 it (it < ITERS) of the wave's TPW rows
// (row0, row0 + 1, ...; pair c belongs to row row0 + c / total); a pair past
// the end gets at[it] = nullptr.
template <class T, int VW, int ITERS, bool kPow2, int TPW>
__device__ __forceinline__ void load_pairs(const RopeArgs<T> a, int64_t row0, int lane, int base, int total,
                                           int cpp, Chunk<T, VW> (&lo)[ITERS], Chunk<T, VW> (&hi)[ITERS],
                                           T* (&at)[ITERS], int (&jj)[ITERS], int (&tt)[ITERS]) {
#pragma unroll
  for (int it = 0; it < ITERS; ++it) {
    int c = base + lane + it * kWave;
    const int t = TPW == 1 ? 0 : (c >= total ? 1 : 0);
    c -= t * total;
    const int64_t row = row0 + t;
    at[it] = nullptr;
    jj[it] = 0;
    tt[it] = t;
    if (row < a.rows && c < total) {
      int h, j;
      split_chunk<kPow2>(c, cpp, a.cpp_shift, h, j);
      T* head = h < a.heads0 ? a.x0 + (row * a.heads0 + h) * a.dim : a.x1 + (row * a.heads1 + (h - a.heads0)) * a.dim;
      at[it] = head + j * VW;
      jj[it] = j;
      lo[it].load(at[it]);
      hi[it].load(at[it] + a.half);
    }
  }
}

// TPW rows (tokens) per wave: 2 for long prefill batches, so each lane
// keeps more 128-bit loads in flight; 1 otherwise. The LDS table holds the
// wave's TPW rows of cos/sin, sized at launch (kRopeWaves * TPW * 2 * half
// floats).
template <class T, int VW, int ITERS, bool kPow2, int TPW>
__global__ __launch_bounds__(kRopeBlock) void rope_rows(RopeArgs<T> a) {
  extern __shared__ __attribute__((aligned(16))) float table[];
  const int wave = wave_in_block();
  const int lane = threadIdx.x & (kWave - 1);
  const int64_t row0 = (static_cast<int64_t>(blockIdx.x) * kRopeWaves + wave) * TPW;
  const bool active = row0 < a.rows;
  const int cpp = a.half / VW;  // chunk pairs per head
  const int total = (a.heads0 + a.heads1) * cpp;  // chunk pairs per row
  float* wave_table = table + wave * TPW * 2 * a.half;

  // The first batch of Q/K loads goes out before anything else: the rows'
  // coordinates and frequencies are read after it, so no wave spends a
  // dependent round trip on its positions before its first data request
  // (reading them first cost RoPE on Q/K [8192, 16+4, 128] 5%).
  Chunk<T, VW> lo[ITERS], hi[ITERS];
  T* at[ITERS];
  int jj[ITERS], tt[ITERS];
  load_pairs<T, VW, ITERS, kPow2, TPW>(a, row0, lane, 0, total, cpp, lo, hi, at, jj, tt);

#pragma unroll
  for (int t = 0; t < TPW; ++t) {
    const int64_t row = row0 + t;
    if (row < a.rows) {
      int64_t tk, pg;
      if (a.state != nullptr) {
        tk = a.state->tok;
        pg = a.state->page;
      } else {
        tk = a.tok != nullptr ? a.tok[row] : a.one_tok;
        pg = a.page != nullptr ? a.page[row] : a.one_page;
      }
      if (a.page_mod > 0) pg = ((pg % a.page_mod) + a.page_mod) % a.page_mod;
      const float ft = static_cast<float>(tk), fp = static_cast<float>(pg);
      float* cosv = wave_table + t * 2 * a.half;
      float* sinv = cosv + a.half;
      for (int p = lane; p < a.half; p += kWave) {
        const float angle = p < a.n_tok ? ft * a.inv_tok[p] : fp * a.inv_page[p - a.n_tok];
        float sn, cs;
        sincosf(angle, &sn, &cs);
        cosv[p] = cs;
        sinv[p] = sn;
      }
    }
  }
  __syncthreads();
  if (!active) return;

  for (int base = 0; base < TPW * total; base += kWave * ITERS) {
    if (base > 0) load_pairs<T, VW, ITERS, kPow2, TPW>(a, row0, lane, base, total, cpp, lo, hi, at, jj, tt);
#pragma unroll
    for (int it = 0; it < ITERS; ++it) {
      if (at[it] != nullptr) {
        const float* cosv = wave_table + tt[it] * 2 * a.half;
        const float* sinv = cosv + a.half;
        float va[VW], vb[VW], cs[VW], sn[VW];
        lo[it].widen(va);
        hi[it].widen(vb);
        load_f32<VW>(cosv + jj[it] * VW, cs);
        load_f32<VW>(sinv + jj[it] * VW, sn);
        float ra[VW], rb[VW];
        {
#pragma clang fp contract(off)
#pragma unroll
          for (int e = 0; e < VW; ++e) {
            ra[e] = va[e] * cs[e] - vb[e] * sn[e];
            rb[e] = vb[e] * cs[e] + va[e] * sn[e];
          }
        }
        lo[it].narrow(ra);
        hi[it].narrow(rb);
        lo[it].store(at[it]);
        hi[it].store(at[it] + a.half);
      }
    }
  }
}

template <class T, int VW, bool kPow2, int TPW>
void launch_rope_iters(const RopeArgs<T>& a, int iters, hipStream_t s) {
  const int64_t waves = (a.rows + TPW - 1) / TPW;
  const unsigned blocks = static_cast<unsigned>((waves + kRopeWaves - 1) / kRopeWaves);
  const size_t lds = static_cast<size_t>(kRopeWaves) * TPW * 2 * a.half * sizeof(float);
  switch (iters) {
    case 1: rope_rows<T, VW, 1, kPow2, TPW><<<blocks, kRopeBlock, lds, s>>>(a); break;
    case 2: rope_rows<T, VW, 2, kPow2, TPW><<<blocks, kRopeBlock, lds, s>>>(a); break;
    case 3: rope_rows<T, VW, 3, kPow2, TPW><<<blocks, kRopeBlock, lds, s>>>(a); break;
    case 4: rope_rows<T, VW, 4, kPow2, TPW><<<blocks, kRopeBlock, lds, s>>>(a); break;
    case 5: rope_rows<T, VW, 5, kPow2, TPW><<<blocks, kRopeBlock, lds, s>>>(a); break;
    default: rope_rows<T, VW, 6, kPow2, TPW><<<blocks, kRopeBlock, lds, s>>>(a); break;
  }
}

// Two rows per wave once there are enough rows to fill the GPU with half as
// many waves, and when the two rows' chunk pairs fit in 6 loads per lane.
constexpr int64_t kPairRows = 2048;

template <class T, int VW>
void launch_rope_vw(RopeArgs<T>& a, hipStream_t s) {
  const int cpp = a.half / VW;
  const int total = (a.heads0 + a.heads1) * cpp;
  const bool pow2 = (cpp & (cpp - 1)) == 0;
  a.cpp_shift = pow2 ? __builtin_ctz(static_cast<unsigned>(cpp)) : -1;
  const bool pair = a.rows >= kPairRows && 2 * total <= 6 * kWave;
  const int per_wave = pair ? 2 * total : total;
  int iters = (per_wave + kWave - 1) / kWave;
  if (iters > 6) iters = 6;
  if (pair) {
    if (pow2) launch_rope_iters<T, VW, true, 2>(a, iters, s);
    else launch_rope_iters<T, VW, false, 2>(a, iters, s);
  } else {
    if (pow2) launch_rope_iters<T, VW, true, 1>(a, iters, s);
    else launch_rope_iters<T, VW, false, 1>(a, iters, s);
  }
}

template <class T>
int launch_rope(const char* what, void* stream, T* x0, int64_t heads0, T* x1, int64_t heads1, int64_t rows,
                int64_t dim, const int64_t* tok, const int64_t* page, const float* inv_tok, int64_t n_tok,
                const float* inv_page, int64_t n_page, int64_t page_mod, int64_t one_tok, int64_t one_page,
                const uocr_rocm_step_state* state) {
  UOCR_REQUIRE(rows >= 0 && rows < (int64_t{1} << 31), what, "rows must be in [0, 2^31)");
  UOCR_REQUIRE(heads0 >= 0 && heads1 >= 0, what, "heads must be >= 0");
  UOCR_REQUIRE(dim > 0 && dim % 2 == 0 && dim / 2 <= kMaxHalf, what, "dim must be even and in [2, 512]");
  UOCR_REQUIRE(n_tok >= 0 && n_page >= 0 && n_tok + n_page == dim / 2, what, "n_tok + n_page must equal dim / 2");
  UOCR_REQUIRE((heads0 + heads1) * (dim / 2) < (int64_t{1} << 30), what, "heads * dim too large");
  if (rows == 0 || heads0 + heads1 == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(heads0 == 0 || x0 != nullptr, what, "null x");
  UOCR_REQUIRE(heads1 == 0 || x1 != nullptr, what, "null k");
  UOCR_REQUIRE(n_tok == 0 || inv_tok != nullptr, what, "null inv_tok");
  UOCR_REQUIRE(n_page == 0 || inv_page != nullptr, what, "null inv_page");
  UOCR_REQUIRE(heads0 == 0 || heads1 == 0 || x0 != x1, what, "q and k must be distinct buffers");

  RopeArgs<T> a{};
  a.x0 = heads0 > 0 ? x0 : x1;
  a.heads0 = static_cast<int>(heads0 > 0 ? heads0 : heads1);
  a.x1 = heads0 > 0 ? x1 : nullptr;
  a.heads1 = static_cast<int>(heads0 > 0 ? heads1 : 0);
  a.rows = rows;
  a.dim = static_cast<int>(dim);
  a.half = static_cast<int>(dim / 2);
  a.tok = tok;
  a.page = page;
  a.inv_tok = inv_tok;
  a.n_tok = static_cast<int>(n_tok);
  a.inv_page = inv_page;
  a.page_mod = page_mod;
  a.one_tok = one_tok;
  a.one_page = one_page;
  a.state = state;

  constexpr int kV = kVec<T>;
  // 16-byte chunks need every head half to start on a 16-byte boundary.
  const bool vec = a.half % kV == 0 && aligned16(a.x0) && (a.x1 == nullptr || aligned16(a.x1));
  clear_launch_error();
  // Row pieces of kPieceRows tokens (one piece below a million tokens).
  for_each_piece(rows, kPieceRows, [&](int64_t r0, int64_t rn) {
    RopeArgs<T> p = a;
    p.rows = rn;
    p.x0 = a.x0 + r0 * a.heads0 * dim;
    p.x1 = a.x1 != nullptr ? a.x1 + r0 * a.heads1 * dim : nullptr;
    p.tok = a.tok != nullptr ? a.tok + r0 : nullptr;
    p.page = a.page != nullptr ? a.page + r0 : nullptr;
    if (vec) {
      launch_rope_vw<T, kV>(p, as_stream(stream));
    } else {
      launch_rope_vw<T, 1>(p, as_stream(stream));
    }
  });
  return check_launch(what);
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_rope(void* stream, float* x, int64_t rows, int64_t heads, int64_t dim, const int64_t* tok,
                   const int64_t* page, const float* inv_tok, int64_t n_tok, const float* inv_page, int64_t n_page,
                   int64_t page_mod, int64_t one_tok, int64_t one_page) {
  return launch_rope<float>("uocr_rocm_rope", stream, x, heads, nullptr, 0, rows, dim, tok, page, inv_tok, n_tok,
                            inv_page, n_page, page_mod, one_tok, one_page, nullptr);
}

int uocr_rocm_rope_bf16(void* stream, uint16_t* x, int64_t rows, int64_t heads, int64_t dim, const int64_t* tok,
                        const int64_t* page, const float* inv_tok, int64_t n_tok, const float* inv_page,
                        int64_t n_page, int64_t page_mod, int64_t one_tok, int64_t one_page) {
  return launch_rope<uint16_t>("uocr_rocm_rope_bf16", stream, x, heads, nullptr, 0, rows, dim, tok, page, inv_tok,
                               n_tok, inv_page, n_page, page_mod, one_tok, one_page, nullptr);
}

int uocr_rocm_rope_qk(void* stream, float* q, int64_t q_heads, float* k, int64_t k_heads, int64_t rows, int64_t dim,
                      const int64_t* tok, const int64_t* page, const float* inv_tok, int64_t n_tok,
                      const float* inv_page, int64_t n_page, int64_t page_mod, int64_t one_tok, int64_t one_page) {
  return launch_rope<float>("uocr_rocm_rope_qk", stream, q, q_heads, k, k_heads, rows, dim, tok, page, inv_tok, n_tok,
                            inv_page, n_page, page_mod, one_tok, one_page, nullptr);
}

int uocr_rocm_rope_qk_bf16(void* stream, uint16_t* q, int64_t q_heads, uint16_t* k, int64_t k_heads, int64_t rows,
                           int64_t dim, const int64_t* tok, const int64_t* page, const float* inv_tok, int64_t n_tok,
                           const float* inv_page, int64_t n_page, int64_t page_mod, int64_t one_tok,
                           int64_t one_page) {
  return launch_rope<uint16_t>("uocr_rocm_rope_qk_bf16", stream, q, q_heads, k, k_heads, rows, dim, tok, page,
                               inv_tok, n_tok, inv_page, n_page, page_mod, one_tok, one_page, nullptr);
}

int uocr_rocm_rope_step(void* stream, float* x, int64_t heads, int64_t dim, const uocr_rocm_step_state* state,
                        const float* inv_tok, int64_t n_tok, const float* inv_page, int64_t page_mod) {
  UOCR_REQUIRE(state != nullptr, "uocr_rocm_rope_step", "null state");
  return launch_rope<float>("uocr_rocm_rope_step", stream, x, heads, nullptr, 0, 1, dim, nullptr, nullptr, inv_tok,
                            n_tok, inv_page, dim / 2 - n_tok, page_mod, 0, 0, state);
}

int uocr_rocm_rope_qk_step(void* stream, float* q, int64_t q_heads, float* k, int64_t k_heads, int64_t dim,
                           const uocr_rocm_step_state* state, const float* inv_tok, int64_t n_tok,
                           const float* inv_page, int64_t page_mod) {
  UOCR_REQUIRE(state != nullptr, "uocr_rocm_rope_qk_step", "null state");
  return launch_rope<float>("uocr_rocm_rope_qk_step", stream, q, q_heads, k, k_heads, 1, dim, nullptr, nullptr,
                            inv_tok, n_tok, inv_page, dim / 2 - n_tok, page_mod, 0, 0, state);
}

int uocr_rocm_rope_qk_step_bf16(void* stream, uint16_t* q, int64_t q_heads, uint16_t* k, int64_t k_heads,
                                int64_t dim, const uocr_rocm_step_state* state, const float* inv_tok, int64_t n_tok,
                                const float* inv_page, int64_t page_mod) {
  UOCR_REQUIRE(state != nullptr, "uocr_rocm_rope_qk_step_bf16", "null state");
  return launch_rope<uint16_t>("uocr_rocm_rope_qk_step_bf16", stream, q, q_heads, k, k_heads, 1, dim, nullptr,
                               nullptr, inv_tok, n_tok, inv_page, dim / 2 - n_tok, page_mod, 0, 0, state);
}

}  // extern "C"
