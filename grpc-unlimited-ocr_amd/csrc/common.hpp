// common.hpp: device helpers shared by the gfx950 kernels (bf16 rounding,
// 128-bit row chunks, wave64 DPP reductions) and the host-side status
// plumbing of the C ABI.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <string>

#include "uocr_rocm.h"

namespace uocr_rocm {

// ---- launch geometry ------------------------------------------------------

constexpr int kWave = 64;                        // CDNA wavefront width
constexpr int kBlock = 256;                      // 4 waves per workgroup
constexpr int kWavesPerBlock = kBlock / kWave;   // one row per wave

// The wave's index in its workgroup as a wave-uniform value (an SGPR): row
// and head base pointers formed from it stay scalar, so each lane's address
// is one 32-bit offset from a scalar base (global_load ... v_off, s[base])
// instead of a 64-bit vector address.
__device__ __forceinline__ int wave_in_block() {
  return __builtin_amdgcn_readfirstlane(static_cast<int>(threadIdx.x / kWave));
}

// ---- bf16 -----------------------------------------------------------------

// bf16 -> fp32 is exact: the 16 bits become the top half of a binary32.
__device__ __forceinline__ float bf16_lo(uint32_t pair) { return __uint_as_float(pair << 16); }
__device__ __forceinline__ float bf16_hi(uint32_t pair) { return __uint_as_float(pair & 0xffff0000u); }
__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// fp32 -> bf16 with gfx950's v_cvt_pk_bf16_f32, two values per instruction.
// On every one of the 2^32 fp32 bit patterns it gives the reference's
// rounding (src/tensor/dtype.h:39-46): nearest even, a NaN keeps its sign
// and top payload bits and gets the quiet bit, denormals are kept
// (tests/cpp/bf16_cvt_probe.hip checks all of them on the device).
typedef __bf16 bf16x2_t __attribute__((ext_vector_type(2)));
typedef float f32x2_t __attribute__((ext_vector_type(2)));

__device__ __forceinline__ uint32_t pack_bf16(float lo, float hi) {
  return __builtin_bit_cast(uint32_t, __builtin_convertvector(f32x2_t{lo, hi}, bf16x2_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return static_cast<uint16_t>(pack_bf16(f, 0.0f)); }

// ---- row chunks -------------------------------------------------------------
// A Chunk<T, VW> is VW consecutive elements of storage type T (float or
// bf16 bits in uint16_t). VW = 16 / sizeof(T) is one 128-bit global load or
// store (global_load_dwordx4); VW = 1 is the scalar path for rows whose width
// or base address does not allow 16-byte chunks. Activations are touched
// once per op, so chunks move with nontemporal loads and stores (the `nt`
// streaming hint), which keep them from displacing reused data in the
// caches; norm weights and rope tables use ordinary loads.

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <class V>
__device__ __forceinline__ V stream_load(const V* p) {
  return __builtin_nontemporal_load(p);
}
template <class V>
__device__ __forceinline__ void stream_store(V* p, V v) {
  __builtin_nontemporal_store(v, p);
}

template <class T, int VW>
struct Chunk;

template <>
struct Chunk<float, 4> {
  u32x4 raw;
  __device__ __forceinline__ void load(const float* p) { raw = stream_load(reinterpret_cast<const u32x4*>(p)); }
  __device__ __forceinline__ void store(float* p) const { stream_store(reinterpret_cast<u32x4*>(p), raw); }
  __device__ __forceinline__ void widen(float (&v)[4]) const {
    v[0] = __uint_as_float(raw.x);
    v[1] = __uint_as_float(raw.y);
    v[2] = __uint_as_float(raw.z);
    v[3] = __uint_as_float(raw.w);
  }
  __device__ __forceinline__ void narrow(const float (&v)[4]) {
    raw = u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])};
  }
  __device__ __forceinline__ void clear() { raw = u32x4{0u, 0u, 0u, 0u}; }
};

template <>
struct Chunk<uint16_t, 8> {
  u32x4 raw;
  __device__ __forceinline__ void load(const uint16_t* p) { raw = stream_load(reinterpret_cast<const u32x4*>(p)); }
  __device__ __forceinline__ void store(uint16_t* p) const { stream_store(reinterpret_cast<u32x4*>(p), raw); }
  __device__ __forceinline__ void widen(float (&v)[8]) const {
    v[0] = bf16_lo(raw.x);
    v[1] = bf16_hi(raw.x);
    v[2] = bf16_lo(raw.y);
    v[3] = bf16_hi(raw.y);
    v[4] = bf16_lo(raw.z);
    v[5] = bf16_hi(raw.z);
    v[6] = bf16_lo(raw.w);
    v[7] = bf16_hi(raw.w);
  }
  __device__ __forceinline__ void narrow(const float (&v)[8]) {
    raw = u32x4{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3]), pack_bf16(v[4], v[5]), pack_bf16(v[6], v[7])};
  }
  __device__ __forceinline__ void clear() { raw = u32x4{0u, 0u, 0u, 0u}; }
};

// A raw buffer resource over `bytes` bytes at `base` (gfx950 word 3: raw
// 32-bit dwords, no swizzle). Accesses through it take a 32-bit byte offset;
// the hardware drops a store past `bytes` and returns zero for such a load.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t buffer_rsrc(const void* base, uint32_t bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), 0, bytes, 0x00020000);
}

// Cache-policy bits of a buffer access on gfx950 (the instruction's sc0, nt
// and sc1 modifiers).
constexpr int kPolicySc0 = 1, kPolicyNt = 2, kPolicySc1 = 16;

// A 128-bit store through a buffer resource with policy bits `kPolicy`.
template <int kPolicy>
__device__ __forceinline__ void buffer_store16(__amdgpu_buffer_rsrc_t r, uint32_t offset, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, offset, 0, kPolicy);
}

// Four bf16 (8 bytes): an fp32 row chunk's worth of a bf16 table row.
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <>
struct Chunk<uint16_t, 4> {
  u32x2 raw;
  __device__ __forceinline__ void load(const uint16_t* p) { raw = stream_load(reinterpret_cast<const u32x2*>(p)); }
  __device__ __forceinline__ void store(uint16_t* p) const { stream_store(reinterpret_cast<u32x2*>(p), raw); }
  __device__ __forceinline__ void widen(float (&v)[4]) const {
    v[0] = bf16_lo(raw.x);
    v[1] = bf16_hi(raw.x);
    v[2] = bf16_lo(raw.y);
    v[3] = bf16_hi(raw.y);
  }
  __device__ __forceinline__ void narrow(const float (&v)[4]) { raw = u32x2{pack_bf16(v[0], v[1]), pack_bf16(v[2], v[3])}; }
  __device__ __forceinline__ void clear() { raw = u32x2{0u, 0u}; }
};

template <>
struct Chunk<float, 1> {
  float raw;
  __device__ __forceinline__ void load(const float* p) { raw = stream_load(p); }
  __device__ __forceinline__ void store(float* p) const { stream_store(p, raw); }
  __device__ __forceinline__ void widen(float (&v)[1]) const { v[0] = raw; }
  __device__ __forceinline__ void narrow(const float (&v)[1]) { raw = v[0]; }
  __device__ __forceinline__ void clear() { raw = 0.0f; }
};

template <>
struct Chunk<uint16_t, 1> {
  uint16_t raw;
  __device__ __forceinline__ void load(const uint16_t* p) { raw = stream_load(p); }
  __device__ __forceinline__ void store(uint16_t* p) const { stream_store(p, raw); }
  __device__ __forceinline__ void widen(float (&v)[1]) const { v[0] = bf16_to_f32(raw); }
  __device__ __forceinline__ void narrow(const float (&v)[1]) { raw = f32_to_bf16(v[0]); }
  __device__ __forceinline__ void clear() { raw = 0; }
};

// ---- row stores without a branch ---------------------------------------------
// A store through a buffer resource at an offset at or past the resource's
// size is dropped by the hardware. A row kernel therefore stores every chunk
// it holds unconditionally: kDropOffset for a chunk past the row's end, and a
// zero-size resource for a wave past the last row. A store inside a branch
// would make the compiler wait for every earlier store and load (vmcnt(0))
// before the next use of a loaded chunk, since it cannot tell whether the
// store was issued; unconditional stores keep those waits exact. Nontemporal
// policy, as Chunk::store.
constexpr uint32_t kDropOffset = 0x80000000u;

__device__ __forceinline__ void buffer_store_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x4 v) {
  __builtin_amdgcn_raw_buffer_store_b128(v, r, off, 0, kPolicyNt);
}
__device__ __forceinline__ void buffer_store_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, u32x2 v) {
  __builtin_amdgcn_raw_buffer_store_b64(v, r, off, 0, kPolicyNt);
}
__device__ __forceinline__ void buffer_store_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, float v) {
  __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), r, off, 0, kPolicyNt);
}
__device__ __forceinline__ void buffer_store_nt(__amdgpu_buffer_rsrc_t r, uint32_t off, uint16_t v) {
  __builtin_amdgcn_raw_buffer_store_b16(v, r, off, 0, kPolicyNt);
}

// Chunk c at byte offset `off` of the resource (kDropOffset: nothing stored).
template <class T, int VW>
__device__ __forceinline__ void store_chunk(__amdgpu_buffer_rsrc_t r, uint32_t off, const Chunk<T, VW>& c) {
  buffer_store_nt(r, off, c.raw);
}

// VW fp32 values (norm weights, cos/sin tables) in 128-bit pieces when VW is
// a multiple of 4; `p` must then be 16-byte aligned.
template <int VW>
__device__ __forceinline__ void load_f32(const float* p, float (&v)[VW]) {
  if constexpr (VW % 4 == 0) {
#pragma unroll
    for (int q = 0; q < VW / 4; ++q) {
      const u32x4 r = *reinterpret_cast<const u32x4*>(p + 4 * q);
      v[4 * q + 0] = __uint_as_float(r.x);
      v[4 * q + 1] = __uint_as_float(r.y);
      v[4 * q + 2] = __uint_as_float(r.z);
      v[4 * q + 3] = __uint_as_float(r.w);
    }
  } else {
#pragma unroll
    for (int e = 0; e < VW; ++e) v[e] = p[e];
  }
}

// Elements per 128-bit chunk for a storage type.
template <class T>
constexpr int kVec = 16 / static_cast<int>(sizeof(T));

// ---- activations shared by several kernels -----------------------------------

// silu(g) u = g sigmoid(g) u with sigmoid(g) = 1 / (1 + e^-g); e^-g is
// 2^(-g log2 e) on v_exp_f32 and the reciprocal is v_rcp_f32 (1 ulp each),
// as in the reference's ops.cpp:40,163-167 and feed_forward.cpp:21-22.
// g -> -inf gives 1 / inf = 0 and g * 0, as the reference does.
__device__ __forceinline__ float silu_mul_f(float g, float u) {
  const float e = __builtin_amdgcn_exp2f(g * -1.4426950408889634f);
  const float sig = __builtin_amdgcn_rcpf(1.0f + e);
  return (g * sig) * u;
}

// ---- wave64 reductions ------------------------------------------------------
// A butterfly over DPP lane permutations inside each 16-lane row, then the
// four row totals read through readlane (SGPRs). Every lane of the wave must
// be active. The result is wave-uniform and has the same bits in every lane;
// its summation order is fixed, so a row's result never depends on which
// wave or launch computed it.

template <int kCtrl>
__device__ __forceinline__ float dpp_f32(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), kCtrl, 0xF, 0xF, false));
}

// A workgroup barrier that orders LDS only: every wave's LDS accesses before
// it complete before any wave passes it, while global loads and stores stay
// in flight across it (__syncthreads waits for those as well). For a
// workgroup whose waves share data through LDS alone.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup", "local");
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup", "local");
}

__device__ __forceinline__ float wave_sum(float v) {
  v += dpp_f32<0xB1>(v);   // quad_perm [1,0,3,2]: partner lane ^ 1
  v += dpp_f32<0x4E>(v);   // quad_perm [2,3,0,1]: partner lane ^ 2
  v += dpp_f32<0x141>(v);  // row_half_mirror: the two quads of each 8 lanes
  v += dpp_f32<0x140>(v);  // row_mirror: the two halves of each 16-lane row
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max(float v) {
  v = fmaxf(v, dpp_f32<0xB1>(v));
  v = fmaxf(v, dpp_f32<0x4E>(v));
  v = fmaxf(v, dpp_f32<0x141>(v));
  v = fmaxf(v, dpp_f32<0x140>(v));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

// Row totals over 64-chunk groups held by WPR waves (wave wr holds groups
// wr, wr + WPR, ...; `part[k]` is this lane's partial for group wr + WPR k).
// Each group reduces with one wave butterfly; the group results fold left to
// right in group order (through the row's LDS slot `red`, kMaxGroups floats,
// when WPR > 1), so the result depends only on the row, never on WPR. kMax
// folds with max (an exact, order-free fold), else with +. Every wave of the
// block must call it the same number of times.
constexpr int kMaxGroups = 64;  // 4 waves x 16 chunks per lane

template <int WPR, int VPL, bool kMax = false>
__device__ __forceinline__ float fold_groups(const float (&part)[VPL], int wr, int groups, float* red) {
  float g[VPL];
#pragma unroll
  for (int k = 0; k < VPL; ++k) g[k] = kMax ? wave_max(part[k]) : wave_sum(part[k]);
  if constexpr (WPR == 1) {
    float total = g[0];
#pragma unroll
    for (int k = 1; k < VPL; ++k) {
      if (k < groups) total = kMax ? fmaxf(total, g[k]) : total + g[k];
    }
    return total;
  } else {
    if ((threadIdx.x & (kWave - 1)) == 0) {
#pragma unroll
      for (int k = 0; k < VPL; ++k) {
        const int grp = wr + WPR * k;
        if (grp < groups) red[grp] = g[k];
      }
    }
    __syncthreads();
    float total = red[0];
    for (int i = 1; i < groups; ++i) total = kMax ? fmaxf(total, red[i]) : total + red[i];
    __syncthreads();  // red is reused by the next fold
    return total;
  }
}

// Sum over the kBlock threads of a workgroup; `lds` holds kWavesPerBlock
// floats. Every thread of the block must call it.
__device__ __forceinline__ float block_sum(float v, float* lds) {
  v = wave_sum(v);
  if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = v;
  __syncthreads();
  const float total = (lds[0] + lds[1]) + (lds[2] + lds[3]);
  __syncthreads();
  return total;
}

__device__ __forceinline__ float block_max(float v, float* lds) {
  v = wave_max(v);
  if ((threadIdx.x & (kWave - 1)) == 0) lds[threadIdx.x / kWave] = v;
  __syncthreads();
  const float total = fmaxf(fmaxf(lds[0], lds[1]), fmaxf(lds[2], lds[3]));
  __syncthreads();
  return total;
}

// Rows below this count leave most of the GPU idle at one wave per row, so
// row kernels spread each row over 4 waves instead.
constexpr int64_t kFewRows = 2048;

inline int vpl_bucket(int64_t groups) {
  if (groups <= 1) return 1;
  if (groups <= 2) return 2;
  if (groups <= 4) return 4;
  if (groups <= 8) return 8;
  return 16;
}

// t / d for t < 2^32 as the high word of t * magic, magic = ceil(2^64 / d)
// (reciprocal_magic); d == 1 passes magic = 0.
__device__ __forceinline__ uint32_t div_by_magic(uint32_t t, uint64_t magic) {
  return magic == 0 ? t : static_cast<uint32_t>(__umul64hi(static_cast<uint64_t>(t), magic));
}

// ceil(2^64 / d) for 2 <= d < 2^32, as floor((2^64 - 1) / d) + 1: for d not
// a power of two, d does not divide 2^64 and the floor equals floor(2^64 / d);
// for d = 2^k the floor is 2^(64-k) - 1. Then floor(t * m / 2^64) = t / d for
// every t < 2^32, because the excess t * (m - 2^64 / d) / 2^64 < 2^-32 < 1 / d.
inline uint64_t reciprocal_magic(uint32_t d) {
  if (d <= 1) return 0;
  return ~uint64_t{0} / d + 1;
}

// ---- XCD-aware block order --------------------------------------------------------
// MI355X dispatches consecutive workgroups round-robin over its 8 XCDs, each
// with its own L2. xcd_block(b, n) renumbers block b of n so that XCD x walks
// one contiguous range of the logical blocks: blocks that share data (rows
// that read the same mask row) then meet in one L2. A bijection on [0, n).
constexpr unsigned kXcds = 8;

__device__ __forceinline__ unsigned xcd_block(unsigned b, unsigned n) {
  const unsigned xcd = b % kXcds, local = b / kXcds;
  const unsigned per = n / kXcds, extra = n % kXcds;
  return xcd * per + (xcd < extra ? xcd : extra) + local;
}

// ---- host side ----------------------------------------------------------------

// Records "<what>: <detail>" as this thread's last error and returns `status`.
int fail(int status, const char* what, const std::string& detail);
// UOCR_ROCM_OK, or UOCR_ROCM_RUNTIME_ERROR with the HIP error string.
int check_hip(hipError_t err, const char* what);
// Reports a failed launch through hipGetLastError.
int check_launch(const char* what);
// Clears a stale launch error left by earlier work on this thread.
inline void clear_launch_error() { (void)hipGetLastError(); }

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// The plain bf16 product through the BLAS library (gemm_library.hip):
// UOCR_ROCM_OK, kLibraryDeclined when the product is not one it takes (the
// caller runs the tile kernels), or an error status.
constexpr int kLibraryDeclined = -1;
int library_linear_bf16(const char* what, hipStream_t s, const uint16_t* x, int64_t m, int64_t k,
                        const uint16_t* w, int64_t n, const float* bias, float* y, bool accumulate);

inline hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

inline unsigned blocks_for_rows(int64_t rows) {
  return static_cast<unsigned>((rows + kWavesPerBlock - 1) / kWavesPerBlock);
}

// ---- launches in pieces -----------------------------------------------------------
// One dispatch holds at most 2^32 - 1 work-items. An op over more rows (or
// chunks) than one launch of modest size reaches runs as consecutive
// launches over contiguous pieces: fn(first, count) for pieces of at most
// `piece` units covering [0, total), in order; one call with count 0 when
// total is 0. A piece of kPieceRows rows is at most 2^28 work-items (256
// threads per row on the widest path) and kPieceChunks 128-bit chunks 2^28
// work-items; both are gigabytes of data, so the extra launches cost
// nothing measurable.
constexpr int64_t kPieceRows = int64_t{1} << 20;
constexpr int64_t kPieceChunks = int64_t{1} << 28;

// ---- split-K decode attention records (decode.hip writes, decode.hip and
// gemv.hip merge) -----------------------------------------------------------------

constexpr float kLog2e = 1.4426950408889634f;

// exp(s - m) through the hardware's base-2 exponential.
__device__ __forceinline__ float exp_shift(float s, float m) { return __builtin_amdgcn_exp2f((s - m) * kLog2e); }

// Live keys per split when the attention walks a routed step's live-key
// segments, and the split count for at most max_live live keys: 32 keys
// each, at most 64 splits (one merge wave).
constexpr int kLiveKeysPerSplit = 32;

inline int segment_splits(int64_t max_live) {
  const int64_t s = (max_live + kLiveKeysPerSplit - 1) / kLiveKeysPerSplit;
  return static_cast<int>(s < 1 ? 1 : (s > kWave ? kWave : s));
}

template <class Fn>
void for_each_piece(int64_t total, int64_t piece, Fn&& fn) {
  int64_t first = 0;
  do {
    const int64_t count = total - first < piece ? total - first : piece;
    fn(first, count);
    first += count;
  } while (first < total);
}

}  // namespace uocr_rocm

#define UOCR_REQUIRE(cond, what, detail)                                  \
  do {                                                                    \
    if (!(cond)) return ::uocr_rocm::fail(UOCR_ROCM_INVALID_ARGUMENT, what, detail); \
  } while (0)
