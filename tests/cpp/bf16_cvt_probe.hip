// Exhaustive check that gfx950's packed conversion v_cvt_pk_bf16_f32 (what
// clang emits for __builtin_convertvector(float2 -> __bf16 x2)) rounds every
// one of the 2^32 fp32 bit patterns exactly as the reference's f32_to_bf16
// does (src/tensor/dtype.h:39-46): nearest even, NaN quieted with 0x0040 and
// its top bits kept, denormals kept. The kernels may use the instruction
// only because this holds. Prints the mismatch count and the first few
// mismatching patterns; exit 0 when there are none, 1 otherwise, 77 without
// a device.
//
// Bounds: the grid-stride loop covers [0, 2^32) with a 64-bit counter; every
// store goes to counters[lane] or samples[slot] with lane < 64 and slot
// clamped below kSamples.

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>

namespace {

constexpr int kSamples = 16;

typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

__device__ uint32_t rne_reference(uint32_t u) {
  if ((u & 0x7fffffffu) > 0x7f800000u) return ((u >> 16) | 0x40u) & 0xffffu;
  return ((u + 0x7fffu + ((u >> 16) & 1u)) >> 16) & 0xffffu;
}

__global__ void probe(unsigned long long* counters, uint32_t* samples) {
  const uint64_t total = uint64_t{1} << 32;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * blockDim.x;
  const unsigned lane = threadIdx.x & 63u;
  unsigned long long bad = 0;
  for (uint64_t i = static_cast<uint64_t>(blockIdx.x) * blockDim.x + threadIdx.x; i < total; i += 2 * stride) {
    // Two patterns per conversion: i and i + stride (when in range).
    const uint32_t a = static_cast<uint32_t>(i);
    const uint64_t j = i + stride;
    const uint32_t b = static_cast<uint32_t>(j < total ? j : i);
    const f32x2 v = {__uint_as_float(a), __uint_as_float(b)};
    const uint32_t hw = __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2));
    const bool bad_a = (hw & 0xffffu) != rne_reference(a);
    const bool bad_b = (hw >> 16) != rne_reference(b);
    if (bad_a || bad_b) {
      const unsigned long long slot = atomicAdd(&counters[64], 1ull);
      if (slot < kSamples) samples[slot] = bad_a ? a : b;
    }
    bad += static_cast<unsigned long long>(bad_a) + static_cast<unsigned long long>(bad_b && j < total);
  }
  atomicAdd(&counters[lane], bad);
}

}  // namespace

int main() {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    std::fprintf(stderr, "SKIP: no HIP device\n");
    return 77;
  }
  unsigned long long* counters = nullptr;
  uint32_t* samples = nullptr;
  if (hipMalloc(&counters, 65 * sizeof(unsigned long long)) != hipSuccess ||
      hipMalloc(&samples, kSamples * sizeof(uint32_t)) != hipSuccess) {
    std::fprintf(stderr, "hipMalloc failed\n");
    return 2;
  }
  (void)hipMemset(counters, 0, 65 * sizeof(unsigned long long));
  (void)hipMemset(samples, 0, kSamples * sizeof(uint32_t));
  probe<<<4096, 256>>>(counters, samples);
  if (hipDeviceSynchronize() != hipSuccess) {
    std::fprintf(stderr, "probe failed: %s\n", hipGetErrorString(hipGetLastError()));
    return 2;
  }
  unsigned long long host[65] = {0};
  uint32_t bad_bits[kSamples] = {0};
  (void)hipMemcpy(host, counters, sizeof host, hipMemcpyDeviceToHost);
  (void)hipMemcpy(bad_bits, samples, sizeof bad_bits, hipMemcpyDeviceToHost);
  unsigned long long mismatches = 0;
  for (int l = 0; l < 64; ++l) mismatches += host[l];
  std::printf("v_cvt_pk_bf16_f32 vs reference RNE over 2^32 patterns: %llu mismatches\n", mismatches);
  const unsigned long long shown = host[64] < kSamples ? host[64] : kSamples;
  for (unsigned long long s = 0; s < shown; ++s) std::printf("  mismatch at 0x%08x\n", bad_bits[s]);
  (void)hipFree(counters);
  (void)hipFree(samples);
  return mismatches == 0 ? 0 : 1;
}
