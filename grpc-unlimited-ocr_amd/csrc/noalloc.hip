// noalloc.hip: uocr_rocm_attend_step_noalloc, the decode attention of
// uocr_rocm_attend_step with its split records kept in a fixed device array
// instead of a caller's scratch buffer, for callers that cannot allocate.
//
// The records live in `scratch`, a file-scope device array of
// kNoAllocScratchFloats floats (4 MiB) that every GPU the library runs on
// holds until the process ends. Its device address is looked up once per
// device (hipGetSymbolAddress, with that device current) on the entry
// point's first call there, and that address, never the array's name, is
// what the kernels receive. Every call on one GPU shares that GPU's array:
// the partial kernel writes every record the merge reads, so nothing needs
// clearing between calls, but calls that overlap on one GPU (two streams, or
// two host threads) race on it.

#include <mutex>

#include "common.hpp"

namespace uocr_rocm {

int attend_step_f32(const char* what, void* stream, const float* q, const float* k_cache, const float* v_cache,
                    int64_t heads, int64_t hd, const float* mask, float scale, const uocr_rocm_step_state* state,
                    float* scratch, int64_t capacity, float* out);

namespace {

constexpr int64_t kNoAllocScratchFloats = int64_t{1} << 20;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) float scratch[kNoAllocScratchFloats];

std::mutex g_scratch_mutex;
float* g_scratch_address[kMaxDevices];  // per device; null until looked up

// The current device's address of `scratch`.
int scratch_address(const char* what, float** address) {
  int device = -1;
  if (const int st = check_hip(hipGetDevice(&device), what)) return st;
  UOCR_REQUIRE(device >= 0 && device < kMaxDevices, what, "device ordinal above 63");
  std::lock_guard<std::mutex> lock(g_scratch_mutex);
  if (g_scratch_address[device] == nullptr) {
    void* p = nullptr;
    if (const int st = check_hip(hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)), what)) return st;
    UOCR_REQUIRE(p != nullptr, what, "no device address for the scratch array");
    g_scratch_address[device] = static_cast<float*>(p);
  }
  *address = g_scratch_address[device];
  return UOCR_ROCM_OK;
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

int uocr_rocm_attend_step_noalloc(void* stream, const float* q, const float* k_cache, const float* v_cache,
                                  int64_t heads, int64_t hd, const float* mask, float scale,
                                  const uocr_rocm_step_state* state, int64_t capacity, float* out) {
  constexpr const char* kWhat = "uocr_rocm_attend_step_noalloc";
  UOCR_REQUIRE(heads >= 0 && hd >= 0, kWhat, "heads and hd must be >= 0");
  if (heads == 0 || hd == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(capacity >= 1, kWhat, "capacity must be >= 1");
  const int64_t need = uocr_rocm_attend_scratch_floats(heads, hd, capacity);
  UOCR_REQUIRE(need <= kNoAllocScratchFloats, kWhat,
               "the split records of this (heads, hd, capacity) exceed the fixed 1048576-float scratch array; "
               "use uocr_rocm_attend_step with a scratch buffer");
  float* records = nullptr;
  if (const int st = scratch_address(kWhat, &records)) return st;
  return attend_step_f32(kWhat, stream, q, k_cache, v_cache, heads, hd, mask, scale, state, records, capacity, out);
}

}  // extern "C"
