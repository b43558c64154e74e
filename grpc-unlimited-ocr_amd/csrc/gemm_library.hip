// gemm_library.hip: the plain prefill projection y[m, n] = x[m, k] . w[n, k]^T
// (+ bias[n]) with x and w bf16 and y fp32 through hipBLASLt, the ROCm
// counterpart of the cuBLAS call inside the reference's cuda::linear
// (src/backend/cuda/ops.cu:268-287: a bf16 GEMM with fp32 compute, then the
// bias). The hand-written tile kernels (gemm.hip) keep the products with an
// activation epilogue into bf16 or a row scatter, fp32 x, and few rows; this
// path takes the plain products (bias, and an add into y, allowed) of at
// least kLibraryMinRows rows, where the library's tiles run about 1.6x the
// hand-written ones (865 against 537 TFLOP/s over a dense decoder layer's
// four projections at 4096 rows, random bf16 operands).
//
// In hipBLASLt's column-major terms y^T [n, m] = w [k, n]^T . x^T [k, m]:
// A = w transposed (lda k), B = x (ldb k), D = y (ldd n), and the bias
// epilogue adds bias[n] to every column of D, one fp32 rounding after the
// sum as the reference's separate bias pass. The product runs without a
// workspace, so no algorithm splits k over one (every candidate this path
// takes is GSU0); the results are deterministic from call to call.
//
// With accumulate the product is added to y (beta 1, C = D = y):
// y + (sum + bias) up to the order of the two additions.
//
// Plans are kept per (device, m, n, k, bias). A new shape's first call,
// when its stream is not capturing a graph and the call does not accumulate
// (the timing runs overwrite y), times up to kCandidates of the library's
// heuristic candidates on that stream (one warm-up and two timed runs each,
// so the call waits for the stream) and keeps the fastest; otherwise it
// takes the heuristic's first. UOCR_ROCM_GEMM=tiles in the environment
// sends every product to the hand-written kernels.

#include <hipblaslt/hipblaslt.h>

#include <cstdlib>
#include <cstring>
#include <map>
#include <mutex>
#include <tuple>

#include "common.hpp"

namespace uocr_rocm {

constexpr int64_t kLibraryMinRows = 128;
constexpr int kCandidates = 8;

namespace {

struct Plan {
  hipblasLtMatmulDesc_t desc = nullptr;
  hipblasLtMatrixLayout_t a = nullptr, b = nullptr, d = nullptr;
  hipblasLtMatmulAlgo_t algo{};
};

struct Library {
  std::mutex mu;
  std::map<int, hipblasLtHandle_t> handles;  // per device
  std::map<std::tuple<int, int64_t, int64_t, int64_t, bool>, Plan> plans;
};

Library& library() {
  static Library* lib = new Library;  // never destroyed: kernels may be in flight at exit
  return *lib;
}

bool tiles_forced() {
  const char* v = std::getenv("UOCR_ROCM_GEMM");
  return v != nullptr && std::strcmp(v, "tiles") == 0;
}

// Builds the plan (descriptor, layouts, candidates) or returns false when
// the library offers no algorithm.
bool make_plan(hipblasLtHandle_t h, int64_t m, int64_t n, int64_t k, bool bias, Plan& p,
               hipblasLtMatmulHeuristicResult_t (&found)[kCandidates], int& count) {
  if (hipblasLtMatmulDescCreate(&p.desc, HIPBLAS_COMPUTE_32F, HIP_R_32F) != HIPBLAS_STATUS_SUCCESS) return false;
  const hipblasOperation_t ta = HIPBLAS_OP_T, tb = HIPBLAS_OP_N;
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSA, &ta, sizeof(ta));
  hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_TRANSB, &tb, sizeof(tb));
  if (bias) {
    const hipblasLtEpilogue_t epi = HIPBLASLT_EPILOGUE_BIAS;
    const hipDataType bias_type = HIP_R_32F;
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_EPILOGUE, &epi, sizeof(epi));
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_DATA_TYPE, &bias_type, sizeof(bias_type));
  }
  if (hipblasLtMatrixLayoutCreate(&p.a, HIP_R_16BF, static_cast<uint64_t>(k), static_cast<uint64_t>(n), k) !=
          HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.b, HIP_R_16BF, static_cast<uint64_t>(k), static_cast<uint64_t>(m), k) !=
          HIPBLAS_STATUS_SUCCESS ||
      hipblasLtMatrixLayoutCreate(&p.d, HIP_R_32F, static_cast<uint64_t>(n), static_cast<uint64_t>(m), n) !=
          HIPBLAS_STATUS_SUCCESS) {
    return false;
  }
  hipblasLtMatmulPreference_t pref = nullptr;
  if (hipblasLtMatmulPreferenceCreate(&pref) != HIPBLAS_STATUS_SUCCESS) return false;
  const uint64_t no_workspace = 0;
  hipblasLtMatmulPreferenceSetAttribute(pref, HIPBLASLT_MATMUL_PREF_MAX_WORKSPACE_BYTES, &no_workspace,
                                        sizeof(no_workspace));
  count = 0;
  const hipblasStatus_t st =
      hipblasLtMatmulAlgoGetHeuristic(h, p.desc, p.a, p.b, p.d, p.d, pref, kCandidates, found, &count);
  hipblasLtMatmulPreferenceDestroy(pref);
  int usable = 0;
  for (int i = 0; i < count; ++i) {
    if (found[i].state == HIPBLAS_STATUS_SUCCESS && found[i].workspaceSize == 0) found[usable++] = found[i];
  }
  count = usable;
  return st == HIPBLAS_STATUS_SUCCESS && count > 0;
}

hipblasStatus_t run(hipblasLtHandle_t h, const Plan& p, const hipblasLtMatmulAlgo_t& algo, const uint16_t* x,
                    const uint16_t* w, float* y, hipStream_t s, bool accumulate = false) {
  const float alpha = 1.0f, beta = accumulate ? 1.0f : 0.0f;
  return hipblasLtMatmul(h, p.desc, &alpha, w, p.a, x, p.b, &beta, y, p.d, y, p.d, &algo, nullptr, 0, s);
}

}  // namespace

// UOCR_ROCM_OK when the library formed y; kLibraryDeclined when the product
// is not one it takes (the caller runs the tiles); an error status when a
// call into the runtime or the library failed.
int library_linear_bf16(const char* what, hipStream_t s, const uint16_t* x, int64_t m, int64_t k,
                        const uint16_t* w, int64_t n, const float* bias, float* y, bool accumulate) {
  if (m < kLibraryMinRows || k % 8 != 0 || !aligned16(x) || !aligned16(w) || !aligned16(y) || tiles_forced()) {
    return kLibraryDeclined;
  }
  int device = 0;
  if (hipGetDevice(&device) != hipSuccess) return fail(UOCR_ROCM_RUNTIME_ERROR, what, "hipGetDevice failed");
  Library& lib = library();
  std::lock_guard<std::mutex> lock(lib.mu);
  hipblasLtHandle_t& h = lib.handles[device];
  if (h == nullptr && hipblasLtCreate(&h) != HIPBLAS_STATUS_SUCCESS) {
    h = nullptr;
    return kLibraryDeclined;
  }
  const auto key = std::make_tuple(device, m, n, k, bias != nullptr);
  auto it = lib.plans.find(key);
  if (it == lib.plans.end()) {
    Plan p;
    hipblasLtMatmulHeuristicResult_t found[kCandidates];
    int count = 0;
    if (!make_plan(h, m, n, k, bias != nullptr, p, found, count)) return kLibraryDeclined;
    p.algo = found[0].algo;
    hipStreamCaptureStatus capture = hipStreamCaptureStatusNone;
    if (count > 1 && !accumulate && hipStreamIsCapturing(s, &capture) == hipSuccess &&
        capture == hipStreamCaptureStatusNone) {
      if (bias != nullptr) {
        hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
      }
      hipEvent_t e0 = nullptr, e1 = nullptr;
      if (hipEventCreate(&e0) == hipSuccess && hipEventCreate(&e1) == hipSuccess) {
        float best = 0.0f;
        for (int i = 0; i < count; ++i) {
          if (run(h, p, found[i].algo, x, w, y, s) != HIPBLAS_STATUS_SUCCESS) continue;
          if (hipEventRecord(e0, s) != hipSuccess) continue;
          run(h, p, found[i].algo, x, w, y, s);
          run(h, p, found[i].algo, x, w, y, s);
          if (hipEventRecord(e1, s) != hipSuccess) continue;
          float ms = 0.0f;
          if (hipEventSynchronize(e1) != hipSuccess || hipEventElapsedTime(&ms, e0, e1) != hipSuccess) continue;
          if (best == 0.0f || ms < best) {
            best = ms;
            p.algo = found[i].algo;
          }
        }
      }
      if (e0 != nullptr) (void)hipEventDestroy(e0);
      if (e1 != nullptr) (void)hipEventDestroy(e1);
    }
    it = lib.plans.emplace(key, p).first;
  }
  const Plan& p = it->second;
  if (bias != nullptr) {
    hipblasLtMatmulDescSetAttribute(p.desc, HIPBLASLT_MATMUL_DESC_BIAS_POINTER, &bias, sizeof(bias));
  }
  if (run(h, p, p.algo, x, w, y, s, accumulate) != HIPBLAS_STATUS_SUCCESS) {
    return fail(UOCR_ROCM_RUNTIME_ERROR, what, "hipblasLtMatmul failed");
  }
  return UOCR_ROCM_OK;
}

}  // namespace uocr_rocm
