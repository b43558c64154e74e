// runtime.hip: status reporting, devices, streams, memory, graphs and events
// of the C ABI. Replaces the device plumbing of the reference's
// src/backend/cuda/context.{h,cu}: one stream per context, stream-ordered
// allocation, pinned host buffers, and graph capture and replay.

#include <cstdio>
#include <cstring>
#include <string>

#include "common.hpp"

namespace uocr_rocm {
namespace {
thread_local std::string g_last_error;
}

int fail(int status, const char* what, const std::string& detail) {
  g_last_error = std::string(what) + ": " + detail;
  return status;
}

int check_hip(hipError_t err, const char* what) {
  if (err == hipSuccess) return UOCR_ROCM_OK;
  return fail(UOCR_ROCM_RUNTIME_ERROR, what, hipGetErrorString(err));
}

int check_launch(const char* what) {
  const hipError_t err = hipGetLastError();
  if (err == hipSuccess) return UOCR_ROCM_OK;
  return fail(UOCR_ROCM_LAUNCH_ERROR, what, hipGetErrorString(err));
}

namespace {

// Byte fill for Array::zero: 16-byte stores over the aligned body, single
// bytes over the ragged ends. A kernel, not hipMemsetAsync, so that a zero
// recorded into a graph is replayed as a kernel node.
__global__ __launch_bounds__(kBlock) void zero_kernel(uint8_t* p, uint64_t head, uint64_t body16, uint64_t tail) {
  const uint64_t i = static_cast<uint64_t>(blockIdx.x) * kBlock + threadIdx.x;
  const uint64_t stride = static_cast<uint64_t>(gridDim.x) * kBlock;
  for (uint64_t k = i; k < body16; k += stride) {
    *reinterpret_cast<u32x4*>(p + head + 16 * k) = u32x4{0u, 0u, 0u, 0u};
  }
  if (i < head) p[i] = 0;
  if (i < tail) p[head + 16 * body16 + i] = 0;
}

}  // namespace
}  // namespace uocr_rocm

using namespace uocr_rocm;

extern "C" {

const char* uocr_rocm_status_string(int status) {
  switch (status) {
    case UOCR_ROCM_OK: return "ok";
    case UOCR_ROCM_INVALID_ARGUMENT: return "invalid argument";
    case UOCR_ROCM_NO_DEVICE: return "no device";
    case UOCR_ROCM_RUNTIME_ERROR: return "HIP runtime error";
    case UOCR_ROCM_LAUNCH_ERROR: return "kernel launch error";
    default: return "unknown status";
  }
}

const char* uocr_rocm_last_error(void) { return g_last_error.c_str(); }

int uocr_rocm_abi_version(void) { return (1 << 16) | 0; }

int uocr_rocm_device_count(int* count) {
  UOCR_REQUIRE(count != nullptr, "uocr_rocm_device_count", "null count");
  int n = 0;
  *count = hipGetDeviceCount(&n) == hipSuccess ? n : 0;
  (void)hipGetLastError();  // no device is an answer, not an error
  return UOCR_ROCM_OK;
}

int uocr_rocm_device_info(int index, char* name, size_t name_len, int* gfx_arch, int* cu_count, uint64_t* free_bytes,
                          uint64_t* total_bytes) {
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return fail(UOCR_ROCM_NO_DEVICE, "uocr_rocm_device_info", "no HIP device");
  }
  UOCR_REQUIRE(index >= 0 && index < n, "uocr_rocm_device_info", "device index out of range");
  hipDeviceProp_t prop{};
  int st = check_hip(hipGetDeviceProperties(&prop, index), "hipGetDeviceProperties");
  if (st) return st;
  if ((st = check_hip(hipSetDevice(index), "hipSetDevice"))) return st;
  size_t free_b = 0, total_b = 0;
  if ((st = check_hip(hipMemGetInfo(&free_b, &total_b), "hipMemGetInfo"))) return st;
  if (name != nullptr && name_len > 0) {
    std::snprintf(name, name_len, "%s (%s)", prop.name, prop.gcnArchName);
  }
  if (gfx_arch != nullptr) {
    // gcnArchName reads "gfx950:sramecc+:xnack-": report the decimal digits after "gfx".
    int v = 0;
    *gfx_arch = std::sscanf(prop.gcnArchName, "gfx%d", &v) == 1 ? v : 0;
  }
  if (cu_count != nullptr) *cu_count = prop.multiProcessorCount;
  if (free_bytes != nullptr) *free_bytes = free_b;
  if (total_bytes != nullptr) *total_bytes = total_b;
  return UOCR_ROCM_OK;
}

int uocr_rocm_stream_create(int device, void** stream) {
  UOCR_REQUIRE(stream != nullptr, "uocr_rocm_stream_create", "null stream out-pointer");
  int n = 0;
  if (hipGetDeviceCount(&n) != hipSuccess || n == 0) {
    (void)hipGetLastError();
    return fail(UOCR_ROCM_NO_DEVICE, "uocr_rocm_stream_create", "no HIP device");
  }
  UOCR_REQUIRE(device >= 0 && device < n, "uocr_rocm_stream_create", "device index out of range");
  int st = check_hip(hipSetDevice(device), "hipSetDevice");
  if (st) return st;
  // The device pool keeps the blocks Arrays give back instead of returning
  // them to the driver (its default threshold is 0): a model's per-call
  // buffers (a vision layer's scores are 0.8 GB) are taken again at once
  // rather than mapped anew each time. 288 GB of HBM leaves room for it.
  hipMemPool_t pool = nullptr;
  if ((st = check_hip(hipDeviceGetDefaultMemPool(&pool, device), "hipDeviceGetDefaultMemPool"))) return st;
  uint64_t keep = UINT64_MAX;
  if ((st = check_hip(hipMemPoolSetAttribute(pool, hipMemPoolAttrReleaseThreshold, &keep),
                      "hipMemPoolSetAttribute"))) {
    return st;
  }
  hipStream_t s = nullptr;
  // Default priority only: streams of mixed priorities are not used here.
  if ((st = check_hip(hipStreamCreateWithFlags(&s, hipStreamNonBlocking), "hipStreamCreateWithFlags"))) return st;
  *stream = s;
  return UOCR_ROCM_OK;
}

int uocr_rocm_stream_destroy(void* stream) {
  if (stream == nullptr) return UOCR_ROCM_OK;
  int st = check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
  const int st2 = check_hip(hipStreamDestroy(as_stream(stream)), "hipStreamDestroy");
  return st ? st : st2;
}

int uocr_rocm_stream_synchronize(void* stream) {
  return check_hip(hipStreamSynchronize(as_stream(stream)), "hipStreamSynchronize");
}

int uocr_rocm_capture_begin(void* stream) {
  UOCR_REQUIRE(stream != nullptr, "uocr_rocm_capture_begin", "capture needs a created stream, not the null stream");
  return check_hip(hipStreamBeginCapture(as_stream(stream), hipStreamCaptureModeThreadLocal), "hipStreamBeginCapture");
}

namespace {
struct GraphHandle {
  hipGraph_t graph = nullptr;
  hipGraphExec_t exec = nullptr;
};
}  // namespace

int uocr_rocm_capture_end(void* stream, void** graph) {
  UOCR_REQUIRE(stream != nullptr && graph != nullptr, "uocr_rocm_capture_end", "null stream or graph out-pointer");
  auto* g = new GraphHandle;
  int st = check_hip(hipStreamEndCapture(as_stream(stream), &g->graph), "hipStreamEndCapture");
  if (st == UOCR_ROCM_OK) st = check_hip(hipGraphInstantiate(&g->exec, g->graph, nullptr, nullptr, 0), "hipGraphInstantiate");
  if (st != UOCR_ROCM_OK) {
    if (g->graph != nullptr) (void)hipGraphDestroy(g->graph);
    delete g;
    return st;
  }
  *graph = g;
  return UOCR_ROCM_OK;
}

int uocr_rocm_graph_launch(void* graph, void* stream) {
  UOCR_REQUIRE(graph != nullptr, "uocr_rocm_graph_launch", "null graph");
  return check_hip(hipGraphLaunch(static_cast<GraphHandle*>(graph)->exec, as_stream(stream)), "hipGraphLaunch");
}

int uocr_rocm_graph_destroy(void* graph) {
  if (graph == nullptr) return UOCR_ROCM_OK;
  auto* g = static_cast<GraphHandle*>(graph);
  int st = UOCR_ROCM_OK;
  if (g->exec != nullptr) st = check_hip(hipGraphExecDestroy(g->exec), "hipGraphExecDestroy");
  if (g->graph != nullptr) {
    const int st2 = check_hip(hipGraphDestroy(g->graph), "hipGraphDestroy");
    if (!st) st = st2;
  }
  delete g;
  return st;
}

int uocr_rocm_malloc(void** ptr, size_t bytes, void* stream) {
  UOCR_REQUIRE(ptr != nullptr, "uocr_rocm_malloc", "null out-pointer");
  *ptr = nullptr;
  if (bytes == 0) return UOCR_ROCM_OK;
  return check_hip(hipMallocAsync(ptr, bytes, as_stream(stream)), "hipMallocAsync");
}

int uocr_rocm_free(void* ptr, void* stream) {
  if (ptr == nullptr) return UOCR_ROCM_OK;
  return check_hip(hipFreeAsync(ptr, as_stream(stream)), "hipFreeAsync");
}

int uocr_rocm_host_alloc(void** ptr, size_t bytes) {
  UOCR_REQUIRE(ptr != nullptr, "uocr_rocm_host_alloc", "null out-pointer");
  *ptr = nullptr;
  if (bytes == 0) return UOCR_ROCM_OK;
  return check_hip(hipHostMalloc(ptr, bytes, hipHostMallocDefault), "hipHostMalloc");
}

int uocr_rocm_host_free(void* ptr) {
  if (ptr == nullptr) return UOCR_ROCM_OK;
  return check_hip(hipHostFree(ptr), "hipHostFree");
}

int uocr_rocm_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream) {
  if (bytes == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(dst != nullptr && src != nullptr, "uocr_rocm_memcpy", "null pointer");
  hipMemcpyKind k;
  switch (kind) {
    case UOCR_ROCM_H2D: k = hipMemcpyHostToDevice; break;
    case UOCR_ROCM_D2H: k = hipMemcpyDeviceToHost; break;
    case UOCR_ROCM_D2D: k = hipMemcpyDeviceToDevice; break;
    default: return fail(UOCR_ROCM_INVALID_ARGUMENT, "uocr_rocm_memcpy", "unknown copy kind");
  }
  return check_hip(hipMemcpyAsync(dst, src, bytes, k, as_stream(stream)), "hipMemcpyAsync");
}

int uocr_rocm_zero(void* ptr, size_t bytes, void* stream) {
  if (bytes == 0) return UOCR_ROCM_OK;
  UOCR_REQUIRE(ptr != nullptr, "uocr_rocm_zero", "null pointer");
  auto* p = static_cast<uint8_t*>(ptr);
  const uint64_t mis = reinterpret_cast<uintptr_t>(p) & 15u;
  uint64_t head = mis == 0 ? 0 : 16 - mis;
  if (head > bytes) head = bytes;
  const uint64_t body16 = (bytes - head) / 16;
  const uint64_t tail = bytes - head - 16 * body16;
  uint64_t blocks = (body16 + kBlock - 1) / kBlock;
  if (blocks < 1) blocks = 1;
  if (blocks > 65536) blocks = 65536;
  clear_launch_error();
  zero_kernel<<<static_cast<unsigned>(blocks), kBlock, 0, as_stream(stream)>>>(p, head, body16, tail);
  return check_launch("uocr_rocm_zero");
}

int uocr_rocm_event_create(void** event) {
  UOCR_REQUIRE(event != nullptr, "uocr_rocm_event_create", "null out-pointer");
  hipEvent_t e = nullptr;
  const int st = check_hip(hipEventCreate(&e), "hipEventCreate");
  *event = e;
  return st;
}

int uocr_rocm_event_destroy(void* event) {
  if (event == nullptr) return UOCR_ROCM_OK;
  return check_hip(hipEventDestroy(static_cast<hipEvent_t>(event)), "hipEventDestroy");
}

int uocr_rocm_event_record(void* event, void* stream) {
  UOCR_REQUIRE(event != nullptr, "uocr_rocm_event_record", "null event");
  return check_hip(hipEventRecord(static_cast<hipEvent_t>(event), as_stream(stream)), "hipEventRecord");
}

int uocr_rocm_event_elapsed_ms(void* start, void* end, float* ms) {
  UOCR_REQUIRE(start != nullptr && end != nullptr && ms != nullptr, "uocr_rocm_event_elapsed_ms", "null argument");
  int st = check_hip(hipEventSynchronize(static_cast<hipEvent_t>(end)), "hipEventSynchronize");
  if (st) return st;
  return check_hip(hipEventElapsedTime(ms, static_cast<hipEvent_t>(start), static_cast<hipEvent_t>(end)),
                   "hipEventElapsedTime");
}

}  // extern "C"
