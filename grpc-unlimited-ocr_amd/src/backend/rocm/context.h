#pragma once

// The rocm backend's device handles and memory, behind a header with no HIP
// includes: C++23 host code links against the gfx950 kernels through the C
// ABI of include/uocr_rocm.h only. Same shape as the reference's
// src/backend/cuda/context.h:12-123 (Context, Graph, PinnedBuffer, Array),
// so model code written against uocr::cuda reads the same against
// uocr::rocm.

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

namespace uocr::rocm {

struct DeviceInfo {
  std::string name;       // marketing name and gfx target
  int gfx_arch = 0;       // 950 for MI355X
  int compute_units = 0;  // 256 for MI355X
  std::uint64_t free_bytes = 0;
  std::uint64_t total_bytes = 0;
};

// Number of visible devices; 0 when there is no usable HIP runtime or GPU.
int device_count();
DeviceInfo device_info(int index);

// Turns a non-zero C-ABI status into the reference's exception types:
// std::invalid_argument for bad shapes and arguments, std::runtime_error
// ("<what>: <detail>") for runtime and launch failures.
void check(int status);

class Graph;

// One device and one non-blocking stream. Every op runs on this stream in
// order; host reads synchronise explicitly.
class Context {
 public:
  explicit Context(int device = 0);
  ~Context();
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;

  void synchronize() const;

  // Records everything enqueued between the two calls as a graph instead of
  // running it.
  void begin_capture() const;
  std::unique_ptr<Graph> end_capture() const;

  int device() const { return device_; }
  // The hipStream_t, as the C ABI takes it.
  void* stream() const { return stream_; }

 private:
  int device_ = 0;
  void* stream_ = nullptr;
};

// A captured, instantiated sequence of device work, replayed on the
// context's stream.
class Graph {
 public:
  Graph(void* handle, void* stream) : handle_(handle), stream_(stream) {}
  ~Graph();
  Graph(const Graph&) = delete;
  Graph& operator=(const Graph&) = delete;
  void launch() const;

 private:
  void* handle_ = nullptr;
  void* stream_ = nullptr;
};

// Page-locked host memory, so copies to and from the device are enqueued
// without blocking the host.
class PinnedBuffer {
 public:
  explicit PinnedBuffer(std::size_t bytes);
  ~PinnedBuffer();
  PinnedBuffer(const PinnedBuffer&) = delete;
  PinnedBuffer& operator=(const PinnedBuffer&) = delete;
  void* data() const { return data_; }
  std::size_t bytes() const { return bytes_; }

 private:
  void* data_ = nullptr;
  std::size_t bytes_ = 0;
};

// Stream-ordered copies; neither waits.
void copy_to_device(const Context& ctx, void* device_dst, const PinnedBuffer& src, std::size_t bytes);
void copy_to_host(const Context& ctx, PinnedBuffer& dst, const void* device_src, std::size_t bytes);

enum class DType : std::uint8_t { kF32, kBF16, kI64, kI8 };

// Device memory of `count` elements of one type, allocated and freed in
// stream order. Contents are undefined until written.
class Array {
 public:
  Array() = default;
  Array(const Context& ctx, DType type, std::int64_t count);
  ~Array();
  Array(Array&& other) noexcept;
  Array& operator=(Array&& other) noexcept;
  Array(const Array&) = delete;
  Array& operator=(const Array&) = delete;

  // Host fp32 in; stored as `type()` (bf16 rounds to nearest even).
  void upload(const float* host, std::int64_t count, std::int64_t offset = 0);
  // Host bf16 bits in, for kBF16 arrays.
  void upload(const std::uint16_t* host, std::int64_t count, std::int64_t offset = 0);
  // Host indices in, for kI64 arrays.
  void upload(const std::int64_t* host, std::int64_t count, std::int64_t offset = 0);
  // Host bytes in, for kI8 arrays.
  void upload(const std::int8_t* host, std::int64_t count, std::int64_t offset = 0);
  // Device contents widened to fp32 (synchronises the stream).
  std::vector<float> download() const;
  // Raw bf16 bits (synchronises the stream), for kBF16 arrays.
  std::vector<std::uint16_t> download_bf16() const;
  void zero();

  void* data() const { return data_; }
  float* f32() const;
  std::uint16_t* bf16() const;
  std::int64_t* i64() const;
  std::int8_t* i8() const;
  std::int64_t count() const { return count_; }
  DType type() const { return type_; }
  const Context* context() const { return ctx_; }

 private:
  void release() noexcept;

  const Context* ctx_ = nullptr;
  void* data_ = nullptr;
  std::int64_t count_ = 0;
  DType type_ = DType::kF32;
};

}  // namespace uocr::rocm
