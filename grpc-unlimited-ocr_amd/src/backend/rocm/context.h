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

// A device and the one non-blocking HIP stream every op of this backend is
// queued on, in submission order. Nothing here waits for the device unless
// a call says it does (synchronize, the download functions).
class Context {
 public:
  explicit Context(int device = 0);
  ~Context();
  Context(const Context&) = delete;
  Context& operator=(const Context&) = delete;

  void synchronize() const;

  // Between begin_capture and end_capture, work queued on the stream is not
  // executed: it is collected, and end_capture returns it as a replayable
  // graph.
  void begin_capture() const;
  std::unique_ptr<Graph> end_capture() const;

  int device() const { return device_; }
  // The hipStream_t, as the C ABI takes it.
  void* stream() const { return stream_; }

 private:
  int device_ = 0;
  void* stream_ = nullptr;
};

// Work collected by Context::begin_capture / end_capture, instantiated once;
// launch() queues one replay on the stream it was captured from.
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

// Host memory pinned for DMA: a copy between it and the device is queued
// on the stream and the host continues at once.
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

// Queue a copy of `bytes` (at most the pinned buffer's size) behind the
// stream's earlier work and return without waiting for it.
void copy_to_device(const Context& ctx, void* device_dst, const PinnedBuffer& src, std::size_t bytes);
void copy_to_host(const Context& ctx, PinnedBuffer& dst, const void* device_src, std::size_t bytes);
// Queue a copy of `bytes` from one device block to another (non-overlapping).
void copy_on_device(const Context& ctx, void* device_dst, const void* device_src, std::size_t bytes);

enum class DType : std::uint8_t { kF32, kBF16, kI64, kI8 };

// Gives an Array's block back to the device pool on the stream it was taken
// on (the deleter of Array's owning pointer).
struct StreamRelease {
  void* stream = nullptr;
  void operator()(void* p) const noexcept;
};

// `count` device elements of one DType. The block is taken from and given
// back to the device's pool on the context's stream, so its lifetime is
// ordered with the work queued there; it holds garbage until written. A
// moved-from Array owns nothing.
class Array {
 public:
  Array() = default;
  Array(const Context& ctx, DType type, std::int64_t count);
  ~Array() = default;
  Array(Array&&) noexcept = default;
  Array& operator=(Array&&) noexcept = default;
  Array(const Array&) = delete;
  Array& operator=(const Array&) = delete;

  // From host fp32 values: copied as they are into a kF32 array, rounded to
  // bf16 (nearest even) for a kBF16 one. Waits for the copy.
  void upload(const float* host, std::int64_t count, std::int64_t offset = 0);
  // Raw bf16 bit patterns into a kBF16 array. Waits for the copy.
  void upload(const std::uint16_t* host, std::int64_t count, std::int64_t offset = 0);
  // 64-bit integers (indices, positions) into a kI64 array.
  void upload(const std::int64_t* host, std::int64_t count, std::int64_t offset = 0);
  // Signed bytes into a kI8 array.
  void upload(const std::int8_t* host, std::int64_t count, std::int64_t offset = 0);
  // The whole array as fp32 on the host (bf16 widened exactly); waits for
  // the stream.
  std::vector<float> download() const;
  // The bit patterns of a kBF16 array; waits for the stream.
  std::vector<std::uint16_t> download_bf16() const;
  void zero();

  void* data() const { return block_.get(); }
  // Typed views of data(); each throws std::logic_error when the array
  // holds another element type.
  float* f32() const { return typed<float>(DType::kF32); }
  std::uint16_t* bf16() const { return typed<std::uint16_t>(DType::kBF16); }
  std::int64_t* i64() const { return typed<std::int64_t>(DType::kI64); }
  std::int8_t* i8() const { return typed<std::int8_t>(DType::kI8); }
  std::int64_t count() const { return count_; }
  DType type() const { return type_; }
  const Context* context() const { return ctx_; }

 private:
  template <class T>
  T* typed(DType want) const {
    if (type_ != want) type_mismatch(want);
    return static_cast<T*>(block_.get());
  }
  [[noreturn]] void type_mismatch(DType want) const;

  const Context* ctx_ = nullptr;
  std::unique_ptr<void, StreamRelease> block_;
  std::int64_t count_ = 0;
  DType type_ = DType::kF32;
};

}  // namespace uocr::rocm
