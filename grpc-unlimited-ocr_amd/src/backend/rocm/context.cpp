#include "backend/rocm/context.h"

#include <stdexcept>
#include <string>
#include <utility>

#include "backend/rocm/dtype.h"
#include "uocr_rocm.h"

namespace uocr::rocm {
namespace {

std::size_t element_bytes(DType t) {
  switch (t) {
    case DType::kI8: return 1;
    case DType::kBF16: return 2;
    case DType::kF32: return 4;
    case DType::kI64: return 8;
  }
  return 1;
}

}  // namespace

void check(int status) {
  if (status == UOCR_ROCM_OK) return;
  const std::string message = uocr_rocm_last_error();
  if (status == UOCR_ROCM_INVALID_ARGUMENT) throw std::invalid_argument(message);
  throw std::runtime_error(message);
}

int device_count() {
  int n = 0;
  return uocr_rocm_device_count(&n) == UOCR_ROCM_OK ? n : 0;
}

DeviceInfo device_info(int index) {
  char name[256] = {0};
  DeviceInfo info;
  check(uocr_rocm_device_info(index, name, sizeof name, &info.gfx_arch, &info.compute_units, &info.free_bytes,
                              &info.total_bytes));
  info.name = name;
  return info;
}

Context::Context(int device) : device_(device) { check(uocr_rocm_stream_create(device, &stream_)); }

Context::~Context() {
  if (stream_ != nullptr) (void)uocr_rocm_stream_destroy(stream_);
}

void Context::synchronize() const { check(uocr_rocm_stream_synchronize(stream_)); }

void Context::begin_capture() const { check(uocr_rocm_capture_begin(stream_)); }

std::unique_ptr<Graph> Context::end_capture() const {
  void* handle = nullptr;
  check(uocr_rocm_capture_end(stream_, &handle));
  return std::make_unique<Graph>(handle, stream_);
}

Graph::~Graph() { (void)uocr_rocm_graph_destroy(handle_); }

void Graph::launch() const { check(uocr_rocm_graph_launch(handle_, stream_)); }

PinnedBuffer::PinnedBuffer(std::size_t bytes) : bytes_(bytes) { check(uocr_rocm_host_alloc(&data_, bytes)); }

PinnedBuffer::~PinnedBuffer() { (void)uocr_rocm_host_free(data_); }

void copy_to_device(const Context& ctx, void* device_dst, const PinnedBuffer& src, std::size_t bytes) {
  if (bytes > src.bytes()) throw std::invalid_argument("copy_to_device: more bytes than the pinned buffer holds");
  check(uocr_rocm_memcpy(device_dst, src.data(), bytes, UOCR_ROCM_H2D, ctx.stream()));
}

void copy_to_host(const Context& ctx, PinnedBuffer& dst, const void* device_src, std::size_t bytes) {
  if (bytes > dst.bytes()) throw std::invalid_argument("copy_to_host: more bytes than the pinned buffer holds");
  check(uocr_rocm_memcpy(dst.data(), device_src, bytes, UOCR_ROCM_D2H, ctx.stream()));
}

Array::Array(const Context& ctx, DType type, std::int64_t count) : ctx_(&ctx), count_(count), type_(type) {
  if (count < 0) throw std::invalid_argument("Array: negative element count");
  const std::size_t bytes = static_cast<std::size_t>(count) * element_bytes(type);
  check(uocr_rocm_malloc(&data_, bytes, ctx.stream()));
}

void Array::release() noexcept {
  if (data_ != nullptr && ctx_ != nullptr) (void)uocr_rocm_free(data_, ctx_->stream());
  data_ = nullptr;
}

Array::~Array() { release(); }

Array::Array(Array&& o) noexcept
    : ctx_(o.ctx_), data_(std::exchange(o.data_, nullptr)), count_(std::exchange(o.count_, 0)), type_(o.type_) {}

Array& Array::operator=(Array&& o) noexcept {
  if (this != &o) {
    release();
    ctx_ = o.ctx_;
    data_ = std::exchange(o.data_, nullptr);
    count_ = std::exchange(o.count_, 0);
    type_ = o.type_;
  }
  return *this;
}

float* Array::f32() const {
  if (type_ != DType::kF32) throw std::logic_error("Array: not fp32");
  return static_cast<float*>(data_);
}

std::uint16_t* Array::bf16() const {
  if (type_ != DType::kBF16) throw std::logic_error("Array: not bf16");
  return static_cast<std::uint16_t*>(data_);
}

std::int64_t* Array::i64() const {
  if (type_ != DType::kI64) throw std::logic_error("Array: not int64");
  return static_cast<std::int64_t*>(data_);
}

std::int8_t* Array::i8() const {
  if (type_ != DType::kI8) throw std::logic_error("Array: not int8");
  return static_cast<std::int8_t*>(data_);
}

namespace {

void upload_bytes(const Context& ctx, void* dst, const void* src, std::size_t bytes) {
  check(uocr_rocm_memcpy(dst, src, bytes, UOCR_ROCM_H2D, ctx.stream()));
  ctx.synchronize();  // the host buffer may go away when the caller returns
}

void check_range(std::int64_t offset, std::int64_t count, std::int64_t size) {
  if (offset < 0 || count < 0 || offset + count > size) throw std::out_of_range("Array::upload past the end");
}

}  // namespace

void Array::upload(const float* host, std::int64_t count, std::int64_t offset) {
  check_range(offset, count, count_);
  if (type_ == DType::kF32) {
    upload_bytes(*ctx_, f32() + offset, host, static_cast<std::size_t>(count) * 4);
    return;
  }
  std::vector<std::uint16_t> staged(static_cast<std::size_t>(count));
  for (std::int64_t i = 0; i < count; ++i) staged[static_cast<std::size_t>(i)] = f32_to_bf16(host[i]);
  upload_bytes(*ctx_, bf16() + offset, staged.data(), staged.size() * 2);
}

void Array::upload(const std::uint16_t* host, std::int64_t count, std::int64_t offset) {
  check_range(offset, count, count_);
  upload_bytes(*ctx_, bf16() + offset, host, static_cast<std::size_t>(count) * 2);
}

void Array::upload(const std::int64_t* host, std::int64_t count, std::int64_t offset) {
  check_range(offset, count, count_);
  upload_bytes(*ctx_, i64() + offset, host, static_cast<std::size_t>(count) * 8);
}

void Array::upload(const std::int8_t* host, std::int64_t count, std::int64_t offset) {
  check_range(offset, count, count_);
  upload_bytes(*ctx_, i8() + offset, host, static_cast<std::size_t>(count));
}

std::vector<float> Array::download() const {
  if (type_ == DType::kI64 || type_ == DType::kI8) {
    throw std::logic_error("Array::download: integer arrays are not widened");
  }
  std::vector<float> out(static_cast<std::size_t>(count_));
  if (type_ == DType::kF32) {
    check(uocr_rocm_memcpy(out.data(), data_, out.size() * 4, UOCR_ROCM_D2H, ctx_->stream()));
    ctx_->synchronize();
    return out;
  }
  const std::vector<std::uint16_t> bits = download_bf16();
  for (std::size_t i = 0; i < out.size(); ++i) out[i] = bf16_to_f32(bits[i]);
  return out;
}

std::vector<std::uint16_t> Array::download_bf16() const {
  std::vector<std::uint16_t> out(static_cast<std::size_t>(count_));
  check(uocr_rocm_memcpy(out.data(), bf16(), out.size() * 2, UOCR_ROCM_D2H, ctx_->stream()));
  ctx_->synchronize();
  return out;
}

void Array::zero() {
  check(uocr_rocm_zero(data_, static_cast<std::size_t>(count_) * element_bytes(type_), ctx_->stream()));
}

}  // namespace uocr::rocm
