#include "backend/rocm/context.h"

#include <stdexcept>
#include <string>

#include "backend/rocm/dtype.h"
#include "uocr_rocm.h"

namespace uocr::rocm {
namespace {

// Bytes per element, indexed by the DType enumerator's value.
constexpr std::size_t kElementBytes[] = {4, 2, 8, 1};  // kF32, kBF16, kI64, kI8
static_assert(static_cast<int>(DType::kF32) == 0 && static_cast<int>(DType::kBF16) == 1 &&
              static_cast<int>(DType::kI64) == 2 && static_cast<int>(DType::kI8) == 3);

constexpr std::size_t bytes_of(DType t) { return kElementBytes[static_cast<std::size_t>(t)]; }

const char* type_name(DType t) {
  constexpr const char* kNames[] = {"fp32", "bf16", "int64", "int8"};
  return kNames[static_cast<std::size_t>(t)];
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

void copy_on_device(const Context& ctx, void* device_dst, const void* device_src, std::size_t bytes) {
  if (bytes == 0) return;
  check(uocr_rocm_memcpy(device_dst, device_src, bytes, UOCR_ROCM_D2D, ctx.stream()));
}

Array::Array(const Context& ctx, DType type, std::int64_t count)
    : ctx_(&ctx), block_(nullptr, StreamRelease{ctx.stream()}), count_(count), type_(type) {
  if (count < 0) throw std::invalid_argument("Array: the element count must not be negative");
  void* p = nullptr;
  check(uocr_rocm_malloc(&p, static_cast<std::size_t>(count) * bytes_of(type), ctx.stream()));
  block_.reset(p);
}

void StreamRelease::operator()(void* p) const noexcept {
  if (p != nullptr) (void)uocr_rocm_free(p, stream);
}

void Array::type_mismatch(DType want) const {
  throw std::logic_error(std::string("Array: a ") + type_name(want) + " view of an array of " + type_name(type_) +
                         " elements");
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
    check(uocr_rocm_memcpy(out.data(), data(), out.size() * 4, UOCR_ROCM_D2H, ctx_->stream()));
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
  check(uocr_rocm_zero(data(), static_cast<std::size_t>(count_) * bytes_of(type_), ctx_->stream()));
}

}  // namespace uocr::rocm
