#include "model/rocm/dense_decode_step.h"

#include <cmath>
#include <cstring>
#include <stdexcept>
#include <utility>

#include "backend/rocm/decode_ops.h"
#include "backend/rocm/ops.h"

namespace uocr::rocm {

DenseDecodeStep::DenseDecodeStep(const Context& ctx, const DenseDecoderDims& dims, const std::uint16_t* embed,
                                 std::vector<DenseLayerWeights> layers, const float* final_norm,
                                 const std::uint16_t* lm_head)
    : ctx_(ctx),
      dims_(dims),
      embed_(embed),
      layers_(std::move(layers)),
      final_norm_(final_norm),
      lm_head_(lm_head) {
  const auto& d = dims_;
  if (d.hidden <= 0 || d.heads <= 0 || d.head_dim <= 0 || d.ffn <= 0 || d.vocab <= 0 || d.capacity <= 0) {
    throw std::invalid_argument("DenseDecodeStep: every dimension must be positive");
  }
  if (d.head_dim % 2 != 0) throw std::invalid_argument("DenseDecodeStep: head_dim must be even");
  if (embed_ == nullptr || final_norm_ == nullptr || lm_head_ == nullptr) {
    throw std::invalid_argument("DenseDecodeStep: null embedding, final norm or LM head");
  }
  for (const auto& l : layers_) {
    if (l.input_norm == nullptr || l.qkv == nullptr || l.o == nullptr || l.post_norm == nullptr ||
        l.gate == nullptr || l.up == nullptr || l.down == nullptr) {
      throw std::invalid_argument("DenseDecodeStep: null layer weight");
    }
  }
  const std::int64_t width = d.heads * d.head_dim, half = d.head_dim / 2;
  // The token axis's frequency table, as PageRope builds it
  // (src/model/page_rope.cpp:17-19): float(1 / theta^(i / half)) in double.
  std::vector<float> inv(static_cast<std::size_t>(half));
  for (std::int64_t i = 0; i < half; ++i) {
    inv[static_cast<std::size_t>(i)] = static_cast<float>(
        1.0 / std::pow(d.rope_theta, static_cast<double>(i) / static_cast<double>(half)));
  }
  auto f32 = [&](std::int64_t n) { return Array(ctx_, DType::kF32, n); };
  inv_tok_ = f32(half);
  inv_tok_.upload(inv.data(), half);
  state_ = Array(ctx_, DType::kI64, 5);
  x_[0] = f32(d.hidden);
  x_[1] = f32(d.hidden);
  delta_ = f32(d.hidden);
  qkv_ = f32(3 * width);
  attn_ = f32(width);
  o_ = f32(d.hidden);
  act_ = f32(d.ffn);
  logits_ = f32(d.vocab);
  scratch_ = f32(attend_scratch_floats(d.heads, d.head_dim, d.capacity));
  const DType cache_type = d.bf16_cache ? DType::kBF16 : DType::kF32;
  for (std::size_t i = 0; i < layers_.size(); ++i) {
    k_cache_.emplace_back(ctx_, cache_type, d.capacity * width);
    v_cache_.emplace_back(ctx_, cache_type, d.capacity * width);
  }
  reset();
  state_host_ = std::make_unique<PinnedBuffer>(sizeof(StepState));
  logits_host_ = std::make_unique<PinnedBuffer>(static_cast<std::size_t>(d.vocab) * sizeof(float));
  ctx_.synchronize();
  ctx_.begin_capture();
  body();
  graph_ = ctx_.end_capture();
}

DenseDecodeStep::~DenseDecodeStep() = default;

void DenseDecodeStep::reset() {
  for (auto& c : k_cache_) c.zero();
  for (auto& c : v_cache_) c.zero();
  ctx_.synchronize();
}

void DenseDecodeStep::body() {
  const auto& d = dims_;
  const std::int64_t width = d.heads * d.head_dim, half = d.head_dim / 2;
  const auto* st = reinterpret_cast<const StepState*>(state_.data());
  const float scale = 1.0f / std::sqrt(static_cast<float>(d.head_dim));
  // x_[cur] holds the residual stream; a fused prologue that adds a sublayer's
  // output writes the sum to the other buffer (its output must not overlap
  // its inputs).
  int cur = 0;
  embed_step(ctx_, embed_, st, d.hidden, x_[cur].f32());
  const float* pending = nullptr;  // the previous MLP's output, not yet added
  float* q = qkv_.f32();
  float* k = q + width;
  float* v = k + width;
  for (std::size_t li = 0; li < layers_.size(); ++li) {
    const DenseLayerWeights& l = layers_[li];
    float* sum = pending != nullptr ? x_[1 - cur].f32() : nullptr;
    add_rms_norm_gemv_bf16(ctx_, x_[cur].f32(), pending, sum, l.input_norm, d.eps, nullptr, d.hidden, l.qkv,
                           3 * width, nullptr, q);
    if (pending != nullptr) cur = 1 - cur;
    if (d.bf16_cache) {
      attend_rope_kv_step_bf16(ctx_, q, k, v, k_cache_[li].bf16(), v_cache_[li].bf16(), d.heads, d.head_dim, nullptr,
                               scale, st, inv_tok_.f32(), half, nullptr, 0, scratch_.f32(), d.capacity, attn_.f32());
    } else {
      attend_rope_kv_step(ctx_, q, k, v, k_cache_[li].f32(), v_cache_[li].f32(), d.heads, d.head_dim, nullptr, scale,
                          st, inv_tok_.f32(), half, nullptr, 0, scratch_.f32(), d.capacity, attn_.f32());
    }
    gemv_bf16(ctx_, attn_.f32(), width, l.o, d.hidden, nullptr, o_.f32());
    add_rms_norm_swiglu_gemv_bf16(ctx_, x_[cur].f32(), o_.f32(), x_[1 - cur].f32(), l.post_norm, d.eps, nullptr,
                                  d.hidden, l.gate, l.up, d.ffn, act_.f32());
    cur = 1 - cur;
    gemv_bf16(ctx_, act_.f32(), d.ffn, l.down, d.hidden, nullptr, delta_.f32());
    pending = delta_.f32();
  }
  add_rms_norm_gemv_bf16(ctx_, x_[cur].f32(), pending, nullptr, final_norm_, d.eps, nullptr, d.hidden, lm_head_,
                         d.vocab, nullptr, logits_.f32());
}

void DenseDecodeStep::set_state(std::int64_t token, std::int64_t pos) {
  if (token < 0 || token >= dims_.vocab) throw std::invalid_argument("DenseDecodeStep: token outside the vocabulary");
  if (pos < 0 || pos >= dims_.capacity) throw std::invalid_argument("DenseDecodeStep: position outside the cache");
  const StepState s{token, pos, pos, 0, -1};
  std::memcpy(state_host_->data(), &s, sizeof s);
  copy_to_device(ctx_, state_.data(), *state_host_, sizeof s);
}

void DenseDecodeStep::replay() { graph_->launch(); }

std::vector<float> DenseDecodeStep::step(std::int64_t token, std::int64_t pos) {
  set_state(token, pos);
  replay();
  copy_to_host(ctx_, *logits_host_, logits_.data(), logits_host_->bytes());
  ctx_.synchronize();
  const auto* l = static_cast<const float*>(logits_host_->data());
  return {l, l + dims_.vocab};
}

}  // namespace uocr::rocm
