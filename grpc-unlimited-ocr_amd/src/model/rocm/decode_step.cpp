#include "model/rocm/decode_step.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <utility>

#include "backend/rocm/decode_ops.h"
#include "backend/rocm/ops.h"

namespace uocr::rocm {

DecodeStep::DecodeStep(const Context& ctx, const DecoderDims& dims, const std::uint16_t* embed,
                                 std::vector<LayerWeights> layers, const float* final_norm,
                                 const std::uint16_t* lm_head)
    : ctx_(ctx),
      dims_(dims),
      embed_(embed),
      layers_(std::move(layers)),
      final_norm_(final_norm),
      lm_head_(lm_head) {
  const auto& d = dims_;
  if (d.hidden <= 0 || d.heads <= 0 || d.head_dim <= 0 || d.vocab <= 0 || d.capacity <= 0) {
    throw std::invalid_argument("DecodeStep: every dimension must be positive");
  }
  if (d.head_dim % 2 != 0) throw std::invalid_argument("DecodeStep: head_dim must be even");
  if (embed_ == nullptr || final_norm_ == nullptr || lm_head_ == nullptr) {
    throw std::invalid_argument("DecodeStep: null embedding, final norm or LM head");
  }
  std::int64_t max_ffn = 1, max_experts = 1, max_k = 1, max_expert_ffn = 1;
  for (const auto& l : layers_) {
    if (l.input_norm == nullptr || l.qkv == nullptr || l.o == nullptr || l.post_norm == nullptr) {
      throw std::invalid_argument("DecodeStep: null layer weight");
    }
    if (l.moe == nullptr) {
      if (l.gate == nullptr || l.up == nullptr || l.down == nullptr || l.ffn <= 0) {
        throw std::invalid_argument("DecodeStep: a dense layer needs gate, up, down and ffn > 0");
      }
      max_ffn = std::max(max_ffn, l.ffn);
    } else {
      const MoeWeights& m = *l.moe;
      if (m.gate == nullptr || m.gate_stack == nullptr || m.up_stack == nullptr || m.down_stack == nullptr ||
          m.shared_gate == nullptr || m.shared_up == nullptr || m.shared_down == nullptr || m.experts <= 0 ||
          m.top_k <= 0 || m.top_k > m.experts || m.expert_ffn <= 0 || m.shared_ffn <= 0) {
        throw std::invalid_argument("DecodeStep: incomplete mixture-of-experts layer");
      }
      max_ffn = std::max(max_ffn, m.shared_ffn);
      max_experts = std::max(max_experts, m.experts);
      max_k = std::max(max_k, m.top_k);
      max_expert_ffn = std::max(max_expert_ffn, m.expert_ffn);
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
  h_ = f32(d.hidden);
  delta_ = f32(d.hidden);
  qkv_ = f32(3 * width);
  attn_ = f32(width);
  o_ = f32(d.hidden);
  act_ = f32(max_ffn);
  router_logits_ = f32(max_experts);
  expert_ids_ = Array(ctx_, DType::kI64, max_k);
  expert_weights_ = f32(max_k);
  expert_scratch_ = f32(std::max<std::int64_t>(1, expert_scratch_floats(max_k, max_expert_ffn)));
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

DecodeStep::~DecodeStep() = default;

void DecodeStep::reset() {
  for (auto& c : k_cache_) c.zero();
  for (auto& c : v_cache_) c.zero();
  ctx_.synchronize();
}

void DecodeStep::body() {
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
    const LayerWeights& l = layers_[li];
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
    if (l.moe == nullptr) {
      add_rms_norm_swiglu_gemv_bf16(ctx_, x_[cur].f32(), o_.f32(), x_[1 - cur].f32(), l.post_norm, d.eps, nullptr,
                                    d.hidden, l.gate, l.up, l.ffn, act_.f32());
      cur = 1 - cur;
      gemv_bf16(ctx_, act_.f32(), l.ffn, l.down, d.hidden, nullptr, delta_.f32());
    } else {
      // The shared experts' gate/up and the router's logits on h in one
      // launch (the fused prologue also writes h for the routed experts),
      // then the routed experts' sum added to the shared experts' down
      // product (cuda_decoder.cpp:137-152).
      const MoeWeights& m = *l.moe;
      add_rms_norm_swiglu_router_gemv_bf16(ctx_, x_[cur].f32(), o_.f32(), x_[1 - cur].f32(), l.post_norm, d.eps,
                                           h_.f32(), d.hidden, m.shared_gate, m.shared_up, m.shared_ffn, act_.f32(),
                                           m.gate, m.experts, router_logits_.f32());
      cur = 1 - cur;
      moe_ffn_one(ctx_, h_.f32(), d.hidden, m.expert_ffn, m.gate_stack, m.up_stack, m.down_stack, m.experts,
                  router_logits_.f32(), m.top_k, expert_ids_.i64(), expert_weights_.f32(), act_.f32(), m.shared_down,
                  m.shared_ffn, expert_scratch_.f32(), delta_.f32());
    }
    pending = delta_.f32();
  }
  add_rms_norm_gemv_bf16(ctx_, x_[cur].f32(), pending, nullptr, final_norm_, d.eps, nullptr, d.hidden, lm_head_,
                         d.vocab, nullptr, logits_.f32());
}

void DecodeStep::set_state(std::int64_t token, std::int64_t pos) {
  if (token < 0 || token >= dims_.vocab) throw std::invalid_argument("DecodeStep: token outside the vocabulary");
  if (pos < 0 || pos >= dims_.capacity) throw std::invalid_argument("DecodeStep: position outside the cache");
  const StepState s{token, pos, pos, 0, -1};
  std::memcpy(state_host_->data(), &s, sizeof s);
  copy_to_device(ctx_, state_.data(), *state_host_, sizeof s);
}

void DecodeStep::replay() { graph_->launch(); }

std::vector<float> DecodeStep::step(std::int64_t token, std::int64_t pos) {
  set_state(token, pos);
  replay();
  copy_to_host(ctx_, *logits_host_, logits_.data(), logits_host_->bytes());
  ctx_.synchronize();
  const auto* l = static_cast<const float*>(logits_host_->data());
  return {l, l + dims_.vocab};
}

}  // namespace uocr::rocm
