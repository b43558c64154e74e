#include "model/rocm/decode_step.h"

#include <algorithm>
#include <cmath>
#include <cstring>
#include <stdexcept>
#include <string>
#include <utility>

#include "backend/rocm/decode_ops.h"

namespace uocr::rocm {
namespace {

// Work queued between construction and finish() is recorded into a graph;
// when the scope is left by an exception, the capture is ended and its
// partial graph dropped, so the stream can take ordinary work again.
class CaptureScope {
 public:
  explicit CaptureScope(const Context& ctx) : ctx_(ctx) { ctx_.begin_capture(); }
  ~CaptureScope() {
    if (open_) {
      try {
        (void)ctx_.end_capture();
      } catch (...) {
      }
    }
  }
  CaptureScope(const CaptureScope&) = delete;
  CaptureScope& operator=(const CaptureScope&) = delete;
  std::unique_ptr<Graph> finish() {
    open_ = false;
    return ctx_.end_capture();
  }

 private:
  const Context& ctx_;
  bool open_ = true;
};

void need(bool ok, const char* what) {
  if (!ok) throw std::invalid_argument(std::string("DecodeStep: ") + what);
}

bool aligned16(const void* p) { return (reinterpret_cast<std::uintptr_t>(p) & 15u) == 0; }

// The frequencies of PageRope (src/model/page_rope.cpp:9-24): float(1 /
// theta^(i / n)) for i < n, in double.
std::vector<float> rope_table(std::int64_t n, double theta) {
  std::vector<float> inv(static_cast<std::size_t>(n));
  for (std::int64_t i = 0; i < n; ++i) {
    inv[static_cast<std::size_t>(i)] =
        static_cast<float>(1.0 / std::pow(theta, static_cast<double>(i) / static_cast<double>(n)));
  }
  return inv;
}

// The fused norm-prologue GEMVs keep bf16(h) in registers, and the expert
// kernels stage their activations in LDS: the widths they take.
constexpr std::int64_t kFusedMaxK = 2048;
constexpr std::int64_t kGemvMaxK = 12288;
constexpr std::int64_t kMaxExperts = 128, kMaxExpertSlots = 8, kExpertActFloats = 8192;
// The router's launch: block keys staged in LDS, scores of every block.
constexpr std::int64_t kMaxBlockKeys = 64, kMaxIndexDim = 256, kStageFloats = 8192, kMaxTop = 32,
                       kMaxRouteBlocks = 4096, kMaxHeadDim = 256;

bool fused_width(std::int64_t n) { return n % 8 == 0 && n >= 8 && n <= kFusedMaxK; }

}  // namespace

DecodeStep::DecodeStep(const Context& ctx, const DecoderDims& dims, const std::uint16_t* embed,
                       std::vector<LayerWeights> layers, const float* final_norm, const std::uint16_t* lm_head)
    : ctx_(ctx),
      dims_(dims),
      embed_(embed),
      layers_(std::move(layers)),
      final_norm_(final_norm),
      lm_head_(lm_head) {
  validate();
  const auto& d = dims_;
  capacity_blocks_ = (d.capacity + d.router.block_size - 1) / d.router.block_size;
  for (const auto& l : layers_) {
    const bool moe = l.moe != nullptr;
    const std::int64_t f = moe ? l.moe->shared_ffn : l.ffn, part = f * d.hidden;
    Array gu(ctx_, DType::kBF16, 2 * part);
    const auto bytes = static_cast<std::size_t>(part) * sizeof(std::uint16_t);
    copy_on_device(ctx_, gu.bf16(), moe ? l.moe->shared_gate : l.gate, bytes);
    copy_on_device(ctx_, gu.bf16() + part, moe ? l.moe->shared_up : l.up, bytes);
    gate_up_.push_back(std::move(gu));
  }
  std::int64_t max_ffn = 1, max_experts = 1, max_k = 1, max_expert_ffn = 1;
  for (const auto& l : layers_) {
    if (l.moe == nullptr) {
      max_ffn = std::max(max_ffn, l.ffn);
    } else {
      max_ffn = std::max(max_ffn, l.moe->shared_ffn);
      max_experts = std::max(max_experts, l.moe->experts);
      max_k = std::max(max_k, l.moe->top_k);
      max_expert_ffn = std::max(max_expert_ffn, l.moe->expert_ffn);
    }
  }
  const std::int64_t width = d.heads * d.head_dim, half = d.head_dim / 2, n_tok = half - d.page_pairs;
  auto f32 = [&](std::int64_t n) { return Array(ctx_, DType::kF32, n); };
  const auto tok = rope_table(n_tok, d.rope_theta);
  inv_tok_ = f32(std::max<std::int64_t>(n_tok, 1));
  if (n_tok > 0) inv_tok_.upload(tok.data(), n_tok);
  if (d.page_pairs > 0) {
    const auto page = rope_table(d.page_pairs, d.page_theta);
    inv_page_ = f32(d.page_pairs);
    inv_page_.upload(page.data(), d.page_pairs);
  }
  state_ = Array(ctx_, DType::kI64, 5);
  x_[0] = f32(d.hidden);
  x_[1] = f32(d.hidden);
  h_ = f32(d.hidden);
  delta_ = f32(d.hidden);
  proj_ = f32(3 * width + 2 * d.index_dim);
  o_ = f32(d.hidden);
  act_ = f32(max_ffn);
  router_logits_ = f32(max_experts);
  expert_ids_ = Array(ctx_, DType::kI64, max_k);
  expert_weights_ = f32(max_k);
  expert_scratch_ = f32(std::max<std::int64_t>(1, expert_scratch_floats(max_k, max_expert_ffn)));
  logits_ = f32(d.vocab);
  max_live_ = std::max<std::int64_t>(1, std::min(max_live_keys(d.router), d.capacity));
  scratch_ = f32(attend_segments_scratch_floats(d.heads, d.head_dim, max_live_));
  segments_ = f32(kKeySegmentWords);  // int32 words
  block_min_ = Array(ctx_, DType::kI64, capacity_blocks_);
  block_max_ = Array(ctx_, DType::kI64, capacity_blocks_);
  const DType cache_type = d.bf16_cache ? DType::kBF16 : DType::kF32;
  for (std::size_t i = 0; i < layers_.size(); ++i) {
    k_cache_.emplace_back(ctx_, cache_type, d.capacity * width);
    v_cache_.emplace_back(ctx_, cache_type, d.capacity * width);
    router_keys_.emplace_back(ctx_, DType::kF32, d.capacity * d.index_dim);
    summaries_.emplace_back(ctx_, DType::kF32, capacity_blocks_ * d.index_dim);
    if (d.trace) {
      trace_x_in_.push_back(f32(d.hidden));
      trace_rqk_.push_back(f32(2 * d.index_dim));
      trace_z_.push_back(f32(capacity_blocks_));
      trace_mask_.push_back(f32(d.capacity));
      trace_x_mid_.push_back(f32(d.hidden));
    }
  }
  reset();
  state_host_ = std::make_unique<PinnedBuffer>(sizeof(StepState));
  logits_host_ = std::make_unique<PinnedBuffer>(static_cast<std::size_t>(d.vocab) * sizeof(float));
  record();
}

DecodeStep::~DecodeStep() = default;

void DecodeStep::validate() const {
  const auto& d = dims_;
  const auto& r = d.router;
  need(d.hidden > 0 && d.heads > 0 && d.head_dim > 0 && d.vocab > 0 && d.capacity > 0 && d.index_dim > 0,
       "every dimension must be positive");
  need(fused_width(d.hidden), "hidden must be a multiple of 8 in [8, 2048]");
  need(d.head_dim % 2 == 0 && d.head_dim <= kMaxHeadDim, "head_dim must be even and at most 256");
  need(d.heads * d.head_dim <= kGemvMaxK, "heads * head_dim above 12288");
  need(d.index_dim == d.head_dim, "index_dim must equal head_dim (the router keys share the rope table)");
  need(d.index_dim % 4 == 0 && d.index_dim <= kMaxIndexDim, "index_dim must be a multiple of 4 in [4, 256]");
  need(d.page_pairs >= 0 && d.page_pairs < d.head_dim / 2, "page_pairs must leave room for token pairs");
  need(d.page_mod >= 0, "page_mod must be >= 0");
  need(r.block_size >= 1 && r.block_size <= kMaxBlockKeys, "router block_size must be in [1, 64]");
  need(r.block_size * d.index_dim <= kStageFloats, "router block_size * index_dim above 8192");
  need((d.capacity + r.block_size - 1) / r.block_size <= kMaxRouteBlocks, "capacity / block_size above 4096");
  need(r.local_blocks >= 0 && r.local_blocks < (std::int64_t{1} << 24), "router local_blocks out of range");
  need(r.top_m >= 1 && r.top_m <= kMaxTop, "router top_m must be in [1, 32]");
  need(r.top_k >= 1 && r.top_k < (std::int64_t{1} << 24), "router top_k must be >= 1");
  need(r.sigma != 0.0f, "router sigma must not be 0");
  need(embed_ != nullptr && final_norm_ != nullptr && lm_head_ != nullptr, "null embedding, final norm or LM head");
  need(aligned16(embed_) && aligned16(lm_head_), "the embedding and LM head must be 16-byte aligned");
  for (const auto& l : layers_) {
    need(l.input_norm != nullptr && l.qkv != nullptr && l.o != nullptr && l.post_norm != nullptr &&
             l.router_q_norm != nullptr && l.router_k_norm != nullptr && l.head_cls != nullptr,
         "null layer weight");
    need(aligned16(l.qkv) && aligned16(l.o), "layer weights must be 16-byte aligned");
    if (l.moe == nullptr) {
      need(l.gate != nullptr && l.up != nullptr && l.down != nullptr, "a dense layer needs gate, up and down");
      need(l.ffn >= 8 && l.ffn % 8 == 0 && l.ffn <= kGemvMaxK, "a dense layer's ffn must be a multiple of 8 in "
                                                              "[8, 12288]");
      need(aligned16(l.gate) && aligned16(l.up) && aligned16(l.down), "layer weights must be 16-byte aligned");
      continue;
    }
    const MoeWeights& m = *l.moe;
    need(m.gate != nullptr && m.gate_stack != nullptr && m.up_stack != nullptr && m.down_stack != nullptr &&
             m.shared_gate != nullptr && m.shared_up != nullptr && m.shared_down != nullptr,
         "incomplete mixture-of-experts layer");
    need(aligned16(m.gate) && aligned16(m.gate_stack) && aligned16(m.up_stack) && aligned16(m.down_stack) &&
             aligned16(m.shared_gate) && aligned16(m.shared_up) && aligned16(m.shared_down),
         "expert weights must be 16-byte aligned");
    need(m.experts >= 1 && m.experts <= kMaxExperts, "experts must be in [1, 128]");
    need(m.top_k >= 1 && m.top_k <= kMaxExpertSlots && m.top_k <= m.experts, "top_k must be in [1, min(8, experts)]");
    need(fused_width(m.expert_ffn), "expert_ffn must be a multiple of 8 in [8, 2048]");
    need(fused_width(m.shared_ffn), "shared_ffn must be a multiple of 8 in [8, 2048]");
    need(m.top_k * m.expert_ffn + m.shared_ffn <= kExpertActFloats, "top_k * expert_ffn + shared_ffn above 8192");
  }
}

void DecodeStep::record() {
  graph_.reset();
  ctx_.synchronize();
  CaptureScope capture(ctx_);
  body();
  graph_ = capture.finish();
}

void DecodeStep::reset() {
  for (auto& c : k_cache_) c.zero();
  for (auto& c : v_cache_) c.zero();
  for (auto& c : router_keys_) c.zero();
  for (auto& c : summaries_) c.zero();
  ctx_.synchronize();
  length_ = 0;
  last_pos_ = -1;
}

void DecodeStep::reserve(std::int64_t keys) {
  if (keys <= dims_.capacity) return;
  auto& d = dims_;
  const std::int64_t bs = d.router.block_size;
  const std::int64_t capacity = std::max<std::int64_t>(keys, d.capacity * 2 + 1024);
  const std::int64_t blocks = (capacity + bs - 1) / bs;
  need(blocks <= kMaxRouteBlocks, "the cache cannot grow past 4096 router blocks");
  const std::int64_t width = d.heads * d.head_dim, used_blocks = (length_ + bs - 1) / bs;
  // A zeroed array of `count` elements with the first `keep` of `a`'s.
  auto grow = [&](Array& a, DType type, std::int64_t count, std::int64_t keep, std::size_t elem_bytes) {
    Array bigger(ctx_, type, count);
    bigger.zero();
    copy_on_device(ctx_, bigger.data(), a.data(), static_cast<std::size_t>(keep) * elem_bytes);
    a = std::move(bigger);
  };
  const DType cache_type = d.bf16_cache ? DType::kBF16 : DType::kF32;
  const std::size_t cache_bytes = d.bf16_cache ? 2 : 4;
  for (std::size_t i = 0; i < layers_.size(); ++i) {
    grow(k_cache_[i], cache_type, capacity * width, length_ * width, cache_bytes);
    grow(v_cache_[i], cache_type, capacity * width, length_ * width, cache_bytes);
    grow(router_keys_[i], DType::kF32, capacity * d.index_dim, length_ * d.index_dim, 4);
    grow(summaries_[i], DType::kF32, blocks * d.index_dim, used_blocks * d.index_dim, 4);
    if (d.trace) {
      trace_z_[i] = Array(ctx_, DType::kF32, blocks);
      trace_mask_[i] = Array(ctx_, DType::kF32, capacity);
    }
  }
  grow(block_min_, DType::kI64, blocks, prompt_blocks_, 8);
  grow(block_max_, DType::kI64, blocks, prompt_blocks_, 8);
  max_live_ = std::max<std::int64_t>(1, std::min(max_live_keys(d.router), capacity));
  scratch_ = Array(ctx_, DType::kF32, attend_segments_scratch_floats(d.heads, d.head_dim, max_live_));
  d.capacity = capacity;
  capacity_blocks_ = blocks;
  record();  // the buffers moved: the captured step is recorded again
}

void DecodeStep::set_prompt_blocks(const std::vector<std::int64_t>& min_page,
                                   const std::vector<std::int64_t>& max_page) {
  const auto n = static_cast<std::int64_t>(min_page.size());
  need(max_page.size() == min_page.size(), "min_page and max_page differ in length");
  need(n <= capacity_blocks_, "more prompt blocks than the cache holds");
  if (n > 0) {
    block_min_.upload(min_page.data(), n);
    block_max_.upload(max_page.data(), n);
  }
  prompt_blocks_ = n;
  record();
}

void DecodeStep::body() {
  const auto& d = dims_;
  const std::int64_t width = d.heads * d.head_dim, half = d.head_dim / 2, n_tok = half - d.page_pairs;
  const auto* st = reinterpret_cast<const StepState*>(state_.data());
  const float scale = 1.0f / std::sqrt(static_cast<float>(d.head_dim));
  const float* inv_page = d.page_pairs > 0 ? inv_page_.f32() : nullptr;
  const std::int64_t* block_min = prompt_blocks_ > 0 ? block_min_.i64() : nullptr;
  const std::int64_t* block_max = prompt_blocks_ > 0 ? block_max_.i64() : nullptr;
  // x_[cur] holds the residual stream; a fused prologue that adds a sublayer's
  // output writes the sum to the other buffer (its output must not overlap
  // its inputs).
  int cur = 0;
  embed_step(ctx_, embed_, st, d.hidden, x_[cur].f32());
  const float* pending = nullptr;  // the previous MLP's output, not yet added
  float* q = proj_.f32();
  float* k = q + width;
  float* v = k + width;
  float* rq = v + width;
  float* rk = rq + d.index_dim;
  auto* segs = reinterpret_cast<std::int32_t*>(segments_.data());
  for (std::size_t li = 0; li < layers_.size(); ++li) {
    const LayerWeights& l = layers_[li];
    float* sum = pending != nullptr ? x_[1 - cur].f32() : nullptr;
    add_rms_norm_gemv_bf16(ctx_, x_[cur].f32(), pending, sum, l.input_norm, d.eps, nullptr, d.hidden, l.qkv,
                           3 * width + 2 * d.index_dim, nullptr, q);
    if (pending != nullptr) cur = 1 - cur;
    if (d.trace) copy(ctx_, trace_x_in_[li].f32(), x_[cur].f32(), d.hidden);
    // The router half (cuda_decode_step.cpp:22-40): norms, rope, the router
    // key's append, the block's summary, the scores and the key mask.
    route_decode_step(ctx_, rq, rk, l.router_q_norm, l.router_k_norm, d.eps, inv_tok_.f32(), n_tok, inv_page,
                      d.page_mod, l.head_cls, router_keys_[li].f32(), summaries_[li].f32(), d.index_dim, block_min,
                      block_max, prompt_blocks_, st, d.router, d.capacity,
                      d.trace ? trace_mask_[li].f32() : nullptr, d.trace ? trace_z_[li].f32() : nullptr,
                      d.trace ? trace_rqk_[li].f32() : nullptr, segs);
    // The attention's splits leave their records in scratch_; the o
    // projection merges them in its prologue (no merge launch).
    if (d.bf16_cache) {
      attend_rope_kv_step_segments_bf16(ctx_, q, k, v, k_cache_[li].bf16(), v_cache_[li].bf16(), d.heads, d.head_dim,
                                        segs, max_live_, scale, st, inv_tok_.f32(), n_tok, inv_page, d.page_mod,
                                        scratch_.f32(), d.capacity, nullptr);
    } else {
      attend_rope_kv_step_segments(ctx_, q, k, v, k_cache_[li].f32(), v_cache_[li].f32(), d.heads, d.head_dim, segs,
                                   max_live_, scale, st, inv_tok_.f32(), n_tok, inv_page, d.page_mod, scratch_.f32(),
                                   d.capacity, nullptr);
    }
    attend_merge_gemv_bf16(ctx_, scratch_.f32(), d.heads, d.head_dim, max_live_, l.o, d.hidden, nullptr, o_.f32());
    if (l.moe == nullptr) {
      add_rms_norm_swiglu_gemv_bf16(ctx_, x_[cur].f32(), o_.f32(), x_[1 - cur].f32(), l.post_norm, d.eps, nullptr,
                                    d.hidden, l.gate, l.up, l.ffn, act_.f32());
      cur = 1 - cur;
      if (d.trace) copy(ctx_, trace_x_mid_[li].f32(), x_[cur].f32(), d.hidden);
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
      if (d.trace) copy(ctx_, trace_x_mid_[li].f32(), x_[cur].f32(), d.hidden);
      moe_ffn_one(ctx_, h_.f32(), d.hidden, m.expert_ffn, m.gate_stack, m.up_stack, m.down_stack, m.experts,
                  router_logits_.f32(), m.top_k, expert_ids_.i64(), expert_weights_.f32(), act_.f32(), m.shared_down,
                  m.shared_ffn, expert_scratch_.f32(), delta_.f32());
    }
    pending = delta_.f32();
  }
  add_rms_norm_gemv_bf16(ctx_, x_[cur].f32(), pending, nullptr, final_norm_, d.eps, nullptr, d.hidden, lm_head_,
                         d.vocab, nullptr, logits_.f32());
}

void DecodeStep::set_state(std::int64_t token, std::int64_t pos, RopeCoord coord, std::int64_t query_page) {
  need(token >= 0 && token < dims_.vocab, "token outside the vocabulary");
  need(pos >= 0 && pos < dims_.capacity, "position outside the cache");
  const StepState s{token, pos, coord.tok, coord.page, query_page < 0 ? -1 : query_page};
  std::memcpy(state_host_->data(), &s, sizeof s);
  copy_to_device(ctx_, state_.data(), *state_host_, sizeof s);
  last_pos_ = pos;
}

void DecodeStep::replay() { graph_->launch(); }

std::vector<float> DecodeStep::step(std::int64_t token, RopeCoord coord, std::int64_t query_page) {
  set_state(token, length_, coord, query_page);
  replay();
  copy_to_host(ctx_, *logits_host_, logits_.data(), logits_host_->bytes());
  ctx_.synchronize();
  ++length_;
  const auto* l = static_cast<const float*>(logits_host_->data());
  return {l, l + dims_.vocab};
}

const std::vector<std::vector<float>>& DecodeStep::prefill_trace() const {
  if (!dims_.trace) throw std::logic_error("DecodeStep::prefill_trace: built without DecoderDims::trace");
  return prefill_masks_;
}

std::vector<LayerTrace> DecodeStep::trace() const {
  if (!dims_.trace) throw std::logic_error("DecodeStep::trace: built without DecoderDims::trace");
  if (last_pos_ < 0) throw std::logic_error("DecodeStep::trace: no step yet");
  const std::int64_t d = dims_.index_dim, pos = last_pos_;
  const std::int64_t remote = pos / dims_.router.block_size - dims_.router.local_blocks + 1;
  std::vector<LayerTrace> out(layers_.size());
  for (std::size_t li = 0; li < layers_.size(); ++li) {
    LayerTrace& t = out[li];
    t.x_in = trace_x_in_[li].download();
    const auto rqk = trace_rqk_[li].download();
    t.rq.assign(rqk.begin(), rqk.begin() + d);
    t.rk.assign(rqk.begin() + d, rqk.end());
    const auto z = trace_z_[li].download();
    t.z.assign(z.begin(), z.begin() + std::max<std::int64_t>(remote, 0));
    const auto mask = trace_mask_[li].download();
    t.mask.assign(mask.begin(), mask.begin() + pos + 1);
    t.x_mid = trace_x_mid_[li].download();
  }
  return out;
}

}  // namespace uocr::rocm
