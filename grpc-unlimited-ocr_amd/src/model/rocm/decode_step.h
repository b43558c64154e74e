#pragma once

// A whole decode step of the decoder on the rocm backend, captured once as
// a graph and replayed per token, as the reference's CudaDecoder::step
// replays decode_body (src/model/cuda/cuda_decoder.cpp:295-331,
// src/model/cuda/cuda_decode_step.cpp:47-70): the embedding row, every
// layer's attention and MLP with their residual adds and norms, the final
// norm and the LM head, with only the StepState rewritten between tokens.
//
// A layer is the reference's decode layer with rotary attention over the
// whole cache:
//   h = rms(x) w_in;  q, k, v = h Wq, h Wk, h Wv;  rope(q, k) at pos;
//   append k, v;  attn = softmax(q K^T / sqrt(hd)) V;  x += attn Wo;
//   h = rms(x) w_post;  x += mlp(h)
// where mlp is dense, silu(h Wg) * (h Wu) Wd (layer.dense,
// cuda_decoder.cpp:119-124), or a mixture of experts (cuda_decoder.cpp:
// 137-152): the shared experts' MLP plus sum_j s_j expert_j(h) over the top
// k experts of softmax(h W_gate) (fp32 gate). After the last layer logits =
// (rms(x) w_final) W_lm. The reference's block routing (the attention mask
// from summary/scores/route steps) and int8 weights are not part of it.
//
// Launches per step: 1 + per layer 6 (dense) or 7 (mixture of experts) +
// 1. The residual add of each sublayer is the prologue of the next
// projection (the fused GEMVs), rope + both appends + attention are one op
// of two launches, the router's logits are formed in the shared experts'
// gate/up launch, the top k inside the routed experts' gate/up launch, and
// the shared experts' down product and the routed experts' sum in the routed
// experts' down launch.

#include <cstdint>
#include <memory>
#include <vector>

#include "backend/rocm/context.h"

namespace uocr::rocm {

struct DecoderDims {
  std::int64_t hidden = 1280;
  std::int64_t heads = 10;
  std::int64_t head_dim = 128;
  std::int64_t vocab = 129280;
  std::int64_t capacity = 8192;  // key/value positions per layer
  float eps = 1e-6f;
  double rope_theta = 1e4;
  bool bf16_cache = true;  // key/value cache in bf16 (else fp32)
};

// A mixture-of-experts MLP, device weights owned by the caller.
struct MoeWeights {
  const float* gate = nullptr;           // [experts, hidden] fp32 router
  const std::uint16_t* up_stack = nullptr;    // [experts * expert_ffn, hidden]
  const std::uint16_t* gate_stack = nullptr;  // [experts * expert_ffn, hidden]
  const std::uint16_t* down_stack = nullptr;  // [experts * hidden, expert_ffn]
  std::int64_t experts = 64;
  std::int64_t top_k = 6;
  std::int64_t expert_ffn = 896;
  const std::uint16_t* shared_gate = nullptr;  // [shared_ffn, hidden]
  const std::uint16_t* shared_up = nullptr;    // [shared_ffn, hidden]
  const std::uint16_t* shared_down = nullptr;  // [hidden, shared_ffn]
  std::int64_t shared_ffn = 1792;
};

// Device weights of one layer, owned by the caller (bf16 bits, fp32 norms).
// The MLP is dense (gate, up, down, ffn) unless moe is set.
struct LayerWeights {
  const float* input_norm = nullptr;   // [hidden]
  const std::uint16_t* qkv = nullptr;  // [3 * heads * head_dim, hidden]: Wq, Wk, Wv rows stacked
  const std::uint16_t* o = nullptr;    // [hidden, heads * head_dim]
  const float* post_norm = nullptr;    // [hidden]
  const std::uint16_t* gate = nullptr;  // [ffn, hidden]
  const std::uint16_t* up = nullptr;    // [ffn, hidden]
  const std::uint16_t* down = nullptr;  // [hidden, ffn]
  std::int64_t ffn = 896;
  const MoeWeights* moe = nullptr;
};

class DecodeStep {
 public:
  // embed [vocab, hidden] bf16, final_norm [hidden], lm_head [vocab, hidden]
  // bf16; every pointer (and every MoeWeights) stays owned by the caller and
  // must outlive this.
  DecodeStep(const Context& ctx, const DecoderDims& dims, const std::uint16_t* embed, std::vector<LayerWeights> layers,
             const float* final_norm, const std::uint16_t* lm_head);
  ~DecodeStep();
  DecodeStep(const DecodeStep&) = delete;
  DecodeStep& operator=(const DecodeStep&) = delete;

  // Feeds `token` at position `pos` (its rope coordinate; keys 0..pos are
  // attended, pos < capacity) and returns the logits [vocab].
  std::vector<float> step(std::int64_t token, std::int64_t pos);

  // Enqueues one replay on the context's stream without reading the logits
  // back (for timing); the StepState must have been set by set_state. The
  // state goes through one pinned host buffer: call set_state again only
  // after the stream has taken the previous copy (step() synchronises).
  void set_state(std::int64_t token, std::int64_t pos);
  void replay();
  // Zeroes every layer's cache (a new sequence).
  void reset();

 private:
  void body();

  const Context& ctx_;
  DecoderDims dims_;
  const std::uint16_t* embed_;
  std::vector<LayerWeights> layers_;
  const float* final_norm_;
  const std::uint16_t* lm_head_;
  Array inv_tok_, state_, x_[2], h_, delta_, qkv_, attn_, o_, act_, logits_, scratch_;
  Array router_logits_, expert_ids_, expert_weights_, expert_scratch_;
  std::vector<Array> k_cache_, v_cache_;
  std::unique_ptr<PinnedBuffer> state_host_, logits_host_;
  std::unique_ptr<Graph> graph_;
};

}  // namespace uocr::rocm
