#pragma once

// A whole decode step of a dense decoder on the rocm backend, captured once
// as a graph and replayed per token, as the reference's CudaDecoder::step
// replays decode_body (src/model/cuda/cuda_decoder.cpp:295-331,
// src/model/cuda/cuda_decode_step.cpp:47-70): the embedding row, every
// layer's attention and MLP with their residual adds and norms, the final
// norm and the LM head, with only the StepState rewritten between tokens.
//
// The layer is the reference's dense layer (layer.dense,
// cuda_decoder.cpp:119-124) with rotary attention over the whole cache:
//   h = rms(x) w_in;  q, k, v = h Wq, h Wk, h Wv;  rope(q, k) at pos;
//   append k, v;  attn = softmax(q K^T / sqrt(hd)) V;  x += attn Wo;
//   h = rms(x) w_post;  x += (silu(h Wg) * (h Wu)) Wd
// and after the last layer logits = (rms(x) w_final) W_lm. The reference's
// block routing, mixture-of-experts layers and int8 weights are not part of
// it. Each step runs 1 + 6 per layer + 1 launches: the residual add of
// each sublayer is the prologue of the next projection (the fused GEMVs),
// and rope + both appends + attention are one op of two launches.

#include <cstdint>
#include <memory>
#include <vector>

#include "backend/rocm/context.h"

namespace uocr::rocm {

struct DenseDecoderDims {
  std::int64_t hidden = 1280;
  std::int64_t heads = 10;
  std::int64_t head_dim = 128;
  std::int64_t ffn = 896;
  std::int64_t vocab = 129280;
  std::int64_t capacity = 8192;  // key/value positions per layer
  float eps = 1e-6f;
  double rope_theta = 1e4;
  bool bf16_cache = true;  // key/value cache in bf16 (else fp32)
};

// Device weights of one layer, owned by the caller (bf16 bits, fp32 norms).
struct DenseLayerWeights {
  const float* input_norm;   // [hidden]
  const std::uint16_t* qkv;  // [3 * heads * head_dim, hidden]: Wq, Wk, Wv rows stacked
  const std::uint16_t* o;    // [hidden, heads * head_dim]
  const float* post_norm;    // [hidden]
  const std::uint16_t* gate;  // [ffn, hidden]
  const std::uint16_t* up;    // [ffn, hidden]
  const std::uint16_t* down;  // [hidden, ffn]
};

class DenseDecodeStep {
 public:
  // embed [vocab, hidden] bf16, final_norm [hidden], lm_head [vocab, hidden]
  // bf16; every pointer stays owned by the caller and must outlive this.
  DenseDecodeStep(const Context& ctx, const DenseDecoderDims& dims, const std::uint16_t* embed,
                  std::vector<DenseLayerWeights> layers, const float* final_norm, const std::uint16_t* lm_head);
  ~DenseDecodeStep();
  DenseDecodeStep(const DenseDecodeStep&) = delete;
  DenseDecodeStep& operator=(const DenseDecodeStep&) = delete;

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
  DenseDecoderDims dims_;
  const std::uint16_t* embed_;
  std::vector<DenseLayerWeights> layers_;
  const float* final_norm_;
  const std::uint16_t* lm_head_;
  Array inv_tok_, state_, x_[2], delta_, qkv_, attn_, o_, act_, logits_, scratch_;
  std::vector<Array> k_cache_, v_cache_;
  std::unique_ptr<PinnedBuffer> state_host_, logits_host_;
  std::unique_ptr<Graph> graph_;
};

}  // namespace uocr::rocm
