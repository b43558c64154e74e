#pragma once

// The whole model on the rocm backend, loaded by the reference's checkpoint
// tensor names (src/weights/architecture.cpp:38-139): the vision encoder
// (VisionEncoder) and the decoder (DecodeStep with its prefill), each
// weight uploaded once and owned here. This is what the reference's
// ModelEngine::build_backend constructs for GRPC_UOCR_BACKEND=rocm
// (src/service/model_engine.cpp:118-144) in place of CudaVisionEncoder and
// CudaDecoder (src/model/cuda/cuda_vision.cpp:54-115,
// src/model/cuda/cuda_decoder.cpp:33-85): matrices go to the device as
// bf16 (nearest even), norm weights, biases and the mixture-of-experts gate
// as fp32; each decoder layer's q, k, v and router q/k projections are
// stacked into one matrix, and each layer's routed experts into one stack
// per projection, as the fused decode step reads them.

#include <cstdint>
#include <memory>
#include <string>
#include <vector>

#include "backend/rocm/context.h"
#include "model/rocm/decode_step.h"
#include "model/rocm/decoder.h"
#include "model/rocm/vision.h"

namespace uocr::rocm {

// One named tensor as the checkpoint holds it, widened to fp32 on the host.
struct HostTensor {
  std::vector<std::int64_t> shape;
  std::vector<float> data;
};

// Where the weights come from: the reference's WeightSource
// (src/model/weight_source.h:16-21) adapts to this in a few lines.
class TensorSource {
 public:
  virtual ~TensorSource() = default;
  // Throws std::out_of_range naming the tensor when it is absent.
  virtual HostTensor get(const std::string& name) const = 0;
};

// src/weights/architecture.h:19-33 (decoder) beside the vision dims.
struct ModelDims {
  DecoderDims decoder;  // hidden, heads, head_dim, index_dim, vocab, cache capacity, router, rope
  std::int64_t layers = 12;
  std::int64_t dense_ffn = 6848;     // layers below first_moe_layer
  std::int64_t first_moe_layer = 1;
  std::int64_t routed_experts = 64;
  std::int64_t experts_per_token = 6;
  std::int64_t shared_experts = 2;   // their FFN is shared_experts * expert_ffn
  std::int64_t expert_ffn = 896;
  VisionDims vision;
};

class Model {
 public:
  // Uploads every tensor (std::out_of_range if one is missing,
  // std::invalid_argument if a shape differs from the dims).
  Model(const Context& ctx, const TensorSource& weights, const ModelDims& dims = {});
  ~Model();
  Model(const Model&) = delete;
  Model& operator=(const Model&) = delete;

  // The page's image tokens [tokens, hidden] (VisionModel::encode_page).
  std::vector<float> encode_page(const View& global, const std::vector<View>& tiles = {}, std::int64_t tiles_wide = 1,
                                 std::int64_t tiles_high = 1) const;
  // Token embeddings [ids, hidden] (Decoder::embed, src/model/decoder.cpp:85-92).
  std::vector<float> embed(const std::vector<std::int64_t>& ids) const;

  VisionEncoder& vision() { return *vision_; }
  DecodeStep& decoder() { return *decoder_; }
  // The decoder as DecoderModel sees it: embed, prefill per document, step.
  Decoder& decoder_model() { return *session_; }

 private:
  const std::uint16_t* matrix(const std::string& name, std::int64_t rows, std::int64_t cols);
  const float* vector(const std::string& name, std::int64_t n);
  std::vector<float> host(const std::string& name, std::int64_t n) const;
  const std::uint16_t* stacked(const std::vector<std::string>& names, std::int64_t rows, std::int64_t cols);

  const Context& ctx_;
  const TensorSource& src_;
  ModelDims dims_;
  std::vector<Array> owned_;
  std::vector<std::unique_ptr<MoeWeights>> moe_;
  const std::uint16_t* embed_ = nullptr;
  std::unique_ptr<VisionEncoder> vision_;
  std::unique_ptr<DecodeStep> decoder_;
  std::unique_ptr<Decoder> session_;
};

}  // namespace uocr::rocm
