#pragma once

// The rocm backend behind the reference's model interfaces, for the
// reference's own tree: this header includes the reference's headers
// (src/model/*.h, src/tensor/tensor.h, src/weights/architecture.h) and is
// compiled there, beside the service that selects the backend; nothing in
// this library includes it. ModelEngine::build_backend
// (src/service/model_engine.cpp:118-144) and uocr-run --backend
// (tools/uocr_run.cpp:122-141) construct, for GRPC_UOCR_BACKEND=rocm:
//
//   RocmWeights      uocr::rocm::TensorSource over a uocr::WeightSource
//                    (src/model/weight_source.h:16-21): the checkpoint's
//                    tensors by name, fp32 on the host
//   rocm_dims(...)   uocr::rocm::ModelDims from the reference's ModelDims
//                    (src/weights/architecture.h:19-63) and RouterParams
//                    (src/model/block_router.h:17-27)
//   RocmDecoder      uocr::DecoderModel (src/model/decoder_model.h:16-31)
//                    over uocr::rocm::Decoder
//   RocmVisionModel  uocr::VisionModel (src/model/vision_encoder.h:24-38)
//                    over uocr::rocm::VisionEncoder; its encode_page is the
//                    reference's own (the base class's), over encode_view
//
// Each converts the reference's types (Tensor, PromptLayout, RopeCoord,
// BlockPages) to the plain vectors the rocm classes take and back; the work
// runs on the device.

#include <cmath>
#include <cstdint>
#include <string>
#include <utility>
#include <vector>

#include "model/block_router.h"
#include "model/decoder_model.h"
#include "model/page_layout.h"
#include "model/page_rope.h"
#include "model/vision_encoder.h"
#include "model/weight_source.h"
#include "tensor/tensor.h"
#include "weights/architecture.h"

#include "model/rocm/decoder.h"
#include "model/rocm/model.h"
#include "model/rocm/vision.h"

namespace uocr::rocm {

class RocmWeights final : public TensorSource {
 public:
  explicit RocmWeights(const uocr::WeightSource& weights) : weights_(weights) {}
  // Throws std::out_of_range naming the tensor when it is absent (the
  // WeightSource's own contract).
  HostTensor get(const std::string& name) const override {
    const uocr::Tensor t = weights_.get(name);
    return HostTensor{t.shape(), std::vector<float>(t.data(), t.data() + t.numel())};
  }

 private:
  const uocr::WeightSource& weights_;
};

// The reference architecture's dimensions (and its decoder's router) as the
// rocm model takes them; `capacity` is the initial key/value positions per
// layer (the caches grow as the reference's do).
inline ModelDims rocm_dims(const uocr::ModelDims& m, const uocr::RouterParams& router,
                           std::int64_t capacity = 8192) {
  ModelDims d;
  const uocr::DecoderDims& dd = m.decoder;
  d.decoder.hidden = dd.hidden;
  d.decoder.heads = dd.heads;
  d.decoder.head_dim = dd.head_dim;
  d.decoder.index_dim = dd.index_dim;
  d.decoder.vocab = dd.vocab;
  d.decoder.capacity = capacity;
  d.decoder.eps = static_cast<float>(dd.rms_norm_eps);
  d.decoder.router = RouteParams{router.block_size, router.local_blocks, router.top_m, router.top_k,
                                 router.idx_scale,  router.floor,        router.sigma};
  d.layers = dd.layers;
  d.dense_ffn = dd.dense_ffn;
  d.first_moe_layer = dd.first_moe_layer;
  d.routed_experts = dd.routed_experts;
  d.experts_per_token = dd.experts_per_token;
  d.shared_experts = dd.shared_experts;
  d.expert_ffn = dd.expert_ffn;
  SamDims& s = d.vision.sam;
  s.image = m.sam.image;
  s.patch = m.sam.patch;
  s.width = m.sam.width;
  s.layers = m.sam.layers;
  s.heads = m.sam.heads;
  s.mlp = m.sam.mlp;
  s.window = m.sam.window;
  s.global_layers.assign(m.sam.global_layers.begin(), m.sam.global_layers.end());
  s.neck = m.sam.neck;
  s.net2 = m.sam.net2;
  s.net3 = m.sam.net3;
  ClipDims& c = d.vision.clip;
  c.width = m.clip.width;
  c.layers = m.clip.layers;
  c.heads = m.clip.heads;
  c.mlp = m.clip.mlp;
  c.positions = m.clip.positions;
  d.vision.hidden = dd.hidden;
  return d;
}

class RocmDecoder final : public uocr::DecoderModel {
 public:
  explicit RocmDecoder(Decoder& decoder) : decoder_(decoder) {}

  uocr::Tensor embed(const std::vector<std::int64_t>& ids) const override {
    return uocr::Tensor({static_cast<std::int64_t>(ids.size()), decoder_.hidden()}, decoder_.embed(ids));
  }

  std::vector<float> prefill(const uocr::Tensor& embeds, const uocr::PromptLayout& layout) override {
    PromptPlan plan;
    plan.coords.reserve(layout.coords.size());
    for (const uocr::RopeCoord& c : layout.coords) plan.coords.push_back(RopeCoord{c.tok, c.page});
    plan.image_page = layout.image_page;
    plan.query_page = layout.query_page;
    return decoder_.prefill(std::vector<float>(embeds.data(), embeds.data() + embeds.numel()), plan);
  }

  // The prompt's block pages are on the device since prefill (as in
  // CudaDecoder::step), so prompt_blocks is not copied over.
  std::vector<float> step(std::int64_t token, uocr::RopeCoord coord, std::int64_t query_page,
                          const uocr::BlockPages& prompt_blocks) override {
    (void)prompt_blocks;
    return decoder_.step(token, RopeCoord{coord.tok, coord.page}, query_page);
  }

  std::int64_t block_size() const override { return decoder_.block_size(); }

 private:
  Decoder& decoder_;
};

class RocmVisionModel final : public uocr::VisionModel {
 public:
  explicit RocmVisionModel(const VisionEncoder& encoder) : encoder_(encoder) {
    newline_ = uocr::Tensor({encoder.hidden()}, encoder.newline());
    separator_ = uocr::Tensor({encoder.hidden()}, encoder.separator());
  }

  // image [3, S, S] -> [g * g, hidden], g = S / 64.
  uocr::Tensor encode_view(const uocr::Tensor& image) const override {
    const View view{std::vector<float>(image.data(), image.data() + image.numel()), image.dim(2)};
    const std::int64_t g = encoder_.grid(view.size);
    return uocr::Tensor({g * g, encoder_.hidden()}, encoder_.encode_view(view));
  }

 private:
  const VisionEncoder& encoder_;
};

}  // namespace uocr::rocm
