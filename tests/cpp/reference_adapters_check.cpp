// Compiled with -fsyntax-only against the reference's headers (never linked,
// never run): the rocm adapters of model/rocm/reference_adapters.h implement
// the reference's model interfaces with their exact signatures (each member
// is marked override, and a class left abstract fails the static_asserts),
// and the calls the generation loop (src/runtime/generator.cpp) and the
// service (src/service/model_engine.cpp:118-144) make through the base
// classes compile against them.

#include <memory>
#include <type_traits>
#include <vector>

#include "model/decoder.h"
#include "model/rocm/reference_adapters.h"

namespace {

using uocr::rocm::RocmDecoder;
using uocr::rocm::RocmVisionModel;
using uocr::rocm::RocmWeights;

static_assert(std::is_base_of_v<uocr::DecoderModel, RocmDecoder>);
static_assert(std::is_base_of_v<uocr::VisionModel, RocmVisionModel>);
static_assert(std::is_base_of_v<uocr::rocm::TensorSource, RocmWeights>);
static_assert(!std::is_abstract_v<RocmDecoder>);
static_assert(!std::is_abstract_v<RocmVisionModel>);
static_assert(!std::is_abstract_v<RocmWeights>);
static_assert(std::is_final_v<RocmDecoder> && std::is_final_v<RocmVisionModel>);

// What build_backend would do for GRPC_UOCR_BACKEND=rocm, then one page and
// a prompt through the base-class pointers.
[[maybe_unused]] void build_and_drive(const uocr::WeightSource& checkpoint, const uocr::PageViews& page,
                                      const std::vector<std::int64_t>& prompt_ids) {
  const uocr::rocm::Context ctx(0);
  const RocmWeights source(checkpoint);
  uocr::rocm::Model model(ctx, source, uocr::rocm::rocm_dims(uocr::ModelDims{}, uocr::Decoder::default_router()));
  std::unique_ptr<uocr::VisionModel> vision = std::make_unique<RocmVisionModel>(model.vision());
  std::unique_ptr<uocr::DecoderModel> decoder = std::make_unique<RocmDecoder>(model.decoder_model());

  const uocr::Tensor image_tokens = vision->encode_page(page);
  const uocr::Tensor view = vision->encode_view(page.global);
  const uocr::PromptLayout layout = uocr::layout_prompt(prompt_ids);
  const uocr::Tensor embeds = decoder->embed(prompt_ids);
  std::vector<float> logits = decoder->prefill(embeds, layout);
  const uocr::BlockPages blocks = uocr::block_image_pages(layout, decoder->block_size());
  uocr::DecodeState state(layout, prompt_ids);
  const std::int64_t token = 1;
  const uocr::RopeCoord coord = state.advance(token);
  logits = decoder->step(token, coord, state.query_page(), blocks);
  (void)image_tokens;
  (void)view;
}

}  // namespace
