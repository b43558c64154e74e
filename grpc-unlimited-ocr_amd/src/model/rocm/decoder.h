#pragma once

// The decoder as the reference's generation loop and service see a backend
// (uocr::DecoderModel, src/model/decoder_model.h:16-31): token embeddings,
// one prefill per document, then one step per token, over the rocm decode
// step and its prefill (DecodeStep). The reference's own types (Tensor,
// PromptLayout, BlockPages, RopeCoord) stay on the reference's side:
// model/rocm/reference_adapters.h turns them into the plain vectors taken
// here, so this library needs none of the reference's headers.

#include <cstdint>
#include <vector>

#include "backend/rocm/context.h"
#include "model/rocm/decode_step.h"

namespace uocr::rocm {

// The parts of a prompt's page layout the decoder reads (PromptLayout,
// src/model/page_layout.h:22-30), one entry per prompt position.
struct PromptPlan {
  std::vector<RopeCoord> coords;         // rotary coordinate
  std::vector<std::int64_t> image_page;  // page of an image token, else -1
  std::vector<std::int64_t> query_page;  // page a query is confined to, -1 = global
};

// Per key block of block_size prompt positions, the lowest and highest image
// page it holds (-1, -1 when it holds no image token).
struct BlockPages {
  std::vector<std::int64_t> min_page;
  std::vector<std::int64_t> max_page;
};

// block_image_pages (src/model/page_layout.cpp:55-69) over the per-position
// image pages.
BlockPages block_image_pages(const std::vector<std::int64_t>& image_page, std::int64_t block_size);

// One document at a time, as an implementation of DecoderModel keeps its own
// cache (CudaDecoder, src/model/cuda/cuda_decoder.cpp:86-92, 288-330). The
// step, the embedding table and the context stay owned by the caller.
class Decoder {
 public:
  // embed: the bf16 table [vocab, hidden] the step reads.
  Decoder(const Context& ctx, DecodeStep& step, const std::uint16_t* embed, std::int64_t vocab, std::int64_t hidden);

  // Rows of the embedding table [ids, hidden], exact (an id outside the
  // vocabulary gives a zero row).
  std::vector<float> embed(const std::vector<std::int64_t>& ids) const;

  // Starts a document: embeds [positions, hidden] from position 0, the
  // prompt blocks' pages taken from layout.image_page, the caches grown to
  // hold the prompt; returns the next-token logits [vocab].
  std::vector<float> prefill(const std::vector<float>& embeds, const PromptPlan& layout);

  // Feeds `token` at the next position; returns the next-token logits. The
  // prompt's block pages are on the device since prefill, so prompt_blocks
  // is not read (as in CudaDecoder::step). The caches grow when full.
  std::vector<float> step(std::int64_t token, RopeCoord coord, std::int64_t query_page,
                          const BlockPages& prompt_blocks = {});

  std::int64_t block_size() const { return step_.block_size(); }
  std::int64_t hidden() const { return hidden_; }
  std::int64_t vocab() const { return vocab_; }
  std::int64_t length() const { return step_.length(); }
  DecodeStep& decode_step() { return step_; }

 private:
  const Context& ctx_;
  DecodeStep& step_;
  const std::uint16_t* embed_;
  std::int64_t vocab_, hidden_;
};

}  // namespace uocr::rocm
