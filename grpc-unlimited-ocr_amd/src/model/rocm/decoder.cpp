#include "model/rocm/decoder.h"

#include <algorithm>
#include <stdexcept>
#include <string>

#include "backend/rocm/ops.h"

namespace uocr::rocm {
namespace {

void need(bool ok, const char* what) {
  if (!ok) throw std::invalid_argument(std::string("Decoder: ") + what);
}

}  // namespace

BlockPages block_image_pages(const std::vector<std::int64_t>& image_page, std::int64_t block_size) {
  need(block_size >= 1, "block_size must be >= 1");
  const auto n = static_cast<std::int64_t>(image_page.size());
  const std::int64_t blocks = (n + block_size - 1) / block_size;
  BlockPages out{std::vector<std::int64_t>(static_cast<std::size_t>(blocks), -1),
                 std::vector<std::int64_t>(static_cast<std::size_t>(blocks), -1)};
  for (std::int64_t i = 0; i < n; ++i) {
    const std::int64_t page = image_page[static_cast<std::size_t>(i)];
    if (page < 0) continue;  // not an image token
    const auto b = static_cast<std::size_t>(i / block_size);
    out.min_page[b] = out.min_page[b] < 0 ? page : std::min(out.min_page[b], page);
    out.max_page[b] = std::max(out.max_page[b], page);
  }
  return out;
}

Decoder::Decoder(const Context& ctx, DecodeStep& step, const std::uint16_t* embed, std::int64_t vocab,
                 std::int64_t hidden)
    : ctx_(ctx), step_(step), embed_(embed), vocab_(vocab), hidden_(hidden) {
  need(embed != nullptr && vocab > 0 && hidden > 0, "null embedding table or empty shape");
}

std::vector<float> Decoder::embed(const std::vector<std::int64_t>& ids) const {
  const auto n = static_cast<std::int64_t>(ids.size());
  if (n == 0) return {};
  Array idx(ctx_, DType::kI64, n);
  idx.upload(ids.data(), n);
  Array out(ctx_, DType::kF32, n * hidden_);
  gather_rows_bf16(ctx_, embed_, vocab_, idx.i64(), n, hidden_, out.f32());
  return out.download();
}

std::vector<float> Decoder::prefill(const std::vector<float>& embeds, const PromptPlan& layout) {
  const auto rows = static_cast<std::int64_t>(layout.coords.size());
  need(rows >= 1, "an empty prompt");
  need(static_cast<std::int64_t>(embeds.size()) == rows * hidden_, "embeds must be [positions, hidden]");
  need(static_cast<std::int64_t>(layout.image_page.size()) == rows &&
           static_cast<std::int64_t>(layout.query_page.size()) == rows,
       "the layout needs one image page and one query page per position");
  // CudaDecoder::prefill (cuda_decoder.cpp:288-298): a new document from
  // position 0, the prompt blocks' pages on the device, then the prompt pass.
  step_.rewind();
  const BlockPages blocks = block_image_pages(layout.image_page, step_.block_size());
  step_.reserve(rows);  // before the blocks: growth copies the old ones
  step_.set_prompt_blocks(blocks.min_page, blocks.max_page);
  return step_.prefill(embeds, layout.coords, layout.query_page);
}

std::vector<float> Decoder::step(std::int64_t token, RopeCoord coord, std::int64_t query_page,
                                 const BlockPages& prompt_blocks) {
  (void)prompt_blocks;  // on the device since prefill
  step_.reserve(step_.length() + 1);
  return step_.step(token, coord, query_page);
}

}  // namespace uocr::rocm
