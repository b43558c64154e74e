#pragma once

// The vision encoder on the rocm backend: SAM (ViT-B with windowed and
// global relative-position attention, the neck and two stride-2
// convolutions), CLIP over SAM's features, and the projector, with bf16
// weights and fp32 activations (the reference's CudaVisionEncoder,
// src/model/cuda/cuda_vision.{h,cpp}), plus the page token layout of
// VisionModel::encode_page (src/model/vision_encoder.cpp:46-68).
//
// A view [3, S, S] (S a multiple of 64) runs as:
//   x = patches(image) Wpatch + b + pos            [g * g, 768], g = S / 16
//   per block: x += attn(LN1(x)) (global, or per 14 x 14 window of the
//     zero-padded grid), x += lin2(gelu(lin1(LN2(x))))
//   y = LN(x Wneck0); y = LN(conv3x3(y)); y = conv3x3/2(y); y = conv3x3/2(y)
//   c = CLIP([class | y] + pos)                    [1 + g4 * g4, 1024]
//   out = [c[1:] | y] Wproj + b                    [g4 * g4, hidden]
// Activations are kept as rows [positions, channels]; a 3 x 3 convolution
// turns its input to [channels, h, w] once for the patch gather. Every
// matrix product of the projections and convolutions runs on the bf16
// matrix cores (x rounded to bf16, fp32 sums: the reference's linear), k
// split over a workspace where a product has too few tiles (CLIP's 257
// rows); attention is one launch per layer for every head and window
// (scores, bias, softmax and values without the scores reaching memory),
// its output rounded to bf16 for the output projection: SAM's on the bf16
// matrix cores with each fp32 operand split into bf16 hi + lo parts,
// CLIP's on the fp32 matrix cores. The learned position grids and the
// relative-position tables are resized on the host once per grid size, as
// the reference does, and kept on the device.

#include <cstdint>
#include <map>
#include <tuple>
#include <vector>

#include "backend/rocm/context.h"

namespace uocr::rocm {

// src/weights/architecture.h:35-56.
struct SamDims {
  std::int64_t image = 1024;  // the position grid's image size
  std::int64_t patch = 16;
  std::int64_t width = 768;
  std::int64_t layers = 12;
  std::int64_t heads = 12;
  std::int64_t mlp = 3072;
  std::int64_t window = 14;
  std::vector<std::int64_t> global_layers = {2, 5, 8, 11};
  std::int64_t neck = 256;
  std::int64_t net2 = 512;
  std::int64_t net3 = 1024;
};

struct ClipDims {
  std::int64_t width = 1024;
  std::int64_t layers = 24;
  std::int64_t heads = 16;
  std::int64_t mlp = 4096;
  std::int64_t positions = 257;  // 16 x 16 + the class position
};

struct VisionDims {
  SamDims sam;
  ClipDims clip;
  std::int64_t hidden = 1280;  // the decoder's width (the projector's output)
};

// Device weights are owned by the caller (bf16 matrices [out, in], conv
// weights [out, in * kh * kw]; fp32 vectors); the tables the encoder
// resizes per grid are host copies.
struct SamBlockWeights {
  const float* norm1_w = nullptr;
  const float* norm1_b = nullptr;
  const std::uint16_t* qkv = nullptr;  // [3 * width, width]
  const float* qkv_b = nullptr;
  const std::uint16_t* proj = nullptr;  // [width, width]
  const float* proj_b = nullptr;
  std::vector<float> rel_h, rel_w;  // host [2 * span - 1, head_dim]
  const float* norm2_w = nullptr;
  const float* norm2_b = nullptr;
  const std::uint16_t* lin1 = nullptr;  // [mlp, width]
  const float* lin1_b = nullptr;
  const std::uint16_t* lin2 = nullptr;  // [width, mlp]
  const float* lin2_b = nullptr;
};

struct ClipLayerWeights {
  const float* ln1_w = nullptr;
  const float* ln1_b = nullptr;
  const std::uint16_t* qkv = nullptr;  // [3 * width, width]
  const float* qkv_b = nullptr;
  const std::uint16_t* out = nullptr;  // [width, width]
  const float* out_b = nullptr;
  const float* ln2_w = nullptr;
  const float* ln2_b = nullptr;
  const std::uint16_t* fc1 = nullptr;  // [mlp, width]
  const float* fc1_b = nullptr;
  const std::uint16_t* fc2 = nullptr;  // [width, mlp]
  const float* fc2_b = nullptr;
};

struct VisionWeights {
  const std::uint16_t* patch = nullptr;  // [width, 3 * patch * patch]
  const float* patch_b = nullptr;
  std::vector<float> sam_pos;  // host [image / patch, image / patch, width]
  std::vector<SamBlockWeights> sam_blocks;
  const std::uint16_t* neck0 = nullptr;  // [neck, width]
  const float* neck1_w = nullptr;
  const float* neck1_b = nullptr;
  const std::uint16_t* neck2 = nullptr;  // [neck, neck * 9]
  const float* neck3_w = nullptr;
  const float* neck3_b = nullptr;
  const std::uint16_t* net2 = nullptr;  // [net2, neck * 9]
  const std::uint16_t* net3 = nullptr;  // [net3, net2 * 9]
  const float* class_embedding = nullptr;  // [clip width]
  std::vector<float> clip_pos;             // host [positions, clip width]
  const float* pre_ln_w = nullptr;
  const float* pre_ln_b = nullptr;
  std::vector<ClipLayerWeights> clip_layers;
  const std::uint16_t* projector = nullptr;  // [hidden, clip width + net3]
  const float* projector_b = nullptr;
  std::vector<float> newline, separator;  // host [hidden]
};

// One image [3, size, size] on the host.
struct View {
  std::vector<float> pixels;
  std::int64_t size = 0;
};

// Calls are ordered on the context's stream and share the encoder's caches
// and scratch: one thread at a time per encoder (an encoder per stream for
// concurrent views).
class VisionEncoder {
 public:
  // Shapes are checked here (std::invalid_argument); every device pointer
  // stays owned by the caller and must outlive this.
  VisionEncoder(const Context& ctx, const VisionDims& dims, VisionWeights weights);

  // The features of one view: [g * g, hidden] rows on the host, g = size /
  // 64 (CudaVisionEncoder::encode_view, cuda_vision.cpp:268-281).
  std::vector<float> encode_view(const View& image) const;
  // The same into device memory out [g * g, hidden] (nothing read back).
  void encode_view(const float* image_device, std::int64_t size, float* out) const;

  // A page's image tokens (VisionModel::encode_page): with tiles, their
  // grids stitched into one (high * g) x (wide * g) grid, each row followed
  // by the newline; then the global view's rows, each followed by the
  // newline; then the separator. Rows [tokens, hidden].
  std::vector<float> encode_page(const View& global, const std::vector<View>& tiles = {}, std::int64_t tiles_wide = 1,
                                 std::int64_t tiles_high = 1) const;

  // The feature grid of a size x size view: size / 16 through two stride-2
  // 3 x 3 convolutions.
  std::int64_t grid(std::int64_t size) const;
  // The embeddings encode_page places after each grid row and after the page
  // (host [hidden] each).
  const std::vector<float>& newline() const { return w_.newline; }
  const std::vector<float>& separator() const { return w_.separator; }
  std::int64_t hidden() const { return dims_.hidden; }
  // g (g + 1) + 1 tokens for the global grid, plus (tile_grid * wide + 1)
  // (tile_grid * high) with tiles (vision_encoder.cpp:70-77).
  static std::int64_t page_image_tokens(std::int64_t global_grid, std::int64_t tile_grid, std::int64_t tiles_wide,
                                        std::int64_t tiles_high, bool tiled);

 private:
  // y = bf16(x) w^T (+ bias) on the matrix cores, k split over a pool
  // workspace where the product has too few tiles to cover the GPU.
  // (accumulate: y += the product, as the product then an in-place add.)
  void project(const float* x, std::int64_t m, std::int64_t k, const std::uint16_t* w, std::int64_t n,
               const float* bias, float* y, bool accumulate = false) const;
  // The same with x already bf16.
  void project_bf16(const std::uint16_t* xb, std::int64_t m, std::int64_t k, const std::uint16_t* w, std::int64_t n,
                    const float* bias, float* y, bool accumulate = false) const;
  // bf16(gelu_erf(x)) (quick: bf16(quick_gelu(x))) in project()'s scratch.
  const std::uint16_t* activated_bf16(const float* x, std::int64_t n, bool quick) const;
  // bf16(LN(x)) in project()'s scratch, x untouched (null: c above 16384).
  const std::uint16_t* normed_bf16(const float* x, std::int64_t rows, std::int64_t c, const float* w, const float* b,
                                   float eps) const;
  // x += act(LN(x) w1^T + b1) w2^T + b2 (act quick_gelu or gelu_erf), both
  // products' inputs in bf16 and the activation in the first one's epilogue;
  // false, nothing done, where c is above 16384 or not a multiple of 64.
  bool mlp_bf16(float* x, std::int64_t rows, std::int64_t c, const float* ln_w, const float* ln_b, float eps,
                const std::uint16_t* w1, std::int64_t hidden, const float* b1, const std::uint16_t* w2,
                const float* b2, bool quick) const;
  // y = LN(x) w^T + bias, x untouched (`normed`: fp32 room for the wide case).
  void norm_project(const float* x, std::int64_t rows, std::int64_t c, const float* ln_w, const float* ln_b, float eps,
                    Array& normed, const std::uint16_t* w, std::int64_t n, const float* bias, float* y) const;
  void sam_forward(const float* image, std::int64_t size, Array& cells) const;
  void sam_block(std::size_t index, Array& x, std::int64_t g) const;
  // x fp32, or xb (non-null) the same rows already in bf16
  // (accumulate: out += the output projection; out_rows non-null: row r of
  // the projection added into out row out_rows[r], dropped at out_count.)
  void sam_attention(std::size_t index, const float* x, const std::uint16_t* xb, std::int64_t windows, std::int64_t h,
                     std::int64_t w, float* out, bool accumulate, const std::int64_t* out_rows,
                     std::int64_t out_count) const;
  void conv3(const float* hwc, std::int64_t side, std::int64_t in_c, const std::uint16_t* w, std::int64_t out_c,
             int stride, Array& out, std::int64_t& out_side) const;
  void clip_forward(const float* cells, std::int64_t g, Array& x) const;
  const Array& sam_positions(std::int64_t g) const;
  const Array& clip_positions(std::int64_t g) const;
  const Array& rel_table(std::size_t block, bool height, std::int64_t span) const;
  struct Windows {
    Array gather, scatter;  // slot -> grid row (g * g: the zero row); grid row -> slot
    std::int64_t count = 0;
  };
  const Windows& windows(std::int64_t g) const;

  const Context& ctx_;
  VisionDims dims_;
  VisionWeights w_;
  std::vector<bool> global_;
  mutable std::map<std::int64_t, Array> sam_pos_, clip_pos_;
  mutable std::map<std::tuple<std::size_t, bool, std::int64_t>, Array> rel_tables_;
  mutable std::map<std::int64_t, Windows> windows_;
  mutable Array split_ws_, x_bf16_;  // project()'s scratch, grown on demand
  mutable Array act_bf16_;           // mlp_bf16()'s activations, grown on demand
  mutable Array mlp_wide_;           // mlp_bf16()'s fp32 first product (many rows), grown on demand
  // From this many rows on, an MLP's first product runs unfused (the
  // library's product, then the activation pass) instead of through the
  // tile kernel's activation epilogue.
  static constexpr std::int64_t kWideMlpRows = 128;
  mutable std::map<std::int64_t, Array> win_normed_;  // per grid: bf16 norm rows + a zero row
};

// Host table resizes of the encoder (src/backend/reference/ops.cpp:42-86,
// 253-296; src/model/sam_encoder.cpp:52-63).
std::vector<float> resize_bicubic_aa(const std::vector<float>& x, std::int64_t c, std::int64_t h, std::int64_t w,
                                     std::int64_t out_h, std::int64_t out_w);
std::vector<float> resize_linear_rows(const std::vector<float>& x, std::int64_t len, std::int64_t c,
                                      std::int64_t out_len);
std::vector<float> relative_positions(const std::vector<float>& table, std::int64_t d, std::int64_t size);

}  // namespace uocr::rocm
