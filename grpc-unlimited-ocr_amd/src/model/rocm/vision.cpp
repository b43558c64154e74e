// VisionEncoder: the vision encoder on the rocm backend (the reference's
// CudaVisionEncoder, src/model/cuda/cuda_vision.cpp, and
// VisionModel::encode_page, src/model/vision_encoder.cpp:46-68).

#include "model/rocm/vision.h"

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>

#include "backend/rocm/ops.h"

namespace uocr::rocm {
namespace {

constexpr float kSamEps = 1e-6f;
constexpr float kClipEps = 1e-5f;

void need(bool ok, const std::string& what) {
  if (!ok) throw std::invalid_argument("VisionEncoder: " + what);
}

Array f32(const Context& ctx, std::int64_t n) { return Array(ctx, DType::kF32, std::max<std::int64_t>(n, 1)); }

Array upload_f32(const Context& ctx, const std::vector<float>& v) {
  Array a = f32(ctx, static_cast<std::int64_t>(v.size()));
  if (!v.empty()) a.upload(v.data(), static_cast<std::int64_t>(v.size()));
  return a;
}

// [rows, c] <-> [c, rows] of host tables (the position grids go through
// the channel-major layout for the resize).
std::vector<float> rows_to_channels(const std::vector<float>& x, std::int64_t rows, std::int64_t c) {
  std::vector<float> y(x.size());
  for (std::int64_t r = 0; r < rows; ++r)
    for (std::int64_t ch = 0; ch < c; ++ch) y[ch * rows + r] = x[r * c + ch];
  return y;
}

std::vector<float> channels_to_rows(const std::vector<float>& x, std::int64_t rows, std::int64_t c) {
  std::vector<float> y(x.size());
  for (std::int64_t ch = 0; ch < c; ++ch)
    for (std::int64_t r = 0; r < rows; ++r) y[r * c + ch] = x[ch * rows + r];
  return y;
}

// The antialiasing cubic, a = -0.5 (ops.cpp:43-54).
float aa_cubic(float t) {
  constexpr float a = -0.5f;
  t = std::fabs(t);
  if (t < 1.0f) return ((a + 2.0f) * t - (a + 3.0f)) * t * t + 1.0f;
  if (t < 2.0f) return ((a * t - 5.0f * a) * t + 8.0f * a) * t - 4.0f * a;
  return 0.0f;
}

// One axis's filter: for output index i, the first source index and the
// normalised weights of its taps (ops.cpp:60-86).
struct AxisFilter {
  std::vector<std::int64_t> first;
  std::vector<std::vector<float>> weights;
};

AxisFilter axis_filter(std::int64_t in, std::int64_t out) {
  const float scale = static_cast<float>(in) / static_cast<float>(out);
  const float support = scale >= 1.0f ? 2.0f * scale : 2.0f;
  const float invscale = scale >= 1.0f ? 1.0f / scale : 1.0f;
  AxisFilter f;
  f.first.resize(static_cast<std::size_t>(out));
  f.weights.resize(static_cast<std::size_t>(out));
  for (std::int64_t i = 0; i < out; ++i) {
    const float center = scale * (static_cast<float>(i) + 0.5f);
    const std::int64_t lo = std::max<std::int64_t>(static_cast<std::int64_t>(center - support + 0.5f), 0);
    const std::int64_t hi = std::min<std::int64_t>(static_cast<std::int64_t>(center + support + 0.5f), in);
    auto& wv = f.weights[static_cast<std::size_t>(i)];
    f.first[static_cast<std::size_t>(i)] = lo;
    float sum = 0.0f;
    for (std::int64_t j = lo; j < hi; ++j) {
      wv.push_back(aa_cubic((static_cast<float>(j) - center + 0.5f) * invscale));
      sum += wv.back();
    }
    if (sum != 0.0f) {
      for (float& v : wv) v /= sum;
    }
  }
  return f;
}

}  // namespace

std::vector<float> resize_bicubic_aa(const std::vector<float>& x, std::int64_t c, std::int64_t h, std::int64_t w,
                                     std::int64_t out_h, std::int64_t out_w) {
  const AxisFilter fy = axis_filter(h, out_h), fx = axis_filter(w, out_w);
  std::vector<float> out(static_cast<std::size_t>(c * out_h * out_w));
  for (std::int64_t ch = 0; ch < c; ++ch) {
    const float* src = x.data() + ch * h * w;
    for (std::int64_t oy = 0; oy < out_h; ++oy) {
      const auto& wy = fy.weights[static_cast<std::size_t>(oy)];
      const std::int64_t y0 = fy.first[static_cast<std::size_t>(oy)];
      for (std::int64_t ox = 0; ox < out_w; ++ox) {
        const auto& wx = fx.weights[static_cast<std::size_t>(ox)];
        const std::int64_t x0 = fx.first[static_cast<std::size_t>(ox)];
        float acc = 0.0f;
        for (std::size_t a = 0; a < wy.size(); ++a) {
          const float* line = src + (y0 + static_cast<std::int64_t>(a)) * w + x0;
          float along = 0.0f;
          for (std::size_t b = 0; b < wx.size(); ++b) along += line[b] * wx[b];
          acc += along * wy[a];
        }
        out[static_cast<std::size_t>((ch * out_h + oy) * out_w + ox)] = acc;
      }
    }
  }
  return out;
}

std::vector<float> resize_linear_rows(const std::vector<float>& x, std::int64_t len, std::int64_t c,
                                      std::int64_t out_len) {
  const float scale = static_cast<float>(len) / static_cast<float>(out_len);
  std::vector<float> out(static_cast<std::size_t>(out_len * c));
  for (std::int64_t i = 0; i < out_len; ++i) {
    const float pos = std::max(scale * (static_cast<float>(i) + 0.5f) - 0.5f, 0.0f);
    const auto r0 = static_cast<std::int64_t>(pos);
    const std::int64_t r1 = r0 < len - 1 ? r0 + 1 : r0;
    const float b = pos - static_cast<float>(r0), a = 1.0f - b;
    for (std::int64_t e = 0; e < c; ++e) {
      out[static_cast<std::size_t>(i * c + e)] =
          a * x[static_cast<std::size_t>(r0 * c + e)] + b * x[static_cast<std::size_t>(r1 * c + e)];
    }
  }
  return out;
}

std::vector<float> relative_positions(const std::vector<float>& table, std::int64_t d, std::int64_t size) {
  const std::int64_t len = static_cast<std::int64_t>(table.size()) / d, span = 2 * size - 1;
  const std::vector<float> t = len == span ? table : resize_linear_rows(table, len, d, span);
  std::vector<float> out(static_cast<std::size_t>(size * size * d));
  for (std::int64_t q = 0; q < size; ++q)
    for (std::int64_t k = 0; k < size; ++k)
      std::copy_n(t.begin() + (q - k + size - 1) * d, d, out.begin() + (q * size + k) * d);
  return out;
}

VisionEncoder::VisionEncoder(const Context& ctx, const VisionDims& dims, VisionWeights weights)
    : ctx_(ctx), dims_(dims), w_(std::move(weights)) {
  const SamDims& s = dims_.sam;
  const ClipDims& c = dims_.clip;
  need(s.patch >= 1 && s.image % s.patch == 0 && s.width >= 1 && s.heads >= 1 && s.width % s.heads == 0 &&
           s.window >= 1 && s.neck >= 1 && s.net2 >= 1 && s.net3 >= 1 && s.mlp >= 1,
       "bad SAM dims");
  need(s.width / s.heads <= 256, "SAM head dim above 256");
  need(c.width == s.net3, "CLIP width must equal SAM's output channels");
  need(c.heads >= 1 && c.width % c.heads == 0 && c.mlp >= 1 && c.positions >= 2, "bad CLIP dims");
  const auto src = static_cast<std::int64_t>(std::sqrt(static_cast<double>(c.positions - 1)));
  need(src * src == c.positions - 1, "CLIP positions must be a square grid plus one");
  need(static_cast<std::int64_t>(w_.sam_blocks.size()) == s.layers, "one SamBlockWeights per SAM layer");
  need(static_cast<std::int64_t>(w_.clip_layers.size()) == c.layers, "one ClipLayerWeights per CLIP layer");
  const std::int64_t pg = s.image / s.patch, hd = s.width / s.heads;
  need(static_cast<std::int64_t>(w_.sam_pos.size()) == pg * pg * s.width, "sam_pos must be [image/patch]^2 x width");
  need(static_cast<std::int64_t>(w_.clip_pos.size()) == c.positions * c.width, "clip_pos must be [positions, width]");
  need(static_cast<std::int64_t>(w_.newline.size()) == dims_.hidden &&
           static_cast<std::int64_t>(w_.separator.size()) == dims_.hidden,
       "newline and separator must be [hidden]");
  for (std::int64_t i = 0; i < s.layers; ++i) {
    const auto& b = w_.sam_blocks[static_cast<std::size_t>(i)];
    need(!b.rel_h.empty() && b.rel_h.size() % static_cast<std::size_t>(hd) == 0 && b.rel_w.size() % hd == 0 &&
             !b.rel_w.empty(),
         "relative-position tables must be [len, head_dim]");
    global_.push_back(std::find(s.global_layers.begin(), s.global_layers.end(), i) != s.global_layers.end());
  }
}

std::int64_t VisionEncoder::grid(std::int64_t size) const {
  const std::int64_t g = size / dims_.sam.patch, g2 = (g + 2 - 3) / 2 + 1;
  return (g2 + 2 - 3) / 2 + 1;
}

std::int64_t VisionEncoder::page_image_tokens(std::int64_t global_grid, std::int64_t tile_grid,
                                              std::int64_t tiles_wide, std::int64_t tiles_high, bool tiled) {
  std::int64_t tokens = global_grid * (global_grid + 1) + 1;
  if (tiled) tokens += (tile_grid * tiles_wide + 1) * (tile_grid * tiles_high);
  return tokens;
}

const Array& VisionEncoder::sam_positions(std::int64_t g) const {
  if (auto it = sam_pos_.find(g); it != sam_pos_.end()) return it->second;
  const std::int64_t pg = dims_.sam.image / dims_.sam.patch, c = dims_.sam.width;
  std::vector<float> pos = w_.sam_pos;
  if (pg != g) {
    pos = channels_to_rows(resize_bicubic_aa(rows_to_channels(pos, pg * pg, c), c, pg, pg, g, g), g * g, c);
  }
  return sam_pos_.emplace(g, upload_f32(ctx_, pos)).first->second;
}

const Array& VisionEncoder::clip_positions(std::int64_t g) const {
  if (auto it = clip_pos_.find(g); it != clip_pos_.end()) return it->second;
  const std::int64_t c = dims_.clip.width;
  const auto src = static_cast<std::int64_t>(std::sqrt(static_cast<double>(dims_.clip.positions - 1)));
  std::vector<float> pos = w_.clip_pos;
  if (src != g) {
    const std::vector<float> cells(w_.clip_pos.begin() + c, w_.clip_pos.end());
    const std::vector<float> resized =
        channels_to_rows(resize_bicubic_aa(rows_to_channels(cells, src * src, c), c, src, src, g, g), g * g, c);
    pos.assign(w_.clip_pos.begin(), w_.clip_pos.begin() + c);
    pos.insert(pos.end(), resized.begin(), resized.end());
  }
  return clip_pos_.emplace(g, upload_f32(ctx_, pos)).first->second;
}

const Array& VisionEncoder::rel_table(std::size_t block, bool height, std::int64_t span) const {
  const auto key = std::make_tuple(block, height, span);
  if (auto it = rel_tables_.find(key); it != rel_tables_.end()) return it->second;
  const auto& b = w_.sam_blocks[block];
  const std::int64_t hd = dims_.sam.width / dims_.sam.heads;
  return rel_tables_.emplace(key, upload_f32(ctx_, relative_positions(height ? b.rel_h : b.rel_w, hd, span)))
      .first->second;
}

// Windows of a g x g grid in row order, slots in row order within a window
// (sam_encoder.cpp:17-47): gather[slot] is the grid row that fills it (the
// zero row g * g for the padding), scatter[cell] the slot a grid cell went to.
const VisionEncoder::Windows& VisionEncoder::windows(std::int64_t g) const {
  if (auto it = windows_.find(g); it != windows_.end()) return it->second;
  const std::int64_t win = dims_.sam.window, per = (g + win - 1) / win, n = win * win;
  std::vector<std::int64_t> gather(static_cast<std::size_t>(per * per * n), g * g), scatter(static_cast<std::size_t>(g * g));
  for (std::int64_t y = 0; y < g; ++y)
    for (std::int64_t x = 0; x < g; ++x) {
      const std::int64_t slot = ((y / win) * per + x / win) * n + (y % win) * win + x % win;
      gather[static_cast<std::size_t>(slot)] = y * g + x;
      scatter[static_cast<std::size_t>(y * g + x)] = slot;
    }
  Windows w;
  w.count = per * per;
  w.gather = Array(ctx_, DType::kI64, static_cast<std::int64_t>(gather.size()));
  w.gather.upload(gather.data(), static_cast<std::int64_t>(gather.size()));
  w.scatter = Array(ctx_, DType::kI64, g * g);
  w.scatter.upload(scatter.data(), g * g);
  return windows_.emplace(g, std::move(w)).first->second;
}

void VisionEncoder::project(const float* x, std::int64_t m, std::int64_t k, const std::uint16_t* w, std::int64_t n,
                            const float* bias, float* y, bool accumulate) const {
  // Scratch kept across calls (every call is ordered on the one stream):
  // the split-k workspace, and x rounded to bf16.
  auto grown = [&](Array& a, DType type, std::int64_t count) -> Array& {
    if (a.count() < count) a = Array(ctx_, type, count);
    return a;
  };
  const std::int64_t floats = linear_workspace_floats(m, k, n);
  float* ws = floats > 0 ? grown(split_ws_, DType::kF32, floats).f32() : nullptr;
  if (m > 1 && k % 64 == 0 && (n >= k || accumulate)) {
    // x rounded once (the rounding the product applies anyway, bit for bit),
    // then tiles straight from memory into LDS. The pass costs 6 bytes per
    // element of x, so it pays where the product is at least as wide as x,
    // or where it saves the residual add's pass.
    Array& xb = grown(x_bf16_, DType::kBF16, m * k);
    round_bf16(ctx_, x, m * k, xb.bf16());
    project_bf16(xb.bf16(), m, k, w, n, bias, y, accumulate);
    return;
  }
  if (accumulate) {
    Array t = f32(ctx_, m * n);
    linear(ctx_, x, m, k, w, n, bias, t.f32(), ws, floats);
    add_inplace(ctx_, y, t.f32(), m * n);
    return;
  }
  linear(ctx_, x, m, k, w, n, bias, y, ws, floats);
}

void VisionEncoder::project_bf16(const std::uint16_t* xb, std::int64_t m, std::int64_t k, const std::uint16_t* w,
                                 std::int64_t n, const float* bias, float* y, bool accumulate) const {
  const std::int64_t floats = linear_workspace_floats(m, k, n);
  if (floats > 0 && split_ws_.count() < floats) split_ws_ = Array(ctx_, DType::kF32, floats);
  float* ws = floats > 0 ? split_ws_.f32() : nullptr;
  if (accumulate) {
    linear_bf16x_add(ctx_, xb, m, k, w, n, bias, y, ws, floats);
  } else {
    linear_bf16x(ctx_, xb, m, k, w, n, bias, y, ws, floats);
  }
}

// A LayerNorm whose only reader is a projection, straight into bf16 (the
// rounding the projection applies), in project()'s scratch; x untouched.
// Null for rows wider than the one-row kernel's 16384 columns.
const std::uint16_t* VisionEncoder::normed_bf16(const float* x, std::int64_t rows, std::int64_t c, const float* w,
                                                const float* b, float eps) const {
  if (c > 16384) return nullptr;
  if (x_bf16_.count() < rows * c) x_bf16_ = Array(ctx_, DType::kBF16, rows * c);
  layer_norm_to_bf16(ctx_, x, w, b, x_bf16_.bf16(), rows, c, eps);
  return x_bf16_.bf16();
}

// An MLP's activation straight into bf16 (the rounding its second
// projection applies), in project()'s scratch.
// y = LN(x) w^T + bias, x untouched: through bf16 where the one-row kernel
// takes the width, else LN into `normed` (fp32) and project().
void VisionEncoder::norm_project(const float* x, std::int64_t rows, std::int64_t c, const float* ln_w,
                                 const float* ln_b, float eps, Array& normed, const std::uint16_t* w, std::int64_t n,
                                 const float* bias, float* y) const {
  if (const std::uint16_t* xb = normed_bf16(x, rows, c, ln_w, ln_b, eps)) {
    project_bf16(xb, rows, c, w, n, bias, y);
    return;
  }
  copy(ctx_, normed.f32(), x, rows * c);
  layer_norm(ctx_, normed.f32(), ln_w, ln_b, rows, c, eps);
  project(normed.f32(), rows, c, w, n, bias, y);
}

bool VisionEncoder::mlp_bf16(float* x, std::int64_t rows, std::int64_t c, const float* ln_w, const float* ln_b,
                             float eps, const std::uint16_t* w1, std::int64_t hidden, const float* b1,
                             const std::uint16_t* w2, const float* b2, bool quick) const {
  if (c % 64 != 0) return false;
  const std::uint16_t* h = normed_bf16(x, rows, c, ln_w, ln_b, eps);
  if (h == nullptr) return false;
  if (act_bf16_.count() < rows * hidden) act_bf16_ = Array(ctx_, DType::kBF16, rows * hidden);
  if (rows >= kWideMlpRows) {
    // many rows: the first product in fp32 through the library's tiles, then
    // the activation into bf16 as its own pass (the same values as the
    // fused epilogue on the same sums; a 1024-pixel view's 12 SAM and 24
    // CLIP MLPs this way took the view from 6.49 to 6.16 ms)
    if (mlp_wide_.count() < rows * hidden) mlp_wide_ = Array(ctx_, DType::kF32, rows * hidden);
    project_bf16(h, rows, c, w1, hidden, b1, mlp_wide_.f32());
    if (quick) {
      quick_gelu_to_bf16(ctx_, mlp_wide_.f32(), act_bf16_.bf16(), rows * hidden);
    } else {
      gelu_erf_to_bf16(ctx_, mlp_wide_.f32(), act_bf16_.bf16(), rows * hidden);
    }
  } else {
    linear_bf16x_act_bf16(ctx_, h, rows, c, w1, hidden, b1, act_bf16_.bf16(), quick);
  }
  project_bf16(act_bf16_.bf16(), rows, hidden, w2, c, b2, x, true);
  return true;
}

const std::uint16_t* VisionEncoder::activated_bf16(const float* x, std::int64_t n, bool quick) const {
  if (x_bf16_.count() < n) x_bf16_ = Array(ctx_, DType::kBF16, n);
  if (quick) {
    quick_gelu_to_bf16(ctx_, x, x_bf16_.bf16(), n);
  } else {
    gelu_erf_to_bf16(ctx_, x, x_bf16_.bf16(), n);
  }
  return x_bf16_.bf16();
}

// Attention of one block over `windows` windows of h x w tokens, rows
// window-major in x [windows * h * w, width] (cuda_vision.cpp:151-172).
// The operands go head-major ([3, heads, rows, hd]) so that every (head,
// window) pair is one slice: with a head dim of 64 or 128 (the model's 64)
// one launch forms scores, bias, softmax and values on the matrix cores;
// with another multiple of 4, three batched launches (scores, the
// relative-position bias + softmax, values); otherwise head by head over all
// windows, as the reference does.
void VisionEncoder::sam_attention(std::size_t index, const float* x, const std::uint16_t* xb, std::int64_t windows,
                                  std::int64_t h, std::int64_t w, float* out, bool accumulate,
                                  const std::int64_t* out_rows, std::int64_t out_count) const {
  const auto& b = w_.sam_blocks[index];
  const std::int64_t c = dims_.sam.width, heads = dims_.sam.heads, hd = c / heads, n = h * w, rows = windows * n;
  Array qkv = f32(ctx_, rows * 3 * c);
  if (xb != nullptr) {
    project_bf16(xb, rows, c, b.qkv, 3 * c, b.qkv_b, qkv.f32());
  } else {
    project(x, rows, c, b.qkv, 3 * c, b.qkv_b, qkv.f32());
  }
  const Array& rh = rel_table(index, true, h);
  const Array& rw = rel_table(index, false, w);
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  if ((hd == 64 || hd == 128) && h + w <= 256) {
    // one pass on the matrix cores: scores, bias, softmax and values per
    // (head, window) slice without the scores reaching memory; slice (head,
    // window) straight from the window-major qkv rows (one window: a global
    // block), into its rows and columns of the merged output, written in
    // bf16 (the rounding the output projection applies) in project()'s
    // scratch, which the qkv projection above has finished reading
    const std::int64_t slices = heads * windows;
    const std::int64_t dots = attention_rel_pos_workspace_floats(slices, h, w);
    Array table = f32(ctx_, dots);  // the bias's dot products, formed once per slice
    if (x_bf16_.count() < rows * c) x_bf16_ = Array(ctx_, DType::kBF16, rows * c);
    std::uint16_t* merged = x_bf16_.bf16();
    const float* q = qkv.f32();
    attention_rel_pos_windows(ctx_, {q, 3 * c, hd}, n * 3 * c, {q + c, 3 * c, hd}, n * 3 * c, {q + 2 * c, 3 * c, hd},
                              n * 3 * c, merged, c, hd, n * c, heads, windows, h, w, hd, scale, rh.f32(), rw.f32(),
                              table.f32(), dots);
    if (out_rows != nullptr) {
      // window slots added straight back into their grid rows (padding dropped)
      linear_bf16x_add_rows(ctx_, merged, rows, c, b.proj, c, b.proj_b, out, out_rows, out_count);
    } else {
      project_bf16(merged, rows, c, b.proj, c, b.proj_b, out, accumulate);
    }
    return;
  }
  Array merged = f32(ctx_, rows * c);
  if (hd % 4 == 0) {
    const std::int64_t slices = heads * windows, part = heads * rows * hd;
    Array split = f32(ctx_, 3 * part), o = f32(ctx_, part), scores = f32(ctx_, slices * n * n);
    split_heads(ctx_, qkv.f32(), rows, 3, heads, hd, split.f32());
    const float* q = split.f32();
    gemm_nt(ctx_, n, n, hd, scale, q, hd, n * hd, q + part, hd, n * hd, scores.f32(), n, n * n, slices);
    rel_pos_softmax_rows(ctx_, scores.f32(), slices, q, hd, h, w, hd, rh.f32(), rw.f32());
    gemm_nn(ctx_, n, hd, n, scores.f32(), n, n * n, q + 2 * part, hd, n * hd, o.f32(), hd, n * hd, slices);
    merge_heads(ctx_, o.f32(), heads, rows, hd, merged.f32());
  } else {
    Array scores = f32(ctx_, windows * n * n);
    for (std::int64_t head = 0; head < heads; ++head) {
      const float* q = qkv.f32() + head * hd;
      gemm_nt(ctx_, n, n, hd, scale, q, 3 * c, n * 3 * c, q + c, 3 * c, n * 3 * c, scores.f32(), n, n * n, windows);
      rel_pos_softmax_rows(ctx_, scores.f32(), windows, q, 3 * c, h, w, hd, rh.f32(), rw.f32());
      gemm_nn(ctx_, n, hd, n, scores.f32(), n, n * n, q + 2 * c, 3 * c, n * 3 * c, merged.f32() + head * hd, c,
              n * c, windows);
    }
  }
  if (out_rows != nullptr) {
    if (x_bf16_.count() < rows * c) x_bf16_ = Array(ctx_, DType::kBF16, rows * c);
    round_bf16(ctx_, merged.f32(), rows * c, x_bf16_.bf16());
    linear_bf16x_add_rows(ctx_, x_bf16_.bf16(), rows, c, b.proj, c, b.proj_b, out, out_rows, out_count);
    return;
  }
  project(merged.f32(), rows, c, b.proj, c, b.proj_b, out, accumulate);
}

// One SAM block over x [g * g, width] (cuda_vision.cpp:174-202).
void VisionEncoder::sam_block(std::size_t index, Array& x, std::int64_t g) const {
  const auto& b = w_.sam_blocks[index];
  const std::int64_t c = dims_.sam.width, cells = g * g;
  const std::uint16_t* normed_b = global_[index] ? normed_bf16(x.f32(), cells, c, b.norm1_w, b.norm1_b, kSamEps)
                                                 : nullptr;
  if (normed_b != nullptr) {
    // a global block: the norm's only reader is the qkv projection, and the
    // output projection adds straight into the residual stream
    sam_attention(index, nullptr, normed_b, 1, g, g, x.f32(), true, nullptr, 0);
  } else if (!global_[index] && c % 64 == 0 && c <= 16384) {
    // windows (a width of whole 64-column steps): the norm straight into
    // bf16 rows (the rounding the qkv projection applies), gathered into the
    // windows as pairs of bf16; the buffer's row past the grid is zero once
    // and for all (the padding)
    const std::int64_t win = dims_.sam.window;
    const Windows& wi = windows(g);
    const std::int64_t rows = wi.count * win * win;
    auto it = win_normed_.find(g);
    if (it == win_normed_.end()) {
      it = win_normed_.emplace(g, Array(ctx_, DType::kBF16, (cells + 1) * c)).first;
      it->second.zero();
    }
    const Array& nb = it->second;
    layer_norm_to_bf16(ctx_, x.f32(), b.norm1_w, b.norm1_b, nb.bf16(), cells, c, kSamEps);
    Array slots(ctx_, DType::kBF16, rows * c);
    gather_rows(ctx_, reinterpret_cast<const float*>(nb.bf16()), wi.gather.i64(), rows, c / 2,
                reinterpret_cast<float*>(slots.bf16()));
    // the output projection adds each slot back into its grid row of x
    sam_attention(index, nullptr, slots.bf16(), wi.count, win, win, x.f32(), true, wi.gather.i64(), cells);
  } else {
    Array attended = f32(ctx_, cells * c);
    Array normed = f32(ctx_, (cells + 1) * c);  // the extra zero row fills the windows' padding
    normed.zero();
    copy(ctx_, normed.f32(), x.f32(), cells * c);
    layer_norm(ctx_, normed.f32(), b.norm1_w, b.norm1_b, cells, c, kSamEps);
    if (global_[index]) {
      sam_attention(index, normed.f32(), nullptr, 1, g, g, attended.f32(), false, nullptr, 0);
    } else {
      const std::int64_t win = dims_.sam.window;
      const Windows& wi = windows(g);
      const std::int64_t rows = wi.count * win * win;
      Array slots = f32(ctx_, rows * c), out = f32(ctx_, rows * c);
      gather_rows(ctx_, normed.f32(), wi.gather.i64(), rows, c, slots.f32());
      sam_attention(index, slots.f32(), nullptr, wi.count, win, win, out.f32(), false, nullptr, 0);
      gather_rows(ctx_, out.f32(), wi.scatter.i64(), cells, c, attended.f32());
    }
    add_inplace(ctx_, x.f32(), attended.f32(), cells * c);
  }

  if (mlp_bf16(x.f32(), cells, c, b.norm2_w, b.norm2_b, kSamEps, b.lin1, dims_.sam.mlp, b.lin1_b, b.lin2, b.lin2_b,
               false)) {
    return;
  }
  Array wide = f32(ctx_, cells * dims_.sam.mlp);
  if (const std::uint16_t* h2 = normed_bf16(x.f32(), cells, c, b.norm2_w, b.norm2_b, kSamEps)) {
    project_bf16(h2, cells, c, b.lin1, dims_.sam.mlp, b.lin1_b, wide.f32());
  } else {
    Array hidden = f32(ctx_, cells * c);
    copy(ctx_, hidden.f32(), x.f32(), cells * c);
    layer_norm(ctx_, hidden.f32(), b.norm2_w, b.norm2_b, cells, c, kSamEps);
    project(hidden.f32(), cells, c, b.lin1, dims_.sam.mlp, b.lin1_b, wide.f32());
  }
  project_bf16(activated_bf16(wide.f32(), cells * dims_.sam.mlp, false), cells, dims_.sam.mlp, b.lin2, c, b.lin2_b,
               x.f32(), true);
}

// A 3 x 3 convolution (padding 1) of rows hwc [side * side, in_c] into rows
// out [out_side^2, out_c]: to channel-major, the patch gather, the product.
void VisionEncoder::conv3(const float* hwc, std::int64_t side, std::int64_t in_c, const std::uint16_t* w,
                          std::int64_t out_c, int stride, Array& out, std::int64_t& out_side) const {
  Array chw = f32(ctx_, side * side * in_c);
  hwc_to_chw(ctx_, hwc, side, side, in_c, chw.f32());
  out_side = (side + 2 - 3) / stride + 1;
  out = f32(ctx_, out_side * out_side * out_c);
  if ((in_c * 9) % 64 == 0) {
    // the patches straight into bf16 (the rounding the product applies), its
    // tiles straight from memory into LDS
    Array patches(ctx_, DType::kBF16, out_side * out_side * in_c * 9);
    im2col(ctx_, chw.f32(), in_c, side, side, 3, 3, stride, 1, patches.bf16());
    project_bf16(patches.bf16(), out_side * out_side, in_c * 9, w, out_c, nullptr, out.f32());
    return;
  }
  Array patches = f32(ctx_, out_side * out_side * in_c * 9);
  im2col(ctx_, chw.f32(), in_c, side, side, 3, 3, stride, 1, patches.f32());
  project(patches.f32(), out_side * out_side, in_c * 9, w, out_c, nullptr, out.f32());
}

// SAM over one image into cells [g4 * g4, net3] (cuda_vision.cpp:204-237).
void VisionEncoder::sam_forward(const float* image, std::int64_t size, Array& cells) const {
  const SamDims& s = dims_.sam;
  const std::int64_t p = s.patch, g = size / p, c = s.width;
  Array x = f32(ctx_, g * g * c);
  if ((3 * p * p) % 64 == 0) {
    // the patches straight into bf16, as in conv3
    Array cols(ctx_, DType::kBF16, g * g * 3 * p * p);
    im2col(ctx_, image, 3, size, size, p, p, static_cast<int>(p), 0, cols.bf16());
    project_bf16(cols.bf16(), g * g, 3 * p * p, w_.patch, c, w_.patch_b, x.f32());
  } else {
    Array cols = f32(ctx_, g * g * 3 * p * p);
    im2col(ctx_, image, 3, size, size, p, p, static_cast<int>(p), 0, cols.f32());
    project(cols.f32(), g * g, 3 * p * p, w_.patch, c, w_.patch_b, x.f32());
  }
  add_inplace(ctx_, x.f32(), sam_positions(g).f32(), g * g * c);
  for (std::size_t i = 0; i < w_.sam_blocks.size(); ++i) sam_block(i, x, g);

  Array y = f32(ctx_, g * g * s.neck);
  project(x.f32(), g * g, c, w_.neck0, s.neck, nullptr, y.f32());
  layer_norm(ctx_, y.f32(), w_.neck1_w, w_.neck1_b, g * g, s.neck, kSamEps);
  Array z, n2;
  std::int64_t s1 = 0, s2 = 0, s3 = 0;
  conv3(y.f32(), g, s.neck, w_.neck2, s.neck, 1, z, s1);
  layer_norm(ctx_, z.f32(), w_.neck3_w, w_.neck3_b, s1 * s1, s.neck, kSamEps);
  conv3(z.f32(), s1, s.neck, w_.net2, s.net2, 2, n2, s2);
  conv3(n2.f32(), s2, s.net2, w_.net3, s.net3, 2, cells, s3);
}

// CLIP over the cells (cuda_vision.cpp:239-266): x [1 + g * g, width].
void VisionEncoder::clip_forward(const float* cells, std::int64_t g, Array& x) const {
  const ClipDims& cd = dims_.clip;
  const std::int64_t c = cd.width, n = 1 + g * g, heads = cd.heads, hd = c / heads;
  x = f32(ctx_, n * c);
  copy(ctx_, x.f32(), w_.class_embedding, c);
  copy(ctx_, x.f32() + c, cells, g * g * c);
  add_inplace(ctx_, x.f32(), clip_positions(g).f32(), n * c);
  layer_norm(ctx_, x.f32(), w_.pre_ln_w, w_.pre_ln_b, n, c, kClipEps);
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  const bool one_pass = hd == 64 || hd == 128;  // attention on the matrix cores
  const bool split = !one_pass && hd % 4 == 0;   // head-major operands, as in sam_attention
  Array normed = f32(ctx_, n * c), qkv = f32(ctx_, n * 3 * c), scores = f32(ctx_, one_pass ? 1 : heads * n * n);
  Array merged = f32(ctx_, one_pass ? 1 : n * c), wide = f32(ctx_, n * cd.mlp);
  Array merged16(ctx_, DType::kBF16, one_pass ? n * c : 1);
  Array hm = f32(ctx_, split ? 3 * n * c : 1), o = f32(ctx_, split ? n * c : 1);
  for (const auto& l : w_.clip_layers) {
    norm_project(x.f32(), n, c, l.ln1_w, l.ln1_b, kClipEps, normed, l.qkv, 3 * c, l.qkv_b, qkv.f32());
    if (one_pass) {
      // straight from the projection's rows into the heads' columns, in
      // bf16 (the rounding the output projection applies)
      const float* q = qkv.f32();
      attention(ctx_, {q, 3 * c, hd}, {q + c, 3 * c, hd}, {q + 2 * c, 3 * c, hd}, merged16.bf16(), c, hd, heads, n, n,
                hd, scale, nullptr, 0);
      project_bf16(merged16.bf16(), n, c, l.out, c, l.out_b, x.f32(), true);
    } else if (split) {
      split_heads(ctx_, qkv.f32(), n, 3, heads, hd, hm.f32());
      const float* q = hm.f32();
      gemm_nt(ctx_, n, n, hd, scale, q, hd, n * hd, q + n * c, hd, n * hd, scores.f32(), n, n * n, heads);
      softmax_rows(ctx_, scores.f32(), heads * n, n);
      gemm_nn(ctx_, n, hd, n, scores.f32(), n, n * n, q + 2 * n * c, hd, n * hd, o.f32(), hd, n * hd, heads);
      merge_heads(ctx_, o.f32(), heads, n, hd, merged.f32());
      project(merged.f32(), n, c, l.out, c, l.out_b, x.f32(), true);
    } else {
      gemm_nt(ctx_, n, n, hd, scale, qkv.f32(), 3 * c, hd, qkv.f32() + c, 3 * c, hd, scores.f32(), n, n * n, heads);
      softmax_rows(ctx_, scores.f32(), heads * n, n);
      gemm_nn(ctx_, n, hd, n, scores.f32(), n, n * n, qkv.f32() + 2 * c, 3 * c, hd, merged.f32(), c, hd, heads);
      project(merged.f32(), n, c, l.out, c, l.out_b, x.f32(), true);
    }
    if (!mlp_bf16(x.f32(), n, c, l.ln2_w, l.ln2_b, kClipEps, l.fc1, cd.mlp, l.fc1_b, l.fc2, l.fc2_b, true)) {
      norm_project(x.f32(), n, c, l.ln2_w, l.ln2_b, kClipEps, normed, l.fc1, cd.mlp, l.fc1_b, wide.f32());
      project_bf16(activated_bf16(wide.f32(), n * cd.mlp, true), n, cd.mlp, l.fc2, c, l.fc2_b, x.f32(), true);
    }
  }
}

void VisionEncoder::encode_view(const float* image_device, std::int64_t size, float* out) const {
  need(size >= 64 && size % 64 == 0, "image must be [3, S, S] with S a multiple of 64");
  Array cells;
  sam_forward(image_device, size, cells);
  const std::int64_t g = grid(size), n = g * g, cw = dims_.clip.width, sw = dims_.sam.net3;
  Array clip;
  clip_forward(cells.f32(), g, clip);
  Array joined = f32(ctx_, n * (cw + sw));
  concat_cols(ctx_, clip.f32() + cw, cw, cells.f32(), sw, n, joined.f32());  // the class row dropped
  project(joined.f32(), n, cw + sw, w_.projector, dims_.hidden, w_.projector_b, out);
}

std::vector<float> VisionEncoder::encode_view(const View& image) const {
  need(image.size >= 64 && image.size % 64 == 0 &&
           static_cast<std::int64_t>(image.pixels.size()) == 3 * image.size * image.size,
       "image must be [3, S, S] with S a multiple of 64");
  const Array pixels = upload_f32(ctx_, image.pixels);
  const std::int64_t g = grid(image.size);
  Array out = f32(ctx_, g * g * dims_.hidden);
  encode_view(pixels.f32(), image.size, out.f32());
  return out.download();
}

std::vector<float> VisionEncoder::encode_page(const View& global, const std::vector<View>& tiles,
                                              std::int64_t tiles_wide, std::int64_t tiles_high) const {
  const std::int64_t width = dims_.hidden;
  std::vector<float> rows;
  auto append_grid = [&](const float* cells, std::int64_t grid_rows, std::int64_t grid_cols) {
    for (std::int64_t r = 0; r < grid_rows; ++r) {
      rows.insert(rows.end(), cells + r * grid_cols * width, cells + (r + 1) * grid_cols * width);
      rows.insert(rows.end(), w_.newline.begin(), w_.newline.end());
    }
  };
  if (!tiles.empty()) {
    need(static_cast<std::int64_t>(tiles.size()) == tiles_wide * tiles_high,
         "encode_page: tile count does not match the tile grid");
    std::vector<std::vector<float>> feats;
    for (const View& t : tiles) feats.push_back(encode_view(t));
    const std::int64_t g = grid(tiles.front().size), cols = tiles_wide * g;
    for (const View& t : tiles) need(t.size == tiles.front().size, "encode_page: tiles of different sizes");
    std::vector<float> stitched(static_cast<std::size_t>(tiles_high * g * cols * width));
    for (std::int64_t ty = 0; ty < tiles_high; ++ty)
      for (std::int64_t tx = 0; tx < tiles_wide; ++tx) {
        const auto& f = feats[static_cast<std::size_t>(ty * tiles_wide + tx)];
        for (std::int64_t r = 0; r < g; ++r) {
          std::copy_n(f.begin() + r * g * width, g * width,
                      stitched.begin() + ((ty * g + r) * cols + tx * g) * width);
        }
      }
    append_grid(stitched.data(), tiles_high * g, cols);
  }
  const std::vector<float> view = encode_view(global);
  const std::int64_t g = grid(global.size);
  append_grid(view.data(), g, g);
  rows.insert(rows.end(), w_.separator.begin(), w_.separator.end());
  return rows;
}

}  // namespace uocr::rocm
