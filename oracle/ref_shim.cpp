// ref_shim.cpp: a C entry-point harness over the reference's own CPU ops,
// compiled together with the reference sources where they lie
// (src/backend/reference/ops.cpp, src/model/page_rope.cpp) into
// oracle/_ref/libuocr_ref.so by oracle/Makefile.
//
// TEST INFRASTRUCTURE ONLY: tests/test_oracle.py uses it to check the C
// restatement in oracle/uocr_oracle.c bit for bit against the reference's
// code. No product path and no GPU run loads it. This file holds no
// reference code: it only adapts raw pointers to the reference's Tensor.

#include <cstdint>
#include <cstring>
#include <vector>

#include "backend/reference/ops.h"
#include "backend/reference/parallel.h"
#include "model/attention_plan.h"
#include "model/block_router.h"
#include "model/page_rope.h"
#include "tensor/dtype.h"
#include "tensor/tensor.h"

namespace ref = uocr::reference;

namespace {

uocr::Tensor wrap(const float* p, std::vector<std::int64_t> shape) {
  const std::int64_t n = uocr::Tensor::count(shape);
  return uocr::Tensor(std::move(shape), std::vector<float>(p, p + n));
}

void unwrap(const uocr::Tensor& t, float* out) { std::memcpy(out, t.data(), static_cast<std::size_t>(t.numel()) * 4); }

}  // namespace

extern "C" {

__attribute__((visibility("default"))) void ref_set_threads(unsigned t) { ref::set_thread_count(t); }

__attribute__((visibility("default"))) std::uint16_t ref_f32_to_bf16(float v) { return uocr::f32_to_bf16(v); }
__attribute__((visibility("default"))) float ref_bf16_to_f32(std::uint16_t b) { return uocr::bf16_to_f32(b); }

__attribute__((visibility("default"))) void ref_rms_norm(float* x, const float* w, std::int64_t rows,
                                                         std::int64_t cols, float eps) {
  uocr::Tensor t = wrap(x, {rows, cols});
  ref::rms_norm(t, wrap(w, {cols}), eps);
  unwrap(t, x);
}

__attribute__((visibility("default"))) void ref_layer_norm(float* x, const float* w, const float* b,
                                                           std::int64_t rows, std::int64_t cols, float eps) {
  uocr::Tensor t = wrap(x, {rows, cols});
  ref::layer_norm(t, wrap(w, {cols}), wrap(b, {cols}), eps);
  unwrap(t, x);
}

__attribute__((visibility("default"))) void ref_gelu_erf(float* x, std::int64_t n) {
  uocr::Tensor t = wrap(x, {n});
  ref::gelu_erf(t);
  unwrap(t, x);
}

__attribute__((visibility("default"))) void ref_silu(float* x, std::int64_t n) {
  uocr::Tensor t = wrap(x, {n});
  ref::silu(t);
  unwrap(t, x);
}

// PageRope's own frequency tables: inv_tok gets dim/2 - page_pairs entries,
// inv_page gets page_pairs.
__attribute__((visibility("default"))) void ref_rope_tables(std::int64_t dim, double tok_theta, double page_theta,
                                                            std::int64_t page_pairs, float* inv_tok,
                                                            float* inv_page) {
  const uocr::PageRope rope(dim, tok_theta, page_theta, page_pairs, 2);
  std::memcpy(inv_tok, rope.inv_tok().data(), rope.inv_tok().size() * 4);
  std::memcpy(inv_page, rope.inv_page().data(), rope.inv_page().size() * 4);
}

// PageRope::apply over x [rows, width] (width a multiple of dim) at
// coordinates (tok[r], page[r]).
__attribute__((visibility("default"))) void ref_rope_apply(float* x, std::int64_t rows, std::int64_t width,
                                                           std::int64_t dim, double tok_theta, double page_theta,
                                                           std::int64_t page_pairs, std::int64_t page_mod,
                                                           const std::int64_t* tok, const std::int64_t* page) {
  const uocr::PageRope rope(dim, tok_theta, page_theta, page_pairs, page_mod);
  uocr::Tensor t = wrap(x, {rows, width});
  std::vector<uocr::RopeCoord> coords(static_cast<std::size_t>(rows));
  for (std::int64_t r = 0; r < rows; ++r) coords[static_cast<std::size_t>(r)] = {tok[r], page[r]};
  rope.apply(t, coords);
  unwrap(t, x);
}

__attribute__((visibility("default"))) void ref_quick_gelu(float* x, std::int64_t n) {
  uocr::Tensor t = wrap(x, {n});
  ref::quick_gelu(t);
  unwrap(t, x);
}

__attribute__((visibility("default"))) void ref_softmax_rows(float* x, std::int64_t rows, std::int64_t cols) {
  uocr::Tensor t = wrap(x, {rows, cols});
  ref::softmax_rows(t);
  unwrap(t, x);
}

// y [m, n] = linear(x [m, k], w [n, k], bias [n] or null).
__attribute__((visibility("default"))) void ref_linear(const float* x, std::int64_t m, std::int64_t k, const float* w,
                                                       std::int64_t n, const float* bias, float* y) {
  const uocr::Tensor b = bias != nullptr ? wrap(bias, {n}) : uocr::Tensor();
  const uocr::Tensor out = ref::linear(wrap(x, {m, k}), wrap(w, {n, k}), bias != nullptr ? &b : nullptr);
  unwrap(out, y);
}

// out [lq, dv] = attention_head(q [lq, d], k [lk, d], v [lk, dv], bias [lq, lk] or null, scale).
__attribute__((visibility("default"))) void ref_attention_head(const float* q, std::int64_t lq, const float* k,
                                                               std::int64_t lk, std::int64_t d, const float* v,
                                                               std::int64_t dv, const float* bias, float scale,
                                                               float* out) {
  const uocr::Tensor b = bias != nullptr ? wrap(bias, {lq, lk}) : uocr::Tensor();
  const uocr::Tensor o = ref::attention_head(wrap(q, {lq, d}), wrap(k, {lk, d}), wrap(v, {lk, dv}),
                                             bias != nullptr ? &b : nullptr, scale);
  unwrap(o, out);
}

// block_summaries(rk [keys, d], head_cls [d], block_size) -> out [ceil(keys / block_size), d].
__attribute__((visibility("default"))) void ref_block_summaries(const float* rk, std::int64_t keys, std::int64_t d,
                                                                const float* cls, std::int64_t block_size,
                                                                float* out) {
  unwrap(uocr::block_summaries(wrap(rk, {keys, d}), wrap(cls, {d}), block_size), out);
}

// block_scores(rq [lq, d], summaries [nblk, d], q_pos [lq]) -> out [lq, nblk].
__attribute__((visibility("default"))) void ref_block_scores(const float* rq, std::int64_t lq,
                                                             const float* summaries, std::int64_t nblk, std::int64_t d,
                                                             const std::int64_t* q_pos, std::int64_t block_size,
                                                             std::int64_t local_blocks, float* out) {
  uocr::RouterParams p;
  p.block_size = block_size;
  p.local_blocks = local_blocks;
  const std::vector<std::int64_t> pos(q_pos, q_pos + lq);
  unwrap(uocr::block_scores(wrap(rq, {lq, d}), wrap(summaries, {nblk, d}), pos, 0, p), out);
}

__attribute__((visibility("default"))) void ref_entmax15(float* x, std::int64_t n) {
  std::vector<float> v(x, x + n);
  uocr::entmax15(v);
  std::memcpy(x, v.data(), static_cast<std::size_t>(n) * 4);
}

// select_blocks(scores [lq, nblk], candidate [lq, nblk] or null) -> block,
// bias, valid [lq, width]; returns width.
__attribute__((visibility("default"))) std::int64_t ref_select_blocks(
    const float* scores, std::int64_t lq, std::int64_t nblk, const std::uint8_t* candidate, std::int64_t top_m,
    std::int64_t top_k, float idx_scale, float floor_p, float sigma, std::int64_t* block, float* bias,
    std::uint8_t* valid) {
  uocr::RouterParams p;
  p.top_m = top_m;
  p.top_k = top_k;
  p.idx_scale = idx_scale;
  p.floor = floor_p;
  p.sigma = sigma;
  std::vector<std::uint8_t> cand;
  if (candidate != nullptr) cand.assign(candidate, candidate + lq * nblk);
  const uocr::BlockSelection sel = uocr::select_blocks(wrap(scores, {lq, nblk}), cand, p);
  std::memcpy(block, sel.block.data(), sel.block.size() * 8);
  std::memcpy(bias, sel.bias.data(), sel.bias.size() * 4);
  std::memcpy(valid, sel.valid.data(), sel.valid.size());
  return sel.width;
}

// key_mask of a selection (block, bias, valid [rows, width]) -> mask [rows, keys].
__attribute__((visibility("default"))) void ref_key_mask(const std::int64_t* block, const float* bias,
                                                         const std::uint8_t* valid, std::int64_t width,
                                                         std::int64_t rows, std::int64_t first_pos, std::int64_t keys,
                                                         std::int64_t block_size, std::int64_t local_blocks,
                                                         float* mask) {
  uocr::BlockSelection sel;
  sel.width = width;
  sel.block.assign(block, block + rows * width);
  sel.bias.assign(bias, bias + rows * width);
  sel.valid.assign(valid, valid + rows * width);
  uocr::RouterParams p;
  p.block_size = block_size;
  p.local_blocks = local_blocks;
  const std::vector<float> m = uocr::key_mask(sel, rows, first_pos, keys, p);
  std::memcpy(mask, m.data(), m.size() * 4);
}

// out [o, oh, ow] = conv2d(x [c, h, w], weight [o, c, kh, kw], bias [o] or null, stride, pad).
__attribute__((visibility("default"))) void ref_conv2d(const float* x, std::int64_t c, std::int64_t h, std::int64_t w,
                                                       const float* weight, const float* bias, std::int64_t o,
                                                       std::int64_t kh, std::int64_t kw, std::int64_t stride,
                                                       std::int64_t pad, float* out) {
  const uocr::Tensor b = bias != nullptr ? wrap(bias, {o}) : uocr::Tensor();
  const uocr::Tensor y = ref::conv2d(wrap(x, {c, h, w}), wrap(weight, {o, c, kh, kw}), bias != nullptr ? &b : nullptr,
                                     static_cast<int>(stride), static_cast<int>(pad));
  unwrap(y, out);
}

// layer_norm_channels on x [c, h, w] in place.
__attribute__((visibility("default"))) void ref_layer_norm_channels(float* x, const float* w, const float* b,
                                                                    std::int64_t c, std::int64_t h, std::int64_t wd,
                                                                    float eps) {
  uocr::Tensor t = wrap(x, {c, h, wd});
  ref::layer_norm_channels(t, wrap(w, {c}), wrap(b, {c}), eps);
  unwrap(t, x);
}

// out [c, oh, ow] = resize_bicubic_aa(x [c, h, w]).
__attribute__((visibility("default"))) void ref_resize_bicubic_aa(const float* x, std::int64_t c, std::int64_t h,
                                                                  std::int64_t w, std::int64_t oh, std::int64_t ow,
                                                                  float* out) {
  unwrap(ref::resize_bicubic_aa(wrap(x, {c, h, w}), oh, ow), out);
}

// out [out_len, c] = resize_linear_rows(x [len, c]).
__attribute__((visibility("default"))) void ref_resize_linear_rows(const float* x, std::int64_t len, std::int64_t c,
                                                                   std::int64_t out_len, float* out) {
  unwrap(ref::resize_linear_rows(wrap(x, {len, c}), out_len), out);
}

// y [h, w, c] = chw_to_hwc(x [c, h, w]); y [c, h, w] = hwc_to_chw(x [h, w, c]).
__attribute__((visibility("default"))) void ref_chw_to_hwc(const float* x, std::int64_t c, std::int64_t h,
                                                           std::int64_t w, float* y) {
  unwrap(ref::chw_to_hwc(wrap(x, {c, h, w})), y);
}
__attribute__((visibility("default"))) void ref_hwc_to_chw(const float* x, std::int64_t h, std::int64_t w,
                                                           std::int64_t c, float* y) {
  unwrap(ref::hwc_to_chw(wrap(x, {h, w, c})), y);
}

}  // extern "C"
