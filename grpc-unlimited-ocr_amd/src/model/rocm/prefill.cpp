// DecodeStep::prefill: the prompt's pass through the decoder, eager (not
// captured), writing the caches the captured step reads afterwards.

#include <algorithm>
#include <cmath>
#include <stdexcept>
#include <string>
#include <vector>

#include "backend/rocm/decode_ops.h"
#include "backend/rocm/ops.h"
#include "model/rocm/decode_step.h"

namespace uocr::rocm {
namespace {

void need(bool ok, const char* what) {
  if (!ok) throw std::invalid_argument(std::string("DecodeStep::prefill: ") + what);
}

Array ids_on_device(const Context& ctx, const std::vector<std::int64_t>& ids) {
  Array a(ctx, DType::kI64, std::max<std::int64_t>(1, static_cast<std::int64_t>(ids.size())));
  if (!ids.empty()) a.upload(ids.data(), static_cast<std::int64_t>(ids.size()));
  return a;
}

// The bf16 rounding of rows [rows, cols] that every projection of them takes
// (rounded once for all of them).
Array rounded(const Context& ctx, const float* x, std::int64_t n) {
  Array r(ctx, DType::kBF16, n);
  round_bf16(ctx, x, n, r.bf16());
  return r;
}

// y [rows, hidden] = silu(x Wg) * (x Wu) Wd over bf16 weights: gate and up
// [ffn, hidden], down [hidden, ffn] (the reference's mlp,
// cuda_decoder.cpp:117-135); xb is x rounded to bf16.
// The same with gate and up stacked [2 ffn, hidden]: one product gives
// [gate | up] per row, then the SwiGLU over the concatenated rows.
void mlp_stacked(const Context& ctx, const std::uint16_t* xb, std::int64_t rows, std::int64_t hidden,
                 const std::uint16_t* gate_up, const std::uint16_t* down, std::int64_t ffn, float* y) {
  Array gu(ctx, DType::kF32, rows * 2 * ffn), act(ctx, DType::kF32, rows * ffn);
  linear_bf16x(ctx, xb, rows, hidden, gate_up, 2 * ffn, nullptr, gu.f32());
  swiglu(ctx, gu.f32(), act.f32(), rows, ffn);
  const Array ab = rounded(ctx, act.f32(), rows * ffn);
  linear_bf16x(ctx, ab.bf16(), rows, ffn, down, hidden, nullptr, y);
}

void mlp(const Context& ctx, const std::uint16_t* xb, std::int64_t rows, std::int64_t hidden, const std::uint16_t* gate,
         const std::uint16_t* up, const std::uint16_t* down, std::int64_t ffn, float* y) {
  Array g(ctx, DType::kF32, rows * ffn), u(ctx, DType::kF32, rows * ffn);
  linear_bf16x(ctx, xb, rows, hidden, gate, ffn, nullptr, g.f32());
  linear_bf16x(ctx, xb, rows, hidden, up, ffn, nullptr, u.f32());
  silu_mul(ctx, g.f32(), u.f32(), rows * ffn);
  const Array gb = rounded(ctx, g.f32(), rows * ffn);
  linear_bf16x(ctx, gb.bf16(), rows, ffn, down, hidden, nullptr, y);
}

}  // namespace

std::vector<float> DecodeStep::prefill(const std::vector<float>& x_host, const std::vector<RopeCoord>& coords,
                                       const std::vector<std::int64_t>& query_pages) {
  const auto& d = dims_;
  const auto rows = static_cast<std::int64_t>(coords.size());
  const std::int64_t H = d.hidden, W = d.heads * d.head_dim, hd = d.head_dim, D = d.index_dim;
  need(rows >= 1, "no rows");
  need(static_cast<std::int64_t>(x_host.size()) == rows * H, "x must be [rows, hidden]");
  need(query_pages.empty() || static_cast<std::int64_t>(query_pages.size()) == rows,
       "one query page per row, or none");
  const std::int64_t first = length_, keys = first + rows;
  need(keys <= d.capacity, "the prompt runs past the cache (reserve)");
  const std::int64_t bs = d.router.block_size, nblk = (keys + bs - 1) / bs;
  const std::int64_t n_tok = hd / 2 - d.page_pairs;
  const float eps = d.eps;
  auto f32 = [&](std::int64_t n) { return Array(ctx_, DType::kF32, std::max<std::int64_t>(n, 1)); };

  std::vector<std::int64_t> tok(static_cast<std::size_t>(rows)), page(static_cast<std::size_t>(rows));
  for (std::int64_t r = 0; r < rows; ++r) {
    tok[static_cast<std::size_t>(r)] = coords[static_cast<std::size_t>(r)].tok;
    page[static_cast<std::size_t>(r)] = coords[static_cast<std::size_t>(r)].page;
  }
  std::vector<std::int64_t> qp = query_pages;
  if (qp.empty()) qp.assign(static_cast<std::size_t>(rows), -1);
  const Array tok_d = ids_on_device(ctx_, tok), page_d = ids_on_device(ctx_, page), qp_d = ids_on_device(ctx_, qp);
  const float* inv_page = d.page_pairs > 0 ? inv_page_.f32() : nullptr;
  const std::int64_t* block_min = prompt_blocks_ > 0 ? block_min_.i64() : nullptr;
  const std::int64_t* block_max = prompt_blocks_ > 0 ? block_max_.i64() : nullptr;

  Array x = f32(rows * H);
  x.upload(x_host.data(), rows * H);
  Array h = f32(rows * H), delta = f32(rows * H), q = f32(rows * W), rq = f32(rows * D), z = f32(rows * nblk);
  const bool one_pass = hd == 64 || hd == 128;
  const bool split = one_pass && d.split_attention;
  Array mask = f32(rows * keys), scores = f32(one_pass ? 1 : d.heads * rows * keys);
  Array merged = f32(one_pass ? 1 : rows * W);
  // the one-pass attention's bf16 output rows (the o projection's input) and workspace
  Array attn_b(ctx_, DType::kBF16, one_pass ? rows * W : 1);
  const std::int64_t attn_ws_floats = !one_pass ? 1
                                      : split   ? attention_masked_workspace_floats(d.heads, rows, keys, hd)
                                                : attention_workspace_floats(d.heads, rows, keys, hd);
  Array attn_ws = f32(attn_ws_floats);
  // Over a bf16 cache: the new keys and values in fp32 before they are
  // rounded into the cache, and every key and value the prompt attends to
  // widened back from the cache (positions 0 .. keys - 1 gathered in order).
  const bool bf16 = d.bf16_cache;
  Array k_new = f32(bf16 ? rows * W : 1), v_new = f32(bf16 ? rows * W : 1);
  Array k_read = f32(bf16 ? keys * W : 1), v_read = f32(bf16 ? keys * W : 1);
  Array positions;
  if (bf16) {
    std::vector<std::int64_t> all(static_cast<std::size_t>(keys));
    for (std::int64_t i = 0; i < keys; ++i) all[static_cast<std::size_t>(i)] = i;
    positions = ids_on_device(ctx_, all);
  }
  const float inv_sqrt_d = 1.0f / std::sqrt(static_cast<float>(D));
  const float scale = 1.0f / std::sqrt(static_cast<float>(hd));
  prefill_masks_.clear();
  for (std::size_t li = 0; li < layers_.size(); ++li) {
    const LayerWeights& l = layers_[li];
    // input norm (the previous MLP's output added first)
    if (li == 0) {
      copy(ctx_, h.f32(), x.f32(), rows * H);
      rms_norm(ctx_, h.f32(), l.input_norm, rows, H, eps);
    } else {
      add_rms_norm(ctx_, x.f32(), delta.f32(), l.input_norm, h.f32(), rows, H, eps);
    }
    // attention (cuda_decoder.cpp:188-245): the projections, k, v and the
    // router keys straight into the caches at rows first.. (k and v through
    // fp32 rows over a bf16 cache)
    float* kc = bf16 ? k_new.f32() : k_cache_[li].f32() + first * W;
    float* vc = bf16 ? v_new.f32() : v_cache_[li].f32() + first * W;
    float* rkc = router_keys_[li].f32() + first * D;
    const std::uint16_t* wq = l.qkv;
    const std::uint16_t* wk = wq + W * H;
    const std::uint16_t* wv = wk + W * H;
    const std::uint16_t* wrq = wv + W * H;
    const std::uint16_t* wrk = wrq + D * H;
    {
      const Array hb = rounded(ctx_, h.f32(), rows * H);
      linear_bf16x(ctx_, hb.bf16(), rows, H, wq, W, nullptr, q.f32());
      linear_bf16x(ctx_, hb.bf16(), rows, H, wk, W, nullptr, kc);
      linear_bf16x(ctx_, hb.bf16(), rows, H, wv, W, nullptr, vc);
      linear_bf16x(ctx_, hb.bf16(), rows, H, wrq, D, nullptr, rq.f32());
      linear_bf16x(ctx_, hb.bf16(), rows, H, wrk, D, nullptr, rkc);
    }
    router_norm(ctx_, rq.f32(), l.router_q_norm, rows, D, eps);
    router_norm(ctx_, rkc, l.router_k_norm, rows, D, eps);
    for (float* t : {q.f32(), kc}) {
      rope(ctx_, t, rows, d.heads, hd, tok_d.i64(), page_d.i64(), inv_tok_.f32(), n_tok, inv_page, d.page_pairs,
           d.page_mod);
    }
    for (float* t : {rq.f32(), rkc}) {
      rope(ctx_, t, rows, 1, D, tok_d.i64(), page_d.i64(), inv_tok_.f32(), n_tok, inv_page, d.page_pairs,
           d.page_mod);
    }
    const float* k_all = bf16 ? k_read.f32() : k_cache_[li].f32();
    const float* v_all = bf16 ? v_read.f32() : v_cache_[li].f32();
    if (bf16) {
      round_bf16(ctx_, kc, rows * W, k_cache_[li].bf16() + first * W);
      round_bf16(ctx_, vc, rows * W, v_cache_[li].bf16() + first * W);
      gather_rows_bf16(ctx_, k_cache_[li].bf16(), positions.i64(), keys, W, k_read.f32());
      gather_rows_bf16(ctx_, v_cache_[li].bf16(), positions.i64(), keys, W, v_read.f32());
    }
    block_summaries(ctx_, router_keys_[li].f32(), keys, D, l.head_cls, bs, summaries_[li].f32());
    gemm_nt(ctx_, rows, nblk, D, inv_sqrt_d, rq.f32(), D, 0, summaries_[li].f32(), D, 0, z.f32(), nblk, 0, 1);
    route_blocks(ctx_, z.f32(), rows, nblk, first, keys, block_min, block_max, prompt_blocks_, qp_d.i64(), -1,
                 d.router, mask.f32());
    if (d.trace) {
      prefill_masks_.push_back(mask.download());
      prefill_masks_.back().resize(static_cast<std::size_t>(rows * keys));
    }
    if (split) {
      // scores, mask, softmax and values in one pass on the bf16 matrix
      // cores with split operands, each head's columns read in place, the
      // output in bf16 (the rounding the o projection applies to its input)
      attention_masked(ctx_, {q.f32(), W, hd}, {k_all, W, hd}, {v_all, W, hd}, attn_b.bf16(), W, hd, d.heads, rows,
                       keys, hd, scale, mask.f32(), keys, attn_ws.f32(), attn_ws_floats);
      linear_bf16x(ctx_, attn_b.bf16(), rows, W, l.o, H, nullptr, delta.f32());
    } else if (one_pass) {
      // scores, mask, softmax and values in one pass on the fp32 matrix
      // cores, each head's columns read in place, only the key tiles the
      // mask leaves live, the output rounded to bf16 as the o projection
      // takes it
      attention(ctx_, {q.f32(), W, hd}, {k_all, W, hd}, {v_all, W, hd}, attn_b.bf16(), W, hd, d.heads, rows, keys, hd,
                scale, mask.f32(), keys, attn_ws.f32(), attn_ws_floats);
      linear_bf16x(ctx_, attn_b.bf16(), rows, W, l.o, H, nullptr, delta.f32());
    } else {
      gemm_nt(ctx_, rows, keys, hd, scale, q.f32(), W, hd, k_all, W, hd, scores.f32(), keys, rows * keys, d.heads);
      scale_add_mask(ctx_, scores.f32(), 1.0f, mask.f32(), d.heads, rows, keys);
      softmax_rows(ctx_, scores.f32(), d.heads * rows, keys);
      gemm_nn(ctx_, rows, hd, keys, scores.f32(), keys, rows * keys, v_all, W, hd, merged.f32(), W, hd, d.heads);
      const Array mb = rounded(ctx_, merged.f32(), rows * W);
      linear_bf16x(ctx_, mb.bf16(), rows, W, l.o, H, nullptr, delta.f32());
    }
    add_rms_norm(ctx_, x.f32(), delta.f32(), l.post_norm, h.f32(), rows, H, eps);
    const Array hb = rounded(ctx_, h.f32(), rows * H);
    if (l.moe == nullptr) {
      mlp_stacked(ctx_, hb.bf16(), rows, H, gate_up_[li].bf16(), l.down, l.ffn, delta.f32());
      continue;
    }
    // mixture of experts (cuda_decoder.cpp:137-186): the device's softmax
    // top-k per row, each expert over its rows, outputs added in expert order
    const MoeWeights& m = *l.moe;
    Array logits = f32(rows * m.experts), wts = f32(rows * m.top_k);
    Array ids(ctx_, DType::kI64, rows * m.top_k);
    gemm_nt(ctx_, rows, m.experts, H, 1.0f, h.f32(), H, 0, m.gate, H, 0, logits.f32(), m.experts, 0, 1);
    expert_topk(ctx_, logits.f32(), rows, m.experts, m.top_k, ids.i64(), wts.f32());
    std::vector<std::int64_t> ids_h(static_cast<std::size_t>(rows * m.top_k));
    {
      PinnedBuffer pin(ids_h.size() * sizeof(std::int64_t));
      copy_to_host(ctx_, pin, ids.i64(), ids_h.size() * sizeof(std::int64_t));
      ctx_.synchronize();
      std::copy_n(static_cast<const std::int64_t*>(pin.data()), ids_h.size(), ids_h.begin());
    }
    const std::vector<float> wts_h = wts.download();
    std::vector<std::vector<std::int64_t>> rows_of(static_cast<std::size_t>(m.experts));
    std::vector<std::vector<float>> weight_of(static_cast<std::size_t>(m.experts));
    for (std::int64_t r = 0; r < rows; ++r) {
      for (std::int64_t j = 0; j < m.top_k; ++j) {
        const std::size_t at = static_cast<std::size_t>(r * m.top_k + j);
        const std::int64_t e = ids_h[at];
        need(e >= 0 && e < m.experts, "top-k returned an expert outside the stack");
        rows_of[static_cast<std::size_t>(e)].push_back(r);
        weight_of[static_cast<std::size_t>(e)].push_back(wts_h[at]);
      }
    }
    mlp_stacked(ctx_, hb.bf16(), rows, H, gate_up_[li].bf16(), m.shared_down, m.shared_ffn, delta.f32());
    Array routed = f32(rows * H);
    routed.zero();
    for (std::int64_t e = 0; e < m.experts; ++e) {
      const auto& picked = rows_of[static_cast<std::size_t>(e)];
      if (picked.empty()) continue;
      const auto n = static_cast<std::int64_t>(picked.size());
      const Array idx = ids_on_device(ctx_, picked);
      Array w = f32(n);
      w.upload(weight_of[static_cast<std::size_t>(e)].data(), n);
      Array in = f32(n * H), res = f32(n * H);
      gather_rows(ctx_, h.f32(), idx.i64(), n, H, in.f32());
      const Array inb = rounded(ctx_, in.f32(), n * H);
      mlp(ctx_, inb.bf16(), n, H, m.gate_stack + e * m.expert_ffn * H, m.up_stack + e * m.expert_ffn * H,
          m.down_stack + e * H * m.expert_ffn, m.expert_ffn, res.f32());
      scatter_add_rows(ctx_, routed.f32(), idx.i64(), w.f32(), res.f32(), n, H);
    }
    add_inplace(ctx_, delta.f32(), routed.f32(), rows * H);
  }
  add_inplace(ctx_, x.f32(), delta.f32(), rows * H);
  Array last = f32(H), logits = f32(d.vocab);
  copy(ctx_, last.f32(), x.f32() + (rows - 1) * H, H);
  rms_norm(ctx_, last.f32(), final_norm_, 1, H, eps);
  gemv_bf16(ctx_, last.f32(), H, lm_head_, d.vocab, nullptr, logits.f32());
  std::vector<float> out = logits.download();
  length_ = keys;
  return out;
}

}  // namespace uocr::rocm
