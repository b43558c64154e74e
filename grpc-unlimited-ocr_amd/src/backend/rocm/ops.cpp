#include "backend/rocm/ops.h"

#include "uocr_rocm.h"

namespace uocr::rocm {

void add_inplace(const Context& ctx, float* y, const float* x, std::int64_t n) {
  check(uocr_rocm_add_inplace(ctx.stream(), y, x, n));
}

void layer_norm(const Context& ctx, float* x, const float* w, const float* b, std::int64_t rows, std::int64_t cols,
                float eps) {
  check(uocr_rocm_layer_norm(ctx.stream(), x, w, b, rows, cols, eps));
}

void rms_norm(const Context& ctx, float* x, const float* w, std::int64_t rows, std::int64_t cols, float eps) {
  check(uocr_rocm_rms_norm(ctx.stream(), x, w, rows, cols, eps));
}

void gelu_erf(const Context& ctx, float* x, std::int64_t n) { check(uocr_rocm_gelu_erf(ctx.stream(), x, n)); }

void silu_mul(const Context& ctx, float* g, const float* u, std::int64_t n) {
  check(uocr_rocm_silu_mul(ctx.stream(), g, u, n));
}

void rope(const Context& ctx, float* x, std::int64_t rows, std::int64_t heads, std::int64_t dim, const std::int64_t* tok,
          const std::int64_t* page, const float* inv_tok, std::int64_t n_tok, const float* inv_page, std::int64_t n_page,
          std::int64_t page_mod, std::int64_t one_tok, std::int64_t one_page) {
  check(uocr_rocm_rope(ctx.stream(), x, rows, heads, dim, tok, page, inv_tok, n_tok, inv_page, n_page, page_mod,
                       one_tok, one_page));
}

void copy(const Context& ctx, float* dst, const float* src, std::int64_t n) {
  check(uocr_rocm_copy(ctx.stream(), dst, src, n));
}

void gather_rows_bf16(const Context& ctx, const std::uint16_t* table, const std::int64_t* index, std::int64_t rows,
                      std::int64_t cols, float* dst) {
  check(uocr_rocm_gather_rows_bf16(ctx.stream(), table, -1, index, rows, cols, dst));
}

void gather_row_bf16(const Context& ctx, const std::uint16_t* table, std::int64_t one_index, std::int64_t cols,
                     float* dst) {
  check(uocr_rocm_gather_row_bf16(ctx.stream(), table, -1, one_index, cols, dst));
}

void gather_rows_bf16(const Context& ctx, const std::uint16_t* table, std::int64_t table_rows, const std::int64_t* index,
                      std::int64_t rows, std::int64_t cols, float* dst) {
  check(uocr_rocm_gather_rows_bf16(ctx.stream(), table, table_rows, index, rows, cols, dst));
}

void add_rms_norm(const Context& ctx, float* x, const float* delta, const float* w, float* h, std::int64_t rows,
                  std::int64_t cols, float eps) {
  check(uocr_rocm_add_rms_norm(ctx.stream(), x, delta, w, h, rows, cols, eps));
}

void swiglu(const Context& ctx, const float* in, float* out, std::int64_t rows, std::int64_t ffn) {
  check(uocr_rocm_swiglu(ctx.stream(), in, out, rows, ffn));
}

void rope_qk(const Context& ctx, float* q, std::int64_t q_heads, float* k, std::int64_t k_heads, std::int64_t rows,
             std::int64_t dim, const std::int64_t* tok, const std::int64_t* page, const float* inv_tok,
             std::int64_t n_tok, const float* inv_page, std::int64_t n_page, std::int64_t page_mod,
             std::int64_t one_tok, std::int64_t one_page) {
  check(uocr_rocm_rope_qk(ctx.stream(), q, q_heads, k, k_heads, rows, dim, tok, page, inv_tok, n_tok, inv_page, n_page,
                          page_mod, one_tok, one_page));
}

void add_rms_norm_bf16(const Context& ctx, std::uint16_t* x, const std::uint16_t* delta, const float* w,
                       std::uint16_t* h, std::int64_t rows, std::int64_t cols, float eps) {
  check(uocr_rocm_add_rms_norm_bf16(ctx.stream(), x, delta, w, h, rows, cols, eps));
}

void layer_norm_bf16(const Context& ctx, std::uint16_t* x, const float* w, const float* b, std::int64_t rows,
                     std::int64_t cols, float eps) {
  check(uocr_rocm_layer_norm_bf16(ctx.stream(), x, w, b, rows, cols, eps));
}

void gelu_erf_bf16(const Context& ctx, std::uint16_t* x, std::int64_t n) {
  check(uocr_rocm_gelu_erf_bf16(ctx.stream(), x, n));
}

void swiglu_bf16(const Context& ctx, const std::uint16_t* in, std::uint16_t* out, std::int64_t rows,
                 std::int64_t ffn) {
  check(uocr_rocm_swiglu_bf16(ctx.stream(), in, out, rows, ffn));
}

void rope_qk_bf16(const Context& ctx, std::uint16_t* q, std::int64_t q_heads, std::uint16_t* k, std::int64_t k_heads,
                  std::int64_t rows, std::int64_t dim, const std::int64_t* tok, const std::int64_t* page,
                  const float* inv_tok, std::int64_t n_tok, const float* inv_page, std::int64_t n_page,
                  std::int64_t page_mod, std::int64_t one_tok, std::int64_t one_page) {
  check(uocr_rocm_rope_qk_bf16(ctx.stream(), q, q_heads, k, k_heads, rows, dim, tok, page, inv_tok, n_tok, inv_page,
                               n_page, page_mod, one_tok, one_page));
}

void router_norm(const Context& ctx, float* x, const float* w, std::int64_t rows, std::int64_t cols, float eps) {
  check(uocr_rocm_router_norm(ctx.stream(), x, w, rows, cols, eps));
}

void quick_gelu(const Context& ctx, float* x, std::int64_t n) { check(uocr_rocm_quick_gelu(ctx.stream(), x, n)); }

void softmax_rows(const Context& ctx, float* x, std::int64_t rows, std::int64_t cols) {
  check(uocr_rocm_softmax_rows(ctx.stream(), x, rows, cols));
}

void scale_add_mask(const Context& ctx, float* x, float scale, const float* mask, std::int64_t batch, std::int64_t rows,
                    std::int64_t cols) {
  check(uocr_rocm_scale_add_mask(ctx.stream(), x, scale, mask, batch, rows, cols));
}

void gemv_bf16(const Context& ctx, const float* x, std::int64_t k, const std::uint16_t* w, std::int64_t n,
               const float* bias, float* y) {
  check(uocr_rocm_gemv_bf16(ctx.stream(), x, k, w, n, bias, y));
}

void gemm_nt(const Context& ctx, std::int64_t m, std::int64_t n, std::int64_t k, float alpha, const float* a,
             std::int64_t lda, std::int64_t stride_a, const float* b, std::int64_t ldb, std::int64_t stride_b, float* c,
             std::int64_t ldc, std::int64_t stride_c, std::int64_t batch) {
  check(uocr_rocm_gemm_nt(ctx.stream(), m, n, k, alpha, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch));
}

void gemm_nn(const Context& ctx, std::int64_t m, std::int64_t n, std::int64_t k, const float* a, std::int64_t lda,
             std::int64_t stride_a, const float* b, std::int64_t ldb, std::int64_t stride_b, float* c, std::int64_t ldc,
             std::int64_t stride_c, std::int64_t batch) {
  check(uocr_rocm_gemm_nn(ctx.stream(), m, n, k, a, lda, stride_a, b, ldb, stride_b, c, ldc, stride_c, batch));
}

void gather_rows(const Context& ctx, const float* src, const std::int64_t* index, std::int64_t rows, std::int64_t cols,
                 float* dst) {
  check(uocr_rocm_gather_rows(ctx.stream(), src, index, rows, cols, dst));
}

void scatter_add_rows(const Context& ctx, float* dst, const std::int64_t* index, const float* weight, const float* src,
                      std::int64_t rows, std::int64_t cols) {
  check(uocr_rocm_scatter_add_rows(ctx.stream(), dst, index, weight, src, rows, cols));
}

void im2col(const Context& ctx, const float* x, std::int64_t c, std::int64_t h, std::int64_t w, std::int64_t kh,
            std::int64_t kw, int stride, int pad, float* cols) {
  check(uocr_rocm_im2col(ctx.stream(), x, c, h, w, kh, kw, stride, pad, cols));
}

void im2col(const Context& ctx, const float* x, std::int64_t c, std::int64_t h, std::int64_t w, std::int64_t kh,
            std::int64_t kw, int stride, int pad, std::uint16_t* cols) {
  check(uocr_rocm_im2col_bf16(ctx.stream(), x, c, h, w, kh, kw, stride, pad, cols));
}

void chw_to_hwc(const Context& ctx, const float* x, std::int64_t c, std::int64_t h, std::int64_t w, float* y) {
  check(uocr_rocm_chw_to_hwc(ctx.stream(), x, c, h, w, y));
}

void hwc_to_chw(const Context& ctx, const float* x, std::int64_t h, std::int64_t w, std::int64_t c, float* y) {
  check(uocr_rocm_hwc_to_chw(ctx.stream(), x, h, w, c, y));
}

void concat_cols(const Context& ctx, const float* a, std::int64_t ca, const float* b, std::int64_t cb, std::int64_t rows,
                 float* out) {
  check(uocr_rocm_concat_cols(ctx.stream(), a, ca, b, cb, rows, out));
}

void split_heads(const Context& ctx, const float* x, std::int64_t rows, std::int64_t parts, std::int64_t heads,
                 std::int64_t hd, float* y) {
  check(uocr_rocm_split_heads(ctx.stream(), x, rows, parts, heads, hd, y));
}

void merge_heads(const Context& ctx, const float* x, std::int64_t heads, std::int64_t rows, std::int64_t hd, float* y) {
  check(uocr_rocm_merge_heads(ctx.stream(), x, heads, rows, hd, y));
}

void rel_pos_bias(const Context& ctx, const float* q, std::int64_t ldq, std::int64_t h, std::int64_t w, std::int64_t d,
                  const float* rh, const float* rw, float* bias) {
  check(uocr_rocm_rel_pos_bias(ctx.stream(), q, ldq, h, w, d, rh, rw, bias));
}

void rel_pos_softmax_rows(const Context& ctx, float* scores, std::int64_t windows, const float* q, std::int64_t ldq,
                          std::int64_t h, std::int64_t w, std::int64_t d, const float* rh, const float* rw) {
  check(uocr_rocm_rel_pos_softmax_rows(ctx.stream(), scores, windows, q, ldq, h, w, d, rh, rw));
}

void attention(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, float* out, std::int64_t ldo,
               std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd, float scale,
               const float* mask, std::int64_t mask_ld) {
  check(uocr_rocm_attention(ctx.stream(), q.p, q.ld, q.slice, k.p, k.ld, k.slice, v.p, v.ld, v.slice, out, ldo, so,
                            slices, rows, keys, hd, scale, mask, mask_ld));
}

void attention(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, std::uint16_t* out, std::int64_t ldo,
               std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd, float scale,
               const float* mask, std::int64_t mask_ld) {
  check(uocr_rocm_attention_bf16(ctx.stream(), q.p, q.ld, q.slice, k.p, k.ld, k.slice, v.p, v.ld, v.slice, out, ldo,
                                 so, slices, rows, keys, hd, scale, mask, mask_ld));
}

void attention_rel_pos_windows(const Context& ctx, AttnOperand q, std::int64_t wq, AttnOperand k, std::int64_t wk,
                               AttnOperand v, std::int64_t wv, std::uint16_t* out, std::int64_t ldo, std::int64_t so,
                               std::int64_t wo, std::int64_t heads, std::int64_t windows, std::int64_t h,
                               std::int64_t w, std::int64_t hd, float scale, const float* rh, const float* rw,
                               float* workspace, std::int64_t workspace_floats) {
  check(uocr_rocm_attention_rel_pos_windows_bf16_ws(ctx.stream(), q.p, q.ld, q.slice, wq, k.p, k.ld, k.slice, wk, v.p,
                                                    v.ld, v.slice, wv, out, ldo, so, wo, heads, windows, h, w, hd,
                                                    scale, rh, rw, workspace, workspace_floats));
}

std::int64_t attention_workspace_floats(std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd) {
  return uocr_rocm_attention_workspace_floats(slices, rows, keys, hd);
}

void attention(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, std::uint16_t* out, std::int64_t ldo,
               std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd, float scale,
               const float* mask, std::int64_t mask_ld, float* workspace, std::int64_t workspace_floats) {
  check(uocr_rocm_attention_bf16_ws(ctx.stream(), q.p, q.ld, q.slice, k.p, k.ld, k.slice, v.p, v.ld, v.slice, out, ldo,
                                    so, slices, rows, keys, hd, scale, mask, mask_ld, workspace, workspace_floats));
}

std::int64_t attention_masked_workspace_floats(std::int64_t slices, std::int64_t rows, std::int64_t keys,
                                               std::int64_t hd) {
  return uocr_rocm_attention_masked_workspace_floats(slices, rows, keys, hd);
}

void attention_masked(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, std::uint16_t* out,
                      std::int64_t ldo, std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys,
                      std::int64_t hd, float scale, const float* mask, std::int64_t mask_ld, float* workspace,
                      std::int64_t workspace_floats) {
  check(uocr_rocm_attention_masked_bf16_ws(ctx.stream(), q.p, q.ld, q.slice, k.p, k.ld, k.slice, v.p, v.ld, v.slice,
                                           out, ldo, so, slices, rows, keys, hd, scale, mask, mask_ld, workspace,
                                           workspace_floats));
}

std::int64_t attention_rel_pos_workspace_floats(std::int64_t slices, std::int64_t h, std::int64_t w) {
  return uocr_rocm_attention_rel_pos_workspace_floats(slices, h, w);
}

void attention_rel_pos_windows(const Context& ctx, AttnOperand q, std::int64_t wq, AttnOperand k, std::int64_t wk,
                               AttnOperand v, std::int64_t wv, float* out, std::int64_t ldo, std::int64_t so,
                               std::int64_t wo, std::int64_t heads, std::int64_t windows, std::int64_t h,
                               std::int64_t w, std::int64_t hd, float scale, const float* rh, const float* rw,
                               float* workspace, std::int64_t workspace_floats) {
  check(uocr_rocm_attention_rel_pos_windows_ws(ctx.stream(), q.p, q.ld, q.slice, wq, k.p, k.ld, k.slice, wk, v.p, v.ld,
                                               v.slice, wv, out, ldo, so, wo, heads, windows, h, w, hd, scale, rh, rw,
                                               workspace, workspace_floats));
}

void linear(const Context& ctx, const float* x, std::int64_t m, std::int64_t k, const std::uint16_t* w_bf16,
            std::int64_t n, const float* bias, float* y) {
  check(uocr_rocm_linear(ctx.stream(), x, m, k, w_bf16, n, bias, y));
}

std::int64_t linear_workspace_floats(std::int64_t m, std::int64_t k, std::int64_t n) {
  return uocr_rocm_linear_workspace_floats(m, k, n);
}

void linear(const Context& ctx, const float* x, std::int64_t m, std::int64_t k, const std::uint16_t* w_bf16,
            std::int64_t n, const float* bias, float* y, float* workspace, std::int64_t workspace_floats) {
  check(uocr_rocm_linear_ws(ctx.stream(), x, m, k, w_bf16, n, bias, y, workspace, workspace_floats));
}

void linear_bf16x(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k, const std::uint16_t* w_bf16,
                  std::int64_t n, const float* bias, float* y) {
  check(uocr_rocm_linear_bf16x(ctx.stream(), x, m, k, w_bf16, n, bias, y));
}

void linear_bf16x(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                  const std::uint16_t* w_bf16, std::int64_t n, const float* bias, float* y, float* workspace,
                  std::int64_t workspace_floats) {
  check(uocr_rocm_linear_bf16x_ws(ctx.stream(), x, m, k, w_bf16, n, bias, y, workspace, workspace_floats));
}

void linear_bf16x_add(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                      const std::uint16_t* w_bf16, std::int64_t n, const float* bias, float* y, float* workspace,
                      std::int64_t workspace_floats) {
  check(uocr_rocm_linear_bf16x_add_ws(ctx.stream(), x, m, k, w_bf16, n, bias, y, workspace, workspace_floats));
}

void linear_bf16x_add_rows(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                           const std::uint16_t* w_bf16, std::int64_t n, const float* bias, float* y,
                           const std::int64_t* y_row, std::int64_t y_rows) {
  check(uocr_rocm_linear_bf16x_add_rows(ctx.stream(), x, m, k, w_bf16, n, bias, y, y_row, y_rows));
}

void linear_bf16x_act_bf16(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                           const std::uint16_t* w_bf16, std::int64_t n, const float* bias, std::uint16_t* y,
                           bool quick) {
  check(quick ? uocr_rocm_linear_bf16x_quick_gelu_bf16(ctx.stream(), x, m, k, w_bf16, n, bias, y)
              : uocr_rocm_linear_bf16x_gelu_erf_bf16(ctx.stream(), x, m, k, w_bf16, n, bias, y));
}

void round_bf16(const Context& ctx, const float* src, std::int64_t n, std::uint16_t* dst) {
  check(uocr_rocm_round_bf16(ctx.stream(), src, n, dst));
}

void layer_norm_to_bf16(const Context& ctx, const float* x, const float* w, const float* b, std::uint16_t* y,
                        std::int64_t rows, std::int64_t cols, float eps) {
  check(uocr_rocm_layer_norm_to_bf16(ctx.stream(), x, w, b, y, rows, cols, eps));
}

void gelu_erf_to_bf16(const Context& ctx, const float* x, std::uint16_t* y, std::int64_t n) {
  check(uocr_rocm_gelu_erf_to_bf16(ctx.stream(), x, y, n));
}

void quick_gelu_to_bf16(const Context& ctx, const float* x, std::uint16_t* y, std::int64_t n) {
  check(uocr_rocm_quick_gelu_to_bf16(ctx.stream(), x, y, n));
}

void add_rms_norm_gemv_bf16(const Context& ctx, const float* x, const float* delta, float* x_out, const float* w_norm,
                            float eps, float* h_out, std::int64_t k, const std::uint16_t* w, std::int64_t n,
                            const float* bias, float* y) {
  check(uocr_rocm_add_rms_norm_gemv_bf16(ctx.stream(), x, delta, x_out, w_norm, eps, h_out, k, w, n, bias, y));
}

void add_rms_norm_swiglu_gemv_bf16(const Context& ctx, const float* x, const float* delta, float* x_out,
                                   const float* w_norm, float eps, float* h_out, std::int64_t k,
                                   const std::uint16_t* w_gate, const std::uint16_t* w_up, std::int64_t ffn,
                                   float* act) {
  check(uocr_rocm_add_rms_norm_swiglu_gemv_bf16(ctx.stream(), x, delta, x_out, w_norm, eps, h_out, k, w_gate, w_up,
                                                ffn, act));
}

void add_rms_norm_swiglu_router_gemv_bf16(const Context& ctx, const float* x, const float* delta, float* x_out,
                                          const float* w_norm, float eps, float* h_out, std::int64_t k,
                                          const std::uint16_t* w_gate, const std::uint16_t* w_up, std::int64_t ffn,
                                          float* act, const float* router, std::int64_t experts, float* logits) {
  check(uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16(ctx.stream(), x, delta, x_out, w_norm, eps, h_out, k, w_gate,
                                                       w_up, ffn, act, router, experts, logits));
}

void scale_mask_softmax_rows(const Context& ctx, float* x, float scale, const float* mask, std::int64_t batch,
                             std::int64_t rows, std::int64_t cols) {
  check(uocr_rocm_scale_mask_softmax_rows(ctx.stream(), x, scale, mask, batch, rows, cols));
}

void expert_topk(const Context& ctx, const float* logits, std::int64_t rows, std::int64_t experts, std::int64_t k,
                 std::int64_t* ids, float* weights) {
  check(uocr_rocm_expert_topk(ctx.stream(), logits, rows, experts, k, ids, weights));
}

std::int64_t expert_scratch_floats(std::int64_t k, std::int64_t ffn) { return uocr_rocm_expert_scratch_floats(k, ffn); }

void expert_ffn_one(const Context& ctx, const float* x, std::int64_t hidden, std::int64_t ffn,
                    const std::uint16_t* gate, const std::uint16_t* up, const std::uint16_t* down,
                    std::int64_t experts, const std::int64_t* ids, const float* weights, std::int64_t k,
                    const float* base, float* scratch, float* out) {
  check(uocr_rocm_expert_ffn_one(ctx.stream(), x, hidden, ffn, gate, up, down, experts, ids, weights, k, base,
                                 scratch, out));
}

void moe_ffn_one(const Context& ctx, const float* x, std::int64_t hidden, std::int64_t ffn,
                 const std::uint16_t* gate, const std::uint16_t* up, const std::uint16_t* down, std::int64_t experts,
                 const float* logits, std::int64_t k, std::int64_t* ids, float* weights, const float* shared_act,
                 const std::uint16_t* shared_down, std::int64_t shared_ffn, float* scratch, float* out) {
  check(uocr_rocm_moe_ffn_one(ctx.stream(), x, hidden, ffn, gate, up, down, experts, logits, k, ids, weights,
                              shared_act, shared_down, shared_ffn, scratch, out));
}

}  // namespace uocr::rocm
