#pragma once

// The rocm backend's fused layer ops, over raw device pointers so callers
// can address slices. Every op is enqueued on the context's stream; none
// synchronises and none allocates, so every op can be captured in a graph.
// Shapes are row-major, as in the reference backend.
//
// The fp32 entry points keep the names and argument order of the reference's
// uocr::cuda ops (src/backend/cuda/ops.h:30-75), so a model/rocm decoder can
// mirror model/cuda line for line. The fused ops and the bf16-activation
// variants are new; each bf16 op computes in fp32 on the widened inputs and
// rounds once on store (nearest even), so it reduces to its fp32 op.
// Norm weights and biases are fp32 throughout.
//
// Bad shapes throw std::invalid_argument before anything is enqueued;
// runtime and launch failures throw std::runtime_error("<what>: <detail>").

#include <cstdint>

#include "backend/rocm/context.h"

namespace uocr::rocm {

// ---- reference signatures (fp32 activations, bf16 tables) ------------------

void add_inplace(const Context& ctx, float* y, const float* x, std::int64_t n);  // y += x
void layer_norm(const Context& ctx, float* x, const float* w, const float* b, std::int64_t rows, std::int64_t cols,
                float eps);
void rms_norm(const Context& ctx, float* x, const float* w, std::int64_t rows, std::int64_t cols, float eps);
void gelu_erf(const Context& ctx, float* x, std::int64_t n);
void silu_mul(const Context& ctx, float* g, const float* u, std::int64_t n);  // g = silu(g) * u

// Rotary embedding of x [rows, heads * dim] in place: pairs below n_tok
// turn by the row's token coordinate, the rest by its page coordinate
// (mod page_mod). Coordinates come per row from tok / page, or, when those
// are null, from one_tok / one_page for every row.
void rope(const Context& ctx, float* x, std::int64_t rows, std::int64_t heads, std::int64_t dim, const std::int64_t* tok,
          const std::int64_t* page, const float* inv_tok, std::int64_t n_tok, const float* inv_page, std::int64_t n_page,
          std::int64_t page_mod, std::int64_t one_tok = 0, std::int64_t one_page = 0);

// Copies n floats from src to dst, both on the device; the two ranges must
// not overlap.
void copy(const Context& ctx, float* dst, const float* src, std::int64_t n);

// Token embeddings: rows of a bf16 table widened into fp32 rows (exact);
// one_index picks a single row without a device index array. The table's row count is unknown here, so the
// indices are trusted as in the reference; the overloads taking table_rows
// turn an out-of-range device index into a zero row instead.
void gather_rows_bf16(const Context& ctx, const std::uint16_t* table, const std::int64_t* index, std::int64_t rows,
                      std::int64_t cols, float* dst);
void gather_row_bf16(const Context& ctx, const std::uint16_t* table, std::int64_t one_index, std::int64_t cols,
                     float* dst);
void gather_rows_bf16(const Context& ctx, const std::uint16_t* table, std::int64_t table_rows, const std::int64_t* index,
                      std::int64_t rows, std::int64_t cols, float* dst);

// ---- fused ops ----------------------------------------------------------------

// Residual add fused with RMSNorm, per row: s = x + delta; x = s;
// h = w * (s * inv(s)). Replaces add_inplace + copy + rms_norm.
void add_rms_norm(const Context& ctx, float* x, const float* delta, const float* w, float* h, std::int64_t rows,
                  std::int64_t cols, float eps);
// SwiGLU over in [rows, 2 * ffn] laid out [gate | up] per row: out [rows, ffn].
void swiglu(const Context& ctx, const float* in, float* out, std::int64_t rows, std::int64_t ffn);
// rope on Q [rows, q_heads * dim] and K [rows, k_heads * dim] in one launch.
void rope_qk(const Context& ctx, float* q, std::int64_t q_heads, float* k, std::int64_t k_heads, std::int64_t rows,
             std::int64_t dim, const std::int64_t* tok, const std::int64_t* page, const float* inv_tok,
             std::int64_t n_tok, const float* inv_page, std::int64_t n_page, std::int64_t page_mod,
             std::int64_t one_tok = 0, std::int64_t one_page = 0);

// ---- bf16 activations ------------------------------------------------------------

void add_rms_norm_bf16(const Context& ctx, std::uint16_t* x, const std::uint16_t* delta, const float* w,
                       std::uint16_t* h, std::int64_t rows, std::int64_t cols, float eps);
void layer_norm_bf16(const Context& ctx, std::uint16_t* x, const float* w, const float* b, std::int64_t rows,
                     std::int64_t cols, float eps);
void gelu_erf_bf16(const Context& ctx, std::uint16_t* x, std::int64_t n);
void swiglu_bf16(const Context& ctx, const std::uint16_t* in, std::uint16_t* out, std::int64_t rows,
                 std::int64_t ffn);
void rope_qk_bf16(const Context& ctx, std::uint16_t* q, std::int64_t q_heads, std::uint16_t* k, std::int64_t k_heads,
                  std::int64_t rows, std::int64_t dim, const std::int64_t* tok, const std::int64_t* page,
                  const float* inv_tok, std::int64_t n_tok, const float* inv_page, std::int64_t n_page,
                  std::int64_t page_mod, std::int64_t one_tok = 0, std::int64_t one_page = 0);

// ---- row ops beside the path (reference signatures, src/backend/cuda/ops.h:35-46) -------

// The router's norm: non-finite inputs zeroed, scaled by (1 + w), clamped to +-1e4.
void router_norm(const Context& ctx, float* x, const float* w, std::int64_t rows, std::int64_t cols, float eps);
void quick_gelu(const Context& ctx, float* x, std::int64_t n);
// Each row of x [rows, cols] becomes its softmax, in place. A row whose
// entries are all -inf becomes all zeros.
void softmax_rows(const Context& ctx, float* x, std::int64_t rows, std::int64_t cols);
// For every slice b of `batch` [rows, cols] slices of x:
// x[b] = x[b] * scale + mask, the one mask [rows, cols] shared by the slices.
void scale_add_mask(const Context& ctx, float* x, float scale, const float* mask, std::int64_t batch, std::int64_t rows,
                    std::int64_t cols);

// New: scale_add_mask then softmax_rows in one pass over x (bitwise the same).
void scale_mask_softmax_rows(const Context& ctx, float* x, float scale, const float* mask, std::int64_t batch,
                             std::int64_t rows, std::int64_t cols);

// ---- weight streaming (src/backend/cuda/gemv_ops.h:25-26) ---------------------------------

// y[n] = bf16(x) . w[n, :] (+ bias[n]); x fp32 [k] (k <= 12288), w bf16 [n, k].
void gemv_bf16(const Context& ctx, const float* x, std::int64_t k, const std::uint16_t* w, std::int64_t n,
               const float* bias, float* y);
// fp32 products batched over `batch` slices stride_* elements apart:
// c = alpha a[m, k] b[n, k]^T (gemm_nt), c = a[m, k] b[k, n] (gemm_nn).
void gemm_nt(const Context& ctx, std::int64_t m, std::int64_t n, std::int64_t k, float alpha, const float* a,
             std::int64_t lda, std::int64_t stride_a, const float* b, std::int64_t ldb, std::int64_t stride_b, float* c,
             std::int64_t ldc, std::int64_t stride_c, std::int64_t batch);
void gemm_nn(const Context& ctx, std::int64_t m, std::int64_t n, std::int64_t k, const float* a, std::int64_t lda,
             std::int64_t stride_a, const float* b, std::int64_t ldb, std::int64_t stride_b, float* c, std::int64_t ldc,
             std::int64_t stride_c, std::int64_t batch);
// Rows by index: dst[i] = src[index[i]]; dst[index[i]] += weight[i] * src[i], i in order.
void gather_rows(const Context& ctx, const float* src, const std::int64_t* index, std::int64_t rows, std::int64_t cols,
                 float* dst);
void scatter_add_rows(const Context& ctx, float* dst, const std::int64_t* index, const float* weight, const float* src,
                      std::int64_t rows, std::int64_t cols);
// The vision encoder's layout ops: [c, h, w] patches in weight order
// (oh = (h + 2 pad - kh) / stride + 1), the two layout transposes, and rows
// joined side by side.
// New: im2col into bf16 patches (the rounding the convolution's product
// applies), bitwise im2col then round_bf16.
void im2col(const Context& ctx, const float* x, std::int64_t c, std::int64_t h, std::int64_t w, std::int64_t kh,
            std::int64_t kw, int stride, int pad, std::uint16_t* cols);
void im2col(const Context& ctx, const float* x, std::int64_t c, std::int64_t h, std::int64_t w, std::int64_t kh,
            std::int64_t kw, int stride, int pad, float* cols);
void chw_to_hwc(const Context& ctx, const float* x, std::int64_t c, std::int64_t h, std::int64_t w, float* y);
void hwc_to_chw(const Context& ctx, const float* x, std::int64_t h, std::int64_t w, std::int64_t c, float* y);
void concat_cols(const Context& ctx, const float* a, std::int64_t ca, const float* b, std::int64_t cb, std::int64_t rows,
                 float* out);
// New: attention operands to a head-major layout, y [parts, heads, rows, hd]
// from x [rows, parts * heads * hd], and the heads' outputs back to rows.
void split_heads(const Context& ctx, const float* x, std::int64_t rows, std::int64_t parts, std::int64_t heads,
                 std::int64_t hd, float* y);
void merge_heads(const Context& ctx, const float* x, std::int64_t heads, std::int64_t rows, std::int64_t hd, float* y);
// SAM's relative-position bias of one window and head, bias[t, ky w + kx] =
// q_t . rh[qy, ky] + q_t . rw[qx, kx]; and (new) the scores of every window
// of one head replaced by softmax(scores + that bias) in one pass.
void rel_pos_bias(const Context& ctx, const float* q, std::int64_t ldq, std::int64_t h, std::int64_t w, std::int64_t d,
                  const float* rh, const float* rw, float* bias);
void rel_pos_softmax_rows(const Context& ctx, float* scores, std::int64_t windows, const float* q, std::int64_t ldq,
                          std::int64_t h, std::int64_t w, std::int64_t d, const float* rh, const float* rw);
// New: attention in one pass on the matrix cores, fp32: out[s, t] =
// softmax(scale q[s, t] . k[s, :] + mask[t, :]) v[s, :] over `slices` slices
// (row t of slice s at base + s * s_stride + t * ld); mask may be null; and
// the same with SAM's relative-position bias over h x w windows.
struct AttnOperand {
  const float* p;
  std::int64_t ld, slice;
};
void attention(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, float* out, std::int64_t ldo,
               std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd, float scale,
               const float* mask, std::int64_t mask_ld);
// New: the same with the bias's dot products formed beforehand into a
// workspace of attention_rel_pos_workspace_floats(slices, h, w) floats.
std::int64_t attention_rel_pos_workspace_floats(std::int64_t slices, std::int64_t h, std::int64_t w);
// New: over heads x windows slices, operand slice (head, window) at
// p + head * slice + window * window_stride.
void attention_rel_pos_windows(const Context& ctx, AttnOperand q, std::int64_t wq, AttnOperand k, std::int64_t wk,
                               AttnOperand v, std::int64_t wv, float* out, std::int64_t ldo, std::int64_t so,
                               std::int64_t wo, std::int64_t heads, std::int64_t windows, std::int64_t h,
                               std::int64_t w, std::int64_t hd, float scale, const float* rh, const float* rw,
                               float* workspace, std::int64_t workspace_floats);
// New: attention and attention_rel_pos_windows with the output in bf16 (the
// rounding the output projection applies), bitwise the fp32 op then
// round_bf16.
void attention(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, std::uint16_t* out, std::int64_t ldo,
               std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd, float scale,
               const float* mask, std::int64_t mask_ld);
// New: attention with a mask and a workspace of
// attention_workspace_floats(slices, rows, keys, hd) floats: the mask's live
// tiles walked alone, long walks cut into runs merged by a last launch;
// fp32 products, the bf16 output bitwise the fp32 one rounded.
std::int64_t attention_workspace_floats(std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd);
void attention(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, std::uint16_t* out, std::int64_t ldo,
               std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys, std::int64_t hd, float scale,
               const float* mask, std::int64_t mask_ld, float* workspace, std::int64_t workspace_floats);
// New: attention with a mask into bf16 on the bf16 matrix cores with split
// operands, walking only the key tiles the mask leaves live; the workspace
// holds attention_masked_workspace_floats(slices, rows, keys, hd) floats.
std::int64_t attention_masked_workspace_floats(std::int64_t slices, std::int64_t rows, std::int64_t keys,
                                               std::int64_t hd);
void attention_masked(const Context& ctx, AttnOperand q, AttnOperand k, AttnOperand v, std::uint16_t* out,
                      std::int64_t ldo, std::int64_t so, std::int64_t slices, std::int64_t rows, std::int64_t keys,
                      std::int64_t hd, float scale, const float* mask, std::int64_t mask_ld, float* workspace,
                      std::int64_t workspace_floats);
void attention_rel_pos_windows(const Context& ctx, AttnOperand q, std::int64_t wq, AttnOperand k, std::int64_t wk,
                               AttnOperand v, std::int64_t wv, std::uint16_t* out, std::int64_t ldo, std::int64_t so,
                               std::int64_t wo, std::int64_t heads, std::int64_t windows, std::int64_t h,
                               std::int64_t w, std::int64_t hd, float scale, const float* rh, const float* rw,
                               float* workspace, std::int64_t workspace_floats);
// y[m, n] = bf16(x)[m, k] . w[n, k]^T (+ bias[n]) on the matrix cores, fp32
// accumulation (m == 1: the GEMV); the reference's linear.
void linear(const Context& ctx, const float* x, std::int64_t m, std::int64_t k, const std::uint16_t* w_bf16,
            std::int64_t n, const float* bias, float* y);
// New: linear with x already rounded to bf16; round_bf16 does the rounding.
void linear_bf16x(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k, const std::uint16_t* w_bf16,
                  std::int64_t n, const float* bias, float* y);
void round_bf16(const Context& ctx, const float* src, std::int64_t n, std::uint16_t* dst);
// New: y = bf16(gelu_erf(x)) / bf16(quick_gelu(x)), x fp32 and y bf16.
// New: y = bf16(layer_norm(x)) out of place (x fp32 untouched, y bf16).
void layer_norm_to_bf16(const Context& ctx, const float* x, const float* w, const float* b, std::uint16_t* y,
                        std::int64_t rows, std::int64_t cols, float eps);
void gelu_erf_to_bf16(const Context& ctx, const float* x, std::uint16_t* y, std::int64_t n);
void quick_gelu_to_bf16(const Context& ctx, const float* x, std::uint16_t* y, std::int64_t n);
// New: y = bf16(act(bf16(x) w^T + bias)), an MLP's first projection with its
// activation (quick: quick_gelu, else gelu_erf) in the epilogue, bitwise
// linear_bf16x then gelu_erf_to_bf16 / quick_gelu_to_bf16; k % 64 == 0.
void linear_bf16x_act_bf16(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                           const std::uint16_t* w_bf16, std::int64_t n, const float* bias, std::uint16_t* y,
                           bool quick);
// New: linear with a workspace for splitting k where the product has too
// few tiles to cover the GPU (linear_workspace_floats(m, k, n) floats; 0:
// no split is taken).
std::int64_t linear_workspace_floats(std::int64_t m, std::int64_t k, std::int64_t n);
void linear(const Context& ctx, const float* x, std::int64_t m, std::int64_t k, const std::uint16_t* w_bf16,
            std::int64_t n, const float* bias, float* y, float* workspace, std::int64_t workspace_floats);
// New: the same with x already rounded to bf16.
void linear_bf16x(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                  const std::uint16_t* w_bf16, std::int64_t n, const float* bias, float* y, float* workspace,
                  std::int64_t workspace_floats);
// New: y[y_row[r]] += (bf16(x) w^T + bias)[r] for y_row[r] < y_rows.
void linear_bf16x_add_rows(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                           const std::uint16_t* w_bf16, std::int64_t n, const float* bias, float* y,
                           const std::int64_t* y_row, std::int64_t y_rows);
// New: y += bf16(x) w^T (+ bias), as linear_bf16x then add_inplace.
void linear_bf16x_add(const Context& ctx, const std::uint16_t* x, std::int64_t m, std::int64_t k,
                      const std::uint16_t* w_bf16, std::int64_t n, const float* bias, float* y, float* workspace,
                      std::int64_t workspace_floats);

// Fused decode projections (new): add + RMSNorm as the GEMV's prologue,
// optionally a gate/up pair with a SwiGLU epilogue. delta, x_out, w_norm
// and h_out may be null; k is a multiple of 8 in [8, 2048].
void add_rms_norm_gemv_bf16(const Context& ctx, const float* x, const float* delta, float* x_out, const float* w_norm,
                            float eps, float* h_out, std::int64_t k, const std::uint16_t* w, std::int64_t n,
                            const float* bias, float* y);
void add_rms_norm_swiglu_gemv_bf16(const Context& ctx, const float* x, const float* delta, float* x_out,
                                   const float* w_norm, float eps, float* h_out, std::int64_t k,
                                   const std::uint16_t* w_gate, const std::uint16_t* w_up, std::int64_t ffn,
                                   float* act);
// New: the SwiGLU pair above and the fp32 router logits [experts] on the
// unrounded h in one launch, bitwise it followed by uocr_rocm_gemv_f32(h, router).
void add_rms_norm_swiglu_router_gemv_bf16(const Context& ctx, const float* x, const float* delta, float* x_out,
                                          const float* w_norm, float eps, float* h_out, std::int64_t k,
                                          const std::uint16_t* w_gate, const std::uint16_t* w_up, std::int64_t ffn,
                                          float* act, const float* router, std::int64_t experts, float* logits);

// ---- mixture of experts at decode (src/backend/cuda/ops.h:77-90) ------------------

// For each row of router logits [rows, experts]: its softmax, then the k
// largest probabilities (the lower expert index first where two are equal)
// written as ids and weights.
void expert_topk(const Context& ctx, const float* logits, std::int64_t rows, std::int64_t experts, std::int64_t k,
                 std::int64_t* ids, float* weights);
// Floats of scratch that expert_ffn_one needs.
std::int64_t expert_scratch_floats(std::int64_t k, std::int64_t ffn);
// One decode row x through its k routed experts, each expert e a slice of
// the stacked gate, up and down weights: out = the weights[j]-weighted sum
// over j of down_e . (silu(gate_e . x) * (up_e . x)), e = ids[j], with x and
// the activation rounded to bf16 for the products. The
// reference's signature plus `experts` and `scratch`, so nothing is
// allocated and a captured step can hold the call.
// With base set, out = base + the routed sum (base may be out itself).
void expert_ffn_one(const Context& ctx, const float* x, std::int64_t hidden, std::int64_t ffn,
                    const std::uint16_t* gate, const std::uint16_t* up, const std::uint16_t* down,
                    std::int64_t experts, const std::int64_t* ids, const float* weights, std::int64_t k,
                    const float* base, float* scratch, float* out);
// New: the routed experts from the router's logits (the top k formed in
// the launch and written to ids/weights) with the shared experts' down
// product in the same launch: out = shared_down . bf16(shared_act) + routed,
// bitwise expert_topk, the shared GEMV and expert_ffn_one with it as base.
void moe_ffn_one(const Context& ctx, const float* x, std::int64_t hidden, std::int64_t ffn,
                 const std::uint16_t* gate, const std::uint16_t* up, const std::uint16_t* down, std::int64_t experts,
                 const float* logits, std::int64_t k, std::int64_t* ids, float* weights, const float* shared_act,
                 const std::uint16_t* shared_down, std::int64_t shared_ffn, float* scratch, float* out);

// ---- the block router (src/backend/cuda/ops.h:97-124) -----------------------------------

// The block router's parameters; the defaults are the reference decoder's
// (src/model/block_router.h:16-26, src/model/decoder.cpp:58-62).
struct RouteParams {
  std::int64_t block_size = 32;
  std::int64_t local_blocks = 4;
  std::int64_t top_m = 16;
  std::int64_t top_k = 12;
  float idx_scale = 11.3137083f;  // 128 / sqrt(128) in fp32
  float floor = 1e-4f;
  float sigma = 1.0f;
};

// Per block of block_size router keys [s, d]: the head_cls-weighted softmax
// mean of its keys, out [ceil(s / block_size), d].
void block_summaries(const Context& ctx, const float* keys, std::int64_t s, std::int64_t d, const float* head_cls,
                     std::int64_t block_size, float* out);
// The key masks [rows, keys] of prompt rows from block scores z [rows, nblk].
void route_blocks(const Context& ctx, const float* z, std::int64_t rows, std::int64_t nblk, std::int64_t first_pos,
                  std::int64_t keys, const std::int64_t* block_min, const std::int64_t* block_max,
                  std::int64_t prompt_blocks, const std::int64_t* query_page, std::int64_t one_page,
                  const RouteParams& params, float* mask);

}  // namespace uocr::rocm
