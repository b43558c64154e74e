#include "backend/rocm/decode_ops.h"

#include <cstddef>

#include "uocr_rocm.h"

namespace uocr::rocm {
namespace {

// The C ABI reads the same five int64 fields in the same order.
static_assert(sizeof(StepState) == sizeof(uocr_rocm_step_state));
static_assert(offsetof(StepState, token) == offsetof(uocr_rocm_step_state, token));
static_assert(offsetof(StepState, pos) == offsetof(uocr_rocm_step_state, pos));
static_assert(offsetof(StepState, tok) == offsetof(uocr_rocm_step_state, tok));
static_assert(offsetof(StepState, page) == offsetof(uocr_rocm_step_state, page));
static_assert(offsetof(StepState, query_page) == offsetof(uocr_rocm_step_state, query_page));

const uocr_rocm_step_state* abi(const StepState* s) { return reinterpret_cast<const uocr_rocm_step_state*>(s); }

}  // namespace

void embed_step(const Context& ctx, const std::uint16_t* table, const StepState* state, std::int64_t cols, float* dst) {
  check(uocr_rocm_embed_step(ctx.stream(), table, -1, abi(state), cols, dst));
}

void rope_step(const Context& ctx, float* x, std::int64_t heads, std::int64_t dim, const StepState* state,
               const float* inv_tok, std::int64_t n_tok, const float* inv_page, std::int64_t page_mod) {
  check(uocr_rocm_rope_step(ctx.stream(), x, heads, dim, abi(state), inv_tok, n_tok, inv_page, page_mod));
}

void rope_qk_step(const Context& ctx, float* q, std::int64_t q_heads, float* k, std::int64_t k_heads, std::int64_t dim,
                  const StepState* state, const float* inv_tok, std::int64_t n_tok, const float* inv_page,
                  std::int64_t page_mod) {
  check(uocr_rocm_rope_qk_step(ctx.stream(), q, q_heads, k, k_heads, dim, abi(state), inv_tok, n_tok, inv_page,
                               page_mod));
}

void rope_qk_step_bf16(const Context& ctx, std::uint16_t* q, std::int64_t q_heads, std::uint16_t* k,
                       std::int64_t k_heads, std::int64_t dim, const StepState* state, const float* inv_tok,
                       std::int64_t n_tok, const float* inv_page, std::int64_t page_mod) {
  check(uocr_rocm_rope_qk_step_bf16(ctx.stream(), q, q_heads, k, k_heads, dim, abi(state), inv_tok, n_tok, inv_page,
                                    page_mod));
}

void embed_step_bf16(const Context& ctx, const std::uint16_t* table, std::int64_t table_rows, const StepState* state,
                     std::int64_t cols, std::uint16_t* dst) {
  check(uocr_rocm_embed_step_bf16(ctx.stream(), table, table_rows, abi(state), cols, dst));
}

void append_step(const Context& ctx, float* cache, const float* row, std::int64_t width, const StepState* state,
                 std::int64_t capacity) {
  check(uocr_rocm_append_step(ctx.stream(), cache, row, width, abi(state), capacity));
}

std::int64_t attend_scratch_floats(std::int64_t heads, std::int64_t hd, std::int64_t capacity) {
  return uocr_rocm_attend_scratch_floats(heads, hd, capacity);
}

void attend_step(const Context& ctx, const float* q, const float* k_cache, const float* v_cache, std::int64_t heads,
                 std::int64_t hd, const float* mask, float scale, const StepState* state, float* scratch,
                 std::int64_t capacity, float* out) {
  check(uocr_rocm_attend_step(ctx.stream(), q, k_cache, v_cache, heads, hd, mask, scale, abi(state), scratch, capacity,
                              out));
}

void attend_rope_kv_step(const Context& ctx, const float* q, const float* k_row, const float* v_row, float* k_cache,
                         float* v_cache, std::int64_t heads, std::int64_t hd, const float* mask, float scale,
                         const StepState* state, const float* inv_tok, std::int64_t n_tok, const float* inv_page,
                         std::int64_t page_mod, float* scratch, std::int64_t capacity, float* out) {
  check(uocr_rocm_attend_rope_kv_step(ctx.stream(), q, k_row, v_row, k_cache, v_cache, heads, hd, mask, scale,
                                      abi(state), inv_tok, n_tok, inv_page, page_mod, scratch, capacity, out));
}

void embed_add_rms_norm_step(const Context& ctx, const std::uint16_t* table, std::int64_t table_rows,
                             const StepState* state, const float* delta, const float* w, float* x, float* h,
                             std::int64_t cols, float eps) {
  check(uocr_rocm_embed_add_rms_norm_step(ctx.stream(), table, table_rows, abi(state), delta, w, x, h, cols, eps));
}

void attend_rope_kv_step_bf16(const Context& ctx, const float* q, const float* k_row, const float* v_row,
                              std::uint16_t* k_cache, std::uint16_t* v_cache, std::int64_t heads, std::int64_t hd,
                              const float* mask, float scale, const StepState* state, const float* inv_tok,
                              std::int64_t n_tok, const float* inv_page, std::int64_t page_mod, float* scratch,
                              std::int64_t capacity, float* out) {
  check(uocr_rocm_attend_rope_kv_step_bf16(ctx.stream(), q, k_row, v_row, k_cache, v_cache, heads, hd, mask, scale,
                                           abi(state), inv_tok, n_tok, inv_page, page_mod, scratch, capacity, out));
}

namespace {

uocr_rocm_route_params abi(const RouteParams& p) {
  return uocr_rocm_route_params{p.block_size, p.local_blocks, p.top_m, p.top_k, p.idx_scale, p.floor, p.sigma};
}

}  // namespace

void block_summaries(const Context& ctx, const float* keys, std::int64_t s, std::int64_t d, const float* head_cls,
                     std::int64_t block_size, float* out) {
  check(uocr_rocm_block_summaries(ctx.stream(), keys, s, d, head_cls, block_size, out));
}

void route_blocks(const Context& ctx, const float* z, std::int64_t rows, std::int64_t nblk, std::int64_t first_pos,
                  std::int64_t keys, const std::int64_t* block_min, const std::int64_t* block_max,
                  std::int64_t prompt_blocks, const std::int64_t* query_page, std::int64_t one_page,
                  const RouteParams& params, float* mask) {
  const auto p = abi(params);
  check(uocr_rocm_route_blocks(ctx.stream(), z, rows, nblk, first_pos, keys, block_min, block_max, prompt_blocks,
                               query_page, one_page, &p, mask));
}

void summary_step(const Context& ctx, const float* router_keys, std::int64_t d, const float* head_cls,
                  std::int64_t block_size, const StepState* state, std::int64_t max_blocks, float* summaries) {
  check(uocr_rocm_summary_step(ctx.stream(), router_keys, d, head_cls, block_size, abi(state), max_blocks,
                               summaries));
}

void scores_step(const Context& ctx, const float* rq, const float* summaries, std::int64_t d, std::int64_t block_size,
                 const StepState* state, std::int64_t max_blocks, float* z) {
  check(uocr_rocm_scores_step(ctx.stream(), rq, summaries, d, block_size, abi(state), max_blocks, z));
}

void route_step(const Context& ctx, const float* z, std::int64_t max_blocks, const std::int64_t* block_min,
                const std::int64_t* block_max, std::int64_t prompt_blocks, const StepState* state,
                const RouteParams& params, float* mask) {
  const auto p = abi(params);
  check(uocr_rocm_route_step(ctx.stream(), z, max_blocks, block_min, block_max, prompt_blocks, abi(state), &p, mask));
}

void route_decode_step(const Context& ctx, const float* rq, const float* rk, const float* q_norm, const float* k_norm,
                       float eps, const float* inv_tok, std::int64_t n_tok, const float* inv_page,
                       std::int64_t page_mod, const float* head_cls, float* router_keys, float* summaries,
                       std::int64_t d, const std::int64_t* block_min, const std::int64_t* block_max,
                       std::int64_t prompt_blocks, const StepState* state, const RouteParams& params,
                       std::int64_t capacity, float* mask, float* z_out, float* rqk_out, std::int32_t* segments) {
  const auto p = abi(params);
  check(uocr_rocm_route_decode_step_segments(ctx.stream(), rq, rk, q_norm, k_norm, eps, inv_tok, n_tok, inv_page,
                                             page_mod, head_cls, router_keys, summaries, d, block_min, block_max,
                                             prompt_blocks, abi(state), &p, capacity, mask, z_out, rqk_out,
                                             segments));
}

static_assert(kMaxKeySegments == UOCR_ROCM_MAX_KEY_SEGMENTS, "the segment layout of include/uocr_rocm.h");

std::int64_t attend_segments_scratch_floats(std::int64_t heads, std::int64_t hd, std::int64_t max_live) {
  return uocr_rocm_attend_segments_scratch_floats(heads, hd, max_live);
}

void attend_rope_kv_step_segments(const Context& ctx, const float* q, const float* k_row, const float* v_row,
                                  float* k_cache, float* v_cache, std::int64_t heads, std::int64_t hd,
                                  const std::int32_t* segments, std::int64_t max_live, float scale,
                                  const StepState* state, const float* inv_tok, std::int64_t n_tok,
                                  const float* inv_page, std::int64_t page_mod, float* scratch,
                                  std::int64_t capacity, float* out) {
  check(uocr_rocm_attend_rope_kv_step_segments(ctx.stream(), q, k_row, v_row, k_cache, v_cache, heads, hd, segments,
                                               max_live, scale, abi(state), inv_tok, n_tok, inv_page, page_mod,
                                               scratch, capacity, out));
}

void attend_rope_kv_step_segments_bf16(const Context& ctx, const float* q, const float* k_row, const float* v_row,
                                       std::uint16_t* k_cache, std::uint16_t* v_cache, std::int64_t heads,
                                       std::int64_t hd, const std::int32_t* segments, std::int64_t max_live,
                                       float scale, const StepState* state, const float* inv_tok,
                                       std::int64_t n_tok, const float* inv_page, std::int64_t page_mod,
                                       float* scratch, std::int64_t capacity, float* out) {
  check(uocr_rocm_attend_rope_kv_step_segments_bf16(ctx.stream(), q, k_row, v_row, k_cache, v_cache, heads, hd,
                                                    segments, max_live, scale, abi(state), inv_tok, n_tok, inv_page,
                                                    page_mod, scratch, capacity, out));
}

void attend_merge_gemv_bf16(const Context& ctx, const float* scratch, std::int64_t heads, std::int64_t hd,
                            std::int64_t max_live, const std::uint16_t* w, std::int64_t n, const float* bias, float* y,
                            float* x_out) {
  check(uocr_rocm_attend_merge_gemv_bf16(ctx.stream(), scratch, heads, hd, max_live, w, n, bias, y, x_out));
}

}  // namespace uocr::rocm
