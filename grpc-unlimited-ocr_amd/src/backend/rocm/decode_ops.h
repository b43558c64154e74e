#pragma once

// Ops for one decode step whose shapes do not depend on how many tokens came
// before: the fed token and its rope coordinate are read from a StepState on
// the device, so a captured step replays for every token with only the
// StepState rewritten between replays. Same contract as the reference's
// src/backend/cuda/decode_ops.h:17-27.

#include <cstdint>

#include "backend/rocm/context.h"
#include "backend/rocm/ops.h"

namespace uocr::rocm {

// The five int64 words a decode step reads from the device (the layout of
// src/backend/cuda/decode_ops.h:17-23, which the kernels index directly).
struct StepState {
  std::int64_t token;       // id whose embedding row enters the step
  std::int64_t pos;         // cache row written this step; pos + 1 keys are live after it
  std::int64_t tok;         // rotary coordinate on the token axis
  std::int64_t page;        // rotary coordinate on the page axis
  std::int64_t query_page;  // page the block router confines this query to (-1: any)
};

void embed_step(const Context& ctx, const std::uint16_t* table, const StepState* state, std::int64_t cols, float* dst);
void rope_step(const Context& ctx, float* x, std::int64_t heads, std::int64_t dim, const StepState* state,
               const float* inv_tok, std::int64_t n_tok, const float* inv_page, std::int64_t page_mod);

// New: Q and K of the step row in one launch, and the bf16-activation forms.
void rope_qk_step(const Context& ctx, float* q, std::int64_t q_heads, float* k, std::int64_t k_heads, std::int64_t dim,
                  const StepState* state, const float* inv_tok, std::int64_t n_tok, const float* inv_page,
                  std::int64_t page_mod);
void rope_qk_step_bf16(const Context& ctx, std::uint16_t* q, std::int64_t q_heads, std::uint16_t* k,
                       std::int64_t k_heads, std::int64_t dim, const StepState* state, const float* inv_tok,
                       std::int64_t n_tok, const float* inv_page, std::int64_t page_mod);
void embed_step_bf16(const Context& ctx, const std::uint16_t* table, std::int64_t table_rows, const StepState* state,
                     std::int64_t cols, std::uint16_t* dst);

// Writes `row` (width floats) into row state->pos of `cache`
// (src/backend/cuda/decode_ops.h:28-29). With capacity >= 0 a pos outside
// [0, capacity) writes nothing; -1 trusts pos, as the reference does.
void append_step(const Context& ctx, float* cache, const float* row, std::int64_t width, const StepState* state,
                 std::int64_t capacity = -1);
// One query row [heads * hd] attends over cache rows 0..state->pos with an
// optional additive key mask; out [heads * hd] (decode_ops.h:42-47). The
// per-split records go to `scratch`, attend_scratch_floats(heads, hd,
// capacity) floats that the caller owns.
std::int64_t attend_scratch_floats(std::int64_t heads, std::int64_t hd, std::int64_t capacity);
void attend_step(const Context& ctx, const float* q, const float* k_cache, const float* v_cache, std::int64_t heads,
                 std::int64_t hd, const float* mask, float scale, const StepState* state, float* scratch,
                 std::int64_t capacity, float* out);

// New: a bf16 key/value cache (rows rounded to bf16 on append, widened to
// fp32 in the attention); half the cache bytes. The fused step of
// attend_rope_kv_step below over such a cache.
void attend_rope_kv_step_bf16(const Context& ctx, const float* q, const float* k_row, const float* v_row,
                              std::uint16_t* k_cache, std::uint16_t* v_cache, std::int64_t heads, std::int64_t hd,
                              const float* mask, float scale, const StepState* state, const float* inv_tok,
                              std::int64_t n_tok, const float* inv_page, std::int64_t page_mod, float* scratch,
                              std::int64_t capacity, float* out);

// New: the step's embedding row fused with the first norm: x = table[token]
// (+ delta, which may be null), h = rms_norm(x) * w.
void embed_add_rms_norm_step(const Context& ctx, const std::uint16_t* table, std::int64_t table_rows,
                             const StepState* state, const float* delta, const float* w, float* x, float* h,
                             std::int64_t cols, float eps);

// New: rope_qk_step on (q, k_row), the appends of the rotated key and of
// v_row at pos, and attend_step, in attend_step's two launches; q, k_row and
// v_row are left unrotated.
void attend_rope_kv_step(const Context& ctx, const float* q, const float* k_row, const float* v_row, float* k_cache,
                         float* v_cache, std::int64_t heads, std::int64_t hd, const float* mask, float scale,
                         const StepState* state, const float* inv_tok, std::int64_t n_tok, const float* inv_page,
                         std::int64_t page_mod, float* scratch, std::int64_t capacity, float* out);

// ---- the block router of the step (src/backend/cuda/decode_ops.h:30-40) --------------------

// The summary of the block holding pos, into summaries[pos / block_size];
// max_blocks bounds the summaries buffer.
void summary_step(const Context& ctx, const float* router_keys, std::int64_t d, const float* head_cls,
                  std::int64_t block_size, const StepState* state, std::int64_t max_blocks, float* summaries);
// z[b] = rq . summaries[b] / sqrt d for every block up to the one holding pos.
void scores_step(const Context& ctx, const float* rq, const float* summaries, std::int64_t d, std::int64_t block_size,
                 const StepState* state, std::int64_t max_blocks, float* z);
// The routed key mask mask[0..pos] of the step's query from z.
void route_step(const Context& ctx, const float* z, std::int64_t max_blocks, const std::int64_t* block_min,
                const std::int64_t* block_max, std::int64_t prompt_blocks, const StepState* state,
                const RouteParams& params, float* mask);
// New: the router half of the step in one launch (router norms, rope at the
// step's coordinate, the router key's append, summary_step, scores_step and
// route_step), bitwise the separate steps; z_out and rqk_out may be null.
void route_decode_step(const Context& ctx, const float* rq, const float* rk, const float* q_norm, const float* k_norm,
                       float eps, const float* inv_tok, std::int64_t n_tok, const float* inv_page,
                       std::int64_t page_mod, const float* head_cls, float* router_keys, float* summaries,
                       std::int64_t d, const std::int64_t* block_min, const std::int64_t* block_max,
                       std::int64_t prompt_blocks, const StepState* state, const RouteParams& params,
                       std::int64_t capacity, float* mask, float* z_out = nullptr, float* rqk_out = nullptr,
                       std::int32_t* segments = nullptr);

// New: the keys a routed step reads as segments (segments != null above):
// kKeySegmentWords int32, {segment count, live keys, 0, 0} and then per
// segment {first key, keys, bias bits, 0} in key order (the selected blocks,
// clipped at the local window, then the window).
constexpr std::int64_t kMaxKeySegments = 33;
constexpr std::int64_t kKeySegmentWords = 4 * (1 + kMaxKeySegments);
// The most keys the block router lets one step read: the local window and
// top_k (at least one) whole blocks.
inline std::int64_t max_live_keys(const RouteParams& p) {
  return ((p.top_k > 1 ? p.top_k : 1) + p.local_blocks) * p.block_size;
}

// New: attend_rope_kv_step over those segments' keys alone instead of a mask
// (each split walks a run of the live keys); max_live bounds the live keys
// of every call and fixes the split count. Scratch:
// attend_segments_scratch_floats(heads, hd, max_live) floats. With out null
// the splits' records stay in scratch for attend_merge_gemv_bf16.
std::int64_t attend_segments_scratch_floats(std::int64_t heads, std::int64_t hd, std::int64_t max_live);
void attend_rope_kv_step_segments(const Context& ctx, const float* q, const float* k_row, const float* v_row,
                                  float* k_cache, float* v_cache, std::int64_t heads, std::int64_t hd,
                                  const std::int32_t* segments, std::int64_t max_live, float scale,
                                  const StepState* state, const float* inv_tok, std::int64_t n_tok,
                                  const float* inv_page, std::int64_t page_mod, float* scratch,
                                  std::int64_t capacity, float* out);
// The same over a bf16 key/value cache (the rotated key and v_row rounded
// to bf16 on append, cache rows widened to fp32 in the attention).
void attend_rope_kv_step_segments_bf16(const Context& ctx, const float* q, const float* k_row, const float* v_row,
                                       std::uint16_t* k_cache, std::uint16_t* v_cache, std::int64_t heads,
                                       std::int64_t hd, const std::int32_t* segments, std::int64_t max_live,
                                       float scale, const StepState* state, const float* inv_tok,
                                       std::int64_t n_tok, const float* inv_page, std::int64_t page_mod,
                                       float* scratch, std::int64_t capacity, float* out);
// New: y = bf16(the merge of those records) . w^T (+ bias) in one launch,
// bitwise the attention's own merge then gemv_bf16 (the o projection,
// cuda_decode_step.cpp:42-44); x_out (optional) receives the merged row.
void attend_merge_gemv_bf16(const Context& ctx, const float* scratch, std::int64_t heads, std::int64_t hd,
                            std::int64_t max_live, const std::uint16_t* w, std::int64_t n, const float* bias, float* y,
                            float* x_out = nullptr);

}  // namespace uocr::rocm
