#pragma once

// A whole decode step of the decoder on the rocm backend, captured once as
// a graph and replayed per token, as the reference's CudaDecoder::step
// replays decode_body (src/model/cuda/cuda_decoder.cpp:300-330,
// src/model/cuda/cuda_decode_step.cpp:13-70): the embedding row, every
// layer's routed attention and MLP with their residual adds and norms, the
// final norm and the LM head, with only the StepState rewritten between
// tokens.
//
// A layer is the reference's decode layer (decode_attention and the layer
// loop of decode_body):
//   h = rms(x) w_in;  q, k, v, rq, rk = h Wq, h Wk, h Wv, h Wrq, h Wrk;
//   rq, rk = router_norm(rq) w_rq, router_norm(rk) w_rk;
//   rope(q, k, rq, rk) at (tok, page);  append k, v, rk at pos;
//   mask = route(summaries of the router keys, rq, query_page);
//   attn = softmax(q K^T / sqrt(hd) + mask) V;  x += attn Wo;
//   h = rms(x) w_post;  x += mlp(h)
// where route is the block router (the current block's summary, scores of
// the blocks before the local window, candidates from the prompt blocks'
// image pages, top-m 1.5-entmax, the key mask), rope is PageRope (the first
// half - page_pairs pairs on the token axis at 1 / theta^(i / n_tok), the
// rest on the page axis at 1 / page_theta^(i / page_pairs), page taken mod
// page_mod), and mlp is dense, silu(h Wg) * (h Wu) Wd, or a mixture of
// experts: the shared experts' MLP plus sum_j s_j expert_j(h) over the top
// k experts of softmax(h W_gate) (fp32 gate), the routed sum in top-k rank
// order. After the last layer logits = (rms(x) w_final) W_lm. Int8 weights
// are not part of it.
//
// Launches per step: 1 + per layer 7 (dense) or 8 (mixture of experts) +
// 1. The residual add of each sublayer is the prologue of the next
// projection (the fused GEMVs); the five projections of h are one GEMV over
// the stacked rows; the router norms, the router rope, the router key's
// append, the summary, the scores and the route are one launch; rope of q
// and k, both appends and the attention are one op of two launches; the
// router's logits are formed in the shared experts' gate/up launch, the top
// k inside the routed experts' gate/up launch, and the shared experts' down
// product and the routed experts' sum in the routed experts' down launch.
// The router also lists the keys its mask keeps (at most the local window
// and top_k blocks), and the attention's splits walk that list rather than
// every mask entry.

#include <cstdint>
#include <memory>
#include <vector>

#include "backend/rocm/context.h"
#include "backend/rocm/ops.h"

namespace uocr::rocm {

// A row's rotary coordinate (src/model/page_rope.h): the token axis and the
// page axis.
struct RopeCoord {
  std::int64_t tok = 0;
  std::int64_t page = 0;
};

struct DecoderDims {
  std::int64_t hidden = 1280;
  std::int64_t heads = 10;
  std::int64_t head_dim = 128;
  std::int64_t index_dim = 128;  // router query/key width; equal to head_dim (one rope table serves both)
  std::int64_t vocab = 129280;
  std::int64_t capacity = 8192;  // key/value positions per layer
  float eps = 1e-6f;
  double rope_theta = 1e4;   // token axis
  double page_theta = 256.0;  // page axis
  std::int64_t page_pairs = 1;  // rotary pairs on the page axis (0: every pair on the token axis)
  std::int64_t page_mod = 2;    // page coordinate taken mod this (0: as given)
  RouteParams router;           // block size, local window, top m / top k, entmax scale and prior
  bool bf16_cache = false;      // key/value cache in bf16 (half the bytes) instead of the reference's fp32
  // The prompt's attention on the bf16 matrix cores with each fp32 operand
  // split into bf16 hi + lo parts (attention_masked: 4-5x faster over long
  // prompts, each attention output within one bf16 step of the fp32
  // products' rounding) instead of the fp32 products the reference keeps.
  bool split_attention = false;
  bool trace = false;           // keep each layer's intermediate values of the last step (for checking)
};

// A mixture-of-experts MLP, device weights owned by the caller.
struct MoeWeights {
  const float* gate = nullptr;                // [experts, hidden] fp32 router
  const std::uint16_t* up_stack = nullptr;    // [experts * expert_ffn, hidden]
  const std::uint16_t* gate_stack = nullptr;  // [experts * expert_ffn, hidden]
  const std::uint16_t* down_stack = nullptr;  // [experts * hidden, expert_ffn]
  std::int64_t experts = 64;
  std::int64_t top_k = 6;
  std::int64_t expert_ffn = 896;
  const std::uint16_t* shared_gate = nullptr;  // [shared_ffn, hidden]
  const std::uint16_t* shared_up = nullptr;    // [shared_ffn, hidden]
  const std::uint16_t* shared_down = nullptr;  // [hidden, shared_ffn]
  std::int64_t shared_ffn = 1792;
};

// Device weights of one layer, owned by the caller (bf16 bits, fp32 norms).
// The MLP is dense (gate, up, down, ffn) unless moe is set.
struct LayerWeights {
  const float* input_norm = nullptr;  // [hidden]
  // [3 * heads * head_dim + 2 * index_dim, hidden]: the rows of Wq, Wk, Wv,
  // the router's Wq and the router's Wk stacked in that order.
  const std::uint16_t* qkv = nullptr;
  const float* router_q_norm = nullptr;  // [index_dim]
  const float* router_k_norm = nullptr;  // [index_dim]
  const float* head_cls = nullptr;       // [index_dim]: the blocks' summary query
  const std::uint16_t* o = nullptr;      // [hidden, heads * head_dim]
  const float* post_norm = nullptr;      // [hidden]
  const std::uint16_t* gate = nullptr;   // [ffn, hidden]
  const std::uint16_t* up = nullptr;     // [ffn, hidden]
  const std::uint16_t* down = nullptr;   // [hidden, ffn]
  std::int64_t ffn = 896;
  const MoeWeights* moe = nullptr;
};

// One layer's values in the last step, kept when DecoderDims::trace is set.
struct LayerTrace {
  std::vector<float> x_in;   // residual stream entering the layer [hidden]
  std::vector<float> rq;     // router query after norm and rope [index_dim]
  std::vector<float> rk;     // router key after norm and rope [index_dim]
  std::vector<float> z;      // scores of the blocks before the local window
  std::vector<float> mask;   // the key mask [pos + 1]
  std::vector<float> x_mid;  // residual stream after the attention sublayer [hidden]
};

class DecodeStep {
 public:
  // embed [vocab, hidden] bf16, final_norm [hidden], lm_head [vocab, hidden]
  // bf16; every pointer (and every MoeWeights) stays owned by the caller and
  // must outlive this. Every shape is checked against the kernels' limits
  // before the step is captured (std::invalid_argument).
  DecodeStep(const Context& ctx, const DecoderDims& dims, const std::uint16_t* embed, std::vector<LayerWeights> layers,
             const float* final_norm, const std::uint16_t* lm_head);
  ~DecodeStep();
  DecodeStep(const DecodeStep&) = delete;
  DecodeStep& operator=(const DecodeStep&) = delete;

  // The prompt's blocks' image pages (min_page[b] < 0: block b holds no
  // image; block_image_pages, src/model/page_layout.cpp:55-69), which
  // confine a query with query_page >= 0 to the blocks of its page. Re-records
  // the step; none by default.
  void set_prompt_blocks(const std::vector<std::int64_t>& min_page, const std::vector<std::int64_t>& max_page);

  // The prompt rows x [rows, hidden] (host fp32 embeddings) at positions
  // length() .. length() + rows - 1 through every layer, writing the caches,
  // and the logits of the last row (CudaDecoder::run, cuda_decoder.cpp:
  // 248-286; the prompt blocks' pages come from set_prompt_blocks): the
  // projections on the matrix cores, per row the router's block scores and
  // key mask, the masked attention as fp32 products and a row softmax, the
  // dense or mixture-of-experts MLP (the experts' rows gathered by the
  // device's top-k, their outputs scattered back in expert order). coords
  // holds one rotary coordinate per row; query_pages one page per row, or
  // is empty (every row unconfined). Over a bf16 cache the new keys and
  // values are rounded to bf16 as they are cached, and the prompt's
  // attention reads them back from the cache, as the decode steps do. The
  // rows must fit the cache (reserve).
  std::vector<float> prefill(const std::vector<float>& x, const std::vector<RopeCoord>& coords,
                             const std::vector<std::int64_t>& query_pages = {});

  // Grows every layer's caches to hold at least `keys` positions, as
  // CudaDecoder::reserve does (src/model/cuda/cuda_decoder.cpp:94-117): the
  // capacity becomes max(keys, 2 capacity + 1024), the length() rows written
  // so far (and their blocks' summaries and the prompt blocks' pages) are
  // copied over, the position-sized buffers are grown, and the step is
  // recorded again. No-op when keys <= capacity(); std::invalid_argument
  // past 4096 router blocks.
  void reserve(std::int64_t keys);
  std::int64_t capacity() const { return dims_.capacity; }
  std::int64_t block_size() const { return dims_.router.block_size; }
  // A new sequence from position 0 over the same caches (what
  // CudaDecoder::prefill does with its length); nothing is cleared, since
  // no position at or past length() is read.
  void rewind() {
    length_ = 0;
    last_pos_ = -1;
  }

  // Feeds `token` at the next position (length() before the call), rotated
  // at `coord`, its attention routed within query_page's blocks (-1: any
  // block), and returns the logits [vocab] (CudaDecoder::step).
  std::vector<float> step(std::int64_t token, RopeCoord coord, std::int64_t query_page = -1);
  std::int64_t length() const { return length_; }

  // For timing: set_state writes the StepState of a step at `pos` and
  // replay enqueues one replay on the context's stream without reading the
  // logits back or advancing length(). The state goes through one pinned
  // host buffer: call set_state again only after the stream has taken the
  // previous copy (step() synchronises).
  void set_state(std::int64_t token, std::int64_t pos, RopeCoord coord, std::int64_t query_page = -1);
  void replay();
  // Zeroes every layer's caches and the length (a new sequence).
  void reset();

  // The last step's per-layer values; throws std::logic_error unless
  // DecoderDims::trace was set.
  std::vector<LayerTrace> trace() const;
  // The last prefill's key masks, per layer [rows, keys] (keys = the
  // positions after the prompt); throws std::logic_error unless
  // DecoderDims::trace was set.
  const std::vector<std::vector<float>>& prefill_trace() const;

 private:
  void validate() const;
  void record();
  void body();

  const Context& ctx_;
  DecoderDims dims_;
  const std::uint16_t* embed_;
  std::vector<LayerWeights> layers_;
  const float* final_norm_;
  const std::uint16_t* lm_head_;
  std::int64_t length_ = 0, last_pos_ = -1, capacity_blocks_ = 0, prompt_blocks_ = 0;
  Array inv_tok_, inv_page_, state_, x_[2], h_, delta_, proj_, o_, act_, logits_, scratch_;
  Array segments_;  // the router's live keys of the current layer (kKeySegmentWords int32)
  std::int64_t max_live_ = 1;
  Array block_min_, block_max_;
  Array router_logits_, expert_ids_, expert_weights_, expert_scratch_;
  std::vector<Array> k_cache_, v_cache_, router_keys_, summaries_;
  std::vector<Array> trace_x_in_, trace_rqk_, trace_z_, trace_mask_, trace_x_mid_;
  // per layer, the dense MLP's (or the shared experts') gate and up rows
  // stacked [2 ffn, hidden]: the prompt pass forms both in one product
  std::vector<Array> gate_up_;
  std::vector<std::vector<float>> prefill_masks_;
  std::unique_ptr<PinnedBuffer> state_host_, logits_host_;
  std::unique_ptr<Graph> graph_;
};

}  // namespace uocr::rocm
