/*
 * uocr_oracle.h: declarations of the CPU oracle (oracle/uocr_oracle.c), the
 * restatement of the reference's fp32 CPU path. TEST INFRASTRUCTURE ONLY:
 * included by the parity tests, never by the product.
 */
#ifndef UOCR_ORACLE_H_
#define UOCR_ORACLE_H_

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

float orc_bf16_to_f32(uint16_t b);
uint16_t orc_f32_to_bf16(float v);
void orc_f32_to_bf16_array(const float* src, uint16_t* dst, int64_t n);
void orc_bf16_to_f32_array(const uint16_t* src, float* dst, int64_t n);
void orc_set_threads(int t);
int orc_threads(void);
/* fn(ctx, r) for every r in [0, count) over orc_threads() threads, thread t
 * taking rows t, t + T, ... (the reference's parallel_for); a row's result
 * never depends on T. */
typedef void (*orc_row_fn)(void* ctx, int64_t row);
void orc_parallel_rows(int64_t count, orc_row_fn fn, void* ctx);
void orc_rms_norm(float* x, const float* w, int64_t rows, int64_t cols, float eps);
void orc_layer_norm(float* x, const float* w, const float* b, int64_t rows, int64_t cols, float eps);
void orc_gelu_erf(float* x, int64_t n);
void orc_silu(float* x, int64_t n);
void orc_mul_into(float* g, const float* u, int64_t n);
void orc_add_into(float* x, const float* y, int64_t n);
void orc_rope_inv(float* inv, int64_t n, double theta);
void orc_rope_apply(float* x, int64_t rows, int64_t heads, int64_t dim, const int64_t* tok, const int64_t* page,
                    const float* inv_tok, int64_t n_tok, const float* inv_page, int64_t n_page, int64_t page_mod,
                    int64_t one_tok, int64_t one_page);
void orc_embed(const uint16_t* table, const int64_t* ids, int64_t n, int64_t cols, float* dst);
void orc_add_rms_norm(float* x, const float* delta, const float* w, float* h, int64_t rows, int64_t cols, float eps);
void orc_decode_chain(const uint16_t* table, int64_t token, const float* delta, const float* w, float* x, float* h,
                      int64_t cols, float eps, float* q, int64_t q_heads, float* k, int64_t k_heads, int64_t dim,
                      int64_t pos, const float* inv, int64_t n_tok, int64_t reps);
void orc_swiglu(const float* in, float* out, int64_t rows, int64_t ffn);
void orc_router_norm(float* x, const float* w, int64_t rows, int64_t cols, float eps);
void orc_linear(const float* x, int64_t m, int64_t k, const float* w, int64_t n, const float* bias, float* y);
void orc_softmax_rows(float* x, int64_t rows, int64_t cols);
void orc_attention_one(const float* q, const float* k, const float* v, int64_t keys, int64_t width, int64_t heads,
                       int64_t hd, const float* bias, float scale, float* out);
void orc_expert_topk(const float* logits, int64_t rows, int64_t experts, int64_t k, int64_t* ids, float* weights);
void orc_scale_add_mask(float* x, float scale, const float* mask, int64_t batch, int64_t rows, int64_t cols);
void orc_quick_gelu(float* x, int64_t n);
/* The block router (src/model/block_router.cpp, src/model/attention_plan.cpp). */
void orc_block_summaries(const float* rk, int64_t keys, int64_t d, const float* cls, int64_t block_size,
                         float* out);
void orc_block_scores(const float* rq, int64_t lq, const float* summaries, int64_t nblk, int64_t d,
                      const int64_t* q_pos, int64_t block_size, int64_t local_blocks, float* out);
void orc_entmax15(float* x, int64_t n);
int64_t orc_select_blocks(const float* scores, int64_t lq, int64_t nblk, const uint8_t* candidate, int64_t top_m,
                          int64_t top_k, float idx_scale, float floor_p, float sigma, int64_t* block, float* bias,
                          uint8_t* valid);
void orc_key_mask(const int64_t* block, const float* bias, const uint8_t* valid, int64_t width, int64_t rows,
                  int64_t first_pos, int64_t keys, int64_t block_size, int64_t local_blocks, float* mask);
int orc_page_candidates(const int64_t* min_page, const int64_t* max_page, int64_t known, int64_t page, int64_t nblk,
                        uint8_t* out);
void orc_route_one(const float* rq, const float* rk, int64_t pos, int64_t d, const float* cls,
                   const int64_t* min_page, const int64_t* max_page, int64_t known, int64_t query_page,
                   int64_t block_size, int64_t local_blocks, int64_t top_m, int64_t top_k, float idx_scale,
                   float floor_p, float sigma, float* summaries, float* mask);

/* The vision encoder and its ops (oracle/uocr_oracle_vision.c;
 * src/backend/reference/ops.cpp, src/model/sam_encoder.cpp,
 * src/model/clip_encoder.cpp, src/model/vision_encoder.cpp). Weight
 * matrices are fp32 [out, in] (convolutions [out, in * kh * kw]). */
void orc_chw_to_hwc(const float* x, int64_t c, int64_t h, int64_t w, float* y);
void orc_hwc_to_chw(const float* x, int64_t h, int64_t w, int64_t c, float* y);
void orc_concat_cols(const float* a, int64_t ca, const float* b, int64_t cb, int64_t rows, float* out);
void orc_im2col(const float* x, int64_t c, int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t stride, int64_t pad,
                float* cols);
void orc_conv2d(const float* x, int64_t c, int64_t h, int64_t w, const float* weight, const float* bias, int64_t o,
                int64_t kh, int64_t kw, int64_t stride, int64_t pad, float* out);
void orc_layer_norm_channels(float* x, const float* w, const float* b, int64_t c, int64_t h, int64_t wd, float eps);
void orc_attention_head(const float* q, const float* k, const float* v, int64_t lq, int64_t lk, int64_t d, int64_t dv,
                        const float* bias, float scale, float* out);
void orc_resize_bicubic_aa(const float* x, int64_t c, int64_t h, int64_t w, int64_t oh, int64_t ow, float* out);
void orc_resize_linear_rows(const float* x, int64_t len, int64_t c, int64_t out_len, float* out);
void orc_relative_positions(const float* table, int64_t len, int64_t d, int64_t size, float* out);
void orc_rel_pos_bias(const float* q, int64_t ldq, int64_t h, int64_t w, int64_t d, const float* rh, const float* rw,
                      float* bias);

typedef struct {
  int64_t image, patch, width, layers, heads, mlp, window, neck, net2, net3;
} orc_sam_dims;

typedef struct {
  const float *norm1_w, *norm1_b, *qkv_w, *qkv_b, *proj_w, *proj_b;
  const float *rel_h, *rel_w; /* [rel_len, head_dim] each */
  int64_t rel_len;
  const float *norm2_w, *norm2_b, *lin1_w, *lin1_b, *lin2_w, *lin2_b;
  int global;
} orc_sam_block;

typedef struct {
  const float *patch_w, *patch_b; /* [width, 3 * patch * patch], [width] */
  const float* pos_embed;         /* [image / patch, image / patch, width] */
  const orc_sam_block* blocks;    /* [layers] */
  const float *neck0_w, *neck1_w, *neck1_b, *neck2_w, *neck3_w, *neck3_b, *net2_w, *net3_w;
} orc_sam_weights;

typedef struct {
  int64_t width, layers, heads, mlp, positions;
} orc_clip_dims;

typedef struct {
  const float *ln1_w, *ln1_b, *qkv_w, *qkv_b, *out_w, *out_b, *ln2_w, *ln2_b, *fc1_w, *fc1_b, *fc2_w, *fc2_b;
} orc_clip_layer;

typedef struct {
  const float* class_embedding; /* [width] */
  const float* positions;       /* [positions, width] */
  const float *pre_ln_w, *pre_ln_b;
  const orc_clip_layer* layers;
} orc_clip_weights;

typedef struct {
  orc_sam_dims sam_dims;
  orc_sam_weights sam;
  orc_clip_dims clip_dims;
  orc_clip_weights clip;
  const float *projector_w, *projector_b; /* [hidden, clip width + net3] */
  const float *newline, *separator;       /* [hidden] */
  int64_t hidden;
} orc_vision_weights;

/* round_x: round every linear's input to bf16 as the device linear does
 * (0: the reference's CPU arithmetic). */
int64_t orc_sam_forward(const orc_sam_weights* wt, const orc_sam_dims* dm, const float* image, int64_t s, float* out,
                        int round_x);
int orc_clip_forward(const orc_clip_weights* wt, const orc_clip_dims* dm, const float* features, int64_t g, float* x,
                     int round_x);
int64_t orc_encode_view(const orc_vision_weights* wt, const float* image, int64_t s, float* out, int round_x);
int64_t orc_page_image_tokens(int64_t global_grid, int64_t tile_grid, int64_t tiles_wide, int64_t tiles_high,
                              int tiled);
int64_t orc_encode_page(const orc_vision_weights* wt, const float* global, int64_t global_size, const float* tiles,
                        int64_t n_tiles, int64_t tile_size, int64_t tiles_wide, int64_t tiles_high, float* out,
                        int round_x);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_ORACLE_H_ */
