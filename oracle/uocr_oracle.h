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

#ifdef __cplusplus
}
#endif

#endif /* UOCR_ORACLE_H_ */
