/*
 * uocr_oracle.c: CPU restatement of grpc-unlimited-ocr's fp32 reference path
 * for the fused layer ops.
 *
 * TEST INFRASTRUCTURE ONLY. This file is the checker: the parity tests,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg load it to compute
 * the expected values and the CPU baseline time. No product path may load or
 * call it; the product is the HIP library built from grpc-unlimited-ocr_amd/csrc.
 *
 * Each function restates the reference's arithmetic in the reference's
 * order (the fp64 accumulations and the points where values are cast to
 * fp32 matter), citing the file:line it follows. Built with -O3 (the
 * reference's Release build) and -ffp-contract=off, so every fp32 product
 * and sum is rounded on its own as in the reference's x86-64 build.
 *
 * How each function is pinned (tests/test_oracle.py):
 *   bf16 conversions: the reference's known answers (tests/dtype_test.cpp:20-28)
 *     plus an exhaustive comparison with an independent rounding rule.
 *   rms_norm, layer_norm, gelu_erf, silu: the reference's hand-worked values
 *     (tests/ops_test.cpp:26-50), closed forms in fp64 on random rows, and
 *     bit-equality with the reference's own ops.cpp compiled into oracle/_ref.
 *   rope: identity at position 0, per-pair norm, rope(p) then rope(-p),
 *     an fp64 complex-rotation brute force, and bit-equality with the
 *     reference's page_rope.cpp compiled into oracle/_ref.
 *   embed (gather): exact equality with numpy's row take of the widened table.
 *   The composed chains (add + rms_norm, swiglu) are pinned through their
 *   parts and an fp64 closed form of the whole chain.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "uocr_oracle.h"

#define ORC_API __attribute__((visibility("default")))

/* ---- bf16 (src/tensor/dtype.h:32-46) ----------------------------------- */

static inline uint32_t f32_bits(float v) {
  uint32_t u;
  memcpy(&u, &v, 4);
  return u;
}
static inline float bits_f32(uint32_t u) {
  float v;
  memcpy(&v, &u, 4);
  return v;
}

/* bf16_to_f32: the bits become the top half of a binary32 (dtype.h:33-35). */
ORC_API float orc_bf16_to_f32(uint16_t b) { return bits_f32((uint32_t)b << 16); }

/* f32_to_bf16: round to nearest even; NaN keeps its top bits and is made
 * quiet with 0x0040 (dtype.h:39-46). */
ORC_API uint16_t orc_f32_to_bf16(float v) {
  const uint32_t bits = f32_bits(v);
  if ((bits & 0x7fffffffU) > 0x7f800000U) return (uint16_t)((bits >> 16) | 0x0040U);
  const uint32_t rounding = 0x7fffU + ((bits >> 16) & 1U);
  return (uint16_t)((bits + rounding) >> 16);
}

ORC_API void orc_f32_to_bf16_array(const float* src, uint16_t* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_f32_to_bf16(src[i]);
}
ORC_API void orc_bf16_to_f32_array(const uint16_t* src, float* dst, int64_t n) {
  for (int64_t i = 0; i < n; ++i) dst[i] = orc_bf16_to_f32(src[i]);
}

/* ---- threading (src/backend/reference/parallel.h:23-42, ops.cpp:15,88-89)
 * The reference spreads a row loop over thread_count() threads, thread t
 * taking rows t, t + T, t + 2T, ...; each row is computed by one thread with
 * the serial arithmetic, so the result never depends on T. Norms use it;
 * the activations, the add and rope run serially in the reference. */

static int g_threads = 1;
ORC_API void orc_set_threads(int t) { g_threads = t < 1 ? 1 : t; }
ORC_API int orc_threads(void) { return g_threads; }

typedef orc_row_fn row_fn;
typedef struct {
  row_fn fn;
  void* ctx;
  int64_t t, threads, count;
} strip_job;

static void* strip_main(void* arg) {
  const strip_job* j = (const strip_job*)arg;
  for (int64_t i = j->t; i < j->count; i += j->threads) j->fn(j->ctx, i);
  return NULL;
}

void orc_parallel_rows(int64_t count, orc_row_fn fn, void* ctx) {
  int64_t threads = g_threads < count ? g_threads : count;
  if (threads <= 1) {
    for (int64_t i = 0; i < count; ++i) fn(ctx, i);
    return;
  }
  pthread_t* tid = (pthread_t*)malloc((size_t)threads * sizeof(pthread_t));
  strip_job* jobs = (strip_job*)malloc((size_t)threads * sizeof(strip_job));
  int64_t started = 0;
  for (int64_t t = 0; t < threads; ++t) {
    jobs[t] = (strip_job){fn, ctx, t, threads, count};
    if (pthread_create(&tid[t], NULL, strip_main, &jobs[t]) != 0) break;
    ++started;
  }
  /* A thread that could not start leaves its rows to the caller. */
  for (int64_t t = started; t < threads; ++t) strip_main(&jobs[t]);
  for (int64_t t = 0; t < started; ++t) pthread_join(tid[t], NULL);
  free(jobs);
  free(tid);
}

static void parallel_for(int64_t count, row_fn fn, void* ctx) { orc_parallel_rows(count, fn, ctx); }

/* ---- norms --------------------------------------------------------------- */

typedef struct {
  float* x;
  const float* w;
  const float* b;
  int64_t cols;
  float eps;
} norm_ctx;

/* reference::rms_norm, one row (src/backend/reference/ops.cpp:132-140):
 * ss in fp64, inv = float(1 / sqrt(ss / c + eps)) in fp64, then
 * v = w * (v * inv) in fp32. */
static void rms_row(void* p, int64_t r) {
  const norm_ctx* c = (const norm_ctx*)p;
  float* v = c->x + r * c->cols;
  double ss = 0.0;
  for (int64_t i = 0; i < c->cols; ++i) ss += (double)v[i] * v[i];
  const float inv = (float)(1.0 / sqrt(ss / (double)c->cols + c->eps));
  for (int64_t i = 0; i < c->cols; ++i) v[i] = c->w[i] * (v[i] * inv);
}

ORC_API void orc_rms_norm(float* x, const float* w, int64_t rows, int64_t cols, float eps) {
  norm_ctx c = {x, w, NULL, cols, eps};
  parallel_for(rows, rms_row, &c);
}

/* reference::layer_norm, one row (ops.cpp:114-126): two-pass fp64 mean and
 * variance, inv = 1 / sqrt(var + eps) in fp64, then
 * v = float((v - mean) * inv) * w + b with the last product and sum in fp32. */
static void ln_row(void* p, int64_t r) {
  const norm_ctx* c = (const norm_ctx*)p;
  float* v = c->x + r * c->cols;
  double mean = 0.0;
  for (int64_t i = 0; i < c->cols; ++i) mean += v[i];
  mean /= (double)c->cols;
  double var = 0.0;
  for (int64_t i = 0; i < c->cols; ++i) var += (v[i] - mean) * (v[i] - mean);
  var /= (double)c->cols;
  const double inv = 1.0 / sqrt(var + c->eps);
  for (int64_t i = 0; i < c->cols; ++i) v[i] = (float)((v[i] - mean) * inv) * c->w[i] + c->b[i];
}

ORC_API void orc_layer_norm(float* x, const float* w, const float* b, int64_t rows, int64_t cols, float eps) {
  norm_ctx c = {x, w, b, cols, eps};
  parallel_for(rows, ln_row, &c);
}

/* ---- activations (serial, as in the reference) --------------------------- */

/* reference::gelu_erf (ops.cpp:151-155): 0.5f * v * (1 + erf(v * float(M_SQRT1_2)))
 * with std::erf on a float, i.e. erff. */
ORC_API void orc_gelu_erf(float* x, int64_t n) {
  const float k = (float)M_SQRT1_2;
  for (int64_t i = 0; i < n; ++i) {
    const float v = x[i];
    x[i] = 0.5f * v * (1.0f + erff(v * k));
  }
}

/* sigmoid (ops.cpp:40): 1 / (1 + exp(-x)) on a float, i.e. expf. */
static inline float sigmoid(float v) { return 1.0f / (1.0f + expf(-v)); }

/* reference::silu (ops.cpp:163-167): v * sigmoid(v). */
ORC_API void orc_silu(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = x[i] * sigmoid(x[i]);
}

/* g *= u, the multiply of GatedMlp::forward (src/model/feed_forward.cpp:21-22). */
ORC_API void orc_mul_into(float* g, const float* u, int64_t n) {
  for (int64_t i = 0; i < n; ++i) g[i] *= u[i];
}

/* add_into: x += y (src/model/decoder.cpp:39-41). */
ORC_API void orc_add_into(float* x, const float* y, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] += y[i];
}

/* ---- rope ---------------------------------------------------------------- */

/* The frequency table of PageRope's constructor (src/model/page_rope.cpp:17-23):
 * inv[i] = float(1 / pow(theta, i / n)) in fp64. */
ORC_API void orc_rope_inv(float* inv, int64_t n, double theta) {
  for (int64_t i = 0; i < n; ++i) inv[i] = (float)(1.0 / pow(theta, (double)i / (double)n));
}

/* PageRope::apply (src/model/page_rope.cpp:26-56) over x [rows, heads * dim]:
 * per row, the fp32 angle float(tok) * inv_tok[i] (token pairs) or
 * float(page folded mod page_mod) * inv_page[i] (page pairs), cos and sin of
 * the fp32 angle (cosf / sinf), then the rotate-half update of every head:
 * v[i] = a c - b s, v[i + half] = b c + a s. tok / page may be NULL, when
 * every row takes one_tok / one_page (the uocr::cuda::rope convention,
 * src/backend/cuda/ops.h:48-52). Requires n_tok + n_page == dim / 2. */
ORC_API void orc_rope_apply(float* x, int64_t rows, int64_t heads, int64_t dim, const int64_t* tok,
                            const int64_t* page, const float* inv_tok, int64_t n_tok, const float* inv_page,
                            int64_t n_page, int64_t page_mod, int64_t one_tok, int64_t one_page) {
  const int64_t half = dim / 2;
  float* cos_v = (float*)malloc((size_t)(half > 0 ? half : 1) * sizeof(float));
  float* sin_v = (float*)malloc((size_t)(half > 0 ? half : 1) * sizeof(float));
  for (int64_t r = 0; r < rows; ++r) {
    const int64_t tk = tok != NULL ? tok[r] : one_tok;
    const int64_t pg = page != NULL ? page[r] : one_page;
    const float t = (float)tk;
    const float p = (float)(page_mod > 0 ? ((pg % page_mod) + page_mod) % page_mod : pg);
    for (int64_t i = 0; i < n_tok; ++i) {
      const float a = t * inv_tok[i];
      cos_v[i] = cosf(a);
      sin_v[i] = sinf(a);
    }
    for (int64_t i = 0; i < n_page; ++i) {
      const float a = p * inv_page[i];
      cos_v[n_tok + i] = cosf(a);
      sin_v[n_tok + i] = sinf(a);
    }
    float* row = x + r * heads * dim;
    for (int64_t h = 0; h < heads; ++h) {
      float* v = row + h * dim;
      for (int64_t i = 0; i < half; ++i) {
        const float a = v[i], b = v[i + half];
        v[i] = a * cos_v[i] - b * sin_v[i];
        v[i + half] = b * cos_v[i] + a * sin_v[i];
      }
    }
  }
  free(cos_v);
  free(sin_v);
}

/* ---- embedding gather ---------------------------------------------------- */

/* Decoder::embed (src/model/decoder.cpp:85-92) copies rows of the fp32
 * embedding table, which CheckpointWeights::get widened from bf16 at load
 * (src/model/weight_source.cpp:16-23): dst[r] = widen(table[ids[r]]). */
ORC_API void orc_embed(const uint16_t* table, const int64_t* ids, int64_t n, int64_t cols, float* dst) {
  for (int64_t r = 0; r < n; ++r) {
    const uint16_t* src = table + ids[r] * cols;
    for (int64_t i = 0; i < cols; ++i) dst[r * cols + i] = orc_bf16_to_f32(src[i]);
  }
}

/* ---- the composed chains the fused ops replace ---------------------------- */

/* Residual add then norm, the order of Decoder::prefill / step
 * (src/model/decoder.cpp:176-181,196-201) and CudaDecoder::run
 * (src/model/cuda/cuda_decoder.cpp:267-278): x += delta; h = x;
 * h = rms_norm(h, w). */
ORC_API void orc_add_rms_norm(float* x, const float* delta, const float* w, float* h, int64_t rows, int64_t cols,
                              float eps) {
  orc_add_into(x, delta, rows * cols);
  memcpy(h, x, (size_t)(rows * cols) * sizeof(float));
  orc_rms_norm(h, w, rows, cols, eps);
}

/* The batch-1 decode chain of the CPU baseline, `reps` times in one call so
 * that no interpreter overhead sits between the ops: the embedding row of
 * `token` (Decoder::embed, src/model/decoder.cpp:85-92), the residual add
 * and RMSNorm (orc_add_rms_norm above), then rope on q and k at position
 * `pos` (PageRope::apply, src/model/page_rope.cpp:26-56). x receives the
 * embedding row each time, so every repetition does the same work. */
ORC_API void orc_decode_chain(const uint16_t* table, int64_t token, const float* delta, const float* w, float* x,
                              float* h, int64_t cols, float eps, float* q, int64_t q_heads, float* k,
                              int64_t k_heads, int64_t dim, int64_t pos, const float* inv, int64_t n_tok,
                              int64_t reps) {
  for (int64_t r = 0; r < reps; ++r) {
    orc_embed(table, &token, 1, cols, x);
    orc_add_rms_norm(x, delta, w, h, 1, cols, eps);
    orc_rope_apply(q, 1, q_heads, dim, &pos, NULL, inv, n_tok, NULL, 0, 0, 0, 0);
    orc_rope_apply(k, 1, k_heads, dim, &pos, NULL, inv, n_tok, NULL, 0, 0, 0, 0);
  }
}

/* SwiGLU of GatedMlp::forward (src/model/feed_forward.cpp:18-24) on a
 * concatenated [gate | up] row layout: g = silu(gate); g *= up. */
ORC_API void orc_swiglu(const float* in, float* out, int64_t rows, int64_t ffn) {
  for (int64_t r = 0; r < rows; ++r) memcpy(out + r * ffn, in + r * 2 * ffn, (size_t)ffn * sizeof(float));
  orc_silu(out, rows * ffn);
  for (int64_t r = 0; r < rows; ++r) orc_mul_into(out + r * ffn, in + r * 2 * ffn + ffn, ffn);
}

/* ---- the decode-step neighbours and the row ops beside the path ---------- */

/* dot (src/backend/reference/ops.cpp:23-38): eight fp32 partial sums in a
 * fixed order, then ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) + tail. */
static float ref_dot(const float* a, const float* b, int64_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    for (int lane = 0; lane < 8; ++lane) acc[lane] += a[i + lane] * b[i + lane];
  }
  float tail = 0.0f;
  for (; i < n; ++i) tail += a[i] * b[i];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7])) + tail;
}

/* The router's RMSNorm (src/model/decoder.cpp:20-34): non-finite inputs
 * become 0, ss in fp64, inv = float(1 / sqrt(ss / c + eps)), then
 * n = clamp(v * inv, -1e4, 1e4) and v = clamp(n * (1 + w), -1e4, 1e4). */
ORC_API void orc_router_norm(float* x, const float* w, int64_t rows, int64_t cols, float eps) {
  const float clampv = 1.0e4f;
  for (int64_t r = 0; r < rows; ++r) {
    float* v = x + r * cols;
    double ss = 0.0;
    for (int64_t i = 0; i < cols; ++i) {
      if (!isfinite(v[i])) v[i] = 0.0f;
      ss += (double)v[i] * v[i];
    }
    const float inv = (float)(1.0 / sqrt(ss / (double)cols + eps));
    for (int64_t i = 0; i < cols; ++i) {
      float n = v[i] * inv;
      n = n < -clampv ? -clampv : (n > clampv ? clampv : n);
      float y = n * (1.0f + w[i]);
      v[i] = y < -clampv ? -clampv : (y > clampv ? clampv : y);
    }
  }
}

/* linear (ops.cpp:91-109): y[m, n] = dot(x[m], w[n]) (+ bias[n]). The
 * reference's bf16 device paths are compared against this on bf16-rounded
 * x and w (tests/cuda_ops_test.cpp:73-80). */
typedef struct {
  const float* x;
  const float* w;
  const float* bias;
  float* y;
  int64_t k, n;
} linear_ctx;

static void linear_row(void* p, int64_t r) {
  const linear_ctx* c = (const linear_ctx*)p;
  for (int64_t j = 0; j < c->n; ++j) {
    const float sum = ref_dot(c->x + r * c->k, c->w + j * c->k, c->k);
    c->y[r * c->n + j] = c->bias != NULL ? sum + c->bias[j] : sum;
  }
}

/* Rows over orc_threads() threads, as the reference's parallel_for over m. */
ORC_API void orc_linear(const float* x, int64_t m, int64_t k, const float* w, int64_t n, const float* bias, float* y) {
  linear_ctx c = {x, w, bias, y, k, n};
  parallel_for(m, linear_row, &c);
}

/* softmax_rows (ops.cpp:169-187): fp32 max, v = exp(v - peak) in fp32,
 * total in fp64, inv = float(1 / total), v *= inv; a row whose max is -inf
 * (fully masked) becomes zeros. */
ORC_API void orc_softmax_rows(float* x, int64_t rows, int64_t cols) {
  for (int64_t r = 0; r < rows; ++r) {
    float* v = x + r * cols;
    float peak = -INFINITY;
    for (int64_t i = 0; i < cols; ++i) peak = v[i] > peak ? v[i] : peak;
    if (peak == -INFINITY) {
      for (int64_t i = 0; i < cols; ++i) v[i] = 0.0f;
      continue;
    }
    double total = 0.0;
    for (int64_t i = 0; i < cols; ++i) {
      v[i] = expf(v[i] - peak);
      total += v[i];
    }
    const float inv = (float)(1.0 / total);
    for (int64_t i = 0; i < cols; ++i) v[i] *= inv;
  }
}

/* MixtureOfExperts::forward's routing (src/model/feed_forward.cpp:36-53):
 * the gate logits go through softmax_rows, then per row the k experts of
 * highest score, ordered by (score descending, index ascending) as the
 * partial_sort comparator orders them, with the scores as weights
 * (unnormalised). ids and weights [rows, k]. */
ORC_API void orc_expert_topk(const float* logits, int64_t rows, int64_t experts, int64_t k, int64_t* ids,
                             float* weights) {
  float* s = (float*)malloc((size_t)experts * sizeof(float));
  unsigned char* used = (unsigned char*)malloc((size_t)experts);
  for (int64_t r = 0; r < rows; ++r) {
    memcpy(s, logits + r * experts, (size_t)experts * sizeof(float));
    orc_softmax_rows(s, 1, experts);
    memset(used, 0, (size_t)experts);
    for (int64_t j = 0; j < k; ++j) {
      int64_t best = -1;
      for (int64_t e = 0; e < experts; ++e) {
        if (!used[e] && (best < 0 || s[e] > s[best])) best = e;  /* ties keep the lower index */
      }
      used[best] = 1;
      ids[r * k + j] = best;
      weights[r * k + j] = s[best];
    }
  }
  free(used);
  free(s);
}

/* attention_head (ops.cpp:219-251) for one query row per head: for head h,
 * s_j = dot(q_h, k_j,h) * scale (+ bias[j]), softmax as above but with the
 * probabilities p_j = exp(s_j - peak) * inv applied to v, out_h = sum p_j v_j,h;
 * all keys masked gives zeros. q [heads * hd]; k, v [keys, width] with head
 * h at column h * hd; bias [keys] shared by the heads (the decode-step mask);
 * out [heads * hd]. */
ORC_API void orc_attention_one(const float* q, const float* k, const float* v, int64_t keys, int64_t width,
                               int64_t heads, int64_t hd, const float* bias, float scale, float* out) {
  float* scores = (float*)malloc((size_t)(keys > 0 ? keys : 1) * sizeof(float));
  float* kh = (float*)malloc((size_t)(hd > 0 ? hd : 1) * sizeof(float));
  for (int64_t h = 0; h < heads; ++h) {
    float* o = out + h * hd;
    for (int64_t e = 0; e < hd; ++e) o[e] = 0.0f;
    float peak = -INFINITY;
    for (int64_t j = 0; j < keys; ++j) {
      for (int64_t e = 0; e < hd; ++e) kh[e] = k[j * width + h * hd + e];
      float s = ref_dot(q + h * hd, kh, hd) * scale;
      if (bias != NULL) s += bias[j];
      scores[j] = s;
      peak = s > peak ? s : peak;
    }
    if (peak == -INFINITY) continue;
    double total = 0.0;
    for (int64_t j = 0; j < keys; ++j) {
      scores[j] = expf(scores[j] - peak);
      total += scores[j];
    }
    const float inv = (float)(1.0 / total);
    for (int64_t j = 0; j < keys; ++j) {
      const float p = scores[j] * inv;
      for (int64_t e = 0; e < hd; ++e) o[e] += p * v[j * width + h * hd + e];
    }
  }
  free(kh);
  free(scores);
}

/* scale_add_mask (src/backend/cuda/ops.cu:129-132,348-352): for each of
 * `batch` slices of [rows, cols], x = x * scale + mask[r, c] (mask NULL: + 0). */
ORC_API void orc_scale_add_mask(float* x, float scale, const float* mask, int64_t batch, int64_t rows, int64_t cols) {
  const int64_t per = rows * cols;
  for (int64_t b = 0; b < batch; ++b) {
    for (int64_t i = 0; i < per; ++i) x[b * per + i] = x[b * per + i] * scale + (mask != NULL ? mask[i] : 0.0f);
  }
}

/* quick_gelu (ops.cpp:157-161): v * sigmoid(1.702 v). */
ORC_API void orc_quick_gelu(float* x, int64_t n) {
  for (int64_t i = 0; i < n; ++i) x[i] = x[i] * sigmoid(1.702f * x[i]);
}

/* ---- the block router of sparse decode attention ------------------------- */

static inline float clamp_act(float v) { return v < -1.0e4f ? -1.0e4f : (v > 1.0e4f ? 1.0e4f : v); }

/* Block summaries (src/model/block_router.cpp:20-47): for each block of
 * `block_size` router keys rk [keys, d], logits a_t = clamp(dot(rk_t, cls)
 * / sqrt(d)) with the dot summed over e in order, w_t = exp(a_t - max),
 * total = max(sum w_t, 1e-6), out[b] = sum_t (w_t / total) rk_t (summed over
 * t in order, starting from 0). */
ORC_API void orc_block_summaries(const float* rk, int64_t keys, int64_t d, const float* cls, int64_t block_size,
                                 float* out) {
  const int64_t nblk = (keys + block_size - 1) / block_size;
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  float* w = (float*)malloc((size_t)(block_size > 0 ? block_size : 1) * sizeof(float));
  for (int64_t b = 0; b < nblk; ++b) {
    const int64_t first = b * block_size, last = first + block_size < keys ? first + block_size : keys;
    float peak = -3.402823466e+38f;
    for (int64_t t = first; t < last; ++t) {
      float a = 0.0f;
      for (int64_t e = 0; e < d; ++e) a += rk[t * d + e] * cls[e];
      a = clamp_act(a * inv_sqrt_d);
      w[t - first] = a;
      if (a > peak) peak = a;
    }
    float total = 0.0f;
    for (int64_t t = first; t < last; ++t) {
      w[t - first] = expf(w[t - first] - peak);
      total += w[t - first];
    }
    if (total < 1e-6f) total = 1e-6f;
    float* o = out + b * d;
    for (int64_t e = 0; e < d; ++e) o[e] = 0.0f;
    for (int64_t t = first; t < last; ++t) {
      const float p = w[t - first] / total;
      for (int64_t e = 0; e < d; ++e) o[e] += p * rk[t * d + e];
    }
  }
  free(w);
}

/* Block scores (block_router.cpp:49-66): for query i at position q_pos[i],
 * blocks b <= q_pos / block_size - local_blocks score clamp(dot(rq_i, S_b)
 * / sqrt(d)); the rest score -1e9 (kScoreMasked). */
ORC_API void orc_block_scores(const float* rq, int64_t lq, const float* summaries, int64_t nblk, int64_t d,
                              const int64_t* q_pos, int64_t block_size, int64_t local_blocks, float* out) {
  const float inv_sqrt_d = 1.0f / sqrtf((float)d);
  for (int64_t i = 0; i < lq; ++i) {
    const int64_t last_remote = q_pos[i] / block_size - local_blocks;
    for (int64_t b = 0; b < nblk; ++b) {
      if (b > last_remote) {
        out[i * nblk + b] = -1.0e9f;
        continue;
      }
      float z = 0.0f;
      for (int64_t e = 0; e < d; ++e) z += rq[i * d + e] * summaries[b * d + e];
      out[i * nblk + b] = clamp_act(z * inv_sqrt_d);
    }
  }
}

static int desc_float(const void* a, const void* b) {
  const float x = *(const float*)a, y = *(const float*)b;
  return x < y ? 1 : (x > y ? -1 : 0);
}

/* 1.5-entmax of one row in place (block_router.cpp:68-91): halve the
 * shifted row, sort descending, running mean and mean square give the
 * threshold candidates tau_k = mean - sqrt(max((1 - rho (msq - mean^2)) /
 * rho, 0)), the support is the count of tau_k <= sorted_k, and the output
 * is max(x - tau*, 0)^2, all in fp32. */
ORC_API void orc_entmax15(float* x, int64_t n) {
  if (n <= 0) return;
  float peak = x[0];
  for (int64_t i = 1; i < n; ++i) if (x[i] > peak) peak = x[i];
  for (int64_t i = 0; i < n; ++i) x[i] = (x[i] - peak) / 2.0f;
  float* sorted = (float*)malloc((size_t)n * sizeof(float));
  float* tau = (float*)malloc((size_t)n * sizeof(float));
  memcpy(sorted, x, (size_t)n * sizeof(float));
  qsort(sorted, (size_t)n, sizeof(float), desc_float);
  float sum = 0.0f, sum_sq = 0.0f;
  int64_t support = 0;
  for (int64_t k = 0; k < n; ++k) {
    sum += sorted[k];
    sum_sq += sorted[k] * sorted[k];
    const float rho = (float)(k + 1);
    const float mean = sum / rho, mean_sq = sum_sq / rho;
    const float ss = rho * (mean_sq - mean * mean);
    float delta = (1.0f - ss) / rho;
    if (delta < 0.0f) delta = 0.0f;
    tau[k] = mean - sqrtf(delta);
    if (tau[k] <= sorted[k]) ++support;
  }
  const float tau_star = tau[(support > 1 ? support : 1) - 1];
  for (int64_t i = 0; i < n; ++i) {
    float t = x[i] - tau_star;
    if (t < 0.0f) t = 0.0f;
    x[i] = t * t;
  }
  free(sorted);
  free(tau);
}

/* Block selection (block_router.cpp:93-154) for each row of scores [lq,
 * nblk]: a block is a candidate when it is remote (score > -5e8) and allowed
 * (candidate NULL, or candidate[i, b] != 0); a row with no candidate falls
 * back to every remote block. Candidates keep score * idx_scale, the rest
 * -1e4; the top m = clamp(top_m, 1, nblk) in descending order (ties: the
 * lower block first) go through 1.5-entmax; the first k = clamp(top_k, 1,
 * m) are the selection: block, valid (= candidate), logp = log(max(p,
 * floor)), and bias (logp - mean logp of the valid ones) / sigma for valid
 * slots, 0 otherwise. block, bias and valid are [lq, k]; returns k. */
ORC_API int64_t orc_select_blocks(const float* scores, int64_t lq, int64_t nblk, const uint8_t* candidate,
                                  int64_t top_m, int64_t top_k, float idx_scale, float floor_p, float sigma,
                                  int64_t* block, float* bias, uint8_t* valid) {
  const int64_t m = top_m < nblk ? (top_m > 1 ? top_m : 1) : (nblk > 1 ? nblk : 1);
  const int64_t k = top_k < m ? (top_k > 1 ? top_k : 1) : m;
  uint8_t* cand = (uint8_t*)malloc((size_t)(nblk > 0 ? nblk : 1));
  float* x = (float*)malloc((size_t)(nblk > 0 ? nblk : 1) * sizeof(float));
  int64_t* order = (int64_t*)malloc((size_t)(nblk > 0 ? nblk : 1) * sizeof(int64_t));
  float* top = (float*)malloc((size_t)m * sizeof(float));
  float* logp = (float*)malloc((size_t)k * sizeof(float));
  for (int64_t i = 0; i < lq; ++i) {
    const float* row = scores + i * nblk;
    int any = 0;
    for (int64_t b = 0; b < nblk; ++b) {
      const int remote = row[b] > -1.0e9f * 0.5f;
      const int allowed = candidate == NULL || candidate[i * nblk + b] != 0;
      cand[b] = (uint8_t)(remote && allowed);
      any |= remote && allowed;
    }
    if (!any) {
      for (int64_t b = 0; b < nblk; ++b) cand[b] = (uint8_t)(row[b] > -1.0e9f * 0.5f);
    }
    for (int64_t b = 0; b < nblk; ++b) x[b] = cand[b] ? row[b] * idx_scale : -1.0e4f;
    /* order by x descending, ties by the lower index: a stable insertion */
    for (int64_t b = 0; b < nblk; ++b) {
      int64_t j = b;
      while (j > 0 && x[order[j - 1]] < x[b]) {
        order[j] = order[j - 1];
        --j;
      }
      order[j] = b;
    }
    for (int64_t j = 0; j < m; ++j) top[j] = x[order[j]];
    orc_entmax15(top, m);
    int64_t count = 0;
    float logp_sum = 0.0f;
    for (int64_t j = 0; j < k; ++j) {
      const int64_t b = order[j];
      block[i * k + j] = b;
      valid[i * k + j] = cand[b];
      logp[j] = logf(top[j] > floor_p ? top[j] : floor_p);
      if (cand[b]) {
        logp_sum += logp[j];
        ++count;
      }
    }
    const float mu = logp_sum / (float)(count > 1 ? count : 1);
    for (int64_t j = 0; j < k; ++j) bias[i * k + j] = valid[i * k + j] ? (logp[j] - mu) / sigma : 0.0f;
  }
  free(cand);
  free(x);
  free(order);
  free(top);
  free(logp);
  return k;
}

/* The additive key mask of a selection (src/model/attention_plan.cpp:34-56)
 * for queries at first_pos.. over keys 0..keys-1: 0 inside the local window
 * (j > pos - local_blocks * block_size), the block's bias for a key of a
 * valid selected block, -inf elsewhere and past pos. mask [rows, keys]. */
ORC_API void orc_key_mask(const int64_t* block, const float* bias, const uint8_t* valid, int64_t width, int64_t rows,
                          int64_t first_pos, int64_t keys, int64_t block_size, int64_t local_blocks, float* mask) {
  const int64_t nblk = (keys + block_size - 1) / block_size;
  const int64_t window = local_blocks * block_size;
  float* block_bias = (float*)malloc((size_t)(nblk > 0 ? nblk : 1) * sizeof(float));
  for (int64_t i = 0; i < rows; ++i) {
    for (int64_t b = 0; b < nblk; ++b) block_bias[b] = -INFINITY;
    for (int64_t j = 0; j < width; ++j) {
      if (valid[i * width + j]) block_bias[block[i * width + j]] = bias[i * width + j];
    }
    const int64_t pos = first_pos + i;
    float* row = mask + i * keys;
    for (int64_t j = 0; j < keys; ++j) row[j] = -INFINITY;
    for (int64_t j = 0; j <= pos && j < keys; ++j) row[j] = j > pos - window ? 0.0f : block_bias[j / block_size];
  }
  free(block_bias);
}

/* A query's candidate blocks from the prompt's per-block image pages
 * (src/model/decoder.cpp:42-56): block b of the first min(nblk, known)
 * blocks is a candidate when min_page[b] >= 0 and min_page[b] <= page <=
 * max_page[b]. Writes out [nblk] and returns 1; returns 0 (no restriction,
 * out untouched) when page < 0 or no block qualifies. */
ORC_API int orc_page_candidates(const int64_t* min_page, const int64_t* max_page, int64_t known, int64_t page,
                                int64_t nblk, uint8_t* out) {
  if (page < 0) return 0;
  int any = 0;
  for (int64_t b = 0; b < nblk; ++b) out[b] = 0;
  const int64_t n = nblk < known ? nblk : known;
  for (int64_t b = 0; b < n; ++b) {
    if (min_page[b] >= 0 && min_page[b] <= page && page <= max_page[b]) {
      out[b] = 1;
      any = 1;
    }
  }
  return any;
}

/* The routed key mask of one decode query (Decoder::attention for one row,
 * src/model/decoder.cpp:104-120, through the functions above): summaries of
 * the router keys rk [pos + 1, d], scores of rq [d] at position pos, the
 * page candidates of query_page, the selection and its key mask [pos + 1].
 * summaries [ceil((pos + 1) / block_size), d] receives the summaries. */
ORC_API void orc_route_one(const float* rq, const float* rk, int64_t pos, int64_t d, const float* cls,
                           const int64_t* min_page, const int64_t* max_page, int64_t known, int64_t query_page,
                           int64_t block_size, int64_t local_blocks, int64_t top_m, int64_t top_k, float idx_scale,
                           float floor_p, float sigma, float* summaries, float* mask) {
  const int64_t keys = pos + 1, nblk = (keys + block_size - 1) / block_size;
  orc_block_summaries(rk, keys, d, cls, block_size, summaries);
  float* z = (float*)malloc((size_t)nblk * sizeof(float));
  orc_block_scores(rq, 1, summaries, nblk, d, &pos, block_size, local_blocks, z);
  uint8_t* cand = (uint8_t*)malloc((size_t)nblk);
  const int restricted = orc_page_candidates(min_page, max_page, known, query_page, nblk, cand);
  int64_t* block = (int64_t*)malloc((size_t)(top_k > 0 ? top_k : 1) * sizeof(int64_t) + 64);
  float* bias = (float*)malloc((size_t)(top_k > 0 ? top_k : 1) * sizeof(float) + 64);
  uint8_t* valid = (uint8_t*)malloc((size_t)(top_k > 0 ? top_k : 1) + 64);
  const int64_t width =
      orc_select_blocks(z, 1, nblk, restricted ? cand : NULL, top_m, top_k, idx_scale, floor_p, sigma, block, bias, valid);
  orc_key_mask(block, bias, valid, width, 1, pos, keys, block_size, local_blocks, mask);
  free(z);
  free(cand);
  free(block);
  free(bias);
  free(valid);
}
