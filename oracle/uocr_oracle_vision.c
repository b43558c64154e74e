/*
 * uocr_oracle_vision.c: CPU restatement of the reference's vision encoder
 * (SAM ViT with its neck and stride-2 convolutions, the CLIP transformer
 * over SAM's features, the projector and the page token layout) and of the
 * reference ops it is built from.
 *
 * TEST INFRASTRUCTURE ONLY. This file is part of the checker: the parity
 * tests load it to compute expected values. No product path may load or
 * call it.
 *
 * Each function restates the reference's arithmetic in the reference's
 * order, citing the file:line it follows. Built with -O3 and
 * -ffp-contract=off like the rest of the oracle.
 *
 * How each function is pinned (tests/test_oracle_vision.py):
 *   im2col, conv2d, chw_to_hwc, hwc_to_chw, layer_norm_channels,
 *   attention_head, resize_bicubic_aa, resize_linear_rows: bit-equality with
 *     the reference's own ops.cpp compiled into oracle/_ref, plus closed
 *     forms (a 1x1 convolution is a linear; the transposes invert each
 *     other; bicubic resize to the same size is the identity and keeps a
 *     constant image constant; linear resize hits the end rows).
 *   relative_positions (sam_encoder.cpp, not buildable here: <format>):
 *     entry [q][k] equals table row q - k + size - 1 when no resize is
 *     needed, and equals the resized table's row otherwise.
 *   rel_pos_bias: an fp64 brute force of q . rh[qy, ky] + q . rw[qx, kx].
 *   The encoder (sam_forward, clip_forward, encode_view, encode_page): the
 *     reference's own layout checks (tests/vision_test.cpp: token counts,
 *     a newline closing every grid row, the separator last), residual
 *     identities (zero sublayer weights leave the stream unchanged), and
 *     each part above.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#include "uocr_oracle.h"

#define ORC_API __attribute__((visibility("default")))

static void* xalloc(size_t n) { return calloc(n > 0 ? n : 1, 1); }
#define FLOATS(n) ((float*)xalloc((size_t)(n) * sizeof(float)))

/* dot (src/backend/reference/ops.cpp:23-38): eight fp32 partial sums in a
 * fixed order, then ((a0+a1)+(a2+a3))+((a4+a5)+(a6+a7)) + tail. */
static float vdot(const float* a, const float* b, int64_t n) {
  float acc[8] = {0, 0, 0, 0, 0, 0, 0, 0};
  int64_t i = 0;
  for (; i + 8 <= n; i += 8) {
    for (int lane = 0; lane < 8; ++lane) acc[lane] += a[i + lane] * b[i + lane];
  }
  float tail = 0.0f;
  for (; i < n; ++i) tail += a[i] * b[i];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7])) + tail;
}

/* linear with the device path's input rounding when round_x is set: the
 * reference's cuda::linear rounds x to bf16 before its products
 * (src/backend/cuda/ops.h:14-17); reference::linear (ops.cpp:91-109) does not. */
static void lin(const float* x, int64_t m, int64_t k, const float* w, int64_t n, const float* bias, float* y,
                int round_x) {
  if (!round_x) {
    orc_linear(x, m, k, w, n, bias, y);
    return;
  }
  float* xr = FLOATS(m * k);
  for (int64_t i = 0; i < m * k; ++i) xr[i] = orc_bf16_to_f32(orc_f32_to_bf16(x[i]));
  orc_linear(xr, m, k, w, n, bias, y);
  free(xr);
}

/* ---- layout ops (src/backend/reference/ops.cpp:298-312) ------------------ */

/* chw_to_hwc: x [c, h, w] -> y [h, w, c]. */
ORC_API void orc_chw_to_hwc(const float* x, int64_t c, int64_t h, int64_t w, float* y) {
  for (int64_t ch = 0; ch < c; ++ch)
    for (int64_t p = 0; p < h * w; ++p) y[p * c + ch] = x[ch * h * w + p];
}

/* hwc_to_chw: x [h, w, c] -> y [c, h, w]. */
ORC_API void orc_hwc_to_chw(const float* x, int64_t h, int64_t w, int64_t c, float* y) {
  for (int64_t p = 0; p < h * w; ++p)
    for (int64_t ch = 0; ch < c; ++ch) y[ch * h * w + p] = x[p * c + ch];
}

/* concat_cols (src/backend/cuda/ops.h:65-67): out[r] = a[r] (ca values)
 * followed by b[r] (cb values). */
ORC_API void orc_concat_cols(const float* a, int64_t ca, const float* b, int64_t cb, int64_t rows, float* out) {
  for (int64_t r = 0; r < rows; ++r) {
    memcpy(out + r * (ca + cb), a + r * ca, (size_t)ca * sizeof(float));
    memcpy(out + r * (ca + cb) + ca, b + r * cb, (size_t)cb * sizeof(float));
  }
}

/* ---- convolution (ops.cpp:189-217) --------------------------------------- */

/* im2col of conv2d (ops.cpp:198-212): one row per output position
 * (oy, ox), its columns in the weight's [c, kh, kw] order, zero outside
 * the image. x [c, h, w] -> cols [oh * ow, c * kh * kw]. */
ORC_API void orc_im2col(const float* x, int64_t c, int64_t h, int64_t w, int64_t kh, int64_t kw, int64_t stride,
                        int64_t pad, float* cols) {
  const int64_t oh = (h + 2 * pad - kh) / stride + 1, ow = (w + 2 * pad - kw) / stride + 1;
  for (int64_t oy = 0; oy < oh; ++oy) {
    for (int64_t ox = 0; ox < ow; ++ox) {
      float* col = cols + (oy * ow + ox) * c * kh * kw;
      for (int64_t ci = 0; ci < c; ++ci) {
        for (int64_t ky = 0; ky < kh; ++ky) {
          const int64_t iy = oy * stride - pad + ky;
          for (int64_t kx = 0; kx < kw; ++kx) {
            const int64_t ix = ox * stride - pad + kx;
            const int inside = iy >= 0 && iy < h && ix >= 0 && ix < w;
            *col++ = inside ? x[(ci * h + iy) * w + ix] : 0.0f;
          }
        }
      }
    }
  }
}

/* conv2d (ops.cpp:189-217): im2col, linear against the weight flattened to
 * [o, c * kh * kw] (+ bias), then the [oh, ow, o] result back to
 * [o, oh, ow]. round_x rounds the patches to bf16 as the device linear does. */
static void conv2d_x(const float* x, int64_t c, int64_t h, int64_t w, const float* weight, const float* bias,
                     int64_t o, int64_t kh, int64_t kw, int64_t stride, int64_t pad, float* out, int round_x) {
  const int64_t oh = (h + 2 * pad - kh) / stride + 1, ow = (w + 2 * pad - kw) / stride + 1;
  const int64_t patch = c * kh * kw;
  float* cols = FLOATS(oh * ow * patch);
  float* hwc = FLOATS(oh * ow * o);
  orc_im2col(x, c, h, w, kh, kw, stride, pad, cols);
  lin(cols, oh * ow, patch, weight, o, bias, hwc, round_x);
  orc_hwc_to_chw(hwc, oh, ow, o, out);
  free(hwc);
  free(cols);
}

ORC_API void orc_conv2d(const float* x, int64_t c, int64_t h, int64_t w, const float* weight, const float* bias,
                        int64_t o, int64_t kh, int64_t kw, int64_t stride, int64_t pad, float* out) {
  conv2d_x(x, c, h, w, weight, bias, o, kh, kw, stride, pad, out, 0);
}

/* layer_norm_channels (ops.cpp:143-149): x [c, h, w] normalised over c at
 * every position (to HWC, layer_norm over rows, back to CHW). */
ORC_API void orc_layer_norm_channels(float* x, const float* w, const float* b, int64_t c, int64_t h, int64_t wd,
                                     float eps) {
  float* hwc = FLOATS(c * h * wd);
  orc_chw_to_hwc(x, c, h, wd, hwc);
  orc_layer_norm(hwc, w, b, h * wd, c, eps);
  orc_hwc_to_chw(hwc, h, wd, c, x);
  free(hwc);
}

/* ---- attention (ops.cpp:219-251) ------------------------------------------ */

/* attention_head: q [lq, d], k [lk, d], v [lk, dv], bias [lq, lk] or NULL;
 * s_j = dot(q_i, k_j) * scale (+ bias[i][j]); peak; e_j = exp(s_j - peak)
 * in fp32 with the total in fp64; inv = float(1 / total); out_i += (e_j *
 * inv) v_j in key order. A row whose every score is -inf stays zero. */
typedef struct {
  const float *q, *k, *v, *bias;
  float* out;
  int64_t lk, d, dv;
  float scale;
} attn_ctx;

static void attention_row(void* p, int64_t i) {
  const attn_ctx* c = (const attn_ctx*)p;
  const int64_t lk = c->lk, d = c->d, dv = c->dv;
  float* o = c->out + i * dv;
  for (int64_t e = 0; e < dv; ++e) o[e] = 0.0f;
  float* s = FLOATS(lk);
  float peak = -INFINITY;
  for (int64_t j = 0; j < lk; ++j) {
    float sj = vdot(c->q + i * d, c->k + j * d, d) * c->scale;
    if (c->bias != NULL) sj += c->bias[i * lk + j];
    s[j] = sj;
    peak = sj > peak ? sj : peak;
  }
  if (peak != -INFINITY) {
    double total = 0.0;
    for (int64_t j = 0; j < lk; ++j) {
      s[j] = expf(s[j] - peak);
      total += s[j];
    }
    const float inv = (float)(1.0 / total);
    for (int64_t j = 0; j < lk; ++j) {
      const float pj = s[j] * inv;
      for (int64_t e = 0; e < dv; ++e) o[e] += pj * c->v[j * dv + e];
    }
  }
  free(s);
}

/* Query rows over orc_threads() threads, as the reference's parallel_for
 * over lq (ops.cpp:225). */
ORC_API void orc_attention_head(const float* q, const float* k, const float* v, int64_t lq, int64_t lk, int64_t d,
                                int64_t dv, const float* bias, float scale, float* out) {
  attn_ctx c = {q, k, v, bias, out, lk, d, dv, scale};
  orc_parallel_rows(lq, attention_row, &c);
}

/* ---- resizes (ops.cpp:42-86, 253-296) ------------------------------------- */

/* The antialiasing cubic with a = -0.5 (ops.cpp:43-54). */
static float cubic_aa(float x) {
  const float a = -0.5f;
  x = fabsf(x);
  if (x < 1.0f) return ((a + 2.0f) * x - (a + 3.0f)) * x * x + 1.0f;
  if (x < 2.0f) return ((a * x - 5.0f * a) * x + 8.0f * a) * x - 4.0f * a;
  return 0.0f;
}

/* The taps of one output index (ops.cpp:60-86): centre scale * (i + 0.5),
 * support 2 * scale when shrinking (2 otherwise), taps over [lo, hi) with
 * weights cubic((j - centre + 0.5) * invscale), normalised by their fp32 sum
 * when it is nonzero. Tap list i holds its weights at w + i * in. */
typedef struct {
  int64_t first, count;
} taps_t;

static void aa_taps(int64_t in, int64_t out, taps_t* taps, float* w) {
  const float scale = (float)in / (float)out;
  const float support = scale >= 1.0f ? 2.0f * scale : 2.0f;
  const float invscale = scale >= 1.0f ? 1.0f / scale : 1.0f;
  for (int64_t i = 0; i < out; ++i) {
    const float center = scale * ((float)i + 0.5f);
    int64_t lo = (int64_t)(center - support + 0.5f);
    if (lo < 0) lo = 0;
    int64_t hi = (int64_t)(center + support + 0.5f);
    if (hi > in) hi = in;
    taps_t* t = &taps[i];
    float* tw = w + i * in;
    t->first = lo;
    t->count = 0;
    float total = 0.0f;
    for (int64_t j = lo; j < hi; ++j) {
      const float wv = cubic_aa(((float)j - center + 0.5f) * invscale);
      tw[t->count++] = wv;
      total += wv;
    }
    if (total != 0.0f) {
      for (int64_t q = 0; q < t->count; ++q) tw[q] /= total;
    }
  }
}

/* resize_bicubic_aa (ops.cpp:253-278): x [c, h, w] -> out [c, oh, ow]; per
 * output pixel, for each row tap the fp32 sum of the column taps, then the
 * fp32 sum of those weighted by the row taps. */
ORC_API void orc_resize_bicubic_aa(const float* x, int64_t c, int64_t h, int64_t w, int64_t oh, int64_t ow,
                                   float* out) {
  taps_t* rows = (taps_t*)xalloc((size_t)oh * sizeof(taps_t));
  taps_t* cols = (taps_t*)xalloc((size_t)ow * sizeof(taps_t));
  float* rw = FLOATS(oh * h);
  float* cw = FLOATS(ow * w);
  aa_taps(h, oh, rows, rw);
  aa_taps(w, ow, cols, cw);
  for (int64_t ch = 0; ch < c; ++ch) {
    const float* src = x + ch * h * w;
    float* dst = out + ch * oh * ow;
    for (int64_t oy = 0; oy < oh; ++oy) {
      const taps_t* ry = &rows[oy];
      const float* wy = rw + oy * h;
      for (int64_t ox = 0; ox < ow; ++ox) {
        const taps_t* rx = &cols[ox];
        const float* wx = cw + ox * w;
        float acc = 0.0f;
        for (int64_t a = 0; a < ry->count; ++a) {
          const float* line = src + (ry->first + a) * w + rx->first;
          float line_acc = 0.0f;
          for (int64_t b = 0; b < rx->count; ++b) line_acc += line[b] * wx[b];
          acc += line_acc * wy[a];
        }
        dst[oy * ow + ox] = acc;
      }
    }
  }
  free(cw);
  free(rw);
  free(cols);
  free(rows);
}

/* resize_linear_rows (ops.cpp:280-296): x [len, c] -> out [out_len, c];
 * row i samples src = max(scale * (i + 0.5) - 0.5, 0) with scale = len /
 * out_len: rows i0 = int(src) and i0 + 1 (i0 at the last row), weights
 * 1 - (src - i0) and src - i0, v = l0 * a + l1 * b in fp32. */
ORC_API void orc_resize_linear_rows(const float* x, int64_t len, int64_t c, int64_t out_len, float* out) {
  const float scale = (float)len / (float)out_len;
  for (int64_t i = 0; i < out_len; ++i) {
    float src = scale * ((float)i + 0.5f) - 0.5f;
    if (src < 0.0f) src = 0.0f;
    const int64_t i0 = (int64_t)src;
    const int64_t i1 = i0 + (i0 < len - 1 ? 1 : 0);
    const float l1 = src - (float)i0;
    const float l0 = 1.0f - l1;
    for (int64_t e = 0; e < c; ++e) out[i * c + e] = l0 * x[i0 * c + e] + l1 * x[i1 * c + e];
  }
}

/* relative_positions (src/model/sam_encoder.cpp:52-63): the table resized
 * linearly to 2 * size - 1 rows when its length differs, then out[q][k] =
 * row q - k + size - 1: out [size, size, d]. */
ORC_API void orc_relative_positions(const float* table, int64_t len, int64_t d, int64_t size, float* out) {
  const int64_t span = 2 * size - 1;
  float* resized = NULL;
  const float* t = table;
  if (len != span) {
    resized = FLOATS(span * d);
    orc_resize_linear_rows(table, len, d, span, resized);
    t = resized;
  }
  for (int64_t q = 0; q < size; ++q)
    for (int64_t k = 0; k < size; ++k) memcpy(out + (q * size + k) * d, t + (q - k + size - 1) * d, (size_t)d * 4);
  free(resized);
}

/* SAM's decomposed relative-position bias for one head of one window
 * (sam_encoder.cpp:163-183): for query t = qy * w + qx, by[ky] = sum_e
 * q_t[e] rh[qy, ky, e] and bx[kx] = sum_e q_t[e] rw[qx, kx, e] (fp32, in e
 * order), bias[t][ky * w + kx] = by[ky] + bx[kx]. q rows ldq apart. */
ORC_API void orc_rel_pos_bias(const float* q, int64_t ldq, int64_t h, int64_t w, int64_t d, const float* rh,
                              const float* rw, float* bias) {
  const int64_t n = h * w;
  float* by = FLOATS(h);
  float* bx = FLOATS(w);
  for (int64_t t = 0; t < n; ++t) {
    const int64_t qy = t / w, qx = t % w;
    const float* qt = q + t * ldq;
    for (int64_t ky = 0; ky < h; ++ky) {
      const float* r = rh + (qy * h + ky) * d;
      float s = 0.0f;
      for (int64_t e = 0; e < d; ++e) s += qt[e] * r[e];
      by[ky] = s;
    }
    for (int64_t kx = 0; kx < w; ++kx) {
      const float* r = rw + (qx * w + kx) * d;
      float s = 0.0f;
      for (int64_t e = 0; e < d; ++e) s += qt[e] * r[e];
      bx[kx] = s;
    }
    for (int64_t ky = 0; ky < h; ++ky)
      for (int64_t kx = 0; kx < w; ++kx) bias[t * n + ky * w + kx] = by[ky] + bx[kx];
  }
  free(bx);
  free(by);
}

/* ---- SAM (src/model/sam_encoder.cpp) -------------------------------------- */

/* Multi-head attention over one window of h x w tokens (sam_encoder.cpp:
 * 150-197): qkv = x Wqkv + b as [n, (3, heads, hd)], per head the
 * relative-position bias from the unscaled query and attention_head with
 * scale 1 / sqrt(hd), the heads' outputs side by side, then the projection. */
static void sam_attention(const orc_sam_block* b, const orc_sam_dims* dm, const float* x, int64_t h, int64_t w,
                          float* out, int round_x) {
  const int64_t n = h * w, c = dm->width, heads = dm->heads, hd = c / heads;
  float* qkv = FLOATS(n * 3 * c);
  lin(x, n, c, b->qkv_w, 3 * c, b->qkv_b, qkv, round_x);
  float* rh = FLOATS(h * h * hd);
  float* rw = FLOATS(w * w * hd);
  orc_relative_positions(b->rel_h, b->rel_len, hd, h, rh);
  orc_relative_positions(b->rel_w, b->rel_len, hd, w, rw);
  const float scale = 1.0f / sqrtf((float)hd);
  float* q = FLOATS(n * hd);
  float* k = FLOATS(n * hd);
  float* v = FLOATS(n * hd);
  float* bias = FLOATS(n * n);
  float* o = FLOATS(n * hd);
  float* merged = FLOATS(n * c);
  for (int64_t head = 0; head < heads; ++head) {
    for (int64_t t = 0; t < n; ++t) {
      memcpy(q + t * hd, qkv + t * 3 * c + head * hd, (size_t)hd * 4);
      memcpy(k + t * hd, qkv + t * 3 * c + c + head * hd, (size_t)hd * 4);
      memcpy(v + t * hd, qkv + t * 3 * c + 2 * c + head * hd, (size_t)hd * 4);
    }
    orc_rel_pos_bias(q, hd, h, w, hd, rh, rw, bias);
    orc_attention_head(q, k, v, n, n, hd, hd, bias, scale, o);
    for (int64_t t = 0; t < n; ++t) memcpy(merged + t * c + head * hd, o + t * hd, (size_t)hd * 4);
  }
  lin(merged, n, c, b->proj_w, c, b->proj_b, out, round_x);
  free(merged);
  free(o);
  free(bias);
  free(v);
  free(k);
  free(q);
  free(rw);
  free(rh);
  free(qkv);
}

/* One block (sam_encoder.cpp:133-160) over x [g, g, c] in place:
 * x += attn(LN1(x)) (global, or in win x win windows of the zero-padded
 * grid, windows in row order, slots in row order), then
 * x += lin2(gelu(lin1(LN2(x)))). */
static void sam_block(const orc_sam_block* b, const orc_sam_dims* dm, float* x, int64_t g, int round_x) {
  const int64_t c = dm->width, cells = g * g;
  float* normed = FLOATS(cells * c);
  memcpy(normed, x, (size_t)(cells * c) * 4);
  orc_layer_norm(normed, b->norm1_w, b->norm1_b, cells, c, 1e-6f);
  float* attended = FLOATS(cells * c);
  if (b->global) {
    sam_attention(b, dm, normed, g, g, attended, round_x);
  } else {
    const int64_t win = dm->window, nw = (g + win - 1) / win, n = win * win;
    float* windows = FLOATS(nw * nw * n * c); /* zero padding */
    float* out = FLOATS(nw * nw * n * c);
    for (int64_t y = 0; y < g; ++y)
      for (int64_t xx = 0; xx < g; ++xx) {
        const int64_t window = (y / win) * nw + xx / win, slot = (y % win) * win + xx % win;
        memcpy(windows + (window * n + slot) * c, normed + (y * g + xx) * c, (size_t)c * 4);
      }
    for (int64_t i = 0; i < nw * nw; ++i) sam_attention(b, dm, windows + i * n * c, win, win, out + i * n * c, round_x);
    for (int64_t y = 0; y < g; ++y)
      for (int64_t xx = 0; xx < g; ++xx) {
        const int64_t window = (y / win) * nw + xx / win, slot = (y % win) * win + xx % win;
        memcpy(attended + (y * g + xx) * c, out + (window * n + slot) * c, (size_t)c * 4);
      }
    free(out);
    free(windows);
  }
  orc_add_into(x, attended, cells * c);
  memcpy(normed, x, (size_t)(cells * c) * 4);
  orc_layer_norm(normed, b->norm2_w, b->norm2_b, cells, c, 1e-6f);
  float* wide = FLOATS(cells * dm->mlp);
  lin(normed, cells, c, b->lin1_w, dm->mlp, b->lin1_b, wide, round_x);
  orc_gelu_erf(wide, cells * dm->mlp);
  lin(wide, cells, dm->mlp, b->lin2_w, c, b->lin2_b, normed, round_x);
  orc_add_into(x, normed, cells * c);
  free(wide);
  free(attended);
  free(normed);
}

/* SamEncoder::forward (sam_encoder.cpp:104-131): image [3, s, s] ->
 * [net3, g4, g4]. Patch embedding (stride = kernel = patch), the learned
 * positions (bicubic-resized from their grid when it differs), the blocks,
 * the neck (1x1 conv, channel LayerNorm, 3x3 conv, channel LayerNorm) and
 * the two stride-2 3x3 convolutions. Returns g4 (or -1 on a bad shape). */
ORC_API int64_t orc_sam_forward(const orc_sam_weights* wt, const orc_sam_dims* dm, const float* image, int64_t s,
                                float* out, int round_x) {
  const int64_t p = dm->patch, c = dm->width, pg = dm->image / dm->patch;
  if (s % 64 != 0 || s < 64) return -1;
  const int64_t g = s / p;
  float* chw = FLOATS(c * g * g);
  conv2d_x(image, 3, s, s, wt->patch_w, wt->patch_b, c, p, p, p, 0, chw, round_x);
  float* x = FLOATS(g * g * c);
  orc_chw_to_hwc(chw, c, g, g, x);
  float* pos = FLOATS(g * g * c);
  if (pg == g) {
    memcpy(pos, wt->pos_embed, (size_t)(g * g * c) * 4);
  } else {
    float* src = FLOATS(c * pg * pg);
    float* dst = FLOATS(c * g * g);
    orc_hwc_to_chw(wt->pos_embed, pg, pg, c, src);
    orc_resize_bicubic_aa(src, c, pg, pg, g, g, dst);
    orc_chw_to_hwc(dst, c, g, g, pos);
    free(dst);
    free(src);
  }
  orc_add_into(x, pos, g * g * c);
  for (int64_t i = 0; i < dm->layers; ++i) sam_block(&wt->blocks[i], dm, x, g, round_x);

  const int64_t nk = dm->neck;
  float* xc = FLOATS(c * g * g);
  orc_hwc_to_chw(x, g, g, c, xc);
  float* y = FLOATS(nk * g * g);
  conv2d_x(xc, c, g, g, wt->neck0_w, NULL, nk, 1, 1, 1, 0, y, round_x);
  orc_layer_norm_channels(y, wt->neck1_w, wt->neck1_b, nk, g, g, 1e-6f);
  float* z = FLOATS(nk * g * g);
  conv2d_x(y, nk, g, g, wt->neck2_w, NULL, nk, 3, 3, 1, 1, z, round_x);
  orc_layer_norm_channels(z, wt->neck3_w, wt->neck3_b, nk, g, g, 1e-6f);
  const int64_t g2 = (g + 2 - 3) / 2 + 1, g4 = (g2 + 2 - 3) / 2 + 1;
  float* n2 = FLOATS(dm->net2 * g2 * g2);
  conv2d_x(z, nk, g, g, wt->net2_w, NULL, dm->net2, 3, 3, 2, 1, n2, round_x);
  conv2d_x(n2, dm->net2, g2, g2, wt->net3_w, NULL, dm->net3, 3, 3, 2, 1, out, round_x);
  free(n2);
  free(z);
  free(y);
  free(xc);
  free(pos);
  free(x);
  free(chw);
  return g4;
}

/* ---- CLIP (src/model/clip_encoder.cpp) ------------------------------------ */

/* ClipEncoder::forward (clip_encoder.cpp:60-97): features [width, g, g] ->
 * x [1 + g * g, width]: the class embedding then the cells in row order,
 * plus the learned positions (the class position kept, the grid bicubic-
 * resized when it differs), pre-LayerNorm (eps 1e-5), then per layer
 * x += out(attn(LN1(x))) (no bias, scale 1 / sqrt(hd)) and
 * x += fc2(quick_gelu(fc1(LN2(x)))). Returns 0, or -1 on a bad shape. */
ORC_API int orc_clip_forward(const orc_clip_weights* wt, const orc_clip_dims* dm, const float* features, int64_t g,
                             float* x, int round_x) {
  const int64_t c = dm->width, n = 1 + g * g, heads = dm->heads, hd = c / heads;
  const int64_t src = (int64_t)sqrt((double)(dm->positions - 1));
  memcpy(x, wt->class_embedding, (size_t)c * 4);
  orc_chw_to_hwc(features, c, g, g, x + c);
  float* pos = FLOATS(n * c);
  if (src == g) {
    memcpy(pos, wt->positions, (size_t)(n * c) * 4);
  } else {
    float* a = FLOATS(c * src * src);
    float* bb = FLOATS(c * g * g);
    orc_hwc_to_chw(wt->positions + c, src, src, c, a);
    orc_resize_bicubic_aa(a, c, src, src, g, g, bb);
    memcpy(pos, wt->positions, (size_t)c * 4);
    orc_chw_to_hwc(bb, c, g, g, pos + c);
    free(bb);
    free(a);
  }
  orc_add_into(x, pos, n * c);
  orc_layer_norm(x, wt->pre_ln_w, wt->pre_ln_b, n, c, 1e-5f);
  const float scale = 1.0f / sqrtf((float)hd);
  float* normed = FLOATS(n * c);
  float* qkv = FLOATS(n * 3 * c);
  float* q = FLOATS(n * hd);
  float* k = FLOATS(n * hd);
  float* v = FLOATS(n * hd);
  float* o = FLOATS(n * hd);
  float* merged = FLOATS(n * c);
  float* proj = FLOATS(n * c);
  float* wide = FLOATS(n * dm->mlp);
  for (int64_t li = 0; li < dm->layers; ++li) {
    const orc_clip_layer* l = &wt->layers[li];
    memcpy(normed, x, (size_t)(n * c) * 4);
    orc_layer_norm(normed, l->ln1_w, l->ln1_b, n, c, 1e-5f);
    lin(normed, n, c, l->qkv_w, 3 * c, l->qkv_b, qkv, round_x);
    for (int64_t head = 0; head < heads; ++head) {
      for (int64_t t = 0; t < n; ++t) {
        memcpy(q + t * hd, qkv + t * 3 * c + head * hd, (size_t)hd * 4);
        memcpy(k + t * hd, qkv + t * 3 * c + c + head * hd, (size_t)hd * 4);
        memcpy(v + t * hd, qkv + t * 3 * c + 2 * c + head * hd, (size_t)hd * 4);
      }
      orc_attention_head(q, k, v, n, n, hd, hd, NULL, scale, o);
      for (int64_t t = 0; t < n; ++t) memcpy(merged + t * c + head * hd, o + t * hd, (size_t)hd * 4);
    }
    lin(merged, n, c, l->out_w, c, l->out_b, proj, round_x);
    orc_add_into(x, proj, n * c);
    memcpy(normed, x, (size_t)(n * c) * 4);
    orc_layer_norm(normed, l->ln2_w, l->ln2_b, n, c, 1e-5f);
    lin(normed, n, c, l->fc1_w, dm->mlp, l->fc1_b, wide, round_x);
    orc_quick_gelu(wide, n * dm->mlp);
    lin(wide, n, dm->mlp, l->fc2_w, c, l->fc2_b, proj, round_x);
    orc_add_into(x, proj, n * c);
  }
  free(wide);
  free(proj);
  free(merged);
  free(o);
  free(v);
  free(k);
  free(q);
  free(qkv);
  free(normed);
  free(pos);
  return 0;
}

/* ---- the view and the page (src/model/vision_encoder.cpp) ----------------- */

/* VisionEncoder::encode_view (vision_encoder.cpp:32-44): SAM, CLIP over
 * SAM's features, then per cell [clip row t + 1 (the class row dropped) |
 * SAM cell t] through the projector: out [g * g, hidden]. Returns g, or -1. */
ORC_API int64_t orc_encode_view(const orc_vision_weights* wt, const float* image, int64_t s, float* out,
                                int round_x) {
  const orc_sam_dims* sd = &wt->sam_dims;
  const int64_t g0 = s / sd->patch, g2 = (g0 + 2 - 3) / 2 + 1, g = (g2 + 2 - 3) / 2 + 1;
  float* sam = FLOATS(sd->net3 * g * g);
  if (orc_sam_forward(&wt->sam, sd, image, s, sam, round_x) != g) return -1;
  const int64_t cw = wt->clip_dims.width, sw = sd->net3, n = g * g;
  float* clip = FLOATS((1 + n) * cw);
  if (orc_clip_forward(&wt->clip, &wt->clip_dims, sam, g, clip, round_x) != 0) return -1;
  float* cells = FLOATS(n * sw);
  orc_chw_to_hwc(sam, sw, g, g, cells);
  float* joined = FLOATS(n * (cw + sw));
  orc_concat_cols(clip + cw, cw, cells, sw, n, joined);
  lin(joined, n, cw + sw, wt->projector_w, wt->hidden, wt->projector_b, out, round_x);
  free(joined);
  free(cells);
  free(clip);
  free(sam);
  return g;
}

/* The page's image tokens (vision_encoder.cpp:70-77): g (g + 1) + 1 for
 * the global view, plus (tile_g * wide + 1) (tile_g * high) when tiled. */
ORC_API int64_t orc_page_image_tokens(int64_t global_grid, int64_t tile_grid, int64_t tiles_wide, int64_t tiles_high,
                                      int tiled) {
  int64_t tokens = global_grid * (global_grid + 1) + 1;
  if (tiled) tokens += (tile_grid * tiles_wide + 1) * (tile_grid * tiles_high);
  return tokens;
}

/* VisionModel::encode_page (vision_encoder.cpp:46-68): with tiles, the
 * tiles' grids stitched into one (high * g) x (wide * g) grid, each of its
 * rows followed by the newline; then the global view's grid rows, each
 * followed by the newline; then the separator. tiles holds tiles_wide *
 * tiles_high images of tile_size (none when n_tiles is 0). Writes the rows
 * to out (sized by orc_page_image_tokens) and returns their count, or -1. */
ORC_API int64_t orc_encode_page(const orc_vision_weights* wt, const float* global, int64_t global_size,
                                const float* tiles, int64_t n_tiles, int64_t tile_size, int64_t tiles_wide,
                                int64_t tiles_high, float* out, int round_x) {
  const int64_t width = wt->hidden;
  int64_t rows = 0;
  if (n_tiles > 0) {
    if (n_tiles != tiles_wide * tiles_high) return -1;
    const int64_t g0 = tile_size / wt->sam_dims.patch, g2 = (g0 + 2 - 3) / 2 + 1, g = (g2 + 2 - 3) / 2 + 1;
    float* feats = FLOATS(n_tiles * g * g * width);
    for (int64_t i = 0; i < n_tiles; ++i) {
      if (orc_encode_view(wt, tiles + i * 3 * tile_size * tile_size, tile_size, feats + i * g * g * width,
                          round_x) != g)
        return -1;
    }
    const int64_t cols = tiles_wide * g;
    for (int64_t ty = 0; ty < tiles_high; ++ty)
      for (int64_t r = 0; r < g; ++r) {
        for (int64_t tx = 0; tx < tiles_wide; ++tx) {
          const float* tile = feats + (ty * tiles_wide + tx) * g * g * width;
          memcpy(out + rows * width, tile + r * g * width, (size_t)(g * width) * 4);
          rows += g;
        }
        memcpy(out + rows * width, wt->newline, (size_t)width * 4);
        rows += 1;
      }
    (void)cols;
    free(feats);
  }
  const int64_t g0 = global_size / wt->sam_dims.patch, g2 = (g0 + 2 - 3) / 2 + 1, g = (g2 + 2 - 3) / 2 + 1;
  float* view = FLOATS(g * g * width);
  if (orc_encode_view(wt, global, global_size, view, round_x) != g) return -1;
  for (int64_t r = 0; r < g; ++r) {
    memcpy(out + rows * width, view + r * g * width, (size_t)(g * width) * 4);
    rows += g;
    memcpy(out + rows * width, wt->newline, (size_t)width * 4);
    rows += 1;
  }
  memcpy(out + rows * width, wt->separator, (size_t)width * 4);
  rows += 1;
  free(view);
  return rows;
}
