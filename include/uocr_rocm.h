/*
 * uocr_rocm.h: the C ABI of the MI355X (gfx950) `rocm` backend for
 * grpc-unlimited-ocr's fused layer ops.
 *
 * Plain C: raw device pointers, explicit int64 shapes, row-major layouts, an
 * opaque stream handle, and an int status instead of exceptions. The C++23
 * layer in src/backend/rocm/ (namespace uocr::rocm) wraps these calls with the
 * same free-function shapes as the reference's uocr::cuda backend and turns a
 * non-zero status into the reference's exception types.
 *
 * Conventions shared by every entry point:
 *   - `stream` is a hipStream_t (from uocr_rocm_stream_create, or any stream
 *     the caller owns on the current device). Ops are enqueued on it in order;
 *     none synchronises and none allocates, so every op can be recorded into a
 *     graph between uocr_rocm_capture_begin and uocr_rocm_capture_end.
 *   - bf16 is IEEE binary32's top half stored as uint16_t; every conversion
 *     from fp32 rounds to nearest even and keeps NaN quiet (bits>>16 | 0x40),
 *     as the reference's f32_to_bf16 does (src/tensor/dtype.h:39-46).
 *   - fp32 ops compute in fp32. bf16 ops widen to fp32, compute in fp32 and
 *     round once on store. Norm weights (gamma, beta) are fp32 in both cases,
 *     as the reference stores them (src/model/cuda/device_params.h:35-37).
 *   - Shapes are validated before anything is enqueued. A bad shape, a null
 *     pointer with a non-empty shape, a misaligned pointer that the op needs
 *     aligned, or an unsupported size returns UOCR_ROCM_INVALID_ARGUMENT and
 *     enqueues nothing, where the reference throws std::invalid_argument
 *     (src/backend/cuda/decode_ops.cu:239, ops.cu:569,655). Empty shapes
 *     (rows == 0 or n == 0) are valid no-ops.
 *   - uocr_rocm_last_error() returns this thread's message for the last
 *     failing call ("<what>: <detail>"), the shape of the reference's check()
 *     messages (src/backend/cuda/context.cu:24-28).
 */
#ifndef UOCR_ROCM_H_
#define UOCR_ROCM_H_

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#if defined(__GNUC__)
#define UOCR_ROCM_API __attribute__((visibility("default")))
#else
#define UOCR_ROCM_API
#endif

/* ---- status ------------------------------------------------------------ */

enum uocr_rocm_status {
  UOCR_ROCM_OK = 0,
  UOCR_ROCM_INVALID_ARGUMENT = 1, /* reference: std::invalid_argument        */
  UOCR_ROCM_NO_DEVICE = 2,        /* reference: device_count() == 0 (skip 77) */
  UOCR_ROCM_RUNTIME_ERROR = 3,    /* a HIP runtime call failed               */
  UOCR_ROCM_LAUNCH_ERROR = 4      /* hipGetLastError() after a launch failed */
};

/* Static name of a status code. */
UOCR_ROCM_API const char* uocr_rocm_status_string(int status);
/* This thread's message for its last failing call ("" if none). */
UOCR_ROCM_API const char* uocr_rocm_last_error(void);
/* ABI version, bumped when an entry point changes: (major << 16) | minor. */
UOCR_ROCM_API int uocr_rocm_abi_version(void);

/* ---- device, stream, memory, graphs ------------------------------------ */

/* Replaces uocr::cuda::device_count (src/backend/cuda/context.h:22-23,
 * context.cu:36-39): *count = 0 and UOCR_ROCM_OK when no usable device. */
UOCR_ROCM_API int uocr_rocm_device_count(int* count);

/* Replaces uocr::cuda::device_info (context.h:14-24, context.cu:41-48).
 * `name` receives at most name_len-1 chars plus NUL; gfx_arch is e.g. 950. */
UOCR_ROCM_API int uocr_rocm_device_info(int index, char* name, size_t name_len, int* gfx_arch, int* cu_count,
                                        uint64_t* free_bytes, uint64_t* total_bytes);

/* Replaces Context's stream (context.h:30-49, context.cu:50-53,65-75): a
 * non-blocking stream at the default priority on `device`. */
UOCR_ROCM_API int uocr_rocm_stream_create(int device, void** stream);
UOCR_ROCM_API int uocr_rocm_stream_destroy(void* stream);
UOCR_ROCM_API int uocr_rocm_stream_synchronize(void* stream);

/* Replaces Context::begin_capture / end_capture and Graph::launch
 * (context.h:39-63, context.cu:77-102): everything enqueued on `stream`
 * between the two calls is recorded, instantiated into *graph, and replayed
 * by uocr_rocm_graph_launch. */
UOCR_ROCM_API int uocr_rocm_capture_begin(void* stream);
UOCR_ROCM_API int uocr_rocm_capture_end(void* stream, void** graph);
UOCR_ROCM_API int uocr_rocm_graph_launch(void* graph, void* stream);
UOCR_ROCM_API int uocr_rocm_graph_destroy(void* graph);

/* Replaces Array's stream-ordered allocation (context.cu:120-127). */
UOCR_ROCM_API int uocr_rocm_malloc(void** ptr, size_t bytes, void* stream);
UOCR_ROCM_API int uocr_rocm_free(void* ptr, void* stream);
/* Replaces PinnedBuffer (context.h:67-79, context.cu:104-110). */
UOCR_ROCM_API int uocr_rocm_host_alloc(void** ptr, size_t bytes);
UOCR_ROCM_API int uocr_rocm_host_free(void* ptr);

/* Stream-ordered copies; neither waits. Replaces copy_to_device /
 * copy_to_host (context.h:81-83, context.cu:112-118) and, for device to
 * device, uocr::cuda::copy's memcpy (ops.h:68-69, ops.cu:264-266). */
enum uocr_rocm_copy_kind { UOCR_ROCM_H2D = 1, UOCR_ROCM_D2H = 2, UOCR_ROCM_D2D = 3 };
UOCR_ROCM_API int uocr_rocm_memcpy(void* dst, const void* src, size_t bytes, int kind, void* stream);

/* Replaces Array::zero (context.cu:212-216) with a fill kernel rather than a
 * memset node, so that it replays correctly inside a captured graph. */
UOCR_ROCM_API int uocr_rocm_zero(void* ptr, size_t bytes, void* stream);

/* Timing events on a stream (for benches; the reference has none). */
UOCR_ROCM_API int uocr_rocm_event_create(void** event);
UOCR_ROCM_API int uocr_rocm_event_destroy(void* event);
UOCR_ROCM_API int uocr_rocm_event_record(void* event, void* stream);
UOCR_ROCM_API int uocr_rocm_event_elapsed_ms(void* start, void* end, float* ms);

/* ---- the decode step's device state ------------------------------------ */

/* Same layout as uocr::cuda::StepState (src/backend/cuda/decode_ops.h:17-23):
 * the length-dependent values of one decode step, read on the device so a
 * captured step replays for every token. */
typedef struct uocr_rocm_step_state {
  int64_t token;      /* id whose embedding row enters the step          */
  int64_t pos;        /* cache row written this step (pos + 1 live keys) */
  int64_t tok;        /* rotary coordinate on the token axis             */
  int64_t page;       /* rotary coordinate on the page axis              */
  int64_t query_page; /* page the block router confines the query to, or -1 */
} uocr_rocm_step_state;

/* The block router's parameters (the reference's RouteParams,
 * src/backend/cuda/ops.h:112-120, and RouterParams,
 * src/model/block_router.h:16-26): keys per block (<= 64), blocks of the
 * always-attended local window, the entmax window (top_m <= 32), the blocks
 * read (top_k), the score scale, the probability floor and the bias scale. */
typedef struct uocr_rocm_route_params {
  int64_t block_size;
  int64_t local_blocks;
  int64_t top_m;
  int64_t top_k;
  float idx_scale;
  float floor;
  float sigma;
} uocr_rocm_route_params;

/* ---- fp32 ops: the reference's uocr::cuda signatures ------------------- */

/* y[i] += x[i]. Replaces add_inplace (src/backend/cuda/ops.h:30,
 * ops.cu:33-36,311-313); CPU form add_into (src/model/decoder.cpp:39-41). */
UOCR_ROCM_API int uocr_rocm_add_inplace(void* stream, float* y, const float* x, int64_t n);

/* dst = src, n fp32 elements, device to device. Replaces copy (ops.h:68-69). */
UOCR_ROCM_API int uocr_rocm_copy(void* stream, float* dst, const float* src, int64_t n);

/* In place, per row of x [rows, cols]: x = w * (x * inv),
 * inv = 1/sqrt(mean(x^2) + eps). Replaces rms_norm (ops.h:34,
 * ops.cu:39-81,324-326); oracle src/backend/reference/ops.cpp:129-141. */
UOCR_ROCM_API int uocr_rocm_rms_norm(void* stream, float* x, const float* w, int64_t rows, int64_t cols, float eps);

/* In place, per row: x = ((x - mean) * inv) * w + b, inv = 1/sqrt(var + eps),
 * with the mean and the variance of the row (two-pass over registers).
 * Replaces layer_norm (ops.h:32-33, ops.cu:319-322); oracle ops.cpp:111-127. */
UOCR_ROCM_API int uocr_rocm_layer_norm(void* stream, float* x, const float* w, const float* b, int64_t rows,
                                       int64_t cols, float eps);

/* In place: x = 0.5 x (1 + erf(x / sqrt 2)). Replaces gelu_erf (ops.h:37,
 * ops.cu:83-89,332-334); oracle ops.cpp:151-155. */
UOCR_ROCM_API int uocr_rocm_gelu_erf(void* stream, float* x, int64_t n);

/* g = silu(g) * u = (g * (1 / (1 + exp(-g)))) * u. Replaces silu_mul
 * (ops.h:39, ops.cu:91-94,340-342); oracle ops.cpp:40,163-167 plus the
 * multiply of src/model/feed_forward.cpp:18-24. */
UOCR_ROCM_API int uocr_rocm_silu_mul(void* stream, float* g, const float* u, int64_t n);

/* Two-axis rotate-half rope in place on x [rows, heads * dim], one (tok, page)
 * coordinate per row; tok/page may be null, then every row uses one_tok /
 * one_page. Pair p < n_tok turns by float(tok) * inv_tok[p], pair
 * p >= n_tok by float(page mod page_mod) * inv_page[p - n_tok]; requires
 * n_tok + n_page == dim / 2, dim even, dim <= 512. Replaces rope (ops.h:48-52,
 * ops.cu:134-151,354-360); oracle src/model/page_rope.cpp:26-56. The plain
 * rope of one frequency table is n_tok = dim / 2, n_page = 0. */
UOCR_ROCM_API int uocr_rocm_rope(void* stream, float* x, int64_t rows, int64_t heads, int64_t dim, const int64_t* tok,
                                 const int64_t* page, const float* inv_tok, int64_t n_tok, const float* inv_page,
                                 int64_t n_page, int64_t page_mod, int64_t one_tok, int64_t one_page);

/* dst[r, :] = widen(table[index[r], :]), bit-exact (bf16 -> fp32 is a
 * 16-bit shift). Replaces gather_rows_bf16 (ops.h:72-73, ops.cu:177-181,
 * 382-386); oracle Decoder::embed (src/model/decoder.cpp:85-92) over the
 * table widened at load (src/model/weight_source.cpp:16-23).
 * table_rows >= 0 bounds-checks every index: an index outside
 * [0, table_rows) yields a zero row instead of a read past the table.
 * table_rows < 0 trusts the caller, as the reference does. */
UOCR_ROCM_API int uocr_rocm_gather_rows_bf16(void* stream, const uint16_t* table, int64_t table_rows,
                                             const int64_t* index, int64_t rows, int64_t cols, float* dst);

/* One row by a host index. Replaces gather_row_bf16 (ops.h:74-75,
 * ops.cu:589-592,647-651). */
UOCR_ROCM_API int uocr_rocm_gather_row_bf16(void* stream, const uint16_t* table, int64_t table_rows,
                                            int64_t one_index, int64_t cols, float* dst);

/* One row by state->token, read on the device. Replaces embed_step
 * (src/backend/cuda/decode_ops.h:25, decode_ops.cu:26-29,203-206). */
UOCR_ROCM_API int uocr_rocm_embed_step(void* stream, const uint16_t* table, int64_t table_rows,
                                       const uocr_rocm_step_state* state, int64_t cols, float* dst);

/* rope of one row x [heads * dim] at (state->tok, state->page), read on the
 * device; the page table has dim / 2 - n_tok entries. Replaces rope_step
 * (decode_ops.h:26-27, decode_ops.cu:31-47,208-212). */
UOCR_ROCM_API int uocr_rocm_rope_step(void* stream, float* x, int64_t heads, int64_t dim,
                                      const uocr_rocm_step_state* state, const float* inv_tok, int64_t n_tok,
                                      const float* inv_page, int64_t page_mod);

/* ---- fused ops (new; no single reference counterpart) ------------------ */

/* Residual add fused with RMSNorm, per row of [rows, cols]:
 *   s = x + delta (fp32);  x = s;  h = w * (s * inv),  inv from s.
 * Replaces the chain add_inplace + copy + rms_norm composed at
 * src/model/cuda/cuda_decoder.cpp:267-278 and cuda_decode_step.cpp:54-65
 * (CPU form src/model/decoder.cpp:176-181,196-201): one read of x and delta,
 * one write of x and h, instead of five full passes. */
UOCR_ROCM_API int uocr_rocm_add_rms_norm(void* stream, float* x, const float* delta, const float* w, float* h,
                                         int64_t rows, int64_t cols, float eps);

/* SwiGLU over a concatenated [gate | up] input: in [rows, 2 * ffn] row-major,
 * out [rows, ffn] = silu(gate) * up. Replaces the gate/up pair +
 * silu_mul of CudaDecoder::mlp (src/model/cuda/cuda_decoder.cpp:119-135) and
 * GatedMlp::forward (src/model/feed_forward.cpp:18-24). */
UOCR_ROCM_API int uocr_rocm_swiglu(void* stream, const float* in, float* out, int64_t rows, int64_t ffn);

/* rope on Q [rows, q_heads * dim] and K [rows, k_heads * dim] in one launch,
 * sharing each row's cos/sin across all q_heads + k_heads heads. Same
 * arithmetic and arguments as uocr_rocm_rope; k may be null when k_heads is
 * 0. Replaces the per-tensor rope calls of CudaDecoder::attention
 * (src/model/cuda/cuda_decoder.cpp:213-220). */
UOCR_ROCM_API int uocr_rocm_rope_qk(void* stream, float* q, int64_t q_heads, float* k, int64_t k_heads, int64_t rows,
                                    int64_t dim, const int64_t* tok, const int64_t* page, const float* inv_tok,
                                    int64_t n_tok, const float* inv_page, int64_t n_page, int64_t page_mod,
                                    int64_t one_tok, int64_t one_page);

/* rope_qk for one decode row at (state->tok, state->page). Replaces the
 * rope_step pair of decode_attention (src/model/cuda/cuda_decode_step.cpp:27-28). */
UOCR_ROCM_API int uocr_rocm_rope_qk_step(void* stream, float* q, int64_t q_heads, float* k, int64_t k_heads,
                                         int64_t dim, const uocr_rocm_step_state* state, const float* inv_tok,
                                         int64_t n_tok, const float* inv_page, int64_t page_mod);

/* ---- bf16-activation variants (new) ------------------------------------
 * Same arithmetic as the fp32 entry point of the same name on the widened
 * inputs, rounded to bf16 once on store; each reduces to its fp32 op. */

UOCR_ROCM_API int uocr_rocm_rms_norm_bf16(void* stream, uint16_t* x, const float* w, int64_t rows, int64_t cols,
                                          float eps);
UOCR_ROCM_API int uocr_rocm_add_rms_norm_bf16(void* stream, uint16_t* x, const uint16_t* delta, const float* w,
                                              uint16_t* h, int64_t rows, int64_t cols, float eps);
UOCR_ROCM_API int uocr_rocm_layer_norm_bf16(void* stream, uint16_t* x, const float* w, const float* b, int64_t rows,
                                            int64_t cols, float eps);
/* New: y = bf16(layer_norm(x)) out of place, x fp32 [rows, cols] read only and
 * y bf16 [rows, cols] (nearest even), cols up to 16384: a LayerNorm whose
 * only reader is a projection, with the rounding the projection applies to
 * its input (the reference's layer_norm then linear, ops.h:14-17,32-33);
 * bitwise uocr_rocm_layer_norm on a copy of x followed by
 * uocr_rocm_round_bf16. */
UOCR_ROCM_API int uocr_rocm_layer_norm_to_bf16(void* stream, const float* x, const float* w, const float* b,
                                               uint16_t* y, int64_t rows, int64_t cols, float eps);
UOCR_ROCM_API int uocr_rocm_gelu_erf_bf16(void* stream, uint16_t* x, int64_t n);
UOCR_ROCM_API int uocr_rocm_swiglu_bf16(void* stream, const uint16_t* in, uint16_t* out, int64_t rows, int64_t ffn);
UOCR_ROCM_API int uocr_rocm_rope_bf16(void* stream, uint16_t* x, int64_t rows, int64_t heads, int64_t dim,
                                      const int64_t* tok, const int64_t* page, const float* inv_tok, int64_t n_tok,
                                      const float* inv_page, int64_t n_page, int64_t page_mod, int64_t one_tok,
                                      int64_t one_page);
UOCR_ROCM_API int uocr_rocm_rope_qk_bf16(void* stream, uint16_t* q, int64_t q_heads, uint16_t* k, int64_t k_heads,
                                         int64_t rows, int64_t dim, const int64_t* tok, const int64_t* page,
                                         const float* inv_tok, int64_t n_tok, const float* inv_page, int64_t n_page,
                                         int64_t page_mod, int64_t one_tok, int64_t one_page);
UOCR_ROCM_API int uocr_rocm_rope_qk_step_bf16(void* stream, uint16_t* q, int64_t q_heads, uint16_t* k,
                                              int64_t k_heads, int64_t dim, const uocr_rocm_step_state* state,
                                              const float* inv_tok, int64_t n_tok, const float* inv_page,
                                              int64_t page_mod);
/* Embedding rows kept in bf16: a bit copy of table rows. */
UOCR_ROCM_API int uocr_rocm_gather_rows_bf16_bf16(void* stream, const uint16_t* table, int64_t table_rows,
                                                  const int64_t* index, int64_t rows, int64_t cols, uint16_t* dst);
UOCR_ROCM_API int uocr_rocm_embed_step_bf16(void* stream, const uint16_t* table, int64_t table_rows,
                                            const uocr_rocm_step_state* state, int64_t cols, uint16_t* dst);

/* ---- row ops beside the path ---------------------------------------------- */

/* The MoE router's norm, in place per row of [rows, cols]: non-finite inputs
 * become 0, inv = 1 / sqrt(mean(x^2) + eps), x = clamp(clamp(x * inv) *
 * (1 + w)) with clamp to [-1e4, 1e4]. Replaces router_norm
 * (src/backend/cuda/ops.h:35-36, ops.cu:39-81 mode 2; CPU form
 * src/model/decoder.cpp:20-34). */
UOCR_ROCM_API int uocr_rocm_router_norm(void* stream, float* x, const float* w, int64_t rows, int64_t cols, float eps);
UOCR_ROCM_API int uocr_rocm_router_norm_bf16(void* stream, uint16_t* x, const float* w, int64_t rows, int64_t cols,
                                             float eps);

/* x = x * sigmoid(1.702 x), in place over n elements. Replaces quick_gelu
 * (src/backend/cuda/ops.h:38). */
UOCR_ROCM_API int uocr_rocm_quick_gelu(void* stream, float* x, int64_t n);
UOCR_ROCM_API int uocr_rocm_quick_gelu_bf16(void* stream, uint16_t* x, int64_t n);

/* Softmax over each row of x [rows, cols] in place (fp32 max, exp(x - max),
 * fp32 total, 1 / total formed in fp64); a row that is all -inf becomes
 * zeros. Replaces softmax_rows (src/backend/cuda/ops.h:41-43). */
UOCR_ROCM_API int uocr_rocm_softmax_rows(void* stream, float* x, int64_t rows, int64_t cols);

/* x[b, r, c] = x[b, r, c] * scale + mask[r, c] for each of `batch` slices of
 * [rows, cols]; mask may be null (+ 0). batch * rows * cols < 2^32 - 256.
 * Replaces scale_add_mask (src/backend/cuda/ops.h:44-46). */
UOCR_ROCM_API int uocr_rocm_scale_add_mask(void* stream, float* x, float scale, const float* mask, int64_t batch,
                                           int64_t rows, int64_t cols);

/* Softmax of the scaled, masked scores in one pass (new): for each of `batch`
 * slices of [rows, cols], x[b, r, :] = softmax(x[b, r, :] * scale + mask[r, :])
 * (mask null: + 0). Bitwise uocr_rocm_scale_add_mask then
 * uocr_rocm_softmax_rows, with one read and one write of x instead of two of
 * each. batch * rows < 2^31. Replaces the pair in CudaDecoder::attention
 * (src/model/cuda/cuda_decoder.cpp:241-242). */
UOCR_ROCM_API int uocr_rocm_scale_mask_softmax_rows(void* stream, float* x, float scale, const float* mask,
                                                    int64_t batch, int64_t rows, int64_t cols);

/* ---- prefill projections ------------------------------------------------------- */

/* y[m, n] = bf16(x)[m, k] . w[n, k]^T (+ bias[n]): x fp32 row-major, rounded
 * to bf16 (nearest even) for the product, w bf16 row-major, fp32
 * accumulation on the matrix cores, fp32 y; the bias (may be null) is added
 * to each finished sum. m == 1 (k <= 12288, k a multiple of 8, x and w
 * 16-byte aligned) goes through uocr_rocm_gemv_bf16. Any k >= 1; rows that
 * are not 16-byte multiples load element by element. Replaces linear
 * (src/backend/cuda/ops.h:14-17). */
UOCR_ROCM_API int uocr_rocm_linear(void* stream, const float* x, int64_t m, int64_t k, const uint16_t* w, int64_t n,
                                   const float* bias, float* y);
/* New: the same product with x already bf16 [m, k] (the rounding done by the
 * producer, e.g. uocr_rocm_round_bf16 once for several projections of one
 * activation); with k a multiple of 64 its tiles go straight from memory
 * into LDS. */
UOCR_ROCM_API int uocr_rocm_linear_bf16x(void* stream, const uint16_t* x, int64_t m, int64_t k, const uint16_t* w,
                                         int64_t n, const float* bias, float* y);
/* New: uocr_rocm_linear and uocr_rocm_linear_bf16x with a workspace of
 * workspace_floats fp32 values: where the m x n tiles are too few to cover
 * the GPU, k is split over the workspace (each split's partial products,
 * then their sum in split order and the bias in one more launch); with a
 * workspace smaller than uocr_rocm_linear_workspace_floats(m, k, n) (0 when
 * no split is taken) the product runs unsplit. Allocates nothing. */
UOCR_ROCM_API int64_t uocr_rocm_linear_workspace_floats(int64_t m, int64_t k, int64_t n);
UOCR_ROCM_API int uocr_rocm_linear_ws(void* stream, const float* x, int64_t m, int64_t k, const uint16_t* w,
                                      int64_t n, const float* bias, float* y, float* workspace,
                                      int64_t workspace_floats);
UOCR_ROCM_API int uocr_rocm_linear_bf16x_ws(void* stream, const uint16_t* x, int64_t m, int64_t k, const uint16_t* w,
                                            int64_t n, const float* bias, float* y, float* workspace,
                                            int64_t workspace_floats);
/* New: y += bf16(x) . w^T (+ bias), y fp32 [m, n] read and written: each
 * element becomes y + (sum + bias), bitwise uocr_rocm_linear_bf16x_ws into
 * a temporary followed by uocr_rocm_add_inplace (the reference's linear then
 * add_inplace on a residual stream, ops.h:14-17). Same workspace rule. */
UOCR_ROCM_API int uocr_rocm_linear_bf16x_add_ws(void* stream, const uint16_t* x, int64_t m, int64_t k,
                                                const uint16_t* w, int64_t n, const float* bias, float* y,
                                                float* workspace, int64_t workspace_floats);
/* New: the same with the product's rows scattered: row r is added into y row
 * y_row[r] (device int64 [m]; a value of y_rows or more drops the row), y
 * [y_rows, n]: window slots added back into their grid rows, bitwise the
 * product, the gather of the kept rows and uocr_rocm_add_inplace. Rows
 * mapping to one y row must not repeat (each is written once); k is a
 * multiple of 64 and x, w are 16-byte aligned. */
UOCR_ROCM_API int uocr_rocm_linear_bf16x_add_rows(void* stream, const uint16_t* x, int64_t m, int64_t k,
                                                  const uint16_t* w, int64_t n, const float* bias, float* y,
                                                  const int64_t* y_row, int64_t y_rows);

/* New: dst[i] = bf16(src[i]), nearest even; both 16-byte aligned. */
UOCR_ROCM_API int uocr_rocm_round_bf16(void* stream, const float* src, int64_t n, uint16_t* dst);
/* New: y[i] = bf16(gelu_erf(x[i])) and y[i] = bf16(quick_gelu(x[i])), x
 * fp32 [n] and y bf16 [n] (nearest even): an MLP's activation together with
 * the rounding its second projection applies to its input (the reference's
 * gelu_erf / quick_gelu then linear, ops.h:14-17,37-38), bitwise the fp32
 * op followed by uocr_rocm_round_bf16. */
UOCR_ROCM_API int uocr_rocm_gelu_erf_to_bf16(void* stream, const float* x, uint16_t* y, int64_t n);
UOCR_ROCM_API int uocr_rocm_quick_gelu_to_bf16(void* stream, const float* x, uint16_t* y, int64_t n);
/* New: an MLP's first projection with its activation in the epilogue,
 * y = bf16(act(x . w^T + bias)), y bf16 [m, n] (nearest even): the
 * reference's linear then gelu_erf / quick_gelu (ops.h:14-17,37-38) with
 * the rounding the second projection applies to its input, bitwise
 * uocr_rocm_linear_bf16x followed by uocr_rocm_gelu_erf_to_bf16 /
 * uocr_rocm_quick_gelu_to_bf16 without the fp32 [m, n] between them. k is a
 * multiple of 64 and x, w are 16-byte aligned. */
UOCR_ROCM_API int uocr_rocm_linear_bf16x_gelu_erf_bf16(void* stream, const uint16_t* x, int64_t m, int64_t k,
                                                       const uint16_t* w, int64_t n, const float* bias,
                                                       uint16_t* y);
UOCR_ROCM_API int uocr_rocm_linear_bf16x_quick_gelu_bf16(void* stream, const uint16_t* x, int64_t m, int64_t k,
                                                         const uint16_t* w, int64_t n, const float* bias,
                                                         uint16_t* y);

/* c[s] = alpha a[s] . b[s]^T (gemm_nt: a [m, k], b [n, k]) or c[s] = a[s] . b[s]
 * (gemm_nn: a [m, k], b [k, n]), fp32, row-major with leading dimensions
 * lda / ldb / ldc, for `batch` slices s whose operands sit stride_a /
 * stride_b / stride_c elements apart. Replaces gemm_nt and gemm_nn
 * (src/backend/cuda/ops.h:19-27). */
UOCR_ROCM_API int uocr_rocm_gemm_nt(void* stream, int64_t m, int64_t n, int64_t k, float alpha, const float* a,
                                    int64_t lda, int64_t stride_a, const float* b, int64_t ldb, int64_t stride_b,
                                    float* c, int64_t ldc, int64_t stride_c, int64_t batch);
UOCR_ROCM_API int uocr_rocm_gemm_nn(void* stream, int64_t m, int64_t n, int64_t k, const float* a, int64_t lda,
                                    int64_t stride_a, const float* b, int64_t ldb, int64_t stride_b, float* c,
                                    int64_t ldc, int64_t stride_c, int64_t batch);

/* dst[i] = src[index[i]] for rows [cols] (fp32); and dst[index[i]] +=
 * weight[i] * src[i] for i in order (an index may repeat). Indices are
 * trusted, as in the reference. Replace gather_rows and scatter_add_rows
 * (src/backend/cuda/ops.h:56-60). */
UOCR_ROCM_API int uocr_rocm_gather_rows(void* stream, const float* src, const int64_t* index, int64_t rows,
                                        int64_t cols, float* dst);
UOCR_ROCM_API int uocr_rocm_scatter_add_rows(void* stream, float* dst, const int64_t* index, const float* weight,
                                             const float* src, int64_t rows, int64_t cols);

/* ---- the vision encoder's layout and attention-bias ops ------------------------- */

/* cols [oh * ow, c * kh * kw] = the patches of x [c, h, w] in the weight's
 * [c, kh, kw] column order, zero outside the image, oh = (h + 2 pad - kh) /
 * stride + 1 (ow alike). Replaces im2col (src/backend/cuda/ops.h:54-56). */
UOCR_ROCM_API int uocr_rocm_im2col(void* stream, const float* x, int64_t c, int64_t h, int64_t w, int64_t kh,
                                   int64_t kw, int64_t stride, int64_t pad, float* cols);
/* New: the same with cols bf16 (nearest even): the patches with the
 * rounding the convolution's linear applies to them, bitwise im2col then
 * uocr_rocm_round_bf16 (the reference's im2col then linear,
 * cuda_vision.cpp:204-237). */
UOCR_ROCM_API int uocr_rocm_im2col_bf16(void* stream, const float* x, int64_t c, int64_t h, int64_t w, int64_t kh,
                                        int64_t kw, int64_t stride, int64_t pad, uint16_t* cols);

/* y [h, w, c] = x [c, h, w] and y [c, h, w] = x [h, w, c] (out of place).
 * Replace chw_to_hwc and hwc_to_chw (src/backend/cuda/ops.h:57-58). */
UOCR_ROCM_API int uocr_rocm_chw_to_hwc(void* stream, const float* x, int64_t c, int64_t h, int64_t w, float* y);
UOCR_ROCM_API int uocr_rocm_hwc_to_chw(void* stream, const float* x, int64_t h, int64_t w, int64_t c, float* y);

/* out[r] = a[r] (ca values) followed by b[r] (cb values), rows of fp32.
 * Replaces concat_cols (src/backend/cuda/ops.h:65-67). */
UOCR_ROCM_API int uocr_rocm_concat_cols(void* stream, const float* a, int64_t ca, const float* b, int64_t cb,
                                        int64_t rows, float* out);

/* New: y [parts, heads, rows, hd] = x [rows, parts, heads, hd] and y [rows,
 * heads, hd] = x [heads, rows, hd] (fp32, hd a multiple of 4, 16-byte
 * aligned, exact): the attention operands in a head-major layout, so that
 * one batched product covers every head (and window) with one stride, and
 * the heads' outputs back to rows. No counterpart in the reference, which
 * launches its products head by head (src/model/cuda/cuda_vision.cpp:
 * 159-170, 252-254). */
UOCR_ROCM_API int uocr_rocm_split_heads(void* stream, const float* x, int64_t rows, int64_t parts, int64_t heads,
                                        int64_t hd, float* y);
UOCR_ROCM_API int uocr_rocm_merge_heads(void* stream, const float* x, int64_t heads, int64_t rows, int64_t hd,
                                        float* y);

/* SAM's decomposed relative-position bias for one head of one window:
 * bias[t, ky * w + kx] = q_t . rh[qy, ky] + q_t . rw[qx, kx] for query t =
 * qy * w + qx, q rows ldq apart, rh [h, h, d], rw [w, w, d], bias [h w, h w].
 * d <= 256, h + w <= 2048. Allocates nothing. Replaces rel_pos_bias
 * (src/backend/cuda/ops.h:91-95). */
UOCR_ROCM_API int uocr_rocm_rel_pos_bias(void* stream, const float* q, int64_t ldq, int64_t h, int64_t w, int64_t d,
                                         const float* rh, const float* rw, float* bias);

/* New: scores [windows, h w, h w] of one head in place = softmax over each
 * row of (scores + bias), the bias of uocr_rocm_rel_pos_bias formed inside
 * the row's workgroup from the query rows (window-major, ldq apart: row
 * window * h w + t at q + (window * h w + t) * ldq). The reference's
 * rel_pos_bias + add_inplace + softmax_rows over every window
 * (src/model/cuda/cuda_vision.cpp:161-166) in one pass over the scores. */
UOCR_ROCM_API int uocr_rocm_rel_pos_softmax_rows(void* stream, float* scores, int64_t windows, const float* q,
                                                 int64_t ldq, int64_t h, int64_t w, int64_t d, const float* rh,
                                                 const float* rw);

/* ---- attention in one pass ------------------------------------------------------- */

/* New: out[s, t] = softmax over keys of (scale * q[s, t] . k[s, key] +
 * mask[t, key]) times v[s, key], for slices s (heads, or heads of windows)
 * and query rows t, fp32 on the matrix cores; the scores never reach memory.
 * Row t of slice s of q sits at q + s * sq + t * ldq (k, v, out alike, in
 * elements); hd is 64 or 128; operands 16-byte aligned with strides of
 * whole 16-byte chunks. mask [rows, mask_ld] (shared by the slices, -inf
 * for a key not attended) or null. A row with no finite score gives zeros.
 * Replaces the reference's gemm_nt + scale_add_mask (or bias add) +
 * softmax_rows + gemm_nn sequence (src/model/cuda/cuda_decoder.cpp:88-105,
 * src/model/cuda/cuda_vision.cpp:251-254). */
UOCR_ROCM_API int uocr_rocm_attention(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                                      int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out,
                                      int64_t ldo, int64_t so, int64_t slices, int64_t rows, int64_t keys, int64_t hd,
                                      float scale, const float* mask, int64_t mask_ld);

/* New: the same over SAM's windows of h x w tokens (rows = keys = h w per
 * slice) with the decomposed relative-position bias of
 * uocr_rocm_rel_pos_bias (rh [h, h, hd], rw [w, w, hd], formed from each
 * slice's own query rows; both 16-byte aligned) in place of the mask;
 * h + w <= 256. Replaces the
 * reference's per-head gemm_nt + rel_pos_bias + add_inplace + softmax_rows
 * + gemm_nn (src/model/cuda/cuda_vision.cpp:159-170). */
UOCR_ROCM_API int uocr_rocm_attention_rel_pos(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                                              int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv,
                                              float* out, int64_t ldo, int64_t so, int64_t slices, int64_t h,
                                              int64_t w, int64_t hd, float scale, const float* rh, const float* rw);
/* New: the same with a workspace for the bias's per-query dot products
 * (q . rh[qy, ky] and q . rw[qx, kx] of every slice and query row), formed
 * by one launch that reads each table slice once per slice before the
 * attention, in place of every workgroup forming its own; the workspace
 * holds uocr_rocm_attention_rel_pos_workspace_floats(slices, h, w) floats,
 * 16-byte aligned (a smaller one: the attention forms its own). */
UOCR_ROCM_API int64_t uocr_rocm_attention_rel_pos_workspace_floats(int64_t slices, int64_t h, int64_t w);
/* New: the same over heads x windows slices, slice (head, window) of each
 * operand at base + head * s_ + window * w_ (row stride ld_): the heads
 * and windows straight from a window-major qkv projection's rows [windows *
 * h * w, 3 * width], the output into the merged rows, with no head-major
 * copies. Window strides are multiples of 4 floats; the workspace as for
 * uocr_rocm_attention_rel_pos_ws with slices = heads * windows. */
UOCR_ROCM_API int uocr_rocm_attention_rel_pos_windows_ws(void* stream, const float* q, int64_t ldq, int64_t sq,
                                                         int64_t wq, const float* k, int64_t ldk, int64_t sk,
                                                         int64_t wk, const float* v, int64_t ldv, int64_t sv,
                                                         int64_t wv, float* out, int64_t ldo, int64_t so, int64_t wo,
                                                         int64_t heads, int64_t windows, int64_t h, int64_t w,
                                                         int64_t hd, float scale, const float* rh, const float* rw,
                                                         float* workspace, int64_t workspace_floats);
/* New: uocr_rocm_attention and uocr_rocm_attention_rel_pos_windows_ws with
 * the output in bf16 (nearest even) at the same element offsets (out
 * 16-byte aligned): attention whose only reader is the output projection,
 * with the rounding that projection applies to its input, bitwise the fp32
 * entry followed by uocr_rocm_round_bf16 (the reference's attention then
 * linear, cuda_vision.cpp:151-172, 253-256). */
UOCR_ROCM_API int uocr_rocm_attention_bf16(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                                           int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv,
                                           uint16_t* out, int64_t ldo, int64_t so, int64_t slices, int64_t rows,
                                           int64_t keys, int64_t hd, float scale, const float* mask,
                                           int64_t mask_ld);
/* New: uocr_rocm_attention and uocr_rocm_attention_bf16 with a workspace
 * (uocr_rocm_attention_workspace_floats(slices, rows, keys, hd) floats,
 * 16-byte aligned) for a mask: a first launch marks, per 128 query rows,
 * the 32-key tiles where some mask entry is finite, and the fp32 products
 * walk only those; where the row blocks of all slices leave CUs idle, a
 * block's walk is cut into runs whose (max, total, values) records a last
 * launch combines, so a causal mask's longest walks no longer set the time.
 * fp32 arithmetic throughout (the sums of a cut row in another order); the
 * bf16 entry is bitwise the fp32 one then uocr_rocm_round_bf16. A null mask
 * takes the entries above (the workspace unused). */
UOCR_ROCM_API int64_t uocr_rocm_attention_workspace_floats(int64_t slices, int64_t rows, int64_t keys, int64_t hd);
UOCR_ROCM_API int uocr_rocm_attention_ws(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                                         int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv, float* out,
                                         int64_t ldo, int64_t so, int64_t slices, int64_t rows, int64_t keys,
                                         int64_t hd, float scale, const float* mask, int64_t mask_ld,
                                         float* workspace, int64_t workspace_floats);
UOCR_ROCM_API int uocr_rocm_attention_bf16_ws(void* stream, const float* q, int64_t ldq, int64_t sq, const float* k,
                                              int64_t ldk, int64_t sk, const float* v, int64_t ldv, int64_t sv,
                                              uint16_t* out, int64_t ldo, int64_t so, int64_t slices, int64_t rows,
                                              int64_t keys, int64_t hd, float scale, const float* mask,
                                              int64_t mask_ld, float* workspace, int64_t workspace_floats);
/* New: uocr_rocm_attention_bf16 with a mask, on the bf16 matrix cores with
 * each fp32 operand split into bf16 hi + lo parts (a . b = lo_a hi_b +
 * hi_a lo_b + hi_a hi_b in fp32: about 2^-16 of each product dropped, far
 * below the output's bf16 rounding, so not bitwise the fp32 entry's
 * rounding). Two launches first fill the workspace
 * (uocr_rocm_attention_masked_workspace_floats(slices, rows, keys, hd)
 * floats, 16-byte aligned): a bit per (128 query rows, 32-key tile) where
 * some mask entry is finite, and every key tile split once; the attention
 * stages and multiplies only the live tiles. mask non-null, mask_ld >=
 * keys. The decoder prefill's
 * attention of CudaDecoder::attention (src/model/cuda/cuda_decoder.cpp:
 * 88-105) followed by the bf16 rounding its output projection applies. */
UOCR_ROCM_API int64_t uocr_rocm_attention_masked_workspace_floats(int64_t slices, int64_t rows, int64_t keys,
                                                                 int64_t hd);
UOCR_ROCM_API int uocr_rocm_attention_masked_bf16_ws(void* stream, const float* q, int64_t ldq, int64_t sq,
                                                     const float* k, int64_t ldk, int64_t sk, const float* v,
                                                     int64_t ldv, int64_t sv, uint16_t* out, int64_t ldo, int64_t so,
                                                     int64_t slices, int64_t rows, int64_t keys, int64_t hd,
                                                     float scale, const float* mask, int64_t mask_ld,
                                                     float* workspace, int64_t workspace_floats);
UOCR_ROCM_API int uocr_rocm_attention_rel_pos_windows_bf16_ws(
    void* stream, const float* q, int64_t ldq, int64_t sq, int64_t wq, const float* k, int64_t ldk, int64_t sk,
    int64_t wk, const float* v, int64_t ldv, int64_t sv, int64_t wv, uint16_t* out, int64_t ldo, int64_t so,
    int64_t wo, int64_t heads, int64_t windows, int64_t h, int64_t w, int64_t hd, float scale, const float* rh,
    const float* rw, float* workspace, int64_t workspace_floats);
UOCR_ROCM_API int uocr_rocm_attention_rel_pos_ws(void* stream, const float* q, int64_t ldq, int64_t sq,
                                                 const float* k, int64_t ldk, int64_t sk, const float* v, int64_t ldv,
                                                 int64_t sv, float* out, int64_t ldo, int64_t so, int64_t slices,
                                                 int64_t h, int64_t w, int64_t hd, float scale, const float* rh,
                                                 const float* rw, float* workspace, int64_t workspace_floats);

/* ---- decode-step neighbours ---------------------------------------------------- */

/* y[n] = bf16(x) . w[n, :] (+ bias[n]): x fp32 [k] rounded to bf16 (nearest
 * even) before the product, w bf16 [n, k] row-major, fp32 accumulation; bias
 * may be null. k <= 12288. Replaces gemv_bf16
 * (src/backend/cuda/gemv_ops.h:25-26); the same product as linear with m = 1
 * (src/backend/cuda/ops.h:14-17). */
UOCR_ROCM_API int uocr_rocm_gemv_bf16(void* stream, const float* x, int64_t k, const uint16_t* w, int64_t n,
                                      const float* bias, float* y);

/* cache[state->pos, :] = row, rows `width` floats wide. With capacity >= 0 a
 * position outside [0, capacity) writes nothing; capacity < 0 leaves the
 * upper bound unchecked, as the reference does (a negative position never
 * writes). Replaces append_step (src/backend/cuda/decode_ops.h:28-29). */
UOCR_ROCM_API int uocr_rocm_append_step(void* stream, float* cache, const float* row, int64_t width,
                                        const uocr_rocm_step_state* state, int64_t capacity);

/* A bf16 key/value cache (new): the fp32 row is rounded to bf16 (nearest
 * even) as it is appended, and the attention widens the cached keys and
 * values to fp32 (q, the scores, the softmax and out stay fp32). Half the
 * cache bytes of the fp32 forms; otherwise the same contract and the same
 * arithmetic on the bf16-rounded values (a lane holds 8 cache elements
 * instead of 4, so sums associate differently). */
UOCR_ROCM_API int uocr_rocm_append_step_bf16(void* stream, uint16_t* cache, const float* row, int64_t width,
                                             const uocr_rocm_step_state* state, int64_t capacity);
UOCR_ROCM_API int uocr_rocm_attend_step_bf16(void* stream, const float* q, const uint16_t* k_cache,
                                             const uint16_t* v_cache, int64_t heads, int64_t hd, const float* mask,
                                             float scale, const uocr_rocm_step_state* state, float* scratch,
                                             int64_t capacity, float* out);

/* Floats of scratch that uocr_rocm_attend_step needs for (heads, hd,
 * capacity); 0 for an empty shape. Replaces attend_scratch_floats
 * (src/backend/cuda/decode_ops.h:42-43). */
UOCR_ROCM_API int64_t uocr_rocm_attend_scratch_floats(int64_t heads, int64_t hd, int64_t capacity);

/* Masked attention of one query over the keys 0..state->pos of a cache:
 *   out[h] = sum_j p_j v[j, h],  p = softmax_j(q_h . k[j, h] * scale + mask[j])
 * q [heads * hd]; k_cache, v_cache [capacity, heads * hd] with head h at
 * column h * hd; mask [capacity] (null: no mask; -inf masks a key, which is
 * then not read); out [heads * hd]. Keys past capacity are not read. Keys
 * all masked give zeros. scratch holds uocr_rocm_attend_scratch_floats(heads,
 * hd, capacity) floats and must not be shared by overlapping calls.
 * 1 <= hd <= 256. Two launches whose shapes depend only on (heads, hd,
 * capacity), so a captured step replays at every position. Replaces
 * attend_step (src/backend/cuda/decode_ops.h:44-47). */
UOCR_ROCM_API int uocr_rocm_attend_step(void* stream, const float* q, const float* k_cache, const float* v_cache,
                                        int64_t heads, int64_t hd, const float* mask, float scale,
                                        const uocr_rocm_step_state* state, float* scratch, int64_t capacity,
                                        float* out);

/* uocr_rocm_attend_step without the scratch argument: the same kernels and
 * results, with the split records in a fixed device array of 1,048,576
 * floats (4 MiB) that each GPU the library runs on holds until the process
 * ends, so the call allocates nothing (no hipMalloc, hipFree or allocating
 * library routine). It has no counterpart in the reference: it is for
 * callers that cannot allocate (code under HIP graph capture, tight serving
 * loops, harnesses that forbid allocation). A (heads, hd, capacity) whose
 * uocr_rocm_attend_scratch_floats exceeds 1,048,576 is rejected with
 * UOCR_ROCM_INVALID_ARGUMENT. Every call on one GPU shares that GPU's array
 * and leaves its records there; calls that overlap on one GPU (two streams,
 * or two host threads) race on it. */
UOCR_ROCM_API int uocr_rocm_attend_step_noalloc(void* stream, const float* q, const float* k_cache,
                                                const float* v_cache, int64_t heads, int64_t hd, const float* mask,
                                                float scale, const uocr_rocm_step_state* state, int64_t capacity,
                                                float* out);

/* ---- the block router of sparse decode attention ------------------------------
 * Router keys rk [keys, d] and queries rq [d] are fp32, d a multiple of 4 in
 * [4, 256], block_size * d <= 8192; at most 4096 blocks per query row. */

/* Per block of block_size keys of rk [s, d]: the softmax(clamp(rk . head_cls
 * / sqrt d))-weighted mean of its keys, out [ceil(s / block_size), d].
 * Replaces block_summaries (src/backend/cuda/ops.h:97-100). */
UOCR_ROCM_API int uocr_rocm_block_summaries(void* stream, const float* keys, int64_t s, int64_t d,
                                            const float* head_cls, int64_t block_size, float* out);

/* The summary of the block holding state->pos (keys first..pos of the
 * router-key cache), written to summaries[pos / block_size]; a pos past
 * max_blocks blocks writes nothing. Replaces summary_step
 * (src/backend/cuda/decode_ops.h:30-33), with max_blocks added as a bound. */
UOCR_ROCM_API int uocr_rocm_summary_step(void* stream, const float* router_keys, int64_t d, const float* head_cls,
                                         int64_t block_size, const uocr_rocm_step_state* state, int64_t max_blocks,
                                         float* summaries);

/* z[b] = rq . summaries[b] / sqrt d for every block up to the one holding
 * state->pos (at most max_blocks <= 4096). Replaces scores_step
 * (src/backend/cuda/decode_ops.h:34-36). */
UOCR_ROCM_API int uocr_rocm_scores_step(void* stream, const float* rq, const float* summaries, int64_t d,
                                        int64_t block_size, const uocr_rocm_step_state* state, int64_t max_blocks,
                                        float* z);

/* The route of prompt rows: row i (position first_pos + i, page
 * query_page[i] or, when query_page is null, one_page; a negative page is
 * unrestricted) scores the blocks before its local window from z [rows,
 * nblk] (clamped to +-1e4), keeps the blocks holding its page's image tokens
 * (page ranges per prompt block in block_min / block_max; none in range
 * means every block), takes the top_m through 1.5-entmax, reads the first
 * top_k with a log-prior bias, and writes its key mask [keys]: 0 on the
 * local window, the bias on a selected block's keys, -inf elsewhere and
 * past its position. Replaces route_blocks (src/backend/cuda/ops.h:102-124). */
UOCR_ROCM_API int uocr_rocm_route_blocks(void* stream, const float* z, int64_t rows, int64_t nblk, int64_t first_pos,
                                         int64_t keys, const int64_t* block_min, const int64_t* block_max,
                                         int64_t prompt_blocks, const int64_t* query_page, int64_t one_page,
                                         const uocr_rocm_route_params* params, float* mask);

/* The route of the one decode query at state->pos (page state->query_page)
 * from z, writing mask[0..pos]. Replaces route_step
 * (src/backend/cuda/decode_ops.h:37-40). */
UOCR_ROCM_API int uocr_rocm_route_step(void* stream, const float* z, int64_t max_blocks, const int64_t* block_min,
                                       const int64_t* block_max, int64_t prompt_blocks,
                                       const uocr_rocm_step_state* state, const uocr_rocm_route_params* params,
                                       float* mask);

/* New: the router half of a decode step in one launch, bitwise the separate
 * ops: the router norm of rq and rk (weights q_norm, k_norm), rope on both
 * at (state->tok, state->page) with the PageRope tables, rk appended to
 * router_keys [capacity, d] at pos, the summary of the block holding pos,
 * the scores of the blocks before the window and the route into mask
 * [capacity] (keys 0..pos written). z_out (capacity blocks) and rqk_out
 * ([2 d]: rq and rk after norm and rope) are optional outputs for checking.
 * Replaces the router projections' norms and ropes, append_step of the
 * router key, summary_step, scores_step and route_step of
 * CudaDecoder::decode_attention (src/model/cuda/cuda_decode_step.cpp:19-41). */
UOCR_ROCM_API int uocr_rocm_route_decode_step(void* stream, const float* rq, const float* rk, const float* q_norm,
                                              const float* k_norm, float eps, const float* inv_tok, int64_t n_tok,
                                              const float* inv_page, int64_t page_mod, const float* head_cls,
                                              float* router_keys, float* summaries, int64_t d,
                                              const int64_t* block_min, const int64_t* block_max,
                                              int64_t prompt_blocks, const uocr_rocm_step_state* state,
                                              const uocr_rocm_route_params* params, int64_t capacity, float* mask,
                                              float* z_out, float* rqk_out);

/* The keys a routed decode query reads, so that its attention visits them
 * alone (the key segments): int32 [4 (1 + UOCR_ROCM_MAX_KEY_SEGMENTS)],
 * word 0 the segment count, word 1 the live key count, then per segment
 * {first key, key count, bias (fp32 bits), 0} in ascending key order: the
 * valid selected blocks, each clipped at the local window (and at pos), then
 * the window itself, every key with the value the mask gives it. */
#define UOCR_ROCM_MAX_KEY_SEGMENTS 33
/* uocr_rocm_route_decode_step that also writes the mask's live keys as
 * segments (new; the reference has no counterpart: its attend_step walks the
 * whole mask, src/backend/cuda/decode_ops.cu:112-195). The mask is written as
 * before. */
UOCR_ROCM_API int uocr_rocm_route_decode_step_segments(
    void* stream, const float* rq, const float* rk, const float* q_norm, const float* k_norm, float eps,
    const float* inv_tok, int64_t n_tok, const float* inv_page, int64_t page_mod, const float* head_cls,
    float* router_keys, float* summaries, int64_t d, const int64_t* block_min, const int64_t* block_max,
    int64_t prompt_blocks, const uocr_rocm_step_state* state, const uocr_rocm_route_params* params, int64_t capacity,
    float* mask, float* z_out, float* rqk_out, int32_t* segments);

/* ---- fused decode-step ops (new) ---------------------------------------------
 * One launch where the reference's decode step makes several; each gives
 * bitwise the result of the unfused entry points it replaces. */

/* The step's token embedding fused with the first norm:
 *   x = widen(table[state->token]) (+ delta; delta null: no add);
 *   h = w * (x * inv(x)),  one row of `cols`.
 * x and h are written (bf16 variant: rounded once). Bitwise uocr_rocm_embed_step
 * then uocr_rocm_add_rms_norm (or, without delta, a copy and
 * uocr_rocm_rms_norm). A token outside [0, table_rows) gives a zero
 * embedding when table_rows >= 0. Replaces embed_step + copy + rms_norm at
 * the top of decode_body (src/model/cuda/cuda_decode_step.cpp:50-55). */
UOCR_ROCM_API int uocr_rocm_embed_add_rms_norm_step(void* stream, const uint16_t* table, int64_t table_rows,
                                                    const uocr_rocm_step_state* state, const float* delta,
                                                    const float* w, float* x, float* h, int64_t cols, float eps);
UOCR_ROCM_API int uocr_rocm_embed_add_rms_norm_step_bf16(void* stream, const uint16_t* table, int64_t table_rows,
                                                         const uocr_rocm_step_state* state, const uint16_t* delta,
                                                         const float* w, uint16_t* x, uint16_t* h, int64_t cols,
                                                         float eps);

/* add + RMSNorm feeding a bf16 GEMV:
 *   s = x + delta (delta null: s = x);  x_out = s (null: not written);
 *   h = w_norm * (s * inv(s)) (w_norm null: h = s);  h_out = h (null: not written);
 *   y[n] = bf16(h) . w[n, :] (+ bias[n]).
 * Bitwise uocr_rocm_add_rms_norm (or uocr_rocm_rms_norm) then
 * uocr_rocm_gemv_bf16 on h. k is a multiple of 8 in [8, 2048]; every pointer
 * 16-byte aligned; x_out and h_out must not overlap x or delta (every
 * workgroup reads the input row). Replaces add_inplace + copy + rms_norm +
 * apply_weight of the decode step (src/model/cuda/cuda_decode_step.cpp:
 * 18-20,54-59,65-69: the layer's input norm and its projections, the final
 * norm and the LM head). */
UOCR_ROCM_API int uocr_rocm_add_rms_norm_gemv_bf16(void* stream, const float* x, const float* delta, float* x_out,
                                                   const float* w_norm, float eps, float* h_out, int64_t k,
                                                   const uint16_t* w, int64_t n, const float* bias, float* y);

/* The same prologue feeding a gate/up pair with a SwiGLU epilogue:
 *   act[r] = silu(bf16(h) . w_gate[r, :]) * (bf16(h) . w_up[r, :]),  r < ffn.
 * Bitwise the two GEMVs then uocr_rocm_silu_mul. Replaces the residual add,
 * post-attention norm, gate/up projections and silu_mul of the decode step
 * (src/model/cuda/cuda_decode_step.cpp:57-61, cuda_decoder.cpp:119-124). */
UOCR_ROCM_API int uocr_rocm_add_rms_norm_swiglu_gemv_bf16(void* stream, const float* x, const float* delta,
                                                          float* x_out, const float* w_norm, float eps, float* h_out,
                                                          int64_t k, const uint16_t* w_gate, const uint16_t* w_up,
                                                          int64_t ffn, float* act);

/* uocr_rocm_add_rms_norm_swiglu_gemv_bf16 (h_out may be null) and, in the
 * same launch, the router's logits [experts] = router [experts, k] (fp32)
 * . h with h unrounded: bitwise that call followed by uocr_rocm_gemv_f32
 * on h, no bias (the shared experts' gate/up and the gate projection of
 * cuda_decoder.cpp:137-146, which read the same normed row). New: no
 * counterpart op in the reference. ffn >= 1, experts in [1, 2^20]. */
UOCR_ROCM_API int uocr_rocm_add_rms_norm_swiglu_router_gemv_bf16(
    void* stream, const float* x, const float* delta, float* x_out, const float* w_norm, float eps, float* h_out,
    int64_t k, const uint16_t* w_gate, const uint16_t* w_up, int64_t ffn, float* act, const float* router,
    int64_t experts, float* logits);

/* rope on q [heads * hd] and the step's new key k_row [heads * hd] at
 * (state->tok, state->page), append of the rotated key and v_row at
 * state->pos (positions outside [0, capacity) append nothing), and the
 * masked attention of the rotated query over keys 0..pos, in the two
 * launches of uocr_rocm_attend_step. q, k_row and v_row are not modified.
 * Bitwise uocr_rocm_rope_qk_step, two uocr_rocm_append_step and
 * uocr_rocm_attend_step (with rotated copies of q and k_row). hd even,
 * at most 256; rope tables as uocr_rocm_rope_step (n_tok token pairs, the
 * rest page pairs). Replaces the rope_step, append_step and attend_step
 * calls of decode_attention (src/model/cuda/cuda_decode_step.cpp:27-28,
 * 31-32,42-43). */
UOCR_ROCM_API int uocr_rocm_attend_rope_kv_step(void* stream, const float* q, const float* k_row,
                                                const float* v_row, float* k_cache, float* v_cache, int64_t heads,
                                                int64_t hd, const float* mask, float scale,
                                                const uocr_rocm_step_state* state, const float* inv_tok,
                                                int64_t n_tok, const float* inv_page, int64_t page_mod,
                                                float* scratch, int64_t capacity, float* out);
/* The same over a bf16 cache: the rotated key and the value are rounded to
 * bf16 as they are appended and scored as the cache holds them. Bitwise
 * uocr_rocm_rope_qk_step, two uocr_rocm_append_step_bf16 and
 * uocr_rocm_attend_step_bf16. */
UOCR_ROCM_API int uocr_rocm_attend_rope_kv_step_bf16(void* stream, const float* q, const float* k_row,
                                                     const float* v_row, uint16_t* k_cache, uint16_t* v_cache,
                                                     int64_t heads, int64_t hd, const float* mask, float scale,
                                                     const uocr_rocm_step_state* state, const float* inv_tok,
                                                     int64_t n_tok, const float* inv_page, int64_t page_mod,
                                                     float* scratch, int64_t capacity, float* out);

/* uocr_rocm_attend_rope_kv_step over the live keys of a routed step
 * (segments from uocr_rocm_route_decode_step_segments) instead of a mask: the
 * same rope, appends and attention, each split walking a run of the live keys
 * (new; the mask-walking attend_step of the reference,
 * src/backend/cuda/decode_ops.cu:112-195, reads every mask entry). max_live:
 * the most live keys any call of this launch shape has ((max(top_k, 1) +
 * local_blocks) * block_size for the block router); it fixes the split count,
 * so a captured step keeps its launch shape. scratch holds
 * uocr_rocm_attend_segments_scratch_floats(heads, hd, max_live) floats. With
 * out null the splits' records stay in scratch, unmerged, for
 * uocr_rocm_attend_merge_gemv_bf16. */
UOCR_ROCM_API int64_t uocr_rocm_attend_segments_scratch_floats(int64_t heads, int64_t hd, int64_t max_live);
UOCR_ROCM_API int uocr_rocm_attend_rope_kv_step_segments(void* stream, const float* q, const float* k_row,
                                                         const float* v_row, float* k_cache, float* v_cache,
                                                         int64_t heads, int64_t hd, const int32_t* segments,
                                                         int64_t max_live, float scale,
                                                         const uocr_rocm_step_state* state, const float* inv_tok,
                                                         int64_t n_tok, const float* inv_page, int64_t page_mod,
                                                         float* scratch, int64_t capacity, float* out);
/* The same over a bf16 cache (as uocr_rocm_attend_rope_kv_step_bf16). */
UOCR_ROCM_API int uocr_rocm_attend_rope_kv_step_segments_bf16(void* stream, const float* q, const float* k_row,
                                                              const float* v_row, uint16_t* k_cache,
                                                              uint16_t* v_cache, int64_t heads, int64_t hd,
                                                              const int32_t* segments, int64_t max_live, float scale,
                                                              const uocr_rocm_step_state* state,
                                                              const float* inv_tok, int64_t n_tok,
                                                              const float* inv_page, int64_t page_mod, float* scratch,
                                                              int64_t capacity, float* out);
/* y = bf16(merge) . w^T (+ bias), w bf16 [n, heads * hd], where merge is
 * the attention row that uocr_rocm_attend_rope_kv_step_segments (called with
 * out null and the same heads, hd and max_live) left as split records in
 * scratch: bitwise its own merge followed by uocr_rocm_gemv_bf16, in one
 * launch (new; the reference's decode step runs attend_step, whose last
 * kernel merges the splits, then the o projection's gemv_bf16,
 * src/model/cuda/cuda_decode_step.cpp:42-44). heads * hd a multiple of 8, at
 * most 2048. x_out (optional, [heads * hd]) receives the merged row. */
UOCR_ROCM_API int uocr_rocm_attend_merge_gemv_bf16(void* stream, const float* scratch, int64_t heads, int64_t hd,
                                                   int64_t max_live, const uint16_t* w, int64_t n, const float* bias,
                                                   float* y, float* x_out);

/* ---- mixture of experts at decode ------------------------------------------ */

/* The gate's routing (src/backend/cuda/ops.h:77-81, the rule of
 * src/model/feed_forward.cpp:36-53): softmax over each row of logits
 * [rows, experts], then the k highest scores, the lower index first on a
 * tie, as ids [rows, k] (descending) and their unnormalised scores weights
 * [rows, k]. experts <= 128, 1 <= k <= experts. A row of -inf logits scores
 * every expert 0. */
UOCR_ROCM_API int uocr_rocm_expert_topk(void* stream, const float* logits, int64_t rows, int64_t experts, int64_t k,
                                        int64_t* ids, float* weights);

/* Floats of scratch that uocr_rocm_expert_ffn_one needs: k * ffn. */
UOCR_ROCM_API int64_t uocr_rocm_expert_scratch_floats(int64_t k, int64_t ffn);

/* One decode row x [hidden] through its k routed experts (ops.h:82-90;
 * gemv_ops.cu:144-191), weights stacked by expert: gate/up
 * [experts * ffn, hidden], down [experts * hidden, ffn] bf16:
 *   out[c] = sum_j weights[j] (down[ids[j]] [c] . bf16(act_j)),
 *   act_j = silu(gate[ids[j]] . bf16(x)) * (up[ids[j]] . bf16(x)).
 * Bitwise, per slot, uocr_rocm_add_rms_norm_swiglu_gemv_bf16 (no norm) on
 * the expert's gate/up rows and uocr_rocm_gemv_bf16 on its down rows, the
 * products summed in slot order as w * d then +. New beside the reference's
 * signature: `experts` (an id outside [0, experts) contributes nothing),
 * `base` (null, or a vector added last: out[c] = base[c] + sum, bitwise
 * the shared experts' output followed by add_inplace of the routed sum,
 * cuda_decoder.cpp:149-151; base may be out itself) and `scratch`
 * (uocr_rocm_expert_scratch_floats(k, ffn) floats for act), so the call
 * allocates nothing. hidden and ffn multiples of 8 in [8, 2048],
 * k <= 8 and k * ffn <= 8192; two launches. */
UOCR_ROCM_API int uocr_rocm_expert_ffn_one(void* stream, const float* x, int64_t hidden, int64_t ffn,
                                           const uint16_t* gate, const uint16_t* up, const uint16_t* down,
                                           int64_t experts, const int64_t* ids, const float* weights, int64_t k,
                                           const float* base, float* scratch, float* out);

/* The mixture-of-experts MLP of a decode row after its shared experts'
 * gate/up and its router logits [experts] (uocr_rocm_gemv_f32): the top k
 * of the logits as uocr_rocm_expert_topk forms them (written to ids and
 * weights), the routed experts as uocr_rocm_expert_ffn_one, and the shared
 * experts' down product (shared_down [hidden, shared_ffn] against
 * bf16(shared_act)) formed in the same launch as the routed down products:
 * out = shared + routed. Bitwise uocr_rocm_expert_topk, then
 * uocr_rocm_gemv_bf16(shared_act, shared_down), then uocr_rocm_expert_ffn_one
 * with that as base (cuda_decoder.cpp:137-152, whose top-k launch, shared
 * down GEMV and add_inplace this folds in); two launches. experts <= 128,
 * shared_ffn a multiple of 8 in [8, 2048], k * ffn + shared_ffn <= 8192. */
UOCR_ROCM_API int uocr_rocm_moe_ffn_one(void* stream, const float* x, int64_t hidden, int64_t ffn,
                                       const uint16_t* gate, const uint16_t* up, const uint16_t* down,
                                       int64_t experts, const float* logits, int64_t k, int64_t* ids, float* weights,
                                       const float* shared_act, const uint16_t* shared_down, int64_t shared_ffn,
                                       float* scratch, float* out);

/* y[n] = x . w[n, :] (+ bias[n]) with fp32 weights, x not rounded: the
 * mixture-of-experts gate logits, which the reference forms from fp32 gate
 * weights with an fp32 GEMM (moe_gate_f32, src/model/cuda/cuda_decoder.cpp:
 * 141-142; linear, src/backend/reference/ops.cpp:91-108). */
UOCR_ROCM_API int uocr_rocm_gemv_f32(void* stream, const float* x, int64_t k, const float* w, int64_t n,
                                     const float* bias, float* y);

#ifdef __cplusplus
}
#endif

#endif /* UOCR_ROCM_H_ */
