/*
 * needle_hip.h -- C ABI of libneedle_hip.so, the MI355X (gfx950) decode
 * backend for needle.js.
 *
 * The ABI is flat C: opaque handles, plain pointers and sizes.  Every call
 * returns an nd_status; on failure nd_last_error(ctx) holds a message.  The
 * host binding maps ND_ERR_INVALID to NeedleError("INVALID_CACT"),
 * ND_ERR_OVERFLOW to NeedleError("CONTEXT_OVERFLOW") and every other failure
 * to NeedleError("BACKEND_UNAVAILABLE") (errors.ts:1-32).
 *
 * Two flavours of each operator exist:
 *   - host-pointer calls (no suffix) copy inputs to HBM, run, copy results
 *     back and synchronise -- the shape of InferenceBackend's synchronous
 *     methods (backend.ts:82-110);
 *   - device-pointer calls (suffix _d) take HBM pointers and a HIP stream
 *     (NULL = the context's own stream) and only enqueue work; the caller
 *     synchronises (nd_sync or its own stream sync).
 *
 * Reference paths are relative to packages/needle.js/src/ of needle.js.
 * A context is used by one host thread at a time (the reference runtime
 * awaits every backend call in sequence, runtime.ts:613-632).
 */
#ifndef NEEDLE_HIP_H
#define NEEDLE_HIP_H

#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

typedef int32_t nd_status;
#define ND_OK 0
#define ND_ERR_INVALID 1     /* bad shape, range or id: INVALID_CACT */
#define ND_ERR_BACKEND 2     /* HIP failure, no device, disposed: BACKEND_UNAVAILABLE */
#define ND_ERR_OVERFLOW 3    /* position beyond the runtime length: CONTEXT_OVERFLOW */
#define ND_ERR_NOMEM 4       /* HBM allocation failed: BACKEND_UNAVAILABLE */

typedef struct nd_ctx nd_ctx;
typedef struct nd_mat nd_mat;
typedef struct nd_kv nd_kv;

/* ------------------------------------------------------------ lifecycle */

/* Creates a backend context on HIP device `device`.  Replaces backend
 * construction in resolveBackend (model/model.ts:162-200) and the device
 * acquisition of createTypeGPUBackend (backends/typegpu.ts:155-205). */
nd_status nd_create(int32_t device, nd_ctx** out);

/* Frees every matrix, cache and buffer of the context.  Idempotent on NULL.
 * InferenceBackend.dispose (backends/backend.ts:109). */
nd_status nd_destroy(nd_ctx* ctx);

/* Message of the last failure on this context ("" if none).  With ctx ==
 * NULL returns the message of the last failed nd_create. */
const char* nd_last_error(const nd_ctx* ctx);

/* Waits for all work enqueued on the context's stream. */
nd_status nd_sync(nd_ctx* ctx);

/* The context's HIP stream (a hipStream_t), for callers that enqueue _d
 * calls and time them with events. */
void* nd_stream(nd_ctx* ctx);

/* ------------------------------------------------------------- weights */

/* Uploads one int8 matrix: W int8 [n][k] row-major, scales f32 [n][k/g]
 * (one scale per row and group of g columns; g == k gives per-row scales).
 * Requires k % g == 0, g % 16 == 0, k % 16 == 0.  This is the int8 form of
 * CqMatrix (model/cact.ts:61-75); the backend caches it in HBM the way the
 * TypeGPU backend uploads each matrix once (backends/typegpu.ts:390-410). */
nd_status nd_mat_upload_i8(nd_ctx* ctx, const int8_t* w, const float* scales, uint32_t n,
                           uint32_t k, uint32_t g, nd_mat** out);

/* Same, from HBM pointers (the matrix keeps its own copy). */
nd_status nd_mat_upload_i8_d(nd_ctx* ctx, const int8_t* w_dev, const float* scales_dev,
                             uint32_t n, uint32_t k, uint32_t g, nd_mat** out);

nd_status nd_mat_free(nd_ctx* ctx, nd_mat* mat);

/* HBM addresses of a matrix's codes and scales (for building graphs). */
nd_status nd_mat_info(const nd_mat* mat, const int8_t** w_dev, const float** scales_dev,
                      uint32_t* n, uint32_t* k, uint32_t* g);

/* ------------------------------------------------- a1: quantized matvec */

/* y[b][r - row_start] = sum_g s[r][g] * sum_{c in g} W[r][c] * x[b][c] for
 * rows [row_start, row_start + row_count) and b < batch; x is [batch][k],
 * y is [batch][row_count].  InferenceBackend.matvec with a MatrixRowRange
 * (backends/backend.ts:88-93, backends/cpu.ts:12-16; arithmetic of
 * backends/cq.ts:106-156).  batch > 1 is the batched-activation form. */
nd_status nd_matvec(nd_ctx* ctx, const nd_mat* mat, const float* x, uint32_t batch,
                    uint32_t row_start, uint32_t row_count, float* y);
nd_status nd_matvec_d(nd_ctx* ctx, const nd_mat* mat, const float* x_dev, uint32_t batch,
                      uint32_t row_start, uint32_t row_count, float* y_dev, void* stream);

/* One matvec request of a batch: MatvecRequest (backends/backend.ts:11-15). */
typedef struct nd_matvec_job {
  const nd_mat* mat;
  const float* x;      /* host pointer, [k] */
  uint32_t row_start;
  uint32_t row_count;
  float* y;            /* host pointer, [row_count] */
} nd_matvec_job;

/* Runs independent matvecs with one host synchronisation.
 * InferenceBackend.matvecBatch (backends/backend.ts:95-101). */
nd_status nd_matvec_batch(nd_ctx* ctx, const nd_matvec_job* jobs, uint32_t count);

/* out[c] = W[row][c] * s[row][c / g] for c < k.  InferenceBackend.row
 * (backends/backend.ts:106-107; backends/cq.ts:243-295). */
nd_status nd_row(nd_ctx* ctx, const nd_mat* mat, uint32_t row, float* out);
nd_status nd_row_d(nd_ctx* ctx, const nd_mat* mat, uint32_t row, float* out_dev, void* stream);

/* --------------------------------------- a2/a3: int8 KV cache, attention */

#define ND_KV_INT8 0
#define ND_KV_FLOAT32 1

/* Allocates a zeroed cache in HBM: codes [layers][kv_heads][alloc][head_dim]
 * (int8, or f32 in ND_KV_FLOAT32 mode) and scales [layers][kv_heads][alloc]
 * with alloc = window > 0 ? min(max_length, sink + window) : max_length and
 * sink clamped to max_length.  Mirrors NeedleRuntime.reset's allocation
 * (model/runtime.ts:150-205) and ResidentExecutionSession.reset
 * (backends/backend.ts:67).  head_dim must be 64. */
nd_status nd_kv_create(nd_ctx* ctx, uint32_t layers, uint32_t kv_heads, uint32_t head_dim,
                       uint32_t max_length, uint32_t sink, uint32_t window, uint32_t mode,
                       nd_kv** out);
nd_status nd_kv_free(nd_ctx* ctx, nd_kv* kv);

/* Zeroes codes and scales (a fresh runtime.reset without reallocation). */
nd_status nd_kv_clear(nd_ctx* ctx, nd_kv* kv);

/* Slots per (layer, head) and the HBM addresses of the cache arrays. */
nd_status nd_kv_info(const nd_kv* kv, uint32_t* alloc, void** k_codes_dev, void** v_codes_dev,
                     float** k_scales_dev, float** v_scales_dev);

/* Quantizes and stores `count` consecutive positions [position, position +
 * count) of one layer.  k, v are [count][kv_heads][head_dim] f32.  Per
 * vector: m = max(1e-12, max|x|) and s = m / 127 in float64, stored scale
 * f32(s), code = roundTiesToEven(x / s) with a float64 division -- bit-exact
 * with NeedleRuntime.#storeKV (model/runtime.ts:679-717, 901-907) and its
 * slot map #kvSlot (:659-664).  Within one call a later position that maps
 * to the same ring slot wins, as with sequential stores.  count == 1 is the
 * decode append; count > 1 is the bulk append of a prefill. */
nd_status nd_kv_store(nd_ctx* ctx, nd_kv* kv, uint32_t layer, uint32_t position, uint32_t count,
                      const float* k, const float* v);
nd_status nd_kv_store_d(nd_ctx* ctx, nd_kv* kv, uint32_t layer, uint32_t position,
                        uint32_t count, const float* k_dev, const float* v_dev, void* stream);

/* Copies one (layer, head)'s codes [alloc][head_dim] and scales [alloc] to
 * the host (codes are int8, or f32 in ND_KV_FLOAT32 mode). */
nd_status nd_kv_read(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t head,
                     void* k_codes, void* v_codes, float* k_scales, float* v_scales);

/* Single-query attention of query position `position` over the visible
 * positions [0, min(sink, position + 1)) and [max(prefix, position + 1 -
 * window), position] (all of [0, position] when window == 0).  q and out are
 * [q_heads][head_dim]; query head h reads KV head h / (q_heads / kv_heads);
 * scores are q.k * scale_k / sqrt(head_dim), softmax, out = sum w * v *
 * scale_v.  NeedleRuntime.#attention (model/runtime.ts:719-786) with
 * softmaxInPlace (model/math.ts:46-60). */
nd_status nd_attention(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                       const float* q, uint32_t q_heads, float* out);
nd_status nd_attention_d(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                         const float* q_dev, uint32_t q_heads, float* out_dev, void* stream);

/* ------------------------------------------- a4: masked argmax selection */

/* selectToken (model/runtime.ts:880-899) with argmax (model/math.ts:140-151)
 * and logSoftmaxAt (model/math.ts:153-160): allowed == NULL selects the
 * first maximum of all logits; otherwise the first maximum over `allowed` in
 * list order (strict '>', so ties keep the earlier entry; a NaN first entry
 * is kept, later NaNs never win).  log_probability = logit - max - log(sum
 * exp(logit - max)) over the full vocabulary in float64.  An empty list or an
 * id >= vocab is ND_ERR_INVALID. */
nd_status nd_select(nd_ctx* ctx, const float* logits, uint32_t vocab, const uint32_t* allowed,
                    uint32_t count, uint32_t* id, double* log_probability);

/* Batched selection over `batch` rows of logits [batch][vocab] with an
 * optional allowed-id bitmask [batch][ceil(vocab/32)] (bit id&31 of word
 * id>>5; NULL = unconstrained).  The bitmask is the ascending allowed list
 * that Needle.complete builds (tools/agent.ts:164-183).  Writes ids[batch]
 * and log_probabilities[batch] in HBM; a row whose mask is empty gets id
 * 0xFFFFFFFF and log-probability NaN. */
nd_status nd_select_mask_d(nd_ctx* ctx, const float* logits_dev, uint32_t batch, uint32_t vocab,
                           const uint32_t* mask_dev, uint32_t* ids_dev,
                           double* log_probabilities_dev, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* NEEDLE_HIP_H */
