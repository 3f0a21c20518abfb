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
#define ND_ERR_UNSUPPORTED 5 /* valid record this backend does not run: UNSUPPORTED_CACT */

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

/* Workgroup placement, no counterpart in the reference.  Several kernels
 * hand partial results between the workgroups of one launch through one
 * XCD's L2 (the attention chunk merge, the k-slice matvec sum, the split-k
 * GEMM sum, the Needle 2 fused layer launch); that needs the dispatcher to
 * place workgroup L of a launch on the XCD of workgroup L % 8.  nd_create
 * checks this on its device (every workgroup of three probe launches reads
 * its XCC id); when it does not hold, those kernels run their agent-scope
 * forms (and Needle 2 its separate layer launches) instead.  *probed
 * (when not NULL) receives 1 when every device probed so far passed.
 * Test hook: enable == 0 selects the agent-scope forms although the probe
 * passed, enable == 1 restores the probe's choice; it applies to launches
 * enqueued (and Needle 2 step graphs captured) after the call, process-wide. */
nd_status nd_test_xcd_local(nd_ctx* ctx, int32_t enable, uint32_t* probed);

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

/* Uploads one Cactus-Quant matrix as the archive stores it (CqMatrix,
 * model/cact.ts:61-75, parsed at cact.ts:346-396): packed codes
 * [n][row_bytes] with row_bytes = kpad * pb / 8 (kpad = k rounded up to a
 * multiple of g, pb = bits, or 2 for the ternary width bits = 5), binary16
 * norms [n][kpad / g], and the width's codebook (2^bits floats: the
 * archive's entries [0, 4) for CQ2, [4, 12) for CQ3, [12, 28) for CQ4,
 * cact.ts:272-276; ignored and may be NULL for ternary).  Codes are read
 * low bits first; 3-bit rows are one little-endian bit stream.  The matrix
 * works with nd_matvec / nd_matvec_d / nd_matvec_batch (cqMatvec,
 * backends/cq.ts:106-231: per-group Walsh-Hadamard input rotation, then the
 * codebook dot products times the group norms) and nd_row / nd_row_d
 * (dequantizeCqRow, cq.ts:234-295); nd_matmul and the model builders take
 * int8 matrices only.  g must be a power of two (else ND_ERR_UNSUPPORTED,
 * as cact.ts:350-359); this backend further needs g >= 8 and kpad <= 8192
 * after rounding up to a multiple of 32 (ND_ERR_UNSUPPORTED otherwise).
 * Calls on one context share one buffer of rotated inputs: enqueue them on
 * one stream. */
nd_status nd_mat_upload_cq(nd_ctx* ctx, const uint8_t* packed, const uint16_t* norms,
                           const float* codebook, uint32_t n, uint32_t k, uint32_t g,
                           uint32_t bits, nd_mat** out);

/* Width (0 for int8 matrices), stored row width in codes (kpad rounded up
 * to a multiple of 32) and stored packed row bytes. */
nd_status nd_mat_cq_info(const nd_mat* mat, uint32_t* bits, uint32_t* kpad, uint32_t* row_bytes);

/* HBM addresses of a matrix's codes and scales (for building graphs). */
nd_status nd_mat_info(const nd_mat* mat, const int8_t** w_dev, const float** scales_dev,
                      uint32_t* n, uint32_t* k, uint32_t* g);

/* ------------------------------------------------- a1: quantized matvec */

/* y[b][r - row_start] = sum_g s[r][g] * sum_{c in g} W[r][c] * x[b][c] for
 * rows [row_start, row_start + row_count) and b < batch; x is [batch][k],
 * y is [batch][row_count].  InferenceBackend.matvec with a MatrixRowRange
 * (backends/backend.ts:88-93, backends/cpu.ts:12-16; arithmetic of
 * backends/cq.ts:106-156).  batch > 1 is the batched-activation form.
 * Batches of 3 or more on int8 matrices (g a multiple of 32) share the
 * context's workspace of partial sums and arrival counters: enqueue such
 * calls of one context on one stream. */
nd_status nd_matvec(nd_ctx* ctx, const nd_mat* mat, const float* x, uint32_t batch,
                    uint32_t row_start, uint32_t row_count, float* y);
nd_status nd_matvec_d(nd_ctx* ctx, const nd_mat* mat, const float* x_dev, uint32_t batch,
                      uint32_t row_start, uint32_t row_count, float* y_dev, void* stream);

/* y[m][n] = s[n] * sum_c W[n][c] * x[m][c] for m < rows on int8 MFMA: the
 * batched matvec of InferenceBackend.matvec over `rows` activation vectors
 * (the skinny GEMM of batched decode and prefill).  Each fp32 row of x is
 * split exactly into three int8 digit planes with a power-of-two scale
 * (representation error <= 2^-22 of the row's largest magnitude) and every
 * plane is multiplied with int32 accumulation.  Requires per-row scales
 * (g == k), k % 64 == 0 and k <= 2048.  With accumulate != 0, y += instead. */
nd_status nd_matmul(nd_ctx* ctx, const nd_mat* mat, const float* x, uint32_t rows, float* y);
nd_status nd_matmul_d(nd_ctx* ctx, const nd_mat* mat, const float* x_dev, uint32_t rows,
                      float* y_dev, uint32_t accumulate, void* stream);

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

/* Calibration, no counterpart in the reference: reads `bytes` (a nonzero
 * multiple of 16) at the 16-byte aligned device address src with the
 * matvec's own load form (non-temporal 128-bit loads) over `blocks`
 * workgroups of 256 threads, and writes one folded word per workgroup to
 * out_dev[blocks].  Gives the read-only streaming rate the weight stream of
 * nd_matvec_d is measured against. */
nd_status nd_stream_read_d(nd_ctx* ctx, const void* src_dev, uint64_t bytes, uint32_t blocks,
                           uint32_t* out_dev, void* stream);

/* Measurement, no counterpart in the reference: nd_matvec_d for batch 1 on
 * an int8 matrix, the same kernel body and launch geometry, with each
 * workgroup's entry time and the time its stores completed (the GPU's 100 MHz
 * constant clock) written to stamps_dev[2 w], stamps_dev[2 w + 1].  The
 * workgroup count goes to *workgroups; more than `capacity` workgroups is
 * ND_ERR_INVALID with nothing launched.  The span from the earliest entry
 * to the latest exit is the kernel's body time. */
nd_status nd_matvec_stamped_d(nd_ctx* ctx, const nd_mat* mat, const float* x_dev,
                              uint32_t row_start, uint32_t row_count, float* y_dev,
                              uint64_t* stamps_dev, uint32_t capacity, uint32_t* workgroups,
                              void* stream);

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
 * softmaxInPlace (model/math.ts:46-60).  A long visible range is split over
 * several workgroups whose partial results meet in the context's workspace
 * (partials and arrival counters): enqueue the _d calls of one context on one
 * stream. */
nd_status nd_attention(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                       const float* q, uint32_t q_heads, float* out);
nd_status nd_attention_d(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                         const float* q_dev, uint32_t q_heads, float* out_dev, void* stream);

/* Measurement, no counterpart in the reference: nd_attention_d's own launch
 * when it takes the XCD-local form with one tile per wave (8 heads x 8192
 * positions does), with thread 0 of each workgroup L reading the GPU's
 * 100 MHz constant clock at entry, after its wave's tiles, after the waves'
 * combine, once the chunk's partials are published, once its arrival is
 * counted and, for the chunk that merges, after the merge, written with
 * the chunk's role (0 counted in, 1 merged) and its XCC id to
 * stamps_dev[8 L .. 8 L + 7].  The workgroup count goes to *workgroups;
 * another launch form, or more than `capacity` workgroups, is
 * ND_ERR_UNSUPPORTED with nothing launched. */
nd_status nd_attention_stamped_d(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                                 const float* q_dev, uint32_t q_heads, float* out_dev,
                                 uint64_t* stamps_dev, uint32_t capacity, uint32_t* workgroups,
                                 void* stream);

/* nd_attention_d without any allocation, for callers that cannot allocate
 * device memory (code under HIP graph capture, tight serving loops, harnesses
 * that forbid hipMalloc).  No counterpart in the reference.  Identical
 * arguments and results; the partial results and arrival counters live in a
 * fixed per-GPU array (1,089,536 bytes, set up by nd_create) instead of the
 * context's workspace, so q_heads is limited to 64 (ND_ERR_INVALID above).
 * Every call on one GPU shares that array: calls that overlap on one GPU --
 * from any context or stream -- race and must be ordered by the caller. */
nd_status nd_attention_static_d(nd_ctx* ctx, const nd_kv* kv, uint32_t layer, uint32_t position,
                                const float* q_dev, uint32_t q_heads, float* out_dev,
                                void* stream);

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
 * 0xFFFFFFFF and log-probability NaN.  Calls on one context share its
 * selection workspace: calls on different streams must not overlap. */
nd_status nd_select_mask_d(nd_ctx* ctx, const float* logits_dev, uint32_t batch, uint32_t vocab,
                           const uint32_t* mask_dev, uint32_t* ids_dev,
                           double* log_probabilities_dev, void* stream);

/* --------------------------------- batched decoder (int8 MFMA, int8 KV) */

typedef struct nd_decoder nd_decoder;
typedef struct nd_batch nd_batch;

/* A decoder built from the reference's per-token primitives: embedding row
 * x sqrt(dim) (model/runtime.ts:305-309); per layer a = rmsNorm(x, attn_norm)
 * (model/math.ts:16-32), q/k/v = Wq/Wk/Wv a, per-head rmsNormSlice with
 * q_norm/k_norm and half-split RoPE (model/runtime.ts:471-500,
 * model/math.ts:94-115), #storeKV and #attention (model/runtime.ts:679-786),
 * x += Wo o, x += Wdown silu(Wup rmsNorm(x, ffn_norm)) (model/math.ts:12-14);
 * logits = embedding . rmsNorm(x, final_norm) (model/runtime.ts:570-577).
 * All matrices are per-row-scaled int8 (g == k) uploaded with
 * nd_mat_upload_i8; norm vectors are host arrays copied at creation.
 * Limits: head_dim 64, heads * 64 == dim, dim and ffn multiples of 64 and at
 * most 2048, heads / kv_heads in {1, 2, 4, 8}. */
typedef struct nd_decoder_desc {
  uint32_t layers, dim, heads, kv_heads, head_dim, ffn, vocab;
  float rope_theta;
  const nd_mat* embedding;            /* [vocab][dim]; tied output projection */
  const nd_mat* const* wq;            /* layers entries, [heads*64][dim] */
  const nd_mat* const* wk;            /* [kv_heads*64][dim] */
  const nd_mat* const* wv;            /* [kv_heads*64][dim] */
  const nd_mat* const* wo;            /* [dim][heads*64] */
  const nd_mat* const* wup;           /* [ffn][dim] */
  const nd_mat* const* wdown;         /* [dim][ffn] */
  const float* attn_norm;             /* [layers][dim] */
  const float* ffn_norm;              /* [layers][dim] */
  const float* q_norm;                /* [layers][64] */
  const float* k_norm;                /* [layers][64] */
  const float* final_norm;            /* [dim] */
} nd_decoder_desc;

/* The matrices stay owned by the caller and must outlive the decoder. */
nd_status nd_decoder_create(nd_ctx* ctx, const nd_decoder_desc* desc, nd_decoder** out);
nd_status nd_decoder_free(nd_ctx* ctx, nd_decoder* dec);

/* `batch` independent sequences decoding together (no batch API exists in the
 * reference: one NeedleRuntime is one sequence, model/runtime.ts:108-140; this
 * is the additive batch extension of the backend).  Owns an int8 KV cache of
 * max_length positions per sequence (no window, no sinks) and all step
 * buffers, allocated once here. */
nd_status nd_batch_create(nd_ctx* ctx, nd_decoder* dec, uint32_t batch, uint32_t max_length,
                          nd_batch** out);
nd_status nd_batch_free(nd_ctx* ctx, nd_batch* batch);

/* The batch's KV cache: sequence s, KV head h is cache head s * kv_heads + h
 * (read it with nd_kv_read). */
nd_kv* nd_batch_kv(nd_batch* batch);

/* Fills positions [0, length) of sequence `seq` in every layer with
 * synthetic int8 rows: for layer l, head h, position p, element i < 64 the
 * code is ((z >> 32) * 255 >> 32) - 127 and the scale lo + (hi - lo) *
 * (z' >> 40) * 2^-24 (float64, stored f32), where z is output ((l * kv_heads
 * + h) * index_stride + p) * 65 + i of the splitmix64 stream of seed_k (K) or
 * seed_v (V), and z' is output ... * 65 + 64. */
nd_status nd_batch_fill_synthetic(nd_ctx* ctx, nd_batch* batch, uint32_t seq, uint64_t seed_k,
                                  uint64_t seed_v, uint32_t length, uint32_t index_stride,
                                  float lo, float hi);

/* Sets each sequence's current token and position and the step counter. */
nd_status nd_batch_set_state(nd_ctx* ctx, nd_batch* batch, const uint32_t* tokens,
                             const uint32_t* positions, uint32_t step);

/* Enqueues one decode step of every sequence (about 10 launches per layer, no
 * allocation, no host synchronisation; capturable in a HIP graph): each
 * sequence runs its current token at its position, appends K/V, and selects
 * the next token with selectToken semantics (model/runtime.ts:880-899); the
 * selected ids become the current tokens and positions advance by one.  With
 * use_masks, the allowed set of sequence b at step t is the bitmask whose bit
 * v is set iff (z_v >> 40) < threshold24 or v is the forced id ((z_vocab >>
 * 32) * vocab >> 32), z being the splitmix64 stream seeded by output
 * t * 65536 + b of the stream of mask_seed (t = the device step counter).
 * max_position must bound every sequence's position in this step. */
nd_status nd_batch_step(nd_ctx* ctx, nd_batch* batch, uint32_t max_position, uint32_t use_masks,
                        uint64_t mask_seed, uint32_t threshold24, void* stream);

/* Copies the current tokens (the last selected ids), positions, the last
 * step's log-probabilities and (optionally) logits [batch][vocab] to the
 * host and synchronises. */
nd_status nd_batch_read(nd_ctx* ctx, nd_batch* batch, uint32_t* tokens, uint32_t* positions,
                        double* log_probabilities, float* logits);

/* Copies the last layer's Q/K/V projections of the last step, [batch]
 * [(heads + 2 kv_heads) * 64] f32 (as nd_prefill_read_projections). */
nd_status nd_batch_read_projections(nd_ctx* ctx, nd_batch* batch, float* out);

/* ------------------------------------------------------------------ prefill */

typedef struct nd_prefill nd_prefill;

/* Buffers for prompts of up to max_tokens positions ending at or before
 * max_context.  The reference has no batched prefill: NeedleRuntime.prefill
 * is one step() per prompt token (model/runtime.ts:227-243). */
nd_status nd_prefill_create(nd_ctx* ctx, nd_decoder* dec, uint32_t max_tokens,
                            uint32_t max_context, nd_prefill** out);
nd_status nd_prefill_free(nd_ctx* ctx, nd_prefill* prefill);

/* Runs `count` prompt tokens at positions [position0, position0 + count)
 * through the decoder in one pass: M-row int8-MFMA GEMMs, every position's
 * K/V quantized into `kv` (int8, window 0, the decoder's layers and KV heads)
 * with #storeKV semantics, then causal attention of each position over [0,
 * its position] of the int8 cache -- what `count` sequential steps read,
 * since a step stores its own K/V before attending (model/runtime.ts:501-502).
 * Writes the last position's logits [vocab] when logits != NULL. */
nd_status nd_prefill_tokens(nd_ctx* ctx, nd_prefill* prefill, nd_kv* kv, const uint32_t* tokens,
                            uint32_t count, uint32_t position0, float* logits);

/* The same in three parts, for callers that time or capture the device work:
 * upload the tokens, enqueue the pass (no allocation, no synchronisation),
 * then copy the logits. */
nd_status nd_prefill_set_tokens(nd_ctx* ctx, nd_prefill* prefill, const uint32_t* tokens,
                                uint32_t count, uint32_t position0);
nd_status nd_prefill_run_d(nd_ctx* ctx, nd_prefill* prefill, nd_kv* kv, void* stream);
nd_status nd_prefill_logits(nd_ctx* ctx, nd_prefill* prefill, float* logits);

/* Runs the pass once on the context's stream with an event after every
 * kernel and returns the summed kernel times by kind: ms[0] the int8 GEMMs
 * (projections and lm head), ms[1] the causal attention, ms[2] the rest
 * (embedding, digit planes, norms, RoPE and the K/V store).  Synchronises.
 * Calibration, no counterpart in the reference. */
nd_status nd_prefill_phase_ms(nd_ctx* ctx, nd_prefill* prefill, nd_kv* kv, float* ms);

/* Copies the last layer's Q/K/V projections of the last pass -- [count]
 * [(heads + 2 kv_heads) * 64] f32, rows q | k | v before the per-head norms
 * and RoPE -- so that a caller can check that the codes stored for the last
 * layer are #storeKV of the values this backend computed (no counterpart in
 * the reference: a read-back of device state, like nd_kv_read). */
nd_status nd_prefill_read_projections(nd_ctx* ctx, nd_prefill* prefill, float* out);

/* Every step records its selected ids and log-probabilities at row t (the
 * step counter) of a [max_length][batch] history in HBM; copies rows
 * [first_step, first_step + steps) to the host and synchronises. */
nd_status nd_batch_history(nd_ctx* ctx, nd_batch* batch, uint32_t first_step, uint32_t steps,
                           uint32_t* ids, double* log_probabilities);

/* ------------------------------------------------------- Needle 2 (batch 1) */

typedef struct nd_needle nd_needle;

/* Needle 2 geometry and weights (model/cact.ts geometry fields; the per-layer
 * tensors read by NeedleRuntime.step, model/runtime.ts:280-583).  Every
 * matrix takes one form, owned by the caller (it must outlive the model):
 * either per-row-scaled int8 (g == k, nd_mat_upload_i8), or -- the shipped
 * archive's form, model/cact.ts:398-562 -- Cactus-Quant (nd_mat_upload_cq),
 * all of the embedding's width and group size, groups of at most 2048 and
 * engram rows of at most 1024 padded codes; a Cactus-Quant model runs every
 * product as cqMatvec and every row gather as dequantizeCqRow
 * (backends/cq.ts:106-295), its prompts in the same batched passes as an
 * int8 model's.  Dense vectors are host arrays copied at creation.
 *   embedding  [vocab][dim], tied output projection (runtime.ts:570-577)
 *   wq, wgate  layers entries of [heads*64][dim]; wk, wv [kv_heads*64][dim]
 *   wo         [dim][heads*64]
 *   phi_pre    [layers*lanes][lanes*dim], phi_post likewise,
 *   phi_res    [layers*lanes*lanes][lanes*dim] (runtime.ts:385-420)
 *   eg_tables  n_sites entries of [engram_tables*engram_slots][engram_sub]
 *   eg_key, eg_value  n_sites entries of [dim][engram_tables*engram_sub]
 * Limits: head_dim 64, lanes <= 4, dim a power of two in [128, 512],
 * hadamard a power of two in [dim, 512], heads / kv_heads in {1, 2, 4, 8}, n_sites <= 4,
 * engram_tables <= 16 and a multiple of n_orders. */
typedef struct nd_needle_desc {
  uint32_t vocab, dim, heads, kv_heads, layers, head_dim, max_length, hadamard, lanes;
  uint32_t kv_window;                  /* 0 = no sliding window */
  uint32_t engram_slots, engram_sub, engram_tables, engram_taps;
  uint32_t n_orders, orders[4];        /* engram n-gram orders */
  uint32_t n_sites, sites[4];          /* layers that inject an engram */
  float rope_theta;
  const nd_mat* embedding;
  const nd_mat* const* wq;
  const nd_mat* const* wk;
  const nd_mat* const* wv;
  const nd_mat* const* wgate;
  const nd_mat* const* wo;
  const nd_mat* phi_pre;
  const nd_mat* phi_post;
  const nd_mat* phi_res;
  const nd_mat* const* eg_tables;
  const nd_mat* const* eg_key;
  const nd_mat* const* eg_value;
  const float* norm_input;         /* [layers][dim] */
  const float* query_norm;         /* [layers][64] */
  const float* key_norm;           /* [layers][64] */
  const float* post_attn_norm;     /* [layers][dim] */
  const float* pre_hadamard_norm;  /* [layers][dim] */
  const float* d1;                 /* [layers][dim] */
  const float* d2;                 /* [layers][hadamard] */
  const float* d3;                 /* [layers][dim] */
  const float* attention_gate;     /* [layers] */
  const float* a_pre;              /* [layers] */
  const float* a_post;             /* [layers] */
  const float* a_res;              /* [layers] */
  const float* b_pre;              /* [layers][lanes] */
  const float* b_post;             /* [layers][lanes] */
  const float* b_res;              /* [layers][lanes][lanes] */
  const float* eg_taps;            /* [n_sites][engram_taps][dim] */
  const float* final_norm;         /* [dim] */
  /* Confidence probe head (CactProbeHead, model/cact.ts:105-112), or
   * probes == NULL for none: probes [probe_count][dim] (1..8), projection
   * [probe_out][probe_count * dim], bias [probe_out].  With a head, every
   * step pools the scaled embedding and each layer's lane mean on the
   * device (OnlineProbePool.add, model/runtime.ts:64-91, fed at
   * runtime.ts:310 and :550). */
  const float* probes;
  uint32_t probe_count, probe_out;
  const float* probe_projection;
  const float* probe_bias;
} nd_needle_desc;

nd_status nd_needle_create(nd_ctx* ctx, const nd_needle_desc* desc, nd_needle** out);
nd_status nd_needle_free(nd_ctx* ctx, nd_needle* model);

/* NeedleRuntime.reset (model/runtime.ts:150-225) and
 * ResidentExecutionSession.reset (backends/backend.ts:17-22, 67): position
 * 0, empty history and engram ring, a KV cache of min(max_length, sink +
 * kv_window) slots per (layer, KV head) (max_length without a window) in
 * the kvCache mode `kv_cache` (ND_KV_INT8 or ND_KV_FLOAT32), and the
 * confidence pool on when collect_confidence != 0 and the model has a probe
 * head.  Errors: CONTEXT_OVERFLOW when max_length is 0 or above the model's
 * max_length; UNSUPPORTED_CACT for a kvCache mode this runtime does not keep
 * (the session's reset() then returns false and the runtime keeps its own
 * cache, runtime.ts:171-205).  The first reset allocates the runtime state
 * for the model's max_length; later resets only clear it.  One reset is
 * driven either by the whole-step calls (nd_needle_step, _prefill,
 * _step_select, _generate) or by the session calls (nd_needle_begin_token
 * ... nd_needle_forward): the first call after a reset decides, and a call
 * of the other kind is INVALID_CACT until the next reset. */
nd_status nd_needle_reset(nd_ctx* ctx, nd_needle* model, uint32_t max_length, uint32_t sink,
                          uint32_t kv_cache, uint32_t collect_confidence);

/* The runtime's KV cache (read it with nd_kv_read), or NULL before reset. */
nd_kv* nd_needle_kv(nd_needle* model);
uint32_t nd_needle_position(const nd_needle* model);

/* The resident confidence (ResidentExecutionSession.residentConfidence,
 * backends/backend.ts:77; computed as NeedleRuntime.confidence,
 * model/runtime.ts:93-104, 641-645): sigmoid of output 0 of the probe head
 * over everything pooled since the last reset.  INVALID_CACT when the model
 * has no confidence head, before reset, or when the reset turned
 * collectConfidence off. */
nd_status nd_needle_confidence(nd_ctx* ctx, nd_needle* model, double* confidence);

/* NeedleRuntime.step (model/runtime.ts:280-583): runs `token` at the current
 * position and advances it; copies the logits [vocab] when logits != NULL.
 * Errors: INVALID_CACT before reset or for token >= vocab, CONTEXT_OVERFLOW
 * at the runtime limit (model/runtime.ts:288-298). */
nd_status nd_needle_step(nd_ctx* ctx, nd_needle* model, uint32_t token, float* logits);

/* NeedleRuntime.prefill (model/runtime.ts:227-243): `count` steps, the last
 * one with logits. */
nd_status nd_needle_prefill(nd_ctx* ctx, nd_needle* model, const uint32_t* tokens,
                            uint32_t count, float* logits);

/* NeedleRuntime.stepSelected (model/runtime.ts:257-278): the step, then
 * selectToken (model/runtime.ts:880-899) over `allowed` (count ascending ids,
 * or all ids when allowed == NULL) on the device; returns the id and its
 * full-vocabulary log-probability. */
nd_status nd_needle_step_select(nd_ctx* ctx, nd_needle* model, uint32_t token,
                                const uint32_t* allowed, uint32_t count, uint32_t* id,
                                double* log_probability);

/* NeedleModel.generate at temperature 0 (model/model.ts:88-153) from token
 * ids: reset(max(count, min(model max_length, count + max_new)), sink), prefill
 * the prompt, then up to max_new greedy tokens, each the argmax of the last
 * logits with its logSoftmaxAt, stepping the model with every token but the
 * last; stops before an `eos` id (pass UINT32_MAX for none).  Every step after
 * the prompt runs as a replay of one HIP graph whose kernels read the token
 * and position from device memory, so the host issues no per-token copies
 * or synchronisation.  Writes *generated ids and log-probabilities. */
nd_status nd_needle_generate(nd_ctx* ctx, nd_needle* model, const uint32_t* prompt,
                             uint32_t count, uint32_t max_new, uint32_t sink, uint32_t eos,
                             uint32_t* ids, double* log_probabilities, uint32_t* generated);

/* stepSelected (model/runtime.ts:257-278) with the allowed set held on the
 * device: the model's mask buffer as nd_needle_grammar_mask left it, plus
 * the `n_settled` ids in `settled` (the undecided pieces the host grammar
 * accepted), then the step and selectToken over that bitmask (the ascending
 * allowed list Needle.complete builds, tools/agent.ts:164-183).  No id list
 * crosses to the device.  INVALID_CACT for a settled id outside the
 * vocabulary, or, after the step as in the reference, for an empty set. */
nd_status nd_needle_step_select_mask(nd_ctx* ctx, nd_needle* model, uint32_t token,
                                     const uint32_t* settled, uint32_t n_settled, uint32_t* id,
                                     double* log_probability);

/* The whole-step calls above run each layer's output projection, the layer
 * mix and the next layer's projection in one launch whose workgroups hand
 * over through bounded waits.  A wait that runs out sets a device status
 * word and its workgroup stores nothing; the call then returns
 * ND_ERR_BACKEND (BACKEND_UNAVAILABLE) with a message naming the wait, and
 * every whole-step call fails the same way until nd_needle_reset clears the
 * word with the launch's counters and flags.
 *
 * Test hook, no counterpart in the reference: makes the mix wait for
 * `extra_arrivals` more output-projection workgroups than the launch has
 * (so with extra_arrivals > 0 its wait runs out) and bounds every wait at
 * `spin_rounds` sleep rounds (0 restores the default, 65536).  Takes effect
 * from the next whole-step call; (0, 0) restores normal operation. */
nd_status nd_needle_test_waits(nd_ctx* ctx, nd_needle* model, uint32_t extra_arrivals,
                               uint32_t spin_rounds);

/* Measurement, no counterpart in the reference: the kernel launches of the
 * decode-step graph (a step with selection, as nd_needle_generate replays
 * it), counted when it was captured; 0 before the first such step. */
nd_status nd_needle_step_launches(nd_ctx* ctx, nd_needle* model, uint32_t* launches);

/* Measurement, no counterpart in the reference: while stamps_dev is set
 * (capacity >= (layers + 1) x 1024 words; an int8 model, or a Cactus-Quant
 * one whose phi matrices share one format), the fused layer
 * launches of direct (not graph-replayed) whole-step calls (nd_needle_step,
 * nd_needle_step_select) run their measurement form: thread 0 of active
 * workgroup k of launch l writes the GPU's 100 MHz clock at entry, when the
 * mix's wait for the output-projection rows ended, when the mix signalled
 * the projection, and at exit to stamps_dev[(64 l + k) x 16 .. + 3], and
 * the mix workgroup after its post norms, each FWHT, the lane update, the
 * pre norm, the phi products, the engram gate and the input norm to words
 * 4 .. 11, and inside the phi products to words 12 .. 14 (int8: the fp16
 * split in LDS, the MFMA chain, the partial rows; Cactus-Quant: the lanes
 * staged, rotated, the rows done); an int8 Wo workgroup when its input and
 * its weights had arrived and its rows were stored to words 4 .. 6 (a
 * Cactus-Quant one: input staged, rows computed, rows stored); a projection workgroup when its
 * wait ended, its input was staged, its rows were computed and its stores had completed to words
 * 4 .. 7; an attention workgroup when its wait ended, q and the gates were
 * issued, the tile math and the waves' combine were done and its output
 * stores had completed to words 4 .. 8 (0 where the role has no such point;
 * workgroups are Wo rows, then the mix, the projection, the attention).
 * NULL turns it off. */
nd_status nd_needle_test_stamps(nd_ctx* ctx, nd_needle* model, uint64_t* stamps_dev,
                                uint32_t capacity);

/* ---------------- ResidentExecutionSession methods (backends/backend.ts:65-80)
 *
 * The session API an unchanged NeedleRuntime.step drives (model/runtime.ts:
 * 314-375, 444-463, 554-564).  The host keeps the position, the token
 * history and the engram hashes; the device keeps the KV cache, the engram
 * ring, the lanes and the confidence pool.  A resident token is
 * nd_needle_prepare_engrams (optional), nd_needle_begin_token, then
 * nd_needle_forward_token (or nd_needle_forward_layer for layers 0..L-1 in
 * order), then nd_needle_finish_token or nd_needle_finish_token_for_selection
 * + nd_needle_select_token.  Calls out of that order are INVALID_CACT. */

/* beginResidentToken(lanes) (backend.ts:69; runtime.ts:327): lanes
 * [lanes][dim], every lane the scaled embedding row (runtime.ts:305-313);
 * lane 0 is the confidence pool's first cell of the token. */
nd_status nd_needle_begin_token(nd_ctx* ctx, nd_needle* model, const float* lanes);

/* prepareResidentEngrams({indices, valid, position}) (backend.ts:46-50, 70;
 * runtime.ts:314-321): the engram lookup of #engramLookup (runtime.ts:
 * 788-818) for `tables` tables; the device gathers the rows, projects the
 * keys and values of every site, and updates and convolves the ring at
 * `position` (#engramStep, runtime.ts:820-877).  Called before
 * nd_needle_begin_token.  Errors: INVALID_CACT for a model without engram
 * layers, a table count other than the model's or an index outside the
 * slots of a valid table; CONTEXT_OVERFLOW at the runtime limit. */
nd_status nd_needle_prepare_engrams(nd_ctx* ctx, nd_needle* model, const uint32_t* indices,
                                    const uint32_t* valid, uint32_t tables, uint32_t position);

/* forwardResidentLayer({layerIndex, position, engramKey?, engramValue?})
 * (backend.ts:58-63, 72; runtime.ts:346-361): layer `layer` of the token at
 * `position` -- the lane mix (runtime.ts:385-441), Q/K/V/gate with the
 * per-head norms and RoPE, #storeKV, gated attention, Wo (:465-505), and the
 * post-attention half of the layer before it (:509-551).  An engram layer
 * takes the host's key and value [dim] (#engramStep results) when the token's
 * engrams were not prepared on the device, and NULL otherwise. */
nd_status nd_needle_forward_layer(nd_ctx* ctx, nd_needle* model, uint32_t layer,
                                  uint32_t position, const float* engram_key,
                                  const float* engram_value);

/* forwardResidentToken({position, engramKeys, engramValues}) (backend.ts:
 * 52-56, 71; runtime.ts:337-345): every layer; engram_keys and
 * engram_values are [n_sites][dim] host arrays, or both NULL when the
 * engrams were prepared on the device. */
nd_status nd_needle_forward_token(nd_ctx* ctx, nd_needle* model, uint32_t position,
                                  const float* engram_keys, const float* engram_values);

/* finishResidentToken(wantLogits) (backend.ts:73; runtime.ts:371-374): the
 * last layer's post half, the lane mean and final norm, the confidence pool,
 * and with want_logits the logits [vocab] copied to `logits`
 * (runtime.ts:570-577). */
nd_status nd_needle_finish_token(nd_ctx* ctx, nd_needle* model, uint32_t want_logits,
                                 float* logits);

/* finishResidentTokenForSelection() (backend.ts:74; runtime.ts:363-369): the
 * same with the logits kept on the device for nd_needle_select_token. */
nd_status nd_needle_finish_token_for_selection(nd_ctx* ctx, nd_needle* model);

/* selectResidentToken(allowedTokenIds?) (backend.ts:75; runtime.ts:555-563):
 * selectToken (runtime.ts:880-899) over those logits -- `count` allowed ids
 * in list order, or every id when allowed == NULL.  Errors: INVALID_CACT for
 * an empty list or an id outside the logits; BACKEND_UNAVAILABLE without
 * logits from nd_needle_finish_token_for_selection. */
nd_status nd_needle_select_token(nd_ctx* ctx, nd_needle* model, const uint32_t* allowed,
                                 uint32_t count, uint32_t* id, double* log_probability);

/* selectResidentToken over the model's mask buffer plus `settled` (as
 * nd_needle_step_select_mask), for the session methods. */
nd_status nd_needle_select_token_mask(nd_ctx* ctx, nd_needle* model, const uint32_t* settled,
                                      uint32_t n_settled, uint32_t* id,
                                      double* log_probability);

/* readResidentLanes() (backend.ts:78): the lanes [lanes][dim] after the
 * last layer run (applying its post half if it is still owed). */
nd_status nd_needle_read_lanes(nd_ctx* ctx, nd_needle* model, float* lanes);

/* forward(request) (backend.ts:24-39, 68; runtime.ts:444-463), the layer of a
 * token that does not run resident: from the runtime's attention input
 * [dim] (the normalized block input), block and update inputs [dim], lanes x
 * [lanes][dim] and the layer's phi rows (phi_post [lanes], phi_residual
 * [lanes][lanes]), runs Q/K/V/gate, norms and RoPE, #storeKV, gated attention
 * and Wo, then the post half, and returns the next lanes ("nextX")
 * [lanes][dim] in next_x. */
nd_status nd_needle_forward(nd_ctx* ctx, nd_needle* model, uint32_t layer, uint32_t position,
                            const float* input, const float* block_input,
                            const float* update_input, const float* x, const float* phi_post,
                            const float* phi_residual, float* next_x);

/* ------------------------------ (f): schema-constrained token masks */

typedef struct nd_pieces nd_pieces;
typedef struct nd_grammar nd_grammar;

/* The tokenizer's pieces for mask generation: piece t is bytes[offsets[t],
 * offsets[t + 1]); eligible[t] = 1 for Normal and Byte pieces
 * (tools/agent.ts:167-168; TokenPieceType, model/tokenizer.ts:21-27). */
nd_status nd_pieces_upload(nd_ctx* ctx, const uint32_t* offsets, const uint8_t* bytes,
                           const uint8_t* eligible, uint32_t vocab, nd_pieces** out);
nd_status nd_pieces_free(nd_ctx* ctx, nd_pieces* pieces);

/* A tool-call grammar program (ToolCallGrammar over its tools' JSON Schemas,
 * tools/grammar.ts:256-797) compiled by the host, as 32-bit words:
 *   header [16]: magic 0x4E444752; (count, word offset) of nodes [28 words
 *     each], values [4], alternatives [1], properties [4], candidates [4],
 *     tools [4]; byte offset and length of the byte pool; word offset of the
 *     pattern automata (0: none), which run up to the byte pool.
 *   node: possible-type bits (string 1, number 2, integer 4, boolean 8,
 *     null 16, array 32, object 64); check flags (1 string constraints,
 *     2 numeric constraints, 4 integer only, 8 enum/const on an array or
 *     object, 16 uniqueItems); minItems; maxItems; items value; property count
 *     (<= 32); first property; required mask; minProperties; maxProperties;
 *     2 reserved; then the value checks (grammar.ts:179-222): flags
 *     (1 minLength, 2 maxLength, 4 format email, 8 format uuid, 16 a string
 *     check the host makes: enum / const / a length that is not a count / a
 *     pattern without an automaton, 32 pattern by its automaton; 256 minimum,
 *     512 maximum, 1024 exclusiveMinimum, 2048 exclusiveMaximum,
 *     4096 multipleOf, 8192 a numeric check the host makes: enum / const / a
 *     bound that is not a number), minLength, maxLength, the pattern
 *     automaton's word offset in the automata + 1 (0: none), minimum,
 *     maximum, exclusiveMinimum, exclusiveMaximum and multipleOf as float64
 *     (two words, low first), 2 reserved.
 *   pattern automaton (`new RegExp(pattern).test(value)` over the value's
 *     UTF-16 code units): states S (<= 1024), classes C, bounds B, 0; B
 *     bounds (first code unit | class << 16, ascending from unit 0); S flags
 *     (bit 0: the units read so far match); S x C next states.  State 0 is
 *     the empty value.
 *   value (a value frame's schema): kind 0 = alternatives (first, count:
 *     node indices in oneOf/anyOf order), 1 = choice (first, count <= 32
 *     candidates: every alternative is const/enum), 2 = too many candidates.
 *   property: name (byte offset, length), value index.
 *   candidate: JSON text (byte offset, length), value kind (0 string,
 *     1 number, 2 boolean, 3 null, 4 array, 5 object).
 *   tool: name (byte offset, length), the parameters' value index.
 * Every index is checked at upload (INVALID_CACT when one points outside). */
nd_status nd_grammar_upload(nd_ctx* ctx, const uint32_t* program, uint32_t n_words,
                            nd_grammar** out);
nd_status nd_grammar_free(nd_ctx* ctx, nd_grammar* grammar);

/* The allowed-token mask of one grammar state: bit t of allowed[t / 32] is
 * set when piece t is eligible, at most `budget` bytes long (65536 minus
 * the output so far, agent.ts:169) and accepted by the grammar from
 * `state`; bit t of undecided[t / 32] instead when the answer needs a check
 * the device does not make (strings under enum/const or under a pattern
 * with no automaton -- backreferences, lookaround, word boundaries --,
 * numbers under enum/const or whose value is not exact in the fast path --
 * more than 2^53 significant or a decimal exponent beyond +-22 --,
 * arrays/objects under enum/const, an array under uniqueItems closing in
 * the piece that completed one of its items, stacks deeper than 24) --
 * the host grammar settles those pieces.  String lengths, patterns with an
 * automaton, the email and uuid formats, and numeric bounds, multipleOf and
 * integrality are decided on the device.
 * state: [24] tool-call phase (0 array-open .. 8 done), literal offset,
 * live tool-name mask, name offset, current tool, used-tool mask, calls,
 * maximum calls, tools, arguments present, arguments complete, the
 * completed value's kind, frame depth (<= 24), 3 reserved; the running
 * summary of the string or number in progress in the top frame (zeros
 * otherwise): for a string, code points after the opening quote (an
 * escaped surrogate pair counts once), word 1 = the \u value being read
 * (bits 0-15) | an escaped high surrogate pending (16) | email state (17-19:
 * 0 start, 1 local part, 2 after '@', 3 domain, 4 after a usable '.',
 * 5 accepting, 6 dead) | uuid characters matched (20-25) | uuid mismatch
 * (26), the UTF-8 code point being assembled, the pattern automaton's
 * state (0 without one); for a number, the
 * mantissa of its significant digits taken while below 10^18 (low, high),
 * k (two's complement: value = mantissa 10^(k + exponent)), the exponent
 * digits (saturating at 999999) | minus (24) | exponent minus (25) | a
 * nonzero digit dropped (26); 4 reserved; then 4 words per
 * JSON frame, bottom first: kind | phase << 8 | flags << 16 (kinds 1 value,
 * 2 string, 3 number, 4 literal, 5 choice, 6 array, 7 object, 8 key), a
 * value or node index (literal: 0 true, 1 false, 2 null), a live/used mask
 * (array: 1 its items are the state's, 2 they are distinct by JSON text),
 * and an offset, count or current key.  Indices in the state are checked
 * by the kernel.  The host-pointer form copies state in and both masks
 * (ceil(vocab / 32) words each) out. */
nd_status nd_grammar_mask(nd_ctx* ctx, const nd_grammar* grammar, const uint32_t* state,
                          uint32_t n_state_words, const nd_pieces* pieces, uint32_t budget,
                          uint32_t* allowed, uint32_t* undecided);
nd_status nd_grammar_mask_d(nd_ctx* ctx, const nd_grammar* grammar, const uint32_t* state_dev,
                            const nd_pieces* pieces, uint32_t budget, uint32_t* allowed_dev,
                            uint32_t* undecided_dev, void* stream);

/* nd_grammar_mask with the allowed mask kept on the device, in the model's
 * mask buffer (pieces over the model's vocabulary), for
 * nd_needle_step_select_mask / nd_needle_select_token_mask: the undecided
 * bits (ceil(vocab / 32) words) and the number of allowed pieces come back
 * to the host, which settles the undecided pieces with its grammar
 * (tools/agent.ts:164-176), raises GRAMMAR_DEAD_END when the two counts sum
 * to zero (agent.ts:177-182), and passes the accepted ids to the selection
 * call.  The model must have been reset. */
nd_status nd_needle_grammar_mask(nd_ctx* ctx, nd_needle* model, const nd_grammar* grammar,
                                 const nd_pieces* pieces, const uint32_t* state,
                                 uint32_t n_state_words, uint32_t budget, uint32_t* undecided,
                                 uint32_t* n_allowed);

#ifdef __cplusplus
}
#endif

#endif /* NEEDLE_HIP_H */
