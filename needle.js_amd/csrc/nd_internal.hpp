// Internal declarations shared by the libneedle_hip translation units.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>
#include <cstdio>
#include <set>
#include <string>

#include "needle_hip.h"
#include "nd_rope.hpp"

struct nd_mat {
  int8_t* w = nullptr;      // [n][k] int8 codes, row-major
  float* scales = nullptr;  // [n][k / g]
  uint32_t n = 0, k = 0, g = 0;
  // Cactus-Quant form (bits != 0; w and scales unused): packed codes
  // [n][row_bytes], binary16 norms [n][kpad / g] and this width's codebook
  // by code (ternary: 0, +c, 0, -c).
  uint32_t bits = 0, kpad = 0, row_bytes = 0;
  uint8_t* packed = nullptr;
  uint16_t* norms = nullptr;
  float cb[16] = {};
};
// Prepared (rotated) input rows of a Cactus-Quant matvec: the context holds
// kCqPreparedRows rows of up to kCqMaxKpad floats, reused in stream order.
constexpr uint32_t kCqPreparedRows = 8;
constexpr uint32_t kCqMaxKpad = 8192;

struct nd_kv {
  uint32_t layers = 0, kv_heads = 0, head_dim = 0, max_length = 0;
  uint32_t sink = 0, window = 0, alloc = 0, mode = ND_KV_INT8;
  void* k = nullptr;  // [layers][kv_heads][alloc][head_dim] int8 (or f32)
  void* v = nullptr;
  float* ks = nullptr;  // [layers][kv_heads][alloc]
  float* vs = nullptr;
};

struct nd_ctx {
  int device = 0;
  hipStream_t stream = nullptr;
  std::string error;
  bool xcd_local = false;  // this device passed the placement probe
  // Device staging for the host-pointer entry points (grown on demand).
  void* stage = nullptr;
  size_t stage_bytes = 0;
  // Pinned host staging for small device-to-host reads (grown on demand).
  void* host_stage = nullptr;
  size_t host_stage_bytes = 0;
  // Split-context attention partials: acc [q_heads][chunks][head_dim] then
  // (max, sum) [q_heads][chunks][2], f32; and one arrival counter per KV head
  // (zeroed at allocation, reset by the kernel that consumes it).
  float* attn_partials = nullptr;
  size_t attn_partial_floats = 0;
  uint32_t* attn_counters = nullptr;
  // Workspace of the batched MFMA matvec (kMatvecSplitBytes).
  void* mv_split = nullptr;
  float* cq_prepared = nullptr;  // [kCqPreparedRows][kCqMaxKpad], on the first CQ upload
  // Digit planes and row factors of nd_matmul_d (grown on demand).
  void* mm_scratch = nullptr;
  size_t mm_scratch_bytes = 0;
  // Row records and counters of split selection (grown on demand, zeroed).
  void* sel_split = nullptr;
  size_t sel_split_bytes = 0;
  std::set<nd_mat*> mats;
  std::set<nd_kv*> kvs;
  std::set<nd_pieces*> pieces;
  std::set<nd_grammar*> grammars;
};

// Token pieces in HBM: byte offsets [vocab + 1], bytes, eligibility [vocab].
struct nd_pieces {
  uint32_t* offsets = nullptr;
  uint8_t* bytes = nullptr;
  uint8_t* eligible = nullptr;
  uint32_t vocab = 0;
};

// A compiled tool-call grammar program in HBM (layout in include/needle_hip.h):
// word offsets of nodes, values, alternatives, properties, candidates and
// tools, the byte offset of the name/candidate bytes, and the table sizes
// the kernel checks state indices against.
struct nd_grammar {
  uint32_t* words = nullptr;
  uint32_t off[6] = {};
  uint32_t bytes_off = 0;
  uint32_t regex_off = 0;  // word offset of the pattern automata (0: none)
  uint32_t n_nodes = 0, n_values = 0, n_tools = 0;
};
hipError_t nd_launch_grammar_mask(const nd_grammar* g, const uint32_t* state, const nd_pieces* pc,
                                  uint32_t budget, uint32_t* allowed, uint32_t* undecided,
                                  hipStream_t s);
// Whether a host grammar state's words hold its header and frames (at most
// 24); records the error on ctx otherwise.
nd_status nd_check_grammar_state(nd_ctx* ctx, const uint32_t* state, uint32_t n_state_words);

// Error helpers: record a message on the context and return a status.
nd_status nd_fail(nd_ctx* ctx, nd_status code, const char* fmt, ...);
nd_status nd_hip_fail(nd_ctx* ctx, hipError_t err, const char* what);

#define ND_HIP(ctx, expr)                                  \
  do {                                                     \
    hipError_t _e = (expr);                                \
    if (_e != hipSuccess) return nd_hip_fail(ctx, _e, #expr); \
  } while (0)

inline hipStream_t nd_pick_stream(nd_ctx* ctx, void* stream) {
  return stream ? reinterpret_cast<hipStream_t>(stream) : ctx->stream;
}

// Workgroup placement.  The XCD-local hand-offs (attention chunk merge,
// k-slice matvec sum, split-k GEMM sum, the Needle 2 fused layer launch)
// keep a merge group's workgroups at one L % 8 and rely on the dispatcher
// handing workgroup L of a launch to the XCD of workgroup L % 8.
// nd_probe_xcd_placement checks that on the current device (every workgroup
// of launches of 8, 64 and 1024 workgroups reads its XCC id) and records
// the result; nd_xcd_local() is true only when every probed device passed
// and the test override (nd_xcd_override) has not switched it off.  False
// selects the agent-scope forms.
hipError_t nd_probe_xcd_placement(hipStream_t s, bool* ok);
bool nd_xcd_local();
void nd_xcd_override(bool off);

// Kernel launchers (each validates nothing: callers check shapes first).
// `split`: kMatvecSplitBytes of device memory that lets batches of 3 or more
// run on MFMA (it holds the per-slice partial sums at k >= 4096 and their
// arrival counters, zero at allocation and left zero by every launch);
// nullptr keeps the vector kernel.  Launches sharing one `split` must be ordered
// (one stream).
constexpr size_t kMatvecPartialBytes = (size_t(4) << 20) - (size_t(64) << 10);
constexpr size_t kMatvecSplitBytes = kMatvecPartialBytes + (size_t(64) << 10);  // + counters
hipError_t nd_launch_matvec(const nd_mat* m, const float* x, uint32_t batch, uint32_t x_stride,
                            uint32_t row_start, uint32_t row_count, float* y, uint32_t y_stride,
                            hipStream_t s, void* split = nullptr);
hipError_t nd_launch_row(const nd_mat* m, uint32_t row, float* out, hipStream_t s);
// Batch-1 vector matvec of an int8 matrix with the entry and exit time of
// every workgroup (two uint64 per workgroup, 100 MHz clock) in stamps; the
// workgroup count goes to *workgroups, and a launch needing more than
// `capacity` workgroups is refused (hipErrorInvalidValue, nothing launched).
hipError_t nd_launch_matvec_stamped(const nd_mat* m, const float* x, uint32_t row_start,
                                    uint32_t row_count, float* y, uint64_t* stamps,
                                    uint32_t capacity, uint32_t* workgroups, hipStream_t s);
// Read-only stream of `bytes` (a multiple of 16) at 16-byte aligned `src`:
// `blocks` workgroups of 256 threads, one folded word each into out[blocks].
hipError_t nd_launch_stream_read(const void* src, uint64_t bytes, uint32_t blocks, uint32_t* out,
                                 hipStream_t s);
// Cactus-Quant matrices (csrc/cq.hip): prepareCqActivation of batch rows of
// x into prepared [batch][kpad]; the matvec of batch rows of x (its own
// input rotation; `prepared` is the context's kCqPreparedRows x kCqMaxKpad
// buffer, used for groups wider than 2048); one dequantized row.
hipError_t nd_launch_cq_prepare(const nd_mat* m, const float* x, uint32_t batch, uint32_t x_stride,
                                float* prepared, hipStream_t s);
hipError_t nd_launch_cq_matvec(const nd_mat* m, const float* x, uint32_t batch, uint32_t x_stride,
                               float* prepared, uint32_t row_start, uint32_t row_count, float* y,
                               uint32_t y_stride, hipStream_t s);
hipError_t nd_launch_cq_row(const nd_mat* m, uint32_t row, float* out, hipStream_t s);

// Visible-position arithmetic of the attention window (runtime.ts:723-728).
struct nd_visible {
  uint32_t prefix;      // positions [0, prefix)
  uint32_t recent_low;  // positions [recent_low, position]
  uint32_t count;       // prefix + position - recent_low + 1
};
nd_visible nd_kv_visible(const nd_kv* kv, uint32_t position);
uint32_t nd_attention_chunks(uint32_t count, uint32_t kv_heads);
size_t nd_attention_partial_floats(uint32_t q_heads, uint32_t kv_heads, uint32_t count);
constexpr uint32_t kMaxAttentionKvHeads = 1024;
constexpr uint32_t kMaxAttentionPositions = 262144;

hipError_t nd_launch_kv_store(const nd_kv* kv, uint32_t layer, uint32_t position, uint32_t first,
                              uint32_t count, const float* k, const float* v, hipStream_t s);
// stamps (measurement form, the XCD-local one-tile launch only): 8 clock
// stamps per workgroup, room for stamp_capacity workgroups; the launch's
// workgroup count goes to *stamp_workgroups (hipErrorInvalidValue when the
// launch takes another form or does not fit).
hipError_t nd_launch_attention(const nd_kv* kv, uint32_t layer, uint32_t position,
                               const float* q, uint32_t q_heads, float* out, float* partials,
                               uint32_t* counters, hipStream_t s, uint64_t* stamps = nullptr,
                               uint32_t stamp_capacity = 0, uint32_t* stamp_workgroups = nullptr);
hipError_t nd_launch_select_list(const float* logits, uint32_t vocab, const uint32_t* allowed,
                                 uint32_t count, uint32_t* id, double* logprob, hipStream_t s);
// `split`: nd_select_split_bytes(batch) of device memory, zero when first
// used and left zero by every launch, that lets each row's vocabulary be
// split over several workgroups (vocab % 32 == 0); nullptr keeps one
// workgroup per row.  Launches sharing one `split` must be ordered.  With
// `adv` and the split form, the launch also advances a decode batch's state
// (tokens[r] = id, positions[r] += 1, history[*step][r] = (id, log-prob) while
// *step < history_steps, then *step += 1) and sets *advanced.
struct nd_select_advance {
  uint32_t* tokens;
  uint32_t* positions;
  uint32_t* step;
  uint32_t* history;
  double* lp_history;
  uint32_t history_steps;
};
size_t nd_select_split_bytes(uint32_t batch);
hipError_t nd_launch_select_mask(const float* logits, uint32_t batch, uint32_t vocab,
                                 const uint32_t* mask, uint32_t* ids, double* logprobs,
                                 hipStream_t s, void* split = nullptr,
                                 const nd_select_advance* adv = nullptr,
                                 bool* advanced = nullptr);

// Digit-sliced int8 MFMA GEMM (gemm.hip): y[m][n] (op)= s_w[n] * A[m] . W[n]
// with A given as digits [3][M][K] and per-row factors fm (digitize first).
// epilogue: 0 store, 1 add into y, 2 store silu.  K % 64 == 0, K <= 2048 for
// digitize.
hipError_t nd_launch_digitize(const float* x, uint32_t ldx, const float* norm, float* norm_out,
                              int8_t* digits, float* fm, uint32_t M, uint32_t K, hipStream_t s);
// Split-k workspace of nd_launch_gemm: partial sums (partial_floats floats)
// and counter_count arrival counters, zero when first used and left zero by
// every launch that completes.  Launches that share a workspace must be
// ordered (one stream).
struct nd_gemm_split {
  float* partials;
  size_t partial_floats;
  uint32_t* counters;
  uint32_t counter_count;
};
hipError_t nd_launch_gemm(const nd_mat* w, const int8_t* digits, const float* fm, float* y,
                          uint32_t ldy, uint32_t M, int epilogue, hipStream_t s,
                          const nd_gemm_split* split = nullptr);
// The same product on fp32 rows x [M][ldx] (optionally RMS-normalized with
// `norm`, math.ts:16-32), digitized per 256-wide chunk inside the launch;
// only for the shapes nd_gemm_f32_fits accepts.  Epilogue 3 (the q/k/v
// projection of a decode step, w->n = (heads + 2 kv_heads) * 64): instead of
// storing y, each 64-column head goes through norm, rope and the cache store
// that `rope` describes (nd_rope.hpp).
bool nd_gemm_f32_fits(const nd_mat* w, const float* x, uint32_t ldx, bool norm, uint32_t M,
                      const nd_gemm_split* split);
hipError_t nd_launch_gemm_f32(const nd_mat* w, const float* x, uint32_t ldx, const float* norm,
                              float* y, uint32_t ldy, uint32_t M, int epilogue, hipStream_t s,
                              const nd_gemm_split* split,
                              const nd::RopeStore* rope = nullptr);
hipError_t nd_launch_attention_batch(const nd_kv* kv, uint32_t layer, const uint32_t* positions,
                                     uint32_t batch, uint32_t seq_kv_heads, uint32_t kv_stride_z,
                                     uint32_t rep, uint32_t max_position, const float* q,
                                     float* out, float* partials, uint32_t* counters,
                                     hipStream_t s, const float* gate = nullptr,
                                     uint32_t gate_ld = 0);
// Attention launches take `counters`: kAttnCounterStride zero-initialized
// words per (query row, KV head) -- from (z * seq_kv_heads + kv head) *
// kAttnCounterStride -- which a launch that splits a row into several chunks
// uses to elect the chunk that merges them (a counter per group of chunks,
// then one per row and head), and leaves at zero again.
constexpr uint32_t kAttnCounterStride = 32;  // 128 bytes: one L2 line per row and head
// Fixed device scratch of nd_attention_static_d (kv_attention.hip): the chunk
// partials of one query row -- acc [q_heads][chunks][64] then (max, sum)
// [q_heads][chunks][2] -- for up to kStaticAttnQHeads query heads and the
// kernel's 64 chunks, then kAttnCounterStride arrival counters per KV head.
constexpr uint32_t kStaticAttnQHeads = 64;
constexpr size_t kStaticAttnPartialWords = (size_t)kStaticAttnQHeads * 64 * (64 + 2);
constexpr size_t kStaticAttnWords =
    kStaticAttnPartialWords + (size_t)kStaticAttnQHeads * kAttnCounterStride;
// Looks the scratch up on `device` (which must be current) once per device;
// nd_attention_scratch returns its HBM address there (nullptr before set-up).
hipError_t nd_attention_scratch_setup(int device);
void* nd_attention_scratch(int device);
//
// One query row whose position is read from device memory (*position <=
// max_position); out = attention * sigmoid(gate) elementwise when gate is set
// (gated attention, model/runtime.ts:503-505).
hipError_t nd_launch_attention_gated(const nd_kv* kv, uint32_t layer, const uint32_t* position,
                                     uint32_t max_position, const float* q, uint32_t q_heads,
                                     const float* gate, float* out, float* partials,
                                     uint32_t* counters, hipStream_t s);
size_t nd_attention_batch_partial_floats(uint32_t batch, uint32_t seq_kv_heads, uint32_t rep,
                                         uint32_t max_count);
