// Batched int8 decoder on HBM-resident weights and KV: the synthetic decoder
// of the batched constrained-decode and prefill workloads, composed from the
// reference primitives (embedding row x sqrt(d), runtime.ts:305-309; per-head
// zero-centred RMS norm and half-split RoPE, runtime.ts:471-500 with
// math.ts:94-115; #storeKV/#attention, runtime.ts:679-786; residual matvecs;
// SiLU MLP, math.ts:12-14; tied logits, runtime.ts:570-577; selectToken over
// an allowed bitmask, runtime.ts:880-899).
//
// One decode step of B sequences is a fixed sequence of kernel launches on one
// stream with no host synchronisation and no allocation, so a caller can
// capture it in a HIP graph; tokens, positions and the step counter advance
// in device memory.
#include <cmath>
#include <vector>

#include "nd_internal.hpp"
#include "nd_rope.hpp"
#include "nd_wave.hpp"

namespace {

constexpr uint32_t kHd = 64;

__device__ __forceinline__ uint64_t sm64_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
__device__ __forceinline__ uint64_t sm64_at(uint64_t seed, uint64_t i) {
  return sm64_mix(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
}

// Wave reductions on DPP and readlane (every lane gets the same value).
__device__ __forceinline__ double wave_sum_d(double v) { return nd::wave_sum(v); }

__device__ __forceinline__ float wave_absmax_js(float v) { return nd::wave_max_js(fabsf(v)); }

// x[m][:] = f32(f32(W[tok][:] * s[tok]) * sqrt(d)), the row() gather and
// embedding scale of runtime.ts:305-309, in float64 like the reference.
__global__ void embed_kernel(const int8_t* __restrict__ W, const float* __restrict__ S,
                             const uint32_t* __restrict__ tokens, uint32_t vocab, uint32_t d,
                             double scale, float* __restrict__ x) {
  const uint32_t m = blockIdx.y, k = blockIdx.x * blockDim.x + threadIdx.x;
  if (k >= d) return;
  const uint32_t tok = tokens[m] < vocab ? tokens[m] : vocab - 1;  // ids are validated on entry
  const float row = (float)W[(size_t)tok * d + k] * S[tok];
  x[(size_t)m * d + k] = (float)((double)row * scale);
}

// One wave per (row m, head slot).  Slots [0, H) are query heads: zero-centred
// RMS norm with q_norm, then RoPE, written to q_out.  Slots [H, H + Hkv) are
// KV heads: k gets k_norm and RoPE, then k and v are quantized into the cache
// at the row's position (#storeKV bit-exact semantics).  Norm and rotation run
// in float64 with f32 stores, as the reference does.
__device__ __forceinline__ void qk_rope_store_item(
    uint32_t m, uint32_t slot, uint32_t lane,
    const float* __restrict__ qkv, uint32_t ld, uint32_t heads, uint32_t kv_heads,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm,
    const double* __restrict__ inv_freq, const double2* __restrict__ rope_tab,
    const uint32_t* __restrict__ positions,
    uint32_t position0, float* __restrict__ q_out, int8_t* __restrict__ Kc,
    int8_t* __restrict__ Vc, float* __restrict__ Ks, float* __restrict__ Vs, uint32_t layer,
    uint32_t cache_heads, uint32_t alloc, uint32_t kv_head_stride) {
  const uint32_t pos = positions ? positions[m] : position0 + m;
  const bool is_q = slot < heads;
  const uint32_t h = is_q ? slot : slot - heads;
  const float* src = qkv + (size_t)m * ld + (is_q ? h * kHd : heads * kHd + h * kHd);
  const float* scale = is_q ? q_norm : k_norm;
  const double x = src[lane];
  // Half-split RoPE: pair (j, j + 32), angle = pos * theta^(-2j/64).
  const uint32_t j = lane & 31;
  double sn, cs;
  if (rope_tab) {  // rope_table_kernel's values for row m: the same sincos
    const double2 sc = rope_tab[(size_t)m * 32 + j];
    sn = sc.x;
    cs = sc.y;
  } else {
    sincos((double)pos * inv_freq[j], &sn, &cs);
  }
  const float rot = nd::norm_rope(x, scale, lane, sn, cs);
  if (is_q) {
    q_out[((size_t)m * heads + h) * kHd + lane] = rot;
    return;
  }
  if (pos >= alloc) return;  // positions are validated on entry; never write past the cache
  // Cache head for row m: (m * kv_head_stride + h) when rows are sequences of
  // a batch (stride = Hkv), or h when rows are consecutive positions.
  const size_t row = ((size_t)layer * cache_heads + (size_t)m * kv_head_stride + h) * alloc + pos;
  nd::quant_store(rot, row, lane, Kc, Ks);
  nd::quant_store(qkv[(size_t)m * ld + (heads + kv_heads) * kHd + h * kHd + lane], row, lane, Vc,
                  Vs);
}

// Workgroup (slot, row m): one wave.
__global__ __launch_bounds__(64) void qk_rope_store_kernel(
    const float* __restrict__ qkv, uint32_t ld, uint32_t heads, uint32_t kv_heads,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm,
    const double* __restrict__ inv_freq, const double2* __restrict__ rope_tab,
    const uint32_t* __restrict__ positions,
    uint32_t position0, float* __restrict__ q_out, int8_t* __restrict__ Kc,
    int8_t* __restrict__ Vc, float* __restrict__ Ks, float* __restrict__ Vs, uint32_t layer,
    uint32_t cache_heads, uint32_t alloc, uint32_t kv_head_stride) {
  qk_rope_store_item(blockIdx.y, blockIdx.x, threadIdx.x, qkv, ld, heads, kv_heads, q_norm,
                     k_norm, inv_freq, rope_tab, positions, position0, q_out, Kc, Vc, Ks, Vs,
                     layer, cache_heads, alloc, kv_head_stride);
}

// (sin, cos) of the RoPE angles pos * inv_freq[j], j < 32, of rows [0, M)
// at positions position0 + m, evaluated as qk_rope_store_kernel evaluates
// them, so that the prefill's layers and heads share one evaluation per row.
__global__ void rope_table_kernel(const double* __restrict__ inv_freq, uint32_t position0,
                                  uint32_t M, double2* __restrict__ tab) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= M * 32) return;
  const uint32_t m = i >> 5, j = i & 31;
  double sn, cs;
  sincos((double)(position0 + m) * inv_freq[j], &sn, &cs);
  tab[i] = make_double2(sn, cs);
}

// Allowed-token bitmask rows for decode step *step of sequence b: id v is
// allowed iff (z_v >> 40) < threshold24 with z the splitmix64 stream seeded by
// splitmix64_at(mask_seed, step * 65536 + b); the id (z_vocab >> 32) * vocab
// >> 32 is always allowed.  One thread per 32-bit word.
__global__ void gen_masks_kernel(uint64_t mask_seed, const uint32_t* __restrict__ step,
                                 uint32_t batch, uint32_t vocab, uint32_t threshold24,
                                 uint32_t* __restrict__ masks) {
  const uint32_t words = (vocab + 31) / 32;
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i >= batch * words) return;
  const uint32_t b = i / words, w = i % words;
  const uint64_t seed = sm64_at(mask_seed, (uint64_t)(*step) * 65536 + b);
  const uint32_t forced = (uint32_t)(((sm64_at(seed, vocab) >> 32) * (uint64_t)vocab) >> 32);
  uint32_t bits = 0;
  for (uint32_t e = 0; e < 32; ++e) {
    const uint32_t v = w * 32 + e;
    if (v >= vocab) break;
    if ((uint32_t)(sm64_at(seed, v) >> 40) < threshold24 || v == forced) bits |= 1u << e;
  }
  masks[i] = bits;
}

// Synthetic prefix rows for sequence `seq`: codes ((z >> 32) * 255 >> 32) -
// 127 and scale lo + (hi - lo) * (z >> 40) * 2^-24 from the stream of the K or
// V seed at index ((l * Hkv + h) * index_stride + p) * 65 + i.
__global__ __launch_bounds__(64) void fill_kv_kernel(uint64_t seed_k, uint64_t seed_v,
                                                     uint32_t seq, uint32_t kv_heads,
                                                     uint32_t cache_heads, uint32_t alloc,
                                                     uint32_t index_stride, float lo, float hi,
                                                     int8_t* __restrict__ Kc,
                                                     int8_t* __restrict__ Vc,
                                                     float* __restrict__ Ks,
                                                     float* __restrict__ Vs) {
  const uint32_t p = blockIdx.x, h = blockIdx.y, l = blockIdx.z, lane = threadIdx.x;
  const uint64_t base = (((uint64_t)l * kv_heads + h) * index_stride + p) * (kHd + 1);
  const size_t row = ((size_t)l * cache_heads + (size_t)seq * kv_heads + h) * alloc + p;
  const uint64_t zk = sm64_at(seed_k, base + lane), zv = sm64_at(seed_v, base + lane);
  Kc[row * kHd + lane] = (int8_t)((int)(((zk >> 32) * 255ull) >> 32) - 127);
  Vc[row * kHd + lane] = (int8_t)((int)(((zv >> 32) * 255ull) >> 32) - 127);
  if (lane == 0) {
    const double uk = (double)(sm64_at(seed_k, base + kHd) >> 40) * (1.0 / 16777216.0);
    const double uv = (double)(sm64_at(seed_v, base + kHd) >> 40) * (1.0 / 16777216.0);
    Ks[row] = (float)((double)lo + ((double)hi - (double)lo) * uk);
    Vs[row] = (float)((double)lo + ((double)hi - (double)lo) * uv);
  }
}

// After selection (one workgroup): feed ids back as the next tokens, record
// them and their log-probabilities in the per-step history, advance the
// positions and then the step counter.
__global__ __launch_bounds__(256) void advance_kernel(
    const uint32_t* __restrict__ ids, const double* __restrict__ logprobs,
    uint32_t* __restrict__ tokens, uint32_t* __restrict__ positions, uint32_t* __restrict__ step,
    uint32_t* __restrict__ history, double* __restrict__ lp_history, uint32_t history_steps,
    uint32_t batch) {
  const uint32_t t = *step;
  for (uint32_t b = threadIdx.x; b < batch; b += blockDim.x) {
    tokens[b] = ids[b];
    positions[b] += 1;
    if (t < history_steps) {
      history[(size_t)t * batch + b] = ids[b];
      lp_history[(size_t)t * batch + b] = logprobs[b];
    }
  }
  __syncthreads();
  if (threadIdx.x == 0) *step = t + 1;
}

}  // namespace

struct nd_decoder {
  uint32_t layers = 0, dim = 0, heads = 0, kv_heads = 0, head_dim = 0, ffn = 0, vocab = 0;
  const nd_mat* embedding = nullptr;
  std::vector<nd_mat> wqkv;  // owned: rows q (heads*64), k (kv_heads*64), v (kv_heads*64)
  std::vector<const nd_mat*> wo, wup, wdown;
  float* norms = nullptr;  // attn [L][d], ffn [L][d], q [L][64], k [L][64], final [d]
  double* inv_freq = nullptr;
  size_t attn_off = 0, ffn_off = 0, q_off = 0, k_off = 0, final_off = 0;
};

struct nd_batch {
  nd_decoder* dec = nullptr;
  uint32_t batch = 0, max_length = 0;
  nd_kv kv;  // kv_heads = batch * dec->kv_heads
  char* arena = nullptr;
  float *x = nullptr, *qkv = nullptr, *q = nullptr, *o = nullptr, *h = nullptr,
        *logits = nullptr, *fm = nullptr, *partials = nullptr;
  int8_t* digits = nullptr;
  uint32_t *counters = nullptr, *masks = nullptr, *tokens = nullptr, *positions = nullptr,
           *step = nullptr, *ids = nullptr, *history = nullptr;
  double *logprobs = nullptr, *lp_history = nullptr;  // history: [max_length][batch]
  nd_gemm_split gsplit{};  // split-k workspace of the step's GEMMs (zeroed counters)
  void* sel_split = nullptr;  // split-selection records and counters (zeroed)
  double2* rope_tab = nullptr;  // (sin, cos) of every cache position: [max_length][32]
};

// Split-k workspace of a batch: up to 512 tiles' worth of partials (16 x 64
// outputs each) and 256 tile counters.
constexpr size_t kSplitPartialFloats = (size_t)512 * 1024;
constexpr uint32_t kSplitCounters = 256;

static inline size_t a256(size_t n) { return (n + 255) & ~size_t(255); }

static nd_status check_weight(nd_ctx* ctx, const nd_mat* m, uint32_t n, uint32_t k,
                              const char* what) {
  if (!m) return nd_fail(ctx, ND_ERR_INVALID, "%s is NULL", what);
  if (m->bits || m->n != n || m->k != k || m->g != k)
    return nd_fail(ctx, ND_ERR_INVALID, "%s is %ux%u (group %u); expected %ux%u per-row scaled",
                   what, m->n, m->k, m->g, n, k);
  return ND_OK;
}

extern "C" {

nd_status nd_decoder_create(nd_ctx* ctx, const nd_decoder_desc* d, nd_decoder** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!d || !out) return nd_fail(ctx, ND_ERR_INVALID, "nd_decoder_create: NULL argument");
  *out = nullptr;
  if (d->head_dim != kHd || d->layers == 0 || d->heads == 0 || d->kv_heads == 0 ||
      d->heads % d->kv_heads != 0 || d->dim % 64 != 0 || d->ffn % 64 != 0 || d->dim > 2048 ||
      d->ffn > 2048 || d->heads * kHd != d->dim)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "decoder geometry: head_dim 64, heads * 64 == dim, dim and ffn multiples of 64 "
                   "and at most 2048");
  const uint32_t rep = d->heads / d->kv_heads;
  if (rep != 1 && rep != 2 && rep != 4 && rep != 8)
    return nd_fail(ctx, ND_ERR_INVALID, "query heads per KV head must be 1, 2, 4 or 8");
  nd_status st = check_weight(ctx, d->embedding, d->vocab, d->dim, "embedding");
  if (st != ND_OK) return st;
  for (uint32_t l = 0; l < d->layers; ++l) {
    if ((st = check_weight(ctx, d->wq[l], d->heads * kHd, d->dim, "wq")) ||
        (st = check_weight(ctx, d->wk[l], d->kv_heads * kHd, d->dim, "wk")) ||
        (st = check_weight(ctx, d->wv[l], d->kv_heads * kHd, d->dim, "wv")) ||
        (st = check_weight(ctx, d->wo[l], d->dim, d->heads * kHd, "wo")) ||
        (st = check_weight(ctx, d->wup[l], d->ffn, d->dim, "wup")) ||
        (st = check_weight(ctx, d->wdown[l], d->dim, d->ffn, "wdown")))
      return st;
  }
  nd_decoder* dec = new nd_decoder();
  dec->layers = d->layers;
  dec->dim = d->dim;
  dec->heads = d->heads;
  dec->kv_heads = d->kv_heads;
  dec->head_dim = d->head_dim;
  dec->ffn = d->ffn;
  dec->vocab = d->vocab;
  dec->embedding = d->embedding;
  const uint32_t qkv_rows = (d->heads + 2 * d->kv_heads) * kHd;
  dec->wqkv.resize(d->layers);
  hipError_t e = hipSuccess;
  for (uint32_t l = 0; l < d->layers && e == hipSuccess; ++l) {
    nd_mat& m = dec->wqkv[l];
    m.n = qkv_rows;
    m.k = d->dim;
    m.g = d->dim;
    e = hipMalloc(&m.w, (size_t)qkv_rows * d->dim);
    if (e == hipSuccess) e = hipMalloc(&m.scales, (size_t)qkv_rows * 4);
    const nd_mat* parts[3] = {d->wq[l], d->wk[l], d->wv[l]};
    size_t row = 0;
    for (const nd_mat* p : parts) {
      if (e == hipSuccess)
        e = hipMemcpyAsync(m.w + row * d->dim, p->w, (size_t)p->n * d->dim, hipMemcpyDeviceToDevice,
                           ctx->stream);
      if (e == hipSuccess)
        e = hipMemcpyAsync(m.scales + row, p->scales, (size_t)p->n * 4, hipMemcpyDeviceToDevice,
                           ctx->stream);
      row += p->n;
    }
    dec->wo.push_back(d->wo[l]);
    dec->wup.push_back(d->wup[l]);
    dec->wdown.push_back(d->wdown[l]);
  }
  const size_t L = d->layers, D = d->dim;
  dec->attn_off = 0;
  dec->ffn_off = L * D;
  dec->q_off = 2 * L * D;
  dec->k_off = 2 * L * D + L * kHd;
  dec->final_off = 2 * L * D + 2 * L * kHd;
  const size_t nf = dec->final_off + D;
  std::vector<float> host(nf);
  for (size_t i = 0; i < L * D; ++i) {
    host[dec->attn_off + i] = d->attn_norm[i];
    host[dec->ffn_off + i] = d->ffn_norm[i];
  }
  for (size_t i = 0; i < L * kHd; ++i) {
    host[dec->q_off + i] = d->q_norm[i];
    host[dec->k_off + i] = d->k_norm[i];
  }
  for (size_t i = 0; i < D; ++i) host[dec->final_off + i] = d->final_norm[i];
  // RoPE frequencies theta^(-2j/64) in float64 (math.ts:94-115).
  std::vector<double> freq(kHd / 2);
  for (uint32_t j = 0; j < kHd / 2; ++j)
    freq[j] = std::pow((double)d->rope_theta, -(2.0 * j) / kHd);
  if (e == hipSuccess) e = hipMalloc(&dec->norms, nf * 4);
  if (e == hipSuccess) e = hipMalloc(&dec->inv_freq, freq.size() * 8);
  if (e == hipSuccess)
    e = hipMemcpyAsync(dec->norms, host.data(), nf * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(dec->inv_freq, freq.data(), freq.size() * 8, hipMemcpyHostToDevice,
                       ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    for (auto& m : dec->wqkv) {
      hipFree(m.w);
      hipFree(m.scales);
    }
    hipFree(dec->norms);
    hipFree(dec->inv_freq);
    delete dec;
    return nd_hip_fail(ctx, e, "decoder upload");
  }
  *out = dec;
  return ND_OK;
}

nd_status nd_decoder_free(nd_ctx* ctx, nd_decoder* dec) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!dec) return ND_OK;
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  for (auto& m : dec->wqkv) {
    hipFree(m.w);
    hipFree(m.scales);
  }
  hipFree(dec->norms);
  hipFree(dec->inv_freq);
  delete dec;
  return ND_OK;
}

nd_status nd_batch_create(nd_ctx* ctx, nd_decoder* dec, uint32_t batch, uint32_t max_length,
                          nd_batch** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!dec || !out || batch == 0 || max_length == 0)
    return nd_fail(ctx, ND_ERR_INVALID, "nd_batch_create: bad argument");
  if (max_length > kMaxAttentionPositions || batch * dec->kv_heads > kMaxAttentionKvHeads)
    return nd_fail(ctx, ND_ERR_INVALID, "batch limits: %u positions, %u KV heads in total",
                   kMaxAttentionPositions, kMaxAttentionKvHeads);
  *out = nullptr;
  nd_batch* b = new nd_batch();
  b->dec = dec;
  b->batch = batch;
  b->max_length = max_length;
  nd_kv& kv = b->kv;
  kv.layers = dec->layers;
  kv.kv_heads = batch * dec->kv_heads;
  kv.head_dim = kHd;
  kv.max_length = max_length;
  kv.sink = 0;
  kv.window = 0;
  kv.alloc = max_length;
  kv.mode = ND_KV_INT8;
  const size_t rows = (size_t)kv.layers * kv.kv_heads * kv.alloc;
  const uint32_t rep = dec->heads / dec->kv_heads;
  const size_t pf = nd_attention_batch_partial_floats(batch, dec->kv_heads, rep, max_length);
  const uint32_t kmax = dec->ffn > dec->dim ? dec->ffn : dec->dim;
  const uint32_t qkv_rows = (dec->heads + 2 * dec->kv_heads) * kHd;
  const uint32_t words = (dec->vocab + 31) / 32;
  size_t sizes[] = {
      a256(rows * kHd), a256(rows * kHd), a256(rows * 4), a256(rows * 4),   // K, V, scales
      a256((size_t)batch * dec->dim * 4),                                    // x
      a256((size_t)batch * qkv_rows * 4),                                    // qkv
      a256((size_t)batch * dec->dim * 4),                                    // q
      a256((size_t)batch * dec->dim * 4),                                    // o
      a256((size_t)batch * dec->ffn * 4),                                    // h
      a256((size_t)batch * dec->vocab * 4),                                  // logits
      a256((size_t)batch * 4),                                               // fm
      a256(pf * 4),                                                          // partials
      a256((size_t)3 * batch * kmax),                                        // digits
      a256((size_t)batch * dec->kv_heads * kAttnCounterStride * 4),          // counters
      a256((size_t)batch * words * 4),                                       // masks
      a256((size_t)batch * 4), a256((size_t)batch * 4), a256(256),           // tokens, positions, step
      a256((size_t)batch * 4), a256((size_t)batch * 8),                      // ids, logprobs
      a256((size_t)max_length * batch * 4), a256((size_t)max_length * batch * 8),   // history
      a256(kSplitPartialFloats * 4), a256((size_t)kSplitCounters * 4),          // GEMM split-k
      a256(nd_select_split_bytes(batch)),                                    // selection
      a256((size_t)max_length * 32 * sizeof(double2))};                      // rope table
  size_t total = 0;
  for (size_t v : sizes) total += v;
  hipError_t e = hipMalloc(&b->arena, total);
  if (e == hipSuccess) e = hipMemsetAsync(b->arena, 0, total, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    if (b->arena) hipFree(b->arena);
    delete b;
    return nd_hip_fail(ctx, e, "batch allocation");
  }
  char* p = b->arena;
  size_t i = 0;
  auto take = [&](void* dst_ptr) {
    *reinterpret_cast<char**>(dst_ptr) = p;
    p += sizes[i++];
  };
  take(&kv.k);
  take(&kv.v);
  take(&kv.ks);
  take(&kv.vs);
  take(&b->x);
  take(&b->qkv);
  take(&b->q);
  take(&b->o);
  take(&b->h);
  take(&b->logits);
  take(&b->fm);
  take(&b->partials);
  take(&b->digits);
  take(&b->counters);
  take(&b->masks);
  take(&b->tokens);
  take(&b->positions);
  take(&b->step);
  take(&b->ids);
  take(&b->logprobs);
  take(&b->history);
  take(&b->lp_history);
  take(&b->gsplit.partials);
  take(&b->gsplit.counters);
  take(&b->sel_split);
  take(&b->rope_tab);
  b->gsplit.partial_floats = kSplitPartialFloats;
  b->gsplit.counter_count = kSplitCounters;
  // RoPE angles of every position the cache holds, evaluated once here as
  // the rope/store kernel evaluates them.
  hipLaunchKernelGGL(rope_table_kernel, dim3((max_length * 32 + 255) / 256), dim3(256), 0,
                     ctx->stream, dec->inv_freq, 0u, max_length, b->rope_tab);
  e = hipGetLastError();
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    hipFree(b->arena);
    delete b;
    return nd_hip_fail(ctx, e, "batch rope table");
  }
  *out = b;
  return ND_OK;
}

nd_status nd_batch_free(nd_ctx* ctx, nd_batch* b) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!b) return ND_OK;
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  hipFree(b->arena);
  delete b;
  return ND_OK;
}

nd_kv* nd_batch_kv(nd_batch* b) { return b ? &b->kv : nullptr; }

nd_status nd_batch_fill_synthetic(nd_ctx* ctx, nd_batch* b, uint32_t seq, uint64_t seed_k,
                                  uint64_t seed_v, uint32_t length, uint32_t index_stride,
                                  float lo, float hi) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!b || seq >= b->batch || length > b->max_length)
    return nd_fail(ctx, ND_ERR_INVALID, "nd_batch_fill_synthetic: bad sequence or length");
  if (length == 0) return ND_OK;
  const nd_decoder* dec = b->dec;
  hipLaunchKernelGGL(fill_kv_kernel, dim3(length, dec->kv_heads, dec->layers), dim3(64), 0,
                     ctx->stream, seed_k, seed_v, seq, dec->kv_heads, b->kv.kv_heads, b->kv.alloc,
                     index_stride, lo, hi, (int8_t*)b->kv.k, (int8_t*)b->kv.v, b->kv.ks, b->kv.vs);
  ND_HIP(ctx, hipGetLastError());
  return ND_OK;
}

nd_status nd_batch_set_state(nd_ctx* ctx, nd_batch* b, const uint32_t* tokens,
                             const uint32_t* positions, uint32_t step) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!b || !tokens || !positions) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  for (uint32_t i = 0; i < b->batch; ++i) {
    if (tokens[i] >= b->dec->vocab)
      return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside the vocabulary", tokens[i]);
    if (positions[i] >= b->max_length)
      return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %u reached runtime limit %u", positions[i],
                     b->max_length);
  }
  ND_HIP(ctx, hipMemcpyAsync(b->tokens, tokens, b->batch * 4, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(b->positions, positions, b->batch * 4, hipMemcpyHostToDevice,
                             ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(b->step, &step, 4, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_batch_read(nd_ctx* ctx, nd_batch* b, uint32_t* tokens, uint32_t* positions,
                        double* logprobs, float* logits) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!b) return nd_fail(ctx, ND_ERR_INVALID, "batch is NULL");
  if (tokens)
    ND_HIP(ctx, hipMemcpyAsync(tokens, b->tokens, b->batch * 4, hipMemcpyDeviceToHost, ctx->stream));
  if (positions)
    ND_HIP(ctx, hipMemcpyAsync(positions, b->positions, b->batch * 4, hipMemcpyDeviceToHost,
                               ctx->stream));
  if (logprobs)
    ND_HIP(ctx, hipMemcpyAsync(logprobs, b->logprobs, b->batch * 8, hipMemcpyDeviceToHost,
                               ctx->stream));
  if (logits)
    ND_HIP(ctx, hipMemcpyAsync(logits, b->logits, (size_t)b->batch * b->dec->vocab * 4,
                               hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_batch_read_projections(nd_ctx* ctx, nd_batch* b, float* out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!b || !out) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  const size_t rows = (size_t)(b->dec->heads + 2 * b->dec->kv_heads) * kHd;
  ND_HIP(ctx, hipMemcpyAsync(out, b->qkv, (size_t)b->batch * rows * 4, hipMemcpyDeviceToHost,
                             ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

// One decode step for all sequences.  Reads tokens/positions/step from device
// memory; with masks == 1 the step's allowed bitmasks are generated on the
// device from mask_seed and applied, otherwise selection is unconstrained.
// `max_position` bounds every sequence's position this step (sizes the
// attention grid); positions beyond it are not read.
nd_status nd_batch_step(nd_ctx* ctx, nd_batch* b, uint32_t max_position, uint32_t use_masks,
                        uint64_t mask_seed, uint32_t threshold24, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!b) return nd_fail(ctx, ND_ERR_INVALID, "batch is NULL");
  if (max_position >= b->max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %u reached runtime limit %u", max_position,
                   b->max_length);
  hipStream_t s = nd_pick_stream(ctx, stream);
  const nd_decoder* dec = b->dec;
  const uint32_t B = b->batch, D = dec->dim, F = dec->ffn;
  const uint32_t qkv_rows = (dec->heads + 2 * dec->kv_heads) * kHd;
  const uint32_t rep = dec->heads / dec->kv_heads;
  hipLaunchKernelGGL(embed_kernel, dim3((D + 255) / 256, B), dim3(256), 0, s, dec->embedding->w,
                     dec->embedding->scales, b->tokens, dec->vocab, D, std::sqrt((double)D), b->x);
  ND_HIP(ctx, hipGetLastError());
  // x (optionally normalized) times w into y: one launch that digitizes its
  // own chunks where the shape allows, else digitize + GEMM.
  auto product = [&](const nd_mat* w, const float* x, const float* norm, float* y, uint32_t ldy,
                     int epi) -> hipError_t {
    if (nd_gemm_f32_fits(w, x, w->k, norm != nullptr, B, &b->gsplit))
      return nd_launch_gemm_f32(w, x, w->k, norm, y, ldy, B, epi, s, &b->gsplit);
    hipError_t e = nd_launch_digitize(x, w->k, norm, nullptr, b->digits, b->fm, B, w->k, s);
    if (e != hipSuccess) return e;
    return nd_launch_gemm(w, b->digits, b->fm, y, ldy, B, epi, s, &b->gsplit);
  };
  for (uint32_t l = 0; l < dec->layers; ++l) {
    const float* attn_norm = dec->norms + dec->attn_off + (size_t)l * D;
    const float* q_norm = dec->norms + dec->q_off + (size_t)l * kHd;
    const float* k_norm = dec->norms + dec->k_off + (size_t)l * kHd;
    if (nd_gemm_f32_fits(&dec->wqkv[l], b->x, D, true, B, &b->gsplit)) {
      // q/k/v projection with norm, rope and the cache store in its epilogue;
      // the last layer's projections are also kept (nd_batch_read_projections).
      const nd::RopeStore rs{dec->heads, dec->kv_heads, q_norm, k_norm, b->rope_tab,
                             b->positions, b->q, (int8_t*)b->kv.k, (int8_t*)b->kv.v, b->kv.ks,
                             b->kv.vs, l, b->kv.kv_heads, b->kv.alloc, dec->kv_heads};
      const bool keep = l + 1 == dec->layers;
      ND_HIP(ctx, nd_launch_gemm_f32(&dec->wqkv[l], b->x, D, attn_norm, keep ? b->qkv : nullptr,
                                     qkv_rows, B, 3, s, &b->gsplit, &rs));
    } else {
      ND_HIP(ctx, product(&dec->wqkv[l], b->x, attn_norm, b->qkv, qkv_rows, 0));
      hipLaunchKernelGGL(qk_rope_store_kernel, dim3(dec->heads + dec->kv_heads, B), dim3(64), 0,
                         s, b->qkv, qkv_rows, dec->heads, dec->kv_heads, q_norm, k_norm,
                         dec->inv_freq, nullptr, b->positions, 0u, b->q, (int8_t*)b->kv.k,
                         (int8_t*)b->kv.v, b->kv.ks, b->kv.vs, l, b->kv.kv_heads, b->kv.alloc,
                         dec->kv_heads);
      ND_HIP(ctx, hipGetLastError());
    }
    ND_HIP(ctx, nd_launch_attention_batch(&b->kv, l, b->positions, B, dec->kv_heads,
                                          dec->kv_heads, rep, max_position, b->q, b->o,
                                          b->partials, b->counters, s));
    ND_HIP(ctx, product(dec->wo[l], b->o, nullptr, b->x, D, 1));
    ND_HIP(ctx, product(dec->wup[l], b->x, dec->norms + dec->ffn_off + (size_t)l * D, b->h, F, 2));
    ND_HIP(ctx, product(dec->wdown[l], b->h, nullptr, b->x, D, 1));
  }
  ND_HIP(ctx, product(dec->embedding, b->x, dec->norms + dec->final_off, b->logits, dec->vocab, 0));
  const uint32_t words = (dec->vocab + 31) / 32;
  if (use_masks) {
    const uint32_t n = B * words;
    hipLaunchKernelGGL(gen_masks_kernel, dim3((n + 255) / 256), dim3(256), 0, s, mask_seed,
                       b->step, B, dec->vocab, threshold24, b->masks);
    ND_HIP(ctx, hipGetLastError());
  }
  const nd_select_advance adv{b->tokens, b->positions, b->step, b->history, b->lp_history,
                              b->max_length};
  bool advanced = false;
  ND_HIP(ctx, nd_launch_select_mask(b->logits, B, dec->vocab, use_masks ? b->masks : nullptr,
                                    b->ids, b->logprobs, s, b->sel_split, &adv, &advanced));
  if (!advanced) {
    hipLaunchKernelGGL(advance_kernel, dim3(1), dim3(256), 0, s, b->ids, b->logprobs, b->tokens,
                       b->positions, b->step, b->history, b->lp_history, b->max_length, B);
    ND_HIP(ctx, hipGetLastError());
  }
  return ND_OK;
}

// ----------------------------------------------------------------- prefill

struct nd_prefill {
  nd_decoder* dec = nullptr;
  uint32_t max_tokens = 0, max_context = 0, count = 0, position0 = 0;
  char* arena = nullptr;
  float *x = nullptr, *qkv = nullptr, *q = nullptr, *o = nullptr, *h = nullptr, *fm = nullptr,
        *partials = nullptr, *logits = nullptr;
  double2* rope = nullptr;  // [max_tokens][32] (sin, cos) of the pass's positions
  int8_t* digits = nullptr;
  uint32_t *tokens = nullptr, *positions = nullptr, *counters = nullptr;
  size_t partial_floats = 0;
};

nd_status nd_prefill_create(nd_ctx* ctx, nd_decoder* dec, uint32_t max_tokens,
                            uint32_t max_context, nd_prefill** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!dec || !out || max_tokens == 0 || max_tokens > 65535 || max_context < max_tokens ||
      max_context > kMaxAttentionPositions)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_prefill_create: 1..65535 tokens and max_context in [tokens, %u]",
                   kMaxAttentionPositions);
  *out = nullptr;
  nd_prefill* p = new nd_prefill();
  p->dec = dec;
  p->max_tokens = max_tokens;
  p->max_context = max_context;
  const size_t M = max_tokens;
  const uint32_t rep = dec->heads / dec->kv_heads;
  const uint32_t qkv_rows = (dec->heads + 2 * dec->kv_heads) * kHd;
  const uint32_t kmax = dec->ffn > dec->dim ? dec->ffn : dec->dim;
  // Chunks of >= 256 positions over at most max_context positions.
  p->partial_floats = nd_attention_batch_partial_floats(max_tokens, dec->kv_heads, rep,
                                                        max_context);
  const size_t sizes[] = {a256(M * dec->dim * 4),  a256(M * qkv_rows * 4), a256(M * dec->dim * 4),
                          a256(M * dec->dim * 4),  a256(M * dec->ffn * 4), a256(M * 4),
                          a256(p->partial_floats * 4), a256((size_t)dec->vocab * 4),
                          a256(3 * M * kmax),      a256(M * 4),            a256(M * 4),
                          a256(M * dec->kv_heads * kAttnCounterStride * 4), a256(M * 32 * 16)};
  size_t total = 0;
  for (size_t v : sizes) total += v;
  hipError_t e = hipMalloc(&p->arena, total);
  if (e == hipSuccess) e = hipMemsetAsync(p->arena, 0, total, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    if (p->arena) hipFree(p->arena);
    delete p;
    return nd_hip_fail(ctx, e, "prefill allocation");
  }
  char* c = p->arena;
  size_t i = 0;
  auto take = [&](void* dst) {
    *reinterpret_cast<char**>(dst) = c;
    c += sizes[i++];
  };
  take(&p->x);
  take(&p->qkv);
  take(&p->q);
  take(&p->o);
  take(&p->h);
  take(&p->fm);
  take(&p->partials);
  take(&p->logits);
  take(&p->digits);
  take(&p->tokens);
  take(&p->positions);
  take(&p->counters);
  take(&p->rope);
  *out = p;
  return ND_OK;
}

nd_status nd_prefill_free(nd_ctx* ctx, nd_prefill* p) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!p) return ND_OK;
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  hipFree(p->arena);
  delete p;
  return ND_OK;
}

static nd_status check_prefill(nd_ctx* ctx, const nd_prefill* p, const nd_kv* kv, uint32_t count,
                               uint32_t position0) {
  if (!p || !kv) return nd_fail(ctx, ND_ERR_INVALID, "prefill or cache is NULL");
  if (count == 0 || count > p->max_tokens)
    return nd_fail(ctx, ND_ERR_INVALID, "prefill of %u tokens (session holds %u)", count,
                   p->max_tokens);
  if (kv->layers != p->dec->layers || kv->kv_heads != p->dec->kv_heads || kv->window != 0 ||
      kv->mode != ND_KV_INT8 || kv->head_dim != kHd)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "prefill cache must be int8, window 0, with the decoder's layers and KV heads");
  if ((uint64_t)position0 + count > kv->max_length || (uint64_t)position0 + count > p->max_context)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Prompt ends at %u but the runtime holds %u (session %u)",
                   position0 + count, kv->max_length, p->max_context);
  return ND_OK;
}

nd_status nd_prefill_set_tokens(nd_ctx* ctx, nd_prefill* p, const uint32_t* tokens, uint32_t count,
                                uint32_t position0) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!p || !tokens || count == 0 || count > p->max_tokens)
    return nd_fail(ctx, ND_ERR_INVALID, "nd_prefill_set_tokens: bad argument");
  std::vector<uint32_t> pos(count);
  for (uint32_t i = 0; i < count; ++i) {
    if (tokens[i] >= p->dec->vocab)
      return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside the vocabulary", tokens[i]);
    pos[i] = position0 + i;
  }
  ND_HIP(ctx, hipMemcpyAsync(p->tokens, tokens, (size_t)count * 4, hipMemcpyHostToDevice, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(p->positions, pos.data(), (size_t)count * 4, hipMemcpyHostToDevice,
                             ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  p->count = count;
  p->position0 = position0;
  return ND_OK;
}

// Phase marks of a timed prefill: an event recorded after each kernel,
// with the kind of work that kernel did (GEMM, attention, other).
struct PrefillMarks {
  enum Kind { kGemm = 0, kAttention = 1, kOther = 2 };
  std::vector<hipEvent_t> events;
  std::vector<int> kinds;
  hipError_t mark(int kind, hipStream_t s) {
    hipEvent_t e;
    hipError_t err = hipEventCreate(&e);
    if (err != hipSuccess) return err;
    events.push_back(e);
    kinds.push_back(kind);
    return hipEventRecord(e, s);
  }
  ~PrefillMarks() {
    for (hipEvent_t e : events) hipEventDestroy(e);
  }
};

static nd_status enqueue_prefill(nd_ctx* ctx, nd_prefill* p, nd_kv* kv, hipStream_t s,
                                 PrefillMarks* marks) {
  const nd_decoder* dec = p->dec;
  const uint32_t M = p->count, D = dec->dim, F = dec->ffn;
  const uint32_t qkv_rows = (dec->heads + 2 * dec->kv_heads) * kHd;
  const uint32_t rep = dec->heads / dec->kv_heads;
  const uint32_t last = p->position0 + M - 1;
  auto mark = [&](int kind) -> hipError_t {
    return marks ? marks->mark(kind, s) : hipSuccess;
  };
  constexpr int G = PrefillMarks::kGemm, A = PrefillMarks::kAttention, O = PrefillMarks::kOther;
  ND_HIP(ctx, mark(O));
  hipLaunchKernelGGL(embed_kernel, dim3((D + 255) / 256, M), dim3(256), 0, s, dec->embedding->w,
                     dec->embedding->scales, p->tokens, dec->vocab, D, std::sqrt((double)D), p->x);
  ND_HIP(ctx, hipGetLastError());
  hipLaunchKernelGGL(rope_table_kernel, dim3((M * 32 + 255) / 256), dim3(256), 0, s, dec->inv_freq,
                     p->position0, M, p->rope);
  ND_HIP(ctx, hipGetLastError());
  ND_HIP(ctx, mark(O));
  for (uint32_t l = 0; l < dec->layers; ++l) {
    ND_HIP(ctx, nd_launch_digitize(p->x, D, dec->norms + dec->attn_off + (size_t)l * D, nullptr,
                                   p->digits, p->fm, M, D, s));
    ND_HIP(ctx, mark(O));
    ND_HIP(ctx, nd_launch_gemm(&dec->wqkv[l], p->digits, p->fm, p->qkv, qkv_rows, M, 0, s));
    ND_HIP(ctx, mark(G));
    hipLaunchKernelGGL(qk_rope_store_kernel, dim3(dec->heads + dec->kv_heads, M), dim3(64), 0, s,
                       p->qkv, qkv_rows, dec->heads, dec->kv_heads,
                       dec->norms + dec->q_off + (size_t)l * kHd,
                       dec->norms + dec->k_off + (size_t)l * kHd, dec->inv_freq, p->rope,
                       nullptr, p->position0, p->q, (int8_t*)kv->k, (int8_t*)kv->v, kv->ks,
                       kv->vs, l, kv->kv_heads, kv->alloc, 0u);
    ND_HIP(ctx, hipGetLastError());
    ND_HIP(ctx, mark(O));
    ND_HIP(ctx, nd_launch_attention_batch(kv, l, p->positions, M, dec->kv_heads, 0u, rep, last,
                                          p->q, p->o, p->partials, p->counters, s));
    ND_HIP(ctx, mark(A));
    ND_HIP(ctx, nd_launch_digitize(p->o, D, nullptr, nullptr, p->digits, p->fm, M, D, s));
    ND_HIP(ctx, mark(O));
    ND_HIP(ctx, nd_launch_gemm(dec->wo[l], p->digits, p->fm, p->x, D, M, 1, s));
    ND_HIP(ctx, mark(G));
    ND_HIP(ctx, nd_launch_digitize(p->x, D, dec->norms + dec->ffn_off + (size_t)l * D, nullptr,
                                   p->digits, p->fm, M, D, s));
    ND_HIP(ctx, mark(O));
    ND_HIP(ctx, nd_launch_gemm(dec->wup[l], p->digits, p->fm, p->h, F, M, 2, s));
    ND_HIP(ctx, mark(G));
    ND_HIP(ctx, nd_launch_digitize(p->h, F, nullptr, nullptr, p->digits, p->fm, M, F, s));
    ND_HIP(ctx, mark(O));
    ND_HIP(ctx, nd_launch_gemm(dec->wdown[l], p->digits, p->fm, p->x, D, M, 1, s));
    ND_HIP(ctx, mark(G));
  }
  ND_HIP(ctx, nd_launch_digitize(p->x + (size_t)(M - 1) * D, D, dec->norms + dec->final_off,
                                 nullptr, p->digits, p->fm, 1, D, s));
  ND_HIP(ctx, mark(O));
  ND_HIP(ctx, nd_launch_gemm(dec->embedding, p->digits, p->fm, p->logits, dec->vocab, 1, 0, s));
  ND_HIP(ctx, mark(G));
  return ND_OK;
}

// Enqueues the prefill of the tokens set by nd_prefill_set_tokens: every
// layer runs as M-row GEMMs on int8 MFMA; all M positions' K/V are quantized
// into the cache first, then each position attends causally over [0, its
// position] of the int8 cache -- the same reads 2048 sequential steps make,
// since a step stores its own K/V before its attention (runtime.ts:501-502).
// The last position's logits stay in HBM (nd_prefill_logits copies them).
nd_status nd_prefill_run_d(nd_ctx* ctx, nd_prefill* p, nd_kv* kv, void* stream) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_prefill(ctx, p, kv, p ? p->count : 0, p ? p->position0 : 0);
  if (st != ND_OK) return st;
  return enqueue_prefill(ctx, p, kv, nd_pick_stream(ctx, stream), nullptr);
}

nd_status nd_prefill_phase_ms(nd_ctx* ctx, nd_prefill* p, nd_kv* kv, float* ms) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!ms) return nd_fail(ctx, ND_ERR_INVALID, "ms is NULL");
  nd_status st = check_prefill(ctx, p, kv, p ? p->count : 0, p ? p->position0 : 0);
  if (st != ND_OK) return st;
  PrefillMarks marks;
  st = enqueue_prefill(ctx, p, kv, ctx->stream, &marks);
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  if (st != ND_OK) return st;
  ms[0] = ms[1] = ms[2] = 0.f;
  for (size_t i = 1; i < marks.events.size(); ++i) {
    float t = 0.f;
    ND_HIP(ctx, hipEventElapsedTime(&t, marks.events[i - 1], marks.events[i]));
    ms[marks.kinds[i]] += t;
  }
  return ND_OK;
}

nd_status nd_prefill_logits(nd_ctx* ctx, nd_prefill* p, float* logits) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!p || !logits) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  ND_HIP(ctx, hipMemcpyAsync(logits, p->logits, (size_t)p->dec->vocab * 4, hipMemcpyDeviceToHost,
                             ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_prefill_read_projections(nd_ctx* ctx, nd_prefill* p, float* out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!p || !out) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  if (p->count == 0) return nd_fail(ctx, ND_ERR_INVALID, "the prefill has not run");
  const size_t rows = (size_t)(p->dec->heads + 2 * p->dec->kv_heads) * kHd;
  ND_HIP(ctx, hipMemcpyAsync(out, p->qkv, (size_t)p->count * rows * 4, hipMemcpyDeviceToHost,
                             ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_prefill_tokens(nd_ctx* ctx, nd_prefill* p, nd_kv* kv, const uint32_t* tokens,
                            uint32_t count, uint32_t position0, float* logits) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_prefill(ctx, p, kv, count, position0);
  if (st != ND_OK) return st;
  if ((st = nd_prefill_set_tokens(ctx, p, tokens, count, position0)) != ND_OK) return st;
  if ((st = nd_prefill_run_d(ctx, p, kv, nullptr)) != ND_OK) return st;
  if (logits) return nd_prefill_logits(ctx, p, logits);
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_batch_history(nd_ctx* ctx, nd_batch* b, uint32_t first_step, uint32_t steps,
                           uint32_t* ids, double* log_probabilities) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!b) return nd_fail(ctx, ND_ERR_INVALID, "batch is NULL");
  if ((uint64_t)first_step + steps > b->max_length)
    return nd_fail(ctx, ND_ERR_INVALID, "history holds steps [0, %u)", b->max_length);
  const size_t off = (size_t)first_step * b->batch, n = (size_t)steps * b->batch;
  if (ids)
    ND_HIP(ctx, hipMemcpyAsync(ids, b->history + off, n * 4, hipMemcpyDeviceToHost, ctx->stream));
  if (log_probabilities)
    ND_HIP(ctx, hipMemcpyAsync(log_probabilities, b->lp_history + off, n * 8,
                               hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

}  // extern "C"
