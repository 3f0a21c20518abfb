// Needle 2 on the GPU at batch 1: the per-token graph of NeedleRuntime.step
// (model/runtime.ts:280-583) with HBM-resident int8 weights, engram ring and
// int8 KV cache (sliding window + sinks).
//
// The token and position live in device memory (`st`, `history`): the step's
// first kernel takes the token (from a kernel argument, from the prompt
// already in `history`, or from the previous step's selection), appends it
// and advances the position, and every later kernel reads the position back.
// So one step's launches form a fixed sequence that is captured once as a
// HIP graph and replayed per token with no host copies.
//
// Per layer the token runs six launches: mhc_pre (one workgroup: lane RMS,
// the lanes*(2+lanes) phi rows, h-pre mix, engram injection, input norm), the
// fused Q/K/V/gate matvec, qk norm + RoPE + KV append, attention with the
// sigmoid(gate) epilogue, the Wo matvec, and mhc_post (one workgroup:
// sandwich norm, Hadamard MLP, h-post, Sinkhorn routing, lane update).  The
// one-workgroup kernels keep the reference's float64-with-f32-stores
// arithmetic, which costs nothing at these sizes.
#include <algorithm>
#include <cmath>
#include <type_traits>
#include <vector>

#include "nd_internal.hpp"

namespace {

constexpr uint32_t kHd = 64;
constexpr int kWg = 1024;

__device__ __forceinline__ double sigmoid_d(double v) {
  if (v >= 0) return 1.0 / (1.0 + exp(-v));
  const double e = exp(v);
  return e / (1.0 + e);
}

// Sum over a workgroup of kWg threads; every thread gets the total.
__device__ __forceinline__ double block_sum_d(double v, double* red) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  __syncthreads();
  if (lane == 0) red[w] = v;
  __syncthreads();
  double r = 0.0;
  for (int i = 0; i < kWg / 64; ++i) r += red[i];
  return r;
}

// JavaScript Math.max over |v| of a wave: NaN wins.
__device__ __forceinline__ float wave_absmax_js(float v) {
  v = fabsf(v);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) {
    const float w = __shfl_xor(v, o, 64);
    v = (v != v || w != w) ? __builtin_nanf("") : (v > w ? v : w);
  }
  return v;
}

// #kvSlot (model/runtime.ts:659-667).
__device__ __forceinline__ uint32_t kv_slot(uint32_t p, uint32_t sink, uint32_t window) {
  if (window == 0 || p < sink) return p;
  return sink + (p - sink) % window;
}

enum TokenSource : uint32_t { kTokenArg = 0, kTokenHistory = 1, kTokenSelected = 2 };

struct BeginArgs {
  uint32_t* st;  // st[0] = next position, st[1] = this step's position
  uint32_t* history;
  double* lp_history;
  const uint32_t* selected_id;
  const double* selected_lp;
  uint32_t token_arg, source;
  const int8_t* emb;
  const float* emb_s;
  uint32_t d, lanes;
  double scale;
  float* x;
  const int8_t* tw[4];
  const float* ts[4];
  uint32_t n_sites, tables, slots, sub, per_order, n_orders;
  uint32_t orders[4];
  float* cat;
};

// Token intake, engram hashing (runtime.ts:788-818), the scaled embedding
// row in every lane (runtime.ts:305-313) and the concatenated engram rows of
// every site (runtime.ts:828-836; zero for a table whose n-gram is not
// complete yet).  One workgroup.
__global__ __launch_bounds__(kWg) void n2_begin_kernel(BeginArgs a) {
  __shared__ uint32_t s_tok, s_pos, s_idx[16], s_valid[16];
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    const uint32_t p = a.st[0];
    uint32_t tok;
    if (a.source == kTokenHistory) {
      tok = a.history[p];
    } else if (a.source == kTokenSelected) {
      tok = *a.selected_id;
      a.history[p] = tok;
      a.lp_history[p] = *a.selected_lp;
    } else {
      tok = a.token_arg;
      a.history[p] = tok;
    }
    a.st[1] = p;
    a.st[0] = p + 1;
    s_tok = tok;
    s_pos = p;
  }
  __syncthreads();
  const uint32_t tok = s_tok, pos = s_pos;
  if (t < a.tables) {
    const uint32_t order = a.orders[t / a.per_order];
    uint32_t hash = 0x9E3779B9u * (t + 1);
    bool valid = true;
    for (uint32_t off = 0; off < order; ++off) {
      const bool in = off <= pos;
      const uint32_t token = off == 0 ? tok : (in ? a.history[pos - off] : 0u);
      hash = (hash ^ token) * 0x01000193u;
      if (off == order - 1) valid = in;
    }
    hash ^= hash >> 15;
    s_idx[t] = hash % a.slots;
    s_valid[t] = valid ? 1u : 0u;
  }
  __syncthreads();
  for (uint32_t k = t; k < a.d; k += kWg) {
    const float row = (float)a.emb[(size_t)tok * a.d + k] * a.emb_s[tok];
    const float v = (float)((double)row * a.scale);
    for (uint32_t l = 0; l < a.lanes; ++l) a.x[(size_t)l * a.d + k] = v;
  }
  const uint32_t per_site = a.tables * a.sub;
  for (uint32_t i = t; i < a.n_sites * per_site; i += kWg) {
    const uint32_t s = i / per_site, j = i % per_site, tb = j / a.sub, c = j % a.sub;
    float v = 0.f;
    if (s_valid[tb]) {
      const size_t row = (size_t)tb * a.slots + s_idx[tb];
      v = (float)a.tw[s][row * a.sub + c] * a.ts[s][row];
    }
    a.cat[i] = v;
  }
}

// runtime.ts:854-872: the value row of this position goes into the ring,
// then the taps mix the ring rows at position - tap * max_order (a slot of a
// non-negative earlier position is always written, so the reference's valid
// flag reduces to prev >= 0).  ekv[s] = [key (d) | value now (d)].
__global__ void n2_engram_conv_kernel(const uint32_t* __restrict__ st,
                                      const float* __restrict__ ekv, float* __restrict__ ring,
                                      const float* __restrict__ taps, uint32_t d, uint32_t depth,
                                      uint32_t n_taps, uint32_t max_order,
                                      float* __restrict__ mixed) {
  const uint32_t s = blockIdx.x, i = threadIdx.x;
  if (i >= d) return;
  const uint32_t pos = st[1];
  float* r = ring + (size_t)s * depth * d;
  r[(size_t)(pos % depth) * d + i] = ekv[(size_t)s * 2 * d + d + i];
  float m = 0.f;
  for (uint32_t tap = 0; tap < n_taps; ++tap) {
    if (tap * max_order > pos) continue;
    const uint32_t ps = (pos - tap * max_order) % depth;
    m = (float)((double)m + (double)taps[((size_t)s * n_taps + tap) * d + i] *
                                (double)r[(size_t)ps * d + i]);
  }
  mixed[(size_t)s * d + i] = m;
}

struct PreArgs {
  const float* x;           // [lanes][d]
  const int8_t* phi_pre;    // this layer's rows
  const float* phi_pre_s;
  const int8_t* phi_post;
  const float* phi_post_s;
  const int8_t* phi_res;
  const float* phi_res_s;
  float a_pre;
  const float* b_pre;       // [lanes]
  const float* ekey;        // engram key of this layer's site, or null
  const float* evalue;
  const float* norm_input;  // [d]
  float* upd;               // out [d]
  float* blk;               // out [d]
  float* ain;               // out [d]
  float* phi_post_out;      // out [lanes]
  float* phi_res_out;       // out [lanes*lanes]
  uint32_t d, lanes, own;
};

// mHC pre-mix (runtime.ts:385-420), engram injection (runtime.ts:422-438)
// and the input norm (runtime.ts:441) in one workgroup.
__global__ __launch_bounds__(kWg) void n2_mhc_pre_kernel(PreArgs a) {
  __shared__ float nl[2048];
  __shared__ float xs[2048];
  __shared__ float phi[24];
  __shared__ float hpre[4];
  __shared__ double red[kWg / 64];
  const uint32_t t = threadIdx.x, D = a.d, L = a.lanes, N = L * D;
  // rmsUnit over all lanes (math.ts:34-44).
  double ss = 0.0;
  for (uint32_t i = t; i < N; i += kWg) {
    const float v = a.x[i];
    xs[i] = v;
    ss += (double)v * (double)v;
  }
  ss = block_sum_d(ss, red);
  const double inv = 1.0 / sqrt(ss / N + 1e-6);
  for (uint32_t i = t; i < N; i += kWg) nl[i] = (float)((double)xs[i] * inv);
  __syncthreads();
  // The phi rows (K = lanes * d): one wave per row, float64 dot, f32 store.
  const uint32_t wave = t >> 6, lane = t & 63, nrows = 2 * L + L * L;
  for (uint32_t r = wave; r < nrows; r += kWg / 64) {
    const int8_t* w;
    float sc;
    if (r < L) {
      w = a.phi_pre + (size_t)r * N;
      sc = a.phi_pre_s[r];
    } else if (r < 2 * L) {
      w = a.phi_post + (size_t)(r - L) * N;
      sc = a.phi_post_s[r - L];
    } else {
      w = a.phi_res + (size_t)(r - 2 * L) * N;
      sc = a.phi_res_s[r - 2 * L];
    }
    double dot = 0.0;
    for (uint32_t i = lane * 4; i < N; i += 256) {
      const char4 c = *reinterpret_cast<const char4*>(w + i);
      dot += (double)c.x * (double)nl[i] + (double)c.y * (double)nl[i + 1] +
             (double)c.z * (double)nl[i + 2] + (double)c.w * (double)nl[i + 3];
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) dot += __shfl_xor(dot, o, 64);
    if (lane == 0) phi[r] = (float)((double)sc * dot);
  }
  __syncthreads();
  if (t < L) {
    const double off = t == a.own ? 4.0 : -4.0;
    hpre[t] = (float)sigmoid_d((double)a.a_pre * (double)phi[t] + (double)a.b_pre[t] + off);
    a.phi_post_out[t] = phi[L + t];
  }
  if (t < L * L) a.phi_res_out[t] = phi[2 * L + t];
  __syncthreads();
  // updateInput = sum_lane hPre[lane] * x[lane].
  float u = 0.f;
  if (t < D) {
    double sum = 0.0;
    for (uint32_t l = 0; l < L; ++l) sum += (double)hpre[l] * (double)xs[l * D + t];
    u = (float)sum;
    a.upd[t] = u;
  }
  float b = u;
  if (a.ekey) {
    // alpha = sigmoid(rmsUnit(u) . rmsUnit(key) / sqrt(d)); block = u + alpha * value.
    const float kk = t < D ? a.ekey[t] : 0.f;
    const double su = block_sum_d(t < D ? (double)u * u : 0.0, red);
    const double sk = block_sum_d(t < D ? (double)kk * kk : 0.0, red);
    const double iu = 1.0 / sqrt(su / D + 1e-6), ik = 1.0 / sqrt(sk / D + 1e-6);
    const float nu = (float)((double)u * iu), nk = (float)((double)kk * ik);
    const double dot = block_sum_d(t < D ? (double)nu * (double)nk : 0.0, red);
    const double alpha = sigmoid_d(dot / sqrt((double)D));
    if (t < D) b = (float)((double)u + alpha * (double)a.evalue[t]);
  }
  if (t < D) a.blk[t] = b;
  // attentionInput = rmsNorm(block, normInput) (math.ts:16-32).
  const double sb = block_sum_d(t < D ? (double)b * b : 0.0, red);
  const double ib = 1.0 / sqrt(sb / D + 1e-6);
  if (t < D) a.ain[t] = (float)((1.0 + (double)a.norm_input[t]) * (double)b * ib);
}

// Query/key head norm + RoPE and the KV append at the ring slot
// (runtime.ts:471-501, #storeKV runtime.ts:679-717).  One wave per head, lane
// = dimension.  qkvg = [q (H*64) | k (Hkv*64) | v (Hkv*64) | gate (H*64)].
__global__ __launch_bounds__(64) void n2_qk_rope_store_kernel(
    const uint32_t* __restrict__ st, const float* __restrict__ qkvg, uint32_t heads,
    uint32_t kv_heads, const float* __restrict__ q_norm, const float* __restrict__ k_norm,
    const double* __restrict__ inv_freq, float* __restrict__ q_out, int8_t* __restrict__ Kc,
    int8_t* __restrict__ Vc, float* __restrict__ Ks, float* __restrict__ Vs, uint32_t layer,
    uint32_t alloc, uint32_t sink, uint32_t window) {
  const uint32_t slot_h = blockIdx.x, lane = threadIdx.x;
  const uint32_t pos = st[1];
  const bool is_q = slot_h < heads;
  const uint32_t h = is_q ? slot_h : slot_h - heads;
  const float* src = qkvg + (is_q ? h * kHd : heads * kHd + h * kHd);
  const float* scale = is_q ? q_norm : k_norm;
  const double x = src[lane];
  double ss = x * x;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
  const double inv = 1.0 / sqrt(ss / kHd + 1e-6);
  const float normed = (float)((1.0 + (double)scale[lane]) * x * inv);
  double sn, cs;
  sincos((double)pos * inv_freq[lane & 31], &sn, &cs);
  const double mine = normed;
  const double other = __shfl_xor(mine, 32, 64);
  const float rot = lane < 32 ? (float)(mine * cs - other * sn) : (float)(mine * cs + other * sn);
  if (is_q) {
    q_out[h * kHd + lane] = rot;
    return;
  }
  const uint32_t slot = kv_slot(pos, sink, window);
  if (slot >= alloc) return;  // the host keeps positions below the runtime limit
  const size_t row = ((size_t)layer * kv_heads + h) * alloc + slot;
  const float vv = qkvg[(heads + kv_heads) * kHd + h * kHd + lane];
  const float ak = wave_absmax_js(rot), av = wave_absmax_js(vv);
  const double mk = (ak != ak) ? (double)ak : fmax(1e-12, (double)ak);
  const double mv = (av != av) ? (double)av : fmax(1e-12, (double)av);
  const double sk = mk / 127.0, sv = mv / 127.0;
  const double ck = rint((double)rot / sk), cv = rint((double)vv / sv);
  Kc[row * kHd + lane] = ck != ck ? (int8_t)0 : (int8_t)(int)ck;
  Vc[row * kHd + lane] = cv != cv ? (int8_t)0 : (int8_t)(int)cv;
  if (lane == 0) {
    Ks[row] = (float)sk;
    Vs[row] = (float)sv;
  }
}

struct PostArgs {
  float* x;                 // [lanes][d], updated in place
  const float* proj;        // Wo output [d]
  const float* blk;
  const float* upd;
  const float* post_norm;   // [d]
  const float* pre_h_norm;  // [d]
  const float* d1;          // [d]
  const float* d2;          // [hdim]
  const float* d3;          // [d]
  float attention_gate;
  const float* phi_post;    // [lanes]
  const float* phi_res;     // [lanes*lanes]
  float a_post, a_res;
  const float* b_post;      // [lanes]
  const float* b_res;       // [lanes*lanes]
  uint32_t d, hdim, lanes, own;
};

// runtime.ts:509-542 with #attentionDelta (runtime.ts:585-611), hadamardMlp
// (math.ts:117-138), fwht (f32 store per butterfly) and sinkhorn
// (math.ts:62-92), in one workgroup.
__global__ __launch_bounds__(kWg) void n2_mhc_post_kernel(PostArgs a) {
  __shared__ float hv[1024];
  __shared__ double red[kWg / 64];
  __shared__ float routing[16];
  __shared__ float hpost[4];
  const uint32_t t = threadIdx.x, D = a.d, H = a.hdim, L = a.lanes;
  // afterAttention = block + sigmoid(gate) * rmsNorm(projected, postNorm).
  const float p = t < D ? a.proj[t] : 0.f;
  const double sp = block_sum_d(t < D ? (double)p * p : 0.0, red);
  const double ip = 1.0 / sqrt(sp / D + 1e-6);
  const double ascale = sigmoid_d((double)a.attention_gate);
  float after = 0.f;
  if (t < D) {
    const float np = (float)((1.0 + (double)a.post_norm[t]) * (double)p * ip);
    after = (float)((double)a.blk[t] + ascale * (double)np);
  }
  const double sa = block_sum_d(t < D ? (double)after * after : 0.0, red);
  const double ia = 1.0 / sqrt(sa / D + 1e-6);
  // Hadamard MLP: FWHT(d1 * x), SiLU(z / sqrt(H) * d2), FWHT, / sqrt(H) * d3.
  if (t < H) {
    float v = 0.f;
    if (t < D) {
      const float pre = (float)((1.0 + (double)a.pre_h_norm[t]) * (double)after * ia);
      v = (float)((double)pre * (double)a.d1[t]);
    }
    hv[t] = v;
  }
  const double inv_root = 1.0 / sqrt((double)H);
  for (int pass = 0; pass < 2; ++pass) {
    __syncthreads();
    for (uint32_t stride = 1; stride < H; stride <<= 1) {
      if (t < H / 2) {
        const uint32_t li = (t / stride) * 2 * stride + t % stride, ri = li + stride;
        const double left = hv[li], right = hv[ri];
        hv[li] = (float)(left + right);
        hv[ri] = (float)(left - right);
      }
      __syncthreads();
    }
    if (pass == 0 && t < H) {
      const double z = (double)hv[t] * inv_root * (double)a.d2[t];
      hv[t] = (float)(z * sigmoid_d(z));
    }
  }
  float delta = 0.f;
  if (t < D) {
    const float mlp = (float)((double)hv[t] * inv_root * (double)a.d3[t]);
    delta = (float)((double)after + (double)mlp - (double)a.upd[t]);
  }
  if (t == 0) {
    for (uint32_t l = 0; l < L; ++l) {
      const double off = l == a.own ? 0.0 : -4.0;
      hpost[l] = (float)(2.0 * sigmoid_d((double)a.a_post * (double)a.phi_post[l] +
                                         (double)a.b_post[l] + off));
    }
    // Sinkhorn: twenty log-space row then column normalizations in float64.
    double r[16];
    for (uint32_t i = 0; i < L * L; ++i)
      r[i] = (double)(float)((double)a.a_res * (double)a.phi_res[i] + (double)a.b_res[i]);
    for (int it = 0; it < 20; ++it) {
      for (uint32_t row = 0; row < L; ++row) {
        double mx = r[row * L];
        for (uint32_t c = 1; c < L; ++c) {
          const double v = r[row * L + c];
          mx = (mx != mx || v != v) ? (double)NAN : fmax(mx, v);
        }
        double sum = 0.0;
        for (uint32_t c = 0; c < L; ++c) sum += exp(r[row * L + c] - mx);
        const double ls = log(sum) + mx;
        for (uint32_t c = 0; c < L; ++c) r[row * L + c] -= ls;
      }
      for (uint32_t c = 0; c < L; ++c) {
        double mx = r[c];
        for (uint32_t row = 1; row < L; ++row) {
          const double v = r[row * L + c];
          mx = (mx != mx || v != v) ? (double)NAN : fmax(mx, v);
        }
        double sum = 0.0;
        for (uint32_t row = 0; row < L; ++row) sum += exp(r[row * L + c] - mx);
        const double ls = log(sum) + mx;
        for (uint32_t row = 0; row < L; ++row) r[row * L + c] -= ls;
      }
    }
    for (uint32_t i = 0; i < L * L; ++i) routing[i] = (float)exp(r[i]);
  }
  __syncthreads();
  if (t < D) {
    float old[4];
    for (uint32_t l = 0; l < L; ++l) old[l] = a.x[(size_t)l * D + t];
    for (uint32_t l = 0; l < L; ++l) {
      double sum = 0.0;
      for (uint32_t src = 0; src < L; ++src) sum += (double)routing[l * L + src] * (double)old[src];
      a.x[(size_t)l * D + t] = (float)(sum + (double)hpost[l] * (double)delta);
    }
  }
}

// runtime.ts:570-576: lane mean, then rmsNorm(finalNorm).
__global__ __launch_bounds__(kWg) void n2_final_kernel(const float* __restrict__ x,
                                                      const float* __restrict__ norm, uint32_t d,
                                                      uint32_t lanes, float* __restrict__ out) {
  __shared__ double red[kWg / 64];
  const uint32_t t = threadIdx.x;
  float m = 0.f;
  if (t < d) {
    double sum = 0.0;
    for (uint32_t l = 0; l < lanes; ++l) sum += x[(size_t)l * d + t];
    m = (float)(sum / lanes);
  }
  const double ss = block_sum_d(t < d ? (double)m * m : 0.0, red);
  const double inv = 1.0 / sqrt(ss / d + 1e-6);
  if (t < d) out[t] = (float)((1.0 + (double)norm[t]) * (double)m * inv);
}

size_t al(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace

struct nd_needle {
  nd_needle_desc d{};
  std::vector<nd_mat> wqkvg;  // owned: rows q | k | v | gate of each layer
  std::vector<nd_mat> ekv;    // owned: rows key | value of each engram site
  std::vector<const nd_mat*> wo, eg_tables;
  const nd_mat *embedding = nullptr, *phi_pre = nullptr, *phi_post = nullptr, *phi_res = nullptr;
  float* params = nullptr;  // dense vectors, offsets below (floats)
  size_t o_norm_input = 0, o_qn = 0, o_kn = 0, o_post = 0, o_preh = 0, o_d1 = 0, o_d2 = 0,
         o_d3 = 0, o_bpre = 0, o_bpost = 0, o_bres = 0, o_taps = 0, o_final = 0;
  std::vector<float> attention_gate, a_pre, a_post, a_res;
  double* inv_freq = nullptr;
  uint32_t max_order = 1, depth = 1;
  // Runtime state (allocated by the first reset for the model's max_length).
  nd_kv kv{};
  char* arena = nullptr;
  size_t state_bytes = 0;  // leading part of the arena cleared by reset
  uint32_t *st = nullptr, *history = nullptr, *sel_id = nullptr, *allowed = nullptr;
  double *lp_history = nullptr, *sel_lp = nullptr;
  float *ring = nullptr, *x = nullptr, *upd = nullptr, *blk = nullptr, *ain = nullptr,
        *qkvg = nullptr, *q = nullptr, *att = nullptr, *proj = nullptr, *phi_post_v = nullptr,
        *phi_res_v = nullptr, *fin = nullptr, *logits = nullptr, *cat = nullptr, *ekv_out = nullptr,
        *evals = nullptr, *partials = nullptr;
  uint32_t max_length = 0, sink = 0, position = 0;
  // Step graphs, valid for (graph_alloc, graph_sink).
  hipGraphExec_t graphs[3] = {nullptr, nullptr, nullptr};
  uint32_t graph_alloc = 0, graph_sink = 0;
};

namespace {

void drop_graphs(nd_needle* n) {
  for (auto& g : n->graphs) {
    if (g) hipGraphExecDestroy(g);
    g = nullptr;
  }
}

// Enqueues one token of NeedleRuntime.step (model/runtime.ts:280-583) on s.
// select: after the logits, selectToken over allowed[0..count) (all ids when
// allowed is null) into sel_id / sel_lp.
hipError_t enqueue_step(nd_needle* n, uint32_t source, uint32_t token, bool want_logits,
                        bool select, const uint32_t* allowed, uint32_t count, hipStream_t s) {
  const nd_needle_desc& d = n->d;
  const uint32_t D = d.dim, ln = d.lanes, qw = d.heads * kHd, kw = d.kv_heads * kHd;
  BeginArgs b{};
  b.st = n->st;
  b.history = n->history;
  b.lp_history = n->lp_history;
  b.selected_id = n->sel_id;
  b.selected_lp = n->sel_lp;
  b.token_arg = token;
  b.source = source;
  b.emb = n->embedding->w;
  b.emb_s = n->embedding->scales;
  b.d = D;
  b.lanes = ln;
  b.scale = std::sqrt((double)D);
  b.x = n->x;
  for (uint32_t si = 0; si < d.n_sites; ++si) {
    b.tw[si] = n->eg_tables[si]->w;
    b.ts[si] = n->eg_tables[si]->scales;
  }
  b.n_sites = d.n_sites;
  b.tables = d.n_sites ? d.engram_tables : 0;
  b.slots = d.engram_slots;
  b.sub = d.engram_sub;
  b.n_orders = d.n_orders;
  b.per_order = d.n_orders ? d.engram_tables / d.n_orders : 1;
  for (uint32_t i = 0; i < d.n_orders; ++i) b.orders[i] = d.orders[i];
  b.cat = n->cat;
  hipLaunchKernelGGL(n2_begin_kernel, dim3(1), dim3(kWg), 0, s, b);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const uint32_t cat = d.engram_tables * d.engram_sub;
  for (uint32_t si = 0; si < d.n_sites; ++si) {
    e = nd_launch_matvec(&n->ekv[si], n->cat + (size_t)si * cat, 1, cat, 0, 2 * D,
                         n->ekv_out + (size_t)si * 2 * D, 2 * D, s);
    if (e != hipSuccess) return e;
  }
  if (d.n_sites) {
    hipLaunchKernelGGL(n2_engram_conv_kernel, dim3(d.n_sites), dim3((D + 63) / 64 * 64), 0, s,
                       n->st, n->ekv_out, n->ring, n->params + n->o_taps, D, n->depth,
                       d.engram_taps, n->max_order, n->evals);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  const size_t K = (size_t)ln * D;
  for (uint32_t l = 0; l < d.layers; ++l) {
    const uint32_t own = l % ln;
    int site = -1;
    for (uint32_t si = 0; si < d.n_sites; ++si)
      if (d.sites[si] == l) site = (int)si;
    PreArgs pa{};
    pa.x = n->x;
    pa.phi_pre = n->phi_pre->w + (size_t)l * ln * K;
    pa.phi_pre_s = n->phi_pre->scales + (size_t)l * ln;
    pa.phi_post = n->phi_post->w + (size_t)l * ln * K;
    pa.phi_post_s = n->phi_post->scales + (size_t)l * ln;
    pa.phi_res = n->phi_res->w + (size_t)l * ln * ln * K;
    pa.phi_res_s = n->phi_res->scales + (size_t)l * ln * ln;
    pa.a_pre = n->a_pre[l];
    pa.b_pre = n->params + n->o_bpre + (size_t)l * ln;
    pa.ekey = site >= 0 ? n->ekv_out + (size_t)site * 2 * D : nullptr;
    pa.evalue = site >= 0 ? n->evals + (size_t)site * D : nullptr;
    pa.norm_input = n->params + n->o_norm_input + (size_t)l * D;
    pa.upd = n->upd;
    pa.blk = n->blk;
    pa.ain = n->ain;
    pa.phi_post_out = n->phi_post_v;
    pa.phi_res_out = n->phi_res_v;
    pa.d = D;
    pa.lanes = ln;
    pa.own = own;
    hipLaunchKernelGGL(n2_mhc_pre_kernel, dim3(1), dim3(kWg), 0, s, pa);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    const nd_mat& wm = n->wqkvg[l];
    if ((e = nd_launch_matvec(&wm, n->ain, 1, D, 0, wm.n, n->qkvg, wm.n, s)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(n2_qk_rope_store_kernel, dim3(d.heads + d.kv_heads), dim3(64), 0, s, n->st,
                       n->qkvg, d.heads, d.kv_heads, n->params + n->o_qn + (size_t)l * kHd,
                       n->params + n->o_kn + (size_t)l * kHd, n->inv_freq, n->q,
                       (int8_t*)n->kv.k, (int8_t*)n->kv.v, n->kv.ks, n->kv.vs, l, n->kv.alloc,
                       n->kv.sink, n->kv.window);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    e = nd_launch_attention_gated(&n->kv, l, n->st + 1, n->max_length - 1, n->q, d.heads,
                                  n->qkvg + qw + 2 * kw, n->att, n->partials, s);
    if (e != hipSuccess) return e;
    if ((e = nd_launch_matvec(n->wo[l], n->att, 1, qw, 0, D, n->proj, D, s)) != hipSuccess)
      return e;
    PostArgs qa{};
    qa.x = n->x;
    qa.proj = n->proj;
    qa.blk = n->blk;
    qa.upd = n->upd;
    qa.post_norm = n->params + n->o_post + (size_t)l * D;
    qa.pre_h_norm = n->params + n->o_preh + (size_t)l * D;
    qa.d1 = n->params + n->o_d1 + (size_t)l * D;
    qa.d2 = n->params + n->o_d2 + (size_t)l * d.hadamard;
    qa.d3 = n->params + n->o_d3 + (size_t)l * D;
    qa.attention_gate = n->attention_gate[l];
    qa.phi_post = n->phi_post_v;
    qa.phi_res = n->phi_res_v;
    qa.a_post = n->a_post[l];
    qa.a_res = n->a_res[l];
    qa.b_post = n->params + n->o_bpost + (size_t)l * ln;
    qa.b_res = n->params + n->o_bres + (size_t)l * ln * ln;
    qa.d = D;
    qa.hdim = d.hadamard;
    qa.lanes = ln;
    qa.own = own;
    hipLaunchKernelGGL(n2_mhc_post_kernel, dim3(1), dim3(kWg), 0, s, qa);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  if (!want_logits && !select) return hipSuccess;
  hipLaunchKernelGGL(n2_final_kernel, dim3(1), dim3(kWg), 0, s, n->x, n->params + n->o_final, D,
                     ln, n->fin);
  if ((e = hipGetLastError()) != hipSuccess) return e;
  e = nd_launch_matvec(n->embedding, n->fin, 1, D, 0, d.vocab, n->logits, d.vocab, s);
  if (e != hipSuccess || !select) return e;
  return nd_launch_select_list(n->logits, d.vocab, allowed, count, n->sel_id, n->sel_lp, s);
}

enum GraphKind { kGraphPrompt = 0, kGraphPromptSelect = 1, kGraphDecodeSelect = 2 };

// Launches the step graph of `kind`, capturing and instantiating it first if
// the cached one was built for another cache geometry.
nd_status launch_graph(nd_ctx* ctx, nd_needle* n, GraphKind kind) {
  if (n->graph_alloc != n->kv.alloc || n->graph_sink != n->kv.sink) {
    drop_graphs(n);
    n->graph_alloc = n->kv.alloc;
    n->graph_sink = n->kv.sink;
  }
  hipStream_t s = ctx->stream;
  if (!n->graphs[kind]) {
    const uint32_t source = kind == kGraphDecodeSelect ? kTokenSelected : kTokenHistory;
    const bool select = kind != kGraphPrompt;
    ND_HIP(ctx, hipStreamBeginCapture(s, hipStreamCaptureModeThreadLocal));
    const hipError_t e = enqueue_step(n, source, 0, select, select, nullptr, 0, s);
    hipGraph_t g = nullptr;
    const hipError_t e2 = hipStreamEndCapture(s, &g);
    if (e != hipSuccess || e2 != hipSuccess) {
      if (g) hipGraphDestroy(g);
      return nd_hip_fail(ctx, e != hipSuccess ? e : e2, "Needle step capture");
    }
    const hipError_t e3 = hipGraphInstantiate(&n->graphs[kind], g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e3 != hipSuccess) {
      n->graphs[kind] = nullptr;
      return nd_hip_fail(ctx, e3, "Needle step graph");
    }
  }
  ND_HIP(ctx, hipGraphLaunch(n->graphs[kind], s));
  return ND_OK;
}

nd_status check_step(nd_ctx* ctx, const nd_needle* n, uint32_t token) {
  if (!n->arena || n->max_length == 0)
    return nd_fail(ctx, ND_ERR_INVALID, "Call runtime.reset() before decoding");
  if (n->position >= n->max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %u reached runtime limit %u", n->position,
                   n->max_length);
  if (token >= n->d.vocab)
    return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside the vocabulary", token);
  return ND_OK;
}

}  // namespace

extern "C" {

nd_status nd_needle_create(nd_ctx* ctx, const nd_needle_desc* d, nd_needle** out) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!d || !out) return nd_fail(ctx, ND_ERR_INVALID, "nd_needle_create: NULL argument");
  *out = nullptr;
  if (d->head_dim != kHd || d->lanes == 0 || d->lanes > 4 || d->dim < 128 || d->dim > 512 ||
      (d->dim & (d->dim - 1)) || d->hadamard > 1024 || d->hadamard < d->dim ||
      (d->hadamard & (d->hadamard - 1)) || d->heads == 0 || d->kv_heads == 0 ||
      d->heads % d->kv_heads || d->heads * kHd > 8192 || d->layers == 0 || d->vocab == 0 ||
      d->max_length == 0 || d->n_sites > 4 || d->n_orders > 4 ||
      (d->n_sites && d->n_orders == 0) || d->engram_tables > 16 ||
      (d->n_orders && d->engram_tables % d->n_orders) ||
      (d->n_sites && (d->engram_taps == 0 || d->engram_slots == 0 || d->engram_sub == 0)))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "Needle geometry outside this kernel set: head_dim 64, lanes <= 4, dim a "
                   "power of two in [128, 512], power-of-two hadamard in [dim, 1024], heads a "
                   "multiple of kv_heads, at most 4 engram sites and orders, tables a multiple "
                   "of orders");
  const uint32_t rep = d->heads / d->kv_heads;
  if (rep != 1 && rep != 2 && rep != 4 && rep != 8)
    return nd_fail(ctx, ND_ERR_INVALID, "query heads per KV head must be 1, 2, 4 or 8");
  for (uint32_t i = 0; i < d->n_orders; ++i)
    if (d->orders[i] == 0) return nd_fail(ctx, ND_ERR_INVALID, "engram orders must be positive");
  for (uint32_t i = 0; i < d->n_sites; ++i)
    if (d->sites[i] >= d->layers)
      return nd_fail(ctx, ND_ERR_INVALID, "engram site past the last layer");
  const uint32_t D = d->dim, L = d->layers, ln = d->lanes, qw = d->heads * kHd,
                 kw = d->kv_heads * kHd, cat = d->engram_tables * d->engram_sub;
  if (d->n_sites && (cat < 128 || cat > 8192 || (cat & (cat - 1))))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "engram tables x sub must be a power of two in [128, 8192]");
  auto check = [&](const nd_mat* m, uint32_t n, uint32_t k, const char* what) -> nd_status {
    if (!m || m->n != n || m->k != k || m->g != k)
      return nd_fail(ctx, ND_ERR_INVALID, "%s must be a per-row-scaled %ux%u int8 matrix", what,
                     n, k);
    return ND_OK;
  };
  nd_status st;
  if ((st = check(d->embedding, d->vocab, D, "embedding")) ||
      (st = check(d->phi_pre, L * ln, ln * D, "phi_pre")) ||
      (st = check(d->phi_post, L * ln, ln * D, "phi_post")) ||
      (st = check(d->phi_res, L * ln * ln, ln * D, "phi_res")))
    return st;
  if (!d->wq || !d->wk || !d->wv || !d->wgate || !d->wo)
    return nd_fail(ctx, ND_ERR_INVALID, "layer matrix arrays must not be NULL");
  for (uint32_t l = 0; l < L; ++l)
    if ((st = check(d->wq[l], qw, D, "wq")) || (st = check(d->wk[l], kw, D, "wk")) ||
        (st = check(d->wv[l], kw, D, "wv")) || (st = check(d->wgate[l], qw, D, "wgate")) ||
        (st = check(d->wo[l], D, qw, "wo")))
      return st;
  if (d->n_sites && (!d->eg_tables || !d->eg_key || !d->eg_value || !d->eg_taps))
    return nd_fail(ctx, ND_ERR_INVALID, "engram arrays must not be NULL");
  for (uint32_t s = 0; s < d->n_sites; ++s)
    if ((st = check(d->eg_tables[s], d->engram_tables * d->engram_slots, d->engram_sub,
                    "engram tables")) ||
        (st = check(d->eg_key[s], D, cat, "engram key")) ||
        (st = check(d->eg_value[s], D, cat, "engram value")))
      return st;
  const float* dense[] = {d->norm_input, d->query_norm, d->key_norm, d->post_attn_norm,
                          d->pre_hadamard_norm, d->d1, d->d2, d->d3, d->attention_gate,
                          d->a_pre, d->a_post, d->a_res, d->b_pre, d->b_post, d->b_res,
                          d->final_norm};
  for (const float* p : dense)
    if (!p) return nd_fail(ctx, ND_ERR_INVALID, "dense Needle parameters must not be NULL");

  nd_needle* n = new nd_needle();
  n->d = *d;
  n->embedding = d->embedding;
  n->phi_pre = d->phi_pre;
  n->phi_post = d->phi_post;
  n->phi_res = d->phi_res;
  hipError_t e = hipSuccess;
  auto concat = [&](nd_mat& m, const nd_mat* const* parts, size_t count) {
    m.n = 0;
    for (size_t i = 0; i < count; ++i) m.n += parts[i]->n;
    m.k = parts[0]->k;
    m.g = m.k;
    if (e == hipSuccess) e = hipMalloc(&m.w, (size_t)m.n * m.k);
    if (e == hipSuccess) e = hipMalloc(&m.scales, (size_t)m.n * 4);
    size_t row = 0;
    for (size_t i = 0; i < count; ++i) {
      const nd_mat* p = parts[i];
      if (e == hipSuccess)
        e = hipMemcpyAsync(m.w + row * m.k, p->w, (size_t)p->n * m.k, hipMemcpyDeviceToDevice,
                           ctx->stream);
      if (e == hipSuccess)
        e = hipMemcpyAsync(m.scales + row, p->scales, (size_t)p->n * 4,
                           hipMemcpyDeviceToDevice, ctx->stream);
      row += p->n;
    }
  };
  n->wqkvg.resize(L);
  for (uint32_t l = 0; l < L; ++l) {
    const nd_mat* parts[4] = {d->wq[l], d->wk[l], d->wv[l], d->wgate[l]};
    concat(n->wqkvg[l], parts, 4);
    n->wo.push_back(d->wo[l]);
  }
  n->ekv.resize(d->n_sites);
  for (uint32_t s = 0; s < d->n_sites; ++s) {
    const nd_mat* parts[2] = {d->eg_key[s], d->eg_value[s]};
    concat(n->ekv[s], parts, 2);
    n->eg_tables.push_back(d->eg_tables[s]);
  }
  std::vector<float> h;
  auto put = [&](const float* src, size_t count) {
    const size_t off = h.size();
    if (src) h.insert(h.end(), src, src + count);
    else h.resize(h.size() + count, 0.f);
    h.resize(al(h.size() * 4) / 4, 0.f);
    return off;
  };
  n->o_norm_input = put(d->norm_input, (size_t)L * D);
  n->o_qn = put(d->query_norm, (size_t)L * kHd);
  n->o_kn = put(d->key_norm, (size_t)L * kHd);
  n->o_post = put(d->post_attn_norm, (size_t)L * D);
  n->o_preh = put(d->pre_hadamard_norm, (size_t)L * D);
  n->o_d1 = put(d->d1, (size_t)L * D);
  n->o_d2 = put(d->d2, (size_t)L * d->hadamard);
  n->o_d3 = put(d->d3, (size_t)L * D);
  n->o_bpre = put(d->b_pre, (size_t)L * ln);
  n->o_bpost = put(d->b_post, (size_t)L * ln);
  n->o_bres = put(d->b_res, (size_t)L * ln * ln);
  n->o_taps = put(d->n_sites ? d->eg_taps : nullptr,
                  (size_t)(d->n_sites ? d->n_sites * d->engram_taps : 1) * D);
  n->o_final = put(d->final_norm, D);
  n->attention_gate.assign(d->attention_gate, d->attention_gate + L);
  n->a_pre.assign(d->a_pre, d->a_pre + L);
  n->a_post.assign(d->a_post, d->a_post + L);
  n->a_res.assign(d->a_res, d->a_res + L);
  // applyRope (math.ts:94-115): angle = position * theta^(-2j/64).
  std::vector<double> freq(kHd / 2);
  for (uint32_t j = 0; j < kHd / 2; ++j)
    freq[j] = std::pow((double)d->rope_theta, -(2.0 * j) / kHd);
  if (e == hipSuccess) e = hipMalloc(&n->params, h.size() * 4);
  if (e == hipSuccess) e = hipMalloc(&n->inv_freq, freq.size() * 8);
  if (e == hipSuccess)
    e = hipMemcpyAsync(n->params, h.data(), h.size() * 4, hipMemcpyHostToDevice, ctx->stream);
  if (e == hipSuccess)
    e = hipMemcpyAsync(n->inv_freq, freq.data(), freq.size() * 8, hipMemcpyHostToDevice,
                       ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  for (uint32_t i = 0; i < d->n_orders; ++i) n->max_order = std::max(n->max_order, d->orders[i]);
  n->depth = d->n_sites ? (d->engram_taps - 1) * n->max_order + 1 : 1;
  if (e != hipSuccess) {
    nd_needle_free(ctx, n);
    return nd_hip_fail(ctx, e, "Needle upload");
  }
  *out = n;
  return ND_OK;
}

nd_status nd_needle_free(nd_ctx* ctx, nd_needle* n) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return ND_OK;
  hipStreamSynchronize(ctx->stream);
  drop_graphs(n);
  if (n->arena) hipFree(n->arena);
  for (auto* v : {&n->wqkvg, &n->ekv})
    for (auto& m : *v) {
      if (m.w) hipFree(m.w);
      if (m.scales) hipFree(m.scales);
    }
  if (n->params) hipFree(n->params);
  if (n->inv_freq) hipFree(n->inv_freq);
  delete n;
  return ND_OK;
}

nd_status nd_needle_reset(nd_ctx* ctx, nd_needle* n, uint32_t max_length, uint32_t sink) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "model is NULL");
  const nd_needle_desc& d = n->d;
  if (max_length == 0 || max_length > d.max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Runtime length %u is outside model limit %u",
                   max_length, d.max_length);
  const uint32_t D = d.dim, ln = d.lanes, qw = d.heads * kHd, kw = d.kv_heads * kHd;
  if (!n->arena) {
    // Sized for the model's max_length so that later resets never allocate.
    const uint32_t cap = d.max_length;
    const size_t rows = (size_t)d.layers * d.kv_heads * cap;
    const size_t pf = nd_attention_batch_partial_floats(1, d.kv_heads, d.heads / d.kv_heads, cap);
    const uint32_t S = d.n_sites ? d.n_sites : 1;
    const uint32_t cat = d.n_sites ? d.engram_tables * d.engram_sub : 1;
    // State first (cleared by every reset), then scratch.
    const size_t sizes[] = {al(64), al((size_t)cap * 4), al((size_t)cap * 8),
                            al((size_t)S * n->depth * D * 4), al(64), al(64),
                            al((size_t)d.vocab * 4), al(rows * kHd), al(rows * kHd), al(rows * 4),
                            al(rows * 4), al((size_t)ln * D * 4), al(D * 4), al(D * 4), al(D * 4),
                            al((size_t)(2 * qw + 2 * kw) * 4), al(qw * 4), al(qw * 4), al(D * 4),
                            al(ln * 4), al(ln * ln * 4), al(D * 4), al((size_t)d.vocab * 4),
                            al((size_t)S * cat * 4), al((size_t)S * 2 * D * 4),
                            al((size_t)S * D * 4), al(pf * 4)};
    size_t total = 0;
    for (size_t v : sizes) total += v;
    ND_HIP(ctx, hipMalloc(&n->arena, total));
    char* p = n->arena;
    size_t i = 0;
    auto take = [&](auto** dst) {
      *dst = reinterpret_cast<std::remove_reference_t<decltype(**dst)>*>(p);
      p += sizes[i++];
    };
    take(&n->st);
    take(&n->history);
    take(&n->lp_history);
    take(&n->ring);
    n->state_bytes = (size_t)(p - n->arena);
    take(&n->sel_id);
    take(&n->sel_lp);
    take(&n->allowed);
    int8_t *kc, *vc;
    take(&kc);
    take(&vc);
    n->kv.k = kc;
    n->kv.v = vc;
    take(&n->kv.ks);
    take(&n->kv.vs);
    take(&n->x);
    take(&n->upd);
    take(&n->blk);
    take(&n->ain);
    take(&n->qkvg);
    take(&n->q);
    take(&n->att);
    take(&n->proj);
    take(&n->phi_post_v);
    take(&n->phi_res_v);
    take(&n->fin);
    take(&n->logits);
    take(&n->cat);
    take(&n->ekv_out);
    take(&n->evals);
    take(&n->partials);
  }
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  ND_HIP(ctx, hipMemsetAsync(n->arena, 0, n->state_bytes, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  n->max_length = max_length;
  n->sink = std::min(sink, max_length);
  n->position = 0;
  nd_kv& kv = n->kv;
  kv.layers = d.layers;
  kv.kv_heads = d.kv_heads;
  kv.head_dim = kHd;
  kv.max_length = max_length;
  kv.sink = n->sink;
  kv.window = d.kv_window;
  kv.alloc = d.kv_window > 0 ? std::min(max_length, n->sink + d.kv_window) : max_length;
  kv.mode = ND_KV_INT8;
  return ND_OK;
}

nd_kv* nd_needle_kv(nd_needle* n) { return n && n->arena && n->max_length ? &n->kv : nullptr; }

uint32_t nd_needle_position(const nd_needle* n) { return n ? n->position : 0; }

nd_status nd_needle_step(nd_ctx* ctx, nd_needle* n, uint32_t token, float* logits) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "model is NULL");
  nd_status st = check_step(ctx, n, token);
  if (st != ND_OK) return st;
  ND_HIP(ctx, enqueue_step(n, kTokenArg, token, logits != nullptr, false, nullptr, 0, ctx->stream));
  ++n->position;
  if (logits)
    ND_HIP(ctx, hipMemcpyAsync(logits, n->logits, (size_t)n->d.vocab * 4, hipMemcpyDeviceToHost,
                               ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_needle_prefill(nd_ctx* ctx, nd_needle* n, const uint32_t* tokens, uint32_t count,
                            float* logits) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || (!tokens && count)) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  if (count == 0) return nd_fail(ctx, ND_ERR_INVALID, "Cannot prefill an empty token sequence");
  if (!n->arena || n->max_length == 0)
    return nd_fail(ctx, ND_ERR_INVALID, "Call runtime.reset() before decoding");
  if (n->max_length - n->position < count)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Prompt has %u tokens but runtime holds %u", count,
                   n->max_length - n->position);
  for (uint32_t i = 0; i < count; ++i)
    if (tokens[i] >= n->d.vocab)
      return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside the vocabulary", tokens[i]);
  ND_HIP(ctx, hipMemcpyAsync(n->history + n->position, tokens, (size_t)count * 4,
                             hipMemcpyHostToDevice, ctx->stream));
  for (uint32_t i = 0; i < count; ++i) {
    const bool last = i + 1 == count;
    ND_HIP(ctx, enqueue_step(n, kTokenHistory, 0, last && logits, false, nullptr, 0, ctx->stream));
    ++n->position;
  }
  if (logits)
    ND_HIP(ctx, hipMemcpyAsync(logits, n->logits, (size_t)n->d.vocab * 4, hipMemcpyDeviceToHost,
                               ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_needle_step_select(nd_ctx* ctx, nd_needle* n, uint32_t token, const uint32_t* allowed,
                                uint32_t count, uint32_t* id, double* logprob) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || !id || !logprob) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  nd_status st = check_step(ctx, n, token);
  if (st != ND_OK) return st;
  if (allowed) {
    // selectToken (runtime.ts:880-899): a non-empty id list inside the logits.
    if (count == 0) return nd_fail(ctx, ND_ERR_INVALID, "Allowed token set is empty");
    if (count > n->d.vocab)
      return nd_fail(ctx, ND_ERR_INVALID, "Allowed token set is larger than the vocabulary");
    for (uint32_t i = 0; i < count; ++i)
      if (allowed[i] >= n->d.vocab)
        return nd_fail(ctx, ND_ERR_INVALID, "Allowed token %u is outside logits", allowed[i]);
    ND_HIP(ctx, hipMemcpyAsync(n->allowed, allowed, (size_t)count * 4, hipMemcpyHostToDevice,
                               ctx->stream));
  }
  ND_HIP(ctx, enqueue_step(n, kTokenArg, token, true, true, allowed ? n->allowed : nullptr,
                           allowed ? count : 0, ctx->stream));
  ++n->position;
  ND_HIP(ctx, hipMemcpyAsync(id, n->sel_id, 4, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(logprob, n->sel_lp, 8, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_needle_generate(nd_ctx* ctx, nd_needle* n, const uint32_t* prompt, uint32_t count,
                             uint32_t max_new, uint32_t sink, uint32_t eos, uint32_t* ids,
                             double* logprobs, uint32_t* generated) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || !prompt || !generated || (max_new && (!ids || !logprobs)))
    return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  *generated = 0;
  if (count == 0) return nd_fail(ctx, ND_ERR_INVALID, "Cannot prefill an empty token sequence");
  const uint32_t model_max = n->d.max_length;
  const uint32_t max_len = (uint32_t)std::min<uint64_t>(model_max, (uint64_t)count + max_new);
  if (count >= max_len && max_new > 0)
    return nd_fail(ctx, ND_ERR_OVERFLOW,
                   "Prompt has %u tokens and leaves no generation room in a %u-token context",
                   count, max_len);
  for (uint32_t i = 0; i < count; ++i)
    if (prompt[i] >= n->d.vocab)
      return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside the vocabulary", prompt[i]);
  nd_status st = nd_needle_reset(ctx, n, std::max(count, max_len), sink);
  if (st != ND_OK) return st;
  ND_HIP(ctx, hipMemcpyAsync(n->history, prompt, (size_t)count * 4, hipMemcpyHostToDevice,
                             ctx->stream));
  const uint32_t n_gen = max_new ? std::min(max_new, max_len - count) : 0;
  for (uint32_t i = 0; i + 1 < count; ++i) {
    if ((st = launch_graph(ctx, n, kGraphPrompt)) != ND_OK) return st;
    ++n->position;
  }
  if ((st = launch_graph(ctx, n, n_gen ? kGraphPromptSelect : kGraphPrompt)) != ND_OK) return st;
  ++n->position;
  // Token k (k < n_gen - 1) is stepped by decode step k, which records it and
  // its log-probability at history[count + k]; the last one stays in the
  // selection buffers.
  for (uint32_t k = 0; k + 1 < n_gen; ++k) {
    if ((st = launch_graph(ctx, n, kGraphDecodeSelect)) != ND_OK) return st;
    ++n->position;
  }
  if (n_gen == 0) {
    ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return ND_OK;
  }
  std::vector<uint32_t> tok(n_gen);
  std::vector<double> lp(n_gen);
  if (n_gen > 1) {
    ND_HIP(ctx, hipMemcpyAsync(tok.data(), n->history + count, (size_t)(n_gen - 1) * 4,
                               hipMemcpyDeviceToHost, ctx->stream));
    ND_HIP(ctx, hipMemcpyAsync(lp.data(), n->lp_history + count, (size_t)(n_gen - 1) * 8,
                               hipMemcpyDeviceToHost, ctx->stream));
  }
  ND_HIP(ctx, hipMemcpyAsync(&tok[n_gen - 1], n->sel_id, 4, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(&lp[n_gen - 1], n->sel_lp, 8, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  uint32_t out = 0;
  for (; out < n_gen && tok[out] != eos; ++out) {
    ids[out] = tok[out];
    logprobs[out] = lp[out];
  }
  *generated = out;
  return ND_OK;
}

}  // extern "C"
