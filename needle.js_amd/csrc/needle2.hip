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
// Per layer the token runs four stages: the previous layer's Wo matvec,
// `mix` (one workgroup: the post-attention half of the previous layer --
// sandwich norm, Hadamard MLP, h-post, Sinkhorn routing, lane update -- then
// this layer's pre-attention half -- lane RMS, the lanes*(2+lanes) phi rows,
// h-pre mix, engram injection, input norm), the Q/K/V/gate matvec with q/k
// norm + RoPE and the KV append in its epilogue, and attention with the
// sigmoid(gate) epilogue.  Where the placement is confirmed they share one
// launch per layer (workgroups on one XCD handing over through its L2),
// else they run as separate launches.  The one-workgroup arithmetic keeps
// the reference's float64-with-f32-stores form except the Sinkhorn
// iterations (fp32).
#include <algorithm>
#include <array>
#include <cmath>
#include <cstring>
#include <type_traits>
#include <vector>

#include "nd_cq.hpp"
#include "nd_attention.hpp"
#include "nd_internal.hpp"
#include "nd_wave.hpp"

namespace {

constexpr uint32_t kHd = 64;
constexpr int kWg = 1024;
constexpr int kMixWg = 512;  // mix kernel: dim <= 512 values per thread role
constexpr uint32_t kPrefillRows = 512;  // positions per batched prefill pass
typedef int i32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
using nd::half8;
using nd::float4v;
using nd::u32x2;

// or_sigmoid / sigmoid (math.ts): 1 / (1 + e^-v) for v >= 0, e^v / (1 + e^v)
// below, with one exp either way (e = e^-|v|), so lanes of either sign share
// one instruction stream.
__device__ __forceinline__ double sigmoid_d(double v) {
  const double e = exp(-fabs(v));
  return (v >= 0 ? 1.0 : e) / (1.0 + e);
}

// Sum over a workgroup of NT threads; every thread gets the total.
template <int NT = kWg>
__device__ __forceinline__ double block_sum_d(double v, double* red) {
  v = nd::wave_sum(v);
  __syncthreads();
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  double r = 0.0;
#pragma unroll
  for (int i = 0; i < NT / 64; ++i) r += red[i];
  return r;
}

// JavaScript Math.max over |v| of a wave: NaN wins.
__device__ __forceinline__ float wave_absmax_js(float v) { return nd::wave_max_js(fabsf(v)); }

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
  const double* inv_freq;  // [32]
  double* rope;            // out: sin then cos of position * inv_freq[j]
  float* cell0;            // confidence pool cell 0 (the scaled embedding), or null
  uint32_t cell_ld;        // its row stride in the batched form
  // Cactus-Quant model: the gathers run in n2_cq_rows_kernel, which reads
  // [tables] indices, [tables] valid flags and the token from here.
  uint32_t* cq_lookup;
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
  if (t < 32) {
    // RoPE angles of this step (math.ts:94-115), shared by every layer.
    double sn, cs;
    sincos((double)pos * a.inv_freq[t], &sn, &cs);
    a.rope[t] = sn;
    a.rope[32 + t] = cs;
  }
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
    if (a.cq_lookup) {
      a.cq_lookup[t] = s_idx[t];
      a.cq_lookup[a.tables + t] = s_valid[t];
    }
  }
  if (a.cq_lookup) {
    if (t == 0) a.cq_lookup[2 * a.tables] = tok;
    return;
  }
  __syncthreads();
  for (uint32_t k = t; k < a.d; k += kWg) {
    const float row = (float)a.emb[(size_t)tok * a.d + k] * a.emb_s[tok];
    const float v = (float)((double)row * a.scale);
    for (uint32_t l = 0; l < a.lanes; ++l) a.x[(size_t)l * a.d + k] = v;
    if (a.cell0) a.cell0[k] = v;
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

// A session step's position (ResidentTokenRequest.position,
// backends/backend.ts:52-56): st[1] = position and st[0] = position + 1, as
// a whole step's intake leaves them, and the RoPE angles of every layer at it
// (math.ts:94-115).
__global__ void n2_position_kernel(uint32_t* __restrict__ st, uint32_t position,
                                   const double* __restrict__ inv_freq, double* __restrict__ rope) {
  const uint32_t t = threadIdx.x;
  if (t == 0) {
    st[0] = position + 1;
    st[1] = position;
  }
  if (t < 32) {
    double sn, cs;
    sincos((double)position * inv_freq[t], &sn, &cs);
    rope[t] = sn;
    rope[32 + t] = cs;
  }
}

// The concatenated engram rows of every site (runtime.ts:828-836) for a
// lookup the host computed (ResidentEngramRequest, backends/backend.ts:
// 46-50: runtime.ts:788-818's indices and valid flags per table, indices
// checked against the slot count on entry); zero for an invalid table.
__global__ __launch_bounds__(kWg) void n2_gather_kernel(BeginArgs a,
                                                         const uint32_t* __restrict__ lookup) {
  const uint32_t per_site = a.tables * a.sub;
  for (uint32_t i = threadIdx.x; i < a.n_sites * per_site; i += kWg) {
    const uint32_t s = i / per_site, j = i % per_site, tb = j / a.sub, c = j % a.sub;
    float v = 0.f;
    if (lookup[a.tables + tb]) {
      const size_t row = (size_t)tb * a.slots + lookup[tb];
      v = (float)a.tw[s][row * a.sub + c] * a.ts[s][row];
    }
    a.cat[i] = v;
  }
}

// The begin kernel's gathers for a Cactus-Quant model (runtime.ts:305-313,
// 828-836), rows dequantized as dequantizeCqRow (cq.ts:243-295):
// workgroup 0 puts the embedding row of *token, times sqrt(d) in float64,
// into every lane (and cell 0 of the confidence pool); workgroup 1 + s *
// tables + t writes table t's row lookup[t] of engram site s into cat, or
// zeros when lookup[tables + t] is 0.
constexpr uint32_t kCqRowMax = 1024;  // padded row width of the embedding and tables
// One matrix whose rows are dequantized: packed rows, binary16 norms,
// padded width, bytes per row, group, code width, 1/sqrt(g) and the
// codebook by code (ternary: 0, +c, 0, -c).
struct CqSource {
  const uint8_t* p;
  const uint16_t* n;
  uint32_t kpad, row_bytes, g, bits;
  double inverse_root;
  float cb[16];
};
struct CqRowsArgs {
  CqSource emb;     // the embedding
  CqSource tab[4];  // each engram site's tables (their own formats)
  const uint32_t* token;   // null: no embedding row (the session's lanes come from the host)
  const uint32_t* lookup;  // [tables] indices, then [tables] valid flags
  uint32_t d, lanes;
  double scale;
  float* x;
  float* cell0;
  uint32_t n_sites, tables, slots, sub;
  float* cat;
  // Batched prefill: position blockIdx.y reads its token and lookups
  // lookup_ld further on and writes its lanes, pool cell and engram rows
  // x_ld, cell_ld and cat_ld further on (all 0 for one step).
  uint32_t lookup_ld, x_ld, cell_ld, cat_ld;
};

__global__ __launch_bounds__(256) void n2_cq_rows_kernel(CqRowsArgs a) {
  __shared__ float v[kCqRowMax];
  const uint32_t b = blockIdx.x, t = threadIdx.x, m = blockIdx.y;
  if (m) {
    a.lookup += (size_t)m * a.lookup_ld;
    if (a.token) a.token += (size_t)m * a.lookup_ld;
    a.x += (size_t)m * a.x_ld;
    if (a.cell0) a.cell0 += (size_t)m * a.cell_ld;
    a.cat += (size_t)m * a.cat_ld;
  }
  // This workgroup's source, copied with constant indices (a runtime index
  // into the argument block would copy it to scratch); its codebook in LDS.
  const uint32_t i = b - 1, s = b ? i / a.tables : 0u, tb = b ? i % a.tables : 0u;
  CqSource src;
  if (b == 0) {
    src = a.emb;
  } else {
    switch (s) {
      case 0: src = a.tab[0]; break;
      case 1: src = a.tab[1]; break;
      case 2: src = a.tab[2]; break;
      default: src = a.tab[3]; break;
    }
  }
  __shared__ float s_cb[16];
  if (t == 0) {
#pragma unroll
    for (int c = 0; c < 16; ++c) s_cb[c] = src.cb[c];
  }
  __syncthreads();
  if (b == 0) {
    if (!a.token) return;
    const uint32_t tok = *a.token;
    nd::cq_dequant_row(src.p + (size_t)tok * src.row_bytes,
                       src.n + (size_t)tok * (src.kpad / src.g), s_cb, src.kpad, src.g, src.bits,
                       src.inverse_root, v);
    for (uint32_t k = t; k < a.d; k += blockDim.x) {
      const float val = (float)((double)v[k] * a.scale);
      for (uint32_t l = 0; l < a.lanes; ++l) a.x[(size_t)l * a.d + k] = val;
      if (a.cell0) a.cell0[k] = val;
    }
    return;
  }
  float* out = a.cat + ((size_t)s * a.tables + tb) * a.sub;
  if (!a.lookup[a.tables + tb]) {
    for (uint32_t c = t; c < a.sub; c += blockDim.x) out[c] = 0.f;
    return;
  }
  const size_t row = (size_t)tb * a.slots + a.lookup[tb];
  nd::cq_dequant_row(src.p + row * src.row_bytes, src.n + row * (src.kpad / src.g), s_cb,
                     src.kpad, src.g, src.bits, src.inverse_root, v);
  for (uint32_t c = t; c < a.sub; c += blockDim.x) out[c] = v[c];
}

// sinkhorn (math.ts:62-92) of an L x L matrix (L <= 4) on the lanes of a
// quad: lane q holds row q.  Each log-space row (column) step r -= logsumexp
// is a division of exp(r) by its row (column) sum, so the twenty iterations
// run on p = exp(r - max) in fp32 with reciprocals; a spread above 80
// between the largest and smallest logit (where exp would underflow in fp32)
// takes the float64 log-space form.  A NaN logit makes every entry NaN, as
// the reference's Math.max does.  Reads the logits from and writes exp(r)
// to io[q * L + c].
__device__ void sinkhorn_quad(float* io, uint32_t L, uint32_t lane) {
  const uint32_t q = lane & 3;
  const bool row_ok = q < L;
  float v[4];
  float mx = -INFINITY, mn = INFINITY;
  bool nan = false;
#pragma unroll
  for (int c = 0; c < 4; ++c) {
    const bool ok = row_ok && (uint32_t)c < L;
    v[c] = ok ? io[q * L + c] : 0.f;
    if (ok) {
      nan = nan || v[c] != v[c];
      mx = fmaxf(mx, v[c]);
      mn = fminf(mn, v[c]);
    }
  }
  mx = fmaxf(mx, nd::dpp<nd::kQuadXor1>(mx));
  mx = fmaxf(mx, nd::dpp<nd::kQuadXor2>(mx));
  mn = fminf(mn, nd::dpp<nd::kQuadXor1>(mn));
  mn = fminf(mn, nd::dpp<nd::kQuadXor2>(mn));
  int any_nan = nan ? 1 : 0;
  any_nan |= __builtin_amdgcn_mov_dpp(any_nan, nd::kQuadXor1, 0xF, 0xF, false);
  any_nan |= __builtin_amdgcn_mov_dpp(any_nan, nd::kQuadXor2, 0xF, 0xF, false);
  float p[4];
  if (any_nan) {
#pragma unroll
    for (int c = 0; c < 4; ++c) p[c] = __builtin_nanf("");
  } else if (mx - mn <= 80.f) {
#pragma unroll
    for (int c = 0; c < 4; ++c) p[c] = (row_ok && (uint32_t)c < L) ? __expf(v[c] - mx) : 0.f;
    for (int it = 0; it < 20; ++it) {
      const float rs = (p[0] + p[1]) + (p[2] + p[3]);
      const float ri = row_ok ? __builtin_amdgcn_rcpf(rs) : 0.f;
#pragma unroll
      for (int c = 0; c < 4; ++c) p[c] *= ri;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float cs = nd::quad_sum(p[c]);
        p[c] *= (uint32_t)c < L ? __builtin_amdgcn_rcpf(cs) : 0.f;
      }
    }
  } else {
    double r[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) r[c] = v[c];
    for (int it = 0; it < 20; ++it) {
      double m = -INFINITY, sum = 0.0;
      for (uint32_t c = 0; c < L; ++c) m = fmax(m, r[c]);
      for (uint32_t c = 0; c < L; ++c) sum += exp(r[c] - m);
      const double ls = log(sum) + m;
#pragma unroll
      for (int c = 0; c < 4; ++c) r[c] -= row_ok ? ls : 0.0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        double cm = row_ok ? r[c] : -INFINITY;
        cm = fmax(cm, nd::dpp<nd::kQuadXor1>(cm));
        cm = fmax(cm, nd::dpp<nd::kQuadXor2>(cm));
        const double cs = nd::quad_sum(row_ok ? exp(r[c] - cm) : 0.0);
        r[c] -= log(cs) + cm;
      }
    }
#pragma unroll
    for (int c = 0; c < 4; ++c) p[c] = (float)exp(r[c]);
  }
  if (lane < 4 && row_ok)
    for (uint32_t c = 0; c < L; ++c) io[q * L + c] = p[c];
}

struct RouteArgs {
  const float* phi_post;  // [lanes], from pre(l)
  const float* phi_res;   // [lanes * lanes]
  float a_post, a_res;
  const float* b_post;
  const float* b_res;
  uint32_t lanes, own;
  float* route;  // out: [lanes * lanes] routing, then [lanes] h-post
};

// h-post and the Sinkhorn routing of layer l (runtime.ts:511-528) on one
// wave; they depend only on pre(l)'s phi values, so they run beside the
// Q/K/V projection instead of inside the next mix kernel.
__device__ void route_wave(const RouteArgs& r, uint32_t lane, float* lds) {
  const uint32_t L = r.lanes;
  if (lane < L * L)
    lds[lane] = (float)((double)r.a_res * (double)r.phi_res[lane] + (double)r.b_res[lane]);
  float hp = 0.f;
  if (lane < L) {
    const double off = lane == r.own ? 0.0 : -4.0;
    hp = (float)(2.0 * sigmoid_d((double)r.a_post * (double)r.phi_post[lane] +
                                 (double)r.b_post[lane] + off));
  }
  __syncthreads();
  if (lane < 64) sinkhorn_quad(lds, L, lane);
  __syncthreads();
  if (lane < L * L) r.route[lane] = lds[lane];
  if (lane < L) r.route[L * L + lane] = hp;
}

// The value of lane (lane ^ M): DPP below 16; for 16 and 32 gfx950's row /
// half swaps (VALU): given the value twice, the 16-swap returns {rows 0, 0,
// 2, 2; rows 1, 1, 3, 3} and the 32-swap {lanes 0..31 twice; lanes 32..63
// twice}.
template <int M>
__device__ __forceinline__ float xor_partner(float v, uint32_t lane) {
  if constexpr (M >= 16) {
    const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(__float_as_uint(v),
                                                              __float_as_uint(v), false, false)
                           : __builtin_amdgcn_permlane32_swap(__float_as_uint(v),
                                                              __float_as_uint(v), false, false);
    return __uint_as_float((lane & M) ? r[0] : r[1]);
  } else {
    return nd::lane_xor<M>(v);
  }
}

// One head of the projection epilogue, one wave, lane = dimension: role 0
// (query) and 1 (key) take the per-head rmsNorm with their scale and the
// half-split RoPE by (sin, cos) of the lane's angle (runtime.ts:471-500,
// math.ts:94-115); role 0
// writes q_dst, roles 1 and 2 (value) quantize into cache row
// head_row + slot with #storeKV's arithmetic (runtime.ts:679-717).
__device__ __forceinline__ void head_epilogue(float val, uint32_t lane, int role, double sn,
                                              double cs, float nscale, float* q_dst,
                                              void* Kc, void* Vc, float* Ks, float* Vs,
                                              size_t head_row, uint32_t slot, uint32_t alloc,
                                              uint32_t f32) {
  float out = val;
  if (role != 2) {
    const double xd = val;
    const double ss = nd::wave_sum(xd * xd);
    const double inv = 1.0 / sqrt(ss / kHd + 1e-6);
    const float nf = (float)((1.0 + (double)nscale) * xd * inv);
    const double normed = nf, other = xor_partner<32>(nf, lane);  // float values, exact in double
    out = lane < 32 ? (float)(normed * cs - other * sn) : (float)(normed * cs + other * sn);
    if (role == 0) {
      q_dst[lane] = out;
      return;
    }
  }
  if (slot >= alloc) return;  // the host keeps positions below the runtime limit
  const size_t crow = head_row + slot;
  if (f32) {  // kvCache "float32": the value itself, scale 1 (runtime.ts:686-692)
    reinterpret_cast<float*>(role == 2 ? Vc : Kc)[crow * kHd + lane] = out;
    if (lane == 0) (role == 2 ? Vs : Ks)[crow] = 1.f;
    return;
  }
  const float am = wave_absmax_js(out);
  const double mx = (am != am) ? (double)am : fmax(1e-12, (double)am);
  const double sc = mx / 127.0;
  const double code = rint((double)out / sc);
  reinterpret_cast<int8_t*>(role == 2 ? Vc : Kc)[crow * kHd + lane] =
      code != code ? (int8_t)0 : (int8_t)(int)code;
  if (lane == 0) (role == 2 ? Vs : Ks)[crow] = (float)sc;
}

// Projection rows of the Q/K/V/gate launch: 64 rows of d <= 512 int8
// columns per workgroup, kQkvTpr threads a row; thread q of row r holds
// bytes [16 kQkvTpr k + 16 q, +16) of the row (k < 32 / kQkvTpr; clamped in
// the row, blocks past d add nothing), so a wave's load covers whole
// 16 kQkvTpr-byte row pieces.  qkv_row_dot takes the fp32 fmas against x in
// LDS in that order and sums the row's threads.
constexpr uint32_t kQkvTpr = 8;
constexpr uint32_t kQkvLoads = 32 / kQkvTpr;
constexpr int kQkvWg = 64 * kQkvTpr;

__device__ __forceinline__ void qkv_row_loads(const int8_t* W, size_t row, uint32_t q,
                                              uint32_t d, i32x4 (&w)[kQkvLoads]) {
  const int8_t* p = W + row * d;
#pragma unroll
  for (uint32_t k = 0; k < kQkvLoads; ++k)
    w[k] = __builtin_nontemporal_load(
        reinterpret_cast<const i32x4*>(p + min(16u * kQkvTpr * k + 16u * q, d - 16)));
}

__device__ __forceinline__ float qkv_row_dot(const i32x4 (&w)[kQkvLoads], const float* xs,
                                             uint32_t q, uint32_t d) {
  float acc = 0.f;
#pragma unroll
  for (uint32_t k = 0; k < kQkvLoads; ++k) {
    const uint32_t off = 16u * kQkvTpr * k + 16u * q;
    if (off < d) {
      int8_t cb[16];
      __builtin_memcpy(cb, &w[k], 16);
#pragma unroll
      for (int j = 0; j < 16; ++j) acc = fmaf((float)cb[j], xs[off + j], acc);
    }
  }
  acc = nd::quad_sum(acc);
  if constexpr (kQkvTpr >= 8) acc += nd::lane_xor<4>(acc);
  if constexpr (kQkvTpr >= 16) acc += nd::lane_xor<8>(acc);
  return acc;
}

// A Cactus-Quant matrix's rows as the projection launch reads them (rows of
// kpad codes, binary16 norms per group, the width's codebook by code).
struct CqRows {
  const uint8_t* packed;
  const uint16_t* norms;
  float cb[16];
  uint32_t g, g_log2, row_bytes, groups;
  float out_scale;  // 1 / sqrt(g)
};

// Rows r and r + 32 of the workgroup's 64 (r = t / 16) of a Cactus-Quant
// product with d <= 512 inputs (cqMatvec, backends/cq.ts:106-231): thread t
// takes 32-code unit u = t % 16 of both rows.  xs holds x with one pad float
// after every 32 (element e at e + e / 32, zeros past d), so the 16 units'
// reads fall in distinct banks.  The unit's inputs are rotated in registers
// -- the butterflies of fastWalshHadamard with strides below min(g, 32), then
// strides 32 .. g / 2 across the lanes holding the group's other units --
// each result one fp32 add or subtract of the reference's two operands; the
// codes index the codebook in LDS; fp32 dots per group times the group's
// norm, summed over the row's 16 lanes, times 1/sqrt(g).  Returns the two
// row values in every lane of the row.
// The operands thread t loads for rows r and r + 32 (r = t / 16) of a
// 64-row block, unit u = t % 16: the packed words (4, 3 or 2 by the code
// width; ternary crumbs as 2) and the norms of the unit's groups.
struct CqRowRegs {
  uint32_t w[2][4];
  uint32_t nb[2][4];
};

__device__ __forceinline__ void cq_rows_load(const CqRows& q, uint32_t bits, size_t row0,
                                             uint32_t units, uint32_t t, CqRowRegs& R) {
  const uint32_t u = t & 15, r = t >> 4;
  const uint32_t uc = u < units ? u : 0;
  const uint32_t words = bits == 4 ? 4u : (bits == 3 ? 3u : 2u);
  const uint32_t ng = q.g < 32 ? 32u >> q.g_log2 : 1u;  // groups in a unit
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    const size_t row = row0 + r + 32u * i;
    const uint32_t* src =
        reinterpret_cast<const uint32_t*>(q.packed + row * q.row_bytes) + uc * words;
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) {
      R.w[i][k] = 0u;
      if (k < words) R.w[i][k] = src[k];
    }
    const uint16_t* nrow = q.norms + row * q.groups + ((uc * 32) >> q.g_log2);
#pragma unroll
    for (uint32_t k = 0; k < 4; ++k) R.nb[i][k] = nrow[k < ng ? k : 0];
  }
}

// The butterflies of fastWalshHadamard (backends/cq.ts:8-27) with strides
// below min(g, 64) over values held one per lane, element e in lane e % 64
// (groups of g are aligned, so a group below 64 values lies in one wave):
// stride s pairs lane i with lane i ^ s, the lower lane takes a + b and the
// upper a - b of the reference's two operands (a the lower element), one
// fp32 add or subtract each.  Every lane of the wave must take part.
__device__ __forceinline__ float cq_rotate_lanes(float v, uint32_t g, uint32_t lane) {
  auto stage = [&](auto m) {
    constexpr int M = decltype(m)::value;
    const float other = xor_partner<M>(v, lane);
    v = (lane & M) ? other - v : v + other;
  };
  if (g > 1) stage(std::integral_constant<int, 1>{});
  if (g > 2) stage(std::integral_constant<int, 2>{});
  if (g > 4) stage(std::integral_constant<int, 4>{});
  if (g > 8) stage(std::integral_constant<int, 8>{});
  if (g > 16) stage(std::integral_constant<int, 16>{});
  if (g > 32) stage(std::integral_constant<int, 32>{});
  return v;
}

// x (kpad <= 512 values: v is thread t's element, zero past the input)
// into xs for cq_rows_dot, by a 512-thread workgroup, one element per
// thread: element e at e + e / 32 (one pad float after every 32, so that the
// 16 units' reads fall in distinct banks), the strides below min(g, 64) of
// the per-group rotation applied (cq_rotate_lanes).  The caller's barrier
// publishes xs.
__device__ __forceinline__ void cq_stage_rotated(float v, uint32_t kpad, uint32_t g, float* xs,
                                                 uint32_t t) {
  static_assert(kQkvWg == 512 && kMixWg == 512, "one input element per thread");
  v = cq_rotate_lanes(v, g, t & 63);
  if (t < kpad) xs[t + (t >> 5)] = v;
}

// Rows r and r + 32 of the workgroup's 64 (r = t / 16) of a Cactus-Quant
// product with d <= 512 inputs (cqMatvec, backends/cq.ts:106-231) from the
// operands cq_rows_load gave thread t (unit u = t % 16 of both rows) and
// the input cq_stage_rotated left in xs.  The group's remaining strides
// (64 .. g / 2, g > 64) run across the lanes holding the group's other
// units, each result one fp32 add or subtract of the reference's two
// operands; the codes index the codebook in LDS; fp32 dots per group times
// the group's norm, summed over the row's 16 lanes, times 1/sqrt(g).
// Returns the two row values in every lane of the row.  G32: g >= 32 (one
// group end per unit); otherwise g is 8 or 16.
template <uint32_t BITS, bool G32>
__device__ __forceinline__ float2 cq_rows_dot(const CqRows& q, const CqRowRegs& R,
                                              uint32_t units, const float* xs, const float* cb,
                                              uint32_t t) {
  const uint32_t u = t & 15;
  const bool active = u < units;
  const uint32_t uc = active ? u : 0;
  float v[32];
#pragma unroll
  for (int c = 0; c < 32; ++c) v[c] = xs[uc * 33 + c];
  if constexpr (G32) {
    auto cross = [&](auto m) {
      constexpr int M = decltype(m)::value;
      const bool right = (t & M) != 0;
#pragma unroll
      for (int c = 0; c < 32; ++c) {
        const float other = nd::lane_xor<M>(v[c]);
        v[c] = right ? other - v[c] : v[c] + other;
      }
    };
    if (q.g > 64) cross(std::integral_constant<int, 2>{});
    if (q.g > 128) cross(std::integral_constant<int, 4>{});
    if (q.g > 256) cross(std::integral_constant<int, 8>{});
  }
  float out[2];
#pragma unroll
  for (int i = 0; i < 2; ++i) {
    float total = 0.f, dot = 0.f;
#pragma unroll
    for (uint32_t c = 0; c < 32; ++c) {
      float w;
      if constexpr (BITS == 4) {
        // The entry's byte offset code * 4: nibble k of a word sits at bits
        // 2..5 of byte k / 2 of the word shifted left by 2 (k even) or right
        // by 2 (k odd).
        const uint32_t word = R.w[i][c >> 3];
        const uint32_t sh = (c & 1) ? word >> 2 : word << 2;
        w = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(cb) +
                                            ((sh >> (8 * ((c & 7) >> 1))) & 0x3cu));
      } else if constexpr (BITS == 3) {
        const uint32_t bit = 3 * c, k = bit >> 5, sh = bit & 31;
        const uint32_t hi = sh > 29 ? R.w[i][k + 1 < 3 ? k + 1 : 2] << (32 - sh) : 0u;
        w = cb[((R.w[i][k] >> sh) | hi) & 7u];
      } else {
        w = cb[(R.w[i][c >> 4] >> (2 * (c & 15))) & 3u];
      }
      dot = fmaf(w, v[c], dot);
      if constexpr (G32) {
        if (c == 31) total = fmaf(nd::cq_half(R.nb[i][0]), dot, total);
      } else if ((c & 7) == 7) {  // a group of 8 or 16 may end here: by selection
        const bool ends = q.g == 8 || (c & 15) == 15;
        const uint32_t h = q.g == 8 ? R.nb[i][c >> 3] : R.nb[i][c >> 4];
        const float with = fmaf(nd::cq_half(h), dot, total);
        total = ends ? with : total;
        dot = ends ? 0.f : dot;
      }
    }
    total = active ? total : 0.f;
    total += nd::lane_xor<1>(total);
    total += nd::lane_xor<2>(total);
    total += nd::lane_xor<4>(total);
    total += nd::lane_xor<8>(total);
    out[i] = total * q.out_scale;
  }
  return float2{out[0], out[1]};
}

// cq_rows_dot by code width (2-bit codes and ternary crumbs as 2) and group
// class.
template <uint32_t BITS>
__device__ __forceinline__ float2 cq_rows_dot_g(const CqRows& q, const CqRowRegs& R,
                                                uint32_t units, const float* xs, const float* cb,
                                                uint32_t t) {
  if (q.g >= 32) return cq_rows_dot<BITS, true>(q, R, units, xs, cb, t);
  return cq_rows_dot<BITS, false>(q, R, units, xs, cb, t);
}

// The fused Q/K/V/gate projection of one layer (runtime.ts:465-470) with the
// per-head norm + RoPE of q and k (runtime.ts:471-500) and #storeKV
// (runtime.ts:679-717) in the epilogue.  Workgroup b computes rows [64 b,
// 64 b + 64) of wqkvg = [q (H*64) | k (Hkv*64) | v (Hkv*64) | gate (H*64)]:
// for int8 rows (BITS 0) eight threads per row (qkv_row_dot), fp32
// accumulation of int8 x fp32 like the matvec, times the row scale; for
// Cactus-Quant rows (BITS 2, 3, 4; ternary crumbs as 2) cq_rows_pair.  q
// heads go to q_out, k and v heads are quantized into the cache at the ring
// slot of the step's position, gate heads go to gate_out as raw projections.
// One more workgroup computes the layer's routing (route_wave).
// Bound on the waits of the fused mix launch (a safety net: a workgroup
// waits only on workgroups dispatched before it, which wait on nothing
// later), in s_sleep(1) rounds.  A wait that runs out sets a bit of the
// runtime's status word and skips every store that depends on it; the word
// stays set until the next reset clears it with the counters and flags, and
// the whole-step calls return an error while it is set (what later launches
// compute from the skipped stores is never reported as a result).
constexpr uint32_t kWoSpin = 1u << 16;
constexpr uint32_t kStatusWoWait = 1u;   // the mix's wait for the Wo rows
constexpr uint32_t kStatusQkvWait = 2u;  // a projection workgroup's wait for the mix
constexpr uint32_t kStatusAttWait = 4u;  // an attention workgroup's wait for the projection
// The mix's signal to the projection workgroups: 1 once its outputs are in
// the L2, or kFlagAbort | 1 when it gave up (they then skip their stores).
// The low 16 bits count the workgroups that have seen it.
constexpr uint32_t kFlagAbort = 1u << 16;
constexpr uint32_t kFlagCount = kFlagAbort - 1;
// Words between the attention workgroups' per-KV-head counters (128 bytes:
// no two share an L2 line, so their atomics do not queue on one address).
constexpr uint32_t kAttStride = 32;

// The projection launch's arguments.
struct QkvParams {
  const int8_t* W;
  const float* S;
  const float* x;
  uint32_t d, heads, kv_heads;
  const uint32_t* st;
  const float* q_norm;
  const float* k_norm;
  const double* rope;
  float* q_out;
  float* gate_out;
  void* Kc;
  void* Vc;
  float* Ks;
  float* Vs;
  uint32_t layer, alloc, sink, window, f32;
  RouteArgs route;
  // Cactus-Quant models: the q, k, v and gate parts, each in its own format
  // (code width cq_bits[i]; a mixed-width archive may differ per part).
  CqRows cq[4];
  uint32_t cq_bits[4];
};

// cq_rows_dot by code width (2-bit codes and ternary crumbs as 2) and group
// class.
__device__ __forceinline__ float2 cq_rows_dot_any(uint32_t bits, const CqRows& q,
                                                  const CqRowRegs& R, uint32_t units,
                                                  const float* xs, const float* cb, uint32_t t) {
  if (bits == 4) return cq_rows_dot_g<4>(q, R, units, xs, cb, t);
  if (bits == 3) return cq_rows_dot_g<3>(q, R, units, xs, cb, t);
  return cq_rows_dot_g<2>(q, R, units, xs, cb, t);
}

// Workgroup b of the projection launch (b == 2 (heads + kv_heads): the
// routing).  CQ: the rows are Cactus-Quant, each 64-row block in its part's
// format (q, k, v, gate).  WAIT (inside the fused mix launch): issue the
// weight rows and
// the epilogue operands, then wait until *flag != 0 -- the mix's signal
// that x and the phi values are in the XCD's L2 -- before reading them (at
// most `spin` rounds).  Each of the `waiters` workgroups then counts itself
// on the flag and the last one clears it, so every launch starts from zero.
// A workgroup whose wait runs out sets kStatusQkvWait in *status; one that
// finds kFlagAbort (the mix gave up) counts itself in; both return without
// storing anything.
//
// att_count (inside the fused launch that also runs layer l's attention):
// every head workgroup counts itself in on its KV head's counter
// (att_count + kAttStride kv head: the query and gate heads of that KV head,
// its key and its value) once its stores (q, the cache row, the gate) have
// completed, or with kFlagAbort when it stores nothing.
// STAMP (measurement form of the fused launch): thread 0 writes the 100 MHz
// clock to marks[0..3] (LDS) when the wait ended, the input was staged, the
// rows were computed and the stores had completed.
template <bool CQ, bool WAIT, bool STAMP = false>
__device__ __forceinline__ void qkv_body(const QkvParams& p, uint32_t b, uint32_t* flag,
                                         uint32_t waiters, uint32_t* status = nullptr,
                                         uint32_t spin = 0, uint32_t* att_count = nullptr,
                                         uint64_t* marks = nullptr) {
  __shared__ float xs[512 + 16];
  __shared__ float rows[64];
  __shared__ float s_cb[16];
  __shared__ uint32_t s_go;
  const uint32_t t = threadIdx.x;
  auto mark = [&](int i) {
    if constexpr (STAMP) {
      if (t == 0) marks[i] = wall_clock64();
    }
  };
  // s_go: 0 the wait ran out, 1 go, 2 the flag carried the abort bit.  A
  // workgroup that saw the flag counts itself on it when it is done
  // (release): the flag is next read by this layer's launch of the next
  // step, so the count stays off this launch's path.
  auto wait = [&]() -> bool {
    if constexpr (WAIT) {
      if (t == 0) {
        uint32_t it = 0, f;
        uint32_t go = 1;
        while ((f = __hip_atomic_load(flag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) == 0) {
          if (++it >= spin) {
            go = 0;
            break;
          }
          __builtin_amdgcn_s_sleep(1);
        }
        if (!go)
          __hip_atomic_fetch_or(status, kStatusQkvWait, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
        else if (f & kFlagAbort)
          go = 2;
        s_go = go;
      }
      __syncthreads();
      mark(0);
      return s_go == 1;
    }
    return true;
  };
  auto release = [&]() {
    if constexpr (WAIT) {
      if (t == 0 && s_go != 0 &&
          (__hip_atomic_fetch_add(flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) &
           kFlagCount) == waiters)
        __hip_atomic_store(flag, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  auto count_in = [&](bool stored) {
    if (att_count) {
      const uint32_t H = p.heads, K = p.kv_heads, rep = H / K;
      const uint32_t kvh = b < H ? b / rep
                         : b < H + K ? b - H
                         : b < H + 2 * K ? b - H - K : (b - H - 2 * K) / rep;
      uint32_t* c = att_count + kAttStride * kvh;
      if (!stored)
        __hip_atomic_fetch_or(c, kFlagAbort, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      __hip_atomic_fetch_add(c, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    }
  };
  if (b == 2 * (p.heads + p.kv_heads)) {
    if (wait()) route_wave(p.route, t, rows);
    release();
    return;
  }
  const uint32_t lane = t & 63;
  const uint32_t d = p.d;
  // The epilogue's operands (written before this launch) are issued here,
  // ahead of the wait, so that they are in registers when the rows are.
  const uint32_t pos = p.st[1];
  const float nscale = b < p.heads ? p.q_norm[lane] : p.k_norm[lane];
  const double rs = p.rope[lane & 31], rc = p.rope[32 + (lane & 31)];
  if constexpr (!CQ) {
    // Loads first: this thread's weight bytes (unconditional, clamped, so
    // they issue back to back), the row scale, then x.
    const size_t row = (size_t)b * kHd + t / kQkvTpr;
    i32x4 wv[kQkvLoads];
    qkv_row_loads(p.W, row, t % kQkvTpr, d, wv);
    const float srow = p.S[row];
    if (!wait()) {
      if (t == 0) count_in(false);
      release();
      return;
    }
    for (uint32_t i = t; i < d; i += kQkvWg) xs[i] = p.x[i];
    __syncthreads();
    mark(1);
    const float acc = qkv_row_dot(wv, xs, t % kQkvTpr, d);
    if (t % kQkvTpr == 0) rows[t / kQkvTpr] = acc * srow;
  } else {
    // The block's part and its first block; the part's descriptor field by
    // field by selection (a runtime index into the argument block, or a copy
    // of a whole descriptor, would go through scratch).
    const uint32_t H = p.heads, K = p.kv_heads;
    const uint32_t part = b < H ? 0u : (b < H + K ? 1u : (b < H + 2 * K ? 2u : 3u));
    const uint32_t first = part == 0 ? 0u : (part == 1 ? H : (part == 2 ? H + K : H + 2 * K));
    auto pick = [part](auto a, auto b, auto c, auto d) {
      return part == 0 ? a : (part == 1 ? b : (part == 2 ? c : d));
    };
    CqRows q;
    q.packed = pick(p.cq[0].packed, p.cq[1].packed, p.cq[2].packed, p.cq[3].packed);
    q.norms = pick(p.cq[0].norms, p.cq[1].norms, p.cq[2].norms, p.cq[3].norms);
    q.g = pick(p.cq[0].g, p.cq[1].g, p.cq[2].g, p.cq[3].g);
    q.g_log2 = pick(p.cq[0].g_log2, p.cq[1].g_log2, p.cq[2].g_log2, p.cq[3].g_log2);
    q.row_bytes = pick(p.cq[0].row_bytes, p.cq[1].row_bytes, p.cq[2].row_bytes,
                       p.cq[3].row_bytes);
    q.groups = pick(p.cq[0].groups, p.cq[1].groups, p.cq[2].groups, p.cq[3].groups);
    q.out_scale = pick(p.cq[0].out_scale, p.cq[1].out_scale, p.cq[2].out_scale,
                       p.cq[3].out_scale);
    const uint32_t bits = pick(p.cq_bits[0], p.cq_bits[1], p.cq_bits[2], p.cq_bits[3]);
    const uint32_t kpad = q.groups << q.g_log2;  // the part's padded row (<= 512)
    // The rows' packed words and norms first (before the wait, as the int8
    // rows), then the part's codebook into LDS.
    CqRowRegs R;
    cq_rows_load(q, bits, (size_t)(b - first) * kHd, kpad / 32, t, R);
    if (t == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i)
        s_cb[i] = pick(p.cq[0].cb[i], p.cq[1].cb[i], p.cq[2].cb[i], p.cq[3].cb[i]);
    }
    if (!wait()) {
      if (t == 0) count_in(false);
      release();
      return;
    }
    cq_stage_rotated(t < d ? p.x[t] : 0.f, kpad, q.g, xs, t);
    __syncthreads();
    mark(1);
    const float2 v = cq_rows_dot_any(bits, q, R, kpad / 32, xs, s_cb, t);
    if ((t & 15) == 0) {
      rows[t >> 4] = v.x;
      rows[(t >> 4) + 32] = v.y;
    }
  }
  __syncthreads();
  mark(2);
  if (t >= 64) return;
  const float val = rows[lane];
  const uint32_t nq = p.heads, nk = p.kv_heads;
  if (b >= nq + 2 * nk) {  // gate head
    p.gate_out[(size_t)(b - nq - 2 * nk) * kHd + lane] = val;
    if (att_count) {
      __builtin_amdgcn_s_waitcnt(0);  // the wave's stores have completed
      mark(3);
      if (lane == 0) count_in(true);
    }
    release();
    return;
  }
  const int role = b < nq ? 0 : (b < nq + nk ? 1 : 2);
  const uint32_t h = role == 0 ? b : (role == 1 ? b - nq : b - nq - nk);
  head_epilogue(val, lane, role, rs, rc, nscale, p.q_out + (size_t)h * kHd, p.Kc, p.Vc, p.Ks, p.Vs,
                ((size_t)p.layer * nk + h) * p.alloc, kv_slot(pos, p.sink, p.window), p.alloc,
                p.f32);
  if (att_count) {
    __builtin_amdgcn_s_waitcnt(0);  // the wave's stores have completed
    mark(3);
    if (lane == 0) count_in(true);
  }
  release();
}

template <bool CQ>
__global__ __launch_bounds__(kQkvWg) void n2_qkv_kernel(QkvParams p) {
  qkv_body<CQ, false>(p, blockIdx.x, nullptr, 0);
}

// A Cactus-Quant Wo (y = W x, x of k <= 512 values, n a multiple of 64
// rows) by 64-row workgroups of cq_rows_pair: the standalone launch
// (n2_wo_cq_kernel) and the fused mix launch run the same body, so both
// give the same bits.
struct WoCq {
  const float* x;
  float* y;
  uint32_t n, k;
  CqRows cq;
};

// Rows [64 k, +64) of w.  count (the fused launch): after the rows are in
// the XCD's L2, add one to *count.  STAMP (measurement form): thread 0
// writes the clock to marks[0..2] (LDS) when the input was staged, the rows
// were computed and the rows were stored.
template <uint32_t BITS, bool STAMP = false>
__device__ __forceinline__ void wo_cq_rows(const WoCq& w, uint32_t k, uint32_t* count,
                                           uint64_t* marks = nullptr) {
  __shared__ float xs[512 + 16];
  __shared__ float s_cb[16];
  const uint32_t t = threadIdx.x;
  auto mark = [&](int i) {
    if constexpr (STAMP) {
      if (t == 0) marks[i] = wall_clock64();
    }
  };
  const uint32_t kpad = w.cq.groups << w.cq.g_log2;  // the padded row (<= 512)
  // The input first (it is in the L2), then the rows' packed words and
  // norms: the rotation's wait for the input then leaves the weight loads in
  // flight.
  const float xv = t < w.k ? w.x[t] : 0.f;
  __builtin_amdgcn_sched_barrier(0);
  CqRowRegs R;
  cq_rows_load(w.cq, BITS, (size_t)k * 64, kpad / 32, t, R);
  __builtin_amdgcn_sched_barrier(0);
  if (t == 0) {  // constant indices into the argument block
#pragma unroll
    for (int i = 0; i < 16; ++i) s_cb[i] = w.cq.cb[i];
  }
  cq_stage_rotated(xv, kpad, w.cq.g, xs, t);
  __syncthreads();
  mark(0);
  const float2 v = cq_rows_dot_g<BITS>(w.cq, R, kpad / 32, xs, s_cb, t);
  if constexpr (STAMP) {
    asm volatile("" ::"v"(v.x), "v"(v.y));
    mark(1);
  }
  if ((t & 15) == 0) {
    const uint32_t r = k * 64 + (t >> 4);
    __hip_atomic_store(w.y + r, v.x, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    __hip_atomic_store(w.y + r + 32, v.y, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  if (count) {
    __builtin_amdgcn_s_waitcnt(0);  // the rows are in the L2
    mark(2);
    __syncthreads();
    if (t == 0) __hip_atomic_fetch_add(count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
}

template <uint32_t BITS>
__global__ __launch_bounds__(kMixWg) void n2_wo_cq_kernel(WoCq w) {
  wo_cq_rows<BITS>(w, blockIdx.x, nullptr);
}

// Layer l's attention inside the fused launch (n2_mix_kernel<*, true>):
// the gated single-chunk attention of nd_launch_attention_gated over an
// int8 cache whose ring fits one 512-position chunk, two query heads per KV
// head -- the same attention_body instance, so the same bits.
struct AttArgs {
  const void* Kc;
  const void* Vc;
  const float* Ks;
  const float* Vs;
  const float* q;
  float* out;
  const float* gate;
  const uint32_t* position;
  uint32_t layer, kv_heads, alloc, sink, window;
};

struct MixArgs {
  float* x;  // [lanes][d]: read, and rewritten when has_post
  uint32_t d, hdim, lanes;
  // log2 of d, lanes * d and lanes when a power of two, else -1 (means over
  // them scale exactly: div_pow2)
  int32_t d_log2, n_log2, l_log2;
  // post-attention half of layer l - 1 (runtime.ts:509-542, #attentionDelta
  // runtime.ts:585-611); routing and h-post come from the route workgroup of
  // the Q/K/V launch of layer l - 1
  uint32_t has_post;
  const float* proj;  // Wo output [d]
  const float* post_norm;
  const float* pre_h_norm;
  const float* d1;
  const float* d2;
  const float* d3;
  double attention_scale;  // sigmoid(attentionGate[l - 1]), float64
  double inv_root_h;       // 1 / sqrt(hdim), float64
  const float* route;  // [lanes * lanes] Sinkhorn routing, then [lanes] h-post
  // pre-attention half of layer l (runtime.ts:385-441)
  uint32_t has_pre, own_pre;
  const int8_t* phi_w[3];  // phi_pre, phi_post, phi_res rows of layer l
  const float* phi_s[3];
  // The same rows as Cactus-Quant matrices (n2_mix_kernel<true>): for layer
  // l's phi_pre, phi_post and phi_res each, its packed rows and binary16
  // norms, codebook by code, width, group, bytes per row, norms per row and
  // 1/sqrt(g) (a mixed-width archive gives each matrix its own).
  const uint8_t* cq_p[3];
  const uint16_t* cq_n[3];
  float cq_cb[3][16];
  uint32_t cq_bits[3], cq_g[3], cq_row_bytes[3], cq_groups[3];
  double cq_inv_root[3];
  float a_pre;
  const float* b_pre;
  uint32_t has_site;  // an engram site injects at layer l
  const float* ekey;  // engram key / mixed value of that site
  const float* evalue;
  double sqrt_d;      // sqrt(d), float64
  float split_scale;  // 2^s with sqrt(lanes * d) * 2^s <= 2^15 (the phi operand split)
  float split_unscale;
  const float* norm_input;
  // lane mean + final norm after the last layer (runtime.ts:570-576)
  uint32_t has_final;
  const float* final_norm;
  float* fin;
  // carried from pre(l) to post(l)
  float* upd;       // [d]
  float* blk;       // [d]
  float* ain;       // [d]
  float* phi_post;  // [lanes]
  float* phi_res;   // [lanes * lanes]
  // Batched prefill: workgroup m works on row m of every per-row buffer
  // (row strides: x lanes * d; proj, blk, upd, ain d; route 20; phi_post
  // lanes; phi_res lanes * lanes; ekey ek_ld; evalue ev_ld) and, with
  // route_out set, also computes layer l's routing into route_out row m.
  uint32_t ek_ld, ev_ld;
  float* route_out;
  float r_a_post, r_a_res;
  const float* r_b_post;
  const float* r_b_res;
  // Confidence pool: after post(l - 1), the lane mean (runtime.ts:543-550)
  // into cell [d] (row stride cell_ld), when not null.  Only workgroup
  // final_row computes the final norm.
  float* cell;
  uint32_t cell_ld, final_row;
  // Wo of layer l - 1 in the same launch (n2_mix_kernel<false, true>): proj =
  // Wo att (codes [wo_n][wo_k], one scale per row), rows in wo_groups
  // workgroups that count in on wo_count.
  const int8_t* wo_w;
  const float* wo_s;
  const float* wo_x;
  uint32_t wo_n, wo_k, wo_groups, wo_tpr_log2;
  uint32_t* wo_count;
  // The mix waits for wo_target arrivals (wo_groups, or more when a test
  // forces the wait to run out), each wait for at most spin rounds; a wait
  // that runs out sets a bit of *status.
  uint32_t wo_target, spin;
  uint32_t* status;
  // ... and layer l's projection: qkv_groups workgroups (qkv_body) after
  // the mix, waiting on qkv_flag, which the mix sets to 1 once the
  // attention input and the phi values are stored (cleared by the last
  // of them).
  QkvParams qkv;
  uint32_t qkv_groups;
  uint32_t* qkv_flag;
  // A Cactus-Quant Wo in the same launch (n2_mix_kernel<true, true>):
  // wo_groups workgroups of wo_cq_rows, codes of wo_bits bits.
  WoCq wo_cq;
  uint32_t wo_bits;
  // ... and layer l's attention: att_groups workgroups (one per KV head)
  // after the projection, each waiting until the att_target projection
  // workgroups of its KV head have counted in on its counter (att_count +
  // kAttStride kv head); it counts itself in after its work and clears the
  // count.
  AttArgs att;
  uint32_t att_groups, att_target;
  uint32_t* att_count;
  // Measurement (n2_mix_kernel<..., STAMP>): 16 clock stamps per active
  // workgroup k (L / 8) at stamps[16 k]: entry, the mix's Wo wait done, the
  // mix's signal to the projection, exit, then the mix's phases (after the
  // post norms, each FWHT, the lane update, the pre norm, the phi products,
  // the engram gate, the input norm) -- 0 where a role has no such point.
  uint64_t* stamps;
};

// Rows [rpw k, +rpw) of proj = Wo att in the fused Wo + mix launch, rpw =
// kMixWg / tpr, tpr = wo_k / 16 threads a row.  Each thread's arithmetic is
// matvec_i8_kernel's for one batch row with one 16-byte segment per thread
// and one scale per row: the segment's 16 inputs and their sum, the codes
// biased to unsigned bytes, d = -128 sum + the fmas, times the row scale;
// the row's threads then add in the same butterfly (lanes 32, 16, ..., 1
// apart, as far as tpr reaches).  So proj holds the bits the separate Wo
// launch gives.  The rows are stored at workgroup scope and the workgroup
// counts itself in: every one of these workgroups and the mix workgroup run
// on one XCD (the launch uses workgroups L % 8 == 0 only), so both stay in
// its L2.
// STAMP (measurement form): thread 0 writes the clock to marks[0..2] (LDS)
// when o had arrived, the weights had arrived, and the rows were stored.
template <bool STAMP = false>
__device__ __forceinline__ void wo_rows(const MixArgs& a, uint32_t k, uint64_t* marks = nullptr) {
  const uint32_t t = threadIdx.x, tpr_log2 = a.wo_tpr_log2, tpr = 1u << tpr_log2;
  auto mark = [&](int i) {
    if constexpr (STAMP) {
      if (t == 0) marks[i] = wall_clock64();
    }
  };
  const uint32_t rpw = kMixWg >> tpr_log2, sub = t >> tpr_log2, lk = t & (tpr - 1);
  const uint32_t row = k * rpw + sub;
  const bool ok = row < a.wo_n;
  const uint32_t r = ok ? row : 0;
  float xr[16];
  const float4* xp = reinterpret_cast<const float4*>(a.wo_x) + lk * 4;
#pragma unroll
  for (int q = 0; q < 4; ++q) {
    const float4 f = xp[q];
    xr[4 * q] = f.x;
    xr[4 * q + 1] = f.y;
    xr[4 * q + 2] = f.z;
    xr[4 * q + 3] = f.w;
  }
  const u32x4 wv = __builtin_nontemporal_load(
      reinterpret_cast<const u32x4*>(a.wo_w + (size_t)r * a.wo_k) + lk);
  const float sv = a.wo_s[r];
  float xs = 0.f;
#pragma unroll
  for (int q = 0; q < 4; ++q) xs += (xr[4 * q] + xr[4 * q + 1]) + (xr[4 * q + 2] + xr[4 * q + 3]);
  if constexpr (STAMP) {
    asm volatile("" ::"v"(xs));
    mark(0);
  }
  const uint32_t words[4] = {wv.x ^ 0x80808080u, wv.y ^ 0x80808080u, wv.z ^ 0x80808080u,
                             wv.w ^ 0x80808080u};
  float d = -128.f * xs;
#pragma unroll
  for (int q = 0; q < 4; ++q)
#pragma unroll
    for (int e = 0; e < 4; ++e) d = fmaf((float)((words[q] >> (8 * e)) & 0xffu), xr[4 * q + e], d);
  if constexpr (STAMP) {
    asm volatile("" ::"v"(d));
    mark(1);
  }
  float sum = 0.f;
  sum += fmaf(sv, d, 0.f);
  if (tpr > 32) sum = nd::sum_xor<32>(sum);
  if (tpr > 16) sum = nd::sum_xor<16>(sum);
  if (tpr > 8) sum += nd::lane_xor<8>(sum);
  if (tpr > 4) sum += nd::lane_xor<4>(sum);
  if (tpr > 2) sum += nd::lane_xor<2>(sum);
  if (tpr > 1) sum += nd::lane_xor<1>(sum);
  if (lk == 0 && ok)
    __hip_atomic_store(const_cast<float*>(a.proj) + row, sum, __ATOMIC_RELAXED,
                       __HIP_MEMORY_SCOPE_WORKGROUP);
  __builtin_amdgcn_s_waitcnt(0);  // the rows are in the L2
  mark(2);
  __syncthreads();
  if (t == 0) __hip_atomic_fetch_add(a.wo_count, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
}


// sigmoid in float64 as the kernels evaluate it (host side: the constants
// a mix launch takes precomputed).
inline double host_sigmoid(double v) {
  if (v >= 0) return 1.0 / (1.0 + std::exp(-v));
  const double e = std::exp(v);
  return e / (1.0 + e);
}

// log2 of n when n is a power of two, else -1.
inline int32_t log2_exact(uint32_t n) {
  if (n == 0 || (n & (n - 1))) return -1;
  int32_t k = 0;
  while ((1u << k) < n) ++k;
  return k;
}

// The mix launch constants derived from the geometry and the layer's gate.
inline void mix_constants(MixArgs& m, uint32_t d, uint32_t hdim, uint32_t lanes, float gate) {
  m.d_log2 = log2_exact(d);
  m.n_log2 = log2_exact(lanes * d);
  m.l_log2 = log2_exact(lanes);
  m.attention_scale = host_sigmoid((double)gate);
  m.inv_root_h = 1.0 / std::sqrt((double)hdim);
  m.sqrt_d = std::sqrt((double)d);
  int s = 0;
  while (std::sqrt((double)lanes * d) * std::ldexp(1.0, s + 1) <= 32768.0) ++s;
  m.split_scale = std::ldexp(1.f, s);
  m.split_unscale = std::ldexp(1.f, -s);
}

// Sums over the kMixWg threads with one LDS barrier each: the partial sums
// alternate between two LDS rows, so a row is rewritten only after the next
// call's barrier, which every reader of the previous call has passed (the
// barrier waits for the wave's own LDS reads first).  mix_sum2 reduces two
// values in the same round.
// s / n in float64: for n = 2^k (log2n = k >= 0) the exact scaling ldexp(s,
// -k), which is the correctly rounded quotient itself; a division otherwise.
__device__ __forceinline__ double div_pow2(double s, int32_t log2n, uint32_t n) {
  return log2n >= 0 ? ldexp(s, -log2n) : s / (double)n;
}

__device__ __forceinline__ double mix_sum(double v, double (*red)[2 * (kMixWg / 64)], int& phase) {
  v = nd::wave_sum(v);
  if ((threadIdx.x & 63) == 0) red[phase][threadIdx.x >> 6] = v;
  nd::lds_barrier();
  double r = 0.0;
#pragma unroll
  for (int i = 0; i < kMixWg / 64; ++i) r += red[phase][i];
  phase ^= 1;
  return r;
}

__device__ __forceinline__ void mix_sum2(double& v, double& w,
                                         double (*red)[2 * (kMixWg / 64)], int& phase) {
  v = nd::wave_sum(v);
  w = nd::wave_sum(w);
  if ((threadIdx.x & 63) == 0) {
    red[phase][threadIdx.x >> 6] = v;
    red[phase][kMixWg / 64 + (threadIdx.x >> 6)] = w;
  }
  nd::lds_barrier();
  double r = 0.0, q = 0.0;
#pragma unroll
  for (int i = 0; i < kMixWg / 64; ++i) {
    r += red[phase][i];
    q += red[phase][kMixWg / 64 + i];
  }
  v = r;
  w = q;
  phase ^= 1;
}

// One FWHT butterfly (fwht, math.ts): the lower element takes mine + other,
// the upper other - mine, each evaluated in float64 and stored as f32.  The
// float64 sum or difference of two f32 values rounded to f32 is the f32 sum
// or difference itself (53 >= 2 * 24 + 2 bits: the double rounding is
// innocuous), so the butterflies run in f32 with the same results.
__device__ __forceinline__ float butterfly(float mine, float other, bool upper) {
  return upper ? other - mine : mine + other;
}

// Walsh-Hadamard transform of hv[0, H) (H <= kMixWg a power of two), one
// value per thread, strides ascending: DPP within rows, swizzle / bpermute
// across them, for strides 1..32.  The strides 64, 128, 256 mix values of
// different waves: after one exchange through the LDS buffer hv (a buffer no
// earlier step of the launch has used), thread t = g + 64 k reads the H / 64
// values g + 64 k' of its column and runs those stages on them in registers
// (the same butterflies, in the same order), keeping element k.  Every
// thread calls it; threads >= H hold zeros.  Returns thread t's transformed
// value; v is its input.
__device__ float fwht_block(float v, float* hv, uint32_t H, uint32_t t) {
  v = butterfly(v, nd::dpp<nd::kQuadXor1>(v), t & 1);
  if (H > 2) v = butterfly(v, nd::dpp<nd::kQuadXor2>(v), t & 2);
  if (H > 4) v = butterfly(v, nd::lane_xor<4>(v), t & 4);
  if (H > 8) v = butterfly(v, nd::lane_xor<8>(v), t & 8);
  if (H > 16) v = butterfly(v, xor_partner<16>(v, t), t & 16);
  if (H > 32) v = butterfly(v, xor_partner<32>(v, t), t & 32);
  if (H <= 64) return v;
  hv[t] = v;
  nd::lds_barrier();
  const uint32_t G = H / 64, g = t & 63, k = t >> 6;  // G <= kMixWg / 64 = 8
  float c[kMixWg / 64];
#pragma unroll
  for (uint32_t i = 0; i < kMixWg / 64; ++i) c[i] = i < G ? hv[g + 64 * i] : 0.f;
#pragma unroll
  for (uint32_t st = 1; st < kMixWg / 64; st <<= 1) {
    if (st < G) {
#pragma unroll
      for (uint32_t i = 0; i < kMixWg / 64; ++i)
        if (!(i & st)) {
          const float a = c[i], b = c[i + st];
          c[i] = a + b;
          c[i + st] = a - b;
        }
    }
  }
  float out = c[0];
#pragma unroll
  for (uint32_t i = 1; i < kMixWg / 64; ++i) out = k == i ? c[i] : out;
  return out;
}

// Cactus-Quant phi rows of the mix kernel, for one code width (2-bit codes and
// ternary crumbs: BITS = 2): wave w takes rows w, w + 8 and w + 16, lane u
// the rows' 32-code unit u, from the packed words w[j] and group norms n[j]
// it loaded at entry, against xu, the lane's 32 rotated inputs.  Each unit
// takes fp32 dots over its four 8-code blocks, each block times its group's
// norm (groups of 8, 16, or 32 and wider) in float64, summed over the wave.
// Element m (0, 1, 2) of a kernel-argument triple, by selection (a runtime
// index into the argument block would copy it to scratch).
template <typename T>
__device__ __forceinline__ T sel3(uint32_t m, T a, T b, T c) {
  return m == 0 ? a : (m == 1 ? b : c);
}

// One Cactus-Quant phi row on a wave: lane u < units holds the row's 32-code
// unit u (packed words w, the norms n of its groups) and the rotated inputs
// xu of that unit; each 8 codes are a dot in fp32 (code from the codebook
// cb in LDS times the input), each group's dots times its binary16 norm in
// float64.  Returns the lane's share of the row (the caller sums the wave).
template <uint32_t BITS>
__device__ __forceinline__ double cq_phi_row(const uint32_t (&w)[4], const uint32_t (&n)[4],
                                             const float (&xu)[32], const float* cb, uint32_t g,
                                             uint32_t units, uint32_t lane) {
  double total = 0.0;
  if (lane < units) {
    float dot8[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t c = 0; c < 32; ++c) {
      float e;
      if constexpr (BITS == 4) {
        // The entry's byte offset code * 4 (as in cq_rows_dot).
        const uint32_t sh = (c & 1) ? w[c >> 3] >> 2 : w[c >> 3] << 2;
        e = *reinterpret_cast<const float*>(reinterpret_cast<const char*>(cb) +
                                            ((sh >> (8 * ((c & 7) >> 1))) & 0x3cu));
      } else if constexpr (BITS == 3) {
        const uint32_t bit = 3 * c, k = bit >> 5, sh = bit & 31;
        const uint32_t hi = sh > 29 ? w[k + 1 < 4 ? k + 1 : 3] << (32 - sh) : 0u;
        e = cb[((w[k] >> sh) | hi) & 7u];
      } else {
        e = cb[(w[c >> 4] >> (2 * (c & 15))) & 3u];
      }
      dot8[c >> 3] = fmaf(e, xu[c], dot8[c >> 3]);
    }
#pragma unroll
    for (int b = 0; b < 4; ++b) {
      const uint32_t nb = g == 8 ? n[b] : (g == 16 ? n[b >> 1] : n[0]);
      total += (double)nd::cq_half(nb) * (double)dot8[b];
    }
  }
  return total;
}

// cq_phi_row by the row's code width (2-bit codes and ternary crumbs as 2).
__device__ __forceinline__ double cq_phi_row_any(uint32_t bits, const uint32_t (&w)[4],
                                                 const uint32_t (&n)[4], const float (&xu)[32],
                                                 const float* cb, uint32_t g, uint32_t units,
                                                 uint32_t lane) {
  if (bits == 4) return cq_phi_row<4>(w, n, xu, cb, g, units, lane);
  if (bits == 3) return cq_phi_row<3>(w, n, xu, cb, g, units, lane);
  return cq_phi_row<2>(w, n, xu, cb, g, units, lane);
}

// The wave's rows w, w + 8, w + 16 (below nrows) of phi matrices that share
// one format: code width BITS, group g, the rotation xu and codebook cb.
template <uint32_t BITS>
__device__ __forceinline__ void cq_phi_rows(const uint32_t (&w)[3][4], const uint32_t (&n)[3][4],
                                            const float (&xu)[32], const float* cb, uint32_t g,
                                            uint32_t units, uint32_t nrows, uint32_t wave,
                                            uint32_t lane, float* phi) {
#pragma unroll
  for (int j = 0; j < 3; ++j) {
    const uint32_t r = wave + 8u * j;
    if (r >= nrows) break;  // uniform over the wave
    const double total = nd::wave_sum(cq_phi_row<BITS>(w[j], n[j], xu, cb, g, units, lane));
    if (lane == 0) phi[r] = (float)total;
  }
}

// prepareCqActivation of one 32-value unit per lane (backends/cq.ts:30-46):
// the butterflies of fastWalshHadamard with strides below min(g, 32) inside
// the unit, strides 32 .. g / 2 across the lanes holding the group's other
// units (each result one fp32 add or subtract of the reference's two
// operands), then times 1/sqrt(g) in float64.
__device__ __forceinline__ void cq_rotate_unit(float (&xu)[32], uint32_t g, double inv_root,
                                               uint32_t lane) {
  const uint32_t gs = g < 32 ? g : 32u;
#pragma unroll
  for (uint32_t st = 1; st < 32; st <<= 1) {
    if (st < gs) {
#pragma unroll
      for (uint32_t c = 0; c < 32; ++c)
        if (!(c & st)) {
          const float x0 = xu[c], x1 = xu[c + st];
          xu[c] = x0 + x1;
          xu[c + st] = x0 - x1;
        }
    }
  }
  auto cross = [&](auto m) {
    constexpr int M = decltype(m)::value;
    const bool right = (lane & M) != 0;
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const float other = nd::lane_xor<M>(xu[c]);
      xu[c] = right ? other - xu[c] : xu[c] + other;
    }
  };
  const uint32_t lpg = g > 32 ? g >> 5 : 1u;  // lanes of a group
  if (lpg > 1) cross(std::integral_constant<int, 1>{});
  if (lpg > 2) cross(std::integral_constant<int, 2>{});
  if (lpg > 4) cross(std::integral_constant<int, 4>{});
  if (lpg > 8) cross(std::integral_constant<int, 8>{});
  if (lpg > 16) cross(std::integral_constant<int, 16>{});
  if (lpg > 32) cross(std::integral_constant<int, 32>{});
#pragma unroll
  for (int c = 0; c < 32; ++c) xu[c] = (float)((double)xu[c] * inv_root);
}

// The strides 64 .. g / 2 (g > 64) of prepareCqActivation over one 32-value
// unit per lane (stride 64 pairs the units two lanes apart), each result one
// fp32 add or subtract of the reference's two operands, then times
// 1/sqrt(g) in float64: the end of cq_rotate_unit for a unit whose strides
// below 64 are done.
__device__ __forceinline__ void cq_rotate_wide(float (&xu)[32], uint32_t g, double inv_root,
                                               uint32_t lane) {
  auto cross = [&](auto m) {
    constexpr int M = decltype(m)::value;
    const bool right = (lane & M) != 0;
#pragma unroll
    for (int c = 0; c < 32; ++c) {
      const float other = nd::lane_xor<M>(xu[c]);
      xu[c] = right ? other - xu[c] : xu[c] + other;
    }
  };
  if (g > 64) cross(std::integral_constant<int, 2>{});
  if (g > 128) cross(std::integral_constant<int, 4>{});
  if (g > 256) cross(std::integral_constant<int, 8>{});
  if (g > 512) cross(std::integral_constant<int, 16>{});
  if (g > 1024) cross(std::integral_constant<int, 32>{});
#pragma unroll
  for (int c = 0; c < 32; ++c) xu[c] = (float)((double)xu[c] * inv_root);
}

// phi operand tiling: the (2 + lanes) * lanes phi rows (<= 24) in tiles of
// 16 weight rows, four waves per tile, each over up to kPhiPairs 64-wide
// k-pairs of the lanes * dim (<= 2048) columns.
constexpr int kPhiPairs = 8;

// The one-workgroup part between two layers: post(l - 1), then pre(l) (or
// the final norm).  Every global operand is loaded at entry, the ones the
// post half needs first and the phi weights last, so the kernel pays about
// one memory latency; after that it runs from registers and LDS, with
// LDS-only barriers (a full barrier would also wait for the phi weight
// stream and for every global store of the launch).
//
// The phi rows (runtime.ts:401-411) run on v_mfma_f32_16x16x32_f16: the
// normalized lanes nl (|nl| < sqrt(lanes * d) by construction) are scaled by
// the power of two split_scale and split into fp16 halves, hi = f16(v) and
// lo = f16(v - hi), which hold v to 22 bits (2^-24 of split_scale absolute
// below 2^-14); the int8 weights are exact in fp16 and the products exact in
// the fp32 accumulator.  A = rows 0 (hi) and 1 (lo), zeros elsewhere; B = 16
// weight rows of the tile; lane l supplies A row l % 16 and B column l % 16,
// eight k of each 32-wide step: for k-pair p, lane block kb = l / 16 loads
// the 16 weight bytes [64 p + 16 kb, +16) and the first MFMA of the pair
// takes bytes [0, 8) of every block, the second [8, 16) (the A halves are
// read at the same k).  D rows 0 and 1 (hi, lo) land in lanes 0..15, outputs
// 0 and 1; the four waves of a tile meet in LDS and the sum is taken in
// float64 times the row scale.
//
// PU (Cactus-Quant): phi_pre, phi_post and phi_res share one format (width,
// group, codebook), so one rotation and one width dispatch serve every row;
// otherwise each row takes its own matrix's format.
// Attention workgroup ah (KV head ah) of the fused launch.  It issues its
// cache tiles at once (every row but this position's is final before the
// launch), then waits until the projection workgroups of its KV head (its
// query and gate heads, key and value) have counted in on its counter (q,
// this position's cache rows and the gate are in the XCD's L2), reads
// the fresh rows again past its L1, runs the gated attention of the KV head with nd_launch_attention_gated's
// instance and arguments for a ring of at most kGatedChunk positions -- the
// same values in the same order, so the same bits -- and clears its counter
// for the next launch.  A wait that runs out sets kStatusAttWait; an abort
// from the projection stores nothing.
// (The hook holds copies of the launch arguments it needs: the address of
// the argument block itself would cost a private copy of it.)
// STAMP: thread 0 writes the clock to marks[i] (LDS): 0 when the wait
// ended, then at the attention body's marks (hook.mark(i)).
template <bool STAMP = false>
struct AttWaitT {
  static constexpr bool kActive = true;
  static constexpr bool kStamp = STAMP;
  uint32_t* count;
  uint32_t* status;
  uint32_t* go;  // an LDS word
  uint32_t target, spin, slot;
  uint64_t* marks;
  __device__ void mark(int i) const {
    if constexpr (STAMP) {
      if (threadIdx.x == 0) marks[i] = wall_clock64();
    }
  }
  __device__ bool wait() const {
    if (threadIdx.x == 0) {
      bool ok = true;
      uint32_t it = 0, v;
      while (((v = __hip_atomic_load(count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)) &
              kFlagCount) < target &&
             !(v & kFlagAbort)) {
        if (++it >= spin) {
          __hip_atomic_fetch_or(status, kStatusAttWait, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
          ok = false;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (v & kFlagAbort) ok = false;
      *go = ok;
      if constexpr (STAMP) marks[0] = wall_clock64();
    }
    __syncthreads();
    return *go != 0;
  }
  __device__ uint32_t fresh_slot() const { return slot; }
  // After the attention: clear the count for the next launch.  The
  // workgroup is its counter's one waiter, and every arrival
  // it waited for has landed, so a plain store does it, with no returning
  // atomic (a round trip through the L2) at the end of the launch's last
  // workgroups.  (After an abort, arrivals may still land; the status bit
  // is then set and the next reset clears the counters.)
  __device__ void release() const {
    if (threadIdx.x == 0)
      __hip_atomic_store(count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
};

// STAMP: marks[0] when the wait ended, [1] when q and the gates were
// issued, [2] after the tile math, [3] after the waves' combine, [4] when the
// output stores had completed (thread 0, LDS).
template <bool STAMP = false>
__device__ __forceinline__ void attention_role(const MixArgs& a, uint32_t ah,
                                               uint64_t* marks = nullptr) {
  __shared__ uint32_t s_att_go;
  const AttArgs& g = a.att;
  const AttWaitT<STAMP> w{a.att_count + kAttStride * ah, a.status, &s_att_go, a.att_target,
                          a.spin, kv_slot(g.position[0], g.sink, g.window), marks};
  nd::att::attention_body<2, false, false, kMixWg / 64, 1, false, false, false, AttWaitT<STAMP>>(
      0u, ah, 0u, g.Kc, g.Vc, g.Ks, g.Vs, g.q, g.out, g.gate, 0u, nullptr, nullptr, nullptr,
      g.layer, g.kv_heads, g.alloc, g.sink, g.window,
      nd::att::Visible{g.alloc, g.alloc, g.alloc}, g.position, 1u, g.kv_heads, 0u,
      nd::att::kGatedChunk, 1u, 0.125f, 1u, 1u, nullptr, w);
  if constexpr (STAMP) {
    __builtin_amdgcn_s_waitcnt(0);
    if (threadIdx.x == 0) marks[4] = wall_clock64();
  }
  w.release();
}

template <bool CQ, bool WO = false, bool PU = true, bool STAMP = false>
__global__ __launch_bounds__(kMixWg) void n2_mix_kernel(MixArgs a) {
  static_assert(kQkvWg == kMixWg, "the fused projection runs on mix-sized workgroups");
  uint64_t stamp[16] = {};
  if constexpr (STAMP) stamp[0] = wall_clock64();
  auto mark = [&](int i) {
    if constexpr (STAMP) stamp[i] = wall_clock64();
  };
  auto put_stamps = [&](uint32_t k) {
    if constexpr (STAMP) {
      if (threadIdx.x == 0) {
        stamp[3] = wall_clock64();
#pragma unroll
        for (int i = 0; i < 16; ++i) a.stamps[16 * k + i] = stamp[i];
      }
    }
  };
  if constexpr (WO) {
    // Workgroups L % 8 == 0 only (one XCD): L / 8 < wo_groups computes Wo
    // rows, L / 8 == wo_groups (dispatched after all of them) runs the mix,
    // the qkv_groups after it the projection, the att_groups after those
    // the attention.  Each waits only on workgroups dispatched before it.
    if (blockIdx.x & 7) return;
    const uint32_t k = blockIdx.x >> 3;
    if (k < a.wo_groups) {
      __shared__ uint64_t s_wo_marks[STAMP ? 4 : 1];
      if constexpr (CQ) {
        if (a.wo_bits == 4)
          wo_cq_rows<4, STAMP>(a.wo_cq, k, a.wo_count, s_wo_marks);
        else if (a.wo_bits == 3)
          wo_cq_rows<3, STAMP>(a.wo_cq, k, a.wo_count, s_wo_marks);
        else
          wo_cq_rows<2, STAMP>(a.wo_cq, k, a.wo_count, s_wo_marks);
      } else {
        wo_rows<STAMP>(a, k, s_wo_marks);
      }
      if constexpr (STAMP) {
        if (threadIdx.x == 0)
          for (int i = 0; i < 3; ++i) stamp[4 + i] = s_wo_marks[i];
      }
      put_stamps(k);
      return;
    }
    if (k > a.wo_groups) {
      const uint32_t qb = k - a.wo_groups - 1;
      __shared__ uint64_t s_marks[STAMP ? 8 : 1];
      if (qb < a.qkv_groups) {
        qkv_body<CQ, true, STAMP>(a.qkv, qb, a.qkv_flag, a.qkv_groups, a.status, a.spin,
                                  a.att_groups ? a.att_count : nullptr, s_marks);
      } else if (qb - a.qkv_groups < a.att_groups) {
        attention_role<STAMP>(a, qb - a.qkv_groups, s_marks);
      }
      if constexpr (STAMP) {
        __syncthreads();
        if (threadIdx.x == 0)
          for (int i = 0; i < 8; ++i) stamp[4 + i] = s_marks[i];
      }
      put_stamps(k);
      return;
    }
  } else if (blockIdx.x) {
    const uint32_t m = blockIdx.x, D0 = a.d, L0 = a.lanes;
    a.x += (size_t)m * L0 * D0;
    a.proj += (size_t)m * D0;
    a.blk += (size_t)m * D0;
    a.upd += (size_t)m * D0;
    a.ain += (size_t)m * D0;
    a.route += (size_t)m * 20;
    a.phi_post += (size_t)m * L0;
    a.phi_res += (size_t)m * L0 * L0;
    a.ekey += (size_t)m * a.ek_ld;
    a.evalue += (size_t)m * a.ev_ld;
    if (a.route_out) a.route_out += (size_t)m * 20;
    if (a.cell) a.cell += (size_t)m * a.cell_ld;
  }
  __shared__ __align__(16) _Float16 s_split[2][2048];  // hi, lo of the scaled nl
  __shared__ float hv1[kMixWg], hv2[kMixWg];
  __shared__ double red[2][2 * (kMixWg / 64)];
  __shared__ __align__(16) float s_part[32][4][2];  // [phi row][wave of the tile][hi, lo]
  __shared__ float phi[24], rt[20];
  __shared__ float s_cqx[CQ ? 2048 + 2048 / 32 : 1];  // rotated lanes, padded
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t D = a.d, L = a.lanes, N = L * D, H = a.hdim;
  const uint32_t nrows = 2 * L + L * L;
  const bool col = t < D;
  int phase = 0;
  // ---- loads, unconditional and in first-use order (every pointer is valid
  // even for a half that is off, indices are clamped in bounds), so the
  // post half waits for its own operands only: post operands and lanes, the
  // phi weights, then the pre operands.  The three phi matrices are picked by
  // uniform selection: indexing the argument block per lane would cost a
  // dependent load.
  const int8_t* const w0 = a.phi_w[0];
  const int8_t* const w1 = a.phi_w[1];
  const int8_t* const w2 = a.phi_w[2];
  const float* const s0 = a.phi_s[0];
  const float* const s1 = a.phi_s[1];
  const float* const s2 = a.phi_s[2];
  const uint32_t tc = min(t, D - 1);
  float p = WO ? 0.f : a.proj[tc];  // WO: read once the Wo rows are in
  const float blk = a.blk[tc], upd = a.upd[tc], post_norm = a.post_norm[tc],
              pre_h = a.pre_h_norm[tc], d1 = a.d1[tc], d3 = a.d3[tc], d2 = a.d2[min(t, H - 1)],
              route = a.route[min(t, L * L + L - 1)];
  float xl[4];
#pragma unroll
  for (int l = 0; l < 4; ++l) xl[l] = a.x[(size_t)min((uint32_t)l, L - 1) * D + tc];
  // phi weights: wave w takes tile w & 1 and k-pairs [ppw (w >> 1), +ppw).
  const uint32_t r16 = lane & 15, kb = lane >> 4;
  const uint32_t tile = wave & 1, kq = wave >> 1;
  const uint32_t prow = tile * 16 + r16;
  const bool prow_ok = prow < nrows;
  const uint32_t pairs = N / 64, ppw = (pairs + 3) / 4;
  const uint32_t pr = prow_ok ? prow : 0;
  const int8_t* wrow = (pr < L ? w0 + (size_t)pr * N
                               : (pr < 2 * L ? w1 + (size_t)(pr - L) * N
                                             : w2 + (size_t)(pr - 2 * L) * N)) + kb * 16;
  // Unconditional loads at clamped (in-bounds) addresses: a predicated load
  // would make the compiler wait for it (and for every older load) at its
  // branch.  Pairs past the wave's share are skipped by the MFMA loop and
  // rows past the phi rows are zeroed there.
  __builtin_amdgcn_sched_barrier(0);
  u32x4 pw[kPhiPairs];
  if constexpr (!CQ) {
#pragma unroll
    for (int i = 0; i < kPhiPairs; ++i) {
      const uint32_t pp = min(kq * ppw + i, pairs - 1);
      pw[i] = *reinterpret_cast<const u32x4*>(wrow + (size_t)pp * 64);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t tr = min(t, nrows - 1);
  const float norm_in = a.norm_input[tc], ekey = a.ekey[tc], evalue = a.evalue[tc],
              fnorm = a.final_norm[tc];
  float psc = 0.f, spre = 0.f;
  if constexpr (!CQ) {
    psc = tr < L ? s0[tr] : (tr < 2 * L ? s1[tr - L] : s2[tr - 2 * L]);
    spre = s0[min(lane, L - 1)];
  }
  const float bpre = a.b_pre[min(lane, L - 1)];
  __shared__ float s_cb[3][16];
  // Cactus-Quant phi rows: wave w takes rows w, w + 8 and w + 16 (rows of
  // phi_pre, phi_post, phi_res in that order; rows w + 8 and w + 16 are
  // always phi_res), lane u the rows' 32-code unit u -- its packed words
  // (bits of them) and the norms of its groups -- loaded here with the
  // other operands, each row in its own matrix's format.
  uint32_t cw[3][4] = {}, cn[3][4] = {};
  if constexpr (CQ) {
    if (t == 0) {  // constant indices into the argument block
#pragma unroll
      for (int m = 0; m < (PU ? 1 : 3); ++m)
#pragma unroll
        for (int i = 0; i < 16; ++i) s_cb[m][i] = a.cq_cb[m][i];
    }
    const uint32_t ul = min(lane, N / 32 - 1);
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const uint32_t r = min(wave + 8u * j, nrows - 1);
      const uint32_t mat = r < L ? 0u : (r < 2 * L ? 1u : 2u);
      const uint32_t rr = r - (mat == 0 ? 0u : (mat == 1 ? L : 2 * L));
      const uint8_t* pm = sel3(mat, a.cq_p[0], a.cq_p[1], a.cq_p[2]);
      const uint16_t* nm = sel3(mat, a.cq_n[0], a.cq_n[1], a.cq_n[2]);
      const uint32_t bits = PU ? a.cq_bits[0] : sel3(mat, a.cq_bits[0], a.cq_bits[1], a.cq_bits[2]);
      const uint32_t g = PU ? a.cq_g[0] : sel3(mat, a.cq_g[0], a.cq_g[1], a.cq_g[2]);
      const uint32_t rb = PU ? a.cq_row_bytes[0]
                             : sel3(mat, a.cq_row_bytes[0], a.cq_row_bytes[1], a.cq_row_bytes[2]);
      const uint32_t ng = PU ? a.cq_groups[0]
                             : sel3(mat, a.cq_groups[0], a.cq_groups[1], a.cq_groups[2]);
      const uint32_t ubw = bits == 4 ? 4u : (bits == 3 ? 3u : 2u);  // words per unit
      const uint32_t gpu = g >= 32 ? 1u : 32u / g;                  // groups per unit
      const uint32_t* prow = reinterpret_cast<const uint32_t*>(pm + (size_t)rr * rb) + ul * ubw;
      const uint16_t* nrow = nm + (size_t)rr * ng + (ul * 32) / g;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if ((uint32_t)k < ubw) cw[j][k] = prow[k];
        if ((uint32_t)k < gpu) cn[j][k] = nrow[k];
      }
    }
  }

  if constexpr (WO) {
    // Every operand above is in flight; wait for the Wo workgroups' count
    // (read past the CU's L1 in the XCD's L2, where they add it), then read
    // their rows the same way, and reset the count for the next launch.
    // When the wait runs out: set the status bit, release the projection
    // workgroups with the abort bit and store nothing.
    __shared__ uint32_t s_go;
    if (t == 0) {
      bool go = true;
      uint32_t it = 0;
      while (__hip_atomic_load(a.wo_count, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) <
             a.wo_target) {
        if (++it >= a.spin) {
          __hip_atomic_fetch_or(a.status, kStatusWoWait, __ATOMIC_RELAXED,
                                __HIP_MEMORY_SCOPE_AGENT);
          go = false;
          break;
        }
        __builtin_amdgcn_s_sleep(1);
      }
      if (!go && a.qkv_groups)
        __hip_atomic_store(a.qkv_flag, kFlagAbort | 1u, __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
      s_go = go;
    }
    __syncthreads();
    if (!s_go) return;
    if constexpr (STAMP) stamp[1] = wall_clock64();
    p = __hip_atomic_load(a.proj + tc, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    if (t == 0) __hip_atomic_store(a.wo_count, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  }
  // ---- post(l - 1)
  if (a.has_post) {
    const double sp = mix_sum(col ? (double)p * p : 0.0, red, phase);
    const double ip = 1.0 / sqrt(div_pow2(sp, a.d_log2, D) + 1e-6);
    float after = 0.f;
    if (col) {
      const float np = (float)((1.0 + (double)post_norm) * (double)p * ip);
      after = (float)((double)blk + a.attention_scale * (double)np);
    }
    if (t < L * L + L) rt[t] = route;  // visible after the next barrier
    const double sa = mix_sum(col ? (double)after * after : 0.0, red, phase);
    const double ia = 1.0 / sqrt(div_pow2(sa, a.d_log2, D) + 1e-6);
    mark(4);
    // hadamardMlp (math.ts:117-138): FWHT(d1 x), SiLU(z / sqrt(H) * d2),
    // FWHT, / sqrt(H) * d3.
    float v = 0.f;
    if (col) {
      const float pre = (float)((1.0 + (double)pre_h) * (double)after * ia);
      v = (float)((double)pre * (double)d1);
    }
    const double inv_root = a.inv_root_h;
    v = fwht_block(v, hv1, H, t);
    mark(5);
    if (t < H) {
      const double z = (double)v * inv_root * (double)d2;
      v = (float)(z * sigmoid_d(z));
    } else {
      v = 0.f;
    }
    v = fwht_block(v, hv2, H, t);
    mark(6);
    if (col) {
      const float mlp = (float)((double)v * inv_root * (double)d3);
      const float delta = (float)((double)after + (double)mlp - (double)upd);
      float nx[4];
#pragma unroll
      for (int l = 0; l < 4; ++l) {
        if ((uint32_t)l >= L) break;
        double sum = 0.0;
#pragma unroll
        for (int s2 = 0; s2 < 4; ++s2)
          if ((uint32_t)s2 < L) sum += (double)rt[l * L + s2] * (double)xl[s2];
        nx[l] = (float)(sum + (double)rt[L * L + l] * (double)delta);
      }
#pragma unroll
      for (int l = 0; l < 4; ++l)
        if ((uint32_t)l < L) {
          xl[l] = nx[l];
          a.x[(size_t)l * D + t] = nx[l];
        }
      if (a.cell) {
        double sum = 0.0;
#pragma unroll
        for (int l = 0; l < 4; ++l)
          if ((uint32_t)l < L) sum += xl[l];
        a.cell[t] = (float)div_pow2(sum, a.l_log2, L);
      }
    }
  }
  if (a.has_final && (WO ? 0u : blockIdx.x) == a.final_row) {
    float m = 0.f;
    if (col) {
      double sum = 0.0;
#pragma unroll
      for (int l = 0; l < 4; ++l)
        if ((uint32_t)l < L) sum += xl[l];
      m = (float)div_pow2(sum, a.l_log2, L);
    }
    const double ss = mix_sum(col ? (double)m * m : 0.0, red, phase);
    const double inv = 1.0 / sqrt(div_pow2(ss, a.d_log2, D) + 1e-6);
    if (col) a.fin[t] = (float)((1.0 + (double)fnorm) * (double)m * inv);
  }
  mark(7);
  if (!a.has_pre) return;

  // ---- pre(l): rmsUnit over all lanes (math.ts:34-44), then the phi rows.
  double ss = 0.0;
#pragma unroll
  for (int l = 0; l < 4; ++l)
    if ((uint32_t)l < L) ss += (double)xl[l] * (double)xl[l];
  ss = mix_sum(col ? ss : 0.0, red, phase);
  const double inv = 1.0 / sqrt(div_pow2(ss, a.n_log2, N) + 1e-6);
  mark(8);
  float pre_phi = 0.f;  // phi_pre row `lane` (lane < lanes): feeds hPre
  if constexpr (CQ) {
    // phi = cqMatvec of the normalized lanes (backends/cq.ts:30-46, 107-231):
    // prepareCqActivation -- per group the butterflies (strides 1 .. g / 2,
    // one fp32 add and subtract per pair), then times 1/sqrt(g) -- and the
    // rows by code width (cq_phi_row_any).  The N <= 2048 normalized values are
    // 64 units of 32, one per lane of a wave: each wave reads them from LDS
    // (one pad float after every 32, so lane u's unit starts at 33 u and a
    // wave's reads fall in distinct banks) and rotates its own copy in
    // registers, strides below 32 inside the unit and strides 32 .. g / 2
    // across the lanes holding the group's other units.
    // PU with d a multiple of 64: thread t holds element l d + t of every
    // lane l, so a group below 64 values lies in one wave and its strides
    // run across the wave's lanes once (cq_rotate_lanes), then times
    // 1/sqrt(g) when the group ends there; each wave then takes the wider
    // groups' strides 64 .. g / 2 across the lanes holding the group's other
    // units, and their scaling.  The same operations on the same operands
    // as cq_rotate_unit, done once instead of once per wave.
    const uint32_t g0 = a.cq_g[0];
    const bool lanes_rot = PU && (D & 63u) == 0;
    if (col) {
#pragma unroll
      for (int l = 0; l < 4; ++l)
        if ((uint32_t)l < L) {
          const uint32_t e = l * D + t;
          float v = (float)((double)xl[l] * inv);
          if (lanes_rot) {
            v = cq_rotate_lanes(v, g0, lane);
            if (g0 <= 64) v = (float)((double)v * a.cq_inv_root[0]);
          }
          s_cqx[e + (e >> 5)] = v;
        }
    }
    nd::lds_barrier();
    mark(12);
    const uint32_t units = N / 32, uc = lane < units ? lane : 0;
    if constexpr (PU) {
      float xu[32];
#pragma unroll
      for (int c = 0; c < 32; ++c) xu[c] = s_cqx[uc * 33 + c];
      if (lanes_rot) {
        if (g0 > 64) cq_rotate_wide(xu, g0, a.cq_inv_root[0], lane);
      } else {
        cq_rotate_unit(xu, g0, a.cq_inv_root[0], lane);
      }
      if constexpr (STAMP) {
#pragma unroll
        for (int c = 0; c < 32; ++c) asm volatile("" ::"v"(xu[c]));
        mark(13);
      }
      if (a.cq_bits[0] == 4)
        cq_phi_rows<4>(cw, cn, xu, s_cb[0], a.cq_g[0], units, nrows, wave, lane, phi);
      else if (a.cq_bits[0] == 3)
        cq_phi_rows<3>(cw, cn, xu, s_cb[0], a.cq_g[0], units, nrows, wave, lane, phi);
      else  // 2-bit codes and ternary crumbs
        cq_phi_rows<2>(cw, cn, xu, s_cb[0], a.cq_g[0], units, nrows, wave, lane, phi);
      mark(14);
    } else {
    // Rows j = 0 take the rotation by their own matrix's group, rows j >= 1
    // (phi_res) by phi_res's; one rotation serves both when the groups agree.
    const uint32_t r0 = wave, mat0 = r0 < L ? 0u : (r0 < 2 * L ? 1u : 2u);
    const uint32_t g0 = sel3(mat0, a.cq_g[0], a.cq_g[1], a.cq_g[2]), gr = a.cq_g[2];
    const bool same = g0 == gr;
    float xa[32], xb[32];
#pragma unroll
    for (int c = 0; c < 32; ++c) xa[c] = s_cqx[uc * 33 + c];
    cq_rotate_unit(xa, g0, sel3(mat0, a.cq_inv_root[0], a.cq_inv_root[1], a.cq_inv_root[2]),
                   lane);
    if (!same) {
#pragma unroll
      for (int c = 0; c < 32; ++c) xb[c] = s_cqx[uc * 33 + c];
      cq_rotate_unit(xb, gr, a.cq_inv_root[2], lane);
    }
#pragma unroll
    for (int j = 0; j < 3; ++j) {
      const uint32_t r = wave + 8u * j;
      if (r >= nrows) break;  // uniform over the wave
      const uint32_t mat = r < L ? 0u : (r < 2 * L ? 1u : 2u);
      const uint32_t bits = sel3(mat, a.cq_bits[0], a.cq_bits[1], a.cq_bits[2]);
      const uint32_t g = sel3(mat, a.cq_g[0], a.cq_g[1], a.cq_g[2]);
      double total;
      if (j == 0 || same)
        total = cq_phi_row_any(bits, cw[j], cn[j], xa, s_cb[mat], g, units, lane);
      else
        total = cq_phi_row_any(bits, cw[j], cn[j], xb, s_cb[mat], g, units, lane);
      total = nd::wave_sum(total);
      if (lane == 0) phi[r] = (float)total;
    }
    }
    nd::lds_barrier();
    if (t < nrows) {
      const float v = phi[t];
      if (t >= L && t < 2 * L) a.phi_post[t - L] = v;
      if (t >= 2 * L) a.phi_res[t - 2 * L] = v;
    }
    pre_phi = phi[min(lane, L - 1)];
  } else {
    if (col) {
  #pragma unroll
      for (int l = 0; l < 4; ++l)
        if ((uint32_t)l < L) {
          const float v = (float)((double)xl[l] * inv) * a.split_scale;
          const _Float16 h = (_Float16)v;
          s_split[0][l * D + t] = h;
          s_split[1][l * D + t] = (_Float16)(v - (float)h);
        }
    }
    nd::lds_barrier();
    mark(12);
    float4v acc = {0.f, 0.f, 0.f, 0.f};
  #pragma unroll
    for (int i = 0; i < kPhiPairs; ++i) {
      const uint32_t pp = kq * ppw + i;
      if ((uint32_t)i < ppw && pp < pairs) {  // uniform over the wave
  #pragma unroll
        for (int h = 0; h < 2; ++h) {
          half8 av = {};
          if (r16 < 2)
            av = *reinterpret_cast<const half8*>(&s_split[r16][pp * 64 + kb * 16 + h * 8]);
          const u32x4 wv = prow_ok ? pw[i] : u32x4{0u, 0u, 0u, 0u};
          const half8 bv = nd::codes_to_half(h ? u32x2{wv.z, wv.w} : u32x2{wv.x, wv.y});
          acc = __builtin_amdgcn_mfma_f32_16x16x32_f16(av, bv, acc, 0, 0, 0);
        }
      }
    }
    mark(13);
    if (lane < 16) {
      s_part[prow][kq][0] = acc[0];
      s_part[prow][kq][1] = acc[1];
    }
    nd::lds_barrier();
    mark(14);
    // phi row r = scale_r * 2^-s * sum over the tile's waves of (hi + lo), in
    // float64; every thread takes the phi_pre rows itself (they feed hPre).
    auto phi_row = [&](uint32_t r, float scale) -> float {
      const float4 q0 = *reinterpret_cast<const float4*>(&s_part[r][0][0]);
      const float4 q1 = *reinterpret_cast<const float4*>(&s_part[r][2][0]);
      const double sum = (((double)q0.x + (double)q0.y) + ((double)q0.z + (double)q0.w)) +
                         (((double)q1.x + (double)q1.y) + ((double)q1.z + (double)q1.w));
      return (float)((double)scale * (sum * (double)a.split_unscale));
    };
    if (t < nrows) {
      const float v = phi_row(t, psc);
      phi[t] = v;  // read by route_wave after later barriers
      if (t >= L && t < 2 * L) a.phi_post[t - L] = v;
      if (t >= 2 * L) a.phi_res[t - 2 * L] = v;
    }
    pre_phi = phi_row(min(lane, L - 1), spre);
  }
  // hPre (runtime.ts:412-417): lane l < lanes of every wave takes lane l's
  // gate, and the wave shares them by readlane (no barrier).
  mark(9);
  float hp = 0.f;
  if (lane < L) {
    const double off = lane == a.own_pre ? 4.0 : -4.0;
    hp = (float)sigmoid_d((double)a.a_pre * (double)pre_phi + (double)bpre + off);
  }
  float hpre[4];
#pragma unroll
  for (int l = 0; l < 4; ++l) hpre[l] = nd::readlane(hp, l);
  // updateInput = sum_lane hPre[lane] * x[lane].
  float u = 0.f;
  if (col) {
    double sum = 0.0;
#pragma unroll
    for (int l = 0; l < 4; ++l)
      if ((uint32_t)l < L) sum += (double)hpre[l] * (double)xl[l];
    u = (float)sum;
    a.upd[t] = u;
  }
  float b = u;
  if (a.has_site) {
    // alpha = sigmoid(rmsUnit(u) . rmsUnit(key) / sqrt(d)); block = u + alpha * value.
    double su = col ? (double)u * u : 0.0, sk = col ? (double)ekey * ekey : 0.0;
    mix_sum2(su, sk, red, phase);
    const double iu = 1.0 / sqrt(div_pow2(su, a.d_log2, D) + 1e-6),
                 ik = 1.0 / sqrt(div_pow2(sk, a.d_log2, D) + 1e-6);
    const float nu = (float)((double)u * iu), nk = (float)((double)ekey * ik);
    const double dot = mix_sum(col ? (double)nu * (double)nk : 0.0, red, phase);
    const double alpha = sigmoid_d(dot / a.sqrt_d);
    if (col) b = (float)((double)u + alpha * (double)evalue);
  }
  mark(10);
  if (col) a.blk[t] = b;
  // attentionInput = rmsNorm(block, normInput) (math.ts:16-32).
  const double sb = mix_sum(col ? (double)b * b : 0.0, red, phase);
  const double ib = 1.0 / sqrt(div_pow2(sb, a.d_log2, D) + 1e-6);
  if (col) a.ain[t] = (float)((1.0 + (double)norm_in) * (double)b * ib);
  mark(11);
  if constexpr (WO) {
    if (a.qkv_groups) {  // the input and the phi values are in the L2: signal
      __builtin_amdgcn_s_waitcnt(0);
      __syncthreads();
      if (t == 0)
        __hip_atomic_store(a.qkv_flag, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      if constexpr (STAMP) stamp[2] = wall_clock64();
    }
  }
  if (a.route_out) {
    RouteArgs r{};
    r.phi_post = phi + L;
    r.phi_res = phi + 2 * L;
    r.a_post = a.r_a_post;
    r.a_res = a.r_a_res;
    r.b_post = a.r_b_post;
    r.b_res = a.r_b_res;
    r.lanes = L;
    r.own = a.own_pre;
    r.route = a.route_out;
    route_wave(r, t, rt);
  }
  if constexpr (WO) put_stamps(blockIdx.x >> 3);
}

// ---------------------------------------------------------------- prefill
// NeedleRuntime.prefill runs one step per prompt token (runtime.ts:227-243).
// The batched form below gives each of M prompt positions its own row and
// runs every layer for all of them at once: the projections become int8
// MFMA GEMMs (digit-sliced, exact to 2^-22 of a row's largest entry), the
// one-workgroup parts become one workgroup per position, and causal
// attention reads the int8 cache, which holds every earlier position because
// each position's K/V is appended before any attention of the layer runs.
// It applies while the prompt's cache slots do not wrap (positions < slots),
// which keeps every position a later query can see in the cache.

// Per position: token from the prompt in `history`, engram hashes, scaled
// embedding in every lane, concatenated engram rows; workgroup 0 advances the
// position counters past the batch.
__global__ __launch_bounds__(kWg) void n2_begin_batch_kernel(BeginArgs a, uint32_t p0,
                                                             uint32_t count,
                                                             uint32_t* __restrict__ positions) {
  __shared__ uint32_t s_idx[16], s_valid[16];
  const uint32_t m = blockIdx.x, t = threadIdx.x, pos = p0 + m;
  const uint32_t tok = a.history[pos];
  if (t == 0) {
    positions[m] = pos;
    if (m == 0) {
      a.st[0] = p0 + count;
      a.st[1] = p0 + count - 1;
    }
  }
  if (t < a.tables) {
    const uint32_t order = a.orders[t / a.per_order];
    uint32_t hash = 0x9E3779B9u * (t + 1);
    bool valid = true;
    for (uint32_t off = 0; off < order; ++off) {
      const bool in = off <= pos;
      const uint32_t token = in ? a.history[pos - off] : 0u;
      hash = (hash ^ token) * 0x01000193u;
      if (off == order - 1) valid = in;
    }
    hash ^= hash >> 15;
    s_idx[t] = hash % a.slots;
    s_valid[t] = valid ? 1u : 0u;
    if (a.cq_lookup) {
      uint32_t* lk = a.cq_lookup + (size_t)m * (2 * a.tables + 1);
      lk[t] = s_idx[t];
      lk[a.tables + t] = s_valid[t];
    }
  }
  if (a.cq_lookup) {  // the rows come from n2_cq_rows_kernel
    if (t == 0) a.cq_lookup[(size_t)m * (2 * a.tables + 1) + 2 * a.tables] = tok;
    return;
  }
  __syncthreads();
  float* x = a.x + (size_t)m * a.lanes * a.d;
  for (uint32_t k = t; k < a.d; k += kWg) {
    const float row = (float)a.emb[(size_t)tok * a.d + k] * a.emb_s[tok];
    const float v = (float)((double)row * a.scale);
    for (uint32_t l = 0; l < a.lanes; ++l) x[(size_t)l * a.d + k] = v;
    if (a.cell0) a.cell0[(size_t)m * a.cell_ld + k] = v;
  }
  const uint32_t per_site = a.tables * a.sub;
  float* cat = a.cat + (size_t)m * a.n_sites * per_site;
  for (uint32_t i = t; i < a.n_sites * per_site; i += kWg) {
    const uint32_t s = i / per_site, j = i % per_site, tb = j / a.sub, c = j % a.sub;
    float v = 0.f;
    if (s_valid[tb]) {
      const size_t row = (size_t)tb * a.slots + s_idx[tb];
      v = (float)a.tw[s][row * a.sub + c] * a.ts[s][row];
    }
    cat[i] = v;
  }
}

// The engram convolution of position p0 + m (runtime.ts:854-872): value rows
// of batch positions come from this batch's projections ekv[m'][s] = [key |
// value], older ones from the ring (which the batch does not touch here).
__global__ void n2_conv_batch_kernel(const float* __restrict__ ekv, const float* __restrict__ ring,
                                     const float* __restrict__ taps, uint32_t d, uint32_t depth,
                                     uint32_t n_taps, uint32_t max_order, uint32_t n_sites,
                                     uint32_t p0, float* __restrict__ mixed) {
  const uint32_t m = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
  if (i >= d) return;
  const uint32_t pos = p0 + m;
  float acc = 0.f;
  for (uint32_t tap = 0; tap < n_taps; ++tap) {
    if (tap * max_order > pos) continue;
    const uint32_t prev = pos - tap * max_order;
    const float v = prev >= p0
        ? ekv[((size_t)(prev - p0) * n_sites + s) * 2 * d + d + i]
        : ring[((size_t)s * depth + prev % depth) * d + i];
    acc = (float)((double)acc + (double)taps[((size_t)s * n_taps + tap) * d + i] * (double)v);
  }
  mixed[((size_t)m * n_sites + s) * d + i] = acc;
}

// After the convolution: the ring keeps the value rows of the batch's last
// `depth` positions.
__global__ void n2_ring_store_kernel(const float* __restrict__ ekv, float* __restrict__ ring,
                                     uint32_t d, uint32_t depth, uint32_t n_sites, uint32_t p0,
                                     uint32_t count) {
  const uint32_t j = blockIdx.x, s = blockIdx.y, i = threadIdx.x;
  const uint32_t first = count > depth ? count - depth : 0;
  const uint32_t m = first + j;
  if (i >= d || m >= count) return;
  const uint32_t pos = p0 + m;
  ring[((size_t)s * depth + pos % depth) * d + i] =
      ekv[((size_t)m * n_sites + s) * 2 * d + d + i];
}

// Query/key norm + RoPE and the K/V append of every batch position: one wave
// per (head, position); qkvg rows [q | k | v | gate] with stride ld.
__global__ __launch_bounds__(64) void n2_rope_store_batch_kernel(
    const float* __restrict__ qkvg, uint32_t ld, uint32_t heads, uint32_t kv_heads,
    const float* __restrict__ q_norm, const float* __restrict__ k_norm,
    const double* __restrict__ inv_freq, uint32_t p0, float* __restrict__ q_out,
    void* __restrict__ Kc, void* __restrict__ Vc, float* __restrict__ Ks,
    float* __restrict__ Vs, uint32_t layer, uint32_t alloc, uint32_t sink, uint32_t window,
    uint32_t f32) {
  const uint32_t b = blockIdx.x, m = blockIdx.y, lane = threadIdx.x, pos = p0 + m;
  const int role = b < heads ? 0 : (b < heads + kv_heads ? 1 : 2);
  const uint32_t h = role == 0 ? b : (role == 1 ? b - heads : b - heads - kv_heads);
  const float val = qkvg[(size_t)m * ld + (size_t)b * kHd + lane];
  double sn, cs;
  sincos((double)pos * inv_freq[lane & 31], &sn, &cs);
  head_epilogue(val, lane, role, sn, cs, role == 0 ? q_norm[lane] : k_norm[lane],
                q_out + ((size_t)m * heads + h) * kHd, Kc, Vc, Ks, Vs,
                ((size_t)layer * kv_heads + h) * alloc, kv_slot(pos, sink, window), alloc, f32);
}

// Confidence pool state (OnlineProbePool, runtime.ts:48-62) for up to
// kMaxProbes probes, float64.  The pool launch runs one workgroup per
// (probe p, 64-column chunk j), and each keeps its own copy of the running
// maximum and denominator ([p][j]: the copies are equal, every workgroup of
// a probe computing them from the same scores) so that no workgroup reads
// what another writes; weighted holds probe p's weighted cell sums.  A
// denominator of 0 means no cell yet (every pooled cell adds at least
// exp(0) = 1 through the maximum's own term).
constexpr uint32_t kMaxProbes = 8;
constexpr uint32_t kMaxChunks = 8;       // d <= 512
struct PoolState {
  double* max;       // [8][8]
  double* den;       // [8][8]
  double* weighted;  // [8][d]
};

// A lane's share of a d-vector (d <= 512): elements lane + 64 k, zero past
// d, loaded together from clamped addresses.
__device__ __forceinline__ void lane_share(const float* __restrict__ v, uint32_t D, uint32_t lane,
                                           float (&out)[8]) {
#pragma unroll
  for (int k = 0; k < 8; ++k) {
    const uint32_t i = lane + 64u * k;
    const float x = v[i < D ? i : D - 1];
    out[k] = i < D ? x : 0.f;
  }
}

// score = (cell . probe) / sqrt(d) in float64 (runtime.ts:66-72), from the
// lane shares of both vectors.
__device__ __forceinline__ double probe_score(const float (&cell)[8], const float (&probe)[8],
                                              double scale) {
  double sum = 0.0;
#pragma unroll
  for (int k = 0; k < 8; ++k) sum += (double)cell[k] * (double)probe[k];
  return nd::wave_sum(sum) * scale;
}

// Scores of C cells for every probe into scores[c][p], one wave per cell
// (the batched prefill's cells; a step's few cells are scored inside the
// pool launch).
__global__ __launch_bounds__(256) void n2_probe_scores_kernel(const float* __restrict__ cells,
                                                              uint32_t C, uint32_t D,
                                                              const float* __restrict__ probes,
                                                              uint32_t P, double scale,
                                                              double* __restrict__ scores) {
  const uint32_t c = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (c >= C) return;
  float cv[8];
  lane_share(cells + (size_t)c * D, D, lane, cv);
  for (uint32_t p = 0; p < P; ++p) {
    float pv[8];
    lane_share(probes + (size_t)p * D, D, lane, pv);
    const double v = probe_score(cv, pv, scale);
    if (lane == 0) scores[(size_t)c * kMaxProbes + p] = v;
  }
}

constexpr uint32_t kPoolThreads = 1024;  // 16 waves, each on every 16th cell

// The online update of runtime.ts:73-90 over C cells at once, in its closed
// form: M' = max(M, max_c s_c); every earlier term is rescaled by
// exp(M - M') (0 before the first cell) and cell c enters with weight
// exp(s_c - M').  Workgroup (p, j) updates probe p's weighted sums of
// columns [64 j, 64 j + 64) and its copy of (M, denominator).
__global__ __launch_bounds__(kPoolThreads) void n2_probe_pool_kernel(const float* __restrict__ cells,
                                                            uint32_t C, uint32_t D,
                                                            const double* __restrict__ scores,
                                                            PoolState ps) {
  constexpr uint32_t kChunk = 1024;
  __shared__ double e[kChunk];
  __shared__ double red[kPoolThreads];
  constexpr uint32_t kSlices = kPoolThreads / 64;
  const uint32_t p = blockIdx.x, j = blockIdx.y, t = threadIdx.x;
  const uint32_t col = j * 64 + (t & 63), slice = t >> 6;
  double* const my_max = ps.max + p * kMaxChunks + j;
  double* const my_den = ps.den + p * kMaxChunks + j;
  const double den_old = *my_den;
  const double m_old = den_old > 0.0 ? *my_max : -INFINITY;
  double mx = -INFINITY;
  for (uint32_t c = t; c < C; c += kPoolThreads) mx = fmax(mx, scores[(size_t)c * kMaxProbes + p]);
  red[t] = mx;
  __syncthreads();
  for (uint32_t w = kPoolThreads / 2; w > 0; w >>= 1) {
    if (t < w) red[t] = fmax(red[t], red[t + w]);
    __syncthreads();
  }
  const double m_new = fmax(m_old, red[0]);
  const double factor = m_old > -INFINITY ? exp(m_old - m_new) : 0.0;
  __syncthreads();
  double acc = 0.0, esum = 0.0;
  for (uint32_t c0 = 0; c0 < C; c0 += kChunk) {
    const uint32_t n = C - c0 < kChunk ? C - c0 : kChunk;
    for (uint32_t c = t; c < n; c += kPoolThreads) {
      const double w = exp(scores[(size_t)(c0 + c) * kMaxProbes + p] - m_new);
      e[c] = w;
      esum += w;
    }
    __syncthreads();
    if (col < D) {
#pragma unroll 16
      for (uint32_t c = slice; c < n; c += kSlices)
        acc += e[c] * (double)cells[(size_t)(c0 + c) * D + col];
    }
    __syncthreads();
  }
  red[t] = acc;
  __syncthreads();
  if (t < 64 && col < D) {
    double sum = red[t];
#pragma unroll
    for (uint32_t q = 1; q < kSlices; ++q) sum += red[t + 64 * q];
    double* w = ps.weighted + (size_t)p * D + col;
    *w = *w * factor + sum;
  }
  __syncthreads();
  red[t] = esum;
  __syncthreads();
  for (uint32_t w = kPoolThreads / 2; w > 0; w >>= 1) {
    if (t < w) red[t] += red[t + w];
    __syncthreads();
  }
  if (t == 0) {
    *my_den = den_old * factor + red[0];
    *my_max = m_new;
  }
}

// The same update for a step's C <= kStepCells cells, scored in the
// launch: every load is issued first (wave w holds lane shares of cells w,
// w + 4, ... and of probe p), the column chunk j of a cell is the share
// element j of the wave that holds it, and the few exponentials are taken
// once per cell.
constexpr uint32_t kStepCells = 32;
__global__ __launch_bounds__(256) void n2_probe_pool_step_kernel(const float* __restrict__ cells,
                                                                 uint32_t C, uint32_t D,
                                                                 const float* __restrict__ probes,
                                                                 double scale, PoolState ps) {
  constexpr int kPerWave = kStepCells / 4;
  __shared__ double sc[kStepCells], wt[kStepCells];
  __shared__ double part[4][64];
  const uint32_t p = blockIdx.x, j = blockIdx.y, t = threadIdx.x, wave = t >> 6, lane = t & 63;
  double* const my_max = ps.max + p * kMaxChunks + j;
  double* const my_den = ps.den + p * kMaxChunks + j;
  double* const my_w = ps.weighted + (size_t)p * D + j * 64 + lane;
  const double den_old = *my_den, m_stored = *my_max;
  const double w_old = j * 64 + lane < D ? *my_w : 0.0;
  float pv[8], cv[kPerWave][8];
  lane_share(probes + (size_t)p * D, D, lane, pv);
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const uint32_t c = wave + 4 * i;
    lane_share(cells + (size_t)(c < C ? c : 0) * D, D, lane, cv[i]);
  }
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const uint32_t c = wave + 4 * i;
    const double v = probe_score(cv[i], pv, scale);
    if (lane == 0 && c < C) sc[c] = v;
  }
  __syncthreads();
  const double m_old = den_old > 0.0 ? m_stored : -INFINITY;
  double m_new = m_old;
  for (uint32_t c = 0; c < C; ++c) m_new = fmax(m_new, sc[c]);
  const double factor = m_old > -INFINITY ? exp(m_old - m_new) : 0.0;
  if (wave == 0) {
    const double w = lane < C ? exp(sc[lane] - m_new) : 0.0;
    if (lane < C) wt[lane] = w;
    const double esum = nd::wave_sum(w);
    if (lane == 0) {
      *my_den = den_old * factor + esum;
      *my_max = m_new;
    }
  }
  __syncthreads();
  double acc = 0.0;
#pragma unroll
  for (int i = 0; i < kPerWave; ++i) {
    const uint32_t c = wave + 4 * i;
    float x = cv[i][0];
#pragma unroll
    for (int k = 1; k < 8; ++k) x = j == (uint32_t)k ? cv[i][k] : x;
    if (c < C) acc += wt[c] * (double)x;
  }
  part[wave][lane] = acc;
  __syncthreads();
  if (wave == 0 && j * 64 + lane < D)
    *my_w = w_old * factor + (((part[0][lane] + part[1][lane]) + part[2][lane]) + part[3][lane]);
}

// output() and confidence() (runtime.ts:93-104, 641-645): pooled =
// f32(weighted / max(denominator, 1e-30)), output 0 = f32(bias + projection
// row 0 . pooled) summed in float64, then its sigmoid in float64.
__global__ __launch_bounds__(256) void n2_probe_head_kernel(PoolState ps, uint32_t P, uint32_t D,
                                                            const float* __restrict__ projection,
                                                            float bias, double* __restrict__ out) {
  __shared__ double red[256];
  const uint32_t t = threadIdx.x;
  double sum = 0.0;
  for (uint32_t j = t; j < P * D; j += 256) {
    const double den = fmax(ps.den[(j / D) * kMaxChunks], 1e-30);
    const float pooled = (float)(ps.weighted[j] / den);
    sum += (double)projection[j] * (double)pooled;
  }
  red[t] = sum;
  __syncthreads();
  for (uint32_t w = 128; w > 0; w >>= 1) {
    if (t < w) red[t] += red[t + w];
    __syncthreads();
  }
  if (t == 0) {
    const float o = (float)((double)bias + red[0]);
    *out = 1.0 / (1.0 + exp(-(double)o));
  }
}

size_t al(size_t n) { return (n + 255) & ~size_t(255); }

}  // namespace

// Pinned staging slots of the session calls.
enum StageSlot : uint32_t {
  kStageLanes = 0,  // begin: lanes [lanes][dim]
  kStageLookup,     // prepare engrams: indices and valid flags
  kStageAllowed,    // selection: allowed ids [vocab]
  kStageForward,    // fallback forward: input, block, update [3][dim], x, phi post, phi res
  kStageEngram,     // host engram key (2 site) and value (2 site + 1) [dim], 4 sites
  kStageSlots = kStageEngram + 8
};

namespace {
// mask |= bit ids[i] for i < n (the ids the host accepted among the
// undecided pieces of a grammar mask).
__global__ void n2_set_bits_kernel(uint32_t* __restrict__ mask, const uint32_t* __restrict__ ids,
                                   uint32_t n) {
  const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
  if (i < n) atomicOr(mask + (ids[i] >> 5), 1u << (ids[i] & 31));
}
}  // namespace

struct nd_needle {
  nd_needle_desc d{};
  bool cq = false;  // every matrix in the Cactus-Quant form (else int8)
  // Owned: rows q | k | v | gate of each layer and key | value of each
  // engram site, concatenated when the parts share one format (int8, or
  // Cactus-Quant of one width, group and padding); otherwise (a mixed-width
  // archive) the entry keeps only its row count and the parts are owned
  // copies in `owned_parts`.
  std::vector<nd_mat> wqkvg;
  std::vector<nd_mat> ekv;
  // Cactus-Quant models: each part as a matrix of its own (views into the
  // concatenation, or the owned copies).
  std::vector<std::array<nd_mat, 4>> qkv_part;
  std::vector<std::array<nd_mat, 2>> ekv_part;
  std::vector<nd_mat> owned_parts;
  bool wo_fused = true;  // every layer's Wo fits the fused launch's rows
  bool phi_uniform = true;  // phi_pre, phi_post, phi_res share one format
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
  uint32_t *st = nullptr, *history = nullptr, *sel_id = nullptr, *allowed = nullptr,
           *counters = nullptr;
  // The allowed-token bitmask of the constrained selection calls: bit t of
  // word t / 32 (nd_needle_grammar_mask fills it; the _mask calls add the
  // ids the host accepted among the undecided ones).
  uint32_t* mask = nullptr;
  // arrivals of the fused launch's Wo rows (word 0) and projection heads
  // (word 32): a 128-byte line each
  uint32_t* wo_count = nullptr;
  uint32_t* qkv_flags = nullptr;  // per layer: the fused launch's mix-done flag
  // Give-ups of the fused launch's bounded waits (kStatus* bits; a line of
  // its own, cleared by reset), its pinned host copy, and the test hook's
  // extra Wo arrivals and spin bound (0: kWoSpin).
  uint32_t* status = nullptr;
  uint32_t* status_host = nullptr;
  uint32_t dbg_extra = 0, dbg_spin = 0;
  uint64_t* dbg_stamps = nullptr;  // measurement: the fused launches' clock stamps
  double *lp_history = nullptr, *sel_lp = nullptr;
  uint32_t* cq_lookup = nullptr;  // CQ model: a step's engram lookups and token
  float *ring = nullptr, *x = nullptr, *upd = nullptr, *blk = nullptr, *ain = nullptr,
        *qkvg = nullptr, *q = nullptr, *att = nullptr, *proj = nullptr, *phi_post_v = nullptr,
        *phi_res_v = nullptr, *fin = nullptr, *logits = nullptr, *cat = nullptr, *ekv_out = nullptr,
        *evals = nullptr, *partials = nullptr, *route = nullptr;
  double* rope = nullptr;
  uint32_t max_length = 0, sink = 0, position = 0;
  // Batched prefill buffers (first prefill), for up to pf_cap positions a pass.
  char* pf_arena = nullptr;
  uint32_t pf_cap = 0;
  float *pf_x = nullptr, *pf_upd = nullptr, *pf_blk = nullptr, *pf_ain = nullptr,
        *pf_phi_post = nullptr, *pf_phi_res = nullptr, *pf_route = nullptr, *pf_qkvg = nullptr,
        *pf_q = nullptr, *pf_att = nullptr, *pf_proj = nullptr, *pf_cat = nullptr,
        *pf_ekv = nullptr, *pf_evals = nullptr, *pf_fm = nullptr, *pf_partials = nullptr;
  int8_t* pf_digits = nullptr;
  uint32_t *pf_positions = nullptr, *pf_counters = nullptr;
  uint32_t* pf_cq_lookup = nullptr;  // CQ model: each position's engram lookups and token
  // Step graphs, valid for (graph_alloc, graph_sink).
  hipGraphExec_t graphs[3] = {nullptr, nullptr, nullptr};
  uint32_t graph_kernels[3] = {0, 0, 0};  // kernel launches each graph holds
  uint32_t graph_alloc = 0, graph_sink = 0, graph_mode = 0;
  // Confidence probe head (absent when the description has no probes):
  // probes [P][d] and projection row 0 [P * d] in params, the pool state in
  // the arena's cleared part, cells of one step (or one prefill pass) and
  // their scores as scratch.
  bool conf = false;
  bool collect = true;  // this reset's collectConfidence
  uint32_t probe_count = 0;
  size_t o_probes = 0, o_pproj = 0;
  float probe_bias0 = 0.f;
  PoolState pool{};
  float *cells = nullptr, *pf_cells = nullptr;
  double *scores = nullptr, *pf_scores = nullptr, *conf_out = nullptr;
  // Which calls drive the runtime since the last reset: 0 none yet, 1 whole
  // steps (nd_needle_step, _prefill, _step_select, _generate), 2 the session
  // methods (ResidentExecutionSession, backends/backend.ts:65-80).
  uint32_t api = 0;
  // Session token in flight: begin called, the next layer to run and the
  // token's position, the post half owed to the last layer run, engrams
  // prepared on the device for this token, logits awaiting selection.
  bool token_open = false, post_pending = false, engrams_ready = false, select_ready = false;
  uint32_t next_layer = 0, token_position = 0;
  uint32_t* lookup = nullptr;  // [2][engram_tables]: indices, valid flags
  // Engram keys and values handed over by the host ([2][sites][dim]; read by
  // the mix launches of the token instead of the device's own when set) and
  // the fallback forward's inputs (input, block, update, x, phi post, phi res).
  float *host_eng = nullptr, *fwd_in = nullptr;
  bool host_engrams = false;
  // Pinned staging of the session's host inputs, one slot per purpose; each
  // slot's event marks the completion of its last copy to the device.
  char* pinned = nullptr;
  size_t stage_off[kStageSlots] = {}, stage_bytes[kStageSlots] = {};
  hipEvent_t stage_done[kStageSlots] = {};
};

namespace {

void drop_graphs(nd_needle* n) {
  for (auto& g : n->graphs) {
    if (g) hipGraphExecDestroy(g);
    g = nullptr;
  }
}

// Pools C cells ([C][d]) into the confidence state: one launch that scores
// a step's few cells itself, else a scoring launch and the update.
hipError_t enqueue_pool(nd_needle* n, const float* cells, uint32_t C, double* scores,
                        hipStream_t s) {
  const uint32_t D = n->d.dim;
  const double scale = 1.0 / std::sqrt((double)D);
  const float* probes = n->params + n->o_probes;
  const dim3 grid(n->probe_count, (D + 63) / 64);
  if (C <= kStepCells) {
    hipLaunchKernelGGL(n2_probe_pool_step_kernel, grid, dim3(256), 0, s, cells, C, D, probes,
                       scale, n->pool);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(n2_probe_scores_kernel, dim3((C + 3) / 4), dim3(256), 0, s, cells, C, D,
                     probes, n->probe_count, scale, scores);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  hipLaunchKernelGGL(n2_probe_pool_kernel, grid, dim3(kPoolThreads), 0, s, cells, C, D, scores,
                     n->pool);
  return hipGetLastError();
}

// Whether this reset pools the confidence cells (a probe head and
// collectConfidence).
inline bool pool_on(const nd_needle* n) { return n->conf && n->collect; }

// The phi rows of layer ql in a mix launch's arguments, in the model's
// matrix form.
void set_phi(const nd_needle* n, uint32_t ql, MixArgs& m) {
  const uint32_t ln = n->d.lanes;
  const size_t K = (size_t)ln * n->d.dim;
  if (n->cq) {
    const nd_mat* pm[3] = {n->phi_pre, n->phi_post, n->phi_res};
    const size_t first[3] = {(size_t)ql * ln, (size_t)ql * ln, (size_t)ql * ln * ln};
    for (int i = 0; i < 3; ++i) {
      m.cq_p[i] = pm[i]->packed + first[i] * pm[i]->row_bytes;
      m.cq_n[i] = pm[i]->norms + first[i] * (pm[i]->kpad / pm[i]->g);
    }
    for (int i = 0; i < 3; ++i) {
      for (int c = 0; c < 16; ++c) m.cq_cb[i][c] = pm[i]->cb[c];
      m.cq_bits[i] = pm[i]->bits;
      m.cq_g[i] = pm[i]->g;
      m.cq_row_bytes[i] = pm[i]->row_bytes;
      m.cq_groups[i] = pm[i]->kpad / pm[i]->g;
      m.cq_inv_root[i] = 1.0 / std::sqrt((double)pm[i]->g);
    }
  } else {
    m.phi_w[0] = n->phi_pre->w + (size_t)ql * ln * K;
    m.phi_s[0] = n->phi_pre->scales + (size_t)ql * ln;
    m.phi_w[1] = n->phi_post->w + (size_t)ql * ln * K;
    m.phi_s[1] = n->phi_post->scales + (size_t)ql * ln;
    m.phi_w[2] = n->phi_res->w + (size_t)ql * ln * ln * K;
    m.phi_s[2] = n->phi_res->scales + (size_t)ql * ln * ln;
  }
}

// The fused launch's waits: the arrivals the mix waits for, the spin bound
// and the status word.
void set_waits(const nd_needle* n, MixArgs& m) {
  m.wo_target = m.wo_groups + n->dbg_extra;
  m.spin = n->dbg_spin ? n->dbg_spin : kWoSpin;
  m.status = n->status;
}

// Halves of a mix launch (enqueue_mix `parts`).
enum MixPart : uint32_t { kMixPost = 1, kMixPre = 2, kMixFinal = 4, kMixCell = 8 };

// Mix launch of layer slot l (l <= layers): post(l - 1) of the previous
// layer with kMixPost (runtime.ts:509-542 with #attentionDelta, :585-611),
// pre(l) of this one with kMixPre when l < layers (runtime.ts:385-441), the
// lane mean plus final norm with kMixFinal (runtime.ts:570-576), and with
// kMixCell (and kMixPost) the lane mean after post(l - 1) into confidence
// cell l when the pool is on.
QkvParams qkv_params(const nd_needle* n, uint32_t l);
bool wo_cq_fits(const nd_mat& w);
WoCq wo_cq_of(const nd_needle* n, const nd_mat& w);

// Whether layer attention can run inside the fused launch: an int8 cache
// whose ring fits the gated attention's one chunk, two query heads per KV
// head (attention_role's instance).
bool att_fusable(const nd_needle* n) {
  return n->kv.mode == ND_KV_INT8 && n->d.heads == 2 * n->d.kv_heads &&
         n->kv.alloc <= nd::att::kGatedChunk;
}

// Layer l's attention in the fused launch (attention_role), with the
// arguments nd_launch_attention_gated gives its kernel.
void set_att(nd_needle* n, uint32_t l, MixArgs& m) {
  m.att = AttArgs{n->kv.k, n->kv.v, n->kv.ks, n->kv.vs, n->q, n->att, n->qkvg, n->st + 1,
                  l, n->d.kv_heads, n->kv.alloc, n->kv.sink, n->kv.window};
  m.att_groups = n->d.kv_heads;
  // per KV head: its query and gate heads, its key and its value
  m.att_target = 2 * (n->d.heads / n->d.kv_heads) + 2;
  m.att_count = n->wo_count + kAttStride;
}

// wo: for an int8 model, layer l - 1's Wo (with the post half) and layer
// l's projection (with the pre half) run in the same launch
// (n2_mix_kernel<false, true>) instead of beside the attention; att (with
// qkv): layer l's attention too.
hipError_t enqueue_mix(nd_needle* n, uint32_t l, uint32_t parts, hipStream_t s, bool wo = false,
                       bool qkv = false, bool att = false) {
  const bool has_post = parts & kMixPost;
  const nd_needle_desc& d = n->d;
  const uint32_t D = d.dim, ln = d.lanes;
  const bool pre = l < d.layers;
  // Every operand pointer is valid whether or not its half runs (the kernel
  // loads them unconditionally): an absent layer reads layer 0's.
  const uint32_t pl = l > 0 ? l - 1 : 0, ql = pre ? l : 0;
  int site = -1;
  for (uint32_t si = 0; si < d.n_sites; ++si)
    if (pre && d.sites[si] == l) site = (int)si;
  MixArgs m{};
  m.x = n->x;
  m.d = D;
  m.hdim = d.hadamard;
  m.lanes = ln;
  m.upd = n->upd;
  m.blk = n->blk;
  m.ain = n->ain;
  m.phi_post = n->phi_post_v;
  m.phi_res = n->phi_res_v;
  m.has_post = has_post;
  m.proj = n->proj;
  m.post_norm = n->params + n->o_post + (size_t)pl * D;
  m.pre_h_norm = n->params + n->o_preh + (size_t)pl * D;
  m.d1 = n->params + n->o_d1 + (size_t)pl * D;
  m.d2 = n->params + n->o_d2 + (size_t)pl * d.hadamard;
  m.d3 = n->params + n->o_d3 + (size_t)pl * D;
  mix_constants(m, D, d.hadamard, ln, n->attention_gate[pl]);
  m.route = n->route;
  m.has_pre = pre && (parts & kMixPre);
  m.own_pre = ql % ln;
  set_phi(n, ql, m);
  m.a_pre = n->a_pre[ql];
  m.b_pre = n->params + n->o_bpre + (size_t)ql * ln;
  m.has_site = site >= 0;
  const uint32_t es = site >= 0 ? (uint32_t)site : 0;
  const uint32_t S = d.n_sites ? d.n_sites : 1;
  m.ekey = n->host_engrams ? n->host_eng + (size_t)es * D : n->ekv_out + (size_t)es * 2 * D;
  m.evalue = n->host_engrams ? n->host_eng + (size_t)(S + es) * D : n->evals + (size_t)es * D;
  m.norm_input = n->params + n->o_norm_input + (size_t)ql * D;
  m.has_final = (parts & kMixFinal) != 0;
  m.final_norm = n->params + n->o_final;
  m.fin = n->fin;
  m.cell = pool_on(n) && has_post && (parts & kMixCell) ? n->cells + (size_t)l * D : nullptr;
  if (wo && n->cq) {
    // One launch on one XCD: layer l - 1's Wo (with the post half), the mix,
    // layer l's projection (with the pre half, when qkv).
    const nd_mat* w = n->wo[pl];
    m.wo_cq = wo_cq_of(n, *w);
    m.wo_bits = w->bits;
    m.wo_groups = has_post ? w->n / 64 : 0;
    m.wo_count = n->wo_count;
    set_waits(n, m);
    if (qkv && m.has_pre) {
      m.qkv = qkv_params(n, l);
      m.qkv_groups = n->wqkvg[l].n / kHd + 1;
      m.qkv_flag = n->qkv_flags + 32 * (size_t)l;
      if (att) set_att(n, l, m);
    }
    const dim3 grid(8 * (m.wo_groups + 1 + m.qkv_groups + m.att_groups));
    if (n->dbg_stamps && n->phi_uniform && grid.x <= 8 * 64) {  // measurement form
      m.stamps = n->dbg_stamps + (size_t)l * 64 * 16;
      hipLaunchKernelGGL((n2_mix_kernel<true, true, true, true>), grid, dim3(kMixWg), 0, s, m);
    } else if (n->phi_uniform) {
      hipLaunchKernelGGL((n2_mix_kernel<true, true, true>), grid, dim3(kMixWg), 0, s, m);
    } else {
      hipLaunchKernelGGL((n2_mix_kernel<true, true, false>), grid, dim3(kMixWg), 0, s, m);
    }
  } else if (n->cq) {
    if (n->phi_uniform)
      hipLaunchKernelGGL((n2_mix_kernel<true, false, true>), dim3(1), dim3(kMixWg), 0, s, m);
    else
      hipLaunchKernelGGL((n2_mix_kernel<true, false, false>), dim3(1), dim3(kMixWg), 0, s, m);
  } else if (wo) {
    // One launch on one XCD: layer l - 1's Wo (with the post half), the mix,
    // layer l's projection (with the pre half, when qkv).
    const nd_mat* w = n->wo[pl];
    m.wo_w = w->w;
    m.wo_s = w->scales;
    m.wo_x = n->att;
    m.wo_n = w->n;
    m.wo_k = w->k;
    while ((1u << m.wo_tpr_log2) < w->k / 16) ++m.wo_tpr_log2;
    m.wo_groups =
        has_post ? (w->n + (kMixWg >> m.wo_tpr_log2) - 1) / (kMixWg >> m.wo_tpr_log2) : 0;
    m.wo_count = n->wo_count;
    set_waits(n, m);
    if (qkv && m.has_pre) {
      m.qkv = qkv_params(n, l);
      m.qkv_groups = n->wqkvg[l].n / kHd + 1;
      m.qkv_flag = n->qkv_flags + 32 * (size_t)l;
      if (att) set_att(n, l, m);
    }
    const dim3 grid(8 * (m.wo_groups + 1 + m.qkv_groups + m.att_groups));
    if (n->dbg_stamps && grid.x <= 8 * 64) {  // measurement: 64 workgroups' stamps per layer
      m.stamps = n->dbg_stamps + (size_t)l * 64 * 16;
      hipLaunchKernelGGL((n2_mix_kernel<false, true, true, true>), grid, dim3(kMixWg), 0, s, m);
    } else {
      hipLaunchKernelGGL((n2_mix_kernel<false, true>), grid, dim3(kMixWg), 0, s, m);
    }
  } else {
    hipLaunchKernelGGL(n2_mix_kernel<false>, dim3(1), dim3(kMixWg), 0, s, m);
  }
  return hipGetLastError();
}

// y = m x (rows [row_start, +row_count) into y[0, row_count)) for either
// matrix form: the int8 matvec, or the Cactus-Quant matvec with its input
// rotation inside the launch (groups <= 2048, checked at create).
hipError_t mv_any(const nd_mat* m, const float* x, uint32_t row_start, uint32_t row_count,
                  float* y, hipStream_t s) {
  if (m->bits)
    return nd_launch_cq_matvec(m, x, 1, m->k, nullptr, row_start, row_count, y, row_count, s);
  return nd_launch_matvec(m, x, 1, m->k, row_start, row_count, y, row_count, s);
}

// The attention block of layer l on the input n->ain: Q/K/V/gate matvec with
// the q/k norms, RoPE and the KV append in its epilogue (plus the layer's
// Sinkhorn routing from the mix's phi rows), gated attention, and Wo into
// n->proj (runtime.ts:465-505).
// The projection launch of layer l: its arguments (input n->ain, the
// routing from the phi values in n->phi_post_v / phi_res_v into n->route).
CqRows cq_rows_of(const nd_mat& wm) {
  CqRows cq{};
  cq.packed = wm.packed;
  cq.norms = wm.norms;
  for (int i = 0; i < 16; ++i) cq.cb[i] = wm.cb[i];
  cq.g = wm.g;
  while ((1u << cq.g_log2) < wm.g) ++cq.g_log2;
  cq.row_bytes = wm.row_bytes;
  cq.groups = wm.kpad / wm.g;
  cq.out_scale = (float)(1.0 / std::sqrt((double)wm.g));
  return cq;
}

// A Cactus-Quant Wo that wo_cq_rows takes (both launches of it use it).
bool wo_cq_fits(const nd_mat& w) { return w.bits && w.kpad <= 512 && w.n % 64 == 0; }

WoCq wo_cq_of(const nd_needle* n, const nd_mat& w) {
  WoCq c{};
  c.x = n->att;
  c.y = n->proj;
  c.n = w.n;
  c.k = w.k;
  c.cq = cq_rows_of(w);
  return c;
}

QkvParams qkv_params(const nd_needle* n, uint32_t l) {
  const nd_needle_desc& d = n->d;
  const uint32_t ln = d.lanes;
  const nd_mat& wm = n->wqkvg[l];
  QkvParams p{};
  p.W = wm.w;
  p.S = wm.scales;
  p.x = n->ain;
  p.d = d.dim;
  p.heads = d.heads;
  p.kv_heads = d.kv_heads;
  p.st = n->st;
  p.q_norm = n->params + n->o_qn + (size_t)l * kHd;
  p.k_norm = n->params + n->o_kn + (size_t)l * kHd;
  p.rope = n->rope;
  p.q_out = n->q;
  p.gate_out = n->qkvg;
  p.Kc = n->kv.k;
  p.Vc = n->kv.v;
  p.Ks = n->kv.ks;
  p.Vs = n->kv.vs;
  p.layer = l;
  p.alloc = n->kv.alloc;
  p.sink = n->kv.sink;
  p.window = n->kv.window;
  p.f32 = n->kv.mode == ND_KV_FLOAT32 ? 1u : 0u;
  RouteArgs& ra = p.route;
  ra.phi_post = n->phi_post_v;
  ra.phi_res = n->phi_res_v;
  ra.a_post = n->a_post[l];
  ra.a_res = n->a_res[l];
  ra.b_post = n->params + n->o_bpost + (size_t)l * ln;
  ra.b_res = n->params + n->o_bres + (size_t)l * ln * ln;
  ra.lanes = ln;
  ra.own = l % ln;
  ra.route = n->route;
  if (n->cq)
    for (int i = 0; i < 4; ++i) {
      p.cq[i] = cq_rows_of(n->qkv_part[l][i]);
      p.cq_bits[i] = n->qkv_part[l][i].bits;
    }
  return p;
}

// with_wo false: Wo is left to the next mix launch (int8 decode steps);
// with_qkv false: the projection runs inside the mix launch too.
hipError_t enqueue_block(nd_needle* n, uint32_t l, hipStream_t s, bool with_wo = true,
                         bool with_qkv = true) {
  const nd_needle_desc& d = n->d;
  const nd_mat& wm = n->wqkvg[l];
  if (with_qkv) {
    auto kern = n->cq ? &n2_qkv_kernel<true> : &n2_qkv_kernel<false>;
    hipLaunchKernelGGL(kern, dim3(wm.n / kHd + 1), dim3(kQkvWg), 0, s, qkv_params(n, l));
    const hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  const hipError_t e =
      nd_launch_attention_gated(&n->kv, l, n->st + 1, n->max_length - 1, n->q, d.heads, n->qkvg,
                                n->att, n->partials, n->counters, s);
  if (e != hipSuccess || !with_wo) return e;
  const nd_mat& w = *n->wo[l];
  if (n->cq && wo_cq_fits(w)) {  // the fused launch's arithmetic
    auto kern = w.bits == 4 ? &n2_wo_cq_kernel<4>
                            : (w.bits == 3 ? &n2_wo_cq_kernel<3> : &n2_wo_cq_kernel<2>);
    hipLaunchKernelGGL(kern, dim3(w.n / 64), dim3(kMixWg), 0, s, wo_cq_of(n, w));
    return hipGetLastError();
  }
  return mv_any(n->wo[l], n->att, 0, d.dim, n->proj, s);
}

// After the final mix: the confidence pool of the step's cells, the logits
// (tied embedding, runtime.ts:577) when tail, and selectToken over
// allowed[0..count) (all ids when allowed is null) when select.
hipError_t enqueue_final(nd_needle* n, bool tail, bool select, const uint32_t* allowed,
                         uint32_t count, hipStream_t s, const uint32_t* mask = nullptr) {
  const nd_needle_desc& d = n->d;
  hipError_t e;
  if (pool_on(n) && (e = enqueue_pool(n, n->cells, d.layers + 1, n->scores, s)) != hipSuccess)
    return e;
  if (!tail) return hipSuccess;
  e = mv_any(n->embedding, n->fin, 0, d.vocab, n->logits, s);
  if (e != hipSuccess || !select) return e;
  if (mask)  // the allowed set as a device bitmask (an empty one gives id 0xFFFFFFFF)
    return nd_launch_select_mask(n->logits, 1, d.vocab, mask, n->sel_id, n->sel_lp, s, nullptr,
                                 nullptr, nullptr);
  return nd_launch_select_list(n->logits, d.vocab, allowed, count, n->sel_id, n->sel_lp, s);
}

// Arguments of the token intake and engram gathers of one step (the token
// and its source are set by the caller).
BeginArgs begin_args(nd_needle* n) {
  const nd_needle_desc& d = n->d;
  BeginArgs b{};
  b.st = n->st;
  b.history = n->history;
  b.lp_history = n->lp_history;
  b.selected_id = n->sel_id;
  b.selected_lp = n->sel_lp;
  b.emb = n->embedding->w;
  b.emb_s = n->embedding->scales;
  b.d = d.dim;
  b.lanes = d.lanes;
  b.scale = std::sqrt((double)d.dim);
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
  b.inv_freq = n->inv_freq;
  b.rope = n->rope;
  b.cell0 = pool_on(n) ? n->cells : nullptr;
  b.cq_lookup = n->cq ? n->cq_lookup : nullptr;
  return b;
}

// The gathers of a Cactus-Quant model's step: the embedding row of *token
// (token null: none) and the engram table rows of `lookup`.
// batch: 0 for one step's rows (n->x, n->cells, n->cat), else the number of
// batched prefill positions (their rows into the prefill buffers).
hipError_t enqueue_cq_rows(nd_needle* n, const uint32_t* token, const uint32_t* lookup,
                           hipStream_t s, uint32_t batch = 0) {
  const nd_needle_desc& d = n->d;
  CqRowsArgs a{};
  auto source = [](const nd_mat* m) {
    CqSource c{};
    c.p = m->packed;
    c.n = m->norms;
    c.kpad = m->kpad;
    c.row_bytes = m->row_bytes;
    c.g = m->g;
    c.bits = m->bits;
    c.inverse_root = 1.0 / std::sqrt((double)m->g);
    for (int i = 0; i < 16; ++i) c.cb[i] = m->cb[i];
    if (m->bits == nd::kCqTernaryBits) {  // dequantizeCqRow's table: c = f32(1.2240064 * 1/sqrt(g))
      const float v = (float)(1.2240064 * c.inverse_root);
      c.cb[0] = 0.f;
      c.cb[1] = v;
      c.cb[2] = 0.f;
      c.cb[3] = -v;
    }
    return c;
  };
  a.emb = source(n->embedding);
  for (uint32_t si = 0; si < d.n_sites; ++si) a.tab[si] = source(n->eg_tables[si]);
  a.token = token;
  a.lookup = lookup;
  a.d = d.dim;
  a.lanes = d.lanes;
  a.scale = std::sqrt((double)d.dim);
  a.x = n->x;
  a.cell0 = pool_on(n) ? n->cells : nullptr;
  a.n_sites = d.n_sites;
  a.tables = d.engram_tables;
  a.slots = d.engram_slots;
  a.sub = d.engram_sub;
  a.cat = n->cat;
  if (batch) {  // the batched prefill's rows, positions in history order
    const uint32_t per_site = d.engram_tables * d.engram_sub;
    a.x = n->pf_x;
    a.cell0 = pool_on(n) ? n->pf_cells : nullptr;
    a.cat = n->pf_cat;
    a.lookup_ld = 2 * d.engram_tables + 1;
    a.x_ld = d.lanes * d.dim;
    a.cell_ld = (d.layers + 1) * d.dim;
    a.cat_ld = (d.n_sites ? d.n_sites : 1) * per_site;
  }
  hipLaunchKernelGGL(n2_cq_rows_kernel, dim3(1 + d.n_sites * d.engram_tables, batch ? batch : 1),
                     dim3(256), 0, s, a);
  return hipGetLastError();
}

// The engram projections of the gathered rows in n->cat (runtime.ts:837-843)
// and the ring update and tap convolution at position st[1] (:854-872):
// keys in n->ekv_out, mixed values in n->evals.
hipError_t enqueue_engrams(nd_needle* n, hipStream_t s) {
  const nd_needle_desc& d = n->d;
  const uint32_t D = d.dim, cat = d.engram_tables * d.engram_sub;
  for (uint32_t si = 0; si < d.n_sites; ++si) {
    const float* x = n->cat + (size_t)si * cat;
    float* y = n->ekv_out + (size_t)si * 2 * D;
    const nd_mat& kv = n->ekv[si];
    hipError_t e;
    if (!kv.bits || kv.packed) {
      e = mv_any(&kv, x, 0, 2 * D, y, s);
    } else {  // key and value of different formats
      e = mv_any(&n->ekv_part[si][0], x, 0, D, y, s);
      if (e == hipSuccess) e = mv_any(&n->ekv_part[si][1], x, 0, D, y + D, s);
    }
    if (e != hipSuccess) return e;
  }
  if (!d.n_sites) return hipSuccess;
  hipLaunchKernelGGL(n2_engram_conv_kernel, dim3(d.n_sites), dim3((D + 63) / 64 * 64), 0, s, n->st,
                     n->ekv_out, n->ring, n->params + n->o_taps, D, n->depth, d.engram_taps,
                     n->max_order, n->evals);
  return hipGetLastError();
}

// Enqueues one token of NeedleRuntime.step (model/runtime.ts:280-583) on s.
// select: after the logits, selectToken over allowed[0..count) (all ids when
// allowed is null) into sel_id / sel_lp.
hipError_t enqueue_step(nd_needle* n, uint32_t source, uint32_t token, bool want_logits,
                        bool select, const uint32_t* allowed, uint32_t count, hipStream_t s,
                        const uint32_t* mask = nullptr) {
  const nd_needle_desc& d = n->d;
  BeginArgs b = begin_args(n);
  b.token_arg = token;
  b.source = source;
  hipLaunchKernelGGL(n2_begin_kernel, dim3(1), dim3(kWg), 0, s, b);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  if (n->cq && (e = enqueue_cq_rows(n, n->cq_lookup + 2 * b.tables, n->cq_lookup, s)) !=
                   hipSuccess)
    return e;
  if ((e = enqueue_engrams(n, s)) != hipSuccess) return e;
  const bool tail = want_logits || select;
  // Launch l (l <= layers) runs post(l - 1) and pre(l); the last one runs
  // post(layers - 1) and the final norm, and only when logits are wanted or
  // the confidence pool takes the last layer's lane mean (otherwise the
  // lanes do not outlive the step).
  for (uint32_t l = 0; l <= d.layers; ++l) {
    const bool pre = l < d.layers;
    if (!pre && !tail && !pool_on(n)) break;
    const uint32_t parts = (l > 0 ? kMixPost | kMixCell : 0) | kMixPre | (!pre && tail ? kMixFinal : 0);
    // Layer l - 1's Wo and layer l's projection run inside mix launch l
    // (when no last mix runs, the last Wo has no reader).
    const uint32_t wo_tpr = n->d.heads * kHd / 16;  // int8 Wo threads a row
    // The fused launch keeps its workgroups on one XCD (workgroups L % 8 ==
    // 0 only): without the confirmed placement the launches stay separate.
    const bool fuse = nd_xcd_local() &&
                      (n->cq ? n->wo_fused
                             : (wo_tpr & (wo_tpr - 1)) == 0 && wo_tpr <= (uint32_t)kMixWg);
    // ... and layer l's attention too when its ring fits one chunk.
    const bool att = fuse && att_fusable(n);
    if ((e = enqueue_mix(n, l, parts, s, fuse, fuse, att)) != hipSuccess) return e;
    if (!pre) break;
    if (att) continue;
    if ((e = enqueue_block(n, l, s, !fuse, !fuse)) != hipSuccess) return e;
  }
  return enqueue_final(n, tail, select, allowed, count, s, mask);
}

enum GraphKind { kGraphPrompt = 0, kGraphPromptSelect = 1, kGraphDecodeSelect = 2 };

// Launches the step graph of `kind`, capturing and instantiating it first if
// the cached one was built for another cache geometry, KV mode or pooling.
nd_status launch_graph(nd_ctx* ctx, nd_needle* n, GraphKind kind) {
  const uint32_t mode = n->kv.mode | (pool_on(n) ? 2u : 0u) | (nd_xcd_local() ? 4u : 0u);
  if (n->graph_alloc != n->kv.alloc || n->graph_sink != n->kv.sink || n->graph_mode != mode) {
    drop_graphs(n);
    n->graph_alloc = n->kv.alloc;
    n->graph_sink = n->kv.sink;
    n->graph_mode = mode;
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
    size_t count = 0;
    hipError_t e3 = hipGraphGetNodes(g, nullptr, &count);
    std::vector<hipGraphNode_t> nodes(count);
    if (e3 == hipSuccess && count) e3 = hipGraphGetNodes(g, nodes.data(), &count);
    uint32_t kernels = 0;
    for (size_t i = 0; e3 == hipSuccess && i < count; ++i) {
      hipGraphNodeType type;
      e3 = hipGraphNodeGetType(nodes[i], &type);
      kernels += type == hipGraphNodeTypeKernel;
    }
    n->graph_kernels[kind] = kernels;
    if (e3 == hipSuccess) e3 = hipGraphInstantiate(&n->graphs[kind], g, nullptr, nullptr, 0);
    hipGraphDestroy(g);
    if (e3 != hipSuccess) {
      n->graphs[kind] = nullptr;
      return nd_hip_fail(ctx, e3, "Needle step graph");
    }
  }
  ND_HIP(ctx, hipGraphLaunch(n->graphs[kind], s));
  return ND_OK;
}

// Buffers of the batched prefill, for up to pf_cap positions per pass.
nd_status ensure_prefill(nd_ctx* ctx, nd_needle* n) {
  if (n->pf_arena) return ND_OK;
  const nd_needle_desc& d = n->d;
  const uint32_t cap = std::min<uint32_t>(d.max_length, kPrefillRows);
  const uint32_t D = d.dim, ln = d.lanes, qw = d.heads * kHd, kw = d.kv_heads * kHd;
  const uint32_t S = d.n_sites ? d.n_sites : 1, cat = d.n_sites ? d.engram_tables * d.engram_sub : 1;
  const uint32_t kmax = std::max(std::max(D, qw), cat);
  const size_t pf = nd_attention_batch_partial_floats(cap, d.kv_heads, d.heads / d.kv_heads,
                                                      d.max_length);
  const size_t sizes[] = {al((size_t)cap * ln * D * 4), al((size_t)cap * D * 4),
                          al((size_t)cap * D * 4),      al((size_t)cap * D * 4),
                          al((size_t)cap * ln * 4),     al((size_t)cap * ln * ln * 4),
                          al((size_t)cap * 20 * 4),     al((size_t)cap * (2 * qw + 2 * kw) * 4),
                          al((size_t)cap * qw * 4),     al((size_t)cap * qw * 4),
                          al((size_t)cap * D * 4),      al((size_t)cap * S * cat * 4),
                          al((size_t)cap * S * 2 * D * 4), al((size_t)cap * S * D * 4),
                          al((size_t)cap * 4),          al(pf * 4),
                          al((size_t)3 * cap * kmax),   al((size_t)cap * 4),
                          al((size_t)cap * d.kv_heads * kAttnCounterStride * 4),
                          n->conf ? al((size_t)cap * (d.layers + 1) * D * 4) : 0,
                          n->conf ? al((size_t)cap * (d.layers + 1) * kMaxProbes * 8) : 0,
                          n->cq ? al((size_t)cap * (2 * d.engram_tables + 1) * 4) : 0};
  size_t total = 0;
  for (size_t v : sizes) total += v;
  hipError_t e = hipMalloc(&n->pf_arena, total);
  if (e == hipSuccess) e = hipMemsetAsync(n->pf_arena, 0, total, ctx->stream);
  if (e == hipSuccess) e = hipStreamSynchronize(ctx->stream);
  if (e != hipSuccess) {
    if (n->pf_arena) hipFree(n->pf_arena);
    n->pf_arena = nullptr;
    return nd_hip_fail(ctx, e, "Needle prefill allocation");
  }
  char* p = n->pf_arena;
  size_t i = 0;
  auto take = [&](auto** dst) {
    *dst = reinterpret_cast<std::remove_reference_t<decltype(**dst)>*>(p);
    p += sizes[i++];
  };
  take(&n->pf_x);
  take(&n->pf_upd);
  take(&n->pf_blk);
  take(&n->pf_ain);
  take(&n->pf_phi_post);
  take(&n->pf_phi_res);
  take(&n->pf_route);
  take(&n->pf_qkvg);
  take(&n->pf_q);
  take(&n->pf_att);
  take(&n->pf_proj);
  take(&n->pf_cat);
  take(&n->pf_ekv);
  take(&n->pf_evals);
  take(&n->pf_fm);
  take(&n->pf_partials);
  take(&n->pf_digits);
  take(&n->pf_positions);
  take(&n->pf_counters);
  take(&n->pf_cells);
  take(&n->pf_scores);
  take(&n->pf_cq_lookup);
  n->pf_cap = cap;
  return ND_OK;
}

// Enqueues `count` prompt tokens (already in history at [position, position
// + count)) as one batched pass; the host checks that the slots do not wrap
// and that count <= pf_cap.  want_logits / select: the last position's
// logits (and selection over all ids) as a step would produce them.
hipError_t enqueue_prefill(nd_needle* n, uint32_t count, bool want_logits, bool select,
                           hipStream_t s) {
  const nd_needle_desc& d = n->d;
  const uint32_t D = d.dim, ln = d.lanes, qw = d.heads * kHd, kw = d.kv_heads * kHd;
  const uint32_t M = count, p0 = n->position, N = ln * D;
  const uint32_t S = d.n_sites ? d.n_sites : 1, cat = d.engram_tables * d.engram_sub;
  const uint32_t qkv_ld = 2 * qw + 2 * kw;
  BeginArgs b{};
  b.st = n->st;
  b.history = n->history;
  b.emb = n->embedding->w;
  b.emb_s = n->embedding->scales;
  b.d = D;
  b.lanes = ln;
  b.scale = std::sqrt((double)D);
  b.x = n->pf_x;
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
  b.cat = n->pf_cat;
  const uint32_t cell_ld = (d.layers + 1) * D;  // cells of one position: [layers + 1][d]
  b.cell0 = pool_on(n) ? n->pf_cells : nullptr;
  b.cell_ld = cell_ld;
  b.cq_lookup = n->cq ? n->pf_cq_lookup : nullptr;
  hipLaunchKernelGGL(n2_begin_batch_kernel, dim3(M), dim3(kWg), 0, s, b, p0, M, n->pf_positions);
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return e;
  const uint32_t lk = 2 * d.engram_tables + 1;
  if (n->cq && (e = enqueue_cq_rows(n, n->pf_cq_lookup + lk - 1, n->pf_cq_lookup, s, M)) !=
                   hipSuccess)
    return e;
  // The batch's products: digit-sliced int8 GEMMs, or for a Cactus-Quant
  // model the CQ matvec over the M rows (the step's arithmetic per row).
  auto product = [&](const nd_mat* w, const float* x, uint32_t x_ld, uint32_t k, float* y,
                     uint32_t y_ld) -> hipError_t {
    if (w->bits)
      return nd_launch_cq_matvec(w, x, M, x_ld, nullptr, 0, w->n, y, y_ld, s);
    hipError_t r = nd_launch_digitize(x, x_ld, nullptr, nullptr, n->pf_digits, n->pf_fm, M, k, s);
    if (r != hipSuccess) return r;
    return nd_launch_gemm(w, n->pf_digits, n->pf_fm, y, y_ld, M, 0, s);
  };
  // Rows of parts concatenated when they share a format, else part by part
  // into their columns of y.
  auto parts_product = [&](const nd_mat& whole, const nd_mat* parts, size_t count,
                           const float* x, uint32_t x_ld, uint32_t k, float* y,
                           uint32_t y_ld) -> hipError_t {
    if (!whole.bits || whole.packed) return product(&whole, x, x_ld, k, y, y_ld);
    uint32_t col = 0;
    for (size_t i = 0; i < count; ++i) {
      const hipError_t r = product(&parts[i], x, x_ld, k, y + col, y_ld);
      if (r != hipSuccess) return r;
      col += parts[i].n;
    }
    return hipSuccess;
  };
  if (d.n_sites) {
    for (uint32_t si = 0; si < d.n_sites; ++si)
      if ((e = parts_product(n->ekv[si], n->cq ? n->ekv_part[si].data() : nullptr, 2,
                             n->pf_cat + (size_t)si * cat, S * cat, cat,
                             n->pf_ekv + (size_t)si * 2 * D, S * 2 * D)) != hipSuccess)
        return e;
    const uint32_t threads = (D + 63) / 64 * 64;
    hipLaunchKernelGGL(n2_conv_batch_kernel, dim3(M, d.n_sites), dim3(threads), 0, s, n->pf_ekv,
                       n->ring, n->params + n->o_taps, D, n->depth, d.engram_taps, n->max_order,
                       d.n_sites, p0, n->pf_evals);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    hipLaunchKernelGGL(n2_ring_store_kernel, dim3(std::min(M, n->depth), d.n_sites), dim3(threads),
                       0, s, n->pf_ekv, n->ring, D, n->depth, d.n_sites, p0, M);
    if ((e = hipGetLastError()) != hipSuccess) return e;
  }
  const bool tail = want_logits || select;
  for (uint32_t l = 0; l <= d.layers; ++l) {
    const bool pre = l < d.layers;
    if (!pre && !tail && !pool_on(n)) break;
    const uint32_t pl = l > 0 ? l - 1 : 0, ql = pre ? l : 0;
    // The final part runs the last row only, unless the confidence pool
    // needs every row's last lane mean.
    const uint32_t rows = pre || pool_on(n) ? M : 1, r0 = pre || pool_on(n) ? 0 : M - 1;
    int site = -1;
    for (uint32_t si = 0; si < d.n_sites; ++si)
      if (pre && d.sites[si] == l) site = (int)si;
    MixArgs m{};
    m.x = n->pf_x + (size_t)r0 * N;
    m.d = D;
    m.hdim = d.hadamard;
    m.lanes = ln;
    m.upd = n->pf_upd + (size_t)r0 * D;
    m.blk = n->pf_blk + (size_t)r0 * D;
    m.ain = n->pf_ain + (size_t)r0 * D;
    m.phi_post = n->pf_phi_post + (size_t)r0 * ln;
    m.phi_res = n->pf_phi_res + (size_t)r0 * ln * ln;
    m.has_post = l > 0;
    m.proj = n->pf_proj + (size_t)r0 * D;
    m.post_norm = n->params + n->o_post + (size_t)pl * D;
    m.pre_h_norm = n->params + n->o_preh + (size_t)pl * D;
    m.d1 = n->params + n->o_d1 + (size_t)pl * D;
    m.d2 = n->params + n->o_d2 + (size_t)pl * d.hadamard;
    m.d3 = n->params + n->o_d3 + (size_t)pl * D;
    mix_constants(m, D, d.hadamard, ln, n->attention_gate[pl]);
    m.route = n->pf_route + (size_t)r0 * 20;
    m.has_pre = pre;
    m.own_pre = ql % ln;
    set_phi(n, ql, m);
    m.a_pre = n->a_pre[ql];
    m.b_pre = n->params + n->o_bpre + (size_t)ql * ln;
    m.has_site = site >= 0;
    m.ekey = n->pf_ekv + (size_t)(site >= 0 ? site : 0) * 2 * D;
    m.evalue = n->pf_evals + (size_t)(site >= 0 ? site : 0) * D;
    m.ek_ld = S * 2 * D;
    m.ev_ld = S * D;
    m.norm_input = n->params + n->o_norm_input + (size_t)ql * D;
    m.has_final = !pre && tail;
    m.final_row = rows - 1;
    m.final_norm = n->params + n->o_final;
    m.fin = n->fin;
    m.cell = pool_on(n) && l > 0 ? n->pf_cells + (size_t)l * D : nullptr;
    m.cell_ld = cell_ld;
    if (pre) {
      m.route_out = n->pf_route;
      m.r_a_post = n->a_post[l];
      m.r_a_res = n->a_res[l];
      m.r_b_post = n->params + n->o_bpost + (size_t)l * ln;
      m.r_b_res = n->params + n->o_bres + (size_t)l * ln * ln;
    }
    auto mix = !n->cq ? &n2_mix_kernel<false>
               : n->phi_uniform ? &n2_mix_kernel<true, false, true>
                                : &n2_mix_kernel<true, false, false>;
    hipLaunchKernelGGL(mix, dim3(rows), dim3(kMixWg), 0, s, m);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    if (!pre) break;
    if ((e = parts_product(n->wqkvg[l], n->cq ? n->qkv_part[l].data() : nullptr, 4, n->pf_ain, D,
                           D, n->pf_qkvg, qkv_ld)) != hipSuccess)
      return e;
    hipLaunchKernelGGL(n2_rope_store_batch_kernel, dim3(d.heads + 2 * d.kv_heads, M), dim3(64), 0,
                       s, n->pf_qkvg, qkv_ld, d.heads, d.kv_heads,
                       n->params + n->o_qn + (size_t)l * kHd, n->params + n->o_kn + (size_t)l * kHd,
                       n->inv_freq, p0, n->pf_q, n->kv.k, n->kv.v, n->kv.ks, n->kv.vs, l,
                       n->kv.alloc, n->kv.sink, n->kv.window,
                       n->kv.mode == ND_KV_FLOAT32 ? 1u : 0u);
    if ((e = hipGetLastError()) != hipSuccess) return e;
    e = nd_launch_attention_batch(&n->kv, l, n->pf_positions, M, d.kv_heads, 0u,
                                  d.heads / d.kv_heads, p0 + M - 1, n->pf_q, n->pf_att,
                                  n->pf_partials, n->pf_counters, s, n->pf_qkvg + qw + 2 * kw,
                                  qkv_ld);
    if (e != hipSuccess) return e;
    if ((e = product(n->wo[l], n->pf_att, qw, qw, n->pf_proj, D)) != hipSuccess) return e;
  }
  if (pool_on(n) && (e = enqueue_pool(n, n->pf_cells, M * (d.layers + 1), n->pf_scores, s)) !=
                     hipSuccess)
    return e;
  if (!tail) return hipSuccess;
  e = mv_any(n->embedding, n->fin, 0, d.vocab, n->logits, s);
  if (e != hipSuccess || !select) return e;
  return nd_launch_select_list(n->logits, d.vocab, nullptr, 0, n->sel_id, n->sel_lp, s);
}

// Runs the prompt tokens already in history at [position, position + count):
// batched passes while the cache slots do not wrap, steps after that.  The
// last token produces logits (and a selection over all ids when select).
nd_status run_prompt(nd_ctx* ctx, nd_needle* n, uint32_t count, bool want_logits, bool select,
                     bool graphs) {
  nd_status st = ensure_prefill(ctx, n);
  if (st != ND_OK) return st;
  hipStream_t s = ctx->stream;
  uint32_t done = 0;
  while (done < count) {
    const uint32_t left = count - done;
    const uint32_t room = n->kv.alloc > n->position ? n->kv.alloc - n->position : 0;
    const uint32_t chunk = std::min(std::min(left, n->pf_cap), room);
    const bool last_pass = chunk == left;
    if (chunk > 0) {
      ND_HIP(ctx, enqueue_prefill(n, chunk, last_pass && want_logits, last_pass && select, s));
      n->position += chunk;
      done += chunk;
      continue;
    }
    // Slots wrap from here on: one step per token.
    const bool last = left == 1;
    if (graphs) {
      if ((st = launch_graph(ctx, n, last && (want_logits || select) ? kGraphPromptSelect
                                                                     : kGraphPrompt)) != ND_OK)
        return st;
    } else {
      ND_HIP(ctx, enqueue_step(n, kTokenHistory, 0, last && want_logits, last && select, nullptr, 0,
                               s));
    }
    ++n->position;
    ++done;
  }
  return ND_OK;
}

// The fused launches' status word: its copy to the pinned host word is
// enqueued before a whole-step call synchronizes, and read after.
hipError_t enqueue_status(nd_needle* n, hipStream_t s) {
  return hipMemcpyAsync(n->status_host, n->status, 4, hipMemcpyDeviceToHost, s);
}

nd_status check_waits(nd_ctx* ctx, const nd_needle* n) {
  const uint32_t v = *n->status_host;
  if (!v) return ND_OK;
  return nd_fail(ctx, ND_ERR_BACKEND,
                 "a bounded wait inside a fused layer launch ran out (%s%s%s%s%s): the results "
                 "of this call are not valid, and every whole-step call fails until reset()",
                 v & kStatusWoWait ? "the layer mix waiting for the output projection rows" : "",
                 (v & kStatusWoWait) && (v & (kStatusQkvWait | kStatusAttWait)) ? "; " : "",
                 v & kStatusQkvWait ? "the projection waiting for the layer mix" : "",
                 (v & kStatusQkvWait) && (v & kStatusAttWait) ? "; " : "",
                 v & kStatusAttWait ? "the attention waiting for the projection" : "");
}

// One reset is driven either by whole-step calls or by the session methods:
// they keep different parts of the runtime state on the device (the token
// history for the engram hashes, or the host's lookups), so mixing them
// would read stale state.
nd_status use_api(nd_ctx* ctx, nd_needle* n, uint32_t api) {
  static const char* const names[] = {"", "whole-step", "session"};
  if (n->api && n->api != api)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "this runtime is driven by %s calls since its reset; call reset() before "
                   "switching to %s calls",
                   names[n->api], names[api]);
  n->api = api;
  return ND_OK;
}

// Copies `bytes` of host memory to dst on s through pinned staging slot k
// (waiting first for that slot's previous copy), so that the caller's buffer
// is free again when this returns and the copy stays asynchronous.
hipError_t stage_copy(nd_needle* n, StageSlot k, void* dst, const void* src, size_t bytes,
                      size_t slot_offset, hipStream_t s) {
  if (slot_offset + bytes > n->stage_bytes[k]) return hipErrorInvalidValue;
  hipError_t e = hipEventSynchronize(n->stage_done[k]);
  if (e != hipSuccess) return e;
  char* slot = n->pinned + n->stage_off[k] + slot_offset;
  std::memcpy(slot, src, bytes);
  if ((e = hipMemcpyAsync(dst, slot, bytes, hipMemcpyHostToDevice, s)) != hipSuccess) return e;
  return hipEventRecord(n->stage_done[k], s);
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
      (d->dim & (d->dim - 1)) || d->hadamard > 512 || d->hadamard < d->dim ||
      (d->hadamard & (d->hadamard - 1)) || d->heads == 0 || d->kv_heads == 0 ||
      d->heads % d->kv_heads || d->heads * kHd > 8192 || d->layers == 0 || d->vocab == 0 ||
      d->max_length == 0 || d->n_sites > 4 || d->n_orders > 4 ||
      (d->n_sites && d->n_orders == 0) || d->engram_tables > 16 ||
      (d->n_orders && d->engram_tables % d->n_orders) ||
      (d->n_sites && (d->engram_taps == 0 || d->engram_slots == 0 || d->engram_sub == 0)))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "Needle geometry outside this kernel set: head_dim 64, lanes <= 4, dim a "
                   "power of two in [128, 512], power-of-two hadamard in [dim, 512], heads a "
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
  // Every matrix in one form: per-row-scaled int8, or (the shipped archive,
  // model/cact.ts:398-562) Cactus-Quant, each matrix with its own width and
  // group as the archive's records carry them (a mixed-bit archive,
  // cact.ts:346-361), groups of at most 2048 (rotated inside the matvec).
  // Rows padded to a multiple of the group must fit the kernel that
  // consumes them: max_kpad codes (q, k, v, gate: 512, one row on 16 lanes
  // of 32 codes; embedding and engram tables: kCqRowMax, a row in LDS; the
  // phi matrices: exactly lanes x dim, the mix's units).
  const bool cq = d->embedding && d->embedding->bits != 0;
  auto check = [&](const nd_mat* m, uint32_t n, uint32_t k, const char* what,
                   uint32_t max_kpad = kCqMaxKpad) -> nd_status {
    if (cq) {
      if (!m || !m->bits || m->n != n || m->k != k || m->g > 2048)
        return nd_fail(ctx, ND_ERR_INVALID,
                       "%s must be a %ux%u Cactus-Quant matrix (group <= 2048)", what, n, k);
      if (m->kpad > max_kpad)
        return nd_fail(ctx, ND_ERR_UNSUPPORTED,
                       "%s rows padded to %u codes (group %u); this runtime takes at most %u", what,
                       m->kpad, m->g, max_kpad);
      return ND_OK;
    }
    if (!m || m->bits || m->n != n || m->k != k || m->g != k)
      return nd_fail(ctx, ND_ERR_INVALID, "%s must be a per-row-scaled %ux%u int8 matrix", what,
                     n, k);
    return ND_OK;
  };
  nd_status st;
  if ((st = check(d->embedding, d->vocab, D, "embedding", kCqRowMax)) ||
      (st = check(d->phi_pre, L * ln, ln * D, "phi_pre", ln * D)) ||
      (st = check(d->phi_post, L * ln, ln * D, "phi_post", ln * D)) ||
      (st = check(d->phi_res, L * ln * ln, ln * D, "phi_res", ln * D)))
    return st;
  if (!d->wq || !d->wk || !d->wv || !d->wgate || !d->wo)
    return nd_fail(ctx, ND_ERR_INVALID, "layer matrix arrays must not be NULL");
  if (d->probes && (d->probe_count == 0 || d->probe_count > kMaxProbes || d->probe_out == 0 ||
                    !d->probe_projection || !d->probe_bias))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "confidence head needs 1..%u probes, at least one output, a projection and a "
                   "bias", kMaxProbes);
  for (uint32_t l = 0; l < L; ++l)
    if ((st = check(d->wq[l], qw, D, "wq", 512)) || (st = check(d->wk[l], kw, D, "wk", 512)) ||
        (st = check(d->wv[l], kw, D, "wv", 512)) || (st = check(d->wgate[l], qw, D, "wgate", 512)) ||
        (st = check(d->wo[l], D, qw, "wo")))
      return st;
  if (d->n_sites && (!d->eg_tables || !d->eg_key || !d->eg_value || !d->eg_taps))
    return nd_fail(ctx, ND_ERR_INVALID, "engram arrays must not be NULL");
  for (uint32_t s = 0; s < d->n_sites; ++s)
    if ((st = check(d->eg_tables[s], d->engram_tables * d->engram_slots, d->engram_sub,
                    "engram tables", kCqRowMax)) ||
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
  n->cq = cq;
  n->embedding = d->embedding;
  n->phi_pre = d->phi_pre;
  n->phi_post = d->phi_post;
  n->phi_res = d->phi_res;
  hipError_t e = hipSuccess;
  auto concat = [&](nd_mat& m, const nd_mat* const* parts, size_t count) {
    m.n = 0;
    for (size_t i = 0; i < count; ++i) m.n += parts[i]->n;
    m.k = parts[0]->k;
    if (cq) {  // rows of packed codes and of norms, one after the other
      const nd_mat* p0 = parts[0];
      m.g = p0->g;
      m.bits = p0->bits;
      m.kpad = p0->kpad;
      m.row_bytes = p0->row_bytes;
      for (int i = 0; i < 16; ++i) m.cb[i] = p0->cb[i];
      const size_t nb = (size_t)(m.kpad / m.g) * 2;  // norm bytes per row
      if (e == hipSuccess) e = hipMalloc(&m.packed, (size_t)m.n * m.row_bytes);
      if (e == hipSuccess) e = hipMalloc(&m.norms, (size_t)m.n * nb);
      size_t row = 0;
      for (size_t i = 0; i < count; ++i) {
        const nd_mat* p = parts[i];
        if (e == hipSuccess)
          e = hipMemcpyAsync(m.packed + row * m.row_bytes, p->packed, (size_t)p->n * m.row_bytes,
                             hipMemcpyDeviceToDevice, ctx->stream);
        if (e == hipSuccess)
          e = hipMemcpyAsync(reinterpret_cast<char*>(m.norms) + row * nb, p->norms,
                             (size_t)p->n * nb, hipMemcpyDeviceToDevice, ctx->stream);
        row += p->n;
      }
      return;
    }
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
  // Parts of one format are concatenated; a Cactus-Quant model also keeps
  // every part as a matrix of its own (a view into the concatenation, or an
  // owned copy when the parts' formats differ).
  auto same_form = [](const nd_mat* a, const nd_mat* b) {
    return a->bits == b->bits && a->g == b->g && a->kpad == b->kpad &&
           a->row_bytes == b->row_bytes && std::memcmp(a->cb, b->cb, sizeof a->cb) == 0;
  };
  auto split = [&](nd_mat& whole, const nd_mat* const* parts, size_t count, nd_mat* out) {
    bool uniform = true;
    for (size_t i = 1; i < count; ++i) uniform = uniform && same_form(parts[0], parts[i]);
    if (!cq || uniform) {
      concat(whole, parts, count);
      if (!cq) return;
      size_t row = 0;
      for (size_t i = 0; i < count; ++i) {
        nd_mat v = whole;
        v.n = parts[i]->n;
        v.packed = whole.packed ? whole.packed + row * whole.row_bytes : nullptr;
        v.norms = whole.norms ? whole.norms + row * (whole.kpad / whole.g) : nullptr;
        out[i] = v;
        row += parts[i]->n;
      }
      return;
    }
    whole.n = 0;
    whole.k = parts[0]->k;
    whole.bits = parts[0]->bits;  // Cactus-Quant, no concatenation (packed stays null)
    for (size_t i = 0; i < count; ++i) {
      whole.n += parts[i]->n;
      nd_mat c;
      concat(c, &parts[i], 1);
      n->owned_parts.push_back(c);
      out[i] = c;
    }
  };
  n->phi_uniform = !cq || (same_form(d->phi_pre, d->phi_post) && same_form(d->phi_pre, d->phi_res));
  n->wqkvg.resize(L);
  n->qkv_part.resize(L);
  for (uint32_t l = 0; l < L; ++l) {
    const nd_mat* parts[4] = {d->wq[l], d->wk[l], d->wv[l], d->wgate[l]};
    split(n->wqkvg[l], parts, 4, n->qkv_part[l].data());
    n->wo.push_back(d->wo[l]);
    n->wo_fused = n->wo_fused && (!cq || wo_cq_fits(*d->wo[l]));
  }
  n->ekv.resize(d->n_sites);
  n->ekv_part.resize(d->n_sites);
  for (uint32_t s = 0; s < d->n_sites; ++s) {
    const nd_mat* parts[2] = {d->eg_key[s], d->eg_value[s]};
    split(n->ekv[s], parts, 2, n->ekv_part[s].data());
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
  if (d->probes) {
    n->conf = true;
    n->probe_count = d->probe_count;
    n->o_probes = put(d->probes, (size_t)d->probe_count * D);
    n->o_pproj = put(d->probe_projection, (size_t)d->probe_count * D);  // row 0
    n->probe_bias0 = d->probe_bias[0];
  }
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
  if (n->pf_arena) hipFree(n->pf_arena);
  for (auto* v : {&n->wqkvg, &n->ekv, &n->owned_parts})
    for (auto& m : *v) {
      if (m.w) hipFree(m.w);
      if (m.scales) hipFree(m.scales);
      if (m.packed) hipFree(m.packed);
      if (m.norms) hipFree(m.norms);
    }
  if (n->params) hipFree(n->params);
  if (n->inv_freq) hipFree(n->inv_freq);
  if (n->pinned) hipHostFree(n->pinned);
  if (n->status_host) hipHostFree(n->status_host);
  for (auto& ev : n->stage_done)
    if (ev) hipEventDestroy(ev);
  delete n;
  return ND_OK;
}

nd_status nd_needle_reset(nd_ctx* ctx, nd_needle* n, uint32_t max_length, uint32_t sink,
                          uint32_t kv_cache, uint32_t collect_confidence) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "model is NULL");
  const nd_needle_desc& d = n->d;
  if (kv_cache != ND_KV_INT8 && kv_cache != ND_KV_FLOAT32)
    return nd_fail(ctx, ND_ERR_INVALID, "unknown kvCache mode %u", kv_cache);
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
    const size_t P8 = kMaxProbes * 8, cb = n->conf ? 1 : 0;
    const size_t sizes[] = {al(64), al((size_t)cap * 4), al((size_t)cap * 8),
                            al((size_t)S * n->depth * D * 4),
                            al((size_t)d.kv_heads * kAttnCounterStride * 4),
                            al((size_t)(1 + d.kv_heads) * kAttStride * 4),
                            al((size_t)d.layers * 128), al(128),
                            cb * al(P8 * kMaxChunks), cb * al(P8 * kMaxChunks),
                            cb * al(P8 * D), al(64), al(64),
                            // K and V sized for float32 rows (kvCache "float32")
                            al((size_t)d.vocab * 4), al((size_t)(d.vocab + 31) / 32 * 4), al(rows * kHd * 4), al(rows * kHd * 4),
                            al(rows * 4),
                            al(rows * 4), al((size_t)ln * D * 4), al(D * 4), al(D * 4), al(D * 4),
                            al((size_t)(2 * qw + 2 * kw) * 4), al(qw * 4), al(qw * 4), al(D * 4),
                            al(ln * 4), al(ln * ln * 4), al(D * 4), al((size_t)d.vocab * 4),
                            al((size_t)S * cat * 4), al((size_t)S * 2 * D * 4),
                            al((size_t)S * D * 4), al(pf * 4), al(20 * 4), al(64 * 8),
                            cb * al((size_t)(d.layers + 1) * D * 4),
                            cb * al((size_t)(d.layers + 1) * P8), cb * al(64), al(32 * 4),
                            al((size_t)2 * S * D * 4),
                            al((size_t)(3 * D + ln * D + ln + ln * ln) * 4),
                            al((2 * 16 + 1) * 4)};
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
    take(&n->counters);
    take(&n->wo_count);
    take(&n->qkv_flags);
    take(&n->status);
    take(&n->pool.max);
    take(&n->pool.den);
    take(&n->pool.weighted);
    n->state_bytes = (size_t)(p - n->arena);
    take(&n->sel_id);
    take(&n->sel_lp);
    take(&n->allowed);
    take(&n->mask);
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
    take(&n->route);
    take(&n->rope);
    take(&n->cells);
    take(&n->scores);
    take(&n->conf_out);
    take(&n->lookup);
    take(&n->host_eng);
    take(&n->fwd_in);
    take(&n->cq_lookup);
  }
  if (!n->pinned) {
    // Pinned staging of the session calls' host inputs.
    const uint32_t S = d.n_sites ? d.n_sites : 1;
    (void)S;
    size_t slot_bytes[kStageSlots] = {al((size_t)ln * D * 4), al(32 * 4),
                                      al((size_t)d.vocab * 4),
                                      al((size_t)(3 * D + ln * D + ln + ln * ln) * 4)};
    for (uint32_t k = kStageEngram; k < kStageSlots; ++k) slot_bytes[k] = al((size_t)D * 4);
    size_t pinned = 0;
    for (uint32_t k = 0; k < kStageSlots; ++k) {
      n->stage_off[k] = pinned;
      n->stage_bytes[k] = slot_bytes[k];
      pinned += slot_bytes[k];
    }
    for (auto& ev : n->stage_done)
      if (!ev) ND_HIP(ctx, hipEventCreateWithFlags(&ev, hipEventDisableTiming));
    ND_HIP(ctx, hipHostMalloc(reinterpret_cast<void**>(&n->pinned), pinned));
  }
  if (!n->status_host) ND_HIP(ctx, hipHostMalloc(reinterpret_cast<void**>(&n->status_host), 64));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  ND_HIP(ctx, hipMemsetAsync(n->arena, 0, n->state_bytes, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  n->max_length = max_length;
  n->sink = std::min(sink, max_length);
  n->position = 0;
  n->collect = collect_confidence != 0;
  n->api = 0;
  n->token_open = n->post_pending = n->engrams_ready = n->select_ready = false;
  n->next_layer = n->token_position = 0;
  nd_kv& kv = n->kv;
  kv.layers = d.layers;
  kv.kv_heads = d.kv_heads;
  kv.head_dim = kHd;
  kv.max_length = max_length;
  kv.sink = n->sink;
  kv.window = d.kv_window;
  kv.alloc = d.kv_window > 0 ? std::min(max_length, n->sink + d.kv_window) : max_length;
  kv.mode = kv_cache;
  return ND_OK;
}

nd_kv* nd_needle_kv(nd_needle* n) { return n && n->arena && n->max_length ? &n->kv : nullptr; }

uint32_t nd_needle_position(const nd_needle* n) { return n ? n->position : 0; }

nd_status nd_needle_confidence(nd_ctx* ctx, nd_needle* n, double* confidence) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || !confidence) return nd_fail(ctx, ND_ERR_INVALID, "nd_needle_confidence: NULL argument");
  if (!n->conf) return nd_fail(ctx, ND_ERR_INVALID, "the model has no confidence head");
  if (!n->arena || !n->max_length)
    return nd_fail(ctx, ND_ERR_INVALID, "runtime is not reset");
  if (!n->collect)
    return nd_fail(ctx, ND_ERR_INVALID, "this reset has collectConfidence off");
  hipLaunchKernelGGL(n2_probe_head_kernel, dim3(1), dim3(256), 0, ctx->stream, n->pool,
                     n->probe_count, n->d.dim, n->params + n->o_pproj, n->probe_bias0, n->conf_out);
  ND_HIP(ctx, hipGetLastError());
  ND_HIP(ctx, hipMemcpyAsync(confidence, n->conf_out, 8, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return ND_OK;
}

nd_status nd_needle_step(nd_ctx* ctx, nd_needle* n, uint32_t token, float* logits) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "model is NULL");
  nd_status st = check_step(ctx, n, token);
  if (st != ND_OK || (st = use_api(ctx, n, 1)) != ND_OK) return st;
  ND_HIP(ctx, enqueue_step(n, kTokenArg, token, logits != nullptr, false, nullptr, 0, ctx->stream));
  ++n->position;
  if (logits)
    ND_HIP(ctx, hipMemcpyAsync(logits, n->logits, (size_t)n->d.vocab * 4, hipMemcpyDeviceToHost,
                               ctx->stream));
  ND_HIP(ctx, enqueue_status(n, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return check_waits(ctx, n);
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
  nd_status st = use_api(ctx, n, 1);
  if (st != ND_OK) return st;
  ND_HIP(ctx, hipMemcpyAsync(n->history + n->position, tokens, (size_t)count * 4,
                             hipMemcpyHostToDevice, ctx->stream));
  st = run_prompt(ctx, n, count, logits != nullptr, false, false);
  if (st != ND_OK) return st;
  if (logits)
    ND_HIP(ctx, hipMemcpyAsync(logits, n->logits, (size_t)n->d.vocab * 4, hipMemcpyDeviceToHost,
                               ctx->stream));
  ND_HIP(ctx, enqueue_status(n, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return check_waits(ctx, n);
}

nd_status nd_needle_step_select(nd_ctx* ctx, nd_needle* n, uint32_t token, const uint32_t* allowed,
                                uint32_t count, uint32_t* id, double* logprob) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || !id || !logprob) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  nd_status st = check_step(ctx, n, token);
  if (st != ND_OK || (st = use_api(ctx, n, 1)) != ND_OK) return st;
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
  ND_HIP(ctx, enqueue_status(n, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  return check_waits(ctx, n);
}

nd_status nd_needle_grammar_mask(nd_ctx* ctx, nd_needle* n, const nd_grammar* g,
                                 const nd_pieces* pc, const uint32_t* state,
                                 uint32_t n_state_words, uint32_t budget, uint32_t* undecided,
                                 uint32_t* n_allowed) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || !g || !pc || !state || !undecided || !n_allowed)
    return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  if (!n->arena) return nd_fail(ctx, ND_ERR_INVALID, "Call runtime.reset() before decoding");
  if (pc->vocab != n->d.vocab)
    return nd_fail(ctx, ND_ERR_INVALID, "the pieces cover %u ids, the model %u", pc->vocab,
                   n->d.vocab);
  const size_t words = ((size_t)n->d.vocab + 31) / 32;
  // The state through the allowed-id list's buffer (at least vocab words).
  if (n_state_words > n->d.vocab)
    return nd_fail(ctx, ND_ERR_INVALID, "grammar state of %u words", n_state_words);
  nd_status st = nd_check_grammar_state(ctx, state, n_state_words);
  if (st != ND_OK) return st;
  hipStream_t s = ctx->stream;
  ND_HIP(ctx, stage_copy(n, kStageAllowed, n->allowed, state, (size_t)n_state_words * 4, 0, s));
  uint32_t* und = n->allowed + ((n_state_words + 63) & ~63u);
  if ((size_t)((n_state_words + 63) & ~63u) + words > n->d.vocab)
    return nd_fail(ctx, ND_ERR_INVALID, "vocabulary too small for the grammar state");
  ND_HIP(ctx, nd_launch_grammar_mask(g, n->allowed, pc, budget, n->mask, und, s));
  std::vector<uint32_t> bits(words);
  ND_HIP(ctx, hipMemcpyAsync(bits.data(), n->mask, words * 4, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipMemcpyAsync(undecided, und, words * 4, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipStreamSynchronize(s));
  uint32_t count = 0;
  for (uint32_t w : bits) count += (uint32_t)__builtin_popcount(w);
  *n_allowed = count;
  return ND_OK;
}

}  // extern "C"

namespace {

// The host's accepted ids among the undecided ones into the model's mask.
nd_status settle_mask(nd_ctx* ctx, nd_needle* n, const uint32_t* settled, uint32_t n_settled) {
  if (n_settled == 0) return ND_OK;
  if (!settled) return nd_fail(ctx, ND_ERR_INVALID, "NULL settled ids");
  if (n_settled > n->d.vocab)
    return nd_fail(ctx, ND_ERR_INVALID, "more settled ids than the vocabulary");
  for (uint32_t i = 0; i < n_settled; ++i)
    if (settled[i] >= n->d.vocab)
      return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside logits", settled[i]);
  hipStream_t s = ctx->stream;
  ND_HIP(ctx, stage_copy(n, kStageAllowed, n->allowed, settled, (size_t)n_settled * 4, 0, s));
  hipLaunchKernelGGL(n2_set_bits_kernel, dim3((n_settled + 255) / 256), dim3(256), 0, s, n->mask,
                     n->allowed, n_settled);
  ND_HIP(ctx, hipGetLastError());
  return ND_OK;
}

}  // namespace

extern "C" {

nd_status nd_needle_step_select_mask(nd_ctx* ctx, nd_needle* n, uint32_t token,
                                     const uint32_t* settled, uint32_t n_settled, uint32_t* id,
                                     double* logprob) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || !id || !logprob) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  nd_status st = check_step(ctx, n, token);
  if (st != ND_OK || (st = use_api(ctx, n, 1)) != ND_OK) return st;
  if ((st = settle_mask(ctx, n, settled, n_settled)) != ND_OK) return st;
  ND_HIP(ctx, enqueue_step(n, kTokenArg, token, true, true, nullptr, 0, ctx->stream, n->mask));
  ++n->position;
  ND_HIP(ctx, hipMemcpyAsync(id, n->sel_id, 4, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, hipMemcpyAsync(logprob, n->sel_lp, 8, hipMemcpyDeviceToHost, ctx->stream));
  ND_HIP(ctx, enqueue_status(n, ctx->stream));
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  if ((st = check_waits(ctx, n)) != ND_OK) return st;
  if (*id == 0xFFFFFFFFu) return nd_fail(ctx, ND_ERR_INVALID, "Allowed token set is empty");
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
  nd_status st = nd_needle_reset(ctx, n, std::max(count, max_len), sink, ND_KV_INT8, n->collect);
  if (st != ND_OK || (st = use_api(ctx, n, 1)) != ND_OK) return st;
  ND_HIP(ctx, hipMemcpyAsync(n->history, prompt, (size_t)count * 4, hipMemcpyHostToDevice,
                             ctx->stream));
  const uint32_t n_gen = max_new ? std::min(max_new, max_len - count) : 0;
  if ((st = run_prompt(ctx, n, count, false, n_gen > 0, true)) != ND_OK) return st;
  // Token k (k < n_gen - 1) is stepped by decode step k, which records it and
  // its log-probability at history[count + k]; the last one stays in the
  // selection buffers.
  for (uint32_t k = 0; k + 1 < n_gen; ++k) {
    if ((st = launch_graph(ctx, n, kGraphDecodeSelect)) != ND_OK) return st;
    ++n->position;
  }
  ND_HIP(ctx, enqueue_status(n, ctx->stream));
  if (n_gen == 0) {
    ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
    return check_waits(ctx, n);
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
  if ((st = check_waits(ctx, n)) != ND_OK) return st;
  uint32_t out = 0;
  for (; out < n_gen && tok[out] != eos; ++out) {
    ids[out] = tok[out];
    logprobs[out] = lp[out];
  }
  *generated = out;
  return ND_OK;
}

nd_status nd_needle_test_waits(nd_ctx* ctx, nd_needle* n, uint32_t extra_arrivals,
                               uint32_t spin_rounds) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "model is NULL");
  if (extra_arrivals > 1024) return nd_fail(ctx, ND_ERR_INVALID, "at most 1024 extra arrivals");
  ND_HIP(ctx, hipStreamSynchronize(ctx->stream));
  drop_graphs(n);  // the launches' arguments change
  n->dbg_extra = extra_arrivals;
  n->dbg_spin = spin_rounds;
  return ND_OK;
}

nd_status nd_needle_step_launches(nd_ctx* ctx, nd_needle* n, uint32_t* launches) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n || !launches) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  *launches = n->graphs[kGraphDecodeSelect] ? n->graph_kernels[kGraphDecodeSelect] : 0;
  return ND_OK;
}

nd_status nd_needle_test_stamps(nd_ctx* ctx, nd_needle* n, uint64_t* stamps, uint32_t capacity) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "NULL model");
  if (stamps && ((n->cq && !n->phi_uniform) || capacity < (n->d.layers + 1) * 64 * 16))
    return nd_fail(ctx, ND_ERR_INVALID,
                   "nd_needle_test_stamps: an int8 model or a Cactus-Quant one whose phi "
                   "matrices share one format, and room for %u stamps",
                   (n->d.layers + 1) * 64 * 16);
  n->dbg_stamps = stamps;
  return ND_OK;
}

}  // extern "C"

// ------------------------------------------------------ session methods
//
// ResidentExecutionSession (backends/backend.ts:65-80) at method granularity,
// as NeedleRuntime.step drives it (model/runtime.ts:314-375, 444-463,
// 554-564): the host keeps the position, the token history and the engram
// hashing; the device keeps the KV cache, the engram ring, the lanes and the
// confidence pool.  A resident token is begin -> (prepare engrams) ->
// forward token (or forward layer 0..L-1) -> finish -> (select).

namespace {

nd_status check_session(nd_ctx* ctx, nd_needle* n) {
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "model is NULL");
  if (!n->arena || !n->max_length)
    return nd_fail(ctx, ND_ERR_INVALID, "Call runtime.reset() before decoding");
  return use_api(ctx, n, 2);
}

int site_of(const nd_needle* n, uint32_t layer) {
  for (uint32_t si = 0; si < n->d.n_sites; ++si)
    if (n->d.sites[si] == layer) return (int)si;
  return -1;
}

hipError_t enqueue_position(nd_needle* n, uint32_t position, hipStream_t s) {
  hipLaunchKernelGGL(n2_position_kernel, dim3(1), dim3(64), 0, s, n->st, position, n->inv_freq,
                     n->rope);
  return hipGetLastError();
}

// The session's final mix (post of the last layer, the lane mean and final
// norm when tail), the pool and the logits.
hipError_t enqueue_session_final(nd_needle* n, bool tail, hipStream_t s) {
  hipError_t e;
  if (tail || pool_on(n)) {
    const uint32_t parts = (n->post_pending ? kMixPost | kMixCell : 0) | (tail ? kMixFinal : 0);
    if ((e = enqueue_mix(n, n->d.layers, parts, s)) != hipSuccess) return e;
    n->post_pending = false;
  }
  return enqueue_final(n, tail, false, nullptr, 0, s);
}

void close_token(nd_needle* n) {
  n->token_open = n->engrams_ready = n->host_engrams = false;
  n->position = n->token_position + 1;
}

}  // namespace

extern "C" {

nd_status nd_needle_begin_token(nd_ctx* ctx, nd_needle* n, const float* lanes) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  if (!lanes) return nd_fail(ctx, ND_ERR_INVALID, "lanes is NULL");
  // A token left open (a runtime that aborted between beginResidentToken and
  // finish, runtime.ts:338-342) is dropped; its position was not advanced.
  const size_t D = n->d.dim;
  hipStream_t s = ctx->stream;
  ND_HIP(ctx, stage_copy(n, kStageLanes, n->x, lanes, (size_t)n->d.lanes * D * 4, 0, s));
  // Every lane holds the scaled embedding (runtime.ts:312-313): cell 0 of the
  // confidence pool (runtime.ts:310).
  if (pool_on(n))
    ND_HIP(ctx, hipMemcpyAsync(n->cells, n->x, D * 4, hipMemcpyDeviceToDevice, s));
  n->token_open = true;
  n->post_pending = n->select_ready = false;
  n->next_layer = 0;
  return ND_OK;
}

nd_status nd_needle_prepare_engrams(nd_ctx* ctx, nd_needle* n, const uint32_t* indices,
                                    const uint32_t* valid, uint32_t tables, uint32_t position) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  const nd_needle_desc& d = n->d;
  if (!d.n_sites) return nd_fail(ctx, ND_ERR_INVALID, "the model has no engram layers");
  if (!indices || !valid) return nd_fail(ctx, ND_ERR_INVALID, "indices or valid is NULL");
  if (tables != d.engram_tables)
    return nd_fail(ctx, ND_ERR_INVALID, "%u engram lookups for %u tables", tables,
                   d.engram_tables);
  if (n->token_open)
    return nd_fail(ctx, ND_ERR_INVALID, "engrams are prepared before the token begins");
  if (position >= n->max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %u reached runtime limit %u", position,
                   n->max_length);
  uint32_t buf[32];
  for (uint32_t t = 0; t < tables; ++t) {
    if (valid[t] && indices[t] >= d.engram_slots)
      return nd_fail(ctx, ND_ERR_INVALID, "engram index %u is outside %u slots", indices[t],
                     d.engram_slots);
    buf[t] = valid[t] ? indices[t] : 0;
    buf[tables + t] = valid[t] ? 1 : 0;
  }
  hipStream_t s = ctx->stream;
  ND_HIP(ctx, stage_copy(n, kStageLookup, n->lookup, buf, (size_t)2 * tables * 4, 0, s));
  ND_HIP(ctx, enqueue_position(n, position, s));
  if (n->cq) {
    ND_HIP(ctx, enqueue_cq_rows(n, nullptr, n->lookup, s));
  } else {
    hipLaunchKernelGGL(n2_gather_kernel, dim3(1), dim3(kWg), 0, s, begin_args(n), n->lookup);
    ND_HIP(ctx, hipGetLastError());
  }
  ND_HIP(ctx, enqueue_engrams(n, s));
  n->engrams_ready = true;
  return ND_OK;
}

nd_status nd_needle_forward_layer(nd_ctx* ctx, nd_needle* n, uint32_t layer, uint32_t position,
                                  const float* engram_key, const float* engram_value) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  const nd_needle_desc& d = n->d;
  if (!n->token_open) return nd_fail(ctx, ND_ERR_INVALID, "Resident layers run after beginResidentToken");
  if (layer != n->next_layer)
    return nd_fail(ctx, ND_ERR_INVALID, "layer %u forwarded out of order (next is %u)", layer,
                   n->next_layer);
  if (position >= n->max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %u reached runtime limit %u", position,
                   n->max_length);
  if (layer > 0 && position != n->token_position)
    return nd_fail(ctx, ND_ERR_INVALID, "layer %u at position %u follows position %u", layer,
                   position, n->token_position);
  hipStream_t s = ctx->stream;
  if (layer == 0) {
    ND_HIP(ctx, enqueue_position(n, position, s));
    n->token_position = position;
  }
  const int site = site_of(n, layer);
  if (site >= 0) {
    const size_t D = d.dim, S = d.n_sites;
    if (engram_key && engram_value) {
      // The host's #engramStep result (runtime.ts:820-877) for this site;
      // the runtime hands these over only when the device did not prepare
      // the token's engrams (runtime.ts:315-325).
      if (n->engrams_ready)
        return nd_fail(ctx, ND_ERR_INVALID, "the engrams of this token were prepared resident");
      ND_HIP(ctx, stage_copy(n, (StageSlot)(kStageEngram + 2 * site), n->host_eng + site * D,
                             engram_key, D * 4, 0, s));
      ND_HIP(ctx, stage_copy(n, (StageSlot)(kStageEngram + 2 * site + 1),
                             n->host_eng + (S + site) * D, engram_value, D * 4, 0, s));
      n->host_engrams = true;
    } else if (!n->engrams_ready) {
      return nd_fail(ctx, ND_ERR_INVALID, "Missing engram values for layer %u", layer);
    }
  }
  const uint32_t parts = (n->post_pending ? kMixPost | kMixCell : 0) | kMixPre;
  ND_HIP(ctx, enqueue_mix(n, layer, parts, s));
  ND_HIP(ctx, enqueue_block(n, layer, s));
  n->post_pending = true;
  ++n->next_layer;
  return ND_OK;
}

nd_status nd_needle_forward_token(nd_ctx* ctx, nd_needle* n, uint32_t position,
                                  const float* engram_keys, const float* engram_values) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  if (!n) return nd_fail(ctx, ND_ERR_INVALID, "model is NULL");
  if ((engram_keys == nullptr) != (engram_values == nullptr))
    return nd_fail(ctx, ND_ERR_INVALID, "engram keys and values come together");
  const size_t D = n->d.dim;
  for (uint32_t l = 0; l < n->d.layers; ++l) {
    const int site = site_of(n, l);
    const float* k = engram_keys && site >= 0 ? engram_keys + site * D : nullptr;
    const float* v = engram_values && site >= 0 ? engram_values + site * D : nullptr;
    const nd_status st = nd_needle_forward_layer(ctx, n, l, position, k, v);
    if (st != ND_OK) return st;
  }
  return ND_OK;
}

nd_status nd_needle_finish_token(nd_ctx* ctx, nd_needle* n, uint32_t want_logits, float* logits) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  if (!n->token_open || n->next_layer != n->d.layers)
    return nd_fail(ctx, ND_ERR_INVALID, "finishResidentToken after every layer (%u of %u ran)",
                   n->token_open ? n->next_layer : 0, n->d.layers);
  if (want_logits && !logits) return nd_fail(ctx, ND_ERR_INVALID, "logits is NULL");
  hipStream_t s = ctx->stream;
  ND_HIP(ctx, enqueue_session_final(n, want_logits != 0, s));
  close_token(n);
  if (!want_logits) return ND_OK;
  ND_HIP(ctx, hipMemcpyAsync(logits, n->logits, (size_t)n->d.vocab * 4, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipStreamSynchronize(s));
  return ND_OK;
}

nd_status nd_needle_finish_token_for_selection(nd_ctx* ctx, nd_needle* n) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  if (!n->token_open || n->next_layer != n->d.layers)
    return nd_fail(ctx, ND_ERR_INVALID,
                   "finishResidentTokenForSelection after every layer (%u of %u ran)",
                   n->token_open ? n->next_layer : 0, n->d.layers);
  ND_HIP(ctx, enqueue_session_final(n, true, ctx->stream));
  close_token(n);
  n->select_ready = true;
  return ND_OK;
}

nd_status nd_needle_select_token(nd_ctx* ctx, nd_needle* n, const uint32_t* allowed,
                                 uint32_t count, uint32_t* id, double* log_probability) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  if (!id || !log_probability) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  if (!n->select_ready)
    return nd_fail(ctx, ND_ERR_BACKEND, "Token selection did not produce a result");
  const uint32_t vocab = n->d.vocab;
  hipStream_t s = ctx->stream;
  if (allowed) {
    // selectToken (runtime.ts:880-899): a non-empty id list inside the logits.
    if (count == 0) return nd_fail(ctx, ND_ERR_INVALID, "Allowed token set is empty");
    if (count > vocab)
      return nd_fail(ctx, ND_ERR_INVALID, "Allowed token set is larger than the vocabulary");
    for (uint32_t i = 0; i < count; ++i)
      if (allowed[i] >= vocab)
        return nd_fail(ctx, ND_ERR_INVALID, "Token %u is outside logits", allowed[i]);
    ND_HIP(ctx, stage_copy(n, kStageAllowed, n->allowed, allowed, (size_t)count * 4, 0, s));
  }
  ND_HIP(ctx, nd_launch_select_list(n->logits, vocab, allowed ? n->allowed : nullptr,
                                    allowed ? count : 0, n->sel_id, n->sel_lp, s));
  n->select_ready = false;
  ND_HIP(ctx, hipMemcpyAsync(id, n->sel_id, 4, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipMemcpyAsync(log_probability, n->sel_lp, 8, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipStreamSynchronize(s));
  return ND_OK;
}

nd_status nd_needle_select_token_mask(nd_ctx* ctx, nd_needle* n, const uint32_t* settled,
                                      uint32_t n_settled, uint32_t* id, double* log_probability) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  if (!id || !log_probability) return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  if (!n->select_ready)
    return nd_fail(ctx, ND_ERR_BACKEND, "Token selection did not produce a result");
  if ((st = settle_mask(ctx, n, settled, n_settled)) != ND_OK) return st;
  hipStream_t s = ctx->stream;
  ND_HIP(ctx, nd_launch_select_mask(n->logits, 1, n->d.vocab, n->mask, n->sel_id, n->sel_lp, s,
                                    nullptr, nullptr, nullptr));
  n->select_ready = false;
  ND_HIP(ctx, hipMemcpyAsync(id, n->sel_id, 4, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipMemcpyAsync(log_probability, n->sel_lp, 8, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipStreamSynchronize(s));
  if (*id == 0xFFFFFFFFu) return nd_fail(ctx, ND_ERR_INVALID, "Allowed token set is empty");
  return ND_OK;
}

nd_status nd_needle_read_lanes(nd_ctx* ctx, nd_needle* n, float* lanes) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  if (!lanes) return nd_fail(ctx, ND_ERR_INVALID, "lanes is NULL");
  hipStream_t s = ctx->stream;
  if (n->token_open && n->post_pending) {
    // The post half owed to the last layer run: the lanes after it.
    ND_HIP(ctx, enqueue_mix(n, n->next_layer, kMixPost | kMixCell, s));
    n->post_pending = false;
  }
  ND_HIP(ctx, hipMemcpyAsync(lanes, n->x, (size_t)n->d.lanes * n->d.dim * 4,
                             hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipStreamSynchronize(s));
  return ND_OK;
}

nd_status nd_needle_forward(nd_ctx* ctx, nd_needle* n, uint32_t layer, uint32_t position,
                            const float* input, const float* block_input,
                            const float* update_input, const float* x, const float* phi_post,
                            const float* phi_residual, float* next_x) {
  if (!ctx) return nd_fail(nullptr, ND_ERR_BACKEND, "context is NULL");
  nd_status st = check_session(ctx, n);
  if (st != ND_OK) return st;
  const nd_needle_desc& d = n->d;
  if (!input || !block_input || !update_input || !x || !phi_post || !phi_residual || !next_x)
    return nd_fail(ctx, ND_ERR_INVALID, "NULL argument");
  if (n->token_open)
    return nd_fail(ctx, ND_ERR_INVALID, "forward() runs a layer of a token not begun resident");
  if (layer >= d.layers)
    return nd_fail(ctx, ND_ERR_INVALID, "layer %u is outside [0, %u)", layer, d.layers);
  if (position >= n->max_length)
    return nd_fail(ctx, ND_ERR_OVERFLOW, "Position %u reached runtime limit %u", position,
                   n->max_length);
  const size_t D = d.dim, ln = d.lanes;
  hipStream_t s = ctx->stream;
  // One staged copy of every input, then their places on the device.
  const float* parts[] = {input, block_input, update_input, x, phi_post, phi_residual};
  float* dsts[] = {n->ain, n->blk, n->upd, n->x, n->phi_post_v, n->phi_res_v};
  const size_t sizes[] = {D, D, D, ln * D, ln, ln * ln};
  size_t off = 0;
  ND_HIP(ctx, hipEventSynchronize(n->stage_done[kStageForward]));
  float* slot = reinterpret_cast<float*>(n->pinned + n->stage_off[kStageForward]);
  for (int i = 0; i < 6; ++i) {
    std::memcpy(slot + off, parts[i], sizes[i] * 4);
    off += sizes[i];
  }
  ND_HIP(ctx, hipMemcpyAsync(n->fwd_in, slot, off * 4, hipMemcpyHostToDevice, s));
  ND_HIP(ctx, hipEventRecord(n->stage_done[kStageForward], s));
  off = 0;
  for (int i = 0; i < 6; ++i) {
    ND_HIP(ctx, hipMemcpyAsync(dsts[i], n->fwd_in + off, sizes[i] * 4, hipMemcpyDeviceToDevice, s));
    off += sizes[i];
  }
  ND_HIP(ctx, enqueue_position(n, position, s));
  // Q/K/V/gate, norms and RoPE, #storeKV, gated attention, Wo (with the
  // layer's routing from the host's phi rows), then the post half: sandwich
  // norm, Hadamard MLP, h-post and the Sinkhorn routing of the lanes -- the
  // next lanes ("nextX", runtime.ts:456-458).
  ND_HIP(ctx, enqueue_block(n, layer, s));
  ND_HIP(ctx, enqueue_mix(n, layer + 1, kMixPost, s));
  ND_HIP(ctx, hipMemcpyAsync(next_x, n->x, ln * D * 4, hipMemcpyDeviceToHost, s));
  ND_HIP(ctx, hipStreamSynchronize(s));
  if (layer + 1 == d.layers) n->position = position + 1;
  return ND_OK;
}

}  // extern "C"
