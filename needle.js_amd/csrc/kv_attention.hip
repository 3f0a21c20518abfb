// Int8 KV-cache append and split-context single-query decode attention.
//
// Cache layout in HBM (per nd_kv): codes [layers][kv_heads][alloc][64] int8,
// scales [layers][kv_heads][alloc] f32, exactly NeedleRuntime's arrays
// (model/runtime.ts:186-204, 666-677).  A 64-dim code row is 64 bytes, so a
// 16-token x 64-dim tile is one contiguous 1 KiB run that a wave reads with
// 128-bit loads.
#include "nd_internal.hpp"

namespace {

constexpr uint32_t kHeadDim = 64;
constexpr uint32_t kChunk = 64;  // visible positions per attention workgroup

__device__ __forceinline__ uint32_t kv_slot(uint32_t position, uint32_t sink, uint32_t window) {
  if (window == 0 || position < sink) return position;
  return sink + (position - sink) % window;
}

// JavaScript Math.max: NaN wins.
__device__ __forceinline__ float js_maxf(float a, float b) {
  if (a != a || b != b) return __builtin_nanf("");
  return a > b ? a : b;
}

__device__ __forceinline__ float wave_max_js(float v) {
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) v = js_maxf(v, __shfl_xor(v, o, 64));
  return v;
}

// Int8Array store of an integral double: NaN -> 0; |v| <= 127 here.
__device__ __forceinline__ int8_t to_int8(double v) { return v != v ? (int8_t)0 : (int8_t)(int)v; }

// One wave per (position, kv head).  #storeKV, model/runtime.ts:697-714:
// m = max(1e-12, max|x|) and s = m / 127 in float64, scale f32(s), code =
// roundTiesToEven(x / s).  The float64 division is IEEE-correctly rounded on
// gfx950 and rint() rounds half to even, which is roundTiesToEven
// (runtime.ts:901-907) for every finite value.
template <bool F32>
__global__ __launch_bounds__(64) void kv_store_kernel(void* __restrict__ Kc, void* __restrict__ Vc,
                                                      float* __restrict__ Ks, float* __restrict__ Vs,
                                                      const float* __restrict__ k,
                                                      const float* __restrict__ v, uint32_t layer,
                                                      uint32_t kv_heads, uint32_t alloc,
                                                      uint32_t sink, uint32_t window,
                                                      uint32_t position, uint32_t count) {
  const uint32_t i = blockIdx.x, h = blockIdx.y, lane = threadIdx.x;
  const uint32_t p = position + i;
  const uint32_t last = position + count - 1;
  // A later position of this call that reuses the ring slot overwrites it.
  if (window > 0 && p >= sink && p + window <= last) return;
  const uint32_t slot = kv_slot(p, sink, window);
  const size_t row = ((size_t)layer * kv_heads + h) * alloc + slot;
  const size_t src = ((size_t)i * kv_heads + h) * kHeadDim + lane;
  const float xk = k[src], xv = v[src];
  if constexpr (F32) {
    reinterpret_cast<float*>(Kc)[row * kHeadDim + lane] = xk;
    reinterpret_cast<float*>(Vc)[row * kHeadDim + lane] = xv;
    if (lane == 0) {
      Ks[row] = 1.f;
      Vs[row] = 1.f;
    }
  } else {
    const float ak = wave_max_js(fabsf(xk)), av = wave_max_js(fabsf(xv));
    const double mk = (ak != ak) ? (double)ak : fmax(1e-12, (double)ak);
    const double mv = (av != av) ? (double)av : fmax(1e-12, (double)av);
    const double sk = mk / 127.0, svv = mv / 127.0;
    reinterpret_cast<int8_t*>(Kc)[row * kHeadDim + lane] = to_int8(rint((double)xk / sk));
    reinterpret_cast<int8_t*>(Vc)[row * kHeadDim + lane] = to_int8(rint((double)xv / svv));
    if (lane == 0) {
      Ks[row] = (float)sk;
      Vs[row] = (float)svv;
    }
  }
}

struct Visible {
  uint32_t prefix, recent_low, count;
};

__device__ __forceinline__ uint32_t logical_at(const Visible& vis, uint32_t t) {
  return t < vis.prefix ? t : vis.recent_low + (t - vis.prefix);
}

__device__ __forceinline__ void decode16(const uint4& w, float* out) {
  const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
  for (int q = 0; q < 4; ++q) {
#pragma unroll
    for (int e = 0; e < 4; ++e)
      out[4 * q + e] = (float)(int8_t)((words[q] >> (8 * e)) & 0xffu);
  }
}

// One wave per (kv head, chunk of 64 visible positions), serving all REP
// query heads of the kv head so that each code byte is read once.
// Lane l owns dims [16*(l&3), +16) of tokens chunk + (l>>2) + 16*k, k < 4.
// Output per query head and chunk: (max score m, sum exp l, acc[64]) or, for
// a single chunk, the normalized result directly.
template <int REP, bool F32>
__global__ __launch_bounds__(64) void attention_chunk_kernel(
    const void* __restrict__ Kc, const void* __restrict__ Vc, const float* __restrict__ Ks,
    const float* __restrict__ Vs, const float* __restrict__ Q, float* __restrict__ out,
    float* __restrict__ partials, uint32_t layer, uint32_t kv_heads, uint32_t alloc, uint32_t sink,
    uint32_t window, Visible vis, uint32_t nchunks, float score_scale) {
  const uint32_t chunk = blockIdx.x, kvh = blockIdx.y, lane = threadIdx.x;
  const uint32_t quad = lane & 3, trow = lane >> 2;
  const size_t head_base = ((size_t)layer * kv_heads + kvh) * alloc;

  float q[REP][16];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const float4* qp = reinterpret_cast<const float4*>(Q + (size_t)(kvh * REP + h) * kHeadDim + quad * 16);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 f = qp[c];
      q[h][4 * c + 0] = f.x;
      q[h][4 * c + 1] = f.y;
      q[h][4 * c + 2] = f.z;
      q[h][4 * c + 3] = f.w;
    }
  }

  float kc[4][16], vc[4][16];
  float ks[4], vs[4];
  bool valid[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t t = chunk * kChunk + trow + 16 * k;
    valid[k] = t < vis.count;
    const uint32_t slot = kv_slot(logical_at(vis, valid[k] ? t : 0), sink, window);
    const size_t row = head_base + slot;
    ks[k] = Ks[row];
    vs[k] = Vs[row];
    if constexpr (F32) {
      const float4* kp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(Kc) + row * kHeadDim + quad * 16);
      const float4* vp = reinterpret_cast<const float4*>(reinterpret_cast<const float*>(Vc) + row * kHeadDim + quad * 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 a = kp[c], b = vp[c];
        kc[k][4 * c + 0] = a.x; kc[k][4 * c + 1] = a.y; kc[k][4 * c + 2] = a.z; kc[k][4 * c + 3] = a.w;
        vc[k][4 * c + 0] = b.x; vc[k][4 * c + 1] = b.y; vc[k][4 * c + 2] = b.z; vc[k][4 * c + 3] = b.w;
      }
    } else {
      const uint4 a = *reinterpret_cast<const uint4*>(reinterpret_cast<const int8_t*>(Kc) + row * kHeadDim + quad * 16);
      const uint4 b = *reinterpret_cast<const uint4*>(reinterpret_cast<const int8_t*>(Vc) + row * kHeadDim + quad * 16);
      decode16(a, kc[k]);
      decode16(b, vc[k]);
    }
  }

  float m[REP], l[REP], p[REP][4];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float mh = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) d = fmaf(q[h][i], kc[k][i], d);
      d += __shfl_xor(d, 1, 64);
      d += __shfl_xor(d, 2, 64);
      const float s = valid[k] ? d * ks[k] * score_scale : -INFINITY;
      p[h][k] = s;
      mh = fmaxf(mh, s);
    }
#pragma unroll
    for (int o = 4; o <= 32; o <<= 1) mh = fmaxf(mh, __shfl_xor(mh, o, 64));
    float lh = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float e = valid[k] ? __expf(p[h][k] - mh) : 0.f;
      p[h][k] = e;
      lh += e;
    }
#pragma unroll
    for (int o = 4; o <= 32; o <<= 1) lh += __shfl_xor(lh, o, 64);
    m[h] = mh;
    l[h] = lh;
  }

  // acc[h*16 + i]: this lane's token rows, dims quad*16 + i.
  constexpr int V = REP * 16;
  float acc[V];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      float a = 0.f;
#pragma unroll
      for (int k = 0; k < 4; ++k) a = fmaf(p[h][k] * vs[k], vc[k][i], a);
      acc[h * 16 + i] = a;
    }
  }
  // Transposing butterfly over the 16 token rows (lane bits 2..5).
  uint32_t idx_base = 0;
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const int c = V >> s;
    const int half = c >> 1;
    const bool upper = (trow >> s) & 1u;
#pragma unroll
    for (int i = 0; i < half; ++i) {
      const float send = upper ? acc[i] : acc[i + half];
      const float keep = upper ? acc[i + half] : acc[i];
      acc[i] = keep + __shfl_xor(send, 4 << s, 64);
    }
    if (upper) idx_base += half;
  }
  // Each lane now holds REP finished sums: indices idx_base + i.
#pragma unroll
  for (int i = 0; i < REP; ++i) {
    const uint32_t idx = idx_base + i;
    const uint32_t h = idx / 16, dim = quad * 16 + (idx % 16);
    const uint32_t qh = kvh * REP + h;
    // Select the per-head m and l without dynamic register indexing.
    float mh = m[0], lh = l[0];
#pragma unroll
    for (int hh = 1; hh < REP; ++hh) {
      if (h == (uint32_t)hh) {
        mh = m[hh];
        lh = l[hh];
      }
    }
    if (nchunks == 1) {
      out[(size_t)qh * kHeadDim + dim] = acc[i] / lh;
    } else {
      float* part = partials + ((size_t)qh * nchunks + chunk) * (2 + kHeadDim);
      part[2 + dim] = acc[i];
      if (dim == 0) {
        part[0] = mh;
        part[1] = lh;
      }
    }
  }
}

// Log-sum-exp merge of the chunk partials: one wave per query head, lane = dim.
__global__ __launch_bounds__(64) void attention_merge_kernel(const float* __restrict__ partials,
                                                             uint32_t nchunks,
                                                             float* __restrict__ out) {
  const uint32_t qh = blockIdx.x, dim = threadIdx.x;
  const float* base = partials + (size_t)qh * nchunks * (2 + kHeadDim);
  float mx = -INFINITY;
  for (uint32_t c = 0; c < nchunks; ++c) mx = fmaxf(mx, base[(size_t)c * (2 + kHeadDim)]);
  float total = 0.f, acc = 0.f;
  for (uint32_t c = 0; c < nchunks; ++c) {
    const float* part = base + (size_t)c * (2 + kHeadDim);
    const float w = __expf(part[0] - mx);
    total = fmaf(w, part[1], total);
    acc = fmaf(w, part[2 + dim], acc);
  }
  out[(size_t)qh * kHeadDim + dim] = acc / total;
}

}  // namespace

nd_visible nd_kv_visible(const nd_kv* kv, uint32_t position) {
  nd_visible v;
  v.prefix = kv->sink < position + 1 ? kv->sink : position + 1;
  v.recent_low = v.prefix;
  if (kv->window > 0 && position + 1 > kv->window && position + 1 - kv->window > v.prefix)
    v.recent_low = position + 1 - kv->window;
  v.count = v.prefix + (position - v.recent_low + 1);
  return v;
}

uint32_t nd_attention_chunks(uint32_t count) { return (count + kChunk - 1) / kChunk; }

size_t nd_attention_partial_floats(uint32_t q_heads, uint32_t count) {
  return (size_t)q_heads * nd_attention_chunks(count) * (2 + kHeadDim);
}

hipError_t nd_launch_kv_store(const nd_kv* kv, uint32_t layer, uint32_t position, uint32_t first,
                              uint32_t count, const float* k, const float* v, hipStream_t s) {
  (void)first;
  if (count == 0) return hipSuccess;
  dim3 grid(count, kv->kv_heads);
  if (kv->mode == ND_KV_FLOAT32)
    hipLaunchKernelGGL(kv_store_kernel<true>, grid, dim3(64), 0, s, kv->k, kv->v, kv->ks, kv->vs,
                       k, v, layer, kv->kv_heads, kv->alloc, kv->sink, kv->window, position, count);
  else
    hipLaunchKernelGGL(kv_store_kernel<false>, grid, dim3(64), 0, s, kv->k, kv->v, kv->ks, kv->vs,
                       k, v, layer, kv->kv_heads, kv->alloc, kv->sink, kv->window, position, count);
  return hipGetLastError();
}

template <int REP, bool F32>
static void launch_chunks(const nd_kv* kv, uint32_t layer, const float* q, float* out,
                          float* partials, const Visible& vis, uint32_t nchunks, hipStream_t s) {
  hipLaunchKernelGGL((attention_chunk_kernel<REP, F32>), dim3(nchunks, kv->kv_heads), dim3(64), 0,
                     s, kv->k, kv->v, kv->ks, kv->vs, q, out, partials, layer, kv->kv_heads,
                     kv->alloc, kv->sink, kv->window, vis, nchunks, 0.125f);
}

template <bool F32>
static hipError_t launch_rep(uint32_t rep, const nd_kv* kv, uint32_t layer, const float* q,
                             float* out, float* partials, const Visible& vis, uint32_t nchunks,
                             hipStream_t s) {
  switch (rep) {
    case 1: launch_chunks<1, F32>(kv, layer, q, out, partials, vis, nchunks, s); break;
    case 2: launch_chunks<2, F32>(kv, layer, q, out, partials, vis, nchunks, s); break;
    case 4: launch_chunks<4, F32>(kv, layer, q, out, partials, vis, nchunks, s); break;
    case 8: launch_chunks<8, F32>(kv, layer, q, out, partials, vis, nchunks, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t nd_launch_attention(const nd_kv* kv, uint32_t layer, uint32_t position,
                               const float* q, uint32_t q_heads, float* out, float* partials,
                               hipStream_t s) {
  const nd_visible nv = nd_kv_visible(kv, position);
  const Visible vis{nv.prefix, nv.recent_low, nv.count};
  const uint32_t nchunks = nd_attention_chunks(nv.count);
  const uint32_t rep = q_heads / kv->kv_heads;
  hipError_t e = kv->mode == ND_KV_FLOAT32
                     ? launch_rep<true>(rep, kv, layer, q, out, partials, vis, nchunks, s)
                     : launch_rep<false>(rep, kv, layer, q, out, partials, vis, nchunks, s);
  if (e != hipSuccess || nchunks == 1) return e;
  hipLaunchKernelGGL(attention_merge_kernel, dim3(q_heads), dim3(64), 0, s, partials, nchunks, out);
  return hipGetLastError();
}
