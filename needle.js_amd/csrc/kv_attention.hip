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

// Visible positions of query `position` (model/runtime.ts:723-728).
__device__ __forceinline__ Visible visible_at(uint32_t position, uint32_t sink, uint32_t window) {
  Visible v;
  v.prefix = sink < position + 1 ? sink : position + 1;
  v.recent_low = v.prefix;
  if (window > 0 && position + 1 > window && position + 1 - window > v.prefix)
    v.recent_low = position + 1 - window;
  v.count = v.prefix + (position - v.recent_low + 1);
  return v;
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

// One workgroup of W waves (W <= 4) per (kv head, chunk of 64*W visible
// positions), serving all REP query heads of the kv head so that each code
// byte is read once.  In wave w, lane l owns dims [16*(l&3), +16) of the
// positions chunk*64W + 64w + (l>>2) + 16k, k < 4, so every 128-bit load of
// the wave reads 16 consecutive 64-byte code rows (1 KiB contiguous).
//
// Each wave reduces its 64 positions to (max m, sum l, acc[64]) per query
// head; the waves are merged through LDS.  With one chunk the workgroup
// writes the normalized output.  Otherwise it writes its partial, and the
// last workgroup of the kv head to finish (device-scope counter, reset by
// that workgroup) merges all chunks with a log-sum-exp combine.
constexpr int kMaxWaves = 4;

template <int REP, bool F32>
__global__ __launch_bounds__(256) void attention_kernel(
    const void* __restrict__ Kc, const void* __restrict__ Vc, const float* __restrict__ Ks,
    const float* __restrict__ Vs, const float* __restrict__ Q, float* __restrict__ out,
    float* __restrict__ part_acc, float* __restrict__ part_ml, uint32_t* __restrict__ counters,
    uint32_t layer, uint32_t kv_heads, uint32_t alloc, uint32_t sink, uint32_t window,
    Visible vis, const uint32_t* __restrict__ positions, uint32_t seq_kv_heads,
    uint32_t max_chunks, float score_scale) {
  // blockIdx.z selects the sequence of a batch: its KV heads are cache heads
  // [z * seq_kv_heads, +seq_kv_heads), its queries rows [z * Hq, +Hq), and its
  // query position is positions[z] (or the single `vis` when positions is null).
  const uint32_t chunk = blockIdx.x, z = blockIdx.z;
  const uint32_t kvh_local = blockIdx.y;
  const uint32_t kvh = z * seq_kv_heads + kvh_local;
  const uint32_t hq = seq_kv_heads * REP;
  const uint32_t wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
  const uint32_t nwaves = blockDim.x >> 6;
  const uint32_t quad = lane & 3, trow = lane >> 2;
  if (positions) {
    if (window == 0 && positions[z] >= alloc) return;  // validated on entry; stay in bounds
    vis = visible_at(positions[z], sink, window);
  }
  // The grid covers max_chunks; a position beyond the launch's bound is a
  // caller error that must not turn into out-of-range partial writes.
  uint32_t nchunks = (vis.count + kChunk * nwaves - 1) / (kChunk * nwaves);
  if (nchunks > max_chunks) nchunks = max_chunks;
  if (chunk >= nchunks) return;
  Q += (size_t)z * hq * kHeadDim;
  out += (size_t)z * hq * kHeadDim;
  const size_t part_base = (size_t)z * hq * max_chunks;
  const size_t head_base = ((size_t)layer * kv_heads + kvh) * alloc;
  const uint32_t tok0 = (chunk * nwaves + wave) * kChunk;

  float kc[4][16], vc[4][16];
  float ks[4], vs[4];
  bool valid[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t t = tok0 + trow + 16 * k;
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

  float q[REP][16];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const float4* qp = reinterpret_cast<const float4*>(Q + (size_t)(kvh_local * REP + h) * kHeadDim + quad * 16);
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const float4 f = qp[c];
      q[h][4 * c + 0] = f.x;
      q[h][4 * c + 1] = f.y;
      q[h][4 * c + 2] = f.z;
      q[h][4 * c + 3] = f.w;
    }
  }

  __shared__ float s_m[kMaxWaves][REP], s_l[kMaxWaves][REP];
  __shared__ float s_acc[kMaxWaves][REP * kHeadDim];

#pragma unroll
  for (int h = 0; h < REP; ++h) {
    float sc[4];
    float mh = -INFINITY;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float d = 0.f;
#pragma unroll
      for (int i = 0; i < 16; ++i) d = fmaf(q[h][i], kc[k][i], d);
      d += __shfl_xor(d, 1, 64);
      d += __shfl_xor(d, 2, 64);
      sc[k] = valid[k] ? d * ks[k] * score_scale : -INFINITY;
      mh = fmaxf(mh, sc[k]);
    }
#pragma unroll
    for (int o = 4; o <= 32; o <<= 1) mh = fmaxf(mh, __shfl_xor(mh, o, 64));
    float lh = 0.f;
    float a[16];
#pragma unroll
    for (int i = 0; i < 16; ++i) a[i] = 0.f;
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const float e = valid[k] ? __expf(sc[k] - mh) : 0.f;
      lh += e;
      const float ev = e * vs[k];
#pragma unroll
      for (int i = 0; i < 16; ++i) a[i] = fmaf(ev, vc[k][i], a[i]);
    }
    // Sum over the 16 token rows (lane bits 2..5); all lanes of a quad end
    // with the full sums of their 16 dims.
#pragma unroll
    for (int o = 4; o <= 32; o <<= 1) {
      lh += __shfl_xor(lh, o, 64);
#pragma unroll
      for (int i = 0; i < 16; ++i) a[i] += __shfl_xor(a[i], o, 64);
    }
    if (trow == 0) {
#pragma unroll
      for (int i = 0; i < 16; ++i) s_acc[wave][h * kHeadDim + quad * 16 + i] = a[i];
      if (quad == 0) {
        s_m[wave][h] = mh;
        s_l[wave][h] = lh;
      }
    }
  }
  __syncthreads();

  // Merge the waves: thread t < REP*64 owns (h, dim).
  const uint32_t t = threadIdx.x;
  float mine_m = -INFINITY, mine_l = 0.f, mine_a = 0.f;
  uint32_t h_t = 0, dim_t = 0;
  for (uint32_t o = t; o < REP * kHeadDim; o += blockDim.x) {
    h_t = o / kHeadDim;
    dim_t = o % kHeadDim;
    float mx = -INFINITY;
    for (uint32_t w = 0; w < nwaves; ++w) mx = fmaxf(mx, s_m[w][h_t]);
    float L = 0.f, A = 0.f;
    for (uint32_t w = 0; w < nwaves; ++w) {
      const float f = (s_m[w][h_t] == -INFINITY) ? 0.f : __expf(s_m[w][h_t] - mx);
      L = fmaf(f, s_l[w][h_t], L);
      A = fmaf(f, s_acc[w][h_t * kHeadDim + dim_t], A);
    }
    const uint32_t qh = kvh_local * REP + h_t;
    if (nchunks == 1) {
      out[(size_t)qh * kHeadDim + dim_t] = A / L;
    } else {
      const size_t pi = part_base + (size_t)qh * max_chunks + chunk;
      part_acc[pi * kHeadDim + dim_t] = A;
      if (dim_t == 0) {
        part_ml[pi * 2 + 0] = mx;
        part_ml[pi * 2 + 1] = L;
      }
    }
    mine_m = mx;
    mine_l = L;
    mine_a = A;
  }
  (void)mine_m; (void)mine_l; (void)mine_a;
  if (nchunks == 1) return;

  // Last-arriving workgroup of this kv head merges every chunk.
  __shared__ uint32_t s_last;
  __threadfence();
  __syncthreads();
  if (t == 0) s_last = (atomicAdd(&counters[kvh], 1u) == nchunks - 1) ? 1u : 0u;
  __syncthreads();
  if (!s_last) return;
  __threadfence();
  if (t == 0) counters[kvh] = 0;  // ready for the next call on this stream

  __shared__ float s_w[1024];
  __shared__ float s_red[16][kHeadDim];
  __shared__ float s_scalar[2];
  for (int h = 0; h < REP; ++h) {
    const uint32_t qh = kvh_local * REP + h;
    const float* ml = part_ml + (part_base + (size_t)qh * max_chunks) * 2;
    // Maximum over chunks.
    float mx = -INFINITY;
    for (uint32_t c = t; c < nchunks; c += blockDim.x) mx = fmaxf(mx, ml[2 * c]);
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) mx = fmaxf(mx, __shfl_xor(mx, o, 64));
    if (lane == 0) s_m[wave][0] = mx;
    __syncthreads();
    mx = s_m[0][0];
    for (uint32_t w = 1; w < nwaves; ++w) mx = fmaxf(mx, s_m[w][0]);
    __syncthreads();
    // Chunk weights and the total.
    float L = 0.f;
    for (uint32_t c = t; c < nchunks; c += blockDim.x) {
      const float f = __expf(ml[2 * c] - mx);
      s_w[c] = f;
      L = fmaf(f, ml[2 * c + 1], L);
    }
#pragma unroll
    for (int o = 32; o >= 1; o >>= 1) L += __shfl_xor(L, o, 64);
    if (lane == 0) s_l[wave][0] = L;
    __syncthreads();
    if (t == 0) {
      float tot = 0.f;
      for (uint32_t w = 0; w < nwaves; ++w) tot += s_l[w][0];
      s_scalar[0] = tot;
    }
    // Weighted sum of chunk accumulators: 16 threads per chunk row (float4 each).
    const uint32_t dq = t & 15, cg = t >> 4, ngroups = blockDim.x >> 4;
    float4 a4 = make_float4(0.f, 0.f, 0.f, 0.f);
    const float* accs = part_acc + (part_base + (size_t)qh * max_chunks) * kHeadDim;
    for (uint32_t c = cg; c < nchunks; c += ngroups) {
      const float4 v = reinterpret_cast<const float4*>(accs + (size_t)c * kHeadDim)[dq];
      const float f = s_w[c];
      a4.x = fmaf(f, v.x, a4.x);
      a4.y = fmaf(f, v.y, a4.y);
      a4.z = fmaf(f, v.z, a4.z);
      a4.w = fmaf(f, v.w, a4.w);
    }
    s_red[cg][dq * 4 + 0] = a4.x;
    s_red[cg][dq * 4 + 1] = a4.y;
    s_red[cg][dq * 4 + 2] = a4.z;
    s_red[cg][dq * 4 + 3] = a4.w;
    __syncthreads();
    if (t < kHeadDim) {
      float sum = 0.f;
      for (uint32_t g2 = 0; g2 < ngroups; ++g2) sum += s_red[g2][t];
      out[(size_t)qh * kHeadDim + t] = sum / s_scalar[0];
    }
    __syncthreads();
  }
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

// Waves per workgroup: enough workgroups to cover the GPU first, then up to
// four waves (256 positions) per workgroup to keep the merge short.
static uint32_t attention_waves(uint32_t count, uint32_t kv_heads) {
  const uint32_t wave_units = (count + kChunk - 1) / kChunk;
  uint32_t w = 1;
  while (w < kMaxWaves && wave_units * kv_heads >= 2u * w * 256u) w <<= 1;
  return w;
}

uint32_t nd_attention_chunks(uint32_t count, uint32_t kv_heads) {
  const uint32_t per = kChunk * attention_waves(count, kv_heads);
  return (count + per - 1) / per;
}

// Upper bound for any visible count <= count (one wave per chunk at worst).
size_t nd_attention_partial_floats(uint32_t q_heads, uint32_t kv_heads, uint32_t count) {
  (void)kv_heads;
  return (size_t)q_heads * ((count + kChunk - 1) / kChunk) * (kHeadDim + 2);
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

struct AttnLaunch {
  const nd_kv* kv;
  uint32_t layer;
  const float* q;
  float* out;
  float* partials;
  uint32_t* counters;
  Visible vis;                 // used when positions == nullptr
  const uint32_t* positions;   // per-sequence query positions, or nullptr
  uint32_t seq_kv_heads;       // KV heads of one sequence
  uint32_t rep;                // query heads per KV head
  uint32_t batch;
  uint32_t max_chunks;
  uint32_t waves;
};

template <int REP, bool F32>
static void launch_attention(const AttnLaunch& a, hipStream_t s) {
  const size_t q_rows = (size_t)a.batch * a.seq_kv_heads * REP;
  float* part_acc = a.partials;
  float* part_ml = a.partials + q_rows * a.max_chunks * kHeadDim;
  hipLaunchKernelGGL((attention_kernel<REP, F32>), dim3(a.max_chunks, a.seq_kv_heads, a.batch),
                     dim3(64 * a.waves), 0, s, a.kv->k, a.kv->v, a.kv->ks, a.kv->vs, a.q, a.out,
                     part_acc, part_ml, a.counters, a.layer, a.kv->kv_heads, a.kv->alloc,
                     a.kv->sink, a.kv->window, a.vis, a.positions, a.seq_kv_heads, a.max_chunks,
                     0.125f);
}

template <bool F32>
static hipError_t launch_rep(const AttnLaunch& a, hipStream_t s) {
  switch (a.rep) {
    case 1: launch_attention<1, F32>(a, s); break;
    case 2: launch_attention<2, F32>(a, s); break;
    case 4: launch_attention<4, F32>(a, s); break;
    case 8: launch_attention<8, F32>(a, s); break;
    default: return hipErrorInvalidValue;
  }
  return hipGetLastError();
}

hipError_t nd_launch_attention(const nd_kv* kv, uint32_t layer, uint32_t position,
                               const float* q, uint32_t q_heads, float* out, float* partials,
                               uint32_t* counters, hipStream_t s) {
  const nd_visible nv = nd_kv_visible(kv, position);
  AttnLaunch a{};
  a.kv = kv;
  a.layer = layer;
  a.q = q;
  a.out = out;
  a.partials = partials;
  a.counters = counters;
  a.vis = Visible{nv.prefix, nv.recent_low, nv.count};
  a.positions = nullptr;
  a.seq_kv_heads = kv->kv_heads;
  a.rep = q_heads / kv->kv_heads;
  a.batch = 1;
  a.waves = attention_waves(nv.count, kv->kv_heads);
  a.max_chunks = (nv.count + kChunk * a.waves - 1) / (kChunk * a.waves);
  return kv->mode == ND_KV_FLOAT32 ? launch_rep<true>(a, s) : launch_rep<false>(a, s);
}

// Batched form: sequence z owns cache heads [z * seq_kv_heads, +seq_kv_heads)
// and queries q[z][seq_kv_heads * rep][64]; its query position is
// positions[z] (device memory), at most max_position.
hipError_t nd_launch_attention_batch(const nd_kv* kv, uint32_t layer, const uint32_t* positions,
                                     uint32_t batch, uint32_t seq_kv_heads, uint32_t rep,
                                     uint32_t max_position, const float* q, float* out,
                                     float* partials, uint32_t* counters, hipStream_t s) {
  const nd_visible nv = nd_kv_visible(kv, max_position);
  AttnLaunch a{};
  a.kv = kv;
  a.layer = layer;
  a.q = q;
  a.out = out;
  a.partials = partials;
  a.counters = counters;
  a.vis = Visible{nv.prefix, nv.recent_low, nv.count};
  a.positions = positions;
  a.seq_kv_heads = seq_kv_heads;
  a.rep = rep;
  a.batch = batch;
  a.waves = attention_waves(nv.count, seq_kv_heads * batch);
  a.max_chunks = (nv.count + kChunk * a.waves - 1) / (kChunk * a.waves);
  return kv->mode == ND_KV_FLOAT32 ? launch_rep<true>(a, s) : launch_rep<false>(a, s);
}

size_t nd_attention_batch_partial_floats(uint32_t batch, uint32_t seq_kv_heads, uint32_t rep,
                                         uint32_t max_count) {
  const uint32_t chunks = (max_count + kChunk - 1) / kChunk;  // bound for every launch
  return (size_t)batch * seq_kv_heads * rep * chunks * (kHeadDim + 2);
}
