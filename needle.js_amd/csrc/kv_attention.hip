// Int8 KV-cache append and single-query decode attention.
//
// Cache layout in HBM (per nd_kv): codes [layers][kv_heads][alloc][64] int8,
// scales [layers][kv_heads][alloc] f32, exactly NeedleRuntime's arrays
// (model/runtime.ts:186-204, 666-677).  A 64-dim code row is 64 bytes, so a
// 16-position x 64-dim tile is one contiguous 1 KiB run that a wave reads
// with 128-bit loads.
#include <mutex>

#include "nd_attention.hpp"
#include "nd_internal.hpp"
#include "nd_wave.hpp"

namespace {

using namespace nd::att;

constexpr uint32_t kWaves = 4;           // waves per attention workgroup
constexpr uint32_t kMinChunk = kWavePositions * kWaves;

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

// The attention launches' kernel: attention_body with its workgroup
// (chunk, KV head, row) taken from the grid.
template <int REP, bool F32, bool QB = false, int KW = 4, int TILES = 0, bool XL = false,
          bool STAMP = false>
__global__ __launch_bounds__(64 * KW) void attention_kernel(
    const void* __restrict__ Kc, const void* __restrict__ Vc, const float* __restrict__ Ks,
    const float* __restrict__ Vs, const float* __restrict__ Q, float* __restrict__ out,
    const float* __restrict__ gate, uint32_t gate_ld, float* __restrict__ part_acc,
    float* __restrict__ part_ml, uint32_t* __restrict__ counters, uint32_t layer,
    uint32_t kv_heads, uint32_t alloc, uint32_t sink, uint32_t window, Visible vis,
    const uint32_t* __restrict__ positions, uint32_t slot_space, uint32_t seq_kv_heads,
    uint32_t kv_stride_z, uint32_t chunk_positions, uint32_t max_chunks, float score_scale,
    uint32_t qrows, uint32_t qgroup, uint64_t* __restrict__ stamps) {
  attention_body<REP, F32, QB, KW, TILES, XL, STAMP, true>(
      0, 0, 0, Kc, Vc, Ks, Vs, Q, out, gate, gate_ld, part_acc, part_ml, counters, layer,
      kv_heads, alloc, sink, window, vis, positions, slot_space, seq_kv_heads, kv_stride_z,
      chunk_positions, max_chunks, score_scale, qrows, qgroup, stamps);
}

// Positions per chunk: the whole visible range when the (row, kv head) pairs
// alone give `target` workgroups, else split so that they do; at least one
// tile per wave.  Splitting costs a publish + count + merge round trip at the
// end, yet more, smaller workgroups win: a single query row aims at 256
// workgroups (32 chunks of 256 per head at 8 heads x 8192: 7.0 us per call
// with the XCD-local merge, 7.95 with the agent-scope one elected in groups
// of 8, 8.9 with that at 128 workgroups and 10.4 at 64) and batches at 8192
// (64 sequences x 8 heads at contexts up to 2176: chunks of 256, 20.3 us per
// layer, vs 21.6 with chunks of 512 at 4096 workgroups; the XCD-local
// layout with each pair's chunks dispatched together: 0.440-0.442 ms per
// decode step against 0.444, chunk-major 0.453).
// One tile per wave also runs the leanest kernel form (73 VGPRs: 6 waves
// per SIMD).
constexpr uint32_t kTargetSingle = 256, kTargetBatch = 8192;
constexpr uint32_t kMaxChunks = 64;  // the merge holds one chunk per lane
static_assert(1 + kMaxChunks / kChunkGroup <= kAttnCounterStride, "group counters fit the stride");
uint32_t chunk_positions_for(uint32_t max_count, uint32_t pairs, uint32_t target,
                             uint32_t min_chunk = kMinChunk) {
  uint32_t want_chunks = pairs >= target ? 1 : (target + pairs - 1) / pairs;
  // Up to two tiles per wave stay in one chunk: the merge round trips cost
  // more than streaming the second, prefetched tile (5.7 vs 6.3 us at 512
  // positions x 8 heads); beyond that, splitting to `target` workgroups is
  // fastest.
  if (max_count <= 2 * kMinChunk) want_chunks = 1;
  if (want_chunks > kMaxChunks) want_chunks = kMaxChunks;
  uint32_t cp = (max_count + want_chunks - 1) / want_chunks;
  cp = (cp + min_chunk - 1) / min_chunk * min_chunk;
  return cp < min_chunk ? min_chunk : cp;
}

struct AttnLaunch {
  const nd_kv* kv;
  uint32_t layer;
  const float* q;
  float* out;
  const float* gate;           // optional: out *= sigmoid(gate); row z at gate + z * gate_ld
  uint32_t gate_ld;
  float* partials;
  uint32_t* counters;          // batch * seq_kv_heads zeros, used when a row has >1 chunk
  Visible vis;                 // used when positions == nullptr
  const uint32_t* positions;   // per-sequence query positions, or nullptr
  uint32_t slot_space;         // one row: iterate cache slots, mask by *positions
  uint32_t seq_kv_heads;       // KV heads of one sequence
  uint32_t kv_stride_z;        // cache-head offset between query rows z
  uint32_t rep;                // query heads per KV head
  uint32_t batch;
  uint32_t max_count;          // bound on every sequence's visible count
  bool qblock;                 // query blocks of a prefill whose positions see [0, position]
  uint64_t* stamps;            // measurement form: 8 stamps per workgroup, or nullptr
  uint32_t stamp_capacity;     // workgroups the stamps hold
  uint32_t* stamp_workgroups;  // out: workgroups launched
};

// Causal prefill attention on MFMA (a prefill whose positions all see [0,
// position] in their own slots; int8 cache).  Workgroup = (block of 64 query
// rows, query head h, KV head h / rep), 16 waves in four groups: wave w
// takes rows [z0 + 16 (w % 4), +16), lane l the row 16 (w % 4) + l % 16, and
// group g = w / 4 the key blocks g, g + 4, ... (64 keys each), so each group
// walks a quarter of the row block's keys (the causal triangle gives the
// last row blocks the most); the four online-softmax states merge through
// LDS at the end.  Each group streams its key blocks through its own pair of
// LDS buffers, converting the codes to fp16 once on the way in (K as
// stored, V transposed to [dim][key]), one barrier per step.  Per block and
// wave:
//   S^T = K Q^T on v_mfma_f32_16x16x32_f16: A = K codes (row = key, exact in
//   fp16), B = Q^T split into fp16 halves hi + lo of q * 2^-e (e: the row's
//   largest magnitude, < 2^e), which hold q to 2^-24 of the row maximum; the
//   product lands as lane l holding keys 4 (l / 16) + c of each 16-key tile
//   for its own row;
//   scores in base 2: (S * (k_scale / 8 * log2 e)) * 2^e, causal mask,
//   online softmax in fp32 with v_exp_f32 (2^x; results below 2^-126 flush
//   to zero, as with __expf) -- NeedleRuntime.#attention
//   (model/runtime.ts:719-786, softmaxInPlace model/math.ts:46-60) with its
//   exponentials taken as 2^(x log2 e);
//   O^T += V^T P'^T: B = P'^T with p' = p * v_scale * 2^f (fp16 halves; f
//   puts the largest v_scale of the visible keys below 2^15 so that both
//   halves stay normal down to 2^-18 of it), which is exactly the layout the
//   S^T product left in the lane (8 keys per lane, the A operand reads V^T at
//   the same keys); A = V^T codes (row = dim).
// The output row is O / (l 2^f), gated when `gate` is set (runtime.ts:503-507).
constexpr uint32_t kPfRows = 64, kPfKeys = 64, kPfGroups = 4, kPfThreads = 256 * kPfGroups;
constexpr uint32_t kKStrideH = 72;   // halves per key row of K in LDS (16-byte aligned rows)
constexpr uint32_t kVtStrideH = 68;  // halves per dim row of V^T in LDS (8-byte aligned rows)
struct PfBuf {
  _Float16 k[kPfKeys * kKStrideH];
  _Float16 vt[kHeadDim * kVtStrideH];
  float ks[kPfKeys];  // k_scale / 8 * log2 e
  float vs[kPfKeys];  // v_scale * 2^f
};

__global__ __launch_bounds__(kPfThreads) void prefill_attention_mfma_kernel(
    const int8_t* __restrict__ Kc, const int8_t* __restrict__ Vc, const float* __restrict__ Ks,
    const float* __restrict__ Vs, const float* __restrict__ Q, float* __restrict__ out,
    const float* __restrict__ gate, uint32_t gate_ld, uint32_t layer, uint32_t kv_heads,
    uint32_t alloc, const uint32_t* __restrict__ positions, uint32_t qrows, uint32_t q_heads,
    uint32_t rep, float score_scale) {
  using nd::half8;
  using nd::float4v;
  using nd::u32x2;
  typedef _Float16 half4 __attribute__((ext_vector_type(4)));
  __shared__ __align__(16) PfBuf s_buf[kPfGroups][2];  // [group][buffer]
  __shared__ uint32_t s_top[kPfThreads / 64];
  __shared__ float s_vmax[kPfThreads / 64];
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t grp = wave >> 2, wq = wave & 3, tg = t & 255;
  const uint32_t r16 = lane & 15, kb = lane >> 4;
  const uint32_t h = blockIdx.y, kvh = h / rep;
  const uint32_t z0 = blockIdx.x * kPfRows;
  const size_t head_base = ((size_t)layer * kv_heads + kvh) * alloc;

  // Keys [0, top): top = 1 + the largest position of the block's rows.
  uint32_t my_top = 0;
  if (t < kPfRows && z0 + t < qrows) my_top = positions[z0 + t] + 1;
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) my_top = max(my_top, (uint32_t)__shfl_xor((int)my_top, o, 64));
  if (lane == 0) s_top[wave] = my_top;
  // This lane's query row and its q values: dims 32 s + 8 kb + [0, 8).
  const uint32_t zq = z0 + 16 * wq + r16;
  const bool q_ok = zq < qrows;
  const uint32_t pos = q_ok ? positions[zq] : 0;
  const float* qp = Q + ((size_t)(q_ok ? zq : 0) * q_heads + h) * kHeadDim + 8 * kb;
  float qv[2][8];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2) {
    const float4 a = *reinterpret_cast<const float4*>(qp + 32 * s2);
    const float4 b = *reinterpret_cast<const float4*>(qp + 32 * s2 + 4);
    qv[s2][0] = a.x; qv[s2][1] = a.y; qv[s2][2] = a.z; qv[s2][3] = a.w;
    qv[s2][4] = b.x; qv[s2][5] = b.y; qv[s2][6] = b.z; qv[s2][7] = b.w;
  }
  // The smallest position of the wave's rows: blocks wholly below it need no mask.
  uint32_t wmin = q_ok ? pos : 0;
#pragma unroll
  for (int o = 8; o >= 1; o >>= 1) wmin = min(wmin, (uint32_t)__shfl_xor((int)wmin, o, 64));
  wmin = __builtin_amdgcn_readfirstlane(wmin);
  __syncthreads();
  uint32_t top = 0;
#pragma unroll
  for (uint32_t w = 0; w < kPfThreads / 64; ++w) top = max(top, s_top[w]);
  if (top > alloc || top == 0) return;  // validated on entry; stay in bounds
  const uint32_t nblocks = (top + kPfKeys - 1) / kPfKeys;

  // The split of q: the row maximum over the four lanes holding the row.
  float qmax = 0.f;
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int e = 0; e < 8; ++e) qmax = fmaxf(qmax, fabsf(qv[s2][e]));
  qmax = nd::max_xor<16>(qmax);
  qmax = nd::max_xor<32>(qmax);
  int qe = 0;
  if (qmax > 0.f && qmax <= 3.4028235e38f) frexpf(qmax, &qe);  // qmax < 2^qe
  const float qdown = ldexpf(1.f, -qe), qup = ldexpf(1.f, qe);
  half8 qh[2], ql[2];
#pragma unroll
  for (int s2 = 0; s2 < 2; ++s2)
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      const float v = qv[s2][e] * qdown;
      const _Float16 hv = (_Float16)v;
      qh[s2][e] = hv;
      ql[s2][e] = (_Float16)(v - (float)hv);
    }

  // The largest v_scale of the visible keys sets the p' scale 2^f.
  float vmax = 0.f;
  for (uint32_t k = t; k < top; k += kPfThreads) vmax = fmaxf(vmax, Vs[head_base + k]);
#pragma unroll
  for (int o = 32; o >= 1; o >>= 1) vmax = fmaxf(vmax, __shfl_xor(vmax, o, 64));
  if (lane == 0) s_vmax[wave] = vmax;
  __syncthreads();
  float vsmax = 0.f;
#pragma unroll
  for (uint32_t w = 0; w < kPfThreads / 64; ++w) vsmax = fmaxf(vsmax, s_vmax[w]);
  int fe = 0;
  if (vsmax > 0.f && vsmax <= 3.4028235e38f) frexpf(vsmax, &fe);  // vsmax < 2^fe
  const float pup = ldexpf(1.f, 15 - fe), pdown = ldexpf(1.f, fe - 15);
  const float ks_mul = score_scale * 1.4426950408889634f;  // scores in base 2

  // Block loads of the group: thread tg takes key tg / 4, bytes [16 (tg %
  // 4), +16) of its K and V rows (keys past top read the last visible slot;
  // they are masked).
  const uint32_t lkey = tg >> 2, lpart = tg & 3;
  uint4 kreg, vreg;
  float ksr = 0.f, vsr = 0.f;
  auto load_block = [&](uint32_t b) {
    const uint32_t key = min(b * kPfKeys + lkey, top - 1);
    const size_t row = head_base + key;
    kreg = *reinterpret_cast<const uint4*>(Kc + row * kHeadDim + 16 * lpart);
    vreg = *reinterpret_cast<const uint4*>(Vc + row * kHeadDim + 16 * lpart);
    if (tg < kPfKeys) {
      const size_t srow = head_base + min(b * kPfKeys + tg, top - 1);
      ksr = Ks[srow];
      vsr = Vs[srow];
    }
  };
  auto store_block = [&](PfBuf& B) {
    const half8 k0 = nd::codes_to_half(u32x2{kreg.x, kreg.y});
    const half8 k1 = nd::codes_to_half(u32x2{kreg.z, kreg.w});
    *reinterpret_cast<half8*>(&B.k[lkey * kKStrideH + 16 * lpart]) = k0;
    *reinterpret_cast<half8*>(&B.k[lkey * kKStrideH + 16 * lpart + 8]) = k1;
    const half8 v0 = nd::codes_to_half(u32x2{vreg.x, vreg.y});
    const half8 v1 = nd::codes_to_half(u32x2{vreg.z, vreg.w});
#pragma unroll
    for (int e = 0; e < 8; ++e) {
      B.vt[(16 * lpart + e) * kVtStrideH + lkey] = v0[e];
      B.vt[(16 * lpart + 8 + e) * kVtStrideH + lkey] = v1[e];
    }
    if (tg < kPfKeys) {
      B.ks[tg] = ksr * ks_mul;
      B.vs[tg] = vsr * pup;
    }
  };
  const uint32_t steps = (nblocks + kPfGroups - 1) / kPfGroups;  // the groups step together
  if (grp < nblocks) {
    load_block(grp);
    store_block(s_buf[grp][0]);
  }
  nd::lds_barrier();

  float m = -INFINITY, l = 0.f;  // m in base 2
  float4v o[4] = {};
  for (uint32_t i = 0; i < steps; ++i) {
    const uint32_t b = kPfGroups * i + grp;
    const bool has = b < nblocks, has_next = b + kPfGroups < nblocks;
    PfBuf& B = s_buf[grp][i & 1];
    if (has_next) load_block(b + kPfGroups);
    if (has) {
      const uint32_t k0 = b * kPfKeys;
      // S^T tiles j: keys k0 + 16 j + 4 kb + c of this lane's row.
      float4v sc[4];
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        sc[j] = float4v{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int s2 = 0; s2 < 2; ++s2) {
          const half8 ka =
              *reinterpret_cast<const half8*>(&B.k[(16 * j + r16) * kKStrideH + 32 * s2 + 8 * kb]);
          sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, qh[s2], sc[j], 0, 0, 0);
          sc[j] = __builtin_amdgcn_mfma_f32_16x16x32_f16(ka, ql[s2], sc[j], 0, 0, 0);
        }
      }
      const bool masked = k0 + kPfKeys - 1 > wmin;  // uniform over the wave
      float bmax = -INFINITY;
#pragma unroll
      for (int j = 0; j < 4; ++j) {
        const float4 ks4 = *reinterpret_cast<const float4*>(&B.ks[16 * j + 4 * kb]);
        const float ksv[4] = {ks4.x, ks4.y, ks4.z, ks4.w};
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          float v = (sc[j][c] * ksv[c]) * qup;
          if (masked) v = (q_ok && k0 + 16 * j + 4 * kb + c <= pos) ? v : -INFINITY;
          sc[j][c] = v;
          bmax = fmaxf(bmax, v);
        }
      }
      bmax = nd::max_xor<16>(bmax);
      bmax = nd::max_xor<32>(bmax);
      const float m_new = fmaxf(m, bmax);
      // While no key has been visible m_new is -inf: subtract 0 instead, so
      // that masked scores give exp2(-inf) = 0 and alpha = 1.
      const float m_sub = m_new == -INFINITY ? 0.f : m_new;
      const float alpha = __builtin_amdgcn_exp2f(m - m_sub);
      m = m_new;
      l *= alpha;
#pragma unroll
      for (int d = 0; d < 4; ++d) o[d] *= alpha;
#pragma unroll
      for (int j = 0; j < 4; ++j)
#pragma unroll
        for (int c = 0; c < 4; ++c) {
          const float e = __builtin_amdgcn_exp2f(sc[j][c] - m_sub);
          sc[j][c] = e;
          l += e;
        }
      // O^T += V^T P'^T over the two 32-key steps.
#pragma unroll
      for (int s2 = 0; s2 < 2; ++s2) {
        const float4 va = *reinterpret_cast<const float4*>(&B.vs[32 * s2 + 4 * kb]);
        const float4 vb = *reinterpret_cast<const float4*>(&B.vs[32 * s2 + 16 + 4 * kb]);
        const float pv[8] = {sc[2 * s2][0] * va.x,     sc[2 * s2][1] * va.y,
                             sc[2 * s2][2] * va.z,     sc[2 * s2][3] * va.w,
                             sc[2 * s2 + 1][0] * vb.x, sc[2 * s2 + 1][1] * vb.y,
                             sc[2 * s2 + 1][2] * vb.z, sc[2 * s2 + 1][3] * vb.w};
        // hi = pv rounded toward zero to fp16, lo = fp16 of the (exact f32)
        // remainder: |pv - hi - lo| <= 2^-22 |pv| while lo is normal.
        half8 ph, pl;
#pragma unroll
        for (int e = 0; e < 8; e += 2) {
          const auto hv = __builtin_amdgcn_cvt_pkrtz(pv[e], pv[e + 1]);
          const auto lv = __builtin_amdgcn_cvt_pkrtz(pv[e] - (float)hv[0], pv[e + 1] - (float)hv[1]);
          ph[e] = hv[0];
          ph[e + 1] = hv[1];
          pl[e] = lv[0];
          pl[e + 1] = lv[1];
        }
#pragma unroll
        for (int d = 0; d < 4; ++d) {
          const _Float16* vt = &B.vt[(16 * d + r16) * kVtStrideH + 32 * s2 + 4 * kb];
          const half4 lo4 = *reinterpret_cast<const half4*>(vt);
          const half4 hi4 = *reinterpret_cast<const half4*>(vt + 16);
          const half8 va8 = {lo4[0], lo4[1], lo4[2], lo4[3], hi4[0], hi4[1], hi4[2], hi4[3]};
          o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va8, ph, o[d], 0, 0, 0);
          o[d] = __builtin_amdgcn_mfma_f32_16x16x32_f16(va8, pl, o[d], 0, 0, 0);
        }
      }
    }
    if (has_next) store_block(s_buf[grp][(i + 1) & 1]);
    nd::lds_barrier();
  }
  // l over the row's four lanes; o[d][c] is dim 16 d + 4 kb + c of the row.
  l = nd::sum_xor<16>(l);
  l = nd::sum_xor<32>(l);
  // Merge: groups 1.. leave (m, l, o) in LDS (the key buffers are free),
  // group 0 combines them with its own and stores the row.
  float* xm = reinterpret_cast<float*>(&s_buf[0][0]);  // [group - 1][wq][18][64]
  static_assert((kPfGroups - 1) * 4 * 18 * 64 * 4 <= sizeof(PfBuf) * kPfGroups * 2, "merge fits");
  if (grp > 0) {
    float* dst = xm + ((grp - 1) * 4 + wq) * 18 * 64 + lane;
    dst[0] = m;
    dst[64] = l;
#pragma unroll
    for (int d = 0; d < 4; ++d)
#pragma unroll
      for (int c = 0; c < 4; ++c) dst[(2 + 4 * d + c) * 64] = o[d][c];
  }
  nd::lds_barrier();
  if (grp > 0 || !q_ok) return;
  {
    float mg[kPfGroups], lg[kPfGroups];
    mg[0] = m;
    lg[0] = l;
    float mt = m;
#pragma unroll
    for (uint32_t g = 1; g < kPfGroups; ++g) {
      const float* src = xm + ((g - 1) * 4 + wq) * 18 * 64 + lane;
      mg[g] = src[0];
      lg[g] = src[64];
      mt = fmaxf(mt, mg[g]);
    }
    float ag[kPfGroups];
#pragma unroll
    for (uint32_t g = 0; g < kPfGroups; ++g) ag[g] = mg[g] == -INFINITY ? 0.f : __builtin_amdgcn_exp2f(mg[g] - mt);
    l = l * ag[0];
#pragma unroll
    for (int d = 0; d < 4; ++d) o[d] *= ag[0];
#pragma unroll
    for (uint32_t g = 1; g < kPfGroups; ++g) {
      const float* src = xm + ((g - 1) * 4 + wq) * 18 * 64 + lane;
      l += lg[g] * ag[g];
#pragma unroll
      for (int d = 0; d < 4; ++d)
#pragma unroll
        for (int c = 0; c < 4; ++c) o[d][c] += src[(2 + 4 * d + c) * 64] * ag[g];
    }
  }
  const size_t obase = ((size_t)zq * q_heads + h) * kHeadDim;
#pragma unroll
  for (int d = 0; d < 4; ++d) {
    float r[4];
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      r[c] = (o[d][c] * pdown) / l;
      if (gate) r[c] *= gate_factor(gate[(size_t)zq * gate_ld + h * kHeadDim + 16 * d + 4 * kb + c]);
    }
    *reinterpret_cast<float4*>(out + obase + 16 * d + 4 * kb) = make_float4(r[0], r[1], r[2], r[3]);
  }
}

template <int REP, bool F32>
hipError_t launch_attention(const AttnLaunch& a, hipStream_t s) {
  if constexpr (REP == 2 && !F32) {
    // The gated single row over a ring that fits one chunk: eight-wave
    // workgroups, the instance the resident Needle 2 step's fused layer
    // launch runs (the same bits either way).
    if (a.slot_space && a.batch == 1 && a.max_count <= kGatedChunk && !a.stamps) {
      hipLaunchKernelGGL((attention_kernel<2, false, false, 8, 1, false>),
                         dim3(1, a.seq_kv_heads, 1), dim3(64 * 8), 0, s, a.kv->k, a.kv->v,
                         a.kv->ks, a.kv->vs, a.q, a.out, a.gate, a.gate_ld, a.partials,
                         a.partials, a.counters, a.layer, a.kv->kv_heads, a.kv->alloc, a.kv->sink,
                         a.kv->window, a.vis, a.positions, a.slot_space, a.seq_kv_heads,
                         a.kv_stride_z, kGatedChunk, 1u, 0.125f, a.batch, 1u, nullptr);
      return hipGetLastError();
    }
  }
  if constexpr ((REP == 1 || REP == 2) && !F32) {
    if (a.qblock) {
      hipLaunchKernelGGL(prefill_attention_mfma_kernel,
                         dim3((a.batch + kPfRows - 1) / kPfRows, a.seq_kv_heads * REP),
                         dim3(kPfThreads), 0, s, reinterpret_cast<const int8_t*>(a.kv->k),
                         reinterpret_cast<const int8_t*>(a.kv->v), a.kv->ks, a.kv->vs, a.q, a.out,
                         a.gate, a.gate_ld, a.layer, a.kv->kv_heads, a.kv->alloc, a.positions,
                         a.batch, a.seq_kv_heads * REP, (uint32_t)REP, 0.125f);
      return hipGetLastError();
    }
    // Query blocks: 4 rows per workgroup (4 positions x 1 head, or 2 x 2).
    if (a.qblock) {
      constexpr int kQb = 4;
      hipLaunchKernelGGL((attention_kernel<kQb, false, true>),
                         dim3(1, a.seq_kv_heads, (a.batch + kQb / REP - 1) / (kQb / REP)),
                         dim3(64 * kWaves), 0, s, a.kv->k, a.kv->v, a.kv->ks, a.kv->vs, a.q,
                         a.out, a.gate, a.gate_ld, nullptr, nullptr, nullptr, a.layer,
                         a.kv->kv_heads, a.kv->alloc, a.kv->sink, a.kv->window, a.vis,
                         a.positions, 0u, a.seq_kv_heads, 0u, a.max_count, 1u, 0.125f, a.batch,
                         (uint32_t)REP, nullptr);
      return hipGetLastError();
    }
  }
  const uint32_t cp = chunk_positions_for(a.max_count, a.batch * a.seq_kv_heads,
                                          a.batch == 1 ? kTargetSingle : kTargetBatch);
  const uint32_t max_chunks = (a.max_count + cp - 1) / cp;
  const uint32_t hq = a.seq_kv_heads * REP;
  float* part_acc = a.partials;
  float* part_ml = a.partials + (size_t)a.batch * hq * max_chunks * kHeadDim;
  // Tiles per wave: cp / kMinChunk (cp is a multiple of it).
  const uint32_t tiles = cp / kMinChunk;
  // The XCD-local forms need the dispatcher's placement (workgroups of one
  // L % 8 on one XCD), confirmed per device when the context is created;
  // without it the chunks merge at the agent coherence point (last form).
  const bool xcd = nd_xcd_local();
  if (xcd && max_chunks > 1 && (a.batch > 1 || a.seq_kv_heads * max_chunks < kTargetSingle)) {
    // Two-wave workgroups on 128-position chunks.  One row whose
    // 256-position chunks leave the launch short of kTargetSingle workgroups
    // (8 heads x 2048: 64) gets twice as many (5.85 against 6.28 us at 2048;
    // at 8192, already 256 workgroups, the four-wave form stays faster).  A
    // batch takes them whenever its rows fit 64 such chunks: ragged rows
    // spread more evenly (64 rows of 32..2048 positions: 0.397 against
    // 0.401 ms per decode step).
    constexpr uint32_t kHalf = kWavePositions * 2;
    const uint32_t cp2 = a.batch == 1
                             ? chunk_positions_for(a.max_count, a.seq_kv_heads, kTargetSingle, kHalf)
                             : kHalf;
    const uint32_t mc2 = (a.max_count + cp2 - 1) / cp2;
    if (cp2 == kHalf && mc2 <= kMaxChunks) {
      if (a.stamps) return hipErrorInvalidValue;  // no measurement form of the two-wave kernel
      float* pm2 = a.partials + (size_t)a.batch * hq * mc2 * kHeadDim;
      const uint32_t gpx = (a.batch * a.seq_kv_heads + 7) / 8;
      hipLaunchKernelGGL((attention_kernel<REP, F32, false, 2, 1, true>), dim3(8 * gpx * mc2),
                         dim3(64 * 2), 0, s, a.kv->k, a.kv->v, a.kv->ks, a.kv->vs, a.q, a.out,
                         a.gate, a.gate_ld, part_acc, pm2, a.counters, a.layer, a.kv->kv_heads,
                         a.kv->alloc, a.kv->sink, a.kv->window, a.vis, a.positions,
                         a.slot_space, a.seq_kv_heads, a.kv_stride_z, cp2, mc2, 0.125f, a.batch,
                         1u, nullptr);
      return hipGetLastError();
    }
  }
  if (xcd && max_chunks > 1) {
    // Rows split into chunks: the XCD-local merge (grid laid out per XCD,
    // see attention_kernel).
    auto kernel = tiles == 1   ? attention_kernel<REP, F32, false, kWaves, 1, true>
                  : tiles == 2 ? attention_kernel<REP, F32, false, kWaves, 2, true>
                               : attention_kernel<REP, F32, false, kWaves, 0, true>;
    const uint32_t gpx = (a.batch * a.seq_kv_heads + 7) / 8;
    if (a.stamps) {  // the measurement form of the same launch (one tile per wave)
      if (tiles != 1 || 8 * gpx * max_chunks > a.stamp_capacity) return hipErrorInvalidValue;
      kernel = attention_kernel<REP, F32, false, kWaves, 1, true, true>;
      *a.stamp_workgroups = 8 * gpx * max_chunks;
    }
    hipLaunchKernelGGL(kernel, dim3(8 * gpx * max_chunks), dim3(64 * kWaves), 0, s, a.kv->k,
                       a.kv->v, a.kv->ks, a.kv->vs, a.q, a.out, a.gate, a.gate_ld, part_acc,
                       part_ml, a.counters, a.layer, a.kv->kv_heads, a.kv->alloc, a.kv->sink,
                       a.kv->window, a.vis, a.positions, a.slot_space, a.seq_kv_heads,
                       a.kv_stride_z, cp, max_chunks, 0.125f, a.batch, 1u, a.stamps);
    return hipGetLastError();
  }
  if (a.stamps) return hipErrorInvalidValue;
  if constexpr (REP <= 2 && !F32) {
    if (max_chunks == 1 && tiles == 2) {
      // One 512-position chunk per (row, KV head): eight waves of one tile
      // each instead of four of two.
      hipLaunchKernelGGL((attention_kernel<REP, F32, false, 8, 1>),
                         dim3(1, a.seq_kv_heads, a.batch), dim3(64 * 8), 0, s, a.kv->k, a.kv->v,
                         a.kv->ks, a.kv->vs, a.q, a.out, a.gate, a.gate_ld, part_acc, part_ml,
                         a.counters, a.layer, a.kv->kv_heads, a.kv->alloc, a.kv->sink,
                         a.kv->window, a.vis, a.positions, a.slot_space, a.seq_kv_heads,
                         a.kv_stride_z, cp, max_chunks, 0.125f, a.batch, 1u, nullptr);
      return hipGetLastError();
    }
  }
  auto kernel = tiles == 1   ? attention_kernel<REP, F32, false, kWaves, 1>
                : tiles == 2 ? attention_kernel<REP, F32, false, kWaves, 2>
                             : attention_kernel<REP, F32, false, kWaves, 0>;
  hipLaunchKernelGGL(kernel, dim3(max_chunks, a.seq_kv_heads, a.batch),
                     dim3(64 * kWaves), 0, s, a.kv->k, a.kv->v, a.kv->ks, a.kv->vs, a.q, a.out,
                     a.gate, a.gate_ld, part_acc, part_ml, a.counters, a.layer, a.kv->kv_heads, a.kv->alloc,
                     a.kv->sink, a.kv->window, a.vis, a.positions, a.slot_space, a.seq_kv_heads,
                     a.kv_stride_z,
                     cp, max_chunks, 0.125f, a.batch, 1u, nullptr);
  return hipGetLastError();
}

template <bool F32>
hipError_t launch_rep(const AttnLaunch& a, hipStream_t s) {
  switch (a.rep) {
    case 1: return launch_attention<1, F32>(a, s);
    case 2: return launch_attention<2, F32>(a, s);
    case 4: return launch_attention<4, F32>(a, s);
    case 8: return launch_attention<8, F32>(a, s);
    default: return hipErrorInvalidValue;
  }
}

}  // namespace

// ------------------------------------------- fixed scratch (no allocation)
//
// The allocation-free attention entry point keeps its chunk partials and
// arrival counters in this array instead of a context buffer.  Every GPU the
// library runs on holds its own copy until the process ends.  Host code never
// passes `scratch` itself to a kernel (in host code it names a host-side
// stand-in): nd_attention_scratch_setup looks up each device's address once,
// and launches take that address.  The counters are cleared at set-up and
// every launch leaves them at zero; the partials are written before they are
// read.  Launches that use the scratch on one GPU must not overlap.
static_assert(kMaxChunks == 64, "the scratch holds 64 chunks per query head");
static __device__ __align__(256) uint32_t scratch[kStaticAttnWords];

namespace {
constexpr int kMaxScratchDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_dev[kMaxScratchDevices] = {};
}  // namespace

hipError_t nd_attention_scratch_setup(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return hipErrorInvalidDevice;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (g_scratch_dev[device]) return hipSuccess;
  void* p = nullptr;
  hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
  if (e != hipSuccess) return e;
  if (!p) return hipErrorInvalidSymbol;
  e = hipMemset(p, 0, kStaticAttnWords * sizeof(uint32_t));
  if (e == hipSuccess) e = hipDeviceSynchronize();
  if (e != hipSuccess) return e;
  g_scratch_dev[device] = p;
  return hipSuccess;
}

void* nd_attention_scratch(int device) {
  if (device < 0 || device >= kMaxScratchDevices) return nullptr;
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  return g_scratch_dev[device];
}

nd_visible nd_kv_visible(const nd_kv* kv, uint32_t position) {
  nd_visible v;
  v.prefix = kv->sink < position + 1 ? kv->sink : position + 1;
  v.recent_low = v.prefix;
  if (kv->window > 0 && position + 1 > kv->window && position + 1 - kv->window > v.prefix)
    v.recent_low = position + 1 - kv->window;
  v.count = v.prefix + (position - v.recent_low + 1);
  return v;
}

uint32_t nd_attention_chunks(uint32_t count, uint32_t kv_heads) {
  const uint32_t cp = chunk_positions_for(count, kv_heads, kTargetSingle);
  return (count + cp - 1) / cp;
}

// Partials for any launch with visible counts <= count (chunks are at least
// kMinChunk positions).
// A single row may take 128-position chunks (two-wave workgroups), batches
// 256-position ones.
size_t nd_attention_partial_floats(uint32_t q_heads, uint32_t kv_heads, uint32_t count) {
  (void)kv_heads;
  const uint32_t unit = kWavePositions * 2;
  return (size_t)q_heads * ((count + unit - 1) / unit) * (kHeadDim + 2);
}

size_t nd_attention_batch_partial_floats(uint32_t batch, uint32_t seq_kv_heads, uint32_t rep,
                                         uint32_t max_count) {
  const uint32_t unit = kWavePositions * 2;  // the two-wave form's chunks
  return (size_t)batch * seq_kv_heads * rep * ((max_count + unit - 1) / unit) * (kHeadDim + 2);
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

hipError_t nd_launch_attention(const nd_kv* kv, uint32_t layer, uint32_t position,
                               const float* q, uint32_t q_heads, float* out, float* partials,
                               uint32_t* counters, hipStream_t s, uint64_t* stamps,
                               uint32_t stamp_capacity, uint32_t* stamp_workgroups) {
  const nd_visible nv = nd_kv_visible(kv, position);
  AttnLaunch a{};
  a.stamps = stamps;
  a.stamp_capacity = stamp_capacity;
  a.stamp_workgroups = stamp_workgroups;
  a.kv = kv;
  a.layer = layer;
  a.q = q;
  a.out = out;
  a.partials = partials;
  a.counters = counters;
  a.vis = Visible{nv.prefix, nv.recent_low, nv.count};
  a.positions = nullptr;
  a.seq_kv_heads = kv->kv_heads;
  a.kv_stride_z = 0;
  a.rep = q_heads / kv->kv_heads;
  a.batch = 1;
  a.max_count = nv.count;
  return kv->mode == ND_KV_FLOAT32 ? launch_rep<true>(a, s) : launch_rep<false>(a, s);
}

// Batched form: query row z reads cache heads [z * kv_stride_z, +seq_kv_heads)
// (kv_stride_z = seq_kv_heads for a batch of sequences, 0 for the positions of
// one prefill) with queries q[z][seq_kv_heads * rep][64] at position
// positions[z] (device memory), at most max_position.
hipError_t nd_launch_attention_batch(const nd_kv* kv, uint32_t layer, const uint32_t* positions,
                                     uint32_t batch, uint32_t seq_kv_heads, uint32_t kv_stride_z,
                                     uint32_t rep, uint32_t max_position, const float* q,
                                     float* out, float* partials, uint32_t* counters,
                                     hipStream_t s, const float* gate, uint32_t gate_ld) {
  const nd_visible nv = nd_kv_visible(kv, max_position);
  AttnLaunch a{};
  a.kv = kv;
  a.layer = layer;
  a.q = q;
  a.out = out;
  a.gate = gate;
  a.gate_ld = gate_ld;
  a.partials = partials;
  a.counters = counters;
  a.vis = Visible{nv.prefix, nv.recent_low, nv.count};
  a.positions = positions;
  a.seq_kv_heads = seq_kv_heads;
  a.kv_stride_z = kv_stride_z;
  a.rep = rep;
  a.batch = batch;
  a.max_count = nv.count;
  // Every position sees [0, position] when no window is outgrown (positions
  // below the window also sit in their own slots).
  a.qblock = kv_stride_z == 0 && (kv->window == 0 || max_position < kv->window) &&
             (rep == 1 || rep == 2) && kv->mode != ND_KV_FLOAT32 && batch >= 64;
  return kv->mode == ND_KV_FLOAT32 ? launch_rep<true>(a, s) : launch_rep<false>(a, s);
}

hipError_t nd_launch_attention_gated(const nd_kv* kv, uint32_t layer, const uint32_t* position,
                                     uint32_t max_position, const float* q, uint32_t q_heads,
                                     const float* gate, float* out, float* partials,
                                     uint32_t* counters, hipStream_t s) {
  (void)max_position;  // slot order covers every slot a position can see
  AttnLaunch a{};
  a.kv = kv;
  a.layer = layer;
  a.q = q;
  a.out = out;
  a.gate = gate;
  a.partials = partials;
  a.counters = counters;
  a.vis = Visible{kv->alloc, kv->alloc, kv->alloc};
  a.positions = position;
  a.slot_space = 1;
  a.seq_kv_heads = kv->kv_heads;
  a.kv_stride_z = 0;
  a.rep = q_heads / kv->kv_heads;
  a.batch = 1;
  a.max_count = kv->alloc;
  return kv->mode == ND_KV_FLOAT32 ? launch_rep<true>(a, s) : launch_rep<false>(a, s);
}
