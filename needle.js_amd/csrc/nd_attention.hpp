// Single-query decode attention over an int8 (or float32) KV cache: the
// workgroup body shared by the attention launches (kv_attention.hip) and the
// fused layer launch of the resident Needle 2 step (needle2.hip), so that
// both compute the same bits.  Cache layout and arithmetic are described
// with attention_body below.
#pragma once

#include "nd_internal.hpp"
#include "nd_wave.hpp"

namespace nd {
namespace att {

constexpr uint32_t kHeadDim = 64;
constexpr uint32_t kWavePositions = 64;  // positions a wave handles per iteration
constexpr uint32_t kChunkGroup = 8;      // chunks per first-level arrival counter
// The gated single-row attention of a ring that fits one chunk runs
// eight-wave workgroups over kGatedChunk positions (its launch and the fused
// layer launch of the resident Needle 2 step use the same instance).
constexpr uint32_t kGatedChunk = 512;

struct Visible {
  uint32_t prefix, recent_low, count;
};

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

typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool F32>
struct Tile {
  // Raw codes (or floats) of 4 positions x 16 dims for K and V, plus scales.
  uint4 k[F32 ? 16 : 4], v[F32 ? 16 : 4];
  float ks[4], vs[4];
};

// Cache slot of visible index t without branches: slot = t below the prefix,
// else r0 + wrap(b0 + t - prefix), wrap(x) = x >= w ? x - w : x.  A sliding
// window (kv_slot) gives r0 = sink, b0 = (recent_low - sink) % window, w =
// window -- the recent indices span fewer than `window` positions, so one
// subtraction wraps them -- and no window r0 = recent_low, b0 = 0, w = 2^32 - 1.
struct Ring {
  uint32_t r0, b0, w;
};

__device__ __forceinline__ Ring ring_of(const Visible& vis, uint32_t sink, uint32_t window) {
  if (window == 0 || vis.recent_low < sink) return Ring{vis.recent_low, 0u, 0xffffffffu};
  return Ring{sink, (vis.recent_low - sink) % window, window};
}

__device__ __forceinline__ uint32_t ring_slot(const Visible& vis, const Ring& ring, uint32_t t) {
  const uint32_t x = ring.b0 + (t - vis.prefix);
  return t < vis.prefix ? t : ring.r0 + (x >= ring.w ? x - ring.w : x);
}

template <bool F32>
__device__ __forceinline__ void load_tile(Tile<F32>& tl, const void* Kc, const void* Vc,
                                          const float* Ks, const float* Vs, size_t head_base,
                                          const Visible& vis, const Ring& ring, uint32_t t0,
                                          uint32_t t_end, uint32_t trow, uint32_t quad) {
  uint32_t slots[4];
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const uint32_t t = t0 + trow + 16 * k;
    slots[k] = ring_slot(vis, ring, t < t_end ? t : t0);
  }
#pragma unroll
  for (int k = 0; k < 4; ++k) {
    const size_t row = head_base + slots[k];
    tl.ks[k] = Ks[row];
    tl.vs[k] = Vs[row];
    if constexpr (F32) {
      const uint4* kp = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(Kc) + row * kHeadDim + quad * 16);
      const uint4* vp = reinterpret_cast<const uint4*>(reinterpret_cast<const float*>(Vc) + row * kHeadDim + quad * 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        tl.k[4 * k + c] = kp[c];
        tl.v[4 * k + c] = vp[c];
      }
    } else {
      // Codes are read once per call: non-temporal loads (6.35 against
      // 7.02 us per call at 8 heads x 8192 positions).
      const u32x4 kk = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          reinterpret_cast<const int8_t*>(Kc) + row * kHeadDim + quad * 16));
      const u32x4 vv = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(
          reinterpret_cast<const int8_t*>(Vc) + row * kHeadDim + quad * 16));
      tl.k[k] = make_uint4(kk[0], kk[1], kk[2], kk[3]);
      tl.v[k] = make_uint4(vv[0], vv[1], vv[2], vv[3]);
    }
  }
}

template <bool F32>
__device__ __forceinline__ void unpack(const Tile<F32>& tl, int k, bool is_v, float* out) {
  if constexpr (F32) {
#pragma unroll
    for (int c = 0; c < 4; ++c) {
      const uint4 w = is_v ? tl.v[4 * k + c] : tl.k[4 * k + c];
      out[4 * c + 0] = __uint_as_float(w.x);
      out[4 * c + 1] = __uint_as_float(w.y);
      out[4 * c + 2] = __uint_as_float(w.z);
      out[4 * c + 3] = __uint_as_float(w.w);
    }
  } else {
    const uint4 w = is_v ? tl.v[k] : tl.k[k];
    const uint32_t words[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
    for (int q = 0; q < 4; ++q) {
#pragma unroll
      for (int e = 0; e < 4; ++e)
        out[4 * q + e] = (float)(int8_t)((words[q] >> (8 * e)) & 0xffu);
    }
  }
}

// Workgroup = 4 waves on one (sequence z, kv head, chunk of `chunk_positions`
// visible positions), serving all REP query heads of the kv head so that each
// code byte is read once.  Wave w walks 64-position tiles w, w+4, ... of the
// chunk with a running (max, sum, acc) per query head (online softmax), and
// prefetches its next tile before working on the current one.  In a tile,
// lane l owns dims [16*(l&3), +16) of positions tile + (l>>2) + 16k, k < 4,
// so each 128-bit load of the wave reads 16 consecutive 64-byte rows.
//
// The waves merge through LDS.  A sequence whose visible positions fit one
// chunk gets its normalized output here; otherwise each chunk publishes
// (max, sum, acc[64]) per query head and the last chunk to finish combines
// them, so one launch always completes the attention.
//
// Scores: (q . k_codes) * k_scale / sqrt(64); softmax; out = sum w * v_codes *
// v_scale -- NeedleRuntime.#attention (model/runtime.ts:719-786) with
// softmaxInPlace (model/math.ts:46-60), evaluated in fp32.
// Output gate of gated attention (model/runtime.ts:503-507): sigmoid(g).
__device__ __forceinline__ float gate_factor(float g) { return 1.f / (1.f + __expf(-g)); }

// QB (a prefill whose positions all see [0, position]: no sliding window,
// or a window no position outgrows): the REP rows are REP / G consecutive
// query positions x the G = qgroup query heads of KV head blockIdx.y --
// row r is query z0 + r / G (z0 = (REP / G) blockIdx.z, rows at or past
// `qrows` absent), head G blockIdx.y + r % G, with its own causal limit --
// so every K/V tile is read once for all of them.
// STAMP (measurement only): thread 0 reads the 100 MHz constant clock at
// entry, after its wave's tiles, after the waves' combine, once the chunk's
// partials are published, once its arrival is counted and (the last chunk)
// after the merge, and writes them with the chunk's role (0 counted in,
// 1 merged) and its XCC id to stamps[8 L .. 8 L + 7] for workgroup L.
// The default of attention_body's `hook`: nothing between the loads and
// the math.
struct NoHook {
  static constexpr bool kActive = false;
  static constexpr bool kStamp = false;  // measurement marks (hook.mark(i))
  __device__ bool wait() const { return true; }
  __device__ uint32_t fresh_slot() const { return 0xFFFFFFFFu; }
  __device__ void mark(int) const {}
};

// hook (kActive, one tile per wave, int8 cache): the workgroup issues its
// tile loads, then every thread calls hook.wait() (false: return without
// storing), then the rows of cache slot hook.fresh_slot() -- written by
// another workgroup of the same launch while the loads were in flight -- are
// read again past the CU's L1, and the query rows are read; then the math.
//
// GRID: the workgroup's (chunk, KV head local to its row, row z) come from
// the grid (the arguments of those names are ignored); otherwise from the
// arguments (a caller that runs one workgroup per (chunk, KV head, row) of
// its own).
template <int REP, bool F32, bool QB = false, int KW = 4, int TILES = 0, bool XL = false,
          bool STAMP = false, bool GRID = true, class Hook = NoHook>
__device__ __forceinline__ void attention_body(
    uint32_t chunk_arg, uint32_t kvh_arg, uint32_t z_arg, const void* Kc, const void* Vc, const float* Ks,
    const float* Vs, const float* Q, float* out,
    const float* gate, uint32_t gate_ld, float* part_acc,
    float* part_ml,
    uint32_t* counters, uint32_t layer, uint32_t kv_heads,
    uint32_t alloc, uint32_t sink, uint32_t window, Visible vis,
    const uint32_t* positions, uint32_t slot_space, uint32_t seq_kv_heads,
    uint32_t kv_stride_z,
    uint32_t chunk_positions, uint32_t max_chunks, float score_scale, uint32_t qrows,
    uint32_t qgroup, uint64_t* stamps, const Hook& hook = Hook()) {
  static_assert(!Hook::kActive || (TILES == 1 && !F32 && !QB),
                "the hook serves the one-tile int8 single-row form");
  uint64_t stamp[6] = {};
  if constexpr (STAMP) stamp[0] = wall_clock64();
  auto put_stamps = [&](uint32_t role) {
    if constexpr (STAMP) {
      if (threadIdx.x == 0) {
        uint64_t* o = stamps + 8 * (size_t)blockIdx.x;
#pragma unroll
        for (int i = 0; i < 6; ++i) o[i] = stamp[i];
        o[6] = role;
        o[7] = (uint32_t)__builtin_amdgcn_s_getreg((3 << 11) | (0 << 6) | 20) & 15u;
      }
    }
  };
  // z indexes query rows: sequences of a batch (kv_stride_z = seq_kv_heads,
  // each with its own cache heads) or positions of one prefill (kv_stride_z
  // = 0, all reading the same cache heads).
  uint32_t chunk, kvh_local, z;
  if constexpr (XL) {
    // A one-dimensional grid laid out so that every chunk of a (row, KV
    // head) pair runs on one XCD: the dispatcher hands workgroup L to XCD
    // L % 8, so pair g = 8 (L / 8 / max_chunks) + L % 8 (row g /
    // seq_kv_heads) and chunk L / 8 % max_chunks -- on each XCD a pair's
    // chunks are dispatched one after another.
    const uint32_t pairs = qrows * seq_kv_heads;
    const uint32_t L = blockIdx.x, sl = L >> 3, g = 8 * (sl / max_chunks) + (L & 7);
    chunk = sl % max_chunks;
    if (g >= pairs) return;
    z = g / seq_kv_heads;
    kvh_local = g % seq_kv_heads;
  } else if constexpr (GRID) {
    chunk = blockIdx.x;
    kvh_local = blockIdx.y;
    z = blockIdx.z;
  } else {
    chunk = chunk_arg;
    kvh_local = kvh_arg;
    z = z_arg;
  }
  const uint32_t kvh = z * kv_stride_z + kvh_local;
  const uint32_t hq = seq_kv_heads * REP;
  // The wave index is uniform: read it into a scalar register so that the
  // tile loop below is scalar control flow.
  const uint32_t wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
  const uint32_t quad = lane & 3, trow = lane >> 2;
  // slot_space (one row, position in device memory): walk the cache slots
  // [0, alloc) in slot order -- vis = {alloc, alloc, alloc} makes logical
  // index = slot -- so the tile loads need not wait for the position; a slot
  // holds a visible position iff slot <= position or the ring is full
  // (position >= alloc).  Otherwise the visible range of the row's position.
  uint32_t spos = 0;
  uint32_t rlim[QB ? REP : 1];  // QB: row r sees cache positions < rlim[r]
  if constexpr (QB) {
    uint32_t top = 0;
#pragma unroll
    for (int r = 0; r < REP; ++r) {
      const uint32_t zr = z * (REP / qgroup) + r / qgroup;
      const uint32_t pr = zr < qrows ? positions[zr] : 0;
      if (zr < qrows && pr >= alloc) return;  // validated on entry; stay in bounds
      rlim[r] = zr < qrows ? pr + 1 : 0;
      top = max(top, rlim[r]);
    }
    vis = Visible{top, top, top};
  } else if (slot_space) {
    spos = positions[z];
  } else if (positions) {
    if (window == 0 && positions[z] >= alloc) return;  // validated on entry; stay in bounds
    vis = visible_at(positions[z], sink, window);
  }
  uint32_t nchunks = (vis.count + chunk_positions - 1) / chunk_positions;
  if (nchunks > max_chunks) nchunks = max_chunks;  // the grid bound; never write past it
  if (chunk >= nchunks) return;
  const uint32_t c_begin = chunk * chunk_positions;
  const uint32_t c_end = min(vis.count, c_begin + chunk_positions);
  if constexpr (!QB) {
    Q += (size_t)z * hq * kHeadDim;
    out += (size_t)z * hq * kHeadDim;
  }
  const size_t head_base = ((size_t)layer * kv_heads + kvh) * alloc;
  // Query row h: head h of this KV head, or (QB) query z REP + h (absent
  // rows read query 0; they are never stored).
  auto qrow = [&](int h) -> size_t {
    if constexpr (QB) {
      const uint32_t zr = z * (REP / qgroup) + h / qgroup;
      return ((size_t)(zr < qrows ? zr : 0) * seq_kv_heads * qgroup + kvh_local * qgroup +
              h % qgroup) * kHeadDim;
    } else {
      return (size_t)(kvh_local * REP + h) * kHeadDim;
    }
  };

  float q[REP][16];
  auto load_q = [&]() __attribute__((always_inline)) {
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      const float4* qp = reinterpret_cast<const float4*>(Q + qrow(h) + quad * 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const float4 f = qp[c];
        q[h][4 * c + 0] = f.x;
        q[h][4 * c + 1] = f.y;
        q[h][4 * c + 2] = f.z;
        q[h][4 * c + 3] = f.w;
      }
    }
  };
  if constexpr (!Hook::kActive) load_q();

  float m[REP], l[REP], acc[REP][16];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    m[h] = -INFINITY;
    l[h] = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) acc[h][i] = 0.f;
  }

  // The tile loads are issued under uniform control flow with a static count
  // of outstanding loads, and no loaded tile is carried from one loop
  // iteration to the next, so that the wait before a tile's math covers that
  // tile only.  (A load under a per-lane condition, or a prefetched tile
  // copied or carried into the next iteration, makes the compiler wait for
  // every outstanding load: one memory round trip per tile.)
  auto tile_math = [&](const Tile<F32>& cur, uint32_t t0) __attribute__((always_inline)) {
    bool valid[4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      const uint32_t ti = t0 + trow + 16 * k;
      valid[k] = ti < c_end && (!slot_space || ti <= spos || spos >= alloc);
    }
    float p[REP][4];
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float kc[16];
      unpack<F32>(cur, k, false, kc);
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        float d = 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) d = fmaf(q[h][i], kc[i], d);
        d = nd::quad_sum(d);
        bool ok = valid[k];
        if constexpr (QB) ok = ok && t0 + trow + 16 * k < rlim[h];
        p[h][k] = ok ? d * cur.ks[k] * score_scale : -INFINITY;
      }
    }
#pragma unroll
    for (int h = 0; h < REP; ++h) {
      float tile_max = fmaxf(fmaxf(p[h][0], p[h][1]), fmaxf(p[h][2], p[h][3]));
      // rows rotated by 4, then 8: the max over lanes i, i - 4, i - 8, i - 12
      // of each 16-lane row, the set lane xor 4 and 8 span
      tile_max = fmaxf(tile_max, nd::dpp<nd::kRowRor4>(tile_max));
      tile_max = fmaxf(tile_max, nd::dpp<nd::kRowRor8>(tile_max));
      tile_max = nd::max_xor<16>(tile_max);
      tile_max = nd::max_xor<32>(tile_max);
      const float m_new = fmaxf(m[h], tile_max);
      // 0 on the first tile with a visible position (m = -inf); 1 while no
      // position has been visible (a tile of unwritten slots: -inf - -inf).
      const float alpha = m_new == -INFINITY ? 1.f : __expf(m[h] - m_new);
      m[h] = m_new;
      l[h] *= alpha;
#pragma unroll
      for (int i = 0; i < 16; ++i) acc[h][i] *= alpha;
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        bool ok = valid[k];
        if constexpr (QB) ok = ok && t0 + trow + 16 * k < rlim[h];
        const float e = ok ? __expf(p[h][k] - m_new) : 0.f;
        p[h][k] = e;
        l[h] += e;
      }
    }
    // Masked positions add exactly nothing, whatever their (possibly never
    // written) slots hold: int8 codes are finite, so a zero weight suffices;
    // float32 rows could hold NaN and are skipped per element.
#pragma unroll
    for (int k = 0; k < 4; ++k) {
      float vc[16];
      unpack<F32>(cur, k, true, vc);
#pragma unroll
      for (int h = 0; h < REP; ++h) {
        const float ev = valid[k] ? p[h][k] * cur.vs[k] : 0.f;
#pragma unroll
        for (int i = 0; i < 16; ++i) {
          if constexpr (F32) acc[h][i] = valid[k] ? fmaf(ev, vc[i], acc[h][i]) : acc[h][i];
          else acc[h][i] = fmaf(ev, vc[i], acc[h][i]);
        }
      }
    }
  };
  constexpr uint32_t kStride = (uint32_t)KW * kWavePositions;
  const Ring ring = ring_of(vis, sink, window);
  const uint32_t t_first = c_begin + wave * kWavePositions;
  // Tiles t_first + kStride j, j < n (n uniform), two per round: both tiles'
  // loads are in flight before the first tile's math.  TILES = 1 or 2: the
  // launch guarantees n <= TILES, and the code is straight-line.
  // Hook: each thread's output gates (the combine's output mapping below),
  // read together with q once the wait is over.
  constexpr int kGateT = REP * kHeadDim >= 64 * KW ? 1 : 64 * KW / (REP * kHeadDim);
  constexpr int kGatePer = REP * kHeadDim >= 64 * KW ? REP * kHeadDim / (64 * KW) : 1;
  float gate_pre[Hook::kActive ? kGatePer : 1];
  if constexpr (Hook::kActive) {
    Tile<F32> ta;
    const bool has = t_first < c_end;
    if (has) load_tile<F32>(ta, Kc, Vc, Ks, Vs, head_base, vis, ring, t_first, c_end, trow, quad);
    if (!hook.wait()) return;
    // The fresh slot's row, past the CU's L1 (device-scope loads hit the L2
    // its writer stored to), issued with q and the gates so that one round
    // trip serves all three.  Slot order: row k of lane group trow holds
    // slot t_first + trow + 16 k, so in the one wave whose tile holds the
    // slot (uniform test) the lanes of row (fresh - t_first) % 16 take it
    // at k = (fresh - t_first) / 16 (uniform); every lane of that wave loads
    // its quad's codes of the row.
    const uint32_t fresh = hook.fresh_slot();
    const bool wave_fresh = has && fresh - t_first < kWavePositions;
    uint32_t fk[4] = {0, 0, 0, 0}, fv[4] = {0, 0, 0, 0};
    float fks = 0.f, fvs = 0.f;
    if (wave_fresh) {
      const size_t row = head_base + fresh;
      const uint32_t* kp = reinterpret_cast<const uint32_t*>(
          reinterpret_cast<const int8_t*>(Kc) + row * kHeadDim + quad * 16);
      const uint32_t* vp = reinterpret_cast<const uint32_t*>(
          reinterpret_cast<const int8_t*>(Vc) + row * kHeadDim + quad * 16);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        fk[c] = __hip_atomic_load(kp + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        fv[c] = __hip_atomic_load(vp + c, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      }
      fks = __hip_atomic_load(Ks + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      fvs = __hip_atomic_load(Vs + row, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
    load_q();
    if (gate) {
#pragma unroll
      for (int u = 0; u < kGatePer; ++u)
        gate_pre[u] = gate[(size_t)z * gate_ld + kvh_local * (REP * kHeadDim) +
                           threadIdx.x / kGateT + u * (64 * KW / kGateT)];
    }
    if (wave_fresh) {
      const uint32_t kf = (fresh - t_first) >> 4;
      const bool mine = trow == ((fresh - t_first) & 15u);
#pragma unroll
      for (int k = 0; k < 4; ++k) {
        if ((uint32_t)k == kf && mine) {
          ta.k[k] = make_uint4(fk[0], fk[1], fk[2], fk[3]);
          ta.v[k] = make_uint4(fv[0], fv[1], fv[2], fv[3]);
          ta.ks[k] = fks;
          ta.vs[k] = fvs;
        }
      }
    }
    if constexpr (Hook::kStamp) hook.mark(1);
    if (has) tile_math(ta, t_first);
    if constexpr (Hook::kStamp) hook.mark(2);
  } else if (t_first < c_end) {
    Tile<F32> ta, tb;
    if constexpr (TILES == 1) {
      load_tile<F32>(ta, Kc, Vc, Ks, Vs, head_base, vis, ring, t_first, c_end, trow, quad);
      __builtin_amdgcn_sched_barrier(0);  // every load issued before the math
      tile_math(ta, t_first);
    } else {
      const uint32_t n = TILES == 2 ? 2u : (c_end - t_first + kStride - 1) / kStride;
      for (uint32_t j = 0; j < n; j += 2) {
        // Past the chunk end the second tile rereads the first one's rows and
        // its math masks every position (it adds nothing); its math is not
        // skipped, so that the compiler cannot sink its loads behind a branch.
        const uint32_t t_a = t_first + j * kStride, t_b = t_a + kStride;
        load_tile<F32>(ta, Kc, Vc, Ks, Vs, head_base, vis, ring, t_a, c_end, trow, quad);
        load_tile<F32>(tb, Kc, Vc, Ks, Vs, head_base, vis, ring, t_b < c_end ? t_b : t_a, c_end,
                       trow, quad);
        __builtin_amdgcn_sched_barrier(0);  // every load issued before the math
        tile_math(ta, t_a);
        tile_math(tb, t_b);
      }
    }
  }
  if constexpr (STAMP) stamp[1] = wall_clock64();

  // Per wave: fold the 16 token rows of each lane's partial sums 4 apart
  // (lane bits 2..3) with DPP, leaving 4 row groups (lane bits 4..5) that go
  // to LDS; l is the same in the 4 lanes of a quad and m in the whole wave.
  // The fold adds the row rotated by 4, then by 8 (one DPP add each): lane
  // j + 12 of a 16-lane row (j < 4) ends with (a[j+12] + a[j+8]) + (a[j+4] +
  // a[j]), the sums a fold by lane xor 4 then 8 leaves in lane j, operand for
  // operand (each add commutes exactly), and it is the lane that stores.
  constexpr int kOut = REP * kHeadDim;  // outputs (head, dim) of the workgroup
  __shared__ float s_m[(uint32_t)KW][REP], s_l[(uint32_t)KW][REP];
  __shared__ float s_part[(uint32_t)KW * 4][kOut];
#pragma unroll
  for (int h = 0; h < REP; ++h) {
    const float lw = nd::wave_sum(quad == 0 ? l[h] : 0.f);
#pragma unroll
    for (int i = 0; i < 16; ++i) {
      acc[h][i] += nd::dpp<nd::kRowRor4>(acc[h][i]);
      acc[h][i] += nd::dpp<nd::kRowRor8>(acc[h][i]);
    }
    if ((trow & 3) == 3) {
      float4* dst = reinterpret_cast<float4*>(&s_part[wave * 4 + (lane >> 4)][h * kHeadDim + quad * 16]);
#pragma unroll
      for (int c = 0; c < 4; ++c)
        dst[c] = make_float4(acc[h][4 * c], acc[h][4 * c + 1], acc[h][4 * c + 2], acc[h][4 * c + 3]);
    }
    if (lane == 0) {
      s_m[wave][h] = m[h];
      s_l[wave][h] = lw;
    }
  }
  __syncthreads();
  if constexpr (STAMP) stamp[2] = wall_clock64();
  if constexpr (Hook::kStamp) hook.mark(3);

  // Combine the waves: kT consecutive threads share output o (REP <= 2), each
  // summing KW * 4 / kT rows scaled by exp(m_wave - max); REP >= 4 gives
  // every thread kPer whole outputs.
  constexpr int kThreads = 64 * KW;
  constexpr int kT = kOut >= kThreads ? 1 : kThreads / kOut;
  constexpr int kPer = kOut >= kThreads ? kOut / kThreads : 1;
  constexpr int kRows = KW * 4 / kT;
  const uint32_t part = threadIdx.x % kT;
  float w_m[kPer], w_l[kPer], w_a[kPer];
  uint32_t w_o[kPer];
#pragma unroll
  for (int u = 0; u < kPer; ++u) {
    const uint32_t o = threadIdx.x / kT + u * (kThreads / kT);
    const uint32_t h = o / kHeadDim;
    float mx = -INFINITY;
#pragma unroll
    for (uint32_t w = 0; w < (uint32_t)KW; ++w) mx = fmaxf(mx, s_m[w][h]);
    float L = 0.f;
#pragma unroll
    for (uint32_t w = 0; w < (uint32_t)KW; ++w)
      L = fmaf((s_m[w][h] == -INFINITY) ? 0.f : __expf(s_m[w][h] - mx), s_l[w][h], L);
    float A = 0.f;
#pragma unroll
    for (int wi = 0; wi < kRows / 4; ++wi) {
      const uint32_t w = part * (kRows / 4) + wi;
      const float fw = (s_m[w][h] == -INFINITY) ? 0.f : __expf(s_m[w][h] - mx);
#pragma unroll
      for (int g = 0; g < 4; ++g) A = fmaf(fw, s_part[w * 4 + g][o], A);
    }
    static_assert(kT <= 8, "at most 8 threads share an output");
    if constexpr (kT >= 2) A += nd::lane_xor<1>(A);
    if constexpr (kT >= 4) A += nd::lane_xor<2>(A);
    if constexpr (kT >= 8) A += nd::lane_xor<4>(A);
    w_m[u] = mx;
    w_l[u] = L;
    w_a[u] = A;
    w_o[u] = o;
  }
  const size_t row0 = (size_t)z * hq + (size_t)kvh_local * REP;
  float* const out_z = out;  // already offset to row z
  const float* const gate_z = gate ? gate + (size_t)z * gate_ld : nullptr;
  if constexpr (QB) {  // one chunk (the launch guarantees it)
    if (part == 0) {
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const uint32_t r = w_o[u] / kHeadDim, zr = z * (REP / qgroup) + r / qgroup;
        if (zr >= qrows) continue;
        const uint32_t oi = (kvh_local * qgroup + r % qgroup) * kHeadDim + w_o[u] % kHeadDim;
        float v = w_a[u] / w_l[u];
        if (gate) v *= gate_factor(gate[(size_t)zr * gate_ld + oi]);
        out[(size_t)zr * seq_kv_heads * qgroup * kHeadDim + oi] = v;
      }
    }
    return;
  }
  if (nchunks == 1) {
    if (part == 0) {
#pragma unroll
      for (int u = 0; u < kPer; ++u) {
        const uint32_t oi = kvh_local * kOut + w_o[u];
        float r = w_a[u] / w_l[u];
        if (gate_z) r *= gate_factor(Hook::kActive ? gate_pre[u] : gate_z[oi]);
        out_z[oi] = r;
      }
    }
    return;
  }
  // Several chunks: publish this chunk's (max, sum, acc) with agent-coherent
  // stores, wait for them, count the chunk in; the last chunk of the (row,
  // KV head) to arrive combines all of them (log-sum-exp) and resets the
  // counter for the next launch.  No workgroup waits for another.  XL: all
  // chunks of the head share one XCD, so the partials and counters stay in
  // its L2 (plain stores, atomics performed there); the merge's agent-scope
  // loads miss the CU's L1 and hit that L2.  Each head's counters fill
  // 128-byte lines of their own.
  constexpr int kPubScope = XL ? __HIP_MEMORY_SCOPE_WORKGROUP : __HIP_MEMORY_SCOPE_AGENT;
  if (part == 0) {
#pragma unroll
    for (int u = 0; u < kPer; ++u) {
      const uint32_t h = w_o[u] / kHeadDim, dim = w_o[u] % kHeadDim;
      const size_t pi = (row0 + h) * max_chunks + chunk;
      __hip_atomic_store(part_acc + pi * kHeadDim + dim, w_a[u], __ATOMIC_RELAXED, kPubScope);
      if (dim == 0) {
        __hip_atomic_store(part_ml + pi * 2, w_m[u], __ATOMIC_RELAXED, kPubScope);
        __hip_atomic_store(part_ml + pi * 2 + 1, w_l[u], __ATOMIC_RELAXED, kPubScope);
      }
    }
  }
  __builtin_amdgcn_s_waitcnt(0);  // every store above has completed
  __syncthreads();
  if constexpr (STAMP) stamp[3] = wall_clock64();
  // Election: rows of more than kChunkGroup chunks count in per group first
  // and the last of each group then on the row's counter, so that no counter
  // serializes more than kChunkGroup arrivals (agent-scope atomics on one
  // address complete ~70 ns apart); XL counts every chunk on the row's
  // counter (atomics in the XCD's L2 do not serialize so).  Each counter is
  // reset by its last arriver.
  __shared__ uint32_t s_last;
  uint32_t* counter = counters + ((size_t)z * seq_kv_heads + kvh_local) * kAttnCounterStride;
  if (threadIdx.x == 0) {
    bool last;
    if (XL || nchunks <= kChunkGroup) {
      last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, kPubScope) == nchunks - 1;
    } else {
      const uint32_t grp = chunk / kChunkGroup;
      const uint32_t ngroups = (nchunks + kChunkGroup - 1) / kChunkGroup;
      const uint32_t members = min(kChunkGroup, nchunks - grp * kChunkGroup);
      uint32_t* gc = counter + 1 + grp;
      last = false;
      if (__hip_atomic_fetch_add(gc, 1u, __ATOMIC_RELAXED, kPubScope) == members - 1) {
        __hip_atomic_store(gc, 0u, __ATOMIC_RELAXED, kPubScope);
        last = __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED, kPubScope) == ngroups - 1;
      }
    }
    s_last = last;
  }
  __syncthreads();
  if constexpr (STAMP) stamp[4] = wall_clock64();
  if (!s_last) {
    put_stamps(0);
    return;
  }

  // Last chunk: wave w merges head w / kWph over chunks c = w % kWph + kWph j
  // (REP < KW) or heads w, w + KW, ... over all chunks.  Lane c holds
  // chunk c's (max, sum) (nchunks <= 64, see chunk_positions_for); lane d
  // accumulates dim d.  The first batch of acc loads is issued together
  // with the (max, sum) loads, so one round trip serves the common case.
  constexpr int kWph = REP >= KW ? 1 : KW / REP;
  constexpr int kHpw = REP > KW ? REP / KW : 1;
  constexpr int kBatch = 16;
  __shared__ float s_fin[(uint32_t)KW][kHeadDim];
  const uint32_t wpart = wave % kWph;
  float fin_l = 0.f;
#pragma unroll
  for (int hh = 0; hh < kHpw; ++hh) {
    const uint32_t h = kWph > 1 ? wave / kWph : wave + hh * (uint32_t)KW;
    const size_t base = (row0 + h) * max_chunks;
    const uint32_t cl = lane < nchunks ? lane : nchunks - 1;
    float mc = __hip_atomic_load(part_ml + (base + cl) * 2, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    float lc = __hip_atomic_load(part_ml + (base + cl) * 2 + 1, __ATOMIC_RELAXED,
                                 __HIP_MEMORY_SCOPE_AGENT);
    float A = 0.f, f = 0.f;
    for (uint32_t j0 = wpart; j0 < nchunks; j0 += kBatch * kWph) {
      float av[kBatch];
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const uint32_t j = min(j0 + u * kWph, nchunks - 1);  // past the end: reread, then drop
        av[u] = __hip_atomic_load(part_acc + (base + j) * kHeadDim + lane, __ATOMIC_RELAXED,
                                  __HIP_MEMORY_SCOPE_AGENT);
      }
      if (j0 == wpart) {
        if (lane >= nchunks) mc = -INFINITY, lc = 0.f;
        float mx = mc;
        mx = fmaxf(mx, nd::lane_xor<1>(mx));
        mx = fmaxf(mx, nd::lane_xor<2>(mx));
        mx = fmaxf(mx, nd::lane_xor<4>(mx));
        mx = fmaxf(mx, nd::lane_xor<8>(mx));
        mx = nd::max_xor<16>(mx);
        mx = nd::max_xor<32>(mx);
        f = mc == -INFINITY ? 0.f : __expf(mc - mx);
        fin_l = nd::wave_sum(f * lc);
      }
#pragma unroll
      for (int u = 0; u < kBatch; ++u) {
        const uint32_t j = j0 + u * kWph;
        if (j < nchunks) A = fmaf(nd::readlane(f, j), av[u], A);
      }
    }
    if constexpr (kWph == 1) {
      const uint32_t oi = kvh_local * kOut + h * kHeadDim + lane;
      float r = A / fin_l;
      if (gate_z) r *= gate_factor(gate_z[oi]);
      out_z[oi] = r;
    } else {
      s_fin[wave][lane] = A;
    }
  }
  if constexpr (kWph > 1) {
    __syncthreads();
    if (wpart == 0) {
      float A = 0.f;
#pragma unroll
      for (int i = 0; i < kWph; ++i) A += s_fin[wave + i][lane];
      const uint32_t oi = kvh_local * kOut + (wave / kWph) * kHeadDim + lane;
      float r = A / fin_l;
      if (gate_z) r *= gate_factor(gate_z[oi]);
      out_z[oi] = r;
    }
  }
  if (threadIdx.x == 0) __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, kPubScope);
  if constexpr (STAMP) {
    __builtin_amdgcn_s_waitcnt(0);  // the outputs are stored
    stamp[5] = wall_clock64();
  }
  put_stamps(1);
}

}  // namespace att
}  // namespace nd
