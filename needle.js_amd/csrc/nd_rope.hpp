// Per-head tail of the q/k/v projections of a decode step: zero-centred RMS
// norm and half-split RoPE of q and k heads, and #storeKV quantization of k
// and v rows into the int8 cache (model/runtime.ts:697-714), on one head row
// held one dimension per lane of a wave.  Shared by the rope/store kernel and
// the q/k/v GEMM's fused epilogue, so both produce the same bits.
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

#include "nd_wave.hpp"

namespace nd {

constexpr uint32_t kRopeHd = 64;

// Destination of a decode step's heads: column heads [0, heads) are query
// heads (normed with q_norm, roped, written to q_out[m][heads][64]), [heads,
// heads + kv_heads) key heads (k_norm, rope, cache) and the next kv_heads
// value heads (cache).  Row m's cache head h is m * kv_head_stride + h of
// cache_heads, at position positions[m] of alloc slots.
struct RopeStore {
  uint32_t heads, kv_heads;
  const float* q_norm;
  const float* k_norm;
  const double2* rope_tab;  // (sin, cos) of pos * inv_freq[j]: [position][32]
  const uint32_t* positions;
  float* q_out;
  int8_t* Kc;
  int8_t* Vc;
  float* Ks;
  float* Vs;
  uint32_t layer, cache_heads, alloc, kv_head_stride;
};

// (1 + scale) * x / sqrt(mean(x^2) + 1e-6) in float64, rounded to f32, then
// the rotation of pair (j, j + 32) by angle (sn, cs), in float64.
__device__ __forceinline__ float norm_rope(double x, const float* __restrict__ scale,
                                           uint32_t lane, double sn, double cs) {
  const double inv = 1.0 / sqrt(wave_sum(x * x) / kRopeHd + 1e-6);
  const float normed = (float)((1.0 + (double)scale[lane]) * x * inv);
  const double mine = normed;
  const double other = __shfl_xor((double)normed, 32, 64);
  return lane < 32 ? (float)(mine * cs - other * sn) : (float)(mine * cs + other * sn);
}

// #storeKV of one row: m = max(1e-12, max|x|), s = m / 127 in float64, scale
// f32(s), code = roundTiesToEven(x / s) (NaN -> 0).
__device__ __forceinline__ void quant_store(float val, size_t row, uint32_t lane,
                                            int8_t* __restrict__ codes,
                                            float* __restrict__ scales) {
  const float a = wave_max_js(fabsf(val));
  const double mm = (a != a) ? (double)a : fmax(1e-12, (double)a);
  const double sc = mm / 127.0;
  const double c = rint((double)val / sc);
  codes[row * kRopeHd + lane] = c != c ? (int8_t)0 : (int8_t)(int)c;
  if (lane == 0) scales[row] = (float)sc;
}

// Rows m[r], r < R, of column head `slot`, value x[r] of this lane's
// dimension; rows with live[r] false are skipped.  pos[r] = positions[m[r]]
// and sc[r] = rope_tab[pos[r]][lane & 31] (q and k heads) and scale[lane]
// (q_norm or k_norm) are loaded by the caller, early.  The R rows are
// independent, so their float64 chains interleave.
template <int R>
__device__ __forceinline__ void rope_store_rows(const float (&x)[R], const uint32_t (&m)[R],
                                                const bool (&live)[R], const uint32_t (&pos)[R],
                                                const double2 (&sc)[R], float scale,
                                                uint32_t slot, uint32_t lane,
                                                const RopeStore& p) {
  const bool is_q = slot < p.heads, is_k = !is_q && slot < p.heads + p.kv_heads;
  if (is_q || is_k) {
    float rot[R];
#pragma unroll
    for (int r = 0; r < R; ++r) {
      const double xd = x[r];
      const double inv = 1.0 / sqrt(wave_sum(xd * xd) / kRopeHd + 1e-6);
      const float normed = (float)((1.0 + (double)scale) * xd * inv);
      const double mine = normed;
      const double other = __shfl_xor((double)normed, 32, 64);
      rot[r] = lane < 32 ? (float)(mine * sc[r].y - other * sc[r].x)
                         : (float)(mine * sc[r].y + other * sc[r].x);
    }
    if (is_q) {
#pragma unroll
      for (int r = 0; r < R; ++r)
        if (live[r]) p.q_out[((size_t)m[r] * p.heads + slot) * kRopeHd + lane] = rot[r];
      return;
    }
    const uint32_t h = slot - p.heads;
#pragma unroll
    for (int r = 0; r < R; ++r) {
      // Positions are validated on entry; never write past the cache.
      if (!live[r] || pos[r] >= p.alloc) continue;
      const size_t row =
          ((size_t)p.layer * p.cache_heads + (size_t)m[r] * p.kv_head_stride + h) * p.alloc +
          pos[r];
      quant_store(rot[r], row, lane, p.Kc, p.Ks);
    }
    return;
  }
  const uint32_t h = slot - p.heads - p.kv_heads;
#pragma unroll
  for (int r = 0; r < R; ++r) {
    if (!live[r] || pos[r] >= p.alloc) continue;
    const size_t row =
        ((size_t)p.layer * p.cache_heads + (size_t)m[r] * p.kv_head_stride + h) * p.alloc +
        pos[r];
    quant_store(x[r], row, lane, p.Vc, p.Vs);
  }
}

}  // namespace nd
