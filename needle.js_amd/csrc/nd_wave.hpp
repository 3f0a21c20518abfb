// Wave64 cross-lane helpers built on DPP moves and readlane, so that a
// reduction costs a few VALU cycles per step instead of the LDS-crossbar
// latency of ds_bpermute (__shfl_xor).
#pragma once

#include <hip/hip_runtime.h>

namespace nd {

// DPP controls (GFX9 encoding).
constexpr int kQuadXor1 = 0xB1;     // quad_perm [1,0,3,2]
constexpr int kQuadXor2 = 0x4E;     // quad_perm [2,3,0,1]
constexpr int kHalfMirror = 0x141;  // lane i of 8 <- lane 7 - i
constexpr int kRowMirror = 0x140;   // lane i of 16 <- lane 15 - i

// Every control used here is a full permutation (each lane reads a lane of
// its own row), so bound_ctrl never applies; given as an update with it set,
// the move folds into the VALU operation that consumes it (v_add_f32_dpp
// and the like: one instruction per reduction step).
template <int CTRL>
__device__ __forceinline__ float dpp(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xF, 0xF, true));
}

template <int CTRL>
__device__ __forceinline__ double dpp(double v) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_mov_dpp((int)b, CTRL, 0xF, 0xF, false);
  const int hi = __builtin_amdgcn_mov_dpp((int)(b >> 32), CTRL, 0xF, 0xF, false);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

__device__ __forceinline__ double readlane(double v, int lane) {
  const long long b = __double_as_longlong(v);
  const int lo = __builtin_amdgcn_readlane((int)b, lane);
  const int hi = __builtin_amdgcn_readlane((int)(b >> 32), lane);
  return __longlong_as_double(((long long)hi << 32) | (unsigned int)lo);
}

__device__ __forceinline__ float readlane(float v, int lane) {
  return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

// Sum of each row of 16 lanes, in every lane of the row.
template <typename T>
__device__ __forceinline__ T row_sum(T v) {
  v += dpp<kQuadXor1>(v);
  v += dpp<kQuadXor2>(v);
  v += dpp<kHalfMirror>(v);
  v += dpp<kRowMirror>(v);
  return v;
}

// Sum over the wave, the same value in every lane: rows of 16 by DPP, then
// ((row0 + row1) + row2) + row3.
template <typename T>
__device__ __forceinline__ T wave_sum(T v) {
  v = row_sum(v);
  return ((readlane(v, 0) + readlane(v, 16)) + readlane(v, 32)) + readlane(v, 48);
}

// Maximum of each row of 16 lanes (fmaxf), in every lane of the row.
__device__ __forceinline__ float row_max(float v) {
  v = fmaxf(v, dpp<kQuadXor1>(v));
  v = fmaxf(v, dpp<kQuadXor2>(v));
  v = fmaxf(v, dpp<kHalfMirror>(v));
  v = fmaxf(v, dpp<kRowMirror>(v));
  return v;
}

typedef _Float16 half8 __attribute__((ext_vector_type(8)));
typedef _Float16 half2v __attribute__((ext_vector_type(2)));
typedef float float4v __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

// Eight int8 codes (bytes 0..7 of w, in order) -> eight exact fp16 values:
// 0x6500 | (c ^ 0x80) is the fp16 number 1408 + c, and one packed
// subtraction per pair removes 1408.
__device__ __forceinline__ half8 codes_to_half(u32x2 w) {
  const uint32_t u0 = w.x ^ 0x80808080u, u1 = w.y ^ 0x80808080u;
  const uint32_t k = 0x65656565u;
  const half2v off = {(_Float16)-1408.f, (_Float16)-1408.f};
  const half2v p0 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(k, u0, 0x04010400u)) + off;
  const half2v p1 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(k, u0, 0x04030402u)) + off;
  const half2v p2 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(k, u1, 0x04010400u)) + off;
  const half2v p3 = __builtin_bit_cast(half2v, __builtin_amdgcn_perm(k, u1, 0x04030402u)) + off;
  return half8{p0[0], p0[1], p1[0], p1[1], p2[0], p2[1], p3[0], p3[1]};
}

// JavaScript Math.max of two numbers (NaN if either is NaN).
__device__ __forceinline__ float js_max(float a, float b) {
  return (a != a || b != b) ? __builtin_nanf("") : (a > b ? a : b);
}

// JavaScript Math.max over the wave (NaN wins), in every lane.
__device__ __forceinline__ float wave_max_js(float v) {
  v = js_max(v, dpp<kQuadXor1>(v));
  v = js_max(v, dpp<kQuadXor2>(v));
  v = js_max(v, dpp<kHalfMirror>(v));
  v = js_max(v, dpp<kRowMirror>(v));
  return js_max(js_max(readlane(v, 0), readlane(v, 16)), js_max(readlane(v, 32), readlane(v, 48)));
}

// Row rotations (lane i of a row of 16 reads lane (i - n) mod 16), checked
// on gfx950.
constexpr int kRowRor4 = 0x124;
constexpr int kRowRor8 = 0x128;   // = lane xor 8
constexpr int kRowRor12 = 0x12C;

// The value of lane (lane xor m), for m in {1, 2, 4, 8, 16, 32}: DPP within a
// row of 16, ds_swizzle (no memory access) for 16, ds_bpermute for 32.
template <int M>
__device__ __forceinline__ float lane_xor(float v) {
  if constexpr (M == 1) return dpp<kQuadXor1>(v);
  else if constexpr (M == 2) return dpp<kQuadXor2>(v);
  else if constexpr (M == 4) {
    const float up = dpp<kRowRor12>(v), down = dpp<kRowRor4>(v);
    return (__lane_id() & 4) ? down : up;
  } else if constexpr (M == 8) return dpp<kRowRor8>(v);
  else if constexpr (M == 16)
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
  else return __shfl_xor(v, 32, 64);
}

// max(v, v of lane i ^ m) for m = 16 or 32 through gfx950's row / half
// swaps (VALU, no trip through the LDS unit): given the value twice, the
// 16-swap returns {rows 0, 0, 2, 2; rows 1, 1, 3, 3} and the 32-swap {lanes
// 0..31 twice; lanes 32..63 twice} (checked on gfx950), so the two results
// hold each lane's value and its partner's in some order, and fmaxf does
// not depend on the order.
template <int M>
__device__ __forceinline__ float max_xor(float v) {
  static_assert(M == 16 || M == 32, "max_xor takes 16 or 32");
  const uint32_t b = __float_as_uint(v);
  const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(b, b, false, false)
                         : __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}

// v + (v of lane i ^ m) for m = 16 or 32 through the same swaps: each lane
// adds its own value and its partner's, in one order or the other, which an
// fp32 add does not depend on -- the same sums as v + lane_xor<m>(v).
template <int M>
__device__ __forceinline__ float sum_xor(float v) {
  static_assert(M == 16 || M == 32, "sum_xor takes 16 or 32");
  const uint32_t b = __float_as_uint(v);
  const auto r = M == 16 ? __builtin_amdgcn_permlane16_swap(b, b, false, false)
                         : __builtin_amdgcn_permlane32_swap(b, b, false, false);
  return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// Workgroup barrier for hand-offs through LDS only: waits for this wave's
// LDS (and scalar) operations, not for its global loads.  __syncthreads()
// also fences global memory, which waits for every load still in flight --
// work that needs only LDS would then wait for a whole weight stream.
__device__ __forceinline__ void lds_barrier() {
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Sum over a quad of lanes (4 consecutive), in every lane of the quad.
template <typename T>
__device__ __forceinline__ T quad_sum(T v) {
  v += dpp<kQuadXor1>(v);
  v += dpp<kQuadXor2>(v);
  return v;
}

// Hand-off of partial results between the workgroups of one launch (the
// attention chunk merge, the k-slice matvec sum, the split-k GEMM sum): each
// workgroup writes its partials with relaxed agent-scope atomic stores, waits
// for them (s_waitcnt vmcnt(0)), meets at a barrier, and one thread counts it
// in with an agent-scope atomic add; the workgroup whose add returns the last
// count reads every partial with relaxed agent-scope atomic loads and resets
// the counter.  On gfx950 these stores and loads are `global_store ... sc1` /
// `global_load ... sc1`, which write to and read from the agent coherence
// point past the XCD's L2, and vmcnt(0) returns only once a store is
// acknowledged there -- so every partial is in place before its workgroup's
// add is issued, and the last arriver's loads issue after its add returns.
// Release/acquire fences at agent scope would state the same order in the
// memory model, but they compile to buffer_wbl2 sc1 / buffer_inv sc1 (a
// write-back and invalidate of the whole XCD L2) and measured +2.4 us per
// attention call at 8 heads x 8192, +7.3 us per batch-8 4096x4096 matvec and
// twice the batch-64 decode step, so they are not used.
//
// XCD-local form (single-row attention, batch matvec slices): the dispatcher
// hands workgroup L of a launch to XCD L % 8, so a grid laid out with every
// member of a merge group at the same L % 8 keeps the group on one XCD.  The
// partials are then stored and counted at workgroup scope (plain stores;
// the atomic, like every global atomic, performed in the L2) and read with
// the agent-scope loads above, which miss the CU's L1 and hit that L2: the
// round trips end in the XCD's L2 instead of the agent coherence point.

}  // namespace nd
