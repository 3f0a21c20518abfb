// Cactus-Quant pieces that the Needle 2 kernels use inside their own launches
// (the standalone CQ kernels are in cq.hip): code extraction from a packed
// row, binary16 norms, the per-group fastWalshHadamard of a row in LDS
// (backends/cq.ts:8-27), and dequantizeCqRow (cq.ts:243-295).  Layout as
// nd_mat's CQ form: rows of kpad codes (a multiple of 32, packed low bits
// first, 3-bit rows one little-endian bit stream, ternary as 2-bit crumbs),
// binary16 norms [n][kpad / g].
#pragma once

#include <hip/hip_runtime.h>

#include <cstdint>

namespace nd {

constexpr uint32_t kCqTernaryBits = 5;

// binary16 bit pattern -> float (float16ToNumber, fp16.ts:5-32; exact).
__device__ __forceinline__ float cq_half(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Code c of a packed row.
__device__ __forceinline__ uint32_t cq_code(const uint8_t* row, uint32_t c, uint32_t bits) {
  if (bits == 2 || bits == kCqTernaryBits) return (row[c >> 2] >> ((c & 3) * 2)) & 3u;
  if (bits == 4) return (row[c >> 1] >> ((c & 1) * 4)) & 15u;
  const uint32_t bit = c * 3, at = bit >> 3, shift = bit & 7;
  const uint32_t word = (uint32_t)row[at] | (shift > 5 ? (uint32_t)row[at + 1] << 8 : 0u);
  return (word >> shift) & 7u;
}

// Per-group FWHT of v[0, len) in LDS by the whole workgroup: strides 1, 2,
// ..., g / 2, one butterfly per pair and a barrier per stage, each result
// one fp32 add or subtract (the reference's Float32Array stores).
__device__ __forceinline__ void cq_fwht_groups(float* v, uint32_t len, uint32_t g) {
  for (uint32_t stride = 1; stride < g; stride <<= 1) {
    for (uint32_t i = threadIdx.x; i < len / 2; i += blockDim.x) {
      const uint32_t block = i / stride, inner = i % stride;
      const uint32_t left = block * 2 * stride + inner, right = left + stride;
      const float a = v[left], b = v[right];
      v[left] = a + b;
      v[right] = a - b;
    }
    __syncthreads();
  }
}

// dequantizeCqRow of one packed row by the whole workgroup into v[0, kpad)
// (LDS): f32(codebook[code] * norm), the butterflies, then f32(value *
// 1/sqrt(g)).  cb: the width's codebook by code (ternary: 0, +c, 0, -c by
// crumb, c = f32(1.2240064 * 1/sqrt(g))).  Ends with a barrier.
__device__ __forceinline__ void cq_dequant_row(const uint8_t* __restrict__ prow,
                                               const uint16_t* __restrict__ nrow,
                                               const float* cb, uint32_t kpad, uint32_t g,
                                               uint32_t bits, double inverse_root, float* v) {
  for (uint32_t c = threadIdx.x; c < kpad; c += blockDim.x)
    v[c] = cb[cq_code(prow, c, bits)] * cq_half(nrow[c / g]);
  __syncthreads();
  cq_fwht_groups(v, kpad, g);
  for (uint32_t c = threadIdx.x; c < kpad; c += blockDim.x)
    v[c] = (float)((double)v[c] * inverse_root);
  __syncthreads();
}

}  // namespace nd
