// Skinny/prefill GEMM on int8 MFMA with exact digit-sliced activations.
//
//   Y[m][n] (op)= s_w[n] * sum_k A[m][k] * W[n][k]
//
// W is an int8 matrix [N][K] with one fp32 scale per row (the reference's
// per-row-scaled int8 matvec, backends/cq.ts:106-156, batched over rows of A).
// The fp32 activations A never meet a lossy cast: each row m is written as
//   A[m][k] ~= 2^(E_m - 21) * (D0 + 256 D1 + 65536 D2)[m][k]
// with E_m = floor(log2(max_k |A[m][k]|)) and balanced int8 digits D0, D1 in
// [-128, 127] and D2 in [-64, 64], so the representation error is at most
// 2^(E_m - 22), i.e. 2^-22 of the row's largest element (about fp32 rounding).
// Each digit plane is multiplied exactly by v_mfma_i32_16x16x64_i8 with int32
// accumulation, and the three exact integer sums are combined in fp32:
//   y = s_w[n] * 2^(E_m - 21) * (C0 + 256 C1 + 65536 C2).
//
// MFMA operand layout (16x16x64 i8): lane l supplies 16 consecutive k of row
// l%16 of each operand, k in [16*(l/16), +16) of the 64-wide step; the
// accumulator's element i of lane l is row 4*(l/16)+i (weight row n) and
// column l%16 (activation row m).  Any k order shared by both operands gives
// the same sum, so both are read straight from row-major memory.
#include "nd_internal.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kKChunk = 256;             // k per LDS stage
constexpr int kLdsRow = kKChunk + 16;    // padded row stride (bank spread)

__device__ __forceinline__ float silu_f(float v) { return v / (1.f + __expf(-v)); }

// MS m-subtiles of 16 and NS n-subtiles of 16 per wave; 4 waves split n.
template <int MS, int NS, int EPI>
__global__ __launch_bounds__(kGemmThreads) void gemm_i8_digits_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ sw, const int8_t* __restrict__ D,
    const float* __restrict__ fm, float* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
    uint32_t ldy) {
  constexpr int TM = 16 * MS;
  constexpr int TN = 4 * 16 * NS;
  __shared__ __attribute__((aligned(16))) int8_t lds[3][TM][kLdsRow];

  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t n0 = blockIdx.x * TN + wave * 16 * NS;
  const uint32_t m0 = blockIdx.y * TM;
  const size_t plane = (size_t)M * K;

  v4i acc[NS][MS][3];
#pragma unroll
  for (int a = 0; a < NS; ++a)
#pragma unroll
    for (int b = 0; b < MS; ++b)
#pragma unroll
      for (int j = 0; j < 3; ++j) acc[a][b][j] = v4i{0, 0, 0, 0};

  const uint32_t lrow = lane & 15, lk = (lane >> 4) * 16;
  for (uint32_t kc = 0; kc < K; kc += kKChunk) {
    const uint32_t kw = (K - kc) < (uint32_t)kKChunk ? (K - kc) : (uint32_t)kKChunk;
    __syncthreads();
    // Stage digits of rows [m0, m0 + TM) and k [kc, kc + kw) into LDS.
    const uint32_t vec_per_row = kw / 16;
    for (uint32_t i = t; i < 3 * TM * vec_per_row; i += kGemmThreads) {
      const uint32_t j = i / (TM * vec_per_row);
      const uint32_t rem = i % (TM * vec_per_row);
      const uint32_t r = rem / vec_per_row, c = rem % vec_per_row;
      uint4 v = make_uint4(0, 0, 0, 0);
      if (m0 + r < M) v = *reinterpret_cast<const uint4*>(D + j * plane + (size_t)(m0 + r) * K + kc + c * 16);
      *reinterpret_cast<uint4*>(&lds[j][r][c * 16]) = v;
    }
    __syncthreads();
    for (uint32_t ks = 0; ks < kw; ks += 64) {
      v4i wa[NS];
#pragma unroll
      for (int a = 0; a < NS; ++a) {
        const uint32_t n = n0 + a * 16 + lrow;
        const uint32_t nn = n < N ? n : N - 1;
        wa[a] = *reinterpret_cast<const v4i*>(W + (size_t)nn * K + kc + ks + lk);
      }
#pragma unroll
      for (int b = 0; b < MS; ++b) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const v4i db = *reinterpret_cast<const v4i*>(&lds[j][b * 16 + lrow][ks + lk]);
#pragma unroll
          for (int a = 0; a < NS; ++a)
            acc[a][b][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[a], db, acc[a][b][j], 0, 0, 0);
        }
      }
    }
  }

  // Epilogue: lane l, element i -> n = n0 + 16a + 4(l/16) + i, m = m0 + 16b + l%16.
#pragma unroll
  for (int a = 0; a < NS; ++a) {
#pragma unroll
    for (int b = 0; b < MS; ++b) {
      const uint32_t m = m0 + b * 16 + lrow;
      if (m >= M) continue;
      const float f = fm[m];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t n = n0 + a * 16 + (lane >> 4) * 4 + i;
        if (n >= N) continue;
        const float c = (float)acc[a][b][0][i] + 256.f * (float)acc[a][b][1][i] +
                        65536.f * (float)acc[a][b][2][i];
        const float v = sw[n] * (f * c);
        float* dst = Y + (size_t)m * ldy + n;
        if constexpr (EPI == 0) *dst = v;
        else if constexpr (EPI == 1) *dst = *dst + v;
        else *dst = silu_f(v);
      }
    }
  }
}

// Row-wise digit split of A (optionally after the zero-centred RMS norm of
// math.ts:16-32): one 256-thread workgroup per row.  Writes D [3][M][K] and
// fm[m] = 2^(E - 21).  With `norm_out`, the normalized row is also stored.
__global__ __launch_bounds__(256) void digitize_kernel(const float* __restrict__ X, uint32_t ldx,
                                                       const float* __restrict__ norm,
                                                       float* __restrict__ norm_out,
                                                       int8_t* __restrict__ D,
                                                       float* __restrict__ fm, uint32_t M,
                                                       uint32_t K) {
  const uint32_t m = blockIdx.x, t = threadIdx.x;
  const float* x = X + (size_t)m * ldx;
  __shared__ float red[8];
  const uint32_t per = (K + 255) / 256;  // K <= 2048 -> per <= 8
  float v[8];
  float ss = 0.f;
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) {
    const uint32_t k = t + i * 256;
    v[i] = (i < per && k < K) ? x[k] : 0.f;
    ss = fmaf(v[i], v[i], ss);
  }
  if (norm) {
    for (int o = 32; o >= 1; o >>= 1) ss += __shfl_xor(ss, o, 64);
    if ((t & 63) == 0) red[t >> 6] = ss;
    __syncthreads();
    ss = red[0] + red[1] + red[2] + red[3];
    __syncthreads();
    const float inv = 1.f / sqrtf(ss / (float)K + 1e-6f);
#pragma unroll
    for (uint32_t i = 0; i < 8; ++i) {
      const uint32_t k = t + i * 256;
      if (i < per && k < K) {
        v[i] = (1.f + norm[k]) * v[i] * inv;
        if (norm_out) norm_out[(size_t)m * K + k] = v[i];
      }
    }
  }
  float amax = 0.f;
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  for (int o = 32; o >= 1; o >>= 1) amax = fmaxf(amax, __shfl_xor(amax, o, 64));
  if ((t & 63) == 0) red[4 + (t >> 6)] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(red[4], red[5]), fmaxf(red[6], red[7]));
  int e = 0;
  if (amax > 0.f) {
    frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
    e -= 1;
  }
  const float up = ldexpf(1.f, 21 - e);
  const size_t plane = (size_t)M * K;
#pragma unroll
  for (uint32_t i = 0; i < 8; ++i) {
    const uint32_t k = t + i * 256;
    if (i < per && k < K) {
      const int X0 = (int)rintf(v[i] * up);  // |X0| < 2^22
      const int d0 = ((X0 + 128) & 255) - 128;
      const int X1 = (X0 - d0) >> 8;
      const int d1 = ((X1 + 128) & 255) - 128;
      const int d2 = (X1 - d1) >> 8;
      D[(size_t)m * K + k] = (int8_t)d0;
      D[plane + (size_t)m * K + k] = (int8_t)d1;
      D[2 * plane + (size_t)m * K + k] = (int8_t)d2;
    }
  }
  if (t == 0) fm[m] = ldexpf(1.f, e - 21);
}

using GemmFn = void (*)(const int8_t*, const float*, const int8_t*, const float*, float*, uint32_t,
                        uint32_t, uint32_t, uint32_t);

template <int EPI>
GemmFn pick(uint32_t ms, uint32_t ns) {
  if (ms == 4) return ns == 2 ? &gemm_i8_digits_kernel<4, 2, EPI> : &gemm_i8_digits_kernel<4, 1, EPI>;
  return ns == 2 ? &gemm_i8_digits_kernel<1, 2, EPI> : &gemm_i8_digits_kernel<1, 1, EPI>;
}

}  // namespace

hipError_t nd_launch_digitize(const float* x, uint32_t ldx, const float* norm, float* norm_out,
                              int8_t* digits, float* fm, uint32_t M, uint32_t K, hipStream_t s) {
  if (M == 0) return hipSuccess;
  hipLaunchKernelGGL(digitize_kernel, dim3(M), dim3(256), 0, s, x, ldx, norm, norm_out, digits, fm,
                     M, K);
  return hipGetLastError();
}

// Tile choice: decode-sized M (<= 64) uses 16-row m tiles so that even
// N = 512 spreads over 32+ workgroups; prefill-sized M uses 64 x 128 tiles.
hipError_t nd_launch_gemm(const nd_mat* w, const int8_t* digits, const float* fm, float* y,
                          uint32_t ldy, uint32_t M, int epilogue, hipStream_t s) {
  if (M == 0) return hipSuccess;
  const uint32_t ms = M > 64 ? 4 : 1;
  const uint32_t ns = (M > 64 || w->n >= 8192) ? 2 : 1;
  const uint32_t tm = 16 * ms, tn = 64 * ns;
  GemmFn f = epilogue == 0 ? pick<0>(ms, ns) : epilogue == 1 ? pick<1>(ms, ns) : pick<2>(ms, ns);
  dim3 grid((w->n + tn - 1) / tn, (M + tm - 1) / tm);
  hipLaunchKernelGGL(f, grid, dim3(kGemmThreads), 0, s, w->w, w->scales, digits, fm, y, M, w->n,
                     w->k, ldy);
  return hipGetLastError();
}
