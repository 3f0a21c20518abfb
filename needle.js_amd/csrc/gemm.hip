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
#include "nd_rope.hpp"
#include "nd_wave.hpp"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

constexpr int kGemmThreads = 256;
constexpr int kKChunk = 256;             // k per LDS stage
constexpr int kLdsRow = kKChunk + 16;    // padded row stride (bank spread)
constexpr int kMaxSplit = 8;             // k slices of a split launch
constexpr uint32_t kMaxNormK = 1024;     // rows the fused norm reads whole

__device__ __forceinline__ float silu_f(float v) { return v / (1.f + __expf(-v)); }

// Digit split of X = rint(v up), |X| <= 2^22, into signed base-256 digits
// X = d0 + 256 d1 + 65536 d2 (d0 = X - 256 round(X / 256) with halves
// rounded up, and so on; d2 in [-64, 64]).  v up + 1.5 2^23 rounds to the
// integer 1.5 2^23 + X (to even on ties, as rint: 1.5 2^23 is even), whose
// bit pattern over [2^23, 2^24] is 0x4B400000 + X; plus 0x408080 its low 24
// bits are X + 0x808080, whose bytes are d_i + 128 -- the digits' bytes
// with bit 7 flipped (no carry crosses a byte).  up = 0 gives zero digits.
__device__ __forceinline__ uint32_t digit_bias(float v, float up) {
  return __float_as_uint(fmaf(v, up, 12582912.f)) + 0x408080u;
}
// Four values' digit_bias words to one word per digit plane (value i in
// byte i): byte permutes, then the bit-7 flips.
__device__ __forceinline__ void digit_words(uint32_t a, uint32_t b, uint32_t c, uint32_t d,
                                            uint32_t& w0, uint32_t& w1, uint32_t& w2) {
  const uint32_t ab = __builtin_amdgcn_perm(b, a, 0x05010400u);   // a0 b0 a1 b1
  const uint32_t cd = __builtin_amdgcn_perm(d, c, 0x05010400u);   // c0 d0 c1 d1
  const uint32_t ab2 = __builtin_amdgcn_perm(b, a, 0x0c0c0602u);  // a2 b2 0 0
  const uint32_t cd2 = __builtin_amdgcn_perm(d, c, 0x0c0c0602u);  // c2 d2 0 0
  w0 = __builtin_amdgcn_perm(cd, ab, 0x05040100u) ^ 0x80808080u;
  w1 = __builtin_amdgcn_perm(cd, ab, 0x07060302u) ^ 0x80808080u;
  w2 = __builtin_amdgcn_perm(cd2, ab2, 0x05040100u) ^ 0x80808080u;
}

// MS m-subtiles of 16 and NS n-subtiles of 16 per wave; 4 waves split n.
// blockIdx.z selects the k slice [z * kslice, +kslice) (kslice = K without a
// split).  Each 256-wide chunk issues its weight loads first and then stages
// the digit planes through LDS, so one round trip serves both.  With
// gridDim.z = S > 1 every workgroup stores its tile's partial sums (fp32 of
// the three exact integer sums) with agent-coherent stores, counts itself in
// on the tile's counter, and the last of the S to arrive adds the partials in
// slice order (deterministic), applies the epilogue and resets the counter.
template <int MS, int NS, int EPI, bool PF>
__global__ __launch_bounds__(kGemmThreads) void gemm_i8_digits_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ sw, const int8_t* __restrict__ D,
    const float* __restrict__ fm, float* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
    uint32_t ldy, uint32_t kslice, float* __restrict__ part, uint32_t* __restrict__ counters) {
  constexpr int TM = 16 * MS;
  constexpr int TN = 4 * 16 * NS;
  constexpr int kSlots = MS * NS * 4;  // outputs per thread
  __shared__ __attribute__((aligned(16))) int8_t lds[3][TM][kLdsRow];

  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t n0 = blockIdx.x * TN + wave * 16 * NS;
  const uint32_t m0 = blockIdx.y * TM;
  const uint32_t S = gridDim.z;
  const uint32_t k_begin = blockIdx.z * kslice;
  const uint32_t k_end = K - k_begin < kslice ? K : k_begin + kslice;
  const size_t plane = (size_t)M * K;

  v4i acc[NS][MS][3];
#pragma unroll
  for (int a = 0; a < NS; ++a)
#pragma unroll
    for (int b = 0; b < MS; ++b)
#pragma unroll
      for (int j = 0; j < 3; ++j) acc[a][b][j] = v4i{0, 0, 0, 0};

  const uint32_t lrow = lane & 15, lk = (lane >> 4) * 16;
  // A chunk's operands in registers: the weights (lane: 16 k of row n) and
  // this thread's share of the digit staging, kDv 16-byte pieces (plane j,
  // row r, piece c of the chunk's 16), all issued together.  With PF the
  // next chunk's are issued before the current chunk's products (one memory
  // round trip overlaps the MFMA work, for twice the operand registers).
  constexpr int kVec = kKChunk / 16;                       // 16-byte pieces per row and plane
  constexpr int kDv = 3 * TM * kVec / kGemmThreads;         // pieces per thread
  static_assert(3 * TM * kVec % kGemmThreads == 0, "the staging divides evenly");
  v4i wa[kKChunk / 64][NS];
  uint4 dv[kDv];
  auto load_chunk = [&](uint32_t kc) {
    const uint32_t kw = (k_end - kc) < (uint32_t)kKChunk ? (k_end - kc) : (uint32_t)kKChunk;
#pragma unroll
    for (int q = 0; q < kKChunk / 64; ++q) {
      const uint32_t ks = (uint32_t)q * 64 < kw ? q * 64 : 0;  // clamped past kw, never used
#pragma unroll
      for (int a = 0; a < NS; ++a) {
        const uint32_t n = n0 + a * 16 + lrow;
        const uint32_t nn = n < N ? n : N - 1;
        wa[q][a] = *reinterpret_cast<const v4i*>(W + (size_t)nn * K + kc + ks + lk);
      }
    }
#pragma unroll
    for (int u = 0; u < kDv; ++u) {
      const uint32_t i = t + u * kGemmThreads;
      const uint32_t j = i / (TM * kVec), r = (i / kVec) % TM, c = i % kVec;
      const uint32_t rr = m0 + r < M ? m0 + r : M - 1;
      const uint32_t cc = c * 16 < kw ? c * 16 : 0;
      dv[u] = *reinterpret_cast<const uint4*>(D + j * plane + (size_t)rr * K + kc + cc);
    }
  };
  load_chunk(k_begin);
  for (uint32_t kc = k_begin; kc < k_end; kc += kKChunk) {
    const uint32_t kw = (k_end - kc) < (uint32_t)kKChunk ? (k_end - kc) : (uint32_t)kKChunk;
    if (!PF && kc != k_begin) load_chunk(kc);
    __syncthreads();  // every wave is done with the previous chunk's digits
#pragma unroll
    for (int u = 0; u < kDv; ++u) {
      const uint32_t i = t + u * kGemmThreads;
      const uint32_t j = i / (TM * kVec), r = (i / kVec) % TM, c = i % kVec;
      // rows past M multiply as zeros (pieces past kw are never read)
      *reinterpret_cast<uint4*>(&lds[j][r][c * 16]) = m0 + r < M ? dv[u] : make_uint4(0, 0, 0, 0);
    }
    v4i wc[kKChunk / 64][NS];
#pragma unroll
    for (int q = 0; q < kKChunk / 64; ++q)
#pragma unroll
      for (int a = 0; a < NS; ++a) wc[q][a] = wa[q][a];
    if (PF && kc + kKChunk < k_end) load_chunk(kc + kKChunk);
    nd::lds_barrier();
#pragma unroll
    for (int q = 0; q < kKChunk / 64; ++q) {
      if ((uint32_t)q * 64 >= kw) break;
#pragma unroll
      for (int b = 0; b < MS; ++b) {
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const v4i db = *reinterpret_cast<const v4i*>(&lds[j][b * 16 + lrow][q * 64 + lk]);
#pragma unroll
          for (int a = 0; a < NS; ++a)
            acc[a][b][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wc[q][a], db, acc[a][b][j], 0, 0, 0);
        }
      }
    }
  }

  // Output (a, b, i) of lane l: n = n0 + 16a + 4(l/16) + i, m = m0 + 16b + l%16.
  auto emit = [&](int a, int b, int i, float c) {
    const uint32_t m = m0 + b * 16 + lrow;
    const uint32_t n = n0 + a * 16 + (lane >> 4) * 4 + i;
    if (m >= M || n >= N) return;
    const float v = sw[n] * (fm[m] * c);
    float* dst = Y + (size_t)m * ldy + n;
    if constexpr (EPI == 0) *dst = v;
    else if constexpr (EPI == 1) *dst = *dst + v;
    else *dst = silu_f(v);
  };
  float cs[kSlots];
#pragma unroll
  for (int a = 0; a < NS; ++a)
#pragma unroll
    for (int b = 0; b < MS; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        cs[(a * MS + b) * 4 + i] = (float)acc[a][b][0][i] + 256.f * (float)acc[a][b][1][i] +
                                   65536.f * (float)acc[a][b][2][i];
  if constexpr (MS == 1 && NS == 1) {  // the decode tile; the launcher splits no other
  if (S > 1) {
    const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
    float* mine = part + ((size_t)tile * S + blockIdx.z) * (TM * TN);
#pragma unroll
    for (int q = 0; q < kSlots; ++q)
      __hip_atomic_store(mine + q * kGemmThreads + t, cs[q], __ATOMIC_RELAXED,
                         __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // every store above has completed
    __syncthreads();
    __shared__ uint32_t s_last;
    if (t == 0)
      s_last = __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED,
                                      __HIP_MEMORY_SCOPE_AGENT) == S - 1;
    __syncthreads();
    if (!s_last) return;
    const float* all = part + (size_t)tile * S * (TM * TN);
    float pv[kMaxSplit][kSlots];
#pragma unroll
    for (int z = 0; z < kMaxSplit; ++z) {
      const uint32_t zc = (uint32_t)z < S ? z : 0;  // past S: reread slice 0, then drop
#pragma unroll
      for (int q = 0; q < kSlots; ++q)
        pv[z][q] = __hip_atomic_load(all + (size_t)zc * (TM * TN) + q * kGemmThreads + t,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int q = 0; q < kSlots; ++q) {
      float sum = pv[0][q];
#pragma unroll
      for (int z = 1; z < kMaxSplit; ++z)
        if ((uint32_t)z < S) sum += pv[z][q];
      cs[q] = sum;
    }
    if (t == 0) __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  }
#pragma unroll
  for (int a = 0; a < NS; ++a)
#pragma unroll
    for (int b = 0; b < MS; ++b)
#pragma unroll
      for (int i = 0; i < 4; ++i) emit(a, b, i, cs[(a * MS + b) * 4 + i]);
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
      const uint32_t u = digit_bias(v[i], up);
      D[(size_t)m * K + k] = (int8_t)(u ^ 0x80u);
      D[plane + (size_t)m * K + k] = (int8_t)((u >> 8) ^ 0x80u);
      D[2 * plane + (size_t)m * K + k] = (int8_t)((u >> 16) ^ 0x80u);
    }
  }
  if (t == 0) fm[m] = ldexpf(1.f, e - 21);
}

// The same split with one wave per row (4 rows per workgroup): lane l holds
// the float4 units l + 64 i of the row (VEC units, K <= 256 VEC), so the
// sum of squares and the maximum are wave reductions on DPP and no barrier
// is needed; each unit's three digit bytes go out as one 32-bit word per
// plane.  Requires 16-byte aligned rows and K % 4 == 0.
template <int VEC>
__global__ __launch_bounds__(256) void digitize_rows_kernel(const float* __restrict__ X,
                                                            uint32_t ldx,
                                                            const float* __restrict__ norm,
                                                            float* __restrict__ norm_out,
                                                            int8_t* __restrict__ D,
                                                            float* __restrict__ fm, uint32_t M,
                                                            uint32_t K) {
  const uint32_t lane = threadIdx.x & 63;
  const uint32_t m = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (m >= M) return;
  const float4* x = reinterpret_cast<const float4*>(X + (size_t)m * ldx);
  const uint32_t units = K / 4;
  float4 v[VEC];
  float4 w[VEC];
  float ss = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const uint32_t u = lane + 64 * i;
    v[i] = u < units ? x[u] : make_float4(0.f, 0.f, 0.f, 0.f);
    if (norm) w[i] = u < units ? reinterpret_cast<const float4*>(norm)[u] : make_float4(0.f, 0.f, 0.f, 0.f);
  }
  if (norm) {
#pragma unroll
    for (int i = 0; i < VEC; ++i)
      ss = fmaf(v[i].x, v[i].x, fmaf(v[i].y, v[i].y, fmaf(v[i].z, v[i].z, fmaf(v[i].w, v[i].w, ss))));
    ss = nd::wave_sum(ss);
    const float inv = 1.f / sqrtf(ss / (float)K + 1e-6f);
#pragma unroll
    for (int i = 0; i < VEC; ++i) {
      v[i].x = (1.f + w[i].x) * v[i].x * inv;
      v[i].y = (1.f + w[i].y) * v[i].y * inv;
      v[i].z = (1.f + w[i].z) * v[i].z * inv;
      v[i].w = (1.f + w[i].w) * v[i].w * inv;
      const uint32_t u = lane + 64 * i;
      if (norm_out && u < units) reinterpret_cast<float4*>(norm_out + (size_t)m * K)[u] = v[i];
    }
  }
  float amax = 0.f;
#pragma unroll
  for (int i = 0; i < VEC; ++i)
    amax = fmaxf(amax, fmaxf(fmaxf(fabsf(v[i].x), fabsf(v[i].y)), fmaxf(fabsf(v[i].z), fabsf(v[i].w))));
  amax = nd::row_max(amax);
  amax = fmaxf(fmaxf(nd::readlane(amax, 0), nd::readlane(amax, 16)),
               fmaxf(nd::readlane(amax, 32), nd::readlane(amax, 48)));
  int e = 0;
  if (amax > 0.f) {
    frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
    e -= 1;
  }
  const float up = ldexpf(1.f, 21 - e);
  const size_t plane = (size_t)M * K;
  uint32_t* d0p = reinterpret_cast<uint32_t*>(D + (size_t)m * K);
  uint32_t* d1p = reinterpret_cast<uint32_t*>(D + plane + (size_t)m * K);
  uint32_t* d2p = reinterpret_cast<uint32_t*>(D + 2 * plane + (size_t)m * K);
#pragma unroll
  for (int i = 0; i < VEC; ++i) {
    const uint32_t u = lane + 64 * i;
    if (u >= units) continue;
    uint32_t w0, w1, w2;
    digit_words(digit_bias(v[i].x, up), digit_bias(v[i].y, up), digit_bias(v[i].z, up),
                digit_bias(v[i].w, up), w0, w1, w2);
    d0p[u] = w0;
    d1p[u] = w1;
    d2p[u] = w2;
  }
  if (lane == 0) fm[m] = ldexpf(1.f, e - 21);
}

// Decode-shaped product (M <= 64 rows per launch, 16 x 64 output tiles) that
// digitizes its own activations: workgroup (n tile, m tile, z) reads the fp32
// rows of its CPW 16 x 256 k chunks [CPW z, CPW z + CPW) (and, with NORM, the
// whole rows for the zero-centred RMS norm of math.ts:16-32), writes the
// three digit planes of each chunk with the chunk's own exponent -- 2^(E -
// 21), max |a| in [2^E, 2^(E+1)) over the row's 256 values, so each value is
// carried to 2^-22 of the chunk's largest -- and multiplies them as the
// kernel above, adding the chunks' scaled sums in k order.  All of its
// chunks' loads are issued together (one memory round trip).  Thread t of
// the staging holds row t / 16, columns [16 (t % 16), +16) of each chunk: a
// row is one DPP row of 16 lanes, so its sum of squares and its maximum are
// DPP reductions.  Slices (gridDim.z = K / (256 CPW)) are combined as in the
// kernel above, each partial already scaled by its chunks' factors.
template <int EPI, bool NORM, int CPW>
__global__ __launch_bounds__(kGemmThreads) void gemm_i8_f32a_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ sw, const float* __restrict__ X,
    uint32_t ldx, const float* __restrict__ norm, float* __restrict__ Y, uint32_t M, uint32_t N,
    uint32_t K, uint32_t ldy, float* __restrict__ part, uint32_t* __restrict__ counters,
    nd::RopeStore rope, uint32_t xcd_local) {
  __shared__ __attribute__((aligned(16))) int8_t lds[CPW][3][16][kLdsRow];
  __shared__ float s_fm[CPW][16];
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t n0 = blockIdx.x * 64 + wave * 16;
  const uint32_t m0 = blockIdx.y * 16;
  const uint32_t S = gridDim.z, kc0 = blockIdx.z * CPW * kKChunk;
  const uint32_t lrow = lane & 15, lk = (lane >> 4) * 16;

  // Weights of the chunks first.
  v4i wa[CPW][kKChunk / 64];
  {
    const uint32_t n = n0 + lrow;
    const int8_t* wr = W + (size_t)(n < N ? n : N - 1) * K + kc0 + lk;
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int q = 0; q < kKChunk / 64; ++q)
        wa[c][q] = *reinterpret_cast<const v4i*>(wr + c * kKChunk + q * 64);
  }
  // Activations: row r of the tile, 16 values of each chunk (and the row's
  // other chunks for the norm; K <= kMaxNormK then).
  const uint32_t r = t >> 4, pc = t & 15;
  const uint32_t m = m0 + r;
  const float* xr = X + (size_t)(m < M ? m : M - 1) * ldx;
  float v[CPW][16];
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    const float4* src = reinterpret_cast<const float4*>(xr + kc0 + c * kKChunk + pc * 16);
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const float4 f = src[q];
      v[c][4 * q] = f.x; v[c][4 * q + 1] = f.y; v[c][4 * q + 2] = f.z; v[c][4 * q + 3] = f.w;
    }
  }
  float4 wn[CPW][4];  // the chunks' norm weights, in flight with the activations
  if constexpr (NORM) {
#pragma unroll
    for (int c = 0; c < CPW; ++c) {
      const float4* src = reinterpret_cast<const float4*>(norm + kc0 + c * kKChunk + pc * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) wn[c][q] = src[q];
    }
  }
  // Epilogue 1's addends (this lane's 4 outputs of y), loaded with the
  // product's operands instead of after the product: no load round trip at
  // the end.
  float e_add[4] = {0.f, 0.f, 0.f, 0.f};
  if constexpr (EPI == 1) {
    const uint32_t mo = m0 + lrow;
    if (mo < M) {
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const uint32_t n = n0 + (lane >> 4) * 4 + i;
        if (n < N) e_add[i] = Y[(size_t)mo * ldy + n];
      }
    }
  }
  // Epilogue 3's operands, loaded after the product's so that they do not
  // delay them: wave w's rows m0 + 4 w + r (w uniform: scalar loads of the
  // positions), the rope angles of this lane's pair and the head's norm
  // weight.
  uint32_t e_m[4] = {}, e_pos[4] = {};
  bool e_live[4] = {};
  double2 e_sc[4] = {};
  float e_scale = 0.f;
  if constexpr (EPI == 3) {
    const uint32_t slot = blockIdx.x, wu = __builtin_amdgcn_readfirstlane(wave);
    const bool rope_head = slot < rope.heads + rope.kv_heads;
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      e_m[r] = m0 + wu * 4 + r;
      e_live[r] = e_m[r] < M;
    }
    if (e_live[3] && (reinterpret_cast<uintptr_t>(rope.positions) & 15) == 0) {
      // One 16-byte scalar load (m0 + 4 w is a multiple of 4).
      const uint4 pv = *reinterpret_cast<const uint4*>(rope.positions + e_m[0]);
      e_pos[0] = pv.x, e_pos[1] = pv.y, e_pos[2] = pv.z, e_pos[3] = pv.w;
    } else {
#pragma unroll
      for (int r = 0; r < 4; ++r) e_pos[r] = rope.positions[e_live[r] ? e_m[r] : M - 1];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      const uint32_t pc = e_pos[r] < rope.alloc ? e_pos[r] : rope.alloc - 1;
      if (rope_head) e_sc[r] = rope.rope_tab[(size_t)pc * 32 + (lane & 31)];
    }
    if (rope_head) e_scale = (slot < rope.heads ? rope.q_norm : rope.k_norm)[lane];
  }
  if constexpr (NORM) {
    // The row's sum of squares in k order of the chunks: own chunks from
    // registers, the others read here.
    float ss = 0.f;
    for (uint32_t c0 = 0; c0 < K; c0 += kKChunk) {
      if (c0 >= kc0 && c0 < kc0 + CPW * kKChunk) {
#pragma unroll
        for (int c = 0; c < CPW; ++c)
          if (c0 == kc0 + c * kKChunk)
#pragma unroll
            for (int i = 0; i < 16; ++i) ss = fmaf(v[c][i], v[c][i], ss);
        continue;
      }
      const float4* o = reinterpret_cast<const float4*>(xr + c0 + pc * 16);
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 f = o[q];
        ss = fmaf(f.x, f.x, fmaf(f.y, f.y, fmaf(f.z, f.z, fmaf(f.w, f.w, ss))));
      }
    }
    ss = nd::row_sum(ss);
    const float inv = 1.f / sqrtf(ss / (float)K + 1e-6f);
#pragma unroll
    for (int c = 0; c < CPW; ++c)
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        const float4 f = wn[c][q];
        v[c][4 * q] = (1.f + f.x) * v[c][4 * q] * inv;
        v[c][4 * q + 1] = (1.f + f.y) * v[c][4 * q + 1] * inv;
        v[c][4 * q + 2] = (1.f + f.z) * v[c][4 * q + 2] * inv;
        v[c][4 * q + 3] = (1.f + f.w) * v[c][4 * q + 3] * inv;
      }
  }
  const bool live = m < M;  // rows past M multiply as zeros
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    float amax = 0.f;
#pragma unroll
    for (int i = 0; i < 16; ++i) amax = fmaxf(amax, fabsf(v[c][i]));
    amax = nd::row_max(amax);
    int e = 0;
    if (amax > 0.f) {
      frexpf(amax, &e);  // amax in [2^(e-1), 2^e)
      e -= 1;
    }
    const float up = live ? ldexpf(1.f, 21 - e) : 0.f;
    uint32_t d0w[4], d1w[4], d2w[4];
#pragma unroll
    for (int j = 0; j < 4; ++j)
      digit_words(digit_bias(v[c][4 * j], up), digit_bias(v[c][4 * j + 1], up),
                  digit_bias(v[c][4 * j + 2], up), digit_bias(v[c][4 * j + 3], up), d0w[j],
                  d1w[j], d2w[j]);
    *reinterpret_cast<uint4*>(&lds[c][0][r][pc * 16]) = make_uint4(d0w[0], d0w[1], d0w[2], d0w[3]);
    *reinterpret_cast<uint4*>(&lds[c][1][r][pc * 16]) = make_uint4(d1w[0], d1w[1], d1w[2], d1w[3]);
    *reinterpret_cast<uint4*>(&lds[c][2][r][pc * 16]) = make_uint4(d2w[0], d2w[1], d2w[2], d2w[3]);
    if (pc == 0) s_fm[c][r] = ldexpf(1.f, e - 21);
  }
  __syncthreads();

  // Lane l, element i: n = n0 + 4 (l / 16) + i, m = m0 + l % 16.
  float cs[4] = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int c = 0; c < CPW; ++c) {
    v4i acc[3] = {v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}, v4i{0, 0, 0, 0}};
#pragma unroll
    for (int q = 0; q < kKChunk / 64; ++q) {
#pragma unroll
      for (int j = 0; j < 3; ++j) {
        const v4i db = *reinterpret_cast<const v4i*>(&lds[c][j][lrow][q * 64 + lk]);
        acc[j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[c][q], db, acc[j], 0, 0, 0);
      }
    }
    const float fm = s_fm[c][lrow];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const float ci = fm * ((float)acc[0][i] + 256.f * (float)acc[1][i] + 65536.f * (float)acc[2][i]);
      cs[i] = c == 0 ? ci : cs[i] + ci;
    }
  }
  if (S > 1) {
    const uint32_t tile = blockIdx.y * gridDim.x + blockIdx.x;
    // Workgroup (x, y, z) runs on XCD (tile + tiles z) % 8: with a multiple
    // of 8 tiles every slice of a tile shares its XCD, and the slice sum
    // stays in that XCD's L2 (workgroup-scope stores and counter; the
    // agent-scope loads below miss the CU's L1 and hit the L2).  xcd_local:
    // the placement was confirmed on this device.
    const bool xl = xcd_local && (gridDim.x * gridDim.y) % 8 == 0;
    float* mine = part + ((size_t)tile * S + blockIdx.z) * 1024;
    if (xl) {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __hip_atomic_store(mine + i * kGemmThreads + t, cs[i], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_WORKGROUP);
    } else {
#pragma unroll
      for (int i = 0; i < 4; ++i)
        __hip_atomic_store(mine + i * kGemmThreads + t, cs[i], __ATOMIC_RELAXED,
                           __HIP_MEMORY_SCOPE_AGENT);
    }
    __builtin_amdgcn_s_waitcnt(0);  // every store above has completed
    __syncthreads();
    __shared__ uint32_t s_last;
    if (t == 0)
      s_last = (xl ? __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_WORKGROUP)
                   : __hip_atomic_fetch_add(counters + tile, 1u, __ATOMIC_RELAXED,
                                            __HIP_MEMORY_SCOPE_AGENT)) == S - 1;
    __syncthreads();
    if (!s_last) return;
    const float* all = part + (size_t)tile * S * 1024;
    float pv[kMaxSplit][4];
#pragma unroll
    for (int z = 0; z < kMaxSplit; ++z) {
      const uint32_t zc = (uint32_t)z < S ? z : 0;  // past S: reread slice 0, then drop
#pragma unroll
      for (int i = 0; i < 4; ++i)
        pv[z][i] = __hip_atomic_load(all + (size_t)zc * 1024 + i * kGemmThreads + t,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float sum = pv[0][i];
#pragma unroll
      for (int z = 1; z < kMaxSplit; ++z)
        if ((uint32_t)z < S) sum += pv[z][i];
      cs[i] = sum;
    }
    if (t == 0) {
      if (xl)
        __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      else
        __hip_atomic_store(counters + tile, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    }
  }
  if constexpr (EPI == 3) {
    // The tile is one head (column tile blockIdx.x) of 16 rows: through LDS
    // to one row per wave pass, one dimension per lane, then norm, rope and
    // the cache store as the rope/store kernel does from the stored tile.
    // Y, when given, also receives the projections themselves.
    __shared__ float s_head[16][65];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const uint32_t n = n0 + (lane >> 4) * 4 + i;  // < N: N is a multiple of 64 here
      const float val = sw[n] * cs[i];
      s_head[lrow][wave * 16 + (lane >> 4) * 4 + i] = val;
      if (Y && m0 + lrow < M) Y[(size_t)(m0 + lrow) * ldy + n] = val;
    }
    __syncthreads();
    float ex[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) ex[r] = s_head[wave * 4 + r][lane];
    // Keep the norm weight's arithmetic here: hoisted next to its early
    // load, it would make the wave wait for every outstanding load there.
    asm volatile("" : "+v"(e_scale));
    nd::rope_store_rows<4>(ex, e_m, e_live, e_pos, e_sc, e_scale, blockIdx.x, lane, rope);
    return;
  }
  const uint32_t mo = m0 + lrow;
  if (mo >= M) return;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const uint32_t n = n0 + (lane >> 4) * 4 + i;
    if (n >= N) continue;
    const float val = sw[n] * cs[i];
    float* dst = Y + (size_t)mo * ldy + n;
    if constexpr (EPI == 0) *dst = val;
    else if constexpr (EPI == 1) *dst = e_add[i] + val;
    else *dst = silu_f(val);
  }
}

// Prompt-sized product with the activations stationary (M >= 1024, K in
// {128, 256, 512}, N % 128 == 0): workgroup (column group g, row tile m) copies the
// three digit planes of its 64 rows over all of K into LDS once (LDS DMA,
// global_load_lds_dwordx4, no registers) and then streams 128-column weight
// strips through them.  Every weight strip is read by the M / 64 row tiles
// and every digit plane by the N / NG column groups, against one read of
// each per 32 x 64 tile pair for the tiled kernel above -- about a quarter
// of its L2 traffic at 2048 x 2048 x 512.  8 waves in two groups take the
// strips alternately (group h: strips h, h + 2, ...), so one group's weight
// loads overlap the other's products; wave w % 4 of a group takes the
// strip's columns [32 (w % 4), +32).  The integer sums are exact and the
// epilogue is the tiled kernel's, so both give the same bits.
//
// LDS layout: 16-byte units, plane j, row r, unit slot p (U = K / 16 per
// row); slot p holds k-unit p ^ (4 (r % 4) & (U - 1)).  A wave's 16-byte
// read takes k-units 4 q + (l / 16) of rows 16 b + l % 16: the rows' four
// residues mod 4 move those units to four different 64-byte bank groups, so
// the 64 lanes fall on all 16 groups of the 64 banks, four lanes each (the
// minimum of four passes for 1 KiB).
constexpr uint32_t kAsRows = 64, kAsMaxK = 512, kAsStrip = 128;
__device__ __forceinline__ uint32_t as_slot(uint32_t u, uint32_t r, uint32_t U) {
  return u ^ ((4u * (r & 3u)) & (U - 1u));
}
template <int EPI>
__global__ __launch_bounds__(512) void gemm_i8_astat_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ sw, const int8_t* __restrict__ D,
    const float* __restrict__ fm, float* __restrict__ Y, uint32_t M, uint32_t N, uint32_t K,
    uint32_t ldy, uint32_t group_cols) {
  __shared__ __attribute__((aligned(16))) int8_t lds[3 * kAsRows * kAsMaxK];
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t half = wave >> 2, wq = wave & 3;
  const uint32_t m0 = blockIdx.y * kAsRows;
  const uint32_t c0 = blockIdx.x * group_cols;
  const uint32_t U = K / 16;  // units per row
  const size_t plane = (size_t)M * K;

  // Stage the tile: 3 * 64 * U units in chunks of 64 (one wave load each).
  {
    const uint32_t chunks = 3 * kAsRows * U / 64;
    for (uint32_t c = wave; c < chunks; c += 8) {
      const uint32_t L = c * 64 + lane;
      const uint32_t j = L / (kAsRows * U), r = (L / U) % kAsRows, pslot = L % U;
      const uint32_t u = as_slot(pslot, r, U);  // the slot map is its own inverse
      const uint32_t row = m0 + r < M ? m0 + r : M - 1;  // rows past M feed only rows past M
      __builtin_amdgcn_global_load_lds(D + j * plane + (size_t)row * K + u * 16,
                                       (__attribute__((address_space(3))) void*)(lds + c * 1024),
                                       16, 0, 0);
    }
  }
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();

  const uint32_t lrow = lane & 15, lk = lane >> 4;
  const uint32_t steps = K / 64;
  for (uint32_t s0 = half * kAsStrip; s0 < group_cols; s0 += 2 * kAsStrip) {
    const uint32_t nb = c0 + s0 + 32 * wq;  // this wave's 32 columns
    // The strip's weights for both 16-column tiles and every k step.
    v4i wa[kAsMaxK / 64][2];
#pragma unroll
    for (int q = 0; q < (int)(kAsMaxK / 64); ++q)
#pragma unroll
      for (int a = 0; a < 2; ++a) {
        const uint32_t n = nb + 16 * a + lrow;
        const uint32_t qs = (uint32_t)q < steps ? q : 0;
        wa[q][a] = *reinterpret_cast<const v4i*>(W + (size_t)(n < N ? n : N - 1) * K + qs * 64 +
                                                 lk * 16);
      }
    v4i acc[2][4][3];
#pragma unroll
    for (int a = 0; a < 2; ++a)
#pragma unroll
      for (int b = 0; b < 4; ++b)
#pragma unroll
        for (int j = 0; j < 3; ++j) acc[a][b][j] = v4i{0, 0, 0, 0};
#pragma unroll
    for (int q = 0; q < (int)(kAsMaxK / 64); ++q) {
      if ((uint32_t)q >= steps) break;
      const uint32_t u = 4 * q + lk;
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t r = 16 * b + lrow;
        const uint32_t pslot = as_slot(u, r, U);
#pragma unroll
        for (int j = 0; j < 3; ++j) {
          const v4i db = *reinterpret_cast<const v4i*>(
              &lds[((j * kAsRows + r) * U + pslot) * 16]);
#pragma unroll
          for (int a = 0; a < 2; ++a)
            acc[a][b][j] = __builtin_amdgcn_mfma_i32_16x16x64_i8(wa[q][a], db, acc[a][b][j], 0, 0, 0);
        }
      }
    }
    // Output (a, b, i) of lane l: n = nb + 16 a + 4 (l / 16) + i, m = m0 + 16 b + l % 16.
#pragma unroll
    for (int a = 0; a < 2; ++a) {
      const uint32_t n = nb + 16 * a + 4 * lk;
      if (n >= N) continue;
      const float4 s4 = *reinterpret_cast<const float4*>(sw + n);
      const float swv[4] = {s4.x, s4.y, s4.z, s4.w};
#pragma unroll
      for (int b = 0; b < 4; ++b) {
        const uint32_t m = m0 + 16 * b + lrow;
        if (m >= M) continue;
        const float f = fm[m];
        float v[4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const float c = (float)acc[a][b][0][i] + 256.f * (float)acc[a][b][1][i] +
                          65536.f * (float)acc[a][b][2][i];
          v[i] = swv[i] * (f * c);
        }
        float4* dst = reinterpret_cast<float4*>(Y + (size_t)m * ldy + n);
        if constexpr (EPI == 1) {
          const float4 o = *dst;
          *dst = make_float4(o.x + v[0], o.y + v[1], o.z + v[2], o.w + v[3]);
        } else if constexpr (EPI == 2) {
          *dst = make_float4(silu_f(v[0]), silu_f(v[1]), silu_f(v[2]), silu_f(v[3]));
        } else {
          *dst = make_float4(v[0], v[1], v[2], v[3]);
        }
      }
    }
  }
}

using F32aFn = void (*)(const int8_t*, const float*, const float*, uint32_t, const float*, float*,
                        uint32_t, uint32_t, uint32_t, uint32_t, float*, uint32_t*, nd::RopeStore,
                        uint32_t);

template <bool NORM, int CPW>
F32aFn pick_f32a(int epilogue) {
  return epilogue == 0 ? &gemm_i8_f32a_kernel<0, NORM, CPW>
       : epilogue == 1 ? &gemm_i8_f32a_kernel<1, NORM, CPW>
       : epilogue == 2 ? &gemm_i8_f32a_kernel<2, NORM, CPW> : &gemm_i8_f32a_kernel<3, NORM, CPW>;
}

using GemmFn = void (*)(const int8_t*, const float*, const int8_t*, const float*, float*, uint32_t,
                        uint32_t, uint32_t, uint32_t, uint32_t, float*, uint32_t*);

template <int EPI>
GemmFn pick(uint32_t ms, uint32_t ns, bool pf) {
  if (ms == 4) {
    if (pf) return ns == 2 ? &gemm_i8_digits_kernel<4, 2, EPI, true> : &gemm_i8_digits_kernel<4, 1, EPI, true>;
    return ns == 2 ? &gemm_i8_digits_kernel<4, 2, EPI, false> : &gemm_i8_digits_kernel<4, 1, EPI, false>;
  }
  if (ms == 2) {
    if (pf) return ns == 2 ? &gemm_i8_digits_kernel<2, 2, EPI, true> : &gemm_i8_digits_kernel<2, 1, EPI, true>;
    return ns == 2 ? &gemm_i8_digits_kernel<2, 2, EPI, false> : &gemm_i8_digits_kernel<2, 1, EPI, false>;
  }
  if (pf) return ns == 2 ? &gemm_i8_digits_kernel<1, 2, EPI, true> : &gemm_i8_digits_kernel<1, 1, EPI, true>;
  return ns == 2 ? &gemm_i8_digits_kernel<1, 2, EPI, false> : &gemm_i8_digits_kernel<1, 1, EPI, false>;
}

}  // namespace

hipError_t nd_launch_digitize(const float* x, uint32_t ldx, const float* norm, float* norm_out,
                              int8_t* digits, float* fm, uint32_t M, uint32_t K, hipStream_t s) {
  if (M == 0) return hipSuccess;
  // One wave per row when rows are 16-byte aligned float4 runs (every caller
  // here); the workgroup-per-row kernel otherwise.
  const bool rows4 = K % 4 == 0 && ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0 &&
                     (!norm || (reinterpret_cast<uintptr_t>(norm) & 15) == 0) &&
                     (!norm_out || (reinterpret_cast<uintptr_t>(norm_out) & 15) == 0) &&
                     (reinterpret_cast<uintptr_t>(digits) & 3) == 0 && K <= 2048;
  if (rows4) {
    const dim3 grid((M + 3) / 4);
    if (K <= 512)
      hipLaunchKernelGGL(digitize_rows_kernel<2>, grid, dim3(256), 0, s, x, ldx, norm, norm_out,
                         digits, fm, M, K);
    else if (K <= 1024)
      hipLaunchKernelGGL(digitize_rows_kernel<4>, grid, dim3(256), 0, s, x, ldx, norm, norm_out,
                         digits, fm, M, K);
    else
      hipLaunchKernelGGL(digitize_rows_kernel<8>, grid, dim3(256), 0, s, x, ldx, norm, norm_out,
                         digits, fm, M, K);
    return hipGetLastError();
  }
  hipLaunchKernelGGL(digitize_kernel, dim3(M), dim3(256), 0, s, x, ldx, norm, norm_out, digits, fm,
                     M, K);
  return hipGetLastError();
}

// Tile choice: decode-sized M (<= 64) uses 16-row m tiles so that even
// N = 512 spreads over 32+ workgroups; prefill-sized M uses 32 x 64 tiles
// (measured at M = 2048 with digitize: 24.2 / 45.3 / 15.7 / 27.9 us for N x K
// = 1536 x 512, 4096 x 512, 512 x 512, 512 x 2048, against 38.9 / 65.3 /
// 21.6 / 43.9 for 64 x 128 tiles and 30.6 / 58.9 / 16.3 / 33.3 for 16 x 64).
// With `split`, a grid of fewer than 256 tiles also splits k (K % 256 == 0)
// into S = 2..8 slices until tiles * S reaches 256, within the workspace
// (16 x 64 tiles only).
hipError_t nd_launch_gemm(const nd_mat* w, const int8_t* digits, const float* fm, float* y,
                          uint32_t ldy, uint32_t M, int epilogue, hipStream_t s,
                          const nd_gemm_split* split) {
  if (M == 0) return hipSuccess;
  // Prompt-sized M with K <= 512: the activation tile stays in LDS.  Column
  // groups of whole 128-column strips, as many as give the row tiles 256
  // workgroups (or fewer when N has fewer strips).
  if (M >= 1024 && (w->k == 128 || w->k == 256 || w->k == 512) && w->n % kAsStrip == 0 &&
      ldy % 4 == 0 &&
      (reinterpret_cast<uintptr_t>(y) & 15) == 0 && (reinterpret_cast<uintptr_t>(digits) & 15) == 0) {
    const uint32_t mt = (M + kAsRows - 1) / kAsRows, strips = w->n / kAsStrip;
    uint32_t groups = (256 + mt - 1) / mt;
    if (groups > strips) groups = strips;
    while (strips % groups) --groups;
    const uint32_t gc = (strips / groups) * kAsStrip;
    const dim3 grid(groups, mt);
    if (epilogue == 0)
      hipLaunchKernelGGL(gemm_i8_astat_kernel<0>, grid, dim3(512), 0, s, w->w, w->scales, digits,
                         fm, y, M, w->n, w->k, ldy, gc);
    else if (epilogue == 1)
      hipLaunchKernelGGL(gemm_i8_astat_kernel<1>, grid, dim3(512), 0, s, w->w, w->scales, digits,
                         fm, y, M, w->n, w->k, ldy, gc);
    else
      hipLaunchKernelGGL(gemm_i8_astat_kernel<2>, grid, dim3(512), 0, s, w->w, w->scales, digits,
                         fm, y, M, w->n, w->k, ldy, gc);
    return hipGetLastError();
  }
  // A wide product at decode M (the 32768-row lm head of a 64-row batch)
  // takes 32 x 128 tiles: 16.1 us with digitize, against 21.2 for 16 x 128
  // tiles with the k prefetch.
  const bool wide = w->n >= 8192 && M <= 64;
  uint32_t ms = M > 64 || wide ? 2 : 1;
  uint32_t ns = wide ? 2 : 1;
  // 32 x 64 tiles only while they still give 256 workgroups (a 128-row
  // prompt through a 1536 x 512 projection would get 96); below that the
  // 16 x 64 tiles spread the product over more CUs.
  if (((w->n + 64 * ns - 1) / (64 * ns)) * ((M + 16 * ms - 1) / (16 * ms)) < 256) ms = ns = 1;
  // The prefetch of the next k chunk pays on the 16-row tiles (split-k
  // decode shapes: 31.2 vs 33.3 us at 512 x 2048); the larger tiles run more
  // workgroups per CU without it.
  const bool pf = ms == 1;
  const uint32_t tm = 16 * ms, tn = 64 * ns;
  GemmFn f = epilogue == 0 ? pick<0>(ms, ns, pf) : epilogue == 1 ? pick<1>(ms, ns, pf)
                                                 : pick<2>(ms, ns, pf);
  dim3 grid((w->n + tn - 1) / tn, (M + tm - 1) / tm, 1);
  const uint32_t tiles = grid.x * grid.y;
  if (split && ms == 1 && ns == 1 && w->k % kKChunk == 0 && tiles <= split->counter_count) {
    const uint32_t chunks = w->k / kKChunk;
    uint32_t S = 1;
    while (S * 2 <= (uint32_t)kMaxSplit && chunks % (S * 2) == 0 && tiles * S < 256 &&
           (size_t)tiles * S * 2 * tm * tn <= split->partial_floats)
      S *= 2;
    grid.z = S;
  }
  hipLaunchKernelGGL(f, grid, dim3(kGemmThreads), 0, s, w->w, w->scales, digits, fm, y, M, w->n,
                     w->k, ldy, w->k / grid.z, split ? split->partials : nullptr,
                     split ? split->counters : nullptr);
  return hipGetLastError();
}

// Decode-shaped product on fp32 activations (optionally RMS-normalized with
// `norm`): one launch instead of digitize + GEMM, for the shapes
// nd_gemm_f32_fits accepts (M <= 64, K % 256 == 0 with K / 256 <= kMaxSplit
// slices, K <= kMaxNormK with a norm, the slices' partials and counters
// within the workspace, 16-byte aligned rows).
bool nd_gemm_f32_fits(const nd_mat* w, const float* x, uint32_t ldx, bool norm, uint32_t M,
                      const nd_gemm_split* split) {
  const uint32_t S = w->k / kKChunk;
  const uint32_t tiles = ((w->n + 63) / 64) * ((M + 15) / 16);
  return M >= 1 && M <= 64 && w->k % kKChunk == 0 && S <= (uint32_t)kMaxSplit &&
         (!norm || w->k <= kMaxNormK) && split &&
         (S == 1 || (tiles <= split->counter_count &&
                     (size_t)tiles * S * 1024 <= split->partial_floats)) &&
         ldx % 4 == 0 && (reinterpret_cast<uintptr_t>(x) & 15) == 0;
}

hipError_t nd_launch_gemm_f32(const nd_mat* w, const float* x, uint32_t ldx, const float* norm,
                              float* y, uint32_t ldy, uint32_t M, int epilogue, hipStream_t s,
                              const nd_gemm_split* split, const nd::RopeStore* rope) {
  if (M == 0) return hipSuccess;
  if (!nd_gemm_f32_fits(w, x, ldx, norm != nullptr, M, split)) return hipErrorInvalidValue;
  if (epilogue == 3 &&
      (!rope || w->n != (rope->heads + 2 * rope->kv_heads) * nd::kRopeHd))
    return hipErrorInvalidValue;
  // Two chunks per workgroup when k has an even number of them: at K = 512
  // the product then needs no cross-workgroup sum, whose round trip costs
  // more than streaming the second chunk.
  const uint32_t chunks = w->k / kKChunk;
  const bool pair = chunks % 2 == 0;
  const uint32_t S = pair ? chunks / 2 : chunks;
  const F32aFn f = pair ? (norm ? pick_f32a<true, 2>(epilogue) : pick_f32a<false, 2>(epilogue))
                        : (norm ? pick_f32a<true, 1>(epilogue) : pick_f32a<false, 1>(epilogue));
  hipLaunchKernelGGL(f, dim3((w->n + 63) / 64, (M + 15) / 16, S), dim3(kGemmThreads), 0, s, w->w,
                     w->scales, x, ldx, norm, y, M, w->n, w->k, ldy, split->partials,
                     split->counters, rope ? *rope : nd::RopeStore{}, nd_xcd_local() ? 1u : 0u);
  return hipGetLastError();
}
