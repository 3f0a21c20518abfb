// Int8-weight matvec for gfx950: y[b][r] = sum_g s[r][g] * sum_{c in g} W[r][c] * x[b][c].
//
// Layout: W int8 [n][k] row-major, s f32 [n][k/g], x f32 [batch][k], y f32 [batch][rows].
// The reference loop is cqMatvecPrepared (backends/cq.ts:106-156): a dot per
// quantization group, scaled by the group's norm and summed per row.
//
// Mapping: a 256-thread workgroup covers `rpp = 256 / tpr` rows per pass and
// RACC passes.  Each thread owns SPT 16-byte segments of the row (one
// 128-bit global load per segment) and keeps the matching x values in
// registers for every row it visits, so x is read once per thread.  Weights
// are streamed with non-temporal 128-bit loads.  Bytes are decoded with the
// unsigned-byte converts: u = b + 128 (byte ^ 0x80), dot = sum u*x - 128*sum x.
// Partial sums (RACC rows x B batch values per thread) are reduced across the
// row's threads through LDS followed by a short DPP butterfly.
#include "nd_internal.hpp"
#include "nd_wave.hpp"

namespace {

constexpr int kThreads = 256;
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <int B, int SPT, int RACC>
__global__ __launch_bounds__(kThreads) void matvec_i8_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ S, const float* __restrict__ X,
    float* __restrict__ Y, uint32_t K, uint32_t groups, uint32_t g16, uint32_t row_start,
    uint32_t row_count, uint32_t tpr_log2, uint32_t x_stride, uint32_t y_stride) {
  constexpr int V = RACC * B;
  const uint32_t t = threadIdx.x;
  const uint32_t tpr = 1u << tpr_log2;
  const uint32_t rpp = kThreads >> tpr_log2;
  const uint32_t sub = t >> tpr_log2;
  const uint32_t lk = t & (tpr - 1);
  const uint32_t row0 = blockIdx.x * rpp * RACC;

  // x first: its loads hit L2 and, since loads complete in issue order, the
  // x sums then overlap the weight loads instead of waiting behind them.
  float xr[B][SPT][16];
  float xs[B][SPT];
#pragma unroll
  for (int b = 0; b < B; ++b) {
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const float4* xp = reinterpret_cast<const float4*>(X + (size_t)b * x_stride) + (lk + j * tpr) * 4;
#pragma unroll
      for (int q = 0; q < 4; ++q) {
        float4 f = xp[q];
        xr[b][j][4 * q + 0] = f.x;
        xr[b][j][4 * q + 1] = f.y;
        xr[b][j][4 * q + 2] = f.z;
        xr[b][j][4 * q + 3] = f.w;
      }
    }
  }

  // Then, per row, the scale and the 16-byte weight segments.
  u32x4 wv[RACC][SPT];
  float sv[RACC][SPT];
  uint32_t grp[SPT];
#pragma unroll
  for (int j = 0; j < SPT; ++j) grp[j] = (lk + j * tpr) / g16;
#pragma unroll
  for (int p = 0; p < RACC; ++p) {
    const uint32_t row = row0 + p * rpp + sub;
    const uint32_t r = row_start + (row < row_count ? row : 0);
    const u32x4* wrow = reinterpret_cast<const u32x4*>(W + (size_t)r * K);
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      sv[p][j] = S[(size_t)r * groups + grp[j]];
      wv[p][j] = __builtin_nontemporal_load(wrow + lk + j * tpr);
    }
  }

#pragma unroll
  for (int b = 0; b < B; ++b) {
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      float sum = 0.f;
#pragma unroll
      for (int q = 0; q < 4; ++q)
        sum += (xr[b][j][4 * q] + xr[b][j][4 * q + 1]) + (xr[b][j][4 * q + 2] + xr[b][j][4 * q + 3]);
      xs[b][j] = sum;
    }
  }

  float acc[V];
#pragma unroll
  for (int i = 0; i < V; ++i) acc[i] = 0.f;

#pragma unroll
  for (int p = 0; p < RACC; ++p) {
#pragma unroll
    for (int j = 0; j < SPT; ++j) {
      const uint32_t words[4] = {wv[p][j].x ^ 0x80808080u, wv[p][j].y ^ 0x80808080u,
                                 wv[p][j].z ^ 0x80808080u, wv[p][j].w ^ 0x80808080u};
      float d[B];
#pragma unroll
      for (int b = 0; b < B; ++b) d[b] = -128.f * xs[b][j];
#pragma unroll
      for (int q = 0; q < 4; ++q) {
#pragma unroll
        for (int e = 0; e < 4; ++e) {
          const float u = (float)((words[q] >> (8 * e)) & 0xffu);
#pragma unroll
          for (int b = 0; b < B; ++b) d[b] = fmaf(u, xr[b][j][4 * q + e], d[b]);
        }
      }
#pragma unroll
      for (int b = 0; b < B; ++b) acc[p * B + b] = fmaf(sv[p][j], d[b], acc[p * B + b]);
    }
  }

  // Reduce each row's partial sums over its tpr threads through LDS.  red is
  // [V][256]: thread t stores its V partials in column t.  Output o = (sub,
  // v) is summed by T = 256 / (rpp * V) threads (a power of two <= 64 that
  // divides 64), each over tpr / T columns, then by a T-lane butterfly.
  __shared__ float red[V * kThreads];
#pragma unroll
  for (int i = 0; i < V; ++i) red[i * kThreads + t] = acc[i];
  __syncthreads();
  const uint32_t outputs = rpp * V;
  const uint32_t T = kThreads / outputs;
  const uint32_t o = t / T, part = t % T;
  const uint32_t osub = o / V, ov = o % V;
  const float* col = red + ov * kThreads + osub * tpr;
  float sum = 0.f;
  for (uint32_t c = part; c < tpr; c += T) sum += col[c];
  // T-lane butterfly: DPP within rows of 16, swizzle / bpermute beyond.
  if (T > 32) sum += nd::lane_xor<32>(sum);
  if (T > 16) sum += nd::lane_xor<16>(sum);
  if (T > 8) sum += nd::lane_xor<8>(sum);
  if (T > 4) sum += nd::lane_xor<4>(sum);
  if (T > 2) sum += nd::lane_xor<2>(sum);
  if (T > 1) sum += nd::lane_xor<1>(sum);
  if (part == 0) {
    const uint32_t p = ov / B, b = ov % B;
    const uint32_t row = row0 + p * rpp + osub;
    if (row < row_count) Y[(size_t)b * y_stride + row] = sum;
  }
}

__global__ void row_kernel(const int8_t* __restrict__ W, const float* __restrict__ S,
                           uint32_t K, uint32_t groups, uint32_t G, uint32_t row,
                           float* __restrict__ out) {
  const uint32_t c = blockIdx.x * blockDim.x + threadIdx.x;
  if (c < K) out[c] = (float)W[(size_t)row * K + c] * S[(size_t)row * groups + c / G];
}

using MatvecFn = void (*)(const int8_t*, const float*, const float*, float*, uint32_t, uint32_t,
                          uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t);

template <int B, int RACC>
MatvecFn pick_spt(uint32_t spt) {
  if constexpr (B <= 4) {
    if (spt == 2) return &matvec_i8_kernel<B, 2, RACC>;
  }
  return &matvec_i8_kernel<B, 1, RACC>;
}

template <int RACC>
MatvecFn pick_b(uint32_t b, uint32_t spt) {
  switch (b) {
    case 1: return pick_spt<1, RACC>(spt);
    case 2: return pick_spt<2, RACC>(spt);
    case 4: return pick_spt<4, RACC>(spt);
    default: return pick_spt<8, RACC>(spt);
  }
}

}  // namespace

// Host-side checks that the kernel's geometry fits the matrix were done by
// the caller (k = 16 * 2^j with 128 <= k <= 8192, g % 16 == 0, k % g == 0).
hipError_t nd_launch_matvec(const nd_mat* m, const float* x, uint32_t batch, uint32_t x_stride,
                            uint32_t row_start, uint32_t row_count, float* y, uint32_t y_stride,
                            hipStream_t s) {
  if (row_count == 0 || batch == 0) return hipSuccess;
  const uint32_t segs = m->k / 16;
  const uint32_t spt = segs > 256 ? segs / 256 : 1;
  const uint32_t tpr = segs / spt;
  uint32_t tpr_log2 = 0;
  while ((1u << tpr_log2) < tpr) ++tpr_log2;
  const uint32_t rpp = kThreads / tpr;
  const uint32_t bmax = 8 / spt;
  const uint32_t groups = m->k / m->g;
  const uint32_t g16 = m->g / 16;
  uint32_t b0 = 0;
  while (b0 < batch) {
    uint32_t left = batch - b0, bc = 1;
    while (bc * 2 <= left && bc * 2 <= bmax) bc *= 2;
    // Rows per pass x batch x passes must give 4..256 outputs per workgroup
    // (the LDS reduction needs T = 256 / outputs <= 64).  8 passes amortize
    // the per-workgroup x loads when there are enough rows.
    uint32_t racc = (bc <= 2 && row_count >= 8 * rpp * 256) ? 8 : 4;
    while (racc > 1 && rpp * racc * bc > kThreads) racc >>= 1;
    const uint32_t blocks = (row_count + rpp * racc - 1) / (rpp * racc);
    MatvecFn f = racc == 8 ? pick_b<8>(bc, spt) : racc == 4 ? pick_b<4>(bc, spt)
               : racc == 2 ? pick_b<2>(bc, spt) : pick_b<1>(bc, spt);
    hipLaunchKernelGGL(f, dim3(blocks), dim3(kThreads), 0, s, m->w, m->scales,
                       x + (size_t)b0 * x_stride, y + (size_t)b0 * y_stride, m->k, groups, g16,
                       row_start, row_count, tpr_log2, x_stride, y_stride);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    b0 += bc;
  }
  return hipSuccess;
}

hipError_t nd_launch_row(const nd_mat* m, uint32_t row, float* out, hipStream_t s) {
  const uint32_t threads = 256;
  hipLaunchKernelGGL(row_kernel, dim3((m->k + threads - 1) / threads), dim3(threads), 0, s, m->w,
                     m->scales, m->k, m->k / m->g, m->g, row, out);
  return hipGetLastError();
}
