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
__device__ __forceinline__ void matvec_i8_body(
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
  // divides 64), each over tpr / T = V columns (all V reads in flight at
  // once), then by a T-lane butterfly.
  __shared__ float red[V * kThreads];
#pragma unroll
  for (int i = 0; i < V; ++i) red[i * kThreads + t] = acc[i];
  __syncthreads();
  const uint32_t outputs = rpp * V;
  const uint32_t T = kThreads / outputs;
  const uint32_t o = t / T, part = t % T;
  const uint32_t osub = o / V, ov = o % V;
  const float* col = red + ov * kThreads + osub * tpr;
  float cv[V];
#pragma unroll
  for (int i = 0; i < V; ++i) cv[i] = col[part + T * i];
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < V; ++i) sum += cv[i];
  // T-lane butterfly: DPP within rows of 16, swizzle / bpermute beyond.
  if (T > 32) sum = nd::sum_xor<32>(sum);
  if (T > 16) sum = nd::sum_xor<16>(sum);
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

template <int B, int SPT, int RACC>
__global__ __launch_bounds__(kThreads) void matvec_i8_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ S, const float* __restrict__ X,
    float* __restrict__ Y, uint32_t K, uint32_t groups, uint32_t g16, uint32_t row_start,
    uint32_t row_count, uint32_t tpr_log2, uint32_t x_stride, uint32_t y_stride) {
  matvec_i8_body<B, SPT, RACC>(W, S, X, Y, K, groups, g16, row_start, row_count, tpr_log2,
                               x_stride, y_stride);
}

// The same body between two reads of the 100 MHz constant clock
// (s_memrealtime): workgroup w writes its entry time and the time its
// stores completed to stamps[2 w], stamps[2 w + 1].  Measurement only: the
// span from the earliest entry to the latest exit is the kernel's body time,
// which excludes the dispatch before its first workgroup and the end-of-
// kernel processing after its last.
template <int B, int SPT, int RACC>
__global__ __launch_bounds__(kThreads) void matvec_i8_stamped_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ S, const float* __restrict__ X,
    float* __restrict__ Y, uint32_t K, uint32_t groups, uint32_t g16, uint32_t row_start,
    uint32_t row_count, uint32_t tpr_log2, uint32_t x_stride, uint32_t y_stride,
    uint64_t* __restrict__ stamps) {
  const uint64_t t0 = wall_clock64();
  matvec_i8_body<B, SPT, RACC>(W, S, X, Y, K, groups, g16, row_start, row_count, tpr_log2,
                               x_stride, y_stride);
  __builtin_amdgcn_s_waitcnt(0);  // this thread's stores have completed
  __syncthreads();
  if (threadIdx.x == 0) {
    const uint64_t t1 = wall_clock64();
    stamps[2 * blockIdx.x] = t0;
    stamps[2 * blockIdx.x + 1] = t1;
  }
}

// Batched form on MFMA (up to 8 rows per launch, g % 32 == 0): fp16 operands with
// the fp32 inputs split exactly enough.  Each workgroup writes into LDS, per
// batch row b with e_b = the exponent of max_k |x[b][k]| (max < 2^e_b),
//   x[b][k] * 2^-e_b = hi + lo,  hi = f16(x * 2^-e_b),  lo = f16(x * 2^-e_b - hi),
// which leaves at most 2^-24 of the row's largest element unrepresented
// (fp32's own rounding step).  Weights are int8, exact in fp16, and fp16 x
// fp16 products are exact in the fp32 MFMA accumulator, so
//   y[b][r] = 2^e_b * sum_g s[r][g] * (sum_{k in g} W[r][k] (hi + lo)[b][k])
// differs from the fp32 dot product only by fp32 accumulation rounding.
//
// v_mfma_f32_16x16x32_f16 with A = the 16 split rows i = (b = i & 7, part =
// i >> 3: hi, lo) and B = 16 weight rows: lane l supplies A row l % 16 and B
// column l % 16, eight k of a 32-wide group, and receives D rows 4 (l / 16)
// + [0, 4) of column l % 16 -- so each lane's four outputs belong to one
// weight row and take one group scale.  Lane block kb = l / 16 holds the
// group's k in [8 kOrder[kb], +8), kOrder = {0, 2, 1, 3}: the order in which
// one 16-byte weight load per lane plus a lane-half swap delivers two groups:
// for a pair of 32-wide groups (2p, 2p + 1), lanes 0..31 (blocks 0, 1) load
// bytes [16 kb, +16) of group 2p and lanes 32..63 the same of group 2p + 1 --
// 64 contiguous bytes per row -- and v_permlane32_swap of (d0, d2) and of
// (d1, d3) gives every lane eight codes of group 2p (k blocks kOrder) and
// eight of group 2p + 1.  The split rows are stored in operand order:
// xs[group][lane] = 8 halves.  Weight loads are issued together and
// unconditionally (addresses clamped, contributions weighted by zero), so
// each MFMA waits only for its operands.
using nd::half8;
using nd::float4v;
using nd::u32x2;
using nd::codes_to_half;
constexpr uint32_t kSplitRows = 8;
// Batch 2 streams faster on the vector kernel (7.5 vs 11 us at 4096 x 4096);
// from 3 rows on (two vector launches) the MFMA path wins.
constexpr uint32_t kMfmaMinBatch = 3;

// Lane block holding k block j of a group (kOrder is its own inverse).
__device__ __forceinline__ uint32_t k_block_lanes(uint32_t j) { return j == 1 ? 2 : j == 2 ? 1 : j; }

constexpr uint32_t kMfmaWaves = 16;

// Cross-wave sum of the MFMA accumulators (already scaled by their split
// exponents) and the store: every wave leaves its four components in red
// ([wave][component][lane], 16 KB of LDS), then wave c < 4 sums component c
// over the waves and adds the lo row to the hi row (lanes l and l + 32) for
// batch row b = 4 (l / 16) + c.
__device__ __forceinline__ void mfma_reduce_store(float4v acc, float* red, uint32_t wave,
                                                  uint32_t lane, uint32_t row0,
                                                  uint32_t row_count, uint32_t bc,
                                                  float* __restrict__ Y, uint32_t y_stride) {
#pragma unroll
  for (int c = 0; c < 4; ++c) red[(wave * 4 + c) * 64 + lane] = acc[c];
  __syncthreads();
  if (wave >= 4) return;
  float sum = 0.f;
#pragma unroll
  for (uint32_t w = 0; w < kMfmaWaves; ++w) sum += red[(w * 4 + wave) * 64 + lane];
  sum = nd::sum_xor<32>(sum);
  const uint32_t b = (lane >> 4) * 4 + wave, row = row0 + (lane & 15);
  if (lane < 32 && row < row_count && b < bc) Y[(size_t)b * y_stride + row] = sum;
}

// k <= 2048: the split done in the workgroup over all of k.  Every
// workgroup reads x (an L2 hit after the first), takes each row's largest
// magnitude, and writes the hi/lo image of x in operand order into LDS (64
// KB at k = 2048) while its weight loads stream in -- one launch, and the
// split's VALU work overlaps the wait for HBM.  Wave w takes the pairs p = w
// + kMfmaWaves i.  Entry e of group g sits
// at g * 64 + (e ^ (g & 15)): a 16-lane write round (16 groups, see the unit
// order below) then covers 16 distinct 16-byte slots, and a wave's read of
// one group stays a permutation within each 256-byte block.
constexpr uint32_t kFusedMaxK = 2048;
constexpr uint32_t kMaxSlices = 16;  // k = 8192 in slices of 512
constexpr int kXUnits = kFusedMaxK / 8 / 128;  // 8-value units of x per thread

template <int NP>
__global__ __launch_bounds__(64 * kMfmaWaves) void matvec_mfma_fused_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ S, const float* __restrict__ X,
    uint32_t x_stride, float* __restrict__ Y, uint32_t K, uint32_t groups, uint32_t gshift,
    uint32_t row_start, uint32_t row_count, uint32_t bc, uint32_t y_stride) {
  __shared__ uint4 s_xs[kFusedMaxK / 32 * 64];
  __shared__ float s_sc[16 * (kFusedMaxK / 32 + 1)];
  __shared__ float s_max[kMfmaWaves];
  __shared__ int s_e[kSplitRows];
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t r16 = lane & 15, kb = lane >> 4;
  const uint32_t row0 = blockIdx.x * 16;
  const uint32_t row = row0 + r16;
  const int8_t* wrow = W + (size_t)(row_start + (row < row_count ? row : row_count - 1)) * K +
                       (kb & 1) * 16 + (kb >> 1) * 32;
  const uint32_t ng = K / 32, npairs = ng / 2;
  const uint32_t per_wave = (npairs + kMfmaWaves - 1) / kMfmaWaves;

  // x: thread t holds row xb = t / 128 and 8-value units j = q + 128 i, with
  // q = 64 h + 4 (l % 16) + l / 16 for lane l of half h of the row's threads.
  const uint32_t xb = t >> 7, upr = K / 8;
  const uint32_t xj = (t & 64) + (lane & 15) * 4 + (lane >> 4);
  const float4* xrow = reinterpret_cast<const float4*>(X + (size_t)(xb < bc ? xb : 0) * x_stride);
  float xv[kXUnits][8];
#pragma unroll
  for (int i = 0; i < kXUnits; ++i) {
    const uint32_t j = xj + 128 * i;
    const uint32_t jj = j < upr ? j : 0;
    const float4 a = xrow[2 * jj], c = xrow[2 * jj + 1];
    const bool ok = j < upr && xb < bc;  // rows past the batch multiply as zeros
    xv[i][0] = ok ? a.x : 0.f; xv[i][1] = ok ? a.y : 0.f;
    xv[i][2] = ok ? a.z : 0.f; xv[i][3] = ok ? a.w : 0.f;
    xv[i][4] = ok ? c.x : 0.f; xv[i][5] = ok ? c.y : 0.f;
    xv[i][6] = ok ? c.z : 0.f; xv[i][7] = ok ? c.w : 0.f;
  }
  // Scales of the 16 rows, [row][group] with a padded row stride.
  const uint32_t sstride = groups + 1;
  constexpr int kSc = 2;  // 16 * groups <= 2048 here
  float sreg[kSc];
#pragma unroll
  for (int i = 0; i < kSc; ++i) {
    const uint32_t e = t + 1024 * i;
    const uint32_t ee = e < 16 * groups ? e : 0;
    const uint32_t r = ee / groups, q = ee % groups;
    const uint32_t srow = row0 + r < row_count ? row0 + r : row_count - 1;
    sreg[i] = S[(size_t)(row_start + srow) * groups + q];
  }

  float4v acc = {0.f, 0.f, 0.f, 0.f};
  u32x4 wv[NP];
  auto load = [&](uint32_t base) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const uint32_t p = wave + kMfmaWaves * (base + i);
      const uint32_t pc = p < npairs ? p : 0;
      wv[i] = __builtin_nontemporal_load(reinterpret_cast<const u32x4*>(wrow + (size_t)pc * 64));
    }
  };
  auto compute = [&](uint32_t base) {
#pragma unroll
    for (int i = 0; i < NP; ++i) {
      const uint32_t p = wave + kMfmaWaves * (base + i);
      const uint32_t pc = p < npairs ? p : 0;
      const auto lo = __builtin_amdgcn_permlane32_swap(wv[i].x, wv[i].z, false, false);
      const auto hi = __builtin_amdgcn_permlane32_swap(wv[i].y, wv[i].w, false, false);
#pragma unroll
      for (int h = 0; h < 2; ++h) {
        const uint32_t g = 2 * pc + h;
        const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(
            __builtin_bit_cast(half8, s_xs[g * 64 + (lane ^ (g & 15))]),
            codes_to_half(u32x2{lo[h], hi[h]}), float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
        const float sv = p < npairs ? s_sc[r16 * sstride + (g >> gshift)] : 0.f;
        acc[0] = fmaf(sv, d[0], acc[0]);
        acc[1] = fmaf(sv, d[1], acc[1]);
        acc[2] = fmaf(sv, d[2], acc[2]);
        acc[3] = fmaf(sv, d[3], acc[3]);
      }
    }
  };
  // Row maxima (rows xb live in waves 2 xb and 2 xb + 1), the split, then
  // the scales to LDS.  The weight loads are issued only once x is here:
  // behind the weight stream x would arrive last and the split could not
  // overlap anything.
  float mx = 0.f;
#pragma unroll
  for (int i = 0; i < kXUnits; ++i)
#pragma unroll
    for (int q = 0; q < 8; ++q) mx = fmaxf(mx, fabsf(xv[i][q]));
  __builtin_amdgcn_sched_barrier(0);
  load(0);
  mx = fmaxf(mx, nd::lane_xor<1>(mx));
  mx = fmaxf(mx, nd::lane_xor<2>(mx));
  mx = fmaxf(mx, nd::lane_xor<4>(mx));
  mx = fmaxf(mx, nd::lane_xor<8>(mx));
  mx = nd::max_xor<16>(mx);
  mx = nd::max_xor<32>(mx);
  if (lane == 0) s_max[wave] = mx;
  nd::lds_barrier();  // the weight loads stay in flight
  const float amax = fmaxf(s_max[2 * xb], s_max[2 * xb + 1]);
  int ex = 0;
  if (amax > 0.f && amax <= 3.4028235e38f) frexpf(amax, &ex);  // amax < 2^ex
  const float down = ldexpf(1.f, -ex);
  if (xj == 0) s_e[xb] = ex;
#pragma unroll
  for (int i = 0; i < kXUnits; ++i) {
    const uint32_t j = xj + 128 * i;
    if (j >= upr) continue;
    half8 hv, lv;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float v = xv[i][q] * down;
      const _Float16 h = (_Float16)v;
      hv[q] = h;
      lv[q] = (_Float16)(v - (float)h);
    }
    const uint32_t g = j >> 2, e = k_block_lanes(j & 3) * 16 + xb;
    s_xs[g * 64 + (e ^ (g & 15))] = __builtin_bit_cast(uint4, hv);
    s_xs[g * 64 + ((e + 8) ^ (g & 15))] = __builtin_bit_cast(uint4, lv);
  }
#pragma unroll
  for (int i = 0; i < kSc; ++i) {
    const uint32_t e = t + 1024 * i;
    if (e < 16 * groups) s_sc[(e / groups) * sstride + e % groups] = sreg[i];
  }
  nd::lds_barrier();

  compute(0);
  for (uint32_t base = NP; base < per_wave; base += NP) {
    load(base);
    compute(base);
  }
  // Output c of lane l belongs to batch row (4 (l / 16) + c) % 8 (ldexp by
  // its exponent: a product with 2^e overflows at e = 128).
#pragma unroll
  for (int c = 0; c < 4; ++c) acc[c] = ldexpf(acc[c], s_e[(4 * kb + c) & 7]);
  __syncthreads();  // every wave is done with s_xs: reuse it for the sums
  mfma_reduce_store(acc, reinterpret_cast<float*>(s_xs), wave, lane, row0, row_count, bc, Y,
                    y_stride);
}

// K-split form of the batched product (k >= 4096): workgroup (row block,
// slice) takes 64 weight rows (4 tiles of 16) over the k-slice [KS s, KS s +
// KS), KS = 256 NP.  Every workgroup of a full-k design reads all of x (128
// KB for 8 fp32 rows at k = 4096) for 64 KB of weights, and the rate at which
// data enters a CU bounds the launch; slicing k cuts x to KS * 32 bytes per
// workgroup (32 KB at KS = 1024) for the same 64 KB of weights.  The split
// into hi/lo halves is taken per (batch row, slice): x * 2^-e_bs with e_bs
// the exponent of the slice's largest magnitude, so the slice's partial sum
// is 2^e_bs times the MFMA sum.  Wave w takes tile w % 4 and the contiguous
// pairs [NP (w / 4), +NP) of the slice.  Partials go to
// P[s][b][row - row_start] with agent-coherent stores; the last slice of a
// row block to count itself in adds the slices in order s = 0, 1, ... (the
// same sum on every run) -- no second launch.
template <int NP>
__global__ __launch_bounds__(64 * kMfmaWaves) void matvec_mfma_slice_kernel(
    const int8_t* __restrict__ W, const float* __restrict__ S, const float* __restrict__ X,
    uint32_t x_stride, float* __restrict__ P, uint32_t* __restrict__ counters,
    float* __restrict__ Y, uint32_t y_stride, uint32_t K, uint32_t groups, uint32_t gshift,
    uint32_t row_start, uint32_t row_count, uint32_t bc, uint32_t xl) {
  constexpr uint32_t KS = 256 * NP, kUnits = KS / 8;  // 8-value units of one batch row
  constexpr uint32_t kSg = KS / 32;                   // 32-wide groups of the slice
  __shared__ uint4 s_xs[kSg * 64];                    // also the cross-wave sums (16 KB)
  __shared__ float s_sc[64 * (kSg + 1)];
  __shared__ float s_max[kMfmaWaves];
  __shared__ int s_e[kSplitRows];
  static_assert(kSg * 64 * 16 >= kMfmaWaves * 4 * 64 * 4, "the sums fit the x image");
  // The grid is laid out so that every slice of a row block runs on one XCD
  // (the dispatcher hands workgroup L to XCD L % 8): row block rb = 8 (L / 8
  // % rpx) + L % 8, slice L / (8 rpx), rpx = ceil(blocks / 8).  The slice sum
  // then stays in that XCD's L2: partials stored and counted at workgroup
  // scope (plain stores, the atomic performed in the L2), read by the last
  // slice with agent-scope loads, which miss the CU's L1 and hit the L2.
  // Without xl (workgroups of one L % 8 not known to share an XCD) the
  // partials and the counter go to the agent coherence point instead.
  const uint32_t nblocks = (row_count + 63) / 64, rpx = (nblocks + 7) / 8;
  const uint32_t L = blockIdx.x, sl = L >> 3, rb = 8 * (sl % rpx) + (L & 7);
  const uint32_t nslices = gridDim.x / (8 * rpx);
  if (rb >= nblocks) return;
  const uint32_t t = threadIdx.x, wave = t >> 6, lane = t & 63;
  const uint32_t r16 = lane & 15, kb = lane >> 4;
  const uint32_t slice = sl / rpx, k0 = slice * KS;
  const uint32_t row0 = rb * 64;
  const uint32_t tile = wave & 3, wq = wave >> 2;

  // x: thread t < 8 kUnits takes batch row xb = t / kUnits, unit j of the
  // slice with j = 64 (u / 64) + 4 (l % 16) + l / 16 for u = t % kUnits, l =
  // u % 64 -- a 16-lane write round then covers 16 distinct groups.
  const bool has_x = t < kSplitRows * kUnits;
  const uint32_t xb = t / kUnits, u = t % kUnits;
  const uint32_t xj = (u & ~63u) + (lane & 15) * 4 + (lane >> 4);
  const float4* xp = reinterpret_cast<const float4*>(
                        X + (size_t)(has_x && xb < bc ? xb : 0) * x_stride + k0) + 2 * xj;
  const float4 xa = xp[0], xc = xp[1];
  // Scales of the 64 rows over the slice's groups, [row][group] padded.
  const uint32_t gs = KS >> gshift >= 32 ? (KS >> gshift) / 32 : 1;  // groups in the slice
  const uint32_t q0 = k0 / (32u << gshift);
  const uint32_t sstride = kSg + 1;
  constexpr int kSc = 64 * kSg / (64 * kMfmaWaves) > 0 ? 64 * kSg / (64 * kMfmaWaves) : 1;
  float sreg[kSc];
#pragma unroll
  for (int i = 0; i < kSc; ++i) {
    const uint32_t e = t + 64 * kMfmaWaves * i;
    const uint32_t ee = e < 64 * gs ? e : 0;
    const uint32_t r = ee / gs, q = ee % gs;
    const uint32_t srow = row0 + r < row_count ? row0 + r : row_count - 1;
    sreg[i] = S[(size_t)(row_start + srow) * groups + q0 + q];
  }
  // Weights: NP pairs of this wave's tile, all in flight at once, issued
  // only after every wave has issued its x and scale loads (a CU serves its
  // waves' loads roughly in issue order: behind the weight stream x would
  // arrive last and the split could not overlap it).
  __builtin_amdgcn_sched_barrier(0);
  __builtin_amdgcn_s_barrier();
  __builtin_amdgcn_sched_barrier(0);
  const uint32_t row = row0 + 16 * tile + r16;
  const int8_t* wrow = W + (size_t)(row_start + (row < row_count ? row : row_count - 1)) * K + k0 +
                       (kb & 1) * 16 + (kb >> 1) * 32;
  u32x4 wv[NP];
#pragma unroll
  for (int i = 0; i < NP; ++i)
    wv[i] = __builtin_nontemporal_load(
        reinterpret_cast<const u32x4*>(wrow + (size_t)(NP * wq + i) * 64));
  __builtin_amdgcn_sched_barrier(0);

  // Slice maxima: a batch row spans kUnits / 64 waves.
  const bool ok = has_x && xb < bc;  // rows past the batch multiply as zeros
  const float xv[8] = {ok ? xa.x : 0.f, ok ? xa.y : 0.f, ok ? xa.z : 0.f, ok ? xa.w : 0.f,
                       ok ? xc.x : 0.f, ok ? xc.y : 0.f, ok ? xc.z : 0.f, ok ? xc.w : 0.f};
  float mx = 0.f;
#pragma unroll
  for (int q = 0; q < 8; ++q) mx = fmaxf(mx, fabsf(xv[q]));
  mx = fmaxf(mx, nd::lane_xor<1>(mx));
  mx = fmaxf(mx, nd::lane_xor<2>(mx));
  mx = fmaxf(mx, nd::lane_xor<4>(mx));
  mx = fmaxf(mx, nd::lane_xor<8>(mx));
  mx = nd::max_xor<16>(mx);
  mx = nd::max_xor<32>(mx);
  if (lane == 0) s_max[wave] = mx;
  nd::lds_barrier();  // the weight loads stay in flight
  if (has_x) {
    constexpr uint32_t kWpr = kUnits / 64;  // waves per batch row
    float amax = 0.f;
#pragma unroll
    for (uint32_t i = 0; i < kWpr; ++i) amax = fmaxf(amax, s_max[xb * kWpr + i]);
    int ex = 0;
    if (amax > 0.f && amax <= 3.4028235e38f) frexpf(amax, &ex);  // amax < 2^ex
    const float down = ldexpf(1.f, -ex);
    if (u == 0) s_e[xb] = ex;
    half8 hv, lv;
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const float v = xv[q] * down;
      const _Float16 h = (_Float16)v;
      hv[q] = h;
      lv[q] = (_Float16)(v - (float)h);
    }
    const uint32_t g = xj >> 2, e = k_block_lanes(xj & 3) * 16 + xb;
    s_xs[g * 64 + (e ^ (g & 15))] = __builtin_bit_cast(uint4, hv);
    s_xs[g * 64 + ((e + 8) ^ (g & 15))] = __builtin_bit_cast(uint4, lv);
  }
#pragma unroll
  for (int i = 0; i < kSc; ++i) {
    const uint32_t e = t + 64 * kMfmaWaves * i;
    if (e < 64 * gs) s_sc[(e / gs) * sstride + e % gs] = sreg[i];
  }
  nd::lds_barrier();

  float4v acc = {0.f, 0.f, 0.f, 0.f};
#pragma unroll
  for (int i = 0; i < NP; ++i) {
    const uint32_t p = NP * wq + i;
    const auto lo = __builtin_amdgcn_permlane32_swap(wv[i].x, wv[i].z, false, false);
    const auto hi = __builtin_amdgcn_permlane32_swap(wv[i].y, wv[i].w, false, false);
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const uint32_t g = 2 * p + h;
      const float4v d = __builtin_amdgcn_mfma_f32_16x16x32_f16(
          __builtin_bit_cast(half8, s_xs[g * 64 + (lane ^ (g & 15))]),
          codes_to_half(u32x2{lo[h], hi[h]}), float4v{0.f, 0.f, 0.f, 0.f}, 0, 0, 0);
      const float sv = s_sc[(16 * tile + r16) * sstride + (g >> gshift)];
      acc[0] = fmaf(sv, d[0], acc[0]);
      acc[1] = fmaf(sv, d[1], acc[1]);
      acc[2] = fmaf(sv, d[2], acc[2]);
      acc[3] = fmaf(sv, d[3], acc[3]);
    }
  }
  // Sum the 4 waves of each tile: red[wave][c][lane]; thread (tile, c, lane)
  // adds its tile's waves, then the lo row onto the hi row (lane + 32).
  float* red = reinterpret_cast<float*>(s_xs);
  __syncthreads();  // every wave is done with the x image
#pragma unroll
  for (int c = 0; c < 4; ++c) red[(wave * 4 + c) * 64 + lane] = acc[c];
  __syncthreads();
  const uint32_t ot = t >> 8, oc = (t >> 6) & 3;
  float sum = 0.f;
#pragma unroll
  for (uint32_t q = 0; q < 4; ++q) sum += red[((4 * q + ot) * 4 + oc) * 64 + lane];
  sum = nd::sum_xor<32>(sum);
  const uint32_t b = (lane >> 4) * 4 + oc, orow = row0 + 16 * ot + (lane & 15);
  if (lane < 32 && orow < row_count && b < bc) {
    float* const pp = P + ((size_t)slice * kSplitRows + b) * row_count + orow;
    if (xl)
      __hip_atomic_store(pp, ldexpf(sum, s_e[b]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
      __hip_atomic_store(pp, ldexpf(sum, s_e[b]), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
  // Count the slice in once its partials are stored (completed in the L2);
  // the last slice of the row block adds all of them in order s = 0, 1, ...
  // and resets the counter for the next launch.  Each row block's counter
  // has a 128-byte line of its own.
  uint32_t* const counter = counters + (size_t)rb * 32;
  __builtin_amdgcn_s_waitcnt(0);
  __syncthreads();
  __shared__ uint32_t s_last;
  if (t == 0)
    s_last = (xl ? __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_WORKGROUP)
                 : __hip_atomic_fetch_add(counter, 1u, __ATOMIC_RELAXED,
                                          __HIP_MEMORY_SCOPE_AGENT)) == nslices - 1;
  __syncthreads();
  if (!s_last) return;
  const uint32_t fb = t >> 6, frow = row0 + (t & 63);
  if (t < 64 * kSplitRows && fb < bc && frow < row_count) {
    float v[kMaxSlices];
#pragma unroll
    for (uint32_t q = 0; q < kMaxSlices; ++q)
      v[q] = q < nslices ? __hip_atomic_load(P + ((size_t)q * kSplitRows + fb) * row_count + frow,
                                             __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                         : 0.f;
    float total = v[0];
#pragma unroll
    for (uint32_t q = 1; q < kMaxSlices; ++q)
      if (q < nslices) total += v[q];
    Y[(size_t)fb * y_stride + frow] = total;
  }
  if (t == 0) {
    if (xl)
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    else
      __hip_atomic_store(counter, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

// Read-only stream over `units` 16-byte units: the matvec's own load form
// (non-temporal 128-bit loads, four in flight per thread), folded by xor into
// one word per workgroup so the loads cannot be dropped.
__global__ __launch_bounds__(kThreads) void stream_read_kernel(const u32x4* __restrict__ src,
                                                               uint64_t units,
                                                               uint32_t* __restrict__ out) {
  const uint64_t stride = (uint64_t)gridDim.x * kThreads;
  uint64_t i = (uint64_t)blockIdx.x * kThreads + threadIdx.x;
  u32x4 f = {0u, 0u, 0u, 0u};
  for (; i + 3 * stride < units; i += 4 * stride) {
    const u32x4 a = __builtin_nontemporal_load(src + i);
    const u32x4 b = __builtin_nontemporal_load(src + i + stride);
    const u32x4 c = __builtin_nontemporal_load(src + i + 2 * stride);
    const u32x4 d = __builtin_nontemporal_load(src + i + 3 * stride);
    f ^= a ^ b ^ c ^ d;
  }
  for (; i < units; i += stride) f ^= __builtin_nontemporal_load(src + i);
  uint32_t w = f.x ^ f.y ^ f.z ^ f.w;
#pragma unroll
  for (int m = 1; m < 64; m <<= 1) w ^= (uint32_t)__shfl_xor((int)w, m, 64);
  __shared__ uint32_t s_w[kThreads / 64];
  if ((threadIdx.x & 63) == 0) s_w[threadIdx.x >> 6] = w;
  __syncthreads();
  if (threadIdx.x == 0) out[blockIdx.x] = s_w[0] ^ s_w[1] ^ s_w[2] ^ s_w[3];
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

// The vector kernel's geometry for the next `left` batch rows of a launch
// over row_count rows: bc batch rows (a power of two, at most 8 / spt),
// spt 16-byte segments per thread, tpr = k / (16 spt) threads a row,
// racc row passes and the workgroup count.
struct VecPlan {
  uint32_t bc, spt, tpr_log2, racc, blocks;
};

VecPlan plan_vector(const nd_mat* m, uint32_t left, uint32_t row_count) {
  VecPlan p{};
  const uint32_t segs = m->k / 16;
  p.spt = segs > 256 ? segs / 256 : 1;
  const uint32_t tpr = segs / p.spt;
  while ((1u << p.tpr_log2) < tpr) ++p.tpr_log2;
  const uint32_t rpp = kThreads / tpr;
  const uint32_t bmax = 8 / p.spt;
  p.bc = 1;
  while (p.bc * 2 <= left && p.bc * 2 <= bmax) p.bc *= 2;
  // Rows per pass x batch x passes must give 4..256 outputs per workgroup
  // (the LDS reduction needs T = 256 / outputs <= 64).  8 passes amortize
  // the per-workgroup x loads when there are enough rows.
  p.racc = (p.bc <= 2 && row_count >= 8 * rpp * 256) ? 8 : 4;
  while (p.racc > 1 && rpp * p.racc * p.bc > kThreads) p.racc >>= 1;
  // Small matrices: fewer passes while that adds workgroups (up to 256),
  // keeping at least 4 outputs per workgroup.
  while (p.racc > 1 && rpp * (p.racc / 2) * p.bc >= 4 &&
         (row_count + rpp * p.racc - 1) / (rpp * p.racc) < 256)
    p.racc >>= 1;
  p.blocks = (row_count + rpp * p.racc - 1) / (rpp * p.racc);
  return p;
}

}  // namespace

// Host-side checks that the kernel's geometry fits the matrix were done by
// the caller (k = 16 * 2^j with 128 <= k <= 8192, g % 16 == 0, k % g == 0).
// With `split` (kMatvecSplitBytes of device memory), batches of 3 or more
// rows of a matrix with g % 32 == 0 run on MFMA, 8 rows per launch: k <=
// 2048 in one fused launch, k >= 4096 as k-slices summed by the last slice
// of each row block (9.2 vs 10.7 us for the fused form at 4096 x 4096 and
// 12.9 vs 17.4 at 4096 x 8192, batch 8; at 4096 x 2048 the fused form wins,
// 6.75 vs 7.1);
// otherwise every row is streamed by the vector kernel.
hipError_t nd_launch_matvec(const nd_mat* m, const float* x, uint32_t batch, uint32_t x_stride,
                            uint32_t row_start, uint32_t row_count, float* y, uint32_t y_stride,
                            hipStream_t s, void* split) {
  if (row_count == 0 || batch == 0) return hipSuccess;
  if (split && batch >= kMfmaMinBatch && m->g % 32 == 0) {
    uint32_t gshift = 0;  // g = 32 << gshift (g divides k, a power of two)
    while ((32u << gshift) < m->g) ++gshift;
    for (uint32_t b0 = 0; b0 < batch; b0 += kSplitRows) {
      const uint32_t bc = batch - b0 < kSplitRows ? batch - b0 : kSplitRows;
      const float* xb = x + (size_t)b0 * x_stride;
      float* yb = y + (size_t)b0 * y_stride;
      if (m->k <= kFusedMaxK) {
        const uint32_t pairs_per_wave = (m->k / 64 + kMfmaWaves - 1) / kMfmaWaves;
        const auto kern = pairs_per_wave >= 2 ? &matvec_mfma_fused_kernel<2>
                                              : &matvec_mfma_fused_kernel<1>;
        hipLaunchKernelGGL(kern, dim3((row_count + 15) / 16), dim3(64 * kMfmaWaves), 0, s, m->w,
                           m->scales, xb, x_stride, yb, m->k, m->k / m->g, gshift, row_start,
                           row_count, bc, y_stride);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
        continue;
      }
      // Slices of 1024 when they give 256 workgroups, else of 512; partials
      // of at most kMatvecPartialBytes per launch (row blocks of 64).
      const bool wide = ((row_count + 63) / 64) * (m->k / 1024) >= 256;
      const uint32_t ks = wide ? 1024 : 512, slices = m->k / ks;
      const size_t cap = kMatvecPartialBytes / sizeof(float) / ((size_t)slices * kSplitRows);
      // Row blocks per launch: within the partials and within the counters
      // (one 32-word line per row block in the split's last 64 KB).
      constexpr size_t kCounterBlocks = (kMatvecSplitBytes - kMatvecPartialBytes) / (32 * 4);
      const uint32_t block = (uint32_t)(std::min(cap / 64, kCounterBlocks) * 64);
      float* P = reinterpret_cast<float*>(split);
      uint32_t* counters = reinterpret_cast<uint32_t*>(reinterpret_cast<char*>(split) +
                                                       kMatvecPartialBytes);
      for (uint32_t r0 = 0; r0 < row_count; r0 += block) {
        const uint32_t rc = row_count - r0 < block ? row_count - r0 : block;
        const auto kern = wide ? &matvec_mfma_slice_kernel<4> : &matvec_mfma_slice_kernel<2>;
        const uint32_t rpx = ((rc + 63) / 64 + 7) / 8;  // row blocks per XCD
        hipLaunchKernelGGL(kern, dim3(8 * rpx * slices), dim3(64 * kMfmaWaves), 0, s, m->w,
                           m->scales, xb, x_stride, P, counters, yb + r0, y_stride, m->k,
                           m->k / m->g, gshift, row_start + r0, rc, bc,
                           nd_xcd_local() ? 1u : 0u);
        hipError_t e = hipGetLastError();
        if (e != hipSuccess) return e;
      }
    }
    return hipSuccess;
  }
  uint32_t b0 = 0;
  while (b0 < batch) {
    const VecPlan p = plan_vector(m, batch - b0, row_count);
    MatvecFn f = p.racc == 8 ? pick_b<8>(p.bc, p.spt) : p.racc == 4 ? pick_b<4>(p.bc, p.spt)
               : p.racc == 2 ? pick_b<2>(p.bc, p.spt) : pick_b<1>(p.bc, p.spt);
    hipLaunchKernelGGL(f, dim3(p.blocks), dim3(kThreads), 0, s, m->w, m->scales,
                       x + (size_t)b0 * x_stride, y + (size_t)b0 * y_stride, m->k, m->k / m->g,
                       m->g / 16, row_start, row_count, p.tpr_log2, x_stride, y_stride);
    hipError_t e = hipGetLastError();
    if (e != hipSuccess) return e;
    b0 += p.bc;
  }
  return hipSuccess;
}

hipError_t nd_launch_matvec_stamped(const nd_mat* m, const float* x, uint32_t row_start,
                                    uint32_t row_count, float* y, uint64_t* stamps,
                                    uint32_t capacity, uint32_t* workgroups, hipStream_t s) {
  const VecPlan p = plan_vector(m, 1, row_count);
  *workgroups = p.blocks;
  if (p.blocks > capacity) return hipErrorInvalidValue;
  decltype(&matvec_i8_stamped_kernel<1, 1, 1>) f;
  const uint32_t key = p.racc * 4 + p.spt;
  switch (key) {
    case 8 * 4 + 2: f = &matvec_i8_stamped_kernel<1, 2, 8>; break;
    case 4 * 4 + 2: f = &matvec_i8_stamped_kernel<1, 2, 4>; break;
    case 2 * 4 + 2: f = &matvec_i8_stamped_kernel<1, 2, 2>; break;
    case 1 * 4 + 2: f = &matvec_i8_stamped_kernel<1, 2, 1>; break;
    case 8 * 4 + 1: f = &matvec_i8_stamped_kernel<1, 1, 8>; break;
    case 4 * 4 + 1: f = &matvec_i8_stamped_kernel<1, 1, 4>; break;
    case 2 * 4 + 1: f = &matvec_i8_stamped_kernel<1, 1, 2>; break;
    default: f = &matvec_i8_stamped_kernel<1, 1, 1>; break;
  }
  hipLaunchKernelGGL(f, dim3(p.blocks), dim3(kThreads), 0, s, m->w, m->scales, x, y, m->k,
                     m->k / m->g, m->g / 16, row_start, row_count, p.tpr_log2, m->k, row_count,
                     stamps);
  return hipGetLastError();
}

hipError_t nd_launch_stream_read(const void* src, uint64_t bytes, uint32_t blocks, uint32_t* out,
                                 hipStream_t s) {
  hipLaunchKernelGGL(stream_read_kernel, dim3(blocks), dim3(kThreads), 0, s,
                     reinterpret_cast<const u32x4*>(src), bytes / 16, out);
  return hipGetLastError();
}

hipError_t nd_launch_row(const nd_mat* m, uint32_t row, float* out, hipStream_t s) {
  const uint32_t threads = 256;
  hipLaunchKernelGGL(row_kernel, dim3((m->k + threads - 1) / threads), dim3(threads), 0, s, m->w,
                     m->scales, m->k, m->k / m->g, m->g, row, out);
  return hipGetLastError();
}
