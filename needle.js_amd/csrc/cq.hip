// Cactus-Quant (CQ2 / CQ3 / CQ4 / ternary) matrices on gfx950: the shipped
// weight format of needle.js (model/cact.ts:61-75, 346-396), multiplied
// without expanding the weights (backends/cq.ts:107-231).
//
// Layout in HBM, as in the archive: packed codes [n][row_bytes] (row_bytes =
// kpad * pb / 8, pb = 2 for ternary records), then binary16 norms
// [n][kpad / g].  Here kpad is the stored width: the archive's (k rounded up
// to the group size g) rounded up to 32 codes, the added codes and their
// groups' norms zero, so every row is whole 32-code units.  The codebook of the matrix's
// width (4, 8 or 16 floats; ternary: 0, +c, 0, -c with c = 1.2240064 /
// sqrt(g)) travels as a kernel argument and is copied to LDS.
//
//  * cq_prepare_kernel: prepareCqActivation (cq.ts:30-46) -- per group the
//    fastWalshHadamard butterflies (cq.ts:8-27) in the reference's stage
//    order with an fp32 result per butterfly, then value * 1/sqrt(g) in
//    float64 with an fp32 store: bit-identical to the reference's Float32Array.
//  * cq_matvec_kernel: thread (sub, u) owns 32-weight unit u of rows row0 +
//    p * rpp + sub; its 32 prepared inputs stay in registers, each row
//    contributes one 8 / 12 / 16-byte load and the unit's binary16 norms;
//    codes index the LDS codebook; fp32 dots per group times the group norm,
//    reduced over the row's threads through LDS and a DPP butterfly.
//  * cq_row_kernel: dequantizeCqRow (cq.ts:243-295): f32(codebook * norm),
//    the same butterflies, f32(value * 1/sqrt(g)); bit-identical.
#include <cmath>

#include "nd_internal.hpp"
#include "nd_wave.hpp"

namespace {

constexpr int kCqThreads = 256;
constexpr uint32_t kTernaryBits = 5;
constexpr double kTernaryCentroid = 1.2240064;  // backends/cq.ts:6

// binary16 bit pattern -> float (float16ToNumber, fp16.ts:5-32; exact).
__device__ __forceinline__ float half_bits_to_float(uint32_t h) {
  return (float)__builtin_bit_cast(_Float16, (uint16_t)h);
}

// Per-group FWHT of v[0, len) in LDS (len = kpad, groups of g): stride 1, 2,
// 4, ... with one butterfly per (pair) and a barrier per stage; each result
// is one fp32 add or subtract, as the reference's Float32Array stores.
__device__ void fwht_groups(float* v, uint32_t len, uint32_t g) {
  for (uint32_t stride = 1; stride < g; stride <<= 1) {
    for (uint32_t i = threadIdx.x; i < len / 2; i += blockDim.x) {
      // Pair i: block of 2*stride, position inside the block's left half.
      const uint32_t block = i / stride, inner = i % stride;
      const uint32_t left = block * 2 * stride + inner, right = left + stride;
      const float a = v[left], b = v[right];
      v[left] = a + b;
      v[right] = a - b;
    }
    __syncthreads();
  }
}

// out[b][0, kpad) = prepareCqActivation(x[b][0, k)) for one batch row per
// workgroup.
__global__ __launch_bounds__(kCqThreads) void cq_prepare_kernel(const float* __restrict__ x,
                                                                uint32_t x_stride, uint32_t k,
                                                                uint32_t kpad, uint32_t g,
                                                                double inverse_root,
                                                                float* __restrict__ out) {
  __shared__ float v[8192];
  const float* xb = x + (size_t)blockIdx.x * x_stride;
  float* ob = out + (size_t)blockIdx.x * kpad;
  for (uint32_t i = threadIdx.x; i < kpad; i += blockDim.x) v[i] = i < k ? xb[i] : 0.f;
  __syncthreads();
  fwht_groups(v, kpad, g);
  for (uint32_t i = threadIdx.x; i < kpad; i += blockDim.x)
    ob[i] = (float)((double)v[i] * inverse_root);
}

// dequantizeCqRow for one row.
struct Codebook {
  float v[16];
};

__device__ __forceinline__ uint32_t code_at(const uint8_t* row, uint32_t c, uint32_t bits) {
  if (bits == 2 || bits == kTernaryBits) return (row[c >> 2] >> ((c & 3) * 2)) & 3u;
  if (bits == 4) return (row[c >> 1] >> ((c & 1) * 4)) & 15u;
  const uint32_t bit = c * 3, at = bit >> 3, shift = bit & 7;
  const uint32_t word = (uint32_t)row[at] | (shift > 5 ? (uint32_t)row[at + 1] << 8 : 0u);
  return (word >> shift) & 7u;
}

__global__ __launch_bounds__(kCqThreads) void cq_row_kernel(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ norms, Codebook cb,
    uint32_t k, uint32_t kpad, uint32_t g, uint32_t bits, uint32_t row_bytes, uint32_t row,
    double inverse_root, float* __restrict__ out) {
  __shared__ float v[8192];
  const uint8_t* prow = packed + (size_t)row * row_bytes;
  const uint32_t groups = kpad / g;
  for (uint32_t c = threadIdx.x; c < kpad; c += blockDim.x) {
    const float norm = half_bits_to_float(norms[(size_t)row * groups + c / g]);
    const uint32_t code = code_at(prow, c, bits);
    // Ternary: crumb 3 -> -c, 1 -> +c, 0 and 2 -> 0 (the record's index
    // mapping into Float32Array([-c, 0, c]), cq.ts:259-273); cb holds them
    // by crumb.
    v[c] = cb.v[code] * norm;
  }
  __syncthreads();
  fwht_groups(v, kpad, g);
  for (uint32_t c = threadIdx.x; c < k; c += blockDim.x)
    out[c] = (float)((double)v[c] * inverse_root);
}

// cb.v[i] for i < N by a select tree over the bits of i (constant indices
// only).
template <int N>
__device__ __forceinline__ float pick_code(const Codebook& cb, uint32_t i) {
  float v[N];
#pragma unroll
  for (int j = 0; j < N; ++j) v[j] = cb.v[j];
#pragma unroll
  for (int half = N / 2, bit = 0; half >= 1; half /= 2, ++bit) {
#pragma unroll
    for (int j = 0; j < half; ++j) v[j] = (i >> bit) & 1u ? v[2 * j + 1] : v[2 * j];
  }
  return v[0];
}

// Rotated inputs of unit u (32 consecutive columns) in registers: the
// butterflies of fastWalshHadamard with strides 1 .. GS / 2 inside the unit
// (GS = min(g, 32)), then strides 32, 64, ... as exchanges with the lanes
// holding the group's other units (lane strides 1 .. lanes_per_group / 2).
// Each result is one fp32 add or subtract of the same two operands as the
// reference's; the 1/sqrt(g) factor is left to the caller.
template <int M>
__device__ __forceinline__ void cross_lane_stage(float (&v)[32]) {
  const bool right = (__lane_id() & M) != 0;
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const float other = nd::lane_xor<M>(v[i]);
    v[i] = right ? other - v[i] : v[i] + other;
  }
}

template <int GS>
__device__ __forceinline__ void rotate_unit(float (&v)[32], uint32_t lanes_per_group) {
#pragma unroll
  for (int st = 1; st < GS; st <<= 1) {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      if ((i & st) == 0) {
        const float a = v[i], b = v[i + st];
        v[i] = a + b;
        v[i + st] = a - b;
      }
    }
  }
  if (lanes_per_group > 1) cross_lane_stage<1>(v);
  if (lanes_per_group > 2) cross_lane_stage<2>(v);
  if (lanes_per_group > 4) cross_lane_stage<4>(v);
  if (lanes_per_group > 8) cross_lane_stage<8>(v);
  if (lanes_per_group > 16) cross_lane_stage<16>(v);
  if (lanes_per_group > 32) cross_lane_stage<32>(v);
}

// y[b][r] for rows [row_start, row_start + row_count), batch row b =
// blockIdx.y.  Thread (sub, u) owns 32-code unit u of rows row0 + i * rpp +
// sub (i < RACC).  UB = bytes of a unit (8: 2-bit and ternary, 12: 3-bit,
// 16: 4-bit); NG = groups in a unit (1 when g >= 32, else 32 / g).
// ROTATE: x is the raw input [k] and each thread rotates its unit in
// registers (g <= 2048: a group's units sit in one wave); otherwise x holds
// rotated rows [kpad] from cq_prepare_kernel.  VEC: x rows are 16-byte
// aligned with k % 4 == 0 (float4 loads), else scalar loads.  Both load
// unconditionally from clamped addresses and zero what lies past the row.  The weight codes and norms
// are issued first among the HBM loads after x, so the rotation overlaps
// their latency; codes index an LDS copy of the codebook; fp32 dots per
// group times the group norm; row sums through LDS and a DPP butterfly,
// times out_scale (1/sqrt(g) for ROTATE, else 1).
// Codes per table lookup for UB-byte units: entries of kE floats indexed by
// kE packed codes.
constexpr int lookup_codes(int ub) { return ub == 8 ? 4 : 2; }

template <int UB, int NG, int RACC, bool ROTATE, bool VEC>
__global__ __launch_bounds__(kCqThreads) void cq_matvec_kernel(
    const uint8_t* __restrict__ packed, const uint16_t* __restrict__ norms, Codebook cb,
    const float* __restrict__ x, uint32_t x_stride, float* __restrict__ y, uint32_t y_stride,
    uint32_t k, uint32_t kpad, uint32_t g_log2, uint32_t row_bytes, uint32_t row_start,
    uint32_t row_count, uint32_t tpr_log2, uint32_t lanes_per_group, float out_scale) {
  constexpr int kGs = 32 / NG;  // weights per group inside a unit
  // Lookup table in LDS: entry i holds the codebook values of the kE codes
  // packed in index i (kE * bits index bits), one read per kE weights.
  constexpr int kPB = UB / 4;                  // bits per code
  constexpr int kE = lookup_codes(UB);         // codes per lookup
  constexpr int kLB = kPB * kE;                // bits per lookup index
  constexpr int kEntries = 1 << kLB;
  constexpr int kLookups = 32 / kE;            // per unit
  __shared__ __align__(16) float tab[kEntries * kE];
  __shared__ float red[RACC * kCqThreads];
  const uint32_t t = threadIdx.x;
  const uint32_t tpr = 1u << tpr_log2, rpp = kCqThreads >> tpr_log2;
  const uint32_t sub = t >> tpr_log2, u = t & (tpr - 1);
  const uint32_t units = kpad / 32, groups = kpad >> g_log2;
  const bool active = u < units;
  const uint32_t uc = active ? u : 0;
  const uint32_t row0 = blockIdx.x * rpp * RACC;
  const float* xb = x + (size_t)blockIdx.y * x_stride;

  // x first (L2-resident, needed first), then the weights; nothing reads
  // x until the weight loads are issued, so the wait for x leaves them in
  // flight.
  float xv[32];
  const uint32_t c0 = u * 32, lim = ROTATE ? k : kpad;
  if constexpr (VEC) {
#pragma unroll
    for (int q = 0; q < 8; ++q) {
      const uint32_t c = c0 + 4 * q;
      const float4 f = *reinterpret_cast<const float4*>(xb + (c < lim ? c : lim - 4));
      xv[4 * q] = f.x;
      xv[4 * q + 1] = f.y;
      xv[4 * q + 2] = f.z;
      xv[4 * q + 3] = f.w;
    }
  } else {
#pragma unroll
    for (int i = 0; i < 32; ++i) {
      const uint32_t c = c0 + i;
      xv[i] = xb[c < lim ? c : lim - 1];
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  uint32_t raw[RACC][UB / 4];
  uint32_t nb[RACC][(NG + 1) / 2];
#pragma unroll
  for (int r = 0; r < RACC; ++r) {
    const uint32_t row = row0 + r * rpp + sub;
    const uint32_t rr = row_start + (row < row_count ? row : 0);
    const uint32_t* src = reinterpret_cast<const uint32_t*>(packed + (size_t)rr * row_bytes +
                                                            (size_t)uc * UB);
#pragma unroll
    for (int w = 0; w < UB / 4; ++w) raw[r][w] = src[w];
    const uint16_t* nrow = norms + (size_t)rr * groups;
    if constexpr (NG == 1) {
      nb[r][0] = nrow[(uc * 32) >> g_log2];
    } else if constexpr (NG == 2) {
      nb[r][0] = *reinterpret_cast<const uint32_t*>(nrow + uc * 2);
    } else {
      const uint2 v = *reinterpret_cast<const uint2*>(nrow + uc * 4);
      nb[r][0] = v.x;
      nb[r][1] = v.y;
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  // The table, while the loads are in flight.  The codebook is read at
  // constant indices (scalar loads of the kernel arguments) and each entry
  // picked with a select tree: no per-lane loads from the argument segment.
  if (t < (uint32_t)kEntries) {
#pragma unroll
    for (int e = 0; e < kE; ++e)
      tab[t * kE + e] = pick_code<(1 << kPB)>(cb, (t >> (e * kPB)) & ((1u << kPB) - 1));
  }
  // Columns past the row (clamped loads above) read as zero.
#pragma unroll
  for (int i = 0; i < 32; ++i) {
    const uint32_t c = VEC ? c0 + (i & ~3) : c0 + i;
    xv[i] = c < lim ? xv[i] : 0.f;
  }
  if constexpr (ROTATE) rotate_unit<kGs>(xv, lanes_per_group);
  __syncthreads();  // tab

  // Codebook values of row r's 32 codes: kLookups table reads (bits
  // kLB * i .. of the unit's 32 * kPB-bit stream).  Row r + 1's reads are
  // issued before row r's products, so LDS latency overlaps the FMAs.
  auto lookup_row = [&](int r, float (&tv)[32]) {
#pragma unroll
    for (int i = 0; i < kLookups; ++i) {
      const int bit = kLB * i, w = bit >> 5, sh = bit & 31;
      const uint32_t b = sh + kLB <= 32
                             ? (raw[r][w] >> sh) & (kEntries - 1u)
                             : ((raw[r][w] >> sh) | (raw[r][w + 1] << (32 - sh))) & (kEntries - 1u);
      const char* at = reinterpret_cast<const char*>(tab) + b * (kE * 4);
      if constexpr (kE == 4) {
        const float4 f = *reinterpret_cast<const float4*>(at);
        tv[4 * i] = f.x;
        tv[4 * i + 1] = f.y;
        tv[4 * i + 2] = f.z;
        tv[4 * i + 3] = f.w;
      } else if constexpr (kE == 2) {
        const float2 f = *reinterpret_cast<const float2*>(at);
        tv[2 * i] = f.x;
        tv[2 * i + 1] = f.y;
      } else {
        tv[i] = *reinterpret_cast<const float*>(at);
      }
    }
  };
  float acc[RACC];
  float tv[2][32];
  lookup_row(0, tv[0]);
#pragma unroll
  for (int r = 0; r < RACC; ++r) {
    if (r + 1 < RACC) lookup_row(r + 1, tv[(r + 1) & 1]);
    __builtin_amdgcn_sched_barrier(0);
    const float(&v)[32] = tv[r & 1];
    float total = 0.f;
#pragma unroll
    for (int s = 0; s < NG; ++s) {
      float d[kE];
#pragma unroll
      for (int e = 0; e < kE; ++e) d[e] = 0.f;
#pragma unroll
      for (int jj = 0; jj < kGs; ++jj) {
        const int j = s * kGs + jj;
        d[jj % kE] = fmaf(v[j], xv[j], d[jj % kE]);
      }
      float dot = d[0];
      if constexpr (kE >= 2) dot += d[1];
      if constexpr (kE == 4) dot += d[2] + d[3];
      const uint32_t h = NG == 1 ? nb[r][0] : (nb[r][s >> 1] >> (16 * (s & 1))) & 0xFFFFu;
      total = fmaf(half_bits_to_float(h), dot, total);
    }
    acc[r] = active ? total : 0.f;
  }

  // Row sums over the row's tpr threads: red is [RACC][256]; T = 256 /
  // (rpp * RACC) threads per output each add tpr / T = RACC columns, then a
  // T-lane butterfly.
#pragma unroll
  for (int r = 0; r < RACC; ++r) red[r * kCqThreads + t] = acc[r];
  __syncthreads();
  const uint32_t outputs = rpp * RACC;
  const uint32_t T = kCqThreads / outputs;
  const uint32_t o = t / T, part = t % T;
  const uint32_t osub = o / RACC, orr = o % RACC;
  const float* col = red + orr * kCqThreads + osub * tpr;
  float sum = 0.f;
#pragma unroll
  for (int i = 0; i < RACC; ++i) sum += col[part + T * i];
  if (T > 32) sum = nd::sum_xor<32>(sum);
  if (T > 16) sum = nd::sum_xor<16>(sum);
  if (T > 8) sum += nd::lane_xor<8>(sum);
  if (T > 4) sum += nd::lane_xor<4>(sum);
  if (T > 2) sum += nd::lane_xor<2>(sum);
  if (T > 1) sum += nd::lane_xor<1>(sum);
  if (part == 0) {
    const uint32_t row = row0 + orr * rpp + osub;
    if (row < row_count) y[(size_t)blockIdx.y * y_stride + row] = sum * out_scale;
  }
}

Codebook codebook_of(const nd_mat* m) {
  Codebook c{};
  for (int i = 0; i < 16; ++i) c.v[i] = m->cb[i];
  return c;
}

using CqFn = void (*)(const uint8_t*, const uint16_t*, Codebook, const float*, uint32_t, float*,
                      uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t, uint32_t,
                      uint32_t, uint32_t, float);

constexpr int kRacc = 8;  // rows per thread: rpp * 8 <= 256 outputs per workgroup
constexpr uint32_t kMaxRotateGroup = 2048;  // 64 lanes of 32 codes

template <int UB, int RACC, bool ROTATE, bool VEC>
CqFn pick_ng(uint32_t g) {
  return g >= 32   ? &cq_matvec_kernel<UB, 1, RACC, ROTATE, VEC>
         : g == 16 ? &cq_matvec_kernel<UB, 2, RACC, ROTATE, VEC>
                   : &cq_matvec_kernel<UB, 4, RACC, ROTATE, VEC>;
}

template <int RACC, bool ROTATE, bool VEC>
CqFn pick_w(const nd_mat* m) {
  return m->bits == 4   ? pick_ng<16, RACC, ROTATE, VEC>(m->g)
         : m->bits == 3 ? pick_ng<12, RACC, ROTATE, VEC>(m->g)
                        : pick_ng<8, RACC, ROTATE, VEC>(m->g);
}

// kRacc rows per thread, or one when kRacc would give the launch fewer than
// 256 workgroups (small matrices: more workgroups, each on fewer rows) and a
// row has at most 64 units.
template <bool ROTATE, bool VEC>
CqFn pick(const nd_mat* m, uint32_t racc) {
  return racc == 1 ? pick_w<1, ROTATE, VEC>(m) : pick_w<kRacc, ROTATE, VEC>(m);
}

}  // namespace

// Geometry checks happened at upload (bits, g a power of two >= 8 with g
// dividing kpad, kpad <= 8192, kpad % 32 == 0).  Rotated inputs are kpad
// wide; columns from k on are zero before the rotation.
hipError_t nd_launch_cq_prepare(const nd_mat* m, const float* x, uint32_t batch, uint32_t x_stride,
                                float* prepared, hipStream_t s) {
  if (batch == 0) return hipSuccess;
  hipLaunchKernelGGL(cq_prepare_kernel, dim3(batch), dim3(kCqThreads), 0, s, x, x_stride, m->k,
                     m->kpad, m->g, 1.0 / std::sqrt((double)m->g), prepared);
  return hipGetLastError();
}

// y[b][r - row_start] for b < batch from x [batch][x_stride].  Groups of
// up to 2048 are rotated inside the matvec (one launch); wider groups are
// rotated by cq_prepare_kernel into `prepared` (kCqPreparedRows rows of
// kCqMaxKpad floats), kCqPreparedRows batch rows at a time.
hipError_t nd_launch_cq_matvec(const nd_mat* m, const float* x, uint32_t batch, uint32_t x_stride,
                               float* prepared, uint32_t row_start, uint32_t row_count, float* y,
                               uint32_t y_stride, hipStream_t s) {
  if (row_count == 0 || batch == 0) return hipSuccess;
  const uint32_t units = m->kpad / 32;
  uint32_t tpr_log2 = 3;  // at least 8 threads per row: rpp * kRacc <= 256 outputs
  while ((1u << tpr_log2) < units) ++tpr_log2;
  const uint32_t rpp = kCqThreads >> tpr_log2;
  // One row per thread keeps a row's threads in one wave (the row sum's
  // butterfly spans T = tpr lanes): rows of at most 64 units.
  const uint32_t racc =
      tpr_log2 <= 6 && (uint64_t)((row_count + rpp * kRacc - 1) / (rpp * kRacc)) * batch < 256
          ? 1u
          : kRacc;
  const uint32_t blocks = (row_count + rpp * racc - 1) / (rpp * racc);
  uint32_t g_log2 = 0;
  while ((1u << g_log2) < m->g) ++g_log2;
  const uint32_t lanes_per_group = m->g > 32 ? m->g / 32 : 1;
  if (m->g <= kMaxRotateGroup) {
    const bool vec = (m->k & 3) == 0 && (x_stride & 3) == 0 &&
                     (reinterpret_cast<uintptr_t>(x) & 15) == 0;
    const CqFn f = vec ? pick<true, true>(m, racc) : pick<true, false>(m, racc);
    hipLaunchKernelGGL(f, dim3(blocks, batch), dim3(kCqThreads), 0, s, m->packed,
                       m->norms, codebook_of(m), x, x_stride, y, y_stride, m->k, m->kpad, g_log2,
                       m->row_bytes, row_start, row_count, tpr_log2, lanes_per_group,
                       (float)(1.0 / std::sqrt((double)m->g)));
    return hipGetLastError();
  }
  for (uint32_t b0 = 0; b0 < batch; b0 += kCqPreparedRows) {
    const uint32_t nb = batch - b0 < kCqPreparedRows ? batch - b0 : kCqPreparedRows;
    hipError_t e = nd_launch_cq_prepare(m, x + (size_t)b0 * x_stride, nb, x_stride, prepared, s);
    if (e != hipSuccess) return e;
    const CqFn f = pick<false, true>(m, racc);
    hipLaunchKernelGGL(f, dim3(blocks, nb), dim3(kCqThreads), 0, s, m->packed,
                       m->norms, codebook_of(m), prepared, m->kpad, y + (size_t)b0 * y_stride,
                       y_stride, m->k, m->kpad, g_log2, m->row_bytes, row_start, row_count,
                       tpr_log2, 1u, 1.0f);
    e = hipGetLastError();
    if (e != hipSuccess) return e;
  }
  return hipSuccess;
}

hipError_t nd_launch_cq_row(const nd_mat* m, uint32_t row, float* out, hipStream_t s) {
  const double inverse_root = 1.0 / std::sqrt((double)m->g);
  Codebook cb = codebook_of(m);
  if (m->bits == kTernaryBits) {  // Float32Array([-c, 0, c]) with c = 1.2240064 * 1/sqrt(g)
    const float c = (float)(kTernaryCentroid * inverse_root);
    cb.v[0] = 0.f;
    cb.v[1] = c;
    cb.v[2] = 0.f;
    cb.v[3] = -c;
  }
  hipLaunchKernelGGL(cq_row_kernel, dim3(1), dim3(kCqThreads), 0, s, m->packed, m->norms, cb,
                     m->k, m->kpad, m->g, m->bits, m->row_bytes, row, inverse_root, out);
  return hipGetLastError();
}
