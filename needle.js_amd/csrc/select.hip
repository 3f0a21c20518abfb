// Constrained-decoding token selection: masked argmax + full-vocabulary
// log-softmax, one workgroup per row of logits.
//
// Semantics (selectToken, model/runtime.ts:880-899; argmax and logSoftmaxAt,
// model/math.ts:140-160): the winner is the first candidate, in candidate
// order, holding the largest value under strict '>' -- so ties keep the
// earliest candidate, a NaN never replaces a finite best, and a NaN first
// candidate is never replaced.  The parallel reduction carries (value,
// order) pairs and keeps the smaller order on equal values, which is the
// same choice.  The log-probability uses max and sum(exp) over all logits in
// float64; any NaN logit makes the maximum (and the result) NaN, as
// Math.max does.
#include "nd_internal.hpp"

namespace {

constexpr int kSelectThreads = 1024;
constexpr uint32_t kNone = 0xFFFFFFFFu;

struct Best {
  float v;
  uint32_t order;  // position in candidate order; kNone = no candidate
};

// True if candidate a should win over b.
__device__ __forceinline__ bool better(const Best& a, const Best& b) {
  if (a.order == kNone) return false;
  if (b.order == kNone) return true;
  if (a.v > b.v) return true;
  if (a.v == b.v) return a.order < b.order;
  if (b.v != b.v) return a.v == a.v;  // NaN best only survives as first candidate (handled by caller)
  return false;
}

__device__ __forceinline__ float js_maxf(float a, float b) {
  if (a != a || b != b) return __builtin_nanf("");
  return a > b ? a : b;
}

// Block reductions: 16 waves -> LDS -> wave 0.
__device__ float block_max_js(float v, float* red) {
  for (int o = 32; o >= 1; o >>= 1) v = js_maxf(v, __shfl_xor(v, o, 64));
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  float r = lane < (int)(blockDim.x >> 6) ? red[lane] : -INFINITY;
  for (int o = 32; o >= 1; o >>= 1) r = js_maxf(r, __shfl_xor(r, o, 64));
  __syncthreads();
  return r;
}

__device__ double block_sum_d(double v, double* red) {
  for (int o = 32; o >= 1; o >>= 1) v += __shfl_xor(v, o, 64);
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) red[w] = v;
  __syncthreads();
  double r = lane < (int)(blockDim.x >> 6) ? red[lane] : 0.0;
  for (int o = 32; o >= 1; o >>= 1) r += __shfl_xor(r, o, 64);
  __syncthreads();
  return r;
}

__device__ Best block_best(Best b, float* redv, uint32_t* redo) {
  for (int o = 32; o >= 1; o >>= 1) {
    Best other{__shfl_xor(b.v, o, 64), (uint32_t)__shfl_xor((int)b.order, o, 64)};
    if (better(other, b)) b = other;
  }
  const int w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  if (lane == 0) {
    redv[w] = b.v;
    redo[w] = b.order;
  }
  __syncthreads();
  Best r{-INFINITY, kNone};
  if (lane < (int)(blockDim.x >> 6)) r = Best{redv[lane], redo[lane]};
  for (int o = 32; o >= 1; o >>= 1) {
    Best other{__shfl_xor(r.v, o, 64), (uint32_t)__shfl_xor((int)r.order, o, 64)};
    if (better(other, r)) r = other;
  }
  __syncthreads();
  return r;
}

// One term e^x, x = logit - max <= 0, of the float64 log-softmax sum: the
// float64 exp while x >= -20, the fast f32 exp below.  The leading term is 1,
// so the terms below e^-20 = 2.1e-9 together hold at most vocab * 2.1e-9 of
// the sum.  __expf is v_exp_f32 of x log2(e) rounded to f32: the rounding
// moves the exponent by at most |x| 1.44 2^-24 (9e-6 at x = -104, where the
// f32 result reaches 0), i.e. a relative error below 1e-5 with the
// instruction's own ulp, and flushed subnormals lose terms below 1.2e-38.
// Together that moves the sum by at most vocab * 2.1e-9 * 1e-5 -- 6.9e-10 at
// a 32768 vocabulary -- and the log-probability by less than 7e-10.  The float64 exp runs only
// while some lane of the wave holds such a term, so a row whose logits
// spread over tens of units (most of the vocabulary below max - 20) costs
// the f32 exp per term.
__device__ __forceinline__ double exp_term(float v, double md) {
  const double x = (double)v - md;
  double e = (double)__expf((float)x);
  if (__any(x >= -20.0)) {
    if (x >= -20.0) e = exp(x);
  }
  return e;
}

// Full-vocabulary max and sum of exp(logit - max), float64 accumulation.
// The first kCache values of each thread (ids t + blockDim.x c) are loaded
// together and kept in registers for the sum; larger vocabularies stream
// the rest.  Each thread still adds its ids in increasing order.
constexpr int kCache = 8;
__device__ void log_normalizer(const float* __restrict__ logits, uint32_t vocab, float* redf,
                               double* redd, float* out_max, double* out_sum) {
  float v[kCache];
#pragma unroll
  for (int c = 0; c < kCache; ++c) {
    const uint32_t i = threadIdx.x + c * blockDim.x;
    v[c] = i < vocab ? logits[i] : -INFINITY;
  }
  float mx = -INFINITY;
#pragma unroll
  for (int c = 0; c < kCache; ++c) mx = js_maxf(mx, v[c]);
  for (uint32_t i = threadIdx.x + kCache * blockDim.x; i < vocab; i += blockDim.x)
    mx = js_maxf(mx, logits[i]);
  mx = block_max_js(mx, redf);
  double sum = 0.0;
  const double md = (double)mx;
#pragma unroll
  for (int c = 0; c < kCache; ++c) {
    const double e = exp_term(v[c], md);
    if (threadIdx.x + c * blockDim.x < vocab) sum += e;
  }
  for (uint32_t i = threadIdx.x + kCache * blockDim.x; i < vocab; i += blockDim.x)
    sum += exp_term(logits[i], md);
  sum = block_sum_d(sum, redd);
  *out_max = mx;
  *out_sum = sum;
}

// Candidate ids from an explicit list (list order) or all ids (allowed == nullptr).
__global__ __launch_bounds__(kSelectThreads) void select_list_kernel(
    const float* __restrict__ logits, uint32_t vocab, const uint32_t* __restrict__ allowed,
    uint32_t count, uint32_t* __restrict__ out_id, double* __restrict__ out_logprob) {
  __shared__ float redf[16];
  __shared__ double redd[16];
  __shared__ uint32_t redo[16];
  __shared__ int bad;
  if (threadIdx.x == 0) bad = 0;
  __syncthreads();
  const uint32_t n = allowed ? count : vocab;
  Best b{-INFINITY, kNone};
  // kCache candidates per thread per round: ids first, then their logits,
  // all loads of a round in flight together (the winner does not depend on
  // the order candidates are seen in: `better` is a total order).
  for (uint32_t base = 0; base < n; base += kCache * blockDim.x) {
    uint32_t ids[kCache];
#pragma unroll
    for (int c = 0; c < kCache; ++c) {
      const uint32_t i = base + threadIdx.x + c * blockDim.x;
      ids[c] = i < n ? (allowed ? allowed[i] : i) : kNone;
    }
    float vals[kCache];
#pragma unroll
    for (int c = 0; c < kCache; ++c) vals[c] = ids[c] < vocab ? logits[ids[c]] : 0.f;
#pragma unroll
    for (int c = 0; c < kCache; ++c) {
      const uint32_t i = base + threadIdx.x + c * blockDim.x;
      if (i >= n) continue;
      if (ids[c] >= vocab) {
        bad = 1;
        continue;
      }
      if (vals[c] != vals[c]) continue;  // a NaN never beats anything
      const Best cand{vals[c], i};
      if (better(cand, b)) b = cand;
    }
  }
  b = block_best(b, redf, redo);
  float mx;
  double sum;
  log_normalizer(logits, vocab, redf, redd, &mx, &sum);
  if (threadIdx.x == 0) {
    if (bad || n == 0) {
      *out_id = kNone;
      *out_logprob = __builtin_nan("");
      return;
    }
    const uint32_t first = allowed ? allowed[0] : 0;
    uint32_t id;
    if (logits[first] != logits[first] || b.order == kNone) id = first;
    else id = allowed ? allowed[b.order] : b.order;
    *out_id = id;
    *out_logprob = (double)logits[id] - (double)mx - log(sum);
  }
}

// Batched form: row r of logits with the ascending allowed set given by bitmask row r.
__global__ __launch_bounds__(kSelectThreads) void select_mask_kernel(
    const float* __restrict__ logits_all, uint32_t vocab, const uint32_t* __restrict__ mask_all,
    uint32_t* __restrict__ ids, double* __restrict__ logprobs) {
  __shared__ float redf[16];
  __shared__ double redd[16];
  __shared__ uint32_t redo[16];
  __shared__ uint32_t first_shared;
  const uint32_t r = blockIdx.x;
  const float* logits = logits_all + (size_t)r * vocab;
  const uint32_t words = (vocab + 31) / 32;
  const uint32_t* mask = mask_all ? mask_all + (size_t)r * words : nullptr;
  if (threadIdx.x == 0) first_shared = kNone;
  __syncthreads();
  Best b{-INFINITY, kNone};
  uint32_t first = kNone;
  for (uint32_t i = threadIdx.x; i < vocab; i += blockDim.x) {
    if (mask && !((mask[i >> 5] >> (i & 31)) & 1u)) continue;
    first = min(first, i);
    const float v = logits[i];
    if (v != v) continue;
    Best c{v, i};
    if (better(c, b)) b = c;
  }
  atomicMin(&first_shared, first);
  b = block_best(b, redf, redo);
  float mx;
  double sum;
  log_normalizer(logits, vocab, redf, redd, &mx, &sum);
  if (threadIdx.x == 0) {
    const uint32_t f = first_shared;
    if (f == kNone) {
      ids[r] = kNone;
      logprobs[r] = __builtin_nan("");
      return;
    }
    const uint32_t id = (logits[f] != logits[f] || b.order == kNone) ? f : b.order;
    ids[r] = id;
    logprobs[r] = (double)logits[id] - (double)mx - log(sum);
  }
}

// Register-resident form for vocab % 32 == 0 and vocab <= 32 * 1024: thread
// t holds ids [32 t, 32 t + 32) -- eight 16-byte loads and one mask word --
// so the row is read once, the masked argmax and the JavaScript max come out
// of one pass and one LDS round, and the float64 exp sum runs from registers.
// Same selection and log-probability as select_mask_kernel.
__global__ __launch_bounds__(kSelectThreads) void select_mask_reg_kernel(
    const float* __restrict__ logits_all, uint32_t vocab, const uint32_t* __restrict__ mask_all,
    uint32_t* __restrict__ ids, double* __restrict__ logprobs) {
  __shared__ float s_v[16], s_mx[16];
  __shared__ uint32_t s_o[16], s_first[16];
  __shared__ double s_sum[16];
  const uint32_t r = blockIdx.x, t = threadIdx.x, w = t >> 6, lane = t & 63;
  const float* logits = logits_all + (size_t)r * vocab;
  const uint32_t words = vocab / 32;
  const bool mine = t < words;
  const uint32_t tc = mine ? t : 0;
  const float4* src = reinterpret_cast<const float4*>(logits + (size_t)tc * 32);
  float v[32];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float4 f = src[q];
    v[4 * q] = f.x;
    v[4 * q + 1] = f.y;
    v[4 * q + 2] = f.z;
    v[4 * q + 3] = f.w;
  }
  const uint32_t m = !mine ? 0u : mask_all ? mask_all[(size_t)r * words + tc] : 0xFFFFFFFFu;
  Best b{-INFINITY, kNone};
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    mx = js_maxf(mx, v[j]);
    if (((m >> j) & 1u) && v[j] == v[j] && (b.order == kNone || v[j] > b.v))
      b = Best{v[j], t * 32 + j};
  }
  if (!mine) mx = -INFINITY;
  uint32_t first = m ? t * 32 + (uint32_t)__builtin_ctz(m) : kNone;
  for (int o = 32; o >= 1; o >>= 1) {
    Best other{__shfl_xor(b.v, o, 64), (uint32_t)__shfl_xor((int)b.order, o, 64)};
    if (better(other, b)) b = other;
    mx = js_maxf(mx, __shfl_xor(mx, o, 64));
    first = min(first, (uint32_t)__shfl_xor((int)first, o, 64));
  }
  if (lane == 0) {
    s_v[w] = b.v;
    s_o[w] = b.order;
    s_mx[w] = mx;
    s_first[w] = first;
  }
  __syncthreads();
  mx = s_mx[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) mx = js_maxf(mx, s_mx[i]);
  double sum = 0.0;
  {
    const double md = (double)mx;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const double e = exp_term(mine ? v[j] : -INFINITY, md);
      if (mine) sum += e;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane == 0) s_sum[w] = sum;
  __syncthreads();
  if (t != 0) return;
  Best best{s_v[0], s_o[0]};
  uint32_t f = s_first[0];
  double total = s_sum[0];
#pragma unroll
  for (int i = 1; i < 16; ++i) {
    const Best other{s_v[i], s_o[i]};
    if (better(other, best)) best = other;
    f = min(f, s_first[i]);
    total += s_sum[i];
  }
  if (f == kNone) {
    ids[r] = kNone;
    logprobs[r] = __builtin_nan("");
    return;
  }
  const uint32_t id = (logits[f] != logits[f] || best.order == kNone) ? f : best.order;
  ids[r] = id;
  logprobs[r] = (double)logits[id] - (double)mx - log(total);
}

// Split form of the register-resident kernel for batches that leave most of
// the chip idle at one workgroup per row: workgroup (sp, r) takes mask words
// [sp * wps, (sp + 1) * wps) of row r (thread t one word: 32 ids), reduces
// them to (best candidate, JavaScript max, first allowed id, float64 sum of
// e^(logit - local max)), publishes that record with agent-coherent stores
// and counts itself in; the last of the row's S workgroups merges the
// records: max over maxima, sum of sum_w * e^(max_w - max) in float64 (a
// part whose maximum is -inf holds only e^-inf = 0 terms), the best record
// by (value, lower id), the smallest first id.  Selection and
// log-probability as select_mask_reg_kernel; the float64 sum is the same
// terms regrouped.  With `adv`, each row's merge also feeds its id back as
// the row's next token, records id and log-probability in the step history,
// advances the row's position, and the last row to finish advances the step
// counter (what a separate advance pass would do).  Every call leaves the
// counters at zero.
constexpr uint32_t kSelSplitMax = 16;
struct SelRecord {
  float bv;
  uint32_t bo;
  float mx;
  uint32_t first;
  double sum;
  double pad;
};
static_assert(sizeof(SelRecord) == 32, "record layout");

__global__ __launch_bounds__(kSelectThreads) void select_mask_split_kernel(
    const float* __restrict__ logits_all, uint32_t vocab, const uint32_t* __restrict__ mask_all,
    uint32_t* __restrict__ ids, double* __restrict__ logprobs, uint32_t wps,
    SelRecord* __restrict__ records, uint32_t* __restrict__ counters, nd_select_advance adv) {
  __shared__ float s_v[16], s_mx[16];
  __shared__ uint32_t s_o[16], s_first[16], s_last;
  __shared__ double s_sum[16];
  const uint32_t sp = blockIdx.x, S = gridDim.x, r = blockIdx.y;
  const uint32_t t = threadIdx.x, w = t >> 6, lane = t & 63, nw = blockDim.x >> 6;
  const float* logits = logits_all + (size_t)r * vocab;
  const uint32_t words = vocab / 32;
  const uint32_t word = sp * wps + t;
  const bool mine = t < wps && word < words;
  const uint32_t wc = mine ? word : 0;
  const float4* src = reinterpret_cast<const float4*>(logits + (size_t)wc * 32);
  float v[32];
#pragma unroll
  for (int q = 0; q < 8; ++q) {
    const float4 f = src[q];
    v[4 * q] = f.x;
    v[4 * q + 1] = f.y;
    v[4 * q + 2] = f.z;
    v[4 * q + 3] = f.w;
  }
  const uint32_t m = !mine ? 0u : mask_all ? mask_all[(size_t)r * words + wc] : 0xFFFFFFFFu;
  Best b{-INFINITY, kNone};
  float mx = -INFINITY;
#pragma unroll
  for (int j = 0; j < 32; ++j) {
    mx = js_maxf(mx, v[j]);
    if (((m >> j) & 1u) && v[j] == v[j] && (b.order == kNone || v[j] > b.v))
      b = Best{v[j], wc * 32 + j};
  }
  if (!mine) mx = -INFINITY;
  uint32_t first = m ? wc * 32 + (uint32_t)__builtin_ctz(m) : kNone;
  for (int o = 32; o >= 1; o >>= 1) {
    Best other{__shfl_xor(b.v, o, 64), (uint32_t)__shfl_xor((int)b.order, o, 64)};
    if (better(other, b)) b = other;
    mx = js_maxf(mx, __shfl_xor(mx, o, 64));
    first = min(first, (uint32_t)__shfl_xor((int)first, o, 64));
  }
  if (lane == 0) {
    s_v[w] = b.v;
    s_o[w] = b.order;
    s_mx[w] = mx;
    s_first[w] = first;
  }
  __syncthreads();
  mx = s_mx[0];
  for (uint32_t i = 1; i < nw; ++i) mx = js_maxf(mx, s_mx[i]);
  double sum = 0.0;
  {
    const double md = (double)mx;
#pragma unroll
    for (int j = 0; j < 32; ++j) {
      const double e = exp_term(mine ? v[j] : -INFINITY, md);
      if (mine) sum += e;
    }
  }
  for (int o = 32; o >= 1; o >>= 1) sum += __shfl_xor(sum, o, 64);
  if (lane == 0) s_sum[w] = sum;
  __syncthreads();
  if (t == 0) {
    Best best{s_v[0], s_o[0]};
    uint32_t f = s_first[0];
    double total = s_sum[0];
    for (uint32_t i = 1; i < nw; ++i) {
      const Best other{s_v[i], s_o[i]};
      if (better(other, best)) best = other;
      f = min(f, s_first[i]);
      total += s_sum[i];
    }
    SelRecord* rec = records + (size_t)r * kSelSplitMax + sp;
    __hip_atomic_store(&rec->bv, best.v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rec->bo, best.order, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rec->mx, mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rec->first, f, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(&rec->sum, total, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __builtin_amdgcn_s_waitcnt(0);  // the record has completed
    const bool last =
        __hip_atomic_fetch_add(counters + r, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
        S - 1;
    if (last) __hip_atomic_store(counters + r, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    s_last = last;
  }
  __syncthreads();
  if (!s_last || w != 0) return;

  // Merge: lane j holds record j.
  const SelRecord* rec = records + (size_t)r * kSelSplitMax + (lane < S ? lane : 0);
  float bv = __hip_atomic_load(&rec->bv, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t bo = __hip_atomic_load(&rec->bo, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  float pm = __hip_atomic_load(&rec->mx, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  uint32_t pf = __hip_atomic_load(&rec->first, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  double ps = __hip_atomic_load(&rec->sum, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  if (lane >= S) {
    bv = -INFINITY;
    bo = kNone;
    pm = -INFINITY;
    pf = kNone;
    ps = 0.0;
  }
  Best best{bv, bo};
  float gm = pm;
  uint32_t f = pf;
  for (int o = 32; o >= 1; o >>= 1) {
    Best other{__shfl_xor(best.v, o, 64), (uint32_t)__shfl_xor((int)best.order, o, 64)};
    if (better(other, best)) best = other;
    gm = js_maxf(gm, __shfl_xor(gm, o, 64));
    f = min(f, (uint32_t)__shfl_xor((int)f, o, 64));
  }
  double term = (lane < S && pm != -INFINITY) ? ps * exp((double)pm - (double)gm) : 0.0;
  for (int o = 32; o >= 1; o >>= 1) term += __shfl_xor(term, o, 64);
  if (lane != 0) return;
  uint32_t id = kNone;
  double lp = __builtin_nan("");
  if (f != kNone) {
    id = (logits[f] != logits[f] || best.order == kNone) ? f : best.order;
    lp = (double)logits[id] - (double)gm - log(term);
  }
  ids[r] = id;
  logprobs[r] = lp;
  if (!adv.tokens) return;
  const uint32_t batch = gridDim.y;
  const uint32_t step = __hip_atomic_load(adv.step, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  adv.tokens[r] = id;
  adv.positions[r] += 1;
  if (step < adv.history_steps) {
    adv.history[(size_t)step * batch + r] = id;
    adv.lp_history[(size_t)step * batch + r] = lp;
  }
  __builtin_amdgcn_s_waitcnt(0);  // this row's read of the step counter has completed
  uint32_t* rows_done = counters + batch;
  if (__hip_atomic_fetch_add(rows_done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) ==
      batch - 1) {
    __hip_atomic_store(rows_done, 0u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
    __hip_atomic_store(adv.step, step + 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
  }
}

}  // namespace

hipError_t nd_launch_select_list(const float* logits, uint32_t vocab, const uint32_t* allowed,
                                 uint32_t count, uint32_t* id, double* logprob, hipStream_t s) {
  hipLaunchKernelGGL(select_list_kernel, dim3(1), dim3(kSelectThreads), 0, s, logits, vocab,
                     allowed, count, id, logprob);
  return hipGetLastError();
}

size_t nd_select_split_bytes(uint32_t batch) {
  return (size_t)batch * kSelSplitMax * sizeof(SelRecord) + ((size_t)batch + 1) * 4;
}

hipError_t nd_launch_select_mask(const float* logits, uint32_t batch, uint32_t vocab,
                                 const uint32_t* mask, uint32_t* ids, double* logprobs,
                                 hipStream_t s, void* split, const nd_select_advance* adv,
                                 bool* advanced) {
  if (advanced) *advanced = false;
  if (batch == 0) return hipSuccess;
  if (split && vocab % 32 == 0) {
    // Parts per row: enough workgroups for ~512 in all, at least 64 words
    // (one wave) per part and at most 1024 words (one workgroup).
    const uint32_t words = vocab / 32;
    uint32_t S = (512 + batch - 1) / batch;
    if (S > words / 64) S = words / 64;
    if (S > kSelSplitMax) S = kSelSplitMax;
    if (S < (words + kSelectThreads - 1) / kSelectThreads)
      S = (words + kSelectThreads - 1) / kSelectThreads;
    if (S >= 2 && S <= kSelSplitMax) {
      const uint32_t wps = (words + S - 1) / S;
      const uint32_t threads = (wps + 63) / 64 * 64;
      SelRecord* records = reinterpret_cast<SelRecord*>(split);
      uint32_t* counters = reinterpret_cast<uint32_t*>(records + (size_t)batch * kSelSplitMax);
      hipLaunchKernelGGL(select_mask_split_kernel, dim3(S, batch), dim3(threads), 0, s, logits,
                         vocab, mask, ids, logprobs, wps, records, counters,
                         adv ? *adv : nd_select_advance{});
      if (advanced) *advanced = adv != nullptr;
      return hipGetLastError();
    }
  }
  if (vocab % 32 == 0 && vocab <= 32u * kSelectThreads)
    hipLaunchKernelGGL(select_mask_reg_kernel, dim3(batch), dim3(kSelectThreads), 0, s, logits,
                       vocab, mask, ids, logprobs);
  else
    hipLaunchKernelGGL(select_mask_kernel, dim3(batch), dim3(kSelectThreads), 0, s, logits, vocab,
                       mask, ids, logprobs);
  return hipGetLastError();
}
