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

// Full-vocabulary max and sum of exp(logit - max), float64 accumulation.
__device__ void log_normalizer(const float* __restrict__ logits, uint32_t vocab, float* redf,
                               double* redd, float* out_max, double* out_sum) {
  float mx = -INFINITY;
  for (uint32_t i = threadIdx.x; i < vocab; i += blockDim.x) mx = js_maxf(mx, logits[i]);
  mx = block_max_js(mx, redf);
  double sum = 0.0;
  const double md = (double)mx;
  for (uint32_t i = threadIdx.x; i < vocab; i += blockDim.x) sum += exp((double)logits[i] - md);
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
  for (uint32_t i = threadIdx.x; i < n; i += blockDim.x) {
    const uint32_t id = allowed ? allowed[i] : i;
    if (id >= vocab) {
      bad = 1;
      continue;
    }
    const float v = logits[id];
    if (v != v) continue;  // a NaN never beats anything
    Best c{v, i};
    if (better(c, b)) b = c;
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

}  // namespace

hipError_t nd_launch_select_list(const float* logits, uint32_t vocab, const uint32_t* allowed,
                                 uint32_t count, uint32_t* id, double* logprob, hipStream_t s) {
  hipLaunchKernelGGL(select_list_kernel, dim3(1), dim3(kSelectThreads), 0, s, logits, vocab,
                     allowed, count, id, logprob);
  return hipGetLastError();
}

hipError_t nd_launch_select_mask(const float* logits, uint32_t batch, uint32_t vocab,
                                 const uint32_t* mask, uint32_t* ids, double* logprobs,
                                 hipStream_t s) {
  if (batch == 0) return hipSuccess;
  hipLaunchKernelGGL(select_mask_kernel, dim3(batch), dim3(kSelectThreads), 0, s, logits, vocab,
                     mask, ids, logprobs);
  return hipGetLastError();
}
