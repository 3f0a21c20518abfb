/*
 * needle_oracle.c -- CPU restatement of the needle.js decode hot path.
 *
 * TEST INFRASTRUCTURE ONLY.  This library is the checker: only tests/,
 * __graft_entry__.smoke() and bench.py's cpu_baseline leg may load it.  The
 * product path (needle.js_amd/) never links, loads or calls it.
 *
 * Every function restates the arithmetic of the reference TypeScript CPU
 * path with JavaScript number semantics: all scalar arithmetic is IEEE
 * binary64 evaluated left to right with no fused multiply-add (build with
 * -ffp-contract=off), and every store into a Float32Array is a
 * round-to-nearest-even conversion to binary32 (a C (float) cast).
 * Reference paths are relative to packages/needle.js/src/ of needle.js.
 *
 * Parity pins (what checks each function beyond re-reading this file):
 *   or_round_ties_even  Python round() on random and tie values; tests/.
 *   or_kv_quantize      invariants |code|<=127, code(absmax)=+-127,
 *                       |x-code*s|<=s/2 in exact rationals, tie cases,
 *                       zero vector; golden vectors in tests/golden/.
 *   or_matvec_i8        closed forms (W==c, x==e_k), dense float64 matmul
 *                       (numpy) on random inputs, batch==single with row
 *                       ranges (mirrors tests/cq.test.ts:74-99).
 *   or_row_i8           elementwise product in numpy (exact).
 *   or_attention        textbook softmax attention in float64 numpy,
 *                       identical keys -> mean of values, L=1 -> V0.
 *   or_select           brute force over allowed ids (Python), NaN and tie
 *                       special cases, scipy logsumexp for log-probability.
 *   or_fwht             Sylvester Hadamard matrix (scipy.linalg.hadamard)
 *                       and self-inverse (tests/cq.test.ts:64-72).
 *   or_f16_to_f32       the binary16 patterns of tests/fp16.test.ts:4-20 and
 *                       numpy's float16 decoding of all 65536 patterns.
 *   or_cq_prepare       explicit Sylvester-matrix products per group.
 *   or_cq_matvec        the fixtures of tests/cq.test.ts:20-61 (direct ==
 *                       dequantized row dot, batch == single with a range),
 *                       codes unpacked independently (numpy bit operations)
 *                       times explicit Hadamard products, closed form for a
 *                       constant code (sqrt(g) * x_0 per group).
 *   or_cq_row           dequantized rows against explicit H (codebook .*
 *                       norm) / sqrt(g); matvec == row . x (the reference
 *                       test's identity).
 *   or_rms_norm, or_rope, or_sigmoid, or_softmax, or_sinkhorn,
 *   or_hadamard_mlp     closed forms in numpy float64 (unit RMS, rotation
 *                       preserves norms and matches complex multiply,
 *                       Sinkhorn output doubly stochastic, H-MLP equals
 *                       explicit matrix products).
 *   decoder steps       composition of the pinned primitives; checked for
 *                       prefill == repeated step and batch == single.
 *   or_synth_prefill    bit-identical to repeated or_synth_step (codes,
 *                       scales, captured vectors, logits) at several thread
 *                       counts and start positions; tests/.
 *   or_kv_capture,      storage only: the captured vectors equal the stored
 *   or_kv_export_raw    inputs and re-quantize to the cache's codes; tests/.
 *   decode checkpoints  equal to or_synth_step logits of the same steps.
 */
#include <math.h>
#include <pthread.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_OK 0
#define OR_INVALID 1
#define OR_OVERFLOW 3

/* JavaScript Math.max of two numbers: NaN if either is NaN, +0 beats -0. */
static double js_max(double a, double b) {
  if (isnan(a) || isnan(b)) return NAN;
  if (a == 0.0 && b == 0.0) return (signbit(a) && signbit(b)) ? -0.0 : 0.0;
  return a > b ? a : b;
}

/* ToInt8 of an integral double (Int8Array store): NaN/inf -> 0, wrap mod 256. */
static int8_t js_to_int8(double v) {
  if (!isfinite(v)) return 0;
  double t = trunc(v);
  double m = fmod(t, 256.0);
  if (m < 0) m += 256.0;
  int iv = (int)m;
  return (int8_t)(iv >= 128 ? iv - 256 : iv);
}

/* runtime.ts:901-907 roundTiesToEven (Math.floor based). */
double or_round_ties_even(double value) {
  double lower = floor(value);
  double fraction = value - lower;
  if (fraction < 0.5) return lower;
  if (fraction > 0.5) return lower + 1;
  /* (lower & 1) uses ToInt32 of lower; NaN & 1 == 0 keeps lower. */
  if (isnan(lower)) return lower;
  int64_t li = (int64_t)fmod(lower, 4294967296.0);
  return ((li & 1) == 0) ? lower : lower + 1;
}

/* ---------------------------------------------------------------- math.ts */

/* math.ts:3-10 */
double or_sigmoid(double value) {
  if (value >= 0) {
    double e = exp(-value);
    return 1 / (1 + e);
  }
  double e = exp(value);
  return e / (1 + e);
}

/* math.ts:12-14 */
double or_silu(double value) { return value * or_sigmoid(value); }

/* math.ts:16-32 rmsNorm (zero-centred: scale stores the offset from 1). */
void or_rms_norm(const float* input, const float* scale, uint32_t n, float* output) {
  double sum_squares = 0;
  for (uint32_t i = 0; i < n; i++) {
    double v = input[i];
    sum_squares += v * v;
  }
  double inverse = 1 / sqrt(sum_squares / n + 1e-6);
  for (uint32_t i = 0; i < n; i++)
    output[i] = (float)((1 + (double)scale[i]) * (double)input[i] * inverse);
}

/* math.ts:34-44 rmsUnit */
void or_rms_unit(const float* input, uint32_t n, float* output) {
  double sum_squares = 0;
  for (uint32_t i = 0; i < n; i++) {
    double v = input[i];
    sum_squares += v * v;
  }
  double inverse = 1 / sqrt(sum_squares / n + 1e-6);
  for (uint32_t i = 0; i < n; i++) output[i] = (float)((double)input[i] * inverse);
}

/* runtime.ts:647-657 #rmsNormSlice (in place, offset slice). */
void or_rms_norm_slice(float* values, uint32_t offset, uint32_t length, const float* scale) {
  double sum_squares = 0;
  for (uint32_t i = 0; i < length; i++) {
    double v = values[offset + i];
    sum_squares += v * v;
  }
  double inverse = 1 / sqrt(sum_squares / length + 1e-6);
  for (uint32_t i = 0; i < length; i++)
    values[offset + i] = (float)((1 + (double)scale[i]) * (double)values[offset + i] * inverse);
}

/* math.ts:46-60 softmaxInPlace */
void or_softmax(float* values, uint32_t length) {
  if (length == 0) return;
  double maximum = values[0];
  for (uint32_t i = 1; i < length; i++) maximum = js_max(maximum, values[i]);
  double total = 0;
  for (uint32_t i = 0; i < length; i++) {
    double v = exp((double)values[i] - maximum);
    values[i] = (float)v;
    total += v;
  }
  double inverse = total > 0 ? 1 / total : 0;
  for (uint32_t i = 0; i < length; i++) values[i] = (float)((double)values[i] * inverse);
}

/* cq.ts:8-27 fastWalshHadamard on values[offset, offset+length). */
int or_fwht(float* values, uint32_t offset, uint32_t length) {
  if (length == 0 || (length & (length - 1)) != 0) return OR_INVALID;
  for (uint32_t stride = 1; stride < length; stride <<= 1) {
    uint32_t block = stride << 1;
    for (uint32_t base = 0; base < length; base += block) {
      for (uint32_t inner = 0; inner < stride; inner++) {
        uint32_t li = offset + base + inner, ri = li + stride;
        double left = values[li], right = values[ri];
        values[li] = (float)(left + right);
        values[ri] = (float)(left - right);
      }
    }
  }
  return OR_OK;
}

/* math.ts:62-92 sinkhorn (log-space, float64 working copy). */
void or_sinkhorn(float* logits, uint32_t size, uint32_t iterations) {
  uint32_t n = size * size;
  double* v = (double*)malloc(sizeof(double) * n);
  for (uint32_t i = 0; i < n; i++) v[i] = logits[i];
  for (uint32_t it = 0; it < iterations; it++) {
    for (uint32_t row = 0; row < size; row++) {
      uint32_t off = row * size;
      double maximum = v[off];
      for (uint32_t c = 1; c < size; c++) maximum = js_max(maximum, v[off + c]);
      double sum = 0;
      for (uint32_t c = 0; c < size; c++) sum += exp(v[off + c] - maximum);
      double log_sum = log(sum) + maximum;
      for (uint32_t c = 0; c < size; c++) v[off + c] = v[off + c] - log_sum;
    }
    for (uint32_t c = 0; c < size; c++) {
      double maximum = v[c];
      for (uint32_t r = 1; r < size; r++) maximum = js_max(maximum, v[r * size + c]);
      double sum = 0;
      for (uint32_t r = 0; r < size; r++) sum += exp(v[r * size + c] - maximum);
      double log_sum = log(sum) + maximum;
      for (uint32_t r = 0; r < size; r++) v[r * size + c] = v[r * size + c] - log_sum;
    }
  }
  for (uint32_t i = 0; i < n; i++) logits[i] = (float)exp(v[i]);
  free(v);
}

/* math.ts:94-115 applyRope: half-split rotation, theta^(-2j/d). */
void or_rope(float* vec, uint32_t heads, uint32_t head_dim, uint32_t position, double theta) {
  uint32_t half = head_dim >> 1;
  for (uint32_t h = 0; h < heads; h++) {
    uint32_t off = h * head_dim;
    for (uint32_t d = 0; d < half; d++) {
      double frequency = pow(theta, -(2.0 * d) / head_dim);
      double angle = position * frequency;
      double c = cos(angle), s = sin(angle);
      double first = vec[off + d], second = vec[off + d + half];
      vec[off + d] = (float)(first * c - second * s);
      vec[off + d + half] = (float)(second * c + first * s);
    }
  }
}

/* math.ts:117-138 hadamardMlp; output has `n` entries, hdim >= n. */
int or_hadamard_mlp(const float* input, uint32_t n, const float* d1, const float* d2,
                    const float* d3, uint32_t hdim, float* output) {
  if (hdim < n) return OR_INVALID;
  float* values = (float*)calloc(hdim, sizeof(float));
  for (uint32_t i = 0; i < n; i++) values[i] = (float)((double)input[i] * (double)d1[i]);
  double inverse_root = 1 / sqrt((double)hdim);
  if (or_fwht(values, 0, hdim) != OR_OK) { free(values); return OR_INVALID; }
  for (uint32_t i = 0; i < hdim; i++)
    values[i] = (float)or_silu((double)values[i] * inverse_root * (double)d2[i]);
  or_fwht(values, 0, hdim);
  for (uint32_t i = 0; i < n; i++)
    output[i] = (float)((double)values[i] * inverse_root * (double)d3[i]);
  free(values);
  return OR_OK;
}

/* math.ts:140-151 argmax: first maximum under strict '>'. */
uint32_t or_argmax(const float* values, uint32_t n) {
  uint32_t best = 0;
  double best_value = n ? (double)values[0] : -INFINITY;
  for (uint32_t i = 1; i < n; i++) {
    double v = values[i];
    if (v > best_value) { best_value = v; best = i; }
  }
  return best;
}

/* math.ts:153-160 logSoftmaxAt over the full vocabulary. */
double or_log_softmax_at(const float* logits, uint32_t n, uint32_t token) {
  double maximum = n ? (double)logits[0] : -INFINITY;
  for (uint32_t i = 1; i < n; i++) maximum = js_max(maximum, logits[i]);
  double sum = 0;
  for (uint32_t i = 0; i < n; i++) sum += exp((double)logits[i] - maximum);
  double at = token < n ? (double)logits[token] : -INFINITY;
  return at - maximum - log(sum);
}

/* runtime.ts:880-899 selectToken.  allowed==NULL -> unconstrained argmax.
 * Returns OR_INVALID for an empty list or an id outside the logits. */
int or_select(const float* logits, uint32_t vocab, const uint32_t* allowed, uint32_t count,
              uint32_t* out_id, double* out_logprob) {
  uint32_t id;
  if (!allowed) {
    id = or_argmax(logits, vocab);
  } else {
    if (count == 0) return OR_INVALID;
    id = allowed[0];
    if (id >= vocab) return OR_INVALID;
    double best = logits[id];
    for (uint32_t i = 1; i < count; i++) {
      uint32_t c = allowed[i];
      if (c >= vocab) return OR_INVALID;
      double v = logits[c];
      if (v > best) { best = v; id = c; }
    }
  }
  *out_id = id;
  *out_logprob = or_log_softmax_at(logits, vocab, id);
  return OR_OK;
}

/* Bitmask form of selectToken used by batched constrained decode: the allowed
 * list is the ascending set of ids whose bit (mask[id>>5] >> (id&31)) & 1 is
 * set, which is how agent.ts:164-183 builds it (ascending token order). */
int or_select_mask(const float* logits, uint32_t vocab, const uint32_t* mask, uint32_t* out_id,
                   double* out_logprob) {
  int found = 0;
  uint32_t id = 0;
  double best = 0;
  for (uint32_t c = 0; c < vocab; c++) {
    if (!((mask[c >> 5] >> (c & 31)) & 1u)) continue;
    double v = logits[c];
    if (!found) { id = c; best = v; found = 1; }
    else if (v > best) { best = v; id = c; }
  }
  if (!found) return OR_INVALID;
  *out_id = id;
  *out_logprob = or_log_softmax_at(logits, vocab, id);
  return OR_OK;
}

/* ------------------------------------------------------- a1: int8 matvec */

/* Int8 variant of CqMatrix: W int8 [N][K] row-major, scales f32 [N][K/G].
 * Restates cqMatvecPrepared's loop shape (cq.ts:106-156): for each row a
 * float64 `dot` per group, `total += norm * dot`, f32 store; the codebook
 * lookup becomes the int8 value and the fp16 group norm the fp32 scale.
 * x and y are [B][K] and [B][row_count]. */
int or_matvec_i8(const int8_t* w, const float* scales, uint32_t n, uint32_t k, uint32_t g,
                 const float* x, uint32_t batch, uint32_t row_start, uint32_t row_count,
                 float* y) {
  if (g == 0 || k % g != 0) return OR_INVALID;
  if ((uint64_t)row_start + row_count > n) return OR_INVALID;
  uint32_t groups = k / g;
  for (uint32_t b = 0; b < batch; b++) {
    const float* xb = x + (size_t)b * k;
    for (uint32_t lr = 0; lr < row_count; lr++) {
      uint32_t r = row_start + lr;
      const int8_t* wr = w + (size_t)r * k;
      double total = 0;
      for (uint32_t grp = 0; grp < groups; grp++) {
        double dot = 0;
        for (uint32_t c = 0; c < g; c++) {
          uint32_t col = grp * g + c;
          dot += (double)wr[col] * (double)xb[col];
        }
        total += (double)scales[(size_t)r * groups + grp] * dot;
      }
      y[(size_t)b * row_count + lr] = (float)total;
    }
  }
  return OR_OK;
}

/* dequantizeCqRow analogue (cq.ts:243-295): out[c] = f32(W[r][c] * s[r][c/G]). */
int or_row_i8(const int8_t* w, const float* scales, uint32_t n, uint32_t k, uint32_t g,
              uint32_t row, float* out) {
  if (g == 0 || k % g != 0 || row >= n) return OR_INVALID;
  uint32_t groups = k / g;
  for (uint32_t c = 0; c < k; c++)
    out[c] = (float)((double)w[(size_t)row * k + c] * (double)scales[(size_t)row * groups + c / g]);
  return OR_OK;
}

/* ------------------------------------- a1 (CQ): Cactus-Quant matrices */

/* fp16.ts:5-32 float16ToNumber: binary16 bit pattern -> binary32 (exact). */
float or_f16_to_f32(uint16_t h) {
  uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
  int32_t exponent = (h >> 10) & 0x1f;
  uint32_t mantissa = h & 0x3ffu, bits;
  if (exponent == 0) {
    if (mantissa == 0) {
      bits = sign;
    } else {
      exponent = 127 - 15 + 1;
      while ((mantissa & 0x400u) == 0) {
        mantissa <<= 1;
        exponent--;
      }
      mantissa &= 0x3ffu;
      bits = sign | ((uint32_t)exponent << 23) | (mantissa << 13);
    }
  } else if (exponent == 0x1f) {
    bits = sign | 0x7f800000u | (mantissa << 13);
  } else {
    bits = sign | ((uint32_t)(exponent - 15 + 127) << 23) | (mantissa << 13);
  }
  float f;
  memcpy(&f, &bits, 4);
  return f;
}

#define OR_TERNARY_BITS 5
static const double kTernaryCentroid = 1.2240064; /* cq.ts:6 */

/* cact.ts:362-378: inputs padded to whole groups; ternary records pack 2-bit
 * crumbs; row byte length = padded inputs * packed bits / 8. */
static int cq_geometry(uint32_t k, uint32_t g, uint32_t bits, uint32_t* kpad, uint32_t* row_bytes) {
  if (g == 0 || (g & (g - 1)) != 0) return OR_INVALID;
  if (bits != 2 && bits != 3 && bits != 4 && bits != OR_TERNARY_BITS) return OR_INVALID;
  uint32_t pb = bits == OR_TERNARY_BITS ? 2 : bits;
  *kpad = (k + g - 1) / g * g;
  if (((uint64_t)*kpad * pb) % 8 != 0) return OR_INVALID;
  *row_bytes = (uint32_t)((uint64_t)*kpad * pb / 8);
  return OR_OK;
}

/* Code (crumb, nibble or 3-bit field) of column c of a packed row: crumbs and
 * nibbles low bits first (cq.ts:143, 169, 194), 3-bit rows one little-endian
 * bitstream read through a 16-bit window (cq.ts:219-224). */
static uint32_t cq_code(const uint8_t* row, uint32_t c, uint32_t bits) {
  if (bits == 2 || bits == OR_TERNARY_BITS) return (row[c >> 2] >> ((c & 3) * 2)) & 3u;
  if (bits == 4) return (row[c >> 1] >> ((c & 1) * 4)) & 15u;
  uint32_t bit = c * 3, at = bit >> 3, shift = bit & 7;
  uint32_t word = (uint32_t)row[at] | ((shift + 3 > 8) ? ((uint32_t)row[at + 1] << 8) : 0u);
  return (word >> shift) & 7u;
}

/* cq.ts:30-46 prepareCqActivation: x zero-padded to kpad, fastWalshHadamard
 * on each group (f32 store after every butterfly), then each value times
 * 1/sqrt(g) in float64 with an f32 store.  out holds kpad values. */
int or_cq_prepare(const float* x, uint32_t k, uint32_t g, float* out) {
  if (g == 0 || (g & (g - 1)) != 0) return OR_INVALID;
  uint32_t kpad = (k + g - 1) / g * g;
  for (uint32_t i = 0; i < kpad; i++) out[i] = i < k ? x[i] : 0.0f;
  const double inverse_root = 1.0 / sqrt((double)g);
  for (uint32_t off = 0; off < kpad; off += g) {
    or_fwht(out, off, g);
    for (uint32_t i = 0; i < g; i++) out[off + i] = (float)((double)out[off + i] * inverse_root);
  }
  return OR_OK;
}

/* cq.ts:107-231 cqMatvecPrepared on or_cq_prepare(x), batch rows of x [B][k]
 * into y [B][row_count].  codebook is the archive's 28 floats: CQ2 [0, 4),
 * CQ3 [4, 12), CQ4 [12, 28) (cact.ts:272-276); norms are binary16 bit
 * patterns [n][kpad / g].  Per row: float64 `dot` per group in the
 * reference's summation order, `total += norm * dot`, f32 store. */
int or_cq_matvec(const uint8_t* packed, const uint16_t* norms, const float* codebook, uint32_t n,
                 uint32_t k, uint32_t g, uint32_t bits, const float* x, uint32_t batch,
                 uint32_t row_start, uint32_t row_count, float* y) {
  uint32_t kpad, row_bytes;
  if (cq_geometry(k, g, bits, &kpad, &row_bytes) != OR_OK) return OR_INVALID;
  if ((uint64_t)row_start + row_count > n) return OR_INVALID;
  const uint32_t groups = kpad / g;
  const double coefficient = kTernaryCentroid / sqrt((double)g);
  const double crumbs[4] = {0.0, coefficient, 0.0, -coefficient};
  const float* cb = bits == 2 ? codebook : bits == 3 ? codebook + 4 : codebook + 12;
  float* prepared = (float*)malloc(sizeof(float) * kpad);
  if (!prepared) return OR_INVALID;
  for (uint32_t b = 0; b < batch; b++) {
    or_cq_prepare(x + (size_t)b * k, k, g, prepared);
    for (uint32_t lr = 0; lr < row_count; lr++) {
      const uint32_t r = row_start + lr;
      const uint8_t* row = packed + (size_t)r * row_bytes;
      double total = 0;
      for (uint32_t grp = 0; grp < groups; grp++) {
        const float* p = prepared + (size_t)grp * g;
        const uint32_t c0 = grp * g;
        double dot = 0;
        if (bits == 2 || bits == OR_TERNARY_BITS) {
          for (uint32_t c = 0; c < g; c += 4) {
            double v[4];
            for (int j = 0; j < 4; j++) {
              uint32_t code = cq_code(row, c0 + c + j, bits);
              v[j] = bits == 2 ? (double)cb[code] : crumbs[code];
            }
            dot += ((v[0] * (double)p[c] + v[1] * (double)p[c + 1]) + v[2] * (double)p[c + 2]) +
                   v[3] * (double)p[c + 3];
          }
        } else if (bits == 4) {
          for (uint32_t c = 0; c < g; c += 2)
            dot += (double)cb[cq_code(row, c0 + c, 4)] * (double)p[c] +
                   (double)cb[cq_code(row, c0 + c + 1, 4)] * (double)p[c + 1];
        } else {
          for (uint32_t c = 0; c < g; c++) dot += (double)cb[cq_code(row, c0 + c, 3)] * (double)p[c];
        }
        total += (double)or_f16_to_f32(norms[(size_t)r * groups + grp]) * dot;
      }
      y[(size_t)b * row_count + lr] = (float)total;
    }
  }
  free(prepared);
  return OR_OK;
}

/* cq.ts:243-295 dequantizeCqRow: per group, f32(codebook[index] * norm) (the
 * ternary codebook is Float32Array([-c, 0, c]) with c = 1.2240064/sqrt(g),
 * crumb 3 -> index 0, crumb i -> i + 1, index 3 reads as 0), the FWHT, then
 * f32(value * 1/sqrt(g)); the first k columns are written. */
int or_cq_row(const uint8_t* packed, const uint16_t* norms, const float* codebook, uint32_t n,
              uint32_t k, uint32_t g, uint32_t bits, uint32_t row, float* out) {
  uint32_t kpad, row_bytes;
  if (cq_geometry(k, g, bits, &kpad, &row_bytes) != OR_OK || row >= n) return OR_INVALID;
  const uint32_t groups = kpad / g;
  const double inverse_root = 1.0 / sqrt((double)g);
  const float ternary[3] = {(float)(-kTernaryCentroid * inverse_root), 0.0f,
                            (float)(kTernaryCentroid * inverse_root)};
  const float* cb = bits == 2 ? codebook : bits == 3 ? codebook + 4 : codebook + 12;
  const uint8_t* prow = packed + (size_t)row * row_bytes;
  float* temporary = (float*)malloc(sizeof(float) * g);
  if (!temporary) return OR_INVALID;
  for (uint32_t grp = 0; grp < groups; grp++) {
    const double norm = (double)or_f16_to_f32(norms[(size_t)row * groups + grp]);
    for (uint32_t c = 0; c < g; c++) {
      const uint32_t code = cq_code(prow, grp * g + c, bits);
      double value;
      if (bits == OR_TERNARY_BITS) {
        const uint32_t index = code == 3 ? 0 : code + 1;
        value = index < 3 ? (double)ternary[index] : 0.0;
      } else {
        value = (double)cb[code];
      }
      temporary[c] = (float)(value * norm);
    }
    or_fwht(temporary, 0, g);
    const uint32_t count = g < k - grp * g ? g : k - grp * g;
    for (uint32_t c = 0; c < count; c++)
      out[grp * g + c] = (float)((double)temporary[c] * inverse_root);
  }
  free(temporary);
  return OR_OK;
}

/* ------------------------------------------------- a2: int8 KV quantizer */

/* One vector of runtime.ts:697-714: m = max(1e-12, max|x|) in float64,
 * s = m/127, stored scale f32(s), code = roundTiesToEven(x/s) as Int8. */
void or_kv_quantize(const float* x, uint32_t n, int8_t* codes, float* scale_out) {
  double maximum = 1e-12;
  for (uint32_t i = 0; i < n; i++) maximum = js_max(maximum, fabs((double)x[i]));
  double scale = maximum / 127;
  *scale_out = (float)scale;
  for (uint32_t i = 0; i < n; i++) codes[i] = js_to_int8(or_round_ties_even((double)x[i] / scale));
}

/* KV cache geometry and slot map, runtime.ts:150-205 and 659-677. */
typedef struct {
  uint32_t layers, kv_heads, head_dim, max_length, sink, window, alloc;
  int float_mode; /* kvCache: "float32" stores raw values, scale 1 */
  int8_t *k8, *v8;
  float *kf, *vf, *ks, *vs;
  /* Test capture: the f32 vectors handed to #storeKV for positions
   * [raw_from, raw_from + raw_count), by position: [layers][kv_heads]
   * [raw_count][head_dim]. */
  float *kraw, *vraw;
  uint32_t raw_from, raw_count;
} or_kv;

or_kv* or_kv_create(uint32_t layers, uint32_t kv_heads, uint32_t head_dim, uint32_t max_length,
                    uint32_t sink, uint32_t window, int float_mode) {
  or_kv* kv = (or_kv*)calloc(1, sizeof(or_kv));
  kv->layers = layers; kv->kv_heads = kv_heads; kv->head_dim = head_dim;
  kv->max_length = max_length;
  kv->sink = sink > max_length ? max_length : sink;
  kv->window = window;
  kv->alloc = window > 0 ? (max_length < kv->sink + window ? max_length : kv->sink + window)
                         : max_length;
  kv->float_mode = float_mode;
  size_t elems = (size_t)layers * kv_heads * kv->alloc * head_dim;
  size_t scales = (size_t)layers * kv_heads * kv->alloc;
  if (float_mode) {
    kv->kf = (float*)calloc(elems, sizeof(float));
    kv->vf = (float*)calloc(elems, sizeof(float));
  } else {
    kv->k8 = (int8_t*)calloc(elems, 1);
    kv->v8 = (int8_t*)calloc(elems, 1);
  }
  kv->ks = (float*)calloc(scales, sizeof(float));
  kv->vs = (float*)calloc(scales, sizeof(float));
  return kv;
}

void or_kv_destroy(or_kv* kv) {
  if (!kv) return;
  free(kv->k8); free(kv->v8); free(kv->kf); free(kv->vf); free(kv->ks); free(kv->vs);
  free(kv->kraw); free(kv->vraw);
  free(kv);
}

/* Keeps, from now on, a copy of every K/V vector stored at a position in
 * [from, from + count) (the values before quantization), for tests that check
 * codes against the exact quotient x / s.  Not part of the reference;
 * storage only. */
int or_kv_capture(or_kv* kv, uint32_t from, uint32_t count) {
  if (count == 0 || (uint64_t)from + count > kv->max_length) return OR_INVALID;
  free(kv->kraw); free(kv->vraw);
  size_t elems = (size_t)kv->layers * kv->kv_heads * count * kv->head_dim;
  kv->kraw = (float*)calloc(elems, sizeof(float));
  kv->vraw = (float*)calloc(elems, sizeof(float));
  kv->raw_from = from;
  kv->raw_count = count;
  return (kv->kraw && kv->vraw) ? OR_OK : OR_INVALID;
}

static size_t kv_raw_base(const or_kv* kv, uint32_t layer, uint32_t head, uint32_t position) {
  return (((size_t)layer * kv->kv_heads + head) * kv->raw_count + (position - kv->raw_from)) *
         kv->head_dim;
}

/* Copies the captured vectors of positions [from, from + count) of one
 * (layer, head): k, v are [count][head_dim]. */
int or_kv_export_raw(const or_kv* kv, uint32_t layer, uint32_t head, uint32_t from, uint32_t count,
                     float* k, float* v) {
  if (!kv->kraw || from < kv->raw_from ||
      (uint64_t)from + count > (uint64_t)kv->raw_from + kv->raw_count ||
      layer >= kv->layers || head >= kv->kv_heads)
    return OR_INVALID;
  size_t base = kv_raw_base(kv, layer, head, from);
  memcpy(k, kv->kraw + base, sizeof(float) * (size_t)count * kv->head_dim);
  memcpy(v, kv->vraw + base, sizeof(float) * (size_t)count * kv->head_dim);
  return OR_OK;
}

uint32_t or_kv_alloc(const or_kv* kv) { return kv->alloc; }

/* runtime.ts:659-664 #kvSlot */
uint32_t or_kv_slot(const or_kv* kv, uint32_t position) {
  if (kv->window == 0) return position;
  if (position < kv->sink) return position;
  return kv->sink + (position - kv->sink) % kv->window;
}

static size_t kv_base(const or_kv* kv, uint32_t layer, uint32_t head, uint32_t slot) {
  return (((size_t)layer * kv->kv_heads + head) * kv->alloc + slot) * kv->head_dim;
}
static size_t kv_scale_index(const or_kv* kv, uint32_t layer, uint32_t head, uint32_t slot) {
  return ((size_t)layer * kv->kv_heads + head) * kv->alloc + slot;
}

/* runtime.ts:679-717 #storeKV: k, v are [kv_heads][head_dim]. */
int or_kv_store(or_kv* kv, uint32_t layer, uint32_t position, const float* k, const float* v) {
  if (layer >= kv->layers || position >= kv->max_length) return OR_INVALID;
  uint32_t slot = or_kv_slot(kv, position);
  for (uint32_t h = 0; h < kv->kv_heads; h++) {
    const float* kh = k + (size_t)h * kv->head_dim;
    const float* vh = v + (size_t)h * kv->head_dim;
    size_t base = kv_base(kv, layer, h, slot), si = kv_scale_index(kv, layer, h, slot);
    if (kv->float_mode) {
      memcpy(kv->kf + base, kh, sizeof(float) * kv->head_dim);
      memcpy(kv->vf + base, vh, sizeof(float) * kv->head_dim);
      kv->ks[si] = 1; kv->vs[si] = 1;
    } else {
      or_kv_quantize(kh, kv->head_dim, kv->k8 + base, kv->ks + si);
      or_kv_quantize(vh, kv->head_dim, kv->v8 + base, kv->vs + si);
    }
    if (kv->kraw && position >= kv->raw_from && position - kv->raw_from < kv->raw_count) {
      size_t rb = kv_raw_base(kv, layer, h, position);
      memcpy(kv->kraw + rb, kh, sizeof(float) * kv->head_dim);
      memcpy(kv->vraw + rb, vh, sizeof(float) * kv->head_dim);
    }
  }
  return OR_OK;
}

/* Copies out the codes (int8, or the float32 rows in float mode) and scales
 * of one (layer, head) for tests. */
void or_kv_export(const or_kv* kv, uint32_t layer, uint32_t head, void* kcodes, void* vcodes,
                  float* kscales, float* vscales) {
  size_t base = kv_base(kv, layer, head, 0), si = kv_scale_index(kv, layer, head, 0);
  if (!kv->float_mode) {
    memcpy(kcodes, kv->k8 + base, (size_t)kv->alloc * kv->head_dim);
    memcpy(vcodes, kv->v8 + base, (size_t)kv->alloc * kv->head_dim);
  } else {
    memcpy(kcodes, kv->kf + base, sizeof(float) * (size_t)kv->alloc * kv->head_dim);
    memcpy(vcodes, kv->vf + base, sizeof(float) * (size_t)kv->alloc * kv->head_dim);
  }
  memcpy(kscales, kv->ks + si, sizeof(float) * kv->alloc);
  memcpy(vscales, kv->vs + si, sizeof(float) * kv->alloc);
}

/* ------------------------------------------- a3: single-query attention */

/* runtime.ts:719-786 #attention with softmaxInPlace (math.ts:46-60).
 * q is [q_heads][head_dim]; out is [q_heads][head_dim]. */
int or_attention(const or_kv* kv, uint32_t layer, uint32_t position, const float* q,
                 uint32_t q_heads, float* out) {
  uint32_t hd = kv->head_dim;
  if (q_heads % kv->kv_heads != 0 || layer >= kv->layers || position >= kv->max_length)
    return OR_INVALID;
  uint32_t reps = q_heads / kv->kv_heads;
  uint32_t prefix = kv->sink < position + 1 ? kv->sink : position + 1;
  uint32_t recent_low = prefix;
  if (kv->window > 0 && position + 1 > kv->window && position + 1 - kv->window > prefix)
    recent_low = position + 1 - kv->window;
  uint32_t count = prefix + (position - recent_low + 1);
  uint32_t* logical = (uint32_t*)malloc(sizeof(uint32_t) * count);
  float* scores = (float*)malloc(sizeof(float) * count);
  uint32_t t = 0;
  for (uint32_t i = 0; i < prefix; i++) logical[t++] = i;
  for (uint32_t i = recent_low; i <= position; i++) logical[t++] = i;
  double inverse_root = 1 / sqrt((double)hd);
  memset(out, 0, sizeof(float) * (size_t)q_heads * hd);
  for (uint32_t kvh = 0; kvh < kv->kv_heads; kvh++) {
    for (uint32_t rep = 0; rep < reps; rep++) {
      uint32_t qh = kvh * reps + rep;
      const float* qv = q + (size_t)qh * hd;
      for (uint32_t ti = 0; ti < count; ti++) {
        uint32_t slot = or_kv_slot(kv, logical[ti]);
        size_t base = kv_base(kv, layer, kvh, slot), si = kv_scale_index(kv, layer, kvh, slot);
        double ks = kv->ks[si];
        double dot = 0;
        if (kv->float_mode) {
          for (uint32_t i = 0; i < hd; i++) dot += (double)qv[i] * (double)kv->kf[base + i];
        } else {
          for (uint32_t i = 0; i < hd; i++) dot += (double)qv[i] * (double)kv->k8[base + i] * ks;
        }
        scores[ti] = (float)(dot * inverse_root);
      }
      or_softmax(scores, count);
      float* o = out + (size_t)qh * hd;
      for (uint32_t ti = 0; ti < count; ti++) {
        uint32_t slot = or_kv_slot(kv, logical[ti]);
        size_t base = kv_base(kv, layer, kvh, slot), si = kv_scale_index(kv, layer, kvh, slot);
        double w = scores[ti];
        if (kv->float_mode) {
          for (uint32_t i = 0; i < hd; i++)
            o[i] = (float)((double)o[i] + w * (double)kv->vf[base + i]);
        } else {
          double vs = kv->vs[si];
          for (uint32_t i = 0; i < hd; i++)
            o[i] = (float)((double)o[i] + w * (double)kv->v8[base + i] * vs);
        }
      }
    }
  }
  free(logical);
  free(scores);
  return OR_OK;
}

/* ------------------------------------------ seeded generators (integers) */

/* splitmix64 output i (0-based) of the stream with 64-bit seed `seed`:
 * mix(seed + (i + 1) * golden).  Shared spec with the synthetic-data module
 * and the GPU generators; pure integer arithmetic, so bit-exact everywhere. */
static uint64_t sm64_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ull;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBull;
  return z ^ (z >> 31);
}
uint64_t or_splitmix64_at(uint64_t seed, uint64_t i) {
  return sm64_mix(seed + (i + 1) * 0x9E3779B97F4A7C15ull);
}

/* Allowed-token bitmask row: id v allowed iff (z_v >> 40) < threshold24,
 * plus the forced id (z_vocab >> 32) * vocab >> 32. */
void or_gen_mask(uint64_t seed, uint32_t vocab, uint32_t threshold24, uint32_t* mask) {
  uint32_t words = (vocab + 31) / 32;
  memset(mask, 0, sizeof(uint32_t) * words);
  for (uint32_t v = 0; v < vocab; v++)
    if ((uint32_t)(or_splitmix64_at(seed, v) >> 40) < threshold24) mask[v >> 5] |= 1u << (v & 31);
  uint32_t forced = (uint32_t)(((or_splitmix64_at(seed, vocab) >> 32) * (uint64_t)vocab) >> 32);
  mask[forced >> 5] |= 1u << (forced & 31);
}

/* Synthetic int8 KV row: code_i = ((z_i >> 32) * 255 >> 32) - 127 and scale
 * = lo + (hi - lo) * (z_n >> 40) * 2^-24 (float64 then f32). */
void or_gen_kv_row(uint64_t seed, uint64_t index, uint32_t n, float lo, float hi, int8_t* codes,
                   float* scale) {
  uint64_t base = index * (uint64_t)(n + 1);
  for (uint32_t i = 0; i < n; i++) {
    uint64_t z = or_splitmix64_at(seed, base + i);
    codes[i] = (int8_t)((int)(((z >> 32) * 255ull) >> 32) - 127);
  }
  uint64_t z = or_splitmix64_at(seed, base + n);
  double u = (double)(z >> 40) * (1.0 / 16777216.0);
  *scale = (float)((double)lo + ((double)hi - (double)lo) * u);
}

/* ------------------------------------------ synthetic decoder */

/* The synthetic 8-layer decoder, composed from the reference primitives: per layer
 *   a = rmsNorm(x, attn_norm)                      math.ts:16-32
 *   q, k, v = Wq a, Wk a, Wv a                     cq.ts:106-156 (int8 form)
 *   per-head rmsNormSlice(q, q_norm), (k, k_norm)  runtime.ts:471-486, 647-657
 *   RoPE(q), RoPE(k) at the position               math.ts:94-115
 *   #storeKV, #attention                            runtime.ts:679-786
 *   x = x + Wo o
 *   f = rmsNorm(x, ffn_norm); x = x + Wdown silu(Wup f)   math.ts:12-14
 * embedding row x sqrt(d) in, tied embedding^T out (runtime.ts:305-309,
 * 570-577).  Matrices are int8 with one f32 scale per row. */
typedef struct {
  const int8_t* w;
  const float* s;
  uint32_t n, k;
} or_mat;

typedef struct {
  uint32_t layers, dim, heads, kv_heads, head_dim, ffn, vocab;
  double rope_theta;
  or_mat embedding;
  const or_mat* wq;
  const or_mat* wk;
  const or_mat* wv;
  const or_mat* wo;
  const or_mat* wup;
  const or_mat* wdown;
  const float* attn_norm; /* [layers][dim] */
  const float* ffn_norm;  /* [layers][dim] */
  const float* q_norm;    /* [layers][head_dim] */
  const float* k_norm;    /* [layers][head_dim] */
  const float* final_norm;
} or_synth;

static void synth_matvec(const or_mat* m, const float* x, float* y) {
  or_matvec_i8(m->w, m->s, m->n, m->k, m->k, x, 1, 0, m->n, y);
}

/* First half of layer l for one token at `position`: attention input, Q/K/V
 * projections, per-head norms, RoPE, then #storeKV.  q receives the rotated
 * query; a, k, v are scratch ([dim], [kv_heads * head_dim] x 2). */
static void synth_layer_qkv(const or_synth* md, or_kv* kv, uint32_t l, uint32_t position,
                            const float* x, float* a, float* q, float* k, float* v) {
  uint32_t d = md->dim, hd = md->head_dim;
  or_rms_norm(x, md->attn_norm + (size_t)l * d, d, a);
  synth_matvec(&md->wq[l], a, q);
  synth_matvec(&md->wk[l], a, k);
  synth_matvec(&md->wv[l], a, v);
  for (uint32_t hh = 0; hh < md->heads; hh++)
    or_rms_norm_slice(q, hh * hd, hd, md->q_norm + (size_t)l * hd);
  for (uint32_t hh = 0; hh < md->kv_heads; hh++)
    or_rms_norm_slice(k, hh * hd, hd, md->k_norm + (size_t)l * hd);
  or_rope(q, md->heads, hd, position, md->rope_theta);
  or_rope(k, md->kv_heads, hd, position, md->rope_theta);
  or_kv_store(kv, l, position, k, v);
}

/* Second half: #attention over the cache, x += Wo o, then the FFN residual.
 * x is updated in place; a, o, p, h are scratch. */
static void synth_layer_out(const or_synth* md, const or_kv* kv, uint32_t l, uint32_t position,
                            float* x, const float* q, float* a, float* o, float* p, float* h) {
  uint32_t d = md->dim;
  or_attention(kv, l, position, q, md->heads, o);
  synth_matvec(&md->wo[l], o, p);
  for (uint32_t i = 0; i < d; i++) x[i] = (float)((double)x[i] + (double)p[i]);
  or_rms_norm(x, md->ffn_norm + (size_t)l * d, d, a);
  synth_matvec(&md->wup[l], a, h);
  for (uint32_t i = 0; i < md->ffn; i++) h[i] = (float)or_silu((double)h[i]);
  synth_matvec(&md->wdown[l], h, p);
  for (uint32_t i = 0; i < d; i++) x[i] = (float)((double)x[i] + (double)p[i]);
}

static void synth_embed(const or_synth* md, uint32_t token, float* x) {
  uint32_t d = md->dim;
  or_row_i8(md->embedding.w, md->embedding.s, md->embedding.n, md->embedding.k,
            md->embedding.k, token, x);
  double es = sqrt((double)d);
  for (uint32_t i = 0; i < d; i++) x[i] = (float)((double)x[i] * es);
}

static void synth_logits(const or_synth* md, const float* x, float* a, float* logits) {
  or_rms_norm(x, md->final_norm, md->dim, a);
  synth_matvec(&md->embedding, a, logits);
}

/* One decode step of one sequence at `position`; logits may be NULL. */
int or_synth_step(const or_synth* md, or_kv* kv, uint32_t token, uint32_t position,
                  float* logits, float* hidden_out) {
  uint32_t d = md->dim, hd = md->head_dim;
  uint32_t qw = md->heads * hd, kw = md->kv_heads * hd;
  if (token >= md->vocab || position >= kv->max_length) return OR_INVALID;
  float* x = (float*)malloc(sizeof(float) * d);
  float* a = (float*)malloc(sizeof(float) * d);
  float* q = (float*)malloc(sizeof(float) * qw);
  float* k = (float*)malloc(sizeof(float) * kw);
  float* v = (float*)malloc(sizeof(float) * kw);
  float* o = (float*)malloc(sizeof(float) * qw);
  float* p = (float*)malloc(sizeof(float) * d);
  float* h = (float*)malloc(sizeof(float) * md->ffn);
  synth_embed(md, token, x);
  for (uint32_t l = 0; l < md->layers; l++) {
    synth_layer_qkv(md, kv, l, position, x, a, q, k, v);
    synth_layer_out(md, kv, l, position, x, q, a, o, p, h);
  }
  if (hidden_out) memcpy(hidden_out, x, sizeof(float) * d);
  if (logits) synth_logits(md, x, a, logits);
  free(x); free(a); free(q); free(k); free(v); free(o); free(p); free(h);
  return OR_OK;
}

/* NeedleRuntime.prefill (runtime.ts:227-243) of `count` tokens at positions
 * [position0, position0 + count): the same per-token arithmetic as `count`
 * calls of or_synth_step, evaluated layer by layer -- first every token's
 * Q/K/V and #storeKV, then every token's attention and residual updates --
 * with the tokens of each half spread over `threads` POSIX threads.  The
 * result is bit-identical to the sequential steps: a step stores its own
 * K/V before it attends (runtime.ts:501-502) and attends to positions <= its
 * own, all of which the first half has stored, and no two positions share a
 * slot (position0 + count <= the cache's slots).  Writes the last position's
 * logits when logits != NULL. */
typedef struct {
  const or_synth* md;
  or_kv* kv;
  const uint32_t* tokens;
  uint32_t count, position0, layer, half;
  float *X, *Q; /* [count][dim], [count][heads * head_dim] */
  uint32_t next;
  pthread_mutex_t lock;
} or_prefill_job;

static void* prefill_worker(void* arg) {
  or_prefill_job* job = (or_prefill_job*)arg;
  const or_synth* md = job->md;
  uint32_t d = md->dim, qw = md->heads * md->head_dim, kw = md->kv_heads * md->head_dim;
  float* a = (float*)malloc(sizeof(float) * d);
  float* k = (float*)malloc(sizeof(float) * kw);
  float* v = (float*)malloc(sizeof(float) * kw);
  float* o = (float*)malloc(sizeof(float) * qw);
  float* p = (float*)malloc(sizeof(float) * d);
  float* h = (float*)malloc(sizeof(float) * md->ffn);
  for (;;) {
    pthread_mutex_lock(&job->lock);
    uint32_t i = job->next++;
    pthread_mutex_unlock(&job->lock);
    if (i >= job->count) break;
    float* x = job->X + (size_t)i * d;
    float* q = job->Q + (size_t)i * qw;
    uint32_t position = job->position0 + i;
    if (job->half == 0) {
      if (job->layer == 0) synth_embed(md, job->tokens[i], x);
      synth_layer_qkv(md, job->kv, job->layer, position, x, a, q, k, v);
    } else {
      synth_layer_out(md, job->kv, job->layer, position, x, q, a, o, p, h);
    }
  }
  free(a); free(k); free(v); free(o); free(p); free(h);
  return NULL;
}

int or_synth_prefill(const or_synth* md, or_kv* kv, const uint32_t* tokens, uint32_t count,
                     uint32_t position0, float* logits, uint32_t threads) {
  if (count == 0 || (uint64_t)position0 + count > kv->alloc ||
      (uint64_t)position0 + count > kv->max_length)
    return OR_INVALID;
  for (uint32_t i = 0; i < count; i++)
    if (tokens[i] >= md->vocab) return OR_INVALID;
  if (threads < 1) threads = 1;
  if (threads > count) threads = count;
  or_prefill_job job;
  memset(&job, 0, sizeof job);
  job.md = md;
  job.kv = kv;
  job.tokens = tokens;
  job.count = count;
  job.position0 = position0;
  job.X = (float*)malloc(sizeof(float) * (size_t)count * md->dim);
  job.Q = (float*)malloc(sizeof(float) * (size_t)count * md->heads * md->head_dim);
  pthread_mutex_init(&job.lock, NULL);
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * threads);
  for (uint32_t l = 0; l < md->layers; l++) {
    for (uint32_t half = 0; half < 2; half++) {
      job.layer = l;
      job.half = half;
      job.next = 0;
      for (uint32_t t = 0; t < threads; t++) pthread_create(&tid[t], NULL, prefill_worker, &job);
      for (uint32_t t = 0; t < threads; t++) pthread_join(tid[t], NULL);
    }
  }
  if (logits) {
    float* a = (float*)malloc(sizeof(float) * md->dim);
    synth_logits(md, job.X + (size_t)(count - 1) * md->dim, a, logits);
    free(a);
  }
  pthread_mutex_destroy(&job.lock);
  free(tid);
  free(job.X);
  free(job.Q);
  return OR_OK;
}

/* Writes positions [0, length) of every (layer, kv head) of `kv` with the
 * synthetic prefix rows: K row (l, h, p) = or_gen_kv_row(seed_k, (l * H + h)
 * * max_length + p, ...), V likewise with seed_v. */
void or_kv_fill_synthetic(or_kv* kv, uint64_t seed_k, uint64_t seed_v, uint32_t length, float lo,
                          float hi) {
  for (uint32_t l = 0; l < kv->layers; l++)
    for (uint32_t h = 0; h < kv->kv_heads; h++)
      for (uint32_t p = 0; p < length; p++) {
        uint64_t index = ((uint64_t)l * kv->kv_heads + h) * kv->max_length + p;
        uint32_t slot = or_kv_slot(kv, p);
        size_t base = kv_base(kv, l, h, slot), si = kv_scale_index(kv, l, h, slot);
        or_gen_kv_row(seed_k, index, kv->head_dim, lo, hi, kv->k8 + base, kv->ks + si);
        or_gen_kv_row(seed_v, index, kv->head_dim, lo, hi, kv->v8 + base, kv->vs + si);
      }
}

/* Constrained batched greedy decode (64 ragged sequences, a seeded allowed-token mask per step):
 * for step t and sequence b, run or_synth_step on the current token at
 * position start[b] + t, build the allowed mask with seed
 * or_splitmix64_at(mask_seed, t * 65536 + b), select with or_select_mask
 * (selectToken over the ascending allowed list), and feed the id back.
 * Sequences are independent and are spread over `threads` POSIX threads;
 * each sequence's arithmetic is the single-sequence oracle's. */

typedef struct {
  const or_synth* md;
  or_kv** kvs;
  const uint32_t* tokens;
  const uint32_t* start;
  uint32_t batch, steps, threshold24;
  uint64_t mask_seed;
  uint32_t* out_ids;    /* [steps][batch] */
  double* out_logprob;  /* [steps][batch] */
  const uint32_t* check_steps; /* steps whose logits are kept (may be NULL) */
  uint32_t n_check;
  float* check_logits;  /* [n_check][batch][vocab] */
  uint32_t next;        /* work counter */
  pthread_mutex_t lock;
  int status;
} or_batch_job;

static void* batch_worker(void* arg) {
  or_batch_job* job = (or_batch_job*)arg;
  const or_synth* md = job->md;
  float* logits = (float*)malloc(sizeof(float) * md->vocab);
  uint32_t* mask = (uint32_t*)malloc(sizeof(uint32_t) * ((md->vocab + 31) / 32));
  for (;;) {
    pthread_mutex_lock(&job->lock);
    uint32_t b = job->next++;
    pthread_mutex_unlock(&job->lock);
    if (b >= job->batch) break;
    uint32_t token = job->tokens[b];
    for (uint32_t t = 0; t < job->steps; t++) {
      if (or_synth_step(md, job->kvs[b], token, job->start[b] + t, logits, NULL) != OR_OK) {
        job->status = OR_INVALID;
        break;
      }
      for (uint32_t c = 0; c < job->n_check; c++)
        if (job->check_steps[c] == t)
          memcpy(job->check_logits + ((size_t)c * job->batch + b) * md->vocab, logits,
                 sizeof(float) * md->vocab);
      or_gen_mask(or_splitmix64_at(job->mask_seed, (uint64_t)t * 65536 + b), md->vocab,
                  job->threshold24, mask);
      uint32_t id;
      double lp;
      or_select_mask(logits, md->vocab, mask, &id, &lp);
      job->out_ids[(size_t)t * job->batch + b] = id;
      job->out_logprob[(size_t)t * job->batch + b] = lp;
      token = id;
    }
  }
  free(logits);
  free(mask);
  return NULL;
}

int or_synth_decode_batch(const or_synth* md, or_kv** kvs, const uint32_t* tokens,
                          const uint32_t* start, uint32_t batch, uint32_t steps,
                          uint64_t mask_seed, uint32_t threshold24, uint32_t* out_ids,
                          double* out_logprob, uint32_t threads, const uint32_t* check_steps,
                          uint32_t n_check, float* check_logits) {
  or_batch_job job = {md, kvs, tokens, start, batch, steps, threshold24, mask_seed,
                      out_ids, out_logprob, check_steps, check_steps ? n_check : 0,
                      check_logits, 0, PTHREAD_MUTEX_INITIALIZER, OR_OK};
  if (threads < 1) threads = 1;
  if (threads > batch) threads = batch;
  pthread_t* tid = (pthread_t*)malloc(sizeof(pthread_t) * threads);
  for (uint32_t i = 0; i < threads; i++) pthread_create(&tid[i], NULL, batch_worker, &job);
  for (uint32_t i = 0; i < threads; i++) pthread_join(tid[i], NULL);
  free(tid);
  return job.status;
}
