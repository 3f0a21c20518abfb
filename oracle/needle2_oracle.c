/*
 * needle2_oracle.c -- CPU restatement of NeedleRuntime.step for the full
 * Needle 2 graph (model/runtime.ts:280-583 of needle.js, CPU path), each
 * matrix either in the int8 form or as the archive's Cactus-Quant matrix
 * (backends/cq.ts:106-295 through or_cq_matvec / or_cq_row).  TEST
 * INFRASTRUCTURE ONLY (see
 * needle_oracle.c for the semantics rules: binary64, no contraction, f32
 * stores).  Builds into liboracle.so with needle_oracle.c.
 *
 * Parity pins: the composition is checked against an independent float64
 * numpy model of the same graph (tests/test_oracle_needle2.py) on a reduced
 * geometry, and prefill == repeated step by construction; every primitive is
 * pinned in needle_oracle.c.  The confidence pool (OnlineProbePool,
 * runtime.ts:48-105) is checked against the closed form of its online
 * update (a softmax over every pooled cell, scipy.special.softmax, then the
 * projection and a sigmoid) on cells recorded from the same steps.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define OR_OK 0
#define OR_INVALID 1
#define OR_OVERFLOW 3

/* Primitives from needle_oracle.c. */
double or_sigmoid(double value);
void or_rms_norm(const float* input, const float* scale, uint32_t n, float* output);
void or_rms_unit(const float* input, uint32_t n, float* output);
void or_rms_norm_slice(float* values, uint32_t offset, uint32_t length, const float* scale);
void or_sinkhorn(float* logits, uint32_t size, uint32_t iterations);
void or_rope(float* vec, uint32_t heads, uint32_t head_dim, uint32_t position, double theta);
int or_hadamard_mlp(const float* input, uint32_t n, const float* d1, const float* d2,
                    const float* d3, uint32_t hdim, float* output);
int or_matvec_i8(const int8_t* w, const float* scales, uint32_t n, uint32_t k, uint32_t g,
                 const float* x, uint32_t batch, uint32_t row_start, uint32_t row_count, float* y);
int or_row_i8(const int8_t* w, const float* scales, uint32_t n, uint32_t k, uint32_t g,
              uint32_t row, float* out);
int or_cq_matvec(const uint8_t* packed, const uint16_t* norms, const float* codebook, uint32_t n,
                 uint32_t k, uint32_t g, uint32_t bits, const float* x, uint32_t batch,
                 uint32_t row_start, uint32_t row_count, float* y);
int or_cq_row(const uint8_t* packed, const uint16_t* norms, const float* codebook, uint32_t n,
              uint32_t k, uint32_t g, uint32_t bits, uint32_t row, float* out);
typedef struct or_kv or_kv;
or_kv* or_kv_create(uint32_t layers, uint32_t kv_heads, uint32_t head_dim, uint32_t max_length,
                    uint32_t sink, uint32_t window, int float_mode);
void or_kv_destroy(or_kv* kv);
int or_kv_store(or_kv* kv, uint32_t layer, uint32_t position, const float* k, const float* v);
int or_attention(const or_kv* kv, uint32_t layer, uint32_t position, const float* q,
                 uint32_t q_heads, float* out);

/* A matrix [n][k]: int8 codes w with per-row scales s, or (bits != 0) the
 * archive's Cactus-Quant form -- packed rows, binary16 norms [n][kpad / g]
 * and the 28-float codebook (CQ2, CQ3, CQ4) -- with w and s unused. */
typedef struct {
  const int8_t* w;
  const float* s;
  uint32_t n, k;
  uint32_t bits, g;
  const uint8_t* packed;
  const uint16_t* norms;
  const float* codebook;
} n2_mat;

typedef struct {
  uint32_t vocab, dim, heads, kv_heads, layers, head_dim, max_length, hadamard, lanes;
  uint32_t engram_slots, engram_sub, engram_tables, engram_taps;
  uint32_t n_orders, n_sites;
  uint32_t orders[4], sites[4];
  double rope_theta;
  uint32_t kv_window;
  n2_mat embedding;
  const n2_mat* wq;   /* [layers] */
  const n2_mat* wk;
  const n2_mat* wv;
  const n2_mat* wgate;
  const n2_mat* wo;
  const float* norm_input;      /* [layers][dim] */
  const float* query_norm;      /* [layers][head_dim] */
  const float* key_norm;        /* [layers][head_dim] */
  const float* post_attn_norm;  /* [layers][dim] */
  const float* attention_gate;  /* [layers] */
  const float* pre_hadamard_norm; /* [layers][dim] */
  const float* d1;              /* [layers][dim] */
  const float* d2;              /* [layers][hadamard] */
  const float* d3;              /* [layers][dim] */
  n2_mat phi_pre;               /* [layers*lanes][lanes*dim] */
  n2_mat phi_post;
  n2_mat phi_res;               /* [layers*lanes*lanes][lanes*dim] */
  const float* a_pre;           /* [layers] */
  const float* a_post;
  const float* a_res;
  const float* b_pre;           /* [layers*lanes] */
  const float* b_post;
  const float* b_res;           /* [layers*lanes*lanes] */
  const n2_mat* eg_tables;      /* [sites], [tables*slots][sub] */
  const n2_mat* eg_key;         /* [sites], [dim][tables*sub] */
  const n2_mat* eg_value;
  const float* eg_taps;         /* [sites][taps][dim] */
  const float* final_norm;
  /* Confidence probe head (CactProbeHead, cact.ts:105-112); probes == NULL
   * when the archive has none. */
  const float* probes;          /* [probe_count][dim] */
  uint32_t probe_count, probe_out;
  const float* probe_projection; /* [probe_out][probe_count * dim] */
  const float* probe_bias;      /* [probe_out] */
} n2_model;

typedef struct {
  const n2_model* md;
  uint32_t max_length, sink, position;
  or_kv* kv;
  uint32_t* history;
  uint32_t history_len;
  float* ring;      /* [sites][depth][dim] */
  uint8_t* valid;   /* [sites][depth] */
  uint32_t depth, engram_position;
  /* OnlineProbePool state (runtime.ts:48-62); cells_out, when set, records
   * every pooled cell (for the closed-form check). */
  double* pool_max;       /* [probe_count] */
  double* pool_den;       /* [probe_count] */
  double* pool_weighted;  /* [probe_count][dim] */
  float* cells_out;
  uint32_t cells_count, cells_cap;
} n2_state;

/* matvec (backends/cpu.ts:12-26, or cq.ts:106-231 for a CQ matrix). */
static void mv(const n2_mat* m, const float* x, uint32_t row_start, uint32_t rows, float* y) {
  if (m->bits)
    or_cq_matvec(m->packed, m->norms, m->codebook, m->n, m->k, m->g, m->bits, x, 1, row_start,
                 rows, y);
  else
    or_matvec_i8(m->w, m->s, m->n, m->k, m->k, x, 1, row_start, rows, y);
}

/* row (backends/cpu.ts:28-31, or dequantizeCqRow, cq.ts:243-295). */
static void mat_row(const n2_mat* m, uint32_t row, float* out) {
  if (m->bits)
    or_cq_row(m->packed, m->norms, m->codebook, m->n, m->k, m->g, m->bits, row, out);
  else
    or_row_i8(m->w, m->s, m->n, m->k, m->k, row, out);
}

/* runtime.ts:150-225 reset: KV allocation (int8, or float32 with
 * float_kv: kvCache "float32", runtime.ts:192-196, 686-692), engram ring
 * depth. */
n2_state* or_n2_create_kv(const n2_model* md, uint32_t max_length, uint32_t sink, int float_kv);
n2_state* or_n2_create(const n2_model* md, uint32_t max_length, uint32_t sink) {
  return or_n2_create_kv(md, max_length, sink, 0);
}

n2_state* or_n2_create_kv(const n2_model* md, uint32_t max_length, uint32_t sink, int float_kv) {
  if (max_length == 0 || max_length > md->max_length) return NULL;
  n2_state* st = (n2_state*)calloc(1, sizeof(n2_state));
  st->md = md;
  st->max_length = max_length;
  st->sink = sink < max_length ? sink : max_length;
  st->kv = or_kv_create(md->layers, md->kv_heads, md->head_dim, max_length, st->sink,
                        md->kv_window, float_kv);
  st->history = (uint32_t*)calloc(max_length, sizeof(uint32_t));
  uint32_t max_order = 1;
  for (uint32_t i = 0; i < md->n_orders; i++)
    if (md->orders[i] > max_order) max_order = md->orders[i];
  st->depth = (md->engram_taps - 1) * max_order + 1;
  st->ring = (float*)calloc((size_t)md->n_sites * st->depth * md->dim, sizeof(float));
  st->valid = (uint8_t*)calloc((size_t)md->n_sites * st->depth, 1);
  if (md->probes && md->probe_count) {
    st->pool_max = (double*)malloc(sizeof(double) * md->probe_count);
    for (uint32_t p = 0; p < md->probe_count; p++) st->pool_max[p] = -INFINITY;
    st->pool_den = (double*)calloc(md->probe_count, sizeof(double));
    st->pool_weighted = (double*)calloc((size_t)md->probe_count * md->dim, sizeof(double));
  }
  return st;
}

/* runtime.ts:64-91 OnlineProbePool.add: per probe, score = (cell . probe) /
 * sqrt(dim) summed in float64, then the online softmax-weighted update of
 * (maximum, denominator, weighted cell sum). */
static void pool_add(n2_state* st, const float* cell) {
  const n2_model* md = st->md;
  if (!st->pool_max) return;
  const uint32_t d = md->dim;
  if (st->cells_out && st->cells_count < st->cells_cap)
    memcpy(st->cells_out + (size_t)st->cells_count++ * d, cell, sizeof(float) * d);
  const double scale = 1.0 / sqrt((double)d);
  for (uint32_t p = 0; p < md->probe_count; p++) {
    double score = 0;
    const float* probe = md->probes + (size_t)p * d;
    for (uint32_t i = 0; i < d; i++) score += (double)cell[i] * (double)probe[i];
    score *= scale;
    const double previous = st->pool_max[p];
    double* w = st->pool_weighted + (size_t)p * d;
    if (score <= previous) {
      const double weight = exp(score - previous);
      st->pool_den[p] = st->pool_den[p] + weight;
      for (uint32_t i = 0; i < d; i++) w[i] = w[i] + weight * (double)cell[i];
    } else {
      const double old = isfinite(previous) ? exp(previous - score) : 0.0;
      st->pool_den[p] = st->pool_den[p] * old + 1;
      for (uint32_t i = 0; i < d; i++) w[i] = w[i] * old + (double)cell[i];
      st->pool_max[p] = score;
    }
  }
}

/* runtime.ts:93-104 output() then runtime.ts:641-645 confidence():
 * pooled = f32(weighted / max(denominator, 1e-30)), denseMatvec with the
 * bias (backends/cq.ts:297-318: float64 sum from the bias, f32 store), and
 * the sigmoid of output 0 in float64. */
int or_n2_confidence(const n2_state* st, double* confidence) {
  const n2_model* md = st->md;
  if (!st->pool_max || md->probe_out == 0) return OR_INVALID;
  const uint32_t d = md->dim, width = md->probe_count * d;
  float* pooled = (float*)malloc(sizeof(float) * width);
  for (uint32_t p = 0; p < md->probe_count; p++) {
    double den = st->pool_den[p] > 1e-30 ? st->pool_den[p] : 1e-30;
    for (uint32_t i = 0; i < d; i++)
      pooled[(size_t)p * d + i] = (float)(st->pool_weighted[(size_t)p * d + i] / den);
  }
  double sum = (double)md->probe_bias[0];
  for (uint32_t j = 0; j < width; j++) sum += (double)md->probe_projection[j] * (double)pooled[j];
  free(pooled);
  *confidence = or_sigmoid((double)(float)sum);
  return OR_OK;
}

/* Records the next `cap` pooled cells into cells ([cap][dim]); count out. */
void or_n2_record_cells(n2_state* st, float* cells, uint32_t cap) {
  st->cells_out = cells;
  st->cells_cap = cap;
  st->cells_count = 0;
}

uint32_t or_n2_recorded_cells(const n2_state* st) { return st->cells_count; }

void or_n2_destroy(n2_state* st) {
  if (!st) return;
  or_kv_destroy(st->kv);
  free(st->history);
  free(st->ring);
  free(st->valid);
  free(st->pool_max);
  free(st->pool_den);
  free(st->pool_weighted);
  free(st);
}

or_kv* or_n2_kv(n2_state* st) { return st->kv; }

/* runtime.ts:788-818 #engramLookup (multiplicative hashing of the history). */
static void engram_lookup(const n2_state* st, uint32_t* indices, uint32_t* valid) {
  const n2_model* md = st->md;
  uint32_t heads_per_order = md->engram_tables / md->n_orders;
  uint32_t table = 0;
  for (uint32_t oi = 0; oi < md->n_orders; oi++) {
    uint32_t order = md->orders[oi];
    for (uint32_t h = 0; h < heads_per_order; h++) {
      uint32_t hash = (uint32_t)(0x9E3779B9u * (uint32_t)(oi * heads_per_order + h + 1));
      int is_valid = 1;
      for (uint32_t off = 0; off < order; off++) {
        int64_t hi = (int64_t)st->history_len - 1 - off;
        uint32_t token = hi >= 0 ? st->history[hi] : 0;
        hash = (uint32_t)((hash ^ token) * 0x01000193u);
        if (off == order - 1) is_valid = hi >= 0;
      }
      hash = hash ^ (hash >> 15);
      indices[table] = hash % md->engram_slots;
      valid[table] = is_valid ? 1 : 0;
      table++;
    }
  }
}

/* One token of NeedleRuntime.step; logits (vocab) may be NULL. */
int or_n2_step(n2_state* st, uint32_t token, float* logits) {
  const n2_model* md = st->md;
  const uint32_t d = md->dim, L = md->lanes, hd = md->head_dim;
  const uint32_t qw = md->heads * hd, kw = md->kv_heads * hd;
  if (st->position >= st->max_length) return OR_OVERFLOW;
  if (token >= md->vocab) return OR_INVALID;
  const uint32_t position = st->position;
  st->history[st->history_len++] = token;

  float* emb = (float*)malloc(sizeof(float) * d);
  float* x = (float*)malloc(sizeof(float) * L * d);
  float* nx = (float*)malloc(sizeof(float) * L * d);
  float* nl = (float*)malloc(sizeof(float) * L * d);
  float* upd = (float*)malloc(sizeof(float) * d);
  float* blk = (float*)malloc(sizeof(float) * d);
  float* ain = (float*)malloc(sizeof(float) * d);
  float* q = (float*)malloc(sizeof(float) * qw);
  float* k = (float*)malloc(sizeof(float) * kw);
  float* v = (float*)malloc(sizeof(float) * kw);
  float* gate = (float*)malloc(sizeof(float) * qw);
  float* att = (float*)malloc(sizeof(float) * qw);
  float* proj = (float*)malloc(sizeof(float) * d);
  float* tmp = (float*)malloc(sizeof(float) * d);
  float* tmp2 = (float*)malloc(sizeof(float) * d);
  float* mlp = (float*)malloc(sizeof(float) * d);
  float* delta = (float*)malloc(sizeof(float) * d);
  float phi_pre[16], phi_post[16], phi_res[64], hpre[16], hpost[16], routing[64];
  const uint32_t cat_n = md->engram_tables * md->engram_sub;
  float* cat = (float*)malloc(sizeof(float) * cat_n);
  float* ekeys = (float*)calloc((size_t)md->n_sites * d, sizeof(float));
  float* evals = (float*)calloc((size_t)md->n_sites * d, sizeof(float));

  /* runtime.ts:305-313 */
  mat_row(&md->embedding, token, emb);
  double es = sqrt((double)d);
  for (uint32_t i = 0; i < d; i++) emb[i] = (float)((double)emb[i] * es);
  pool_add(st, emb); /* runtime.ts:310 */
  for (uint32_t ln = 0; ln < L; ln++) memcpy(x + ln * d, emb, sizeof(float) * d);

  /* runtime.ts:820-877 #engramStep */
  if (md->n_sites > 0) {
    uint32_t indices[16], valid[16];
    engram_lookup(st, indices, valid);
    uint32_t max_order = 1;
    for (uint32_t i = 0; i < md->n_orders; i++)
      if (md->orders[i] > max_order) max_order = md->orders[i];
    for (uint32_t s = 0; s < md->n_sites; s++) {
      memset(cat, 0, sizeof(float) * cat_n);
      for (uint32_t t = 0; t < md->engram_tables; t++)
        if (valid[t]) {
          const n2_mat* tb = &md->eg_tables[s];
          mat_row(tb, t * md->engram_slots + indices[t], cat + t * md->engram_sub);
        }
      mv(&md->eg_key[s], cat, 0, d, ekeys + s * d);
      float* value_now = tmp;
      mv(&md->eg_value[s], cat, 0, d, value_now);
      uint32_t slot = st->engram_position % st->depth;
      memcpy(st->ring + ((size_t)s * st->depth + slot) * d, value_now, sizeof(float) * d);
      st->valid[s * st->depth + slot] = 1;
      float* mixed = evals + s * d;
      memset(mixed, 0, sizeof(float) * d);
      for (uint32_t tap = 0; tap < md->engram_taps; tap++) {
        int64_t prev = (int64_t)st->engram_position - (int64_t)tap * max_order;
        if (prev < 0) continue;
        uint32_t ps = (uint32_t)(prev % st->depth);
        if (!st->valid[s * st->depth + ps]) continue;
        const float* ring = st->ring + ((size_t)s * st->depth + ps) * d;
        const float* taps = md->eg_taps + ((size_t)s * md->engram_taps + tap) * d;
        for (uint32_t i = 0; i < d; i++)
          mixed[i] = (float)((double)mixed[i] + (double)taps[i] * (double)ring[i]);
      }
    }
    st->engram_position++;
  }

  for (uint32_t l = 0; l < md->layers; l++) {
    /* runtime.ts:385-420 mHC pre-mix */
    or_rms_unit(x, L * d, nl);
    mv(&md->phi_pre, nl, l * L, L, phi_pre);
    mv(&md->phi_post, nl, l * L, L, phi_post);
    mv(&md->phi_res, nl, l * L * L, L * L, phi_res);
    uint32_t own = l % L;
    for (uint32_t ln = 0; ln < L; ln++) {
      double off = ln == own ? 4 : -4;
      hpre[ln] = (float)or_sigmoid((double)md->a_pre[l] * (double)phi_pre[ln] +
                                   (double)md->b_pre[l * L + ln] + off);
    }
    for (uint32_t c = 0; c < d; c++) {
      double sum = 0;
      for (uint32_t ln = 0; ln < L; ln++) sum += (double)hpre[ln] * (double)x[ln * d + c];
      upd[c] = (float)sum;
    }
    /* runtime.ts:422-438 engram injection */
    memcpy(blk, upd, sizeof(float) * d);
    for (uint32_t s = 0; s < md->n_sites; s++) {
      if (md->sites[s] != l) continue;
      or_rms_unit(upd, d, tmp);
      or_rms_unit(ekeys + s * d, d, tmp2);
      double dot = 0;
      for (uint32_t i = 0; i < d; i++) dot += (double)tmp[i] * (double)tmp2[i];
      double alpha = or_sigmoid(dot / sqrt((double)d));
      for (uint32_t i = 0; i < d; i++)
        blk[i] = (float)((double)upd[i] + alpha * (double)evals[s * d + i]);
      break;
    }
    /* runtime.ts:441, 465-507 gated GQA */
    or_rms_norm(blk, md->norm_input + (size_t)l * d, d, ain);
    mv(&md->wq[l], ain, 0, qw, q);
    mv(&md->wk[l], ain, 0, kw, k);
    mv(&md->wv[l], ain, 0, kw, v);
    mv(&md->wgate[l], ain, 0, qw, gate);
    for (uint32_t h = 0; h < md->heads; h++)
      or_rms_norm_slice(q, h * hd, hd, md->query_norm + (size_t)l * hd);
    for (uint32_t h = 0; h < md->kv_heads; h++)
      or_rms_norm_slice(k, h * hd, hd, md->key_norm + (size_t)l * hd);
    or_rope(q, md->heads, hd, position, md->rope_theta);
    or_rope(k, md->kv_heads, hd, position, md->rope_theta);
    or_kv_store(st->kv, l, position, k, v);
    or_attention(st->kv, l, position, q, md->heads, att);
    for (uint32_t i = 0; i < qw; i++)
      att[i] = (float)((double)att[i] * or_sigmoid((double)gate[i]));
    mv(&md->wo[l], att, 0, d, proj);
    /* runtime.ts:585-611 #attentionDelta */
    or_rms_norm(proj, md->post_attn_norm + (size_t)l * d, d, tmp);
    double ascale = or_sigmoid((double)md->attention_gate[l]);
    for (uint32_t i = 0; i < d; i++) tmp2[i] = (float)((double)blk[i] + ascale * (double)tmp[i]);
    or_rms_norm(tmp2, md->pre_hadamard_norm + (size_t)l * d, d, tmp);
    or_hadamard_mlp(tmp, d, md->d1 + (size_t)l * d, md->d2 + (size_t)l * md->hadamard,
                    md->d3 + (size_t)l * d, md->hadamard, mlp);
    for (uint32_t i = 0; i < d; i++)
      delta[i] = (float)((double)tmp2[i] + (double)mlp[i] - (double)upd[i]);
    /* runtime.ts:509-542 h-post, Sinkhorn routing, lane update */
    for (uint32_t ln = 0; ln < L; ln++) {
      double off = ln == own ? 0 : -4;
      hpost[ln] = (float)(2 * or_sigmoid((double)md->a_post[l] * (double)phi_post[ln] +
                                         (double)md->b_post[l * L + ln] + off));
    }
    for (uint32_t i = 0; i < L * L; i++)
      routing[i] = (float)((double)md->a_res[l] * (double)phi_res[i] +
                           (double)md->b_res[l * L * L + i]);
    or_sinkhorn(routing, L, 20);
    for (uint32_t ln = 0; ln < L; ln++)
      for (uint32_t c = 0; c < d; c++) {
        double sum = 0;
        for (uint32_t src = 0; src < L; src++)
          sum += (double)routing[ln * L + src] * (double)x[src * d + c];
        nx[ln * d + c] = (float)(sum + (double)hpost[ln] * (double)delta[c]);
      }
    memcpy(x, nx, sizeof(float) * L * d);
    /* runtime.ts:543-550: the lane mean after the layer joins the pool. */
    if (st->pool_max) {
      for (uint32_t c = 0; c < d; c++) {
        double sum = 0;
        for (uint32_t ln = 0; ln < L; ln++) sum += x[ln * d + c];
        tmp[c] = (float)(sum / L);
      }
      pool_add(st, tmp);
    }
  }
  st->position++;
  if (logits) {
    /* runtime.ts:570-577 */
    for (uint32_t c = 0; c < d; c++) {
      double sum = 0;
      for (uint32_t ln = 0; ln < L; ln++) sum += x[ln * d + c];
      tmp[c] = (float)(sum / L);
    }
    or_rms_norm(tmp, md->final_norm, d, tmp2);
    mv(&md->embedding, tmp2, 0, md->vocab, logits);
  }
  free(emb); free(x); free(nx); free(nl); free(upd); free(blk); free(ain); free(q); free(k);
  free(v); free(gate); free(att); free(proj); free(tmp); free(tmp2); free(mlp); free(delta);
  free(cat); free(ekeys); free(evals);
  return OR_OK;
}
