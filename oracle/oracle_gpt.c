// oracle_gpt.c - CPU restatement of the reference's GPT-2 KV-cache decode
// (model.c:437-520) with its pieces: layernorm.c:8-38, the tanh GELU of
// activation.c:43-50, the feed-forward of feedforward.c:9-42, the f32 matmul of
// matrix.c:178-199 and the GPTC tensor order of checkpoint.c:17-44.
//
// TEST INFRASTRUCTURE ONLY (see oracle.h): compiled like the reference (ISO C11,
// no contraction), pinned by tests/test_gpt_oracle.py against fixtures the
// compiled reference wrote (tests/golden/gen_golden.c gpt).
#include <math.h>
#include <pthread.h>
#include <stdlib.h>
#include <string.h>

#include "oracle.h"
#include "synth.h"

// layernorm.c:8-38 for each of `rows` rows: mean and variance as sequential float
// sums in j order, each divided by cols; then (x - mean) * inv_std, then * gamma + beta.
void or_layernorm(const float *x, int rows, int cols, const float *gamma, const float *beta, float eps, float *y) {
  for (int i = 0; i < rows; i++) {
    const float *xr = x + (size_t)i * cols;
    float *yr = y + (size_t)i * cols;
    float mean = 0.0f;
    for (int j = 0; j < cols; j++) mean += xr[j];
    mean /= cols;
    float var = 0.0f;
    for (int j = 0; j < cols; j++) {
      const float d = xr[j] - mean;
      var += d * d;
    }
    var /= cols;
    const float inv_std = 1.0f / sqrtf(var + eps);
    for (int j = 0; j < cols; j++) yr[j] = (xr[j] - mean) * inv_std;
    for (int j = 0; j < cols; j++) yr[j] = yr[j] * gamma[j] + beta[j];
  }
}

// activation.c:43-50, element-wise, with the host libm tanhf
void or_gelu(const float *x, size_t n, float *y) {
  const float k = 0.7978845608028654f;
  for (size_t i = 0; i < n; i++) {
    const float v = x[i];
    const float inner = k * (v + 0.044715f * v * v * v);
    y[i] = 0.5f * v * (1.0f + tanhf(inner));
  }
}

// Tensors of the model in the GPTC order (checkpoint.c:17-44); returns the count.
int or_gpt_tensors(const OrGPT *m, float **list, size_t *sizes) {
  const size_t V = (size_t)m->vocab, dm = (size_t)m->d_model, ff = (size_t)m->d_ff, S = (size_t)m->max_seq;
  int n = 0;
#define PUT(p, sz) do { list[n] = (p); sizes[n] = (sz); n++; } while (0)
  PUT(m->wte, V * dm);
  PUT(m->wpe, S * dm);
  for (int l = 0; l < m->n_layers; l++) {
    OrGBlock *b = &m->blocks[l];
    PUT(b->Wq, dm * dm); PUT(b->Wk, dm * dm); PUT(b->Wv, dm * dm); PUT(b->Wo, dm * dm);
    PUT(b->bq, dm); PUT(b->bk, dm); PUT(b->bv, dm); PUT(b->bo, dm);
    PUT(b->g1, dm); PUT(b->be1, dm); PUT(b->g2, dm); PUT(b->be2, dm);
    PUT(b->W1, dm * ff); PUT(b->bf1, ff); PUT(b->W2, ff * dm); PUT(b->bf2, dm);
  }
  PUT(m->lnf_g, dm);
  PUT(m->lnf_b, dm);
  PUT(m->lm_head, dm * V);
#undef PUT
  return n;
}

int or_gpt_alloc(OrGPT *m, const int32_t cfg[6]) {
  memset(m, 0, sizeof *m);
  m->vocab = cfg[0]; m->d_model = cfg[1]; m->n_heads = cfg[2]; m->n_layers = cfg[3]; m->d_ff = cfg[4];
  m->max_seq = cfg[5];
  const size_t V = (size_t)m->vocab, dm = (size_t)m->d_model, ff = (size_t)m->d_ff, S = (size_t)m->max_seq;
  m->blocks = (OrGBlock*)calloc((size_t)m->n_layers, sizeof(OrGBlock));
  if (!m->blocks) return 1;
#define AL(p, sz) do { (p) = (float*)calloc((sz), sizeof(float)); if (!(p)) return 1; } while (0)
  AL(m->wte, V * dm); AL(m->wpe, S * dm);
  for (int l = 0; l < m->n_layers; l++) {
    OrGBlock *b = &m->blocks[l];
    AL(b->Wq, dm * dm); AL(b->Wk, dm * dm); AL(b->Wv, dm * dm); AL(b->Wo, dm * dm);
    AL(b->bq, dm); AL(b->bk, dm); AL(b->bv, dm); AL(b->bo, dm);
    AL(b->g1, dm); AL(b->be1, dm); AL(b->g2, dm); AL(b->be2, dm);
    AL(b->W1, dm * ff); AL(b->bf1, ff); AL(b->W2, ff * dm); AL(b->bf2, dm);
  }
  AL(m->lnf_g, dm); AL(m->lnf_b, dm); AL(m->lm_head, dm * V);
#undef AL
  return 0;
}

void or_gpt_free(OrGPT *m) {
  if (m->blocks) {
    for (int l = 0; l < m->n_layers; l++) {
      OrGBlock *b = &m->blocks[l];
      float *p[16] = {b->Wq, b->Wk, b->Wv, b->Wo, b->bq, b->bk, b->bv, b->bo,
                      b->g1, b->be1, b->g2, b->be2, b->W1, b->bf1, b->W2, b->bf2};
      for (int i = 0; i < 16; i++) free(p[i]);
    }
  }
  free(m->blocks); free(m->wte); free(m->wpe); free(m->lnf_g); free(m->lnf_b); free(m->lm_head);
  memset(m, 0, sizeof *m);
}

// Seeded weights (synth.h) by GPTC position t: matrices and embeddings N(0, 0.02),
// biases and LayerNorm betas N(0, 0.02), gammas 1 + N(0, 0.1); tensor id = t.
int or_gpt_synth(OrGPT *m, const int32_t cfg[6], uint64_t seed) {
  if (or_gpt_alloc(m, cfg)) { or_gpt_free(m); return 1; }
  float *list[2 + 16 * 64 + 3];
  size_t sizes[2 + 16 * 64 + 3];
  if (m->n_layers > 64) { or_gpt_free(m); return 1; }
  const int n = or_gpt_tensors(m, list, sizes);
  for (int t = 0; t < n; t++) {
    const int in_layer = t >= 2 && t < 2 + 16 * m->n_layers, slot = in_layer ? (t - 2) % 16 : -1;
    const int gamma = (in_layer && (slot == 8 || slot == 10)) || t == n - 3;
    syn_fill(list[t], sizes[t], seed, (uint64_t)t, gamma ? 0.1 : 0.02);
    if (gamma)
      for (size_t i = 0; i < sizes[t]; i++) list[t][i] = 1.0f + list[t][i];
  }
  return 0;
}

uint64_t or_gpt_hash(const OrGPT *m) {
  float *list[2 + 16 * 64 + 3];
  size_t sizes[2 + 16 * 64 + 3];
  const int n = or_gpt_tensors(m, list, sizes);
  uint64_t h = 0;
  for (int t = 0; t < n; t++) h = h * 31 + syn_hash_f32(list[t], sizes[t], 0);
  return h;
}

// model.c:437-448: per layer K and V of (max_seq, d_model)
int or_gkv_create(OrKV *kv, const OrGPT *m) {
  kv->n_layers = m->n_layers; kv->max_seq = m->max_seq; kv->kv_dim = m->d_model; kv->len = 0;
  const size_t n = (size_t)m->n_layers * m->max_seq * m->d_model;
  kv->k = (float*)calloc(n, sizeof(float));
  kv->v = (float*)calloc(n, sizeof(float));
  return (kv->k && kv->v) ? 0 : 1;
}

// model.c:457-520: one token at position kv->len, logits (vocab).
void or_gpt_decode_step(const OrGPT *m, OrKV *kv, int token, float *logits) {
  const int dm = m->d_model, nh = m->n_heads, hd = dm / nh, ff = m->d_ff, pos = kv->len;
  const float scale = 1.0f / sqrtf((float)hd);
  const float eps = 1e-5f;                                         // model.c:15
  float *x = (float*)calloc((size_t)dm, 4), *xn = (float*)calloc((size_t)dm, 4);
  float *q = (float*)calloc((size_t)dm, 4), *k = (float*)calloc((size_t)dm, 4), *v = (float*)calloc((size_t)dm, 4);
  float *cat = (float*)calloc((size_t)dm, 4), *att = (float*)calloc((size_t)dm, 4), *fo = (float*)calloc((size_t)dm, 4);
  float *h = (float*)calloc((size_t)ff, 4), *ha = (float*)calloc((size_t)ff, 4);
  float *sc = (float*)malloc((size_t)(pos + 1) * 4);
  for (int j = 0; j < dm; j++) x[j] = m->wte[(size_t)token * dm + j] + m->wpe[(size_t)pos * dm + j];
  for (int l = 0; l < m->n_layers; l++) {
    const OrGBlock *b = &m->blocks[l];
    float *kc = &kv->k[(size_t)l * kv->max_seq * dm];
    float *vc = &kv->v[(size_t)l * kv->max_seq * dm];
    or_layernorm(x, 1, dm, b->g1, b->be1, eps, xn);
    or_matmul_row(xn, b->Wq, dm, dm, q); for (int j = 0; j < dm; j++) q[j] = q[j] + b->bq[j];
    or_matmul_row(xn, b->Wk, dm, dm, k); for (int j = 0; j < dm; j++) k[j] = k[j] + b->bk[j];
    or_matmul_row(xn, b->Wv, dm, dm, v); for (int j = 0; j < dm; j++) v[j] = v[j] + b->bv[j];
    memcpy(&kc[(size_t)pos * dm], k, (size_t)dm * 4);
    memcpy(&vc[(size_t)pos * dm], v, (size_t)dm * 4);
    for (int hh = 0; hh < nh; hh++) {                               // one query row, every head
      const int off = hh * hd;
      float mx = -INFINITY;
      for (int j = 0; j <= pos; j++) {
        float dot = 0.0f;
        for (int d = 0; d < hd; d++) dot += q[off + d] * kc[(size_t)j * dm + off + d];
        sc[j] = dot * scale;
        if (sc[j] > mx) mx = sc[j];
      }
      float sum = 0.0f;
      for (int j = 0; j <= pos; j++) { sc[j] = expf(sc[j] - mx); sum += sc[j]; }
      for (int d = 0; d < hd; d++) {
        float acc = 0.0f;
        for (int j = 0; j <= pos; j++) acc += (sc[j] / sum) * vc[(size_t)j * dm + off + d];
        cat[off + d] = acc;
      }
    }
    or_matmul_row(cat, b->Wo, dm, dm, att); for (int j = 0; j < dm; j++) att[j] = att[j] + b->bo[j];
    for (int j = 0; j < dm; j++) x[j] = x[j] + att[j];
    or_layernorm(x, 1, dm, b->g2, b->be2, eps, xn);
    or_matmul_row(xn, b->W1, dm, ff, h); for (int j = 0; j < ff; j++) h[j] += b->bf1[j];
    or_gelu(h, (size_t)ff, ha);
    or_matmul_row(ha, b->W2, ff, dm, fo); for (int j = 0; j < dm; j++) fo[j] += b->bf2[j];
    for (int j = 0; j < dm; j++) x[j] = x[j] + fo[j];
  }
  or_layernorm(x, 1, dm, m->lnf_g, m->lnf_b, eps, xn);
  or_matmul_row(xn, m->lm_head, dm, m->vocab, logits);
  kv->len = pos + 1;
  free(sc); free(x); free(xn); free(q); free(k); free(v); free(cat); free(att); free(fo); free(h); free(ha);
}

// Checker for the device tanhf: inputs start..start+count-1 (float bit patterns)
// where got[] differs bitwise from this host's libm tanhf (the function the
// reference's GELU calls).  NaN results compare equal to NaN.
typedef struct { uint32_t start, lo, hi; const float *got; long long bad; } TanhJob;

static void *tanhf_worker(void *arg) {
  TanhJob *j = (TanhJob*)arg;
  long long bad = 0;
  for (uint32_t i = j->lo; i < j->hi; i++) {
    const uint32_t b = j->start + i;
    float x; memcpy(&x, &b, 4);
    const float r = tanhf(x), g = j->got[i];
    uint32_t rb, gb; memcpy(&rb, &r, 4); memcpy(&gb, &g, 4);
    if (rb != gb && !(isnan(r) && isnan(g))) bad++;
  }
  j->bad = bad;
  return NULL;
}

long long or_tanhf_mismatches(uint32_t start, uint32_t count, const float *got) {
  enum { NT = 16 };
  pthread_t th[NT];
  TanhJob jobs[NT];
  const uint32_t per = (count + NT - 1) / NT;
  for (int t = 0; t < NT; t++) {
    uint32_t lo = (uint32_t)t * per, hi = lo + per;
    if (lo > count) lo = count;
    if (hi > count) hi = count;
    jobs[t] = (TanhJob){start, lo, hi, got, 0};
    pthread_create(&th[t], NULL, tanhf_worker, &jobs[t]);
  }
  long long bad = 0;
  for (int t = 0; t < NT; t++) { pthread_join(th[t], NULL); bad += jobs[t].bad; }
  return bad;
}
