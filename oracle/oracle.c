// oracle.c - CPU restatement of the reference's int8 LLaMA decode path.
// TEST INFRASTRUCTURE ONLY (see oracle.h).  Build as ISO C11 (-std=c11): the
// reference relies on that mode's "no floating-point contraction" default.
#define _POSIX_C_SOURCE 200809L
#include "oracle.h"
#include "synth.h"

#include <math.h>
#include <pthread.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <unistd.h>

// ---------------------------------------------------------------------------
// Fork-join pool.  Same decomposition as matrix.c:78-84,152-168: [0,total) is
// cut into n chunks of ceil(total/n); the caller runs the last chunk.  Only the
// timing depends on it: every output column is produced by one thread.
// ---------------------------------------------------------------------------
#define OR_MAX_THREADS 64
#define OR_MM_THRESHOLD (1L << 19)   // matrix.c:34

typedef void (*or_range_fn)(int lo, int hi, void *ctx);

static int P_n = 0, P_started = 0, P_gen = 0, P_left = 0, P_total = 0;
static or_range_fn P_fn;
static void *P_ctx;
static pthread_mutex_t P_mtx = PTHREAD_MUTEX_INITIALIZER;
static pthread_cond_t P_work = PTHREAD_COND_INITIALIZER, P_done = PTHREAD_COND_INITIALIZER;
static pthread_t P_th[OR_MAX_THREADS];
static int P_id[OR_MAX_THREADS];
static int P_req = 0;

static void chunk(int total, int idx, int n, int *lo, int *hi) {
  int per = (total + n - 1) / n;
  int l = idx * per, h = l + per;
  if (l > total) l = total;
  if (h > total) h = total;
  *lo = l; *hi = h;
}

static void *pool_main(void *arg) {
  const int id = *(int*)arg;
  int seen = 0;
  pthread_mutex_lock(&P_mtx);
  for (;;) {
    while (P_gen == seen) pthread_cond_wait(&P_work, &P_mtx);
    seen = P_gen;
    or_range_fn fn = P_fn; void *ctx = P_ctx; int total = P_total, n = P_n;
    pthread_mutex_unlock(&P_mtx);
    int lo, hi; chunk(total, id, n, &lo, &hi);
    if (lo < hi) fn(lo, hi, ctx);
    pthread_mutex_lock(&P_mtx);
    if (--P_left == 0) pthread_cond_signal(&P_done);
  }
  return NULL;
}

void or_set_threads(int n) {
  if (P_started) return;              // fixed once the pool runs
  P_req = n;
}

static void pool_start(void) {
  if (P_started) return;
  int n = P_req;
  if (n <= 0) {
    const char *env = getenv("TF_THREADS");
    if (env && atoi(env) > 0) n = atoi(env);
    else { long c = sysconf(_SC_NPROCESSORS_ONLN); n = c > 0 ? (int)c : 4; }
  }
  if (n > OR_MAX_THREADS) n = OR_MAX_THREADS;
  if (n < 1) n = 1;
  P_n = n;
  for (int i = 0; i < n - 1; i++) {
    P_id[i] = i;
    pthread_create(&P_th[i], NULL, pool_main, &P_id[i]);
    pthread_detach(P_th[i]);
  }
  P_started = 1;
}

int or_get_threads(void) { pool_start(); return P_n; }

static void parallel_for(int total, or_range_fn fn, void *ctx) {
  pool_start();
  if (P_n <= 1 || total < 2) { fn(0, total, ctx); return; }
  pthread_mutex_lock(&P_mtx);
  P_fn = fn; P_ctx = ctx; P_total = total; P_left = P_n - 1; P_gen++;
  pthread_cond_broadcast(&P_work);
  pthread_mutex_unlock(&P_mtx);
  int lo, hi; chunk(total, P_n - 1, P_n, &lo, &hi);
  if (lo < hi) fn(lo, hi, ctx);
  pthread_mutex_lock(&P_mtx);
  while (P_left > 0) pthread_cond_wait(&P_done, &P_mtx);
  pthread_mutex_unlock(&P_mtx);
}

// ---------------------------------------------------------------------------
// quant.c:10-27  per-column symmetric int8 quantization.
// ---------------------------------------------------------------------------
void or_quantize_int8_percol(const float *w, int rows, int cols, int8_t *q, float *scale) {
  for (int j = 0; j < cols; j++) {
    float mx = 0.0f;
    for (int i = 0; i < rows; i++) {
      float a = fabsf(w[(size_t)i * cols + j]);
      if (a > mx) mx = a;
    }
    float s = (mx > 0.0f) ? mx / 127.0f : 1.0f;
    scale[j] = s;
    float inv = 1.0f / s;
    for (int i = 0; i < rows; i++) {
      int v = (int)lrintf(w[(size_t)i * cols + j] * inv);
      if (v > 127) v = 127;
      if (v < -127) v = -127;
      q[(size_t)i * cols + j] = (int8_t)v;
    }
  }
}

// quant.c:29-33
void or_dequantize_int8_percol(const int8_t *q, const float *scale, int rows, int cols, float *w) {
  for (int i = 0; i < rows; i++)
    for (int j = 0; j < cols; j++)
      w[(size_t)i * cols + j] = (float)q[(size_t)i * cols + j] * scale[j];
}

// ---------------------------------------------------------------------------
// matrix.c:354-374  acc[j] = sum_k qa[k] * qw[k*N + j], threaded over columns.
// ---------------------------------------------------------------------------
typedef struct { const int8_t *qa, *qw; int K, N; int32_t *acc; } QAccJob;

static void qacc_range(int j0, int j1, void *ctx) {
  const QAccJob *t = (const QAccJob*)ctx;
  const int K = t->K, N = t->N;
  int32_t *acc = t->acc;
  for (int j = j0; j < j1; j++) acc[j] = 0;
  for (int k = 0; k < K; k++) {
    const int av = t->qa[k];
    const int8_t *qr = &t->qw[(size_t)k * N];
    for (int j = j0; j < j1; j++) acc[j] += av * (int)qr[j];
  }
}

void or_qacc_columns(const int8_t *qa, const int8_t *qw, int K, int N, int32_t *acc) {
  QAccJob t = {qa, qw, K, N, acc};
  if ((size_t)K * N < (size_t)OR_MM_THRESHOLD) { qacc_range(0, N, &t); return; }
  parallel_for(N, qacc_range, &t);
}

// ---------------------------------------------------------------------------
// quant.c:60-85  W8A8 qmatmul: per-row dynamic activation quantization, int32
// accumulation, then C = (as * ws[j]) * (float)acc[j].
// ---------------------------------------------------------------------------
void or_qmatmul_ex(const float *A, int M, const OrQT *W, float *C,
                   int8_t *qa_out, float *as_out, int32_t *acc_out) {
  const int K = W->rows, N = W->cols;
  int32_t *acc = (int32_t*)malloc((size_t)N * sizeof(int32_t));
  int8_t *qa = (int8_t*)malloc((size_t)K);
  const float *ws = W->scale;
  for (int m = 0; m < M; m++) {
    const float *a = &A[(size_t)m * K];
    float mx = 0.0f;
    for (int k = 0; k < K; k++) { float t = fabsf(a[k]); if (t > mx) mx = t; }
    float as = (mx > 0.0f) ? mx / 127.0f : 1.0f;
    float inv = 1.0f / as;
    for (int k = 0; k < K; k++) {
      int v = (int)lrintf(a[k] * inv);
      if (v > 127) v = 127;
      if (v < -127) v = -127;
      qa[k] = (int8_t)v;
    }
    or_qacc_columns(qa, W->q, K, N, acc);
    float *c = &C[(size_t)m * N];
    for (int j = 0; j < N; j++) c[j] = as * ws[j] * (float)acc[j];
    if (qa_out) memcpy(&qa_out[(size_t)m * K], qa, (size_t)K);
    if (as_out) as_out[m] = as;
    if (acc_out) memcpy(&acc_out[(size_t)m * N], acc, (size_t)N * sizeof(int32_t));
  }
  free(acc); free(qa);
}

void or_qmatmul(const float *A, int M, const OrQT *W, float *C) {
  or_qmatmul_ex(A, M, W, C, NULL, NULL, NULL);
}

// rmsnorm.c:7-21  y = (x * r) * gamma,  r = 1 / sqrtf(sum(x*x) * (1/cols) + eps).
void or_rmsnorm(const float *x, int rows, int cols, const float *gamma, float eps, float *y) {
  const float inv_n = 1.0f / (float)cols;
  for (int i = 0; i < rows; i++) {
    const float *xr = &x[(size_t)i * cols];
    float ms = 0.0f;
    for (int j = 0; j < cols; j++) ms += xr[j] * xr[j];
    ms *= inv_n;
    float r = 1.0f / sqrtf(ms + eps);
    for (int j = 0; j < cols; j++) y[(size_t)i * cols + j] = xr[j] * r * gamma[j];
  }
}

// rope.c:48-68  half-split rotary embedding, in place, row i at position pos0 + i.
void or_rope_heads_pos(float *x, int rows, int cols, int n_heads, float base, int pos0) {
  const int hd = cols / n_heads;
  const int h = hd / 2;
  for (int i = 0; i < rows; i++) {
    const int pos = pos0 + i;
    for (int head = 0; head < n_heads; head++) {
      float *xh = &x[(size_t)i * cols + (size_t)head * hd];
      for (int k = 0; k < h; k++) {
        float inv_freq = powf(base, -2.0f * (float)k / (float)hd);
        float ang = (float)pos * inv_freq;
        float c = cosf(ang), s = sinf(ang);
        float x1 = xh[k], x2 = xh[k + h];
        xh[k]     = x1 * c - x2 * s;
        xh[k + h] = x2 * c + x1 * s;
      }
    }
  }
}

// gqa.c:16-50  causal grouped-query attention over a full sequence.
// att: scratch of n floats (one row at a time; the reference keeps H*n*n).
void or_gqa_forward(const float *Q, const float *K, const float *V, int n, int H, int KVH,
                    int hd, float *att, float *O) {
  const int group = H / KVH, qd = H * hd, kd = KVH * hd;
  const float scale = 1.0f / sqrtf((float)hd);
  for (int h = 0; h < H; h++) {
    const int kv = h / group;
    const int qoff = h * hd, koff = kv * hd;
    for (int i = 0; i < n; i++) {
      float maxs = -INFINITY;
      for (int j = 0; j <= i; j++) {
        float dot = 0.0f;
        for (int d = 0; d < hd; d++)
          dot += Q[(size_t)i * qd + qoff + d] * K[(size_t)j * kd + koff + d];
        float s = dot * scale;
        att[j] = s;
        if (s > maxs) maxs = s;
      }
      float sum = 0.0f;
      for (int j = 0; j <= i; j++) { float e = expf(att[j] - maxs); att[j] = e; sum += e; }
      float inv = 1.0f / sum;
      for (int j = 0; j <= i; j++) att[j] *= inv;
      for (int d = 0; d < hd; d++) {
        float o = 0.0f;
        for (int j = 0; j <= i; j++) o += att[j] * V[(size_t)j * kd + koff + d];
        O[(size_t)i * qd + qoff + d] = o;
      }
    }
  }
}

// llama.c:554-576  decode attention of one query row at position pos against the
// cache rows 0..pos.  kc/vc: [max_seq][kvd] of one layer.  sc: pos+1 floats.
void or_attn_decode(const float *q, const float *kc, const float *vc, int kvd, int pos,
                    int n_heads, int n_kv, int hd, float *sc, float *o) {
  const int group = n_heads / n_kv;
  const float scale = 1.0f / sqrtf((float)hd);
  for (int head = 0; head < n_heads; head++) {
    const int kvh = head / group;
    const float *qh = &q[(size_t)head * hd];
    float maxs = -INFINITY;
    for (int jj = 0; jj <= pos; jj++) {
      const float *kj = &kc[(size_t)jj * kvd + (size_t)kvh * hd];
      float dot = 0.0f;
      for (int d = 0; d < hd; d++) dot += qh[d] * kj[d];
      float s = dot * scale;
      sc[jj] = s;
      if (s > maxs) maxs = s;
    }
    float sum = 0.0f;
    for (int jj = 0; jj <= pos; jj++) { float e = expf(sc[jj] - maxs); sc[jj] = e; sum += e; }
    float inv = 1.0f / sum;
    float *oh = &o[(size_t)head * hd];
    for (int d = 0; d < hd; d++) oh[d] = 0.0f;
    for (int jj = 0; jj <= pos; jj++) {
      float w = sc[jj] * inv;
      const float *vj = &vc[(size_t)jj * kvd + (size_t)kvh * hd];
      for (int d = 0; d < hd; d++) oh[d] += w * vj[d];
    }
  }
}

// sampler.c:8-21  first index of the maximum.
int or_argmax(const float *r, int n) {
  int best = 0;
  float best_val = r[0];
  for (int j = 1; j < n; j++)
    if (r[j] > best_val) { best_val = r[j]; best = j; }
  return best;
}

// sampler.c:24-45: xorshift64 state, seed 0 replaced by a fixed odd constant;
// a draw is the top 53 bits scaled to [0, 1) in double, narrowed to float.
uint64_t or_rng_create(uint64_t seed) { return seed ? seed : 0x9E3779B97F4A7C15ULL; }

float or_rng_uniform(uint64_t *state) {
  uint64_t x = *state;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  *state = x;
  return (float)((double)(x >> 11) * (1.0 / 9007199254740992.0));
}

typedef struct { float p; int idx; } OrProb;

// Probability descending, then index ascending: the order a stable sort by
// probability leaves the index-ordered array in (sampler.c:82 sorts with
// glibc's qsort, a merge sort for arrays of this size, which is stable).
static int or_prob_cmp(const void *a, const void *b) {
  const OrProb *x = (const OrProb*)a, *y = (const OrProb*)b;
  if (x->p != y->p) return x->p < y->p ? 1 : -1;
  return (x->idx > y->idx) - (x->idx < y->idx);
}

// sampler.c:54-143
int or_sample_token(const float *l, int V, float temperature, int top_k, float top_p, uint64_t *state) {
  if (temperature <= 0.0f) return or_argmax(l, V);
  float max_l = l[0];
  for (int j = 1; j < V; j++) if (l[j] > max_l) max_l = l[j];
  OrProb *pi = (OrProb*)malloc((size_t)V * sizeof(OrProb));
  if (!pi) abort();
  float sum = 0.0f;
  for (int j = 0; j < V; j++) {
    const float e = expf((l[j] - max_l) / temperature);
    pi[j].p = e;
    pi[j].idx = j;
    sum += e;
  }
  for (int j = 0; j < V; j++) pi[j].p /= sum;
  qsort(pi, (size_t)V, sizeof(OrProb), or_prob_cmp);
  int keep = V;
  if (top_k > 0 && top_k < keep) keep = top_k;
  if (top_p > 0.0f && top_p < 1.0f) {
    float cum = 0.0f;
    int kp = 0;
    for (int i = 0; i < keep; i++) {
      cum += pi[i].p;
      kp++;
      if (cum >= top_p) break;
    }
    keep = kp;
  }
  if (keep < 1) keep = 1;
  float z = 0.0f;
  for (int i = 0; i < keep; i++) z += pi[i].p;
  const float u = or_rng_uniform(state) * z;
  int chosen = pi[keep - 1].idx;
  float acc = 0.0f;
  for (int i = 0; i < keep; i++) {
    acc += pi[i].p;
    if (u <= acc) { chosen = pi[i].idx; break; }
  }
  free(pi);
  return chosen;
}

// ---------------------------------------------------------------------------
// Model construction.
// ---------------------------------------------------------------------------
static int qt_alloc(OrQT *t, int rows, int cols) {
  t->rows = rows; t->cols = cols;
  t->q = (int8_t*)malloc((size_t)rows * cols);
  t->scale = (float*)malloc((size_t)cols * sizeof(float));
  return (t->q && t->scale) ? 0 : 1;
}

static void qt_free(OrQT *t) { free(t->q); free(t->scale); t->q = NULL; t->scale = NULL; }

static float *fvec(int n, float v) {
  float *p = (float*)malloc((size_t)n * sizeof(float));
  if (p) for (int i = 0; i < n; i++) p[i] = v;
  return p;
}

int or_model_alloc(OrModel *m, const int32_t cfg[8], float rope_base, float eps) {
  memset(m, 0, sizeof *m);
  m->vocab = cfg[0]; m->d_model = cfg[1]; m->n_layers = cfg[2]; m->n_heads = cfg[3];
  m->n_kv = cfg[4]; m->head_dim = cfg[5]; m->d_ff = cfg[6]; m->max_seq = cfg[7];
  m->rope_base = rope_base; m->eps = eps;
  const int dm = m->d_model, qd = m->n_heads * m->head_dim, kvd = m->n_kv * m->head_dim;
  int bad = qt_alloc(&m->wte, m->vocab, dm);
  m->blocks = (OrBlock*)calloc((size_t)m->n_layers, sizeof(OrBlock));
  if (!m->blocks) return 1;
  for (int l = 0; l < m->n_layers; l++) {
    OrBlock *b = &m->blocks[l];
    b->attn_norm = fvec(dm, 1.0f); b->ffn_norm = fvec(dm, 1.0f);
    b->b_q = fvec(qd, 0.0f); b->b_k = fvec(kvd, 0.0f); b->b_v = fvec(kvd, 0.0f);
    bad |= qt_alloc(&b->Wq, dm, qd) | qt_alloc(&b->Wk, dm, kvd) | qt_alloc(&b->Wv, dm, kvd);
    bad |= qt_alloc(&b->Wo, qd, dm) | qt_alloc(&b->Wgate, dm, m->d_ff);
    bad |= qt_alloc(&b->Wup, dm, m->d_ff) | qt_alloc(&b->Wdown, m->d_ff, dm);
    if (!b->attn_norm || !b->ffn_norm || !b->b_q || !b->b_k || !b->b_v) bad = 1;
  }
  m->final_norm = fvec(dm, 1.0f);
  bad |= qt_alloc(&m->lm_head, dm, m->vocab);
  return bad || !m->final_norm;
}

void or_model_free(OrModel *m) {
  qt_free(&m->wte);
  for (int l = 0; l < m->n_layers && m->blocks; l++) {
    OrBlock *b = &m->blocks[l];
    free(b->attn_norm); free(b->ffn_norm); free(b->b_q); free(b->b_k); free(b->b_v);
    qt_free(&b->Wq); qt_free(&b->Wk); qt_free(&b->Wv); qt_free(&b->Wo);
    qt_free(&b->Wgate); qt_free(&b->Wup); qt_free(&b->Wdown);
  }
  free(m->blocks); m->blocks = NULL;
  free(m->final_norm); m->final_norm = NULL;
  qt_free(&m->lm_head);
}

static void synth_qt(OrQT *t, float *buf, uint64_t seed, uint64_t tid) {
  syn_fill(buf, (size_t)t->rows * t->cols, seed, tid, 0.02);
  or_quantize_int8_percol(buf, t->rows, t->cols, t->q, t->scale);
}

int or_model_synth(OrModel *m, const int32_t cfg[8], float rope_base, float eps,
                   uint64_t seed, int tied) {
  if (or_model_alloc(m, cfg, rope_base, eps)) return 1;
  const int dm = m->d_model, L = m->n_layers;
  size_t biggest = (size_t)m->vocab * dm;
  size_t ff = (size_t)dm * m->d_ff;
  if (ff > biggest) biggest = ff;
  size_t qo = (size_t)dm * m->n_heads * m->head_dim;     // Wq and Wo when n_heads*head_dim > d_model
  if (qo > biggest) biggest = qo;
  float *buf = (float*)malloc(biggest * sizeof(float));
  if (!buf) return 1;
  synth_qt(&m->wte, buf, seed, 0);
  for (int l = 0; l < L; l++) {
    OrBlock *b = &m->blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    synth_qt(&b->Wq, buf, seed, t0 + 1);
    synth_qt(&b->Wk, buf, seed, t0 + 2);
    synth_qt(&b->Wv, buf, seed, t0 + 3);
    synth_qt(&b->Wo, buf, seed, t0 + 7);
    synth_qt(&b->Wgate, buf, seed, t0 + 9);
    synth_qt(&b->Wup, buf, seed, t0 + 10);
    synth_qt(&b->Wdown, buf, seed, t0 + 11);
  }
  const uint64_t tid_head = 2 + 12 * (uint64_t)L;
  if (tied) {
    // lm_head[k][v] = wte fp32 value at (v, k); regenerate wte then transpose.
    float *w = (float*)malloc((size_t)m->vocab * dm * sizeof(float));
    if (!w) { free(buf); return 1; }
    syn_fill(w, (size_t)m->vocab * dm, seed, 0, 0.02);
    for (int v = 0; v < m->vocab; v++)
      for (int k = 0; k < dm; k++) buf[(size_t)k * m->vocab + v] = w[(size_t)v * dm + k];
    free(w);
    or_quantize_int8_percol(buf, dm, m->vocab, m->lm_head.q, m->lm_head.scale);
  } else {
    synth_qt(&m->lm_head, buf, seed, tid_head);
  }
  free(buf);
  return 0;
}

// llama.c:490-511 (q_llama_quantize_from): the int8 model of an fp32 model:
// every matrix quantized per column (quant.c:10-27), norms and biases copied.
int or_model_quantize_from(OrModel *m, const OrFModel *f) {
  const int32_t cfg[8] = {f->vocab, f->d_model, f->n_layers, f->n_heads, f->n_kv, f->head_dim, f->d_ff, f->max_seq};
  if (or_model_alloc(m, cfg, f->rope_base, f->eps)) return 1;
  const int dm = m->d_model, qd = m->n_heads * m->head_dim, kvd = m->n_kv * m->head_dim;
  or_quantize_int8_percol(f->wte, m->vocab, dm, m->wte.q, m->wte.scale);
  for (int l = 0; l < m->n_layers; l++) {
    const OrFBlock *a = &f->blocks[l];
    OrBlock *b = &m->blocks[l];
    memcpy(b->attn_norm, a->attn_norm, (size_t)dm * sizeof(float));
    memcpy(b->ffn_norm, a->ffn_norm, (size_t)dm * sizeof(float));
    memcpy(b->b_q, a->b_q, (size_t)qd * sizeof(float));
    memcpy(b->b_k, a->b_k, (size_t)kvd * sizeof(float));
    memcpy(b->b_v, a->b_v, (size_t)kvd * sizeof(float));
    or_quantize_int8_percol(a->Wq, dm, qd, b->Wq.q, b->Wq.scale);
    or_quantize_int8_percol(a->Wk, dm, kvd, b->Wk.q, b->Wk.scale);
    or_quantize_int8_percol(a->Wv, dm, kvd, b->Wv.q, b->Wv.scale);
    or_quantize_int8_percol(a->Wo, qd, dm, b->Wo.q, b->Wo.scale);
    or_quantize_int8_percol(a->Wgate, dm, m->d_ff, b->Wgate.q, b->Wgate.scale);
    or_quantize_int8_percol(a->Wup, dm, m->d_ff, b->Wup.q, b->Wup.scale);
    or_quantize_int8_percol(a->Wdown, m->d_ff, dm, b->Wdown.q, b->Wdown.scale);
  }
  memcpy(m->final_norm, f->final_norm, (size_t)dm * sizeof(float));
  or_quantize_int8_percol(f->lm_head, dm, m->vocab, m->lm_head.q, m->lm_head.scale);
  return 0;
}

static uint64_t qt_hash(const OrQT *t, uint64_t salt) {
  return syn_hash_i8(t->q, (size_t)t->rows * t->cols, salt) * 3 +
         syn_hash_f32(t->scale, (size_t)t->cols, salt ^ 0x5CA1E5ULL);
}

uint64_t or_model_hash(const OrModel *m) {
  uint64_t h = qt_hash(&m->wte, 0);
  for (int l = 0; l < m->n_layers; l++) {
    const OrBlock *b = &m->blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    h = h * 31 + qt_hash(&b->Wq, t0 + 1);
    h = h * 31 + qt_hash(&b->Wk, t0 + 2);
    h = h * 31 + qt_hash(&b->Wv, t0 + 3);
    h = h * 31 + qt_hash(&b->Wo, t0 + 7);
    h = h * 31 + qt_hash(&b->Wgate, t0 + 9);
    h = h * 31 + qt_hash(&b->Wup, t0 + 10);
    h = h * 31 + qt_hash(&b->Wdown, t0 + 11);
  }
  return h * 31 + qt_hash(&m->lm_head, 2 + 12 * (uint64_t)m->n_layers);
}

// llama.c:513-526
int or_kv_create(OrKV *kv, const OrModel *m) {
  kv->n_layers = m->n_layers; kv->max_seq = m->max_seq;
  kv->kv_dim = m->n_kv * m->head_dim; kv->len = 0;
  size_t n = (size_t)m->n_layers * m->max_seq * kv->kv_dim;
  kv->k = (float*)malloc(n * sizeof(float));
  kv->v = (float*)malloc(n * sizeof(float));
  return (kv->k && kv->v) ? 0 : 1;
}

void or_kv_free(OrKV *kv) { free(kv->k); free(kv->v); kv->k = kv->v = NULL; }

// llama.c:528-600  one decode step at position kv->len.
void or_decode_step(const OrModel *m, OrKV *kv, int token, float *logits) {
  const int dm = m->d_model, hd = m->head_dim, dff = m->d_ff;
  const int qd = m->n_heads * hd, kvd = m->n_kv * hd;
  const int pos = kv->len;
  float *x = (float*)calloc((size_t)dm, sizeof(float));
  float *xn = (float*)calloc((size_t)dm, sizeof(float));
  float *q = (float*)calloc((size_t)qd, sizeof(float));
  float *k = (float*)calloc((size_t)kvd, sizeof(float));
  float *v = (float*)calloc((size_t)kvd, sizeof(float));
  float *o = (float*)calloc((size_t)qd, sizeof(float));
  float *ao = (float*)calloc((size_t)dm, sizeof(float));
  float *hn = (float*)calloc((size_t)dm, sizeof(float));
  float *f = (float*)calloc((size_t)dm, sizeof(float));
  float *g = (float*)calloc((size_t)dff, sizeof(float));
  float *u = (float*)calloc((size_t)dff, sizeof(float));
  float *sc = (float*)malloc((size_t)(pos + 1) * sizeof(float));

  { const int8_t *qr = &m->wte.q[(size_t)token * dm]; const float *sq = m->wte.scale;
    for (int j = 0; j < dm; j++) x[j] = (float)qr[j] * sq[j]; }

  for (int l = 0; l < m->n_layers; l++) {
    const OrBlock *b = &m->blocks[l];
    float *kc = &kv->k[(size_t)l * kv->max_seq * kvd];
    float *vc = &kv->v[(size_t)l * kv->max_seq * kvd];
    or_rmsnorm(x, 1, dm, b->attn_norm, m->eps, xn);
    or_qmatmul(xn, 1, &b->Wq, q); for (int j = 0; j < qd; j++) q[j] = q[j] + b->b_q[j];
    or_qmatmul(xn, 1, &b->Wk, k); for (int j = 0; j < kvd; j++) k[j] = k[j] + b->b_k[j];
    or_qmatmul(xn, 1, &b->Wv, v); for (int j = 0; j < kvd; j++) v[j] = v[j] + b->b_v[j];
    or_rope_heads_pos(q, 1, qd, m->n_heads, m->rope_base, pos);
    or_rope_heads_pos(k, 1, kvd, m->n_kv, m->rope_base, pos);
    memcpy(&kc[(size_t)pos * kvd], k, (size_t)kvd * sizeof(float));
    memcpy(&vc[(size_t)pos * kvd], v, (size_t)kvd * sizeof(float));
    or_attn_decode(q, kc, vc, kvd, pos, m->n_heads, m->n_kv, hd, sc, o);
    or_qmatmul(o, 1, &b->Wo, ao);
    for (int j = 0; j < dm; j++) x[j] += ao[j];
    or_rmsnorm(x, 1, dm, b->ffn_norm, m->eps, hn);
    or_qmatmul(hn, 1, &b->Wgate, g);
    or_qmatmul(hn, 1, &b->Wup, u);
    for (int j = 0; j < dff; j++) {
      float z = g[j];
      float s = 1.0f / (1.0f + expf(-z));
      g[j] = (z * s) * u[j];
    }
    or_qmatmul(g, 1, &b->Wdown, f);
    for (int j = 0; j < dm; j++) x[j] += f[j];
  }
  or_rmsnorm(x, 1, dm, m->final_norm, m->eps, hn);
  or_qmatmul(hn, 1, &m->lm_head, logits);
  kv->len = pos + 1;

  free(sc); free(x); free(xn); free(q); free(k); free(v); free(o); free(ao);
  free(hn); free(f); free(g); free(u);
}

// ---------------------------------------------------------------------------
// fp32 (LLMA) path: llama.c:296-362 with the f32 matmul of matrix.c:178-190.
// ---------------------------------------------------------------------------
// One row of matrix.c:178-190: c[j] = ((0 + a_0*W_0j) + a_1*W_1j) + ..., k outer,
// j inner (every c[j] sums in k order; products rounded before the add).
void or_matmul_row(const float *a, const float *W, int K, int N, float *c) {
  for (int j = 0; j < N; j++) c[j] = 0.0f;
  for (int k = 0; k < K; k++) {
    const float ak = a[k];
    const float *Wk = &W[(size_t)k * N];
    for (int j = 0; j < N; j++) c[j] += ak * Wk[j];
  }
}

int or_fmodel_synth(OrFModel *m, const int32_t cfg[8], float rope_base, float eps, uint64_t seed, int tied) {
  memset(m, 0, sizeof *m);
  m->vocab = cfg[0]; m->d_model = cfg[1]; m->n_layers = cfg[2]; m->n_heads = cfg[3]; m->n_kv = cfg[4];
  m->head_dim = cfg[5]; m->d_ff = cfg[6]; m->max_seq = cfg[7]; m->rope_base = rope_base; m->eps = eps;
  const size_t dm = (size_t)m->d_model, qd = (size_t)m->n_heads * m->head_dim, kvd = (size_t)m->n_kv * m->head_dim;
  const size_t ff = (size_t)m->d_ff, V = (size_t)m->vocab;
  const int L = m->n_layers;
  m->blocks = (OrFBlock*)calloc((size_t)L, sizeof(OrFBlock));
  m->wte = (float*)malloc(V * dm * 4);
  m->lm_head = (float*)malloc(V * dm * 4);
  m->final_norm = (float*)malloc(dm * 4);
  if (!m->blocks || !m->wte || !m->lm_head || !m->final_norm) return 1;
  syn_fill(m->wte, V * dm, seed, 0, 0.02);
  for (size_t j = 0; j < dm; j++) m->final_norm[j] = 1.0f;
  for (int l = 0; l < L; l++) {
    OrFBlock *b = &m->blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    b->attn_norm = (float*)malloc(dm * 4); b->ffn_norm = (float*)malloc(dm * 4);
    b->b_q = (float*)calloc(qd, 4); b->b_k = (float*)calloc(kvd, 4); b->b_v = (float*)calloc(kvd, 4);
    b->Wq = (float*)malloc(dm * qd * 4); b->Wk = (float*)malloc(dm * kvd * 4); b->Wv = (float*)malloc(dm * kvd * 4);
    b->Wo = (float*)malloc(qd * dm * 4);
    b->Wgate = (float*)malloc(dm * ff * 4); b->Wup = (float*)malloc(dm * ff * 4); b->Wdown = (float*)malloc(ff * dm * 4);
    if (!b->attn_norm || !b->ffn_norm || !b->b_q || !b->b_k || !b->b_v || !b->Wq || !b->Wk || !b->Wv || !b->Wo ||
        !b->Wgate || !b->Wup || !b->Wdown) return 1;
    for (size_t j = 0; j < dm; j++) { b->attn_norm[j] = 1.0f; b->ffn_norm[j] = 1.0f; }
    syn_fill(b->Wq, dm * qd, seed, t0 + 1, 0.02);
    syn_fill(b->Wk, dm * kvd, seed, t0 + 2, 0.02);
    syn_fill(b->Wv, dm * kvd, seed, t0 + 3, 0.02);
    syn_fill(b->Wo, qd * dm, seed, t0 + 7, 0.02);
    syn_fill(b->Wgate, dm * ff, seed, t0 + 9, 0.02);
    syn_fill(b->Wup, dm * ff, seed, t0 + 10, 0.02);
    syn_fill(b->Wdown, ff * dm, seed, t0 + 11, 0.02);
  }
  if (tied) {      // lm_head[k][v] = wte[v][k]
    for (size_t v = 0; v < V; v++)
      for (size_t k = 0; k < dm; k++) m->lm_head[k * V + v] = m->wte[v * dm + k];
  } else {
    syn_fill(m->lm_head, dm * V, seed, 2 + 12 * (uint64_t)L, 0.02);
  }
  return 0;
}

void or_fmodel_free(OrFModel *m) {
  if (m->blocks) {
    for (int l = 0; l < m->n_layers; l++) {
      OrFBlock *b = &m->blocks[l];
      free(b->attn_norm); free(b->ffn_norm); free(b->b_q); free(b->b_k); free(b->b_v);
      free(b->Wq); free(b->Wk); free(b->Wv); free(b->Wo); free(b->Wgate); free(b->Wup); free(b->Wdown);
    }
  }
  free(m->blocks); free(m->wte); free(m->lm_head); free(m->final_norm);
  memset(m, 0, sizeof *m);
}

int or_fkv_create(OrKV *kv, const OrFModel *m) {
  kv->n_layers = m->n_layers; kv->max_seq = m->max_seq;
  kv->kv_dim = m->n_kv * m->head_dim; kv->len = 0;
  size_t n = (size_t)m->n_layers * m->max_seq * kv->kv_dim;
  kv->k = (float*)malloc(n * sizeof(float));
  kv->v = (float*)malloc(n * sizeof(float));
  return (kv->k && kv->v) ? 0 : 1;
}

// llama.c:296-362 (swiglu.c:31-41 for the feed-forward)
void or_f32_decode_step(const OrFModel *m, OrKV *kv, int token, float *logits) {
  const int dm = m->d_model, hd = m->head_dim, dff = m->d_ff;
  const int qd = m->n_heads * hd, kvd = m->n_kv * hd;
  const int pos = kv->len;
  float *x = (float*)calloc((size_t)dm, 4), *xn = (float*)calloc((size_t)dm, 4);
  float *q = (float*)calloc((size_t)qd, 4), *k = (float*)calloc((size_t)kvd, 4), *v = (float*)calloc((size_t)kvd, 4);
  float *o = (float*)calloc((size_t)qd, 4), *ao = (float*)calloc((size_t)dm, 4), *hn = (float*)calloc((size_t)dm, 4);
  float *f = (float*)calloc((size_t)dm, 4), *g = (float*)calloc((size_t)dff, 4), *u = (float*)calloc((size_t)dff, 4);
  float *sc = (float*)malloc((size_t)(pos + 1) * 4);
  for (int j = 0; j < dm; j++) x[j] = m->wte[(size_t)token * dm + j];
  for (int l = 0; l < m->n_layers; l++) {
    const OrFBlock *b = &m->blocks[l];
    float *kc = &kv->k[(size_t)l * kv->max_seq * kvd];
    float *vc = &kv->v[(size_t)l * kv->max_seq * kvd];
    or_rmsnorm(x, 1, dm, b->attn_norm, m->eps, xn);
    or_matmul_row(xn, b->Wq, dm, qd, q); for (int j = 0; j < qd; j++) q[j] = q[j] + b->b_q[j];
    or_matmul_row(xn, b->Wk, dm, kvd, k); for (int j = 0; j < kvd; j++) k[j] = k[j] + b->b_k[j];
    or_matmul_row(xn, b->Wv, dm, kvd, v); for (int j = 0; j < kvd; j++) v[j] = v[j] + b->b_v[j];
    or_rope_heads_pos(q, 1, qd, m->n_heads, m->rope_base, pos);
    or_rope_heads_pos(k, 1, kvd, m->n_kv, m->rope_base, pos);
    memcpy(&kc[(size_t)pos * kvd], k, (size_t)kvd * 4);
    memcpy(&vc[(size_t)pos * kvd], v, (size_t)kvd * 4);
    or_attn_decode(q, kc, vc, kvd, pos, m->n_heads, m->n_kv, hd, sc, o);
    or_matmul_row(o, b->Wo, qd, dm, ao);
    for (int j = 0; j < dm; j++) x[j] += ao[j];
    or_rmsnorm(x, 1, dm, b->ffn_norm, m->eps, hn);
    or_matmul_row(hn, b->Wgate, dm, dff, g);
    or_matmul_row(hn, b->Wup, dm, dff, u);
    for (int j = 0; j < dff; j++) {
      const float z = g[j];
      const float s = 1.0f / (1.0f + expf(-z));
      g[j] = (z * s) * u[j];
    }
    or_matmul_row(g, b->Wdown, dff, dm, f);
    for (int j = 0; j < dm; j++) x[j] += f[j];
  }
  or_rmsnorm(x, 1, dm, m->final_norm, m->eps, hn);
  or_matmul_row(hn, m->lm_head, dm, m->vocab, logits);
  kv->len = pos + 1;
  free(sc); free(x); free(xn); free(q); free(k); free(v); free(o); free(ao); free(hn); free(f); free(g); free(u);
}

// ---------------------------------------------------------------------------
// Checker for the device expf: counts inputs start..start+count-1 (as float bit
// patterns) where got[] differs bitwise from this host's libm expf (the function
// llama.c:567,585 call).  NaN results compare equal to NaN.
// ---------------------------------------------------------------------------
typedef struct { uint32_t start; uint32_t lo, hi; const float *got; long long bad; } ExpJob;

static void *expf_worker(void *arg) {
  ExpJob *j = (ExpJob*)arg;
  long long bad = 0;
  for (uint32_t i = j->lo; i < j->hi; i++) {
    uint32_t b = j->start + i;
    float x; memcpy(&x, &b, 4);
    float r = expf(x), g = j->got[i];
    uint32_t rb, gb; memcpy(&rb, &r, 4); memcpy(&gb, &g, 4);
    if (rb != gb && !(isnan(r) && isnan(g))) bad++;
  }
  j->bad = bad;
  return NULL;
}

long long or_expf_mismatches(uint32_t start, uint32_t count, const float *got) {
  enum { NT = 16 };
  pthread_t th[NT];
  ExpJob jobs[NT];
  uint32_t per = (count + NT - 1) / NT;
  for (int t = 0; t < NT; t++) {
    uint32_t lo = (uint32_t)t * per, hi = lo + per;
    if (lo > count) lo = count;
    if (hi > count) hi = count;
    jobs[t] = (ExpJob){start, lo, hi, got, 0};
    pthread_create(&th[t], NULL, expf_worker, &jobs[t]);
  }
  long long bad = 0;
  for (int t = 0; t < NT; t++) { pthread_join(th[t], NULL); bad += jobs[t].bad; }
  return bad;
}
