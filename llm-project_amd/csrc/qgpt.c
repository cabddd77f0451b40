// qgpt.c - C11 host side of the GPT-2 (GPTC) KV-cache decode on the GPU: the
// reference's model.h / checkpoint.h entry points for that path (model.c:437-520,
// checkpoint.c:62-174) with the same names, argument meaning and errors.
//
// The model stays the reference's host GPT (fp32 tensors in host memory, as
// gpt_load fills them).  Each KVCache takes a device copy of the weights when it
// is created (and again when a different model is passed to gpt_decode_step),
// holds the per-layer caches [head][max_seq][head_dim] in HBM, and replays the
// token's launches as one HIP graph.  Every float operation is the reference's,
// in its order, so the logits are the reference's bit for bit.
#define _POSIX_C_SOURCE 200809L
#include "qgpt.h"
#include "qllama.h"
#include "qhip.h"

#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define GPTC_MAGIC   0x43545047u   // checkpoint.c:9 ('GPTC')
#define GPTC_VERSION 2u            // checkpoint.c:10
#define GPT_LN_EPS   1e-5f         // model.c:15

static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

// ---------------------------------------------------------------------------
// Host model: allocation, the GPTC order, load / save / free
// ---------------------------------------------------------------------------
static Tensor host_tensor(int rows, int cols) {           // zero-filled, like tensor_create
  Tensor t;
  memset(&t, 0, sizeof t);
  t.ndim = cols > 0 ? 2 : 1;
  t.size = (size_t)rows * (size_t)(cols > 0 ? cols : 1);
  t.shape = (int*)malloc(2 * sizeof(int));
  t.data = (float*)calloc(t.size, sizeof(float));
  if (!t.shape || !t.data) { fprintf(stderr, "Error: out of memory (GPT tensor)\n"); exit(EXIT_FAILURE); }
  t.shape[0] = rows;
  t.shape[1] = cols;
  return t;
}

static void host_tensor_free(Tensor *t) {
  free(t->data); free(t->grad); free(t->shape);
  t->data = NULL; t->grad = NULL; t->shape = NULL;
}

// The tensors in the GPTC order (checkpoint.c:17-44): wte, wpe, 16 per layer,
// the final LayerNorm, lm_head.  list holds 5 + 16 * n_layers entries.
static int gpt_list(const GPT *m, Tensor **list) {
  int n = 0;
  list[n++] = (Tensor*)&m->wte;
  list[n++] = (Tensor*)&m->wpe;
  for (int l = 0; l < m->n_layers; l++) {
    BlockWeights *b = &m->blocks[l];
    Tensor *blk[16] = {&b->W_q, &b->W_k, &b->W_v, &b->W_o, &b->b_q, &b->b_k, &b->b_v, &b->b_o,
                       &b->gamma1, &b->beta1, &b->gamma2, &b->beta2, &b->ff_W1, &b->ff_b1, &b->ff_W2, &b->ff_b2};
    for (int i = 0; i < 16; i++) list[n++] = blk[i];
  }
  list[n++] = (Tensor*)&m->ln_f_gamma;
  list[n++] = (Tensor*)&m->ln_f_beta;
  list[n++] = (Tensor*)&m->lm_head;
  return n;
}

// checkpoint.c:117-127: positive bounded dims, whole heads, element counts within int
static int gpt_cfg_valid(const int32_t *c) {
  for (int i = 0; i < 6; i++)
    if (c[i] <= 0 || c[i] > 1000000) return 0;
  const long long vocab = c[0], dm = c[1], heads = c[2], ff = c[4];
  if (dm % heads != 0) return 0;
  if (vocab * dm > INT_MAX || dm * ff > INT_MAX) return 0;
  return 1;
}

// A zero-filled host model of the given config (vocab, d_model, heads, layers, d_ff, max_seq).
static int gpt_alloc(GPT *m, const int32_t *c) {
  memset(m, 0, sizeof *m);
  m->vocab_size = c[0]; m->d_model = c[1]; m->n_heads = c[2]; m->n_layers = c[3]; m->d_ff = c[4];
  m->max_seq_len = c[5];
  const int V = c[0], dm = c[1], ff = c[4], S = c[5];
  m->blocks = (BlockWeights*)calloc((size_t)m->n_layers, sizeof(BlockWeights));
  if (!m->blocks) return 1;
  m->wte = host_tensor(V, dm);
  m->wpe = host_tensor(S, dm);
  for (int l = 0; l < m->n_layers; l++) {
    BlockWeights *b = &m->blocks[l];
    b->W_q = host_tensor(dm, dm); b->W_k = host_tensor(dm, dm); b->W_v = host_tensor(dm, dm);
    b->W_o = host_tensor(dm, dm);
    b->b_q = host_tensor(dm, 0); b->b_k = host_tensor(dm, 0); b->b_v = host_tensor(dm, 0); b->b_o = host_tensor(dm, 0);
    b->gamma1 = host_tensor(dm, 0); b->beta1 = host_tensor(dm, 0);
    b->gamma2 = host_tensor(dm, 0); b->beta2 = host_tensor(dm, 0);
    b->ff_W1 = host_tensor(dm, ff); b->ff_b1 = host_tensor(ff, 0);
    b->ff_W2 = host_tensor(ff, dm); b->ff_b2 = host_tensor(dm, 0);
  }
  m->ln_f_gamma = host_tensor(dm, 0);
  m->ln_f_beta = host_tensor(dm, 0);
  m->lm_head = host_tensor(dm, V);
  return 0;
}

void gpt_free(GPT *m) {
  if (!m || !m->blocks) return;
  Tensor **list = (Tensor**)malloc(sizeof(Tensor*) * (size_t)(5 + 16 * m->n_layers));
  if (list) {
    const int n = gpt_list(m, list);
    for (int i = 0; i < n; i++) host_tensor_free(list[i]);
    free(list);
  }
  free(m->blocks);
  m->blocks = NULL;
}

int gpt_load(const char *path, GPT *out) {
  FILE *f = fopen(path, "rb");
  if (!f) { fprintf(stderr, "Error: cannot open '%s' for reading\n", path); return 1; }
  uint32_t header[2];
  int32_t cfg[6];
  if (fread(header, sizeof(uint32_t), 2, f) != 2 || fread(cfg, sizeof(int32_t), 6, f) != 6) {
    fprintf(stderr, "Error: '%s' is truncated (bad header)\n", path);
    fclose(f);
    return 1;
  }
  if (header[0] != GPTC_MAGIC || header[1] != GPTC_VERSION) {
    fprintf(stderr, "Error: '%s' is not a v%u GPTC checkpoint\n", path, GPTC_VERSION);
    fclose(f);
    return 1;
  }
  if (!gpt_cfg_valid(cfg)) {
    fprintf(stderr, "Error: '%s' has an invalid/unsupported config\n", path);
    fclose(f);
    return 1;
  }
  if (gpt_alloc(out, cfg)) { fclose(f); gpt_free(out); fprintf(stderr, "Error: out of memory loading '%s'\n", path); return 1; }
  Tensor **list = (Tensor**)malloc(sizeof(Tensor*) * (size_t)(5 + 16 * out->n_layers));
  int ok = list != NULL;
  const int n = ok ? gpt_list(out, list) : 0;
  for (int i = 0; i < n && ok; i++) ok = fread(list[i]->data, sizeof(float), list[i]->size, f) == list[i]->size;
  free(list);
  fclose(f);
  if (!ok) {
    fprintf(stderr, "Error: '%s' is truncated (bad weights)\n", path);
    gpt_free(out);
    return 1;
  }
  return 0;
}

// Moves the finished temporary file over dst (checkpoint.c:56-60: where rename
// cannot replace an existing file, remove it first).
static int replace_file(const char *tmp, const char *dst) {
  if (rename(tmp, dst) == 0) return 0;
  remove(dst);
  return rename(tmp, dst);
}

// checkpoint.c:62-103: the bytes go to path.tmp, which is flushed, closed and
// only then renamed over path, so a failed or interrupted save leaves an
// existing checkpoint at path untouched.
int gpt_save(const char *path, const GPT *m) {
  const size_t pl = strlen(path);
  char *tmp = (char*)malloc(pl + 5);
  if (!tmp) { fprintf(stderr, "Error: out of memory saving '%s'\n", path); return 1; }
  memcpy(tmp, path, pl);
  memcpy(tmp + pl, ".tmp", 5);
  FILE *f = fopen(tmp, "wb");
  if (!f) {
    fprintf(stderr, "Error: cannot open '%s' for writing\n", tmp);
    free(tmp);
    return 1;
  }
  const uint32_t header[2] = {GPTC_MAGIC, GPTC_VERSION};
  const int32_t cfg[6] = {m->vocab_size, m->d_model, m->n_heads, m->n_layers, m->d_ff, m->max_seq_len};
  int ok = fwrite(header, sizeof(uint32_t), 2, f) == 2 && fwrite(cfg, sizeof(int32_t), 6, f) == 6;
  Tensor **list = (Tensor**)malloc(sizeof(Tensor*) * (size_t)(5 + 16 * m->n_layers));
  ok = ok && list != NULL;
  const int n = ok ? gpt_list(m, list) : 0;
  for (int i = 0; i < n && ok; i++) ok = fwrite(list[i]->data, sizeof(float), list[i]->size, f) == list[i]->size;
  free(list);
  if (fflush(f) != 0) ok = 0;
  if (fclose(f) != 0) ok = 0;          // deferred write errors (a full disk) surface here
  if (ok) ok = replace_file(tmp, path) == 0;
  if (!ok) {
    remove(tmp);
    fprintf(stderr, "Error: failed while writing '%s'\n", path);
    free(tmp);
    return 1;
  }
  free(tmp);
  return 0;
}

// ---------------------------------------------------------------------------
// Device copy, per cache
// ---------------------------------------------------------------------------
typedef struct {
  const void *key[4];                     // wte, wpe, blocks, lm_head of the host model copied
  int vocab, dm, nh, hd, L, ff, max_seq;
  uint8_t *blob;
  float **wqkv, **bqkv, **wo, **bo, **g1, **be1, **g2, **be2, **w1, **bf1, **w2, **bf2;
  float *wte, *wpe, *lnf_g, *lnf_b, *head;
  float *x, *xn, *qkv, *o, *h, *logits, *scores;
  int *d_state, *d_in;
  float *kbase, *vbase;                   // [L][nh][max_seq][hd]
  int *h_stage;                           // pinned: position, end, token
  void *graph;
} GDev;

static void gdev_free(GDev *g) {
  if (!g) return;
  qhip_sync();
  if (g->graph) qhip_graph_destroy(g->graph);
  qhip_free(g->blob); qhip_free(g->kbase); qhip_free(g->vbase);
  qhip_host_free(g->h_stage);
  free(g->wqkv); free(g->bqkv); free(g->wo); free(g->bo); free(g->g1); free(g->be1); free(g->g2); free(g->be2);
  free(g->w1); free(g->bf1); free(g->w2); free(g->bf2);
  free(g);
}

static int gpt_supported(const GPT *m) {
  const int hd = m->d_model / m->n_heads;
  return hd % 2 == 0 && hd <= 512 && m->d_model <= 8192 && m->d_ff <= qhip_gemv_f32_max_k() &&
         m->max_seq_len <= 16384;
}

// Upload m's weights into g's buffers (the shapes already match).
static int gdev_upload(GDev *g, const GPT *m) {
  const size_t dm = (size_t)g->dm, ff = (size_t)g->ff, V = (size_t)g->vocab;
  size_t big = dm * 3 * dm;
  if (dm * ff > big) big = dm * ff;
  if (dm * V > big) big = dm * V;
  float *tmp = (float*)qhip_malloc(big * 4), *tmp2 = (float*)qhip_malloc(dm * dm * 4);
  int rc = !tmp || !tmp2 || qhip_upload_begin((size_t)32 << 20);
#define JOIN(src, col) (qhip_upload(tmp2, (src)->data, dm * dm * 4) || \
                        qhip_copy2d_d2d(tmp + (col), 3 * dm * 4, tmp2, dm * 4, dm * 4, dm))
  rc = rc || qhip_upload(g->wte, m->wte.data, V * dm * 4) ||
       qhip_upload(g->wpe, m->wpe.data, (size_t)g->max_seq * dm * 4) ||
       qhip_upload(g->lnf_g, m->ln_f_gamma.data, dm * 4) || qhip_upload(g->lnf_b, m->ln_f_beta.data, dm * 4) ||
       qhip_upload(tmp, m->lm_head.data, dm * V * 4) || qhip_to_panels_f32(tmp, (int)dm, (int)V, g->head);
  for (int l = 0; l < g->L && !rc; l++) {
    const BlockWeights *b = &m->blocks[l];
    rc = JOIN(&b->W_q, 0) || JOIN(&b->W_k, dm) || JOIN(&b->W_v, 2 * dm) ||
         qhip_to_panels_f32(tmp, (int)dm, (int)(3 * dm), g->wqkv[l]) ||
         qhip_upload(g->bqkv[l], b->b_q.data, dm * 4) || qhip_upload(g->bqkv[l] + dm, b->b_k.data, dm * 4) ||
         qhip_upload(g->bqkv[l] + 2 * dm, b->b_v.data, dm * 4) ||
         qhip_upload(tmp, b->W_o.data, dm * dm * 4) || qhip_to_panels_f32(tmp, (int)dm, (int)dm, g->wo[l]) ||
         qhip_upload(g->bo[l], b->b_o.data, dm * 4) ||
         qhip_upload(g->g1[l], b->gamma1.data, dm * 4) || qhip_upload(g->be1[l], b->beta1.data, dm * 4) ||
         qhip_upload(g->g2[l], b->gamma2.data, dm * 4) || qhip_upload(g->be2[l], b->beta2.data, dm * 4) ||
         qhip_upload(tmp, b->ff_W1.data, dm * ff * 4) || qhip_to_panels_f32(tmp, (int)dm, (int)ff, g->w1[l]) ||
         qhip_upload(g->bf1[l], b->ff_b1.data, ff * 4) ||
         qhip_upload(tmp, b->ff_W2.data, ff * dm * 4) || qhip_to_panels_f32(tmp, (int)ff, (int)dm, g->w2[l]) ||
         qhip_upload(g->bf2[l], b->ff_b2.data, dm * 4);
  }
#undef JOIN
  if (qhip_upload_end()) rc = 1;
  qhip_free(tmp); qhip_free(tmp2);
  g->key[0] = m->wte.data; g->key[1] = m->wpe.data; g->key[2] = m->blocks; g->key[3] = m->lm_head.data;
  return rc;
}

static GDev *gdev_create(const GPT *m) {
  const int32_t cfg[6] = {m->vocab_size, m->d_model, m->n_heads, m->n_layers, m->d_ff, m->max_seq_len};
  if (!gpt_cfg_valid(cfg) || !gpt_supported(m)) {
    fprintf(stderr, "Error: gpt_kvcache_create: config not supported by the GPU path\n");
    return NULL;
  }
  if (qhip_init() != 0) { fprintf(stderr, "Error: no usable GPU: %s\n", qhip_last_error()); return NULL; }
  GDev *g = (GDev*)calloc(1, sizeof(GDev));
  if (!g) return NULL;
  g->vocab = m->vocab_size; g->dm = m->d_model; g->nh = m->n_heads; g->hd = m->d_model / m->n_heads;
  g->L = m->n_layers; g->ff = m->d_ff; g->max_seq = m->max_seq_len;
  const int L = g->L;
  float ***vecs[12] = {&g->wqkv, &g->bqkv, &g->wo, &g->bo, &g->g1, &g->be1, &g->g2, &g->be2,
                       &g->w1, &g->bf1, &g->w2, &g->bf2};
  for (int i = 0; i < 12; i++) {
    *vecs[i] = (float**)calloc((size_t)L, sizeof(float*));
    if (!*vecs[i]) { gdev_free(g); return NULL; }
  }
  const size_t dm = (size_t)g->dm, ff = (size_t)g->ff, V = (size_t)g->vocab, S = (size_t)g->max_seq;
  size_t off = 0, *lo = (size_t*)calloc((size_t)L * 12, sizeof(size_t));
  if (!lo) { gdev_free(g); return NULL; }
#define TAKE(nfloats) (off += al256((nfloats) * 4), off - al256((nfloats) * 4))
  for (int l = 0; l < L; l++) {
    const size_t n[12] = {qhip_panels_f32_size((int)dm, (int)(3 * dm)), 3 * dm, qhip_panels_f32_size((int)dm, (int)dm),
                          dm, dm, dm, dm, dm, qhip_panels_f32_size((int)dm, (int)ff), ff,
                          qhip_panels_f32_size((int)ff, (int)dm), dm};
    for (int i = 0; i < 12; i++) lo[l * 12 + i] = TAKE(n[i]);
  }
  const size_t o_wte = TAKE(V * dm), o_wpe = TAKE(S * dm), o_lg = TAKE(dm), o_lb = TAKE(dm);
  const size_t o_head = TAKE(qhip_panels_f32_size((int)dm, (int)V));
  const size_t o_x = TAKE(dm), o_xn = TAKE(dm), o_qkv = TAKE(3 * dm), o_o = TAKE(dm), o_h = TAKE(ff);
  const size_t o_logits = TAKE(V), o_sc = TAKE(qhip_attention_scratch(g->nh, g->max_seq));
  const size_t o_st = TAKE(16), o_in = TAKE(S + 1);
#undef TAKE
  g->blob = (uint8_t*)qhip_malloc(off);
  const size_t per = (size_t)L * S * dm;                 // cache floats per K or V
  g->kbase = (float*)qhip_malloc(per * 4);
  g->vbase = (float*)qhip_malloc(per * 4);
  g->h_stage = (int*)qhip_host_alloc(64);
  if (!g->blob || !g->kbase || !g->vbase || !g->h_stage) {
    fprintf(stderr, "Error: device allocation failed: %s\n", qhip_last_error());
    free(lo); gdev_free(g); return NULL;
  }
  uint8_t *b = g->blob;
  for (int l = 0; l < L; l++)
    for (int i = 0; i < 12; i++) (*vecs[i])[l] = (float*)(b + lo[l * 12 + i]);
  free(lo);
  g->wte = (float*)(b + o_wte); g->wpe = (float*)(b + o_wpe); g->lnf_g = (float*)(b + o_lg);
  g->lnf_b = (float*)(b + o_lb); g->head = (float*)(b + o_head);
  g->x = (float*)(b + o_x); g->xn = (float*)(b + o_xn); g->qkv = (float*)(b + o_qkv); g->o = (float*)(b + o_o);
  g->h = (float*)(b + o_h); g->logits = (float*)(b + o_logits); g->scores = (float*)(b + o_sc);
  g->d_state = (int*)(b + o_st); g->d_in = (int*)(b + o_in);
  if (gdev_upload(g, m) || qhip_fill_zero(g->d_in, (S + 1) * 4) || qhip_fill_zero(g->d_state, 64) || qhip_sync()) {
    fprintf(stderr, "Error: upload of the GPT model failed: %s\n", qhip_last_error());
    gdev_free(g);
    return NULL;
  }
  return g;
}

// model.c:462-518 for the token at d_in[pos], pos = d_state[0]
static int enqueue_gpt_step(const GDev *g) {
  const size_t per = (size_t)g->max_seq * g->dm;
  const float scale = 1.0f / sqrtf((float)g->hd);           // model.c:460
  int rc = qhip_gpt_embed(g->wte, g->wpe, g->dm, g->d_in, g->d_state, g->x);
  for (int l = 0; l < g->L && !rc; l++) {
    float *kc = g->kbase + (size_t)l * per, *vc = g->vbase + (size_t)l * per;
    rc |= qhip_layernorm_f32(g->x, g->dm, g->g1[l], g->be1[l], GPT_LN_EPS, g->xn);
    rc |= qhip_gemv_f32(0, 2, g->xn, g->dm, g->wqkv[l], 3 * g->dm, g->qkv, g->bqkv[l]);
    rc |= qhip_gpt_kv_append(g->qkv, g->dm, g->hd, g->max_seq, g->d_state, kc, vc);
    rc |= qhip_attention_div(g->qkv, kc, vc, g->d_state, g->nh, g->nh, g->hd, g->max_seq, scale, g->scores, g->o);
    rc |= qhip_gemv_f32(2, 6, g->o, g->dm, g->wo[l], g->dm, g->x, g->bo[l]);
    rc |= qhip_layernorm_f32(g->x, g->dm, g->g2[l], g->be2[l], GPT_LN_EPS, g->xn);
    rc |= qhip_gemv_f32(3, 7, g->xn, g->dm, g->w1[l], g->ff, g->h, g->bf1[l]);
    rc |= qhip_gemv_f32(2, 9, g->h, g->ff, g->w2[l], g->dm, g->x, g->bf2[l]);
  }
  if (!rc) rc |= qhip_layernorm_f32(g->x, g->dm, g->lnf_g, g->lnf_b, GPT_LN_EPS, g->xn);
  if (!rc) rc |= qhip_gemv_f32(0, 10, g->xn, g->dm, g->head, g->vocab, g->logits, NULL);
  return rc;
}

KVCache gpt_kvcache_create(const GPT *m) {
  KVCache kv;
  memset(&kv, 0, sizeof kv);
  GDev *g = m ? gdev_create(m) : NULL;
  if (!g) abort();
  kv.n_layers = m->n_layers; kv.d_model = m->d_model; kv.n_heads = m->n_heads; kv.max_seq_len = m->max_seq_len;
  kv.len = 0;
  kv.K = (Tensor*)calloc((size_t)m->n_layers, sizeof(Tensor));
  kv.V = (Tensor*)calloc((size_t)m->n_layers, sizeof(Tensor));
  if (!kv.K || !kv.V) { fprintf(stderr, "Error: out of memory (kv)\n"); abort(); }
  const size_t per = (size_t)m->max_seq_len * m->d_model;
  for (int l = 0; l < m->n_layers; l++) {       // device views, [head][max_seq][head_dim]
    kv.K[l].data = g->kbase + (size_t)l * per; kv.K[l].size = per; kv.K[l].ndim = 3;
    kv.V[l].data = g->vbase + (size_t)l * per; kv.V[l].size = per; kv.V[l].ndim = 3;
  }
  kv.dev = g;
  return kv;
}

void gpt_kvcache_free(KVCache *kv) {
  if (!kv) return;
  gdev_free((GDev*)kv->dev);
  free(kv->K); free(kv->V);
  kv->K = kv->V = NULL;
  kv->dev = NULL;
  kv->len = 0;
}

// The cache's device copy of m's weights made again from the host model: for a
// caller that changed weights in place (same buffers), which the step cannot
// see (it copies only when it is given a different model).  Returns 0 on
// success.  The cached keys and values are kept.
int gpt_kvcache_refresh(KVCache *kv, const GPT *m) {
  GDev *g = kv ? (GDev*)kv->dev : NULL;
  if (!m || !g) {
    fprintf(stderr, "Error: gpt_kvcache_refresh: the cache was not made by gpt_kvcache_create\n");
    return 1;
  }
  if (m->vocab_size != g->vocab || m->d_model != g->dm || m->n_heads != g->nh || m->n_layers != g->L ||
      m->d_ff != g->ff || m->max_seq_len != g->max_seq) {
    fprintf(stderr, "Error: gpt_kvcache_refresh: the cache was made for a model of another shape\n");
    return 1;
  }
  if (qhip_sync() || gdev_upload(g, m) || qhip_sync()) {
    fprintf(stderr, "Error: gpt_kvcache_refresh: weight upload failed: %s\n", qhip_last_error());
    return 1;
  }
  return 0;
}

void gpt_decode_step(const GPT *m, KVCache *kv, int token, Tensor *logits) {
  GDev *g = kv ? (GDev*)kv->dev : NULL;
  if (!m || !g || !logits || !logits->data) {
    fprintf(stderr, "Error: gpt_decode_step: the cache was not made by gpt_kvcache_create\n");
    abort();
  }
  if (m->vocab_size != g->vocab || m->d_model != g->dm || m->n_heads != g->nh || m->n_layers != g->L ||
      m->d_ff != g->ff || m->max_seq_len != g->max_seq) {
    fprintf(stderr, "Error: gpt_decode_step: the cache was made for a model of another shape\n");
    abort();
  }
  if (kv->len < 0 || kv->len >= g->max_seq || token < 0 || token >= g->vocab) {
    fprintf(stderr, "Error: gpt_decode_step: position %d / token %d out of range\n", kv->len, token);
    abort();
  }
  // another host model of the same shape: take its weights (the graph reads the same buffers)
  if (g->key[0] != m->wte.data || g->key[1] != m->wpe.data || g->key[2] != m->blocks ||
      g->key[3] != m->lm_head.data) {
    if (qhip_sync() || gdev_upload(g, m) || qhip_sync()) {
      fprintf(stderr, "Error: gpt_decode_step: weight upload failed: %s\n", qhip_last_error());
      abort();
    }
  }
  int *h = g->h_stage;
  h[0] = kv->len; h[1] = kv->len + 1; h[2] = token;
  int rc = qhip_h2d_async(g->d_state, h, 2 * sizeof(int)) || qhip_h2d_async(g->d_in + kv->len, h + 2, sizeof(int));
  if (!rc) {
    if (getenv("QLLAMA_NO_GRAPH") || qhip_profiling()) {
      rc = enqueue_gpt_step(g);
    } else {
      if (!g->graph) {
        void *gr = NULL;
        rc = qhip_capture_begin();
        if (!rc) {
          const int e = enqueue_gpt_step(g);
          rc = qhip_capture_end(&gr) || e;
        }
        if (!rc) g->graph = gr;
        else if (gr) qhip_graph_destroy(gr);
      }
      if (!rc) rc = qhip_graph_launch(g->graph);
    }
  }
  if (rc || qhip_d2h_async(logits->data, g->logits, (size_t)g->vocab * 4) || qhip_sync()) {
    fprintf(stderr, "Error: gpt_decode_step: %s\n", qhip_last_error());
    abort();
  }
  kv->len += 1;
}
