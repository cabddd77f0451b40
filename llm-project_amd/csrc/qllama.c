// qllama.c - C11 host side of the MI355X int8 LLaMA decode path.
//
// Keeps the reference's quantized API (llama.h:114-140, quant.h:15-33) and its
// decode loop structure (llama.c:528-600); every numeric step is a launch into
// the HIP layer (qhip.h).  The whole per-token sequence reads the token and the
// position from device memory, so it is captured once into a HIP graph per
// (model, KV cache) pair and replayed for every token.
#define _POSIX_C_SOURCE 200809L
#include "qllama.h"
#include "qhip.h"

#include <limits.h>
#include <math.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <fcntl.h>
#include <sys/mman.h>
#include <sys/stat.h>
#include <sys/types.h>
#include <unistd.h>

#define LLMQ_MAGIC   0x514D4C4Cu   // llama.c:193
#define QLLAMA_CLS_OTHER 12        // kernel class "other" of the event timing
#define LLMA_VERSION 2u            // llama.c:194

static int pad16(int k) { return (k + 15) & ~15; }
static size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

static void die(const char *what) {
  fprintf(stderr, "Error: %s: %s\n", what, qhip_last_error());
  abort();
}

// ---------------------------------------------------------------------------
// Device model state
// ---------------------------------------------------------------------------
typedef struct {
  int vocab, dm, L, H, KVH, hd, dff, max_seq, qd, kvd, nqkv;
  int kp_dm, kp_qd, kp_ff, kp_max;
  float eps, rope_base, attn_scale;
  uint8_t *blob;
  // per layer (aliases into blob)
  int8_t **wqkv, **wo, **wgu, **wd;
  float **sqkv, **bqkv, **so, **sgu, **sd, **g_attn, **g_ffn;
  int8_t *wte, *head;
  float *wte_s, *head_s, *g_final;
  float *rope_cos, *rope_sin;
  // scratch
  float *x, *qkv, *q, *o, *gu, *logits, *scores, *as, *obm, *hbm, *amax_v;
  int *amax_i;
  int8_t *qa;
  int *d_state;      // [0] pos, [1] fill_end
  int *d_in;         // max_seq + 1 input tokens by position
  int *d_out;        // max_seq argmax ids by position
  int *h_stage;      // pinned staging, max_seq + 2 ints
  float *h_logits;   // pinned staging of the logits (vocab floats): a copy from the device into
                     // pinned memory runs at the link's rate, one into pageable memory does not
  uint64_t gen;      // process-wide generation: identifies this model to the graphs of its caches
  // prompt ingestion (allocated on first use): rows of activations
  int pf_rows;
  float *pf_x, *pf_qkv, *pf_q, *pf_o, *pf_h, *pf_as, *pf_attn;
  int8_t *pf_qa;
  int *pf_work;      // split-K partial sums of the prompt GEMMs (PF_WORK_BYTES)
  // the attention half of a decode layer in one launch (qhip_attn_layer), where served
  int ly_ok;
  float *ly_scratch;
  unsigned *ly_sync;
} QDev;

typedef struct {
  float *kbase, *vbase;
  int mode;            // QLLAMA_MODE_*
  void *fa_scratch;    // fast mode: split-K attention partials and counters
  // a captured graph bakes in the device addresses of the model it was made
  // for; it is reused only while that model (by generation, never by address,
  // which the allocator may hand out again) and the sampler buffers are the same
  void *graph;
  uint64_t graph_gen;
  // sampled step (sampler kernels, then the decode step) for one parameter set
  void *sgraph;
  uint64_t sgraph_gen, sgraph_smp_gen;
  float sg_t, sg_p;
  int sg_k;
  struct FDev *fdev;   // fp32 caches: the device model they belong to
} KVDev;

// Generations start at 1, so a zeroed KVDev matches no model.
static uint64_t g_generation = 0;
static uint64_t next_generation(void) { return ++g_generation; }

static int config_valid(const int32_t *cfg) {
  // Same acceptance rule as llama.c:371-386: positive bounded dims, whole GQA
  // groups, 2-D element counts within int.
  const long long MAXD = 1000000;
  for (int i = 0; i < 8; i++)
    if (cfg[i] <= 0 || cfg[i] > MAXD) return 0;
  const long long vocab = cfg[0], dm = cfg[1], H = cfg[3], KVH = cfg[4], hd = cfg[5], ff = cfg[6];
  if (H % KVH != 0) return 0;
  if (H * hd > MAXD || KVH * hd > MAXD) return 0;
  if (vocab * dm > INT_MAX || dm * ff > INT_MAX || H * hd * dm > INT_MAX) return 0;
  return 1;
}

// Shapes the kernels of this build support (beyond the reference's own checks).
static int config_supported(const int32_t *cfg) {
  const int dm = cfg[1], hd = cfg[5], ff = cfg[6], G = cfg[3] / cfg[4];
  if (hd % 2 != 0 || hd > 512) return 0;
  if (G > 8 || G * hd > 4096) return 0;  // the decode attention serves up to 8 query heads per KV head
  if (dm > 16384 || ff > 32768 || cfg[3] * hd > 32768) return 0;   // rmsnorm holds a row in one block
  if (cfg[7] > 16384) return 0;          // attention keeps a head's softmax weights in LDS
  return 1;
}

static Tensor dev_tensor(float *p, int n) {
  Tensor t;
  t.data = p; t.grad = NULL; t.ndim = 1; t.size = (size_t)n;
  t.shape = (int*)malloc(sizeof(int));
  if (t.shape) t.shape[0] = n;
  return t;
}

static QTensor dev_qt(int8_t *q, float *s, int rows, int cols, int layout) {
  QTensor t;
  t.rows = rows; t.cols = cols; t.q = (signed char*)q; t.scale = s; t.layout = layout;
  t.kpad = layout == QT_LAYOUT_NK ? pad16(rows) : cols;
  return t;
}

static void pf_free(QDev *d) {
  qhip_free(d->pf_x); qhip_free(d->pf_qkv); qhip_free(d->pf_q); qhip_free(d->pf_o);
  qhip_free(d->pf_h); qhip_free(d->pf_as); qhip_free(d->pf_attn); qhip_free(d->pf_qa); qhip_free(d->pf_work);
  d->pf_x = d->pf_qkv = d->pf_q = d->pf_o = d->pf_h = d->pf_as = d->pf_attn = NULL;
  d->pf_qa = NULL;
  d->pf_work = NULL;
  d->pf_rows = 0;
}

static void qdev_free(QDev *d) {
  if (!d) return;
  pf_free(d);
  qhip_free(d->blob);
  qhip_host_free(d->h_stage);
  qhip_host_free(d->h_logits);
  free(d->wqkv); free(d->wo); free(d->wgu); free(d->wd);
  free(d->sqkv); free(d->bqkv); free(d->so); free(d->sgu); free(d->sd);
  free(d->g_attn); free(d->g_ffn);
  free(d);
}

// The host-built RoPE tables (rope.c:58-61 with the host libm).
static int rope_upload(float *dcos, float *dsin, int max_seq, int hd, float base) {
  const int half = hd / 2;
  float *ct = (float*)malloc((size_t)max_seq * half * sizeof(float));
  float *st = (float*)malloc((size_t)max_seq * half * sizeof(float));
  if (!ct || !st) { free(ct); free(st); return 1; }
  for (int pos = 0; pos < max_seq; pos++)
    for (int k = 0; k < half; k++) {
      float inv_freq = powf(base, -2.0f * (float)k / (float)hd);
      float ang = (float)pos * inv_freq;
      ct[(size_t)pos * half + k] = cosf(ang);
      st[(size_t)pos * half + k] = sinf(ang);
    }
  int rc = qhip_h2d(dcos, ct, (size_t)max_seq * half * 4) | qhip_h2d(dsin, st, (size_t)max_seq * half * 4);
  free(ct); free(st);
  return rc;
}

// Allocate one blob holding every weight and the scratch; fill the QLlamaModel
// view (config ints, QTensor / Tensor device views).
static int model_alloc(QLlamaModel *m, const int32_t cfg[8], float rope_base, float eps) {
  memset(m, 0, sizeof *m);
  if (qhip_init() != 0) {
    fprintf(stderr, "Error: no usable GPU: %s\n", qhip_last_error());
    return 1;
  }
  QDev *d = (QDev*)calloc(1, sizeof(QDev));
  if (!d) return 1;
  d->vocab = cfg[0]; d->dm = cfg[1]; d->L = cfg[2]; d->H = cfg[3]; d->KVH = cfg[4];
  d->hd = cfg[5]; d->dff = cfg[6]; d->max_seq = cfg[7];
  d->qd = d->H * d->hd; d->kvd = d->KVH * d->hd; d->nqkv = d->qd + 2 * d->kvd;
  d->kp_dm = pad16(d->dm); d->kp_qd = pad16(d->qd); d->kp_ff = pad16(d->dff);
  d->kp_max = d->kp_dm;
  if (d->kp_qd > d->kp_max) d->kp_max = d->kp_qd;
  if (d->kp_ff > d->kp_max) d->kp_max = d->kp_ff;
  d->eps = eps; d->rope_base = rope_base;
  d->gen = next_generation();
  d->attn_scale = 1.0f / sqrtf((float)d->hd);          // llama.c:532
  const int L = d->L;
  d->wqkv = calloc(L, sizeof(int8_t*)); d->wo = calloc(L, sizeof(int8_t*));
  d->wgu = calloc(L, sizeof(int8_t*)); d->wd = calloc(L, sizeof(int8_t*));
  d->sqkv = calloc(L, sizeof(float*)); d->bqkv = calloc(L, sizeof(float*));
  d->so = calloc(L, sizeof(float*)); d->sgu = calloc(L, sizeof(float*));
  d->sd = calloc(L, sizeof(float*)); d->g_attn = calloc(L, sizeof(float*));
  d->g_ffn = calloc(L, sizeof(float*));
  if (!d->wqkv || !d->wo || !d->wgu || !d->wd || !d->sqkv || !d->bqkv || !d->so || !d->sgu ||
      !d->sd || !d->g_attn || !d->g_ffn) { qdev_free(d); return 1; }

  // --- blob layout ---
  size_t off = 0;
#define TAKE(n) (off += al256(n), off - al256(n))
  size_t *o_wqkv = calloc(L, sizeof(size_t)), *o_wo = calloc(L, sizeof(size_t));
  size_t *o_wgu = calloc(L, sizeof(size_t)), *o_wd = calloc(L, sizeof(size_t));
  size_t *o_s = calloc((size_t)L * 8, sizeof(size_t));
  if (!o_wqkv || !o_wo || !o_wgu || !o_wd || !o_s) { qdev_free(d); return 1; }
  for (int l = 0; l < L; l++) {
    o_wqkv[l] = TAKE((size_t)d->nqkv * d->kp_dm);
    o_wo[l] = TAKE((size_t)d->dm * d->kp_qd);
    o_wgu[l] = TAKE((size_t)2 * d->dff * d->kp_dm);
    o_wd[l] = TAKE((size_t)d->dm * d->kp_ff);
    o_s[l * 8 + 0] = TAKE((size_t)d->nqkv * 4);
    o_s[l * 8 + 1] = TAKE((size_t)d->nqkv * 4);
    o_s[l * 8 + 2] = TAKE((size_t)d->dm * 4);
    o_s[l * 8 + 3] = TAKE((size_t)2 * d->dff * 4);
    o_s[l * 8 + 4] = TAKE((size_t)d->dm * 4);
    o_s[l * 8 + 5] = TAKE((size_t)d->dm * 4);
    o_s[l * 8 + 6] = TAKE((size_t)d->dm * 4);
  }
  size_t o_wte = TAKE((size_t)d->vocab * d->dm);
  size_t o_wte_s = TAKE((size_t)d->dm * 4);
  size_t o_head = TAKE((size_t)d->vocab * d->kp_dm);
  size_t o_head_s = TAKE((size_t)d->vocab * 4);
  size_t o_gf = TAKE((size_t)d->dm * 4);
  const int half = d->hd / 2;
  size_t o_cos = TAKE((size_t)d->max_seq * half * 4);
  size_t o_sin = TAKE((size_t)d->max_seq * half * 4);
  size_t o_x = TAKE((size_t)d->dm * 4);
  size_t o_qkv = TAKE((size_t)d->nqkv * 4);
  size_t o_q = TAKE((size_t)d->qd * 4);
  size_t o_o = TAKE((size_t)d->qd * 4);
  size_t o_gu = TAKE((size_t)2 * d->dff * 4);
  size_t o_logits = TAKE((size_t)d->vocab * 4);
  size_t o_scores = TAKE(qhip_attention_scratch(d->H, d->max_seq) * 4);
  size_t o_as = TAKE(64);
  size_t o_obm = TAKE((size_t)qhip_attention_nbm(d->H, d->hd) * 4);
  size_t o_hbm = TAKE((size_t)qhip_gemv_blocks(d->dff, d->kp_dm) * 4);
  size_t o_amv = TAKE((size_t)qhip_gemv_blocks(d->vocab, d->kp_dm) * 4);
  size_t o_ami = TAKE((size_t)qhip_gemv_blocks(d->vocab, d->kp_dm) * 4);
  size_t o_qa = TAKE((size_t)d->kp_max);
  size_t o_state = TAKE(64);
  size_t o_in = TAKE((size_t)(d->max_seq + 1) * 4);
  size_t o_out = TAKE((size_t)(d->max_seq + 1) * 4);
  size_t o_ly = TAKE(qhip_attn_layer_scratch(d->H, d->KVH, d->hd) * 4);
  size_t o_lys = TAKE(qhip_attn_layer_sync_words(d->KVH) * 4);
#undef TAKE
  d->blob = (uint8_t*)qhip_malloc(off);
  d->h_stage = (int*)qhip_host_alloc((size_t)(d->max_seq + 2) * sizeof(int));
  d->h_logits = (float*)qhip_host_alloc((size_t)d->vocab * sizeof(float));
  if (!d->blob || !d->h_stage || !d->h_logits) {
    fprintf(stderr, "Error: device allocation of %zu bytes failed: %s\n", off, qhip_last_error());
    free(o_wqkv); free(o_wo); free(o_wgu); free(o_wd); free(o_s);
    qdev_free(d);
    return 1;
  }
  uint8_t *b = d->blob;
  for (int l = 0; l < L; l++) {
    d->wqkv[l] = (int8_t*)(b + o_wqkv[l]); d->wo[l] = (int8_t*)(b + o_wo[l]);
    d->wgu[l] = (int8_t*)(b + o_wgu[l]); d->wd[l] = (int8_t*)(b + o_wd[l]);
    d->sqkv[l] = (float*)(b + o_s[l * 8 + 0]); d->bqkv[l] = (float*)(b + o_s[l * 8 + 1]);
    d->so[l] = (float*)(b + o_s[l * 8 + 2]); d->sgu[l] = (float*)(b + o_s[l * 8 + 3]);
    d->sd[l] = (float*)(b + o_s[l * 8 + 4]); d->g_attn[l] = (float*)(b + o_s[l * 8 + 5]);
    d->g_ffn[l] = (float*)(b + o_s[l * 8 + 6]);
  }
  free(o_wqkv); free(o_wo); free(o_wgu); free(o_wd); free(o_s);
  d->wte = (int8_t*)(b + o_wte); d->wte_s = (float*)(b + o_wte_s);
  d->head = (int8_t*)(b + o_head); d->head_s = (float*)(b + o_head_s);
  d->g_final = (float*)(b + o_gf);
  d->rope_cos = (float*)(b + o_cos); d->rope_sin = (float*)(b + o_sin);
  d->x = (float*)(b + o_x); d->qkv = (float*)(b + o_qkv); d->q = (float*)(b + o_q);
  d->o = (float*)(b + o_o); d->gu = (float*)(b + o_gu); d->logits = (float*)(b + o_logits);
  d->scores = (float*)(b + o_scores); d->as = (float*)(b + o_as);
  d->obm = (float*)(b + o_obm); d->hbm = (float*)(b + o_hbm);
  d->amax_v = (float*)(b + o_amv); d->amax_i = (int*)(b + o_ami); d->qa = (int8_t*)(b + o_qa);
  d->d_state = (int*)(b + o_state); d->d_in = (int*)(b + o_in); d->d_out = (int*)(b + o_out);
  d->ly_scratch = (float*)(b + o_ly); d->ly_sync = (unsigned*)(b + o_lys);
  // QLLAMA_NO_ATTN_LAYER=1 keeps the separate QKV, scores and PV kernels (same results)
  d->ly_ok = !getenv("QLLAMA_NO_ATTN_LAYER") && qhip_gemv_norm_ok(d->kp_dm, d->dm) &&
             qhip_attn_layer_ok(d->H, d->KVH, d->hd, d->kp_dm, d->max_seq);
  if (qhip_fill_zero(d->qa, (size_t)d->kp_max) || qhip_fill_zero(d->d_in, (size_t)(d->max_seq + 1) * 4) ||
      qhip_fill_zero(d->d_state, 64) || qhip_fill_zero(d->ly_sync, qhip_attn_layer_sync_words(d->KVH) * 4)) {
    qdev_free(d);
    return 1;
  }

  // --- RoPE tables: the expressions of rope.c:58-61, evaluated on the host with
  // the same libm, so the device reads bit-identical cos/sin values.
  if (rope_upload(d->rope_cos, d->rope_sin, d->max_seq, d->hd, rope_base)) { qdev_free(d); return 1; }

  // --- API view ---
  m->vocab = d->vocab; m->d_model = d->dm; m->n_layers = L; m->n_heads = d->H;
  m->n_kv = d->KVH; m->head_dim = d->hd; m->d_ff = d->dff; m->max_seq = d->max_seq;
  m->rope_base = rope_base; m->eps = eps;
  m->wte = dev_qt(d->wte, d->wte_s, d->vocab, d->dm, QT_LAYOUT_KN);
  m->lm_head = dev_qt(d->head, d->head_s, d->dm, d->vocab, QT_LAYOUT_NK);
  m->final_norm = dev_tensor(d->g_final, d->dm);
  m->blocks = (QLlamaBlock*)calloc((size_t)L, sizeof(QLlamaBlock));
  if (!m->blocks) { qdev_free(d); return 1; }
  for (int l = 0; l < L; l++) {
    QLlamaBlock *bl = &m->blocks[l];
    bl->attn_norm = dev_tensor(d->g_attn[l], d->dm);
    bl->ffn_norm = dev_tensor(d->g_ffn[l], d->dm);
    bl->b_q = dev_tensor(d->bqkv[l], d->qd);
    bl->b_k = dev_tensor(d->bqkv[l] + d->qd, d->kvd);
    bl->b_v = dev_tensor(d->bqkv[l] + d->qd + d->kvd, d->kvd);
    bl->Wq = dev_qt(d->wqkv[l], d->sqkv[l], d->dm, d->qd, QT_LAYOUT_NK);
    bl->Wk = dev_qt(d->wqkv[l] + (size_t)d->qd * d->kp_dm, d->sqkv[l] + d->qd, d->dm, d->kvd, QT_LAYOUT_NK);
    bl->Wv = dev_qt(d->wqkv[l] + (size_t)(d->qd + d->kvd) * d->kp_dm, d->sqkv[l] + d->qd + d->kvd,
                    d->dm, d->kvd, QT_LAYOUT_NK);
    bl->Wo = dev_qt(d->wo[l], d->so[l], d->qd, d->dm, QT_LAYOUT_NK);
    bl->Wgate = dev_qt(d->wgu[l], d->sgu[l], d->dm, d->dff, QT_LAYOUT_NK);
    bl->Wup = dev_qt(d->wgu[l] + (size_t)d->dff * d->kp_dm, d->sgu[l] + d->dff, d->dm, d->dff, QT_LAYOUT_NK);
    bl->Wdown = dev_qt(d->wd[l], d->sd[l], d->dff, d->dm, QT_LAYOUT_NK);
  }
  m->dev = d;
  return 0;
}

static void free_view(QLlamaModel *m) {
  if (m->blocks) {
    for (int l = 0; l < m->n_layers; l++) {
      QLlamaBlock *b = &m->blocks[l];
      free(b->attn_norm.shape); free(b->ffn_norm.shape);
      free(b->b_q.shape); free(b->b_k.shape); free(b->b_v.shape);
    }
  }
  free(m->blocks); m->blocks = NULL;
  free(m->final_norm.shape); m->final_norm.shape = NULL;
}

void q_llama_model_free(QLlamaModel *m) {
  if (!m) return;
  if (m->dev) qhip_sync();
  free_view(m);
  qdev_free((QDev*)m->dev);
  m->dev = NULL;
}

// Norm gains 1, biases 0 (the seeded models and any freshly loaded layer start so).
static int init_vectors(QDev *d) {
  for (int l = 0; l < d->L; l++) {
    if (qhip_fill_f32(d->g_attn[l], (size_t)d->dm, 1.0f) || qhip_fill_f32(d->g_ffn[l], (size_t)d->dm, 1.0f) ||
        qhip_fill_f32(d->bqkv[l], (size_t)d->nqkv, 0.0f)) return 1;
  }
  return qhip_fill_f32(d->g_final, (size_t)d->dm, 1.0f);
}

int q_llama_model_synth(QLlamaModel *out, const int32_t cfg[8], float rope_base, float eps,
                        uint64_t seed, int tied) {
  if (!config_valid(cfg) || !config_supported(cfg)) {
    fprintf(stderr, "Error: invalid/unsupported config\n");
    return 1;
  }
  if (model_alloc(out, cfg, rope_base, eps)) return 1;
  QDev *d = (QDev*)out->dev;
  int rc = init_vectors(d);
  rc |= qhip_synth_quant_kn(seed, 0, d->vocab, d->dm, 0.02, d->wte, d->wte_s);
  for (int l = 0; l < d->L && !rc; l++) {
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    const int kp = d->kp_dm;
    rc |= qhip_synth_quant_nk(seed, t0 + 1, d->dm, d->qd, kp, 0, 0.02, d->wqkv[l], d->sqkv[l]);
    rc |= qhip_synth_quant_nk(seed, t0 + 2, d->dm, d->kvd, kp, 0, 0.02,
                              d->wqkv[l] + (size_t)d->qd * kp, d->sqkv[l] + d->qd);
    rc |= qhip_synth_quant_nk(seed, t0 + 3, d->dm, d->kvd, kp, 0, 0.02,
                              d->wqkv[l] + (size_t)(d->qd + d->kvd) * kp, d->sqkv[l] + d->qd + d->kvd);
    rc |= qhip_synth_quant_nk(seed, t0 + 7, d->qd, d->dm, d->kp_qd, 0, 0.02, d->wo[l], d->so[l]);
    rc |= qhip_synth_quant_nk(seed, t0 + 9, d->dm, d->dff, kp, 0, 0.02, d->wgu[l], d->sgu[l]);
    rc |= qhip_synth_quant_nk(seed, t0 + 10, d->dm, d->dff, kp, 0, 0.02,
                              d->wgu[l] + (size_t)d->dff * kp, d->sgu[l] + d->dff);
    rc |= qhip_synth_quant_nk(seed, t0 + 11, d->dff, d->dm, d->kp_ff, 0, 0.02, d->wd[l], d->sd[l]);
  }
  if (!rc) {
    if (tied) rc = qhip_synth_quant_nk(seed, 0, d->dm, d->vocab, d->kp_dm, 1, 0.02, d->head, d->head_s);
    else rc = qhip_synth_quant_nk(seed, 2 + 12 * (uint64_t)d->L, d->dm, d->vocab, d->kp_dm, 0, 0.02,
                                  d->head, d->head_s);
  }
  if (!rc) rc = qhip_sync();
  if (rc) {
    fprintf(stderr, "Error: synthetic model build failed: %s\n", qhip_last_error());
    q_llama_model_free(out);
    return 1;
  }
  return 0;
}

// Digest of one tensor: the same combination the generator's CPU side uses.
static int qt_digest(const QTensor *t, uint64_t salt, uint64_t *h) {
  uint64_t a = 0, s = 0;
  if (qhip_hash_i8((const int8_t*)t->q, t->rows, t->cols, t->layout == QT_LAYOUT_NK, t->kpad, salt, &a)) return 1;
  if (qhip_hash_f32(t->scale, (size_t)t->cols, salt ^ 0x5CA1E5ULL, &s)) return 1;
  *h = a * 3 + s;
  return 0;
}

uint64_t q_llama_model_hash(const QLlamaModel *m) {
  uint64_t h = 0, t = 0;
  if (qt_digest(&m->wte, 0, &h)) die("model hash");
  for (int l = 0; l < m->n_layers; l++) {
    const QLlamaBlock *b = &m->blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    const QTensor *list[7] = {&b->Wq, &b->Wk, &b->Wv, &b->Wo, &b->Wgate, &b->Wup, &b->Wdown};
    const int off[7] = {1, 2, 3, 7, 9, 10, 11};
    for (int i = 0; i < 7; i++) {
      if (qt_digest(list[i], t0 + (uint64_t)off[i], &t)) die("model hash");
      h = h * 31 + t;
    }
  }
  if (qt_digest(&m->lm_head, 2 + 12 * (uint64_t)m->n_layers, &t)) die("model hash");
  return h * 31 + t;
}

// ---------------------------------------------------------------------------
// Loading: LLMQ v2 (llama.c:603-657 byte order).  The file is mapped, each
// tensor is streamed to HBM through double-buffered pinned staging with async
// copies, and int8 matrices are transposed into the NK layout on the device.
// ---------------------------------------------------------------------------
typedef struct {
  const uint8_t *p;     // mapped file
  size_t size, off;
} FileCur;

static const void *cur_take(FileCur *c, size_t n) {
  if (c->size - c->off < n) return NULL;
  const void *r = c->p + c->off;
  c->off += n;
  return r;
}

// One int8 tensor: cols f32 scales, then rows*cols int8 row-major (llama.c:603-608).
// 1 = truncated, 2 = device error.
static int read_q(FileCur *c, int rows, int cols, int layout_nk, int kpad, int8_t *dq, float *ds, int8_t *dtmp) {
  const void *sc = cur_take(c, (size_t)cols * 4);
  const void *body = cur_take(c, (size_t)rows * cols);
  if (!sc || !body) return 1;
  if (qhip_upload(ds, sc, (size_t)cols * 4)) return 2;
  if (qhip_upload(layout_nk ? dtmp : dq, body, (size_t)rows * cols)) return 2;
  if (layout_nk && qhip_transpose_kn_to_nk(dtmp, rows, cols, kpad, dq)) return 2;
  return 0;
}

static int read_f(FileCur *c, float *dst, int n) {
  const void *v = cur_take(c, (size_t)n * 4);
  if (!v) return 1;
  return qhip_upload(dst, v, (size_t)n * 4) ? 2 : 0;
}

int q_llama_model_load(const char *path, QLlamaModel *out) {
  int fd = open(path, O_RDONLY);
  if (fd < 0) { fprintf(stderr, "Error: cannot open '%s' for reading\n", path); return 1; }
  struct stat stt;
  if (fstat(fd, &stt) != 0) { fprintf(stderr, "Error: cannot open '%s' for reading\n", path); close(fd); return 1; }
  const size_t fsize = (size_t)stt.st_size;
  const size_t hdr = 2 * sizeof(uint32_t) + 8 * sizeof(int32_t) + 2 * sizeof(float);
  uint32_t header[2];
  int32_t cfg[8];
  float fcfg[2];
  if (fsize < hdr || pread(fd, header, sizeof header, 0) != (ssize_t)sizeof header ||
      pread(fd, cfg, sizeof cfg, 8) != (ssize_t)sizeof cfg || pread(fd, fcfg, sizeof fcfg, 40) != (ssize_t)sizeof fcfg) {
    fprintf(stderr, "Error: '%s' is truncated (bad header)\n", path);
    close(fd); return 1;
  }
  if (header[0] != LLMQ_MAGIC || header[1] != LLMA_VERSION) {
    fprintf(stderr, "Error: '%s' is not a v%u int8 LLMQ checkpoint\n", path, LLMA_VERSION);
    close(fd); return 1;
  }
  if (!config_valid(cfg)) {
    fprintf(stderr, "Error: '%s' has an invalid/unsupported config\n", path);
    close(fd); return 1;
  }
  if (!config_supported(cfg)) {
    fprintf(stderr, "Error: '%s' has a config this GPU build does not support\n", path);
    close(fd); return 1;
  }
  void *map = mmap(NULL, fsize, PROT_READ, MAP_PRIVATE, fd, 0);
  close(fd);
  if (map == MAP_FAILED) { fprintf(stderr, "Error: cannot map '%s'\n", path); return 1; }
  (void)posix_madvise(map, fsize, POSIX_MADV_SEQUENTIAL);
  if (model_alloc(out, cfg, fcfg[0], fcfg[1])) { munmap(map, fsize); return 1; }
  QDev *d = (QDev*)out->dev;
  size_t big = (size_t)d->dm * d->dff;                 // largest NK matrix staged for the transpose
  if ((size_t)d->qd * d->dm > big) big = (size_t)d->qd * d->dm;
  if ((size_t)d->vocab * d->dm > big) big = (size_t)d->vocab * d->dm;
  int8_t *dtmp = (int8_t*)qhip_malloc(big);
  FileCur c = {(const uint8_t*)map, fsize, hdr};
  int rc = (!dtmp || qhip_upload_begin((size_t)32 << 20)) ? 2 : 0;
  const int kp = d->kp_dm;
  if (!rc) rc = read_q(&c, d->vocab, d->dm, 0, d->dm, d->wte, d->wte_s, dtmp);
  for (int l = 0; l < d->L && !rc; l++) {
    rc = read_f(&c, d->g_attn[l], d->dm);
    if (!rc) rc = read_q(&c, d->dm, d->qd, 1, kp, d->wqkv[l], d->sqkv[l], dtmp);
    if (!rc) rc = read_q(&c, d->dm, d->kvd, 1, kp, d->wqkv[l] + (size_t)d->qd * kp, d->sqkv[l] + d->qd, dtmp);
    if (!rc) rc = read_q(&c, d->dm, d->kvd, 1, kp, d->wqkv[l] + (size_t)(d->qd + d->kvd) * kp,
                         d->sqkv[l] + d->qd + d->kvd, dtmp);
    if (!rc) rc = read_f(&c, d->bqkv[l], d->qd);
    if (!rc) rc = read_f(&c, d->bqkv[l] + d->qd, d->kvd);
    if (!rc) rc = read_f(&c, d->bqkv[l] + d->qd + d->kvd, d->kvd);
    if (!rc) rc = read_q(&c, d->qd, d->dm, 1, d->kp_qd, d->wo[l], d->so[l], dtmp);
    if (!rc) rc = read_f(&c, d->g_ffn[l], d->dm);
    if (!rc) rc = read_q(&c, d->dm, d->dff, 1, kp, d->wgu[l], d->sgu[l], dtmp);
    if (!rc) rc = read_q(&c, d->dm, d->dff, 1, kp, d->wgu[l] + (size_t)d->dff * kp, d->sgu[l] + d->dff, dtmp);
    if (!rc) rc = read_q(&c, d->dff, d->dm, 1, d->kp_ff, d->wd[l], d->sd[l], dtmp);
  }
  if (!rc) rc = read_f(&c, d->g_final, d->dm);
  if (!rc) rc = read_q(&c, d->dm, d->vocab, 1, kp, d->head, d->head_s, dtmp);
  if (qhip_upload_end() && !rc) rc = 2;
  munmap(map, fsize);
  qhip_free(dtmp);
  if (rc) {
    if (rc == 1) fprintf(stderr, "Error: '%s' is truncated (bad weights)\n", path);
    else fprintf(stderr, "Error: device upload of '%s' failed: %s\n", path, qhip_last_error());
    q_llama_model_free(out);
    return 1;
  }
  return 0;
}

// The writer's side of the same format (tools/convert_llama.py:73-97 with
// int8=True): every int8 matrix as cols f32 scales then rows*cols int8 bytes.
static int write_q(FILE *f, const QTensor *t, int8_t *qh, float *sh) {
  if (q_llama_tensor_export(t, (signed char*)qh, sh)) return 1;
  return fwrite(sh, 4, (size_t)t->cols, f) != (size_t)t->cols ||
         fwrite(qh, 1, (size_t)t->rows * t->cols, f) != (size_t)t->rows * t->cols;
}

static int write_f(FILE *f, const float *dev, int n, float *sh) {
  if (qhip_d2h(sh, dev, (size_t)n * 4)) return 1;
  return fwrite(sh, 4, (size_t)n, f) != (size_t)n;
}

int q_llama_model_save(const QLlamaModel *m, const char *path) {
  const QDev *d = m ? (const QDev*)m->dev : NULL;
  if (!d) { fprintf(stderr, "Error: q_llama_model_save: model not on the GPU\n"); return 1; }
  FILE *f = fopen(path, "wb");
  if (!f) { fprintf(stderr, "Error: cannot open '%s' for writing\n", path); return 1; }
  size_t big = (size_t)d->vocab * d->dm;
  if ((size_t)d->dm * d->dff > big) big = (size_t)d->dm * d->dff;
  if ((size_t)d->qd * d->dm > big) big = (size_t)d->qd * d->dm;
  size_t nf = (size_t)d->vocab;
  if ((size_t)d->dff > nf) nf = (size_t)d->dff;
  if ((size_t)d->nqkv > nf) nf = (size_t)d->nqkv;
  int8_t *qh = (int8_t*)malloc(big);
  float *sh = (float*)malloc(nf * 4);
  const uint32_t header[2] = {LLMQ_MAGIC, LLMA_VERSION};
  const int32_t cfg[8] = {m->vocab, m->d_model, m->n_layers, m->n_heads, m->n_kv, m->head_dim, m->d_ff, m->max_seq};
  const float fcfg[2] = {m->rope_base, m->eps};
  int rc = !qh || !sh || fwrite(header, 4, 2, f) != 2 || fwrite(cfg, 4, 8, f) != 8 || fwrite(fcfg, 4, 2, f) != 2;
  if (!rc) rc = write_q(f, &m->wte, qh, sh);
  for (int l = 0; l < m->n_layers && !rc; l++) {
    const QLlamaBlock *b = &m->blocks[l];
    rc = write_f(f, d->g_attn[l], d->dm, sh) || write_q(f, &b->Wq, qh, sh) || write_q(f, &b->Wk, qh, sh) ||
         write_q(f, &b->Wv, qh, sh) || write_f(f, d->bqkv[l], d->qd, sh) ||
         write_f(f, d->bqkv[l] + d->qd, d->kvd, sh) || write_f(f, d->bqkv[l] + d->qd + d->kvd, d->kvd, sh) ||
         write_q(f, &b->Wo, qh, sh) || write_f(f, d->g_ffn[l], d->dm, sh) || write_q(f, &b->Wgate, qh, sh) ||
         write_q(f, &b->Wup, qh, sh) || write_q(f, &b->Wdown, qh, sh);
  }
  if (!rc) rc = write_f(f, d->g_final, d->dm, sh) || write_q(f, &m->lm_head, qh, sh);
  if (fclose(f) != 0) rc = 1;
  free(qh); free(sh);
  if (rc) { fprintf(stderr, "Error: writing '%s' failed\n", path); return 1; }
  return 0;
}

// llama.c:490-511 on the device: each 2-D weight is uploaded in f32 and
// quantized per output column there; norms and biases are copied as f32.
QLlamaModel q_llama_quantize_from(const LlamaModel *s) {
  QLlamaModel m;
  int32_t cfg[8] = {s->vocab, s->d_model, s->n_layers, s->n_heads, s->n_kv, s->head_dim, s->d_ff, s->max_seq};
  if (!config_valid(cfg) || !config_supported(cfg)) {
    fprintf(stderr, "Error: q_llama_quantize_from: invalid/unsupported config\n");
    abort();
  }
  if (model_alloc(&m, cfg, s->rope_base, s->eps)) die("q_llama_quantize_from");
  QDev *d = (QDev*)m.dev;
  size_t big = (size_t)d->vocab * d->dm;
  if ((size_t)d->dm * d->dff > big) big = (size_t)d->dm * d->dff;
  if ((size_t)d->qd * d->dm > big) big = (size_t)d->qd * d->dm;
  float *dw = (float*)qhip_malloc(big * 4);
  if (!dw) die("q_llama_quantize_from");
#define QUANT(src, rows, cols, nk, kpad, q, sc) \
  do { if (qhip_h2d(dw, (src)->data, (size_t)(rows) * (cols) * 4) || \
           qhip_quantize_percol(dw, rows, cols, nk, kpad, q, sc)) die("q_llama_quantize_from"); } while (0)
#define COPYF(dst, src, n) do { if (qhip_h2d(dst, (src)->data, (size_t)(n) * 4)) die("q_llama_quantize_from"); } while (0)
  const int kp = d->kp_dm;
  QUANT(&s->wte, d->vocab, d->dm, 0, d->dm, d->wte, d->wte_s);
  for (int l = 0; l < d->L; l++) {
    const LlamaBlock *a = &s->blocks[l];
    COPYF(d->g_attn[l], &a->attn_norm, d->dm);
    COPYF(d->g_ffn[l], &a->ffn_norm, d->dm);
    COPYF(d->bqkv[l], &a->b_q, d->qd);
    COPYF(d->bqkv[l] + d->qd, &a->b_k, d->kvd);
    COPYF(d->bqkv[l] + d->qd + d->kvd, &a->b_v, d->kvd);
    QUANT(&a->Wq, d->dm, d->qd, 1, kp, d->wqkv[l], d->sqkv[l]);
    QUANT(&a->Wk, d->dm, d->kvd, 1, kp, d->wqkv[l] + (size_t)d->qd * kp, d->sqkv[l] + d->qd);
    QUANT(&a->Wv, d->dm, d->kvd, 1, kp, d->wqkv[l] + (size_t)(d->qd + d->kvd) * kp, d->sqkv[l] + d->qd + d->kvd);
    QUANT(&a->Wo, d->qd, d->dm, 1, d->kp_qd, d->wo[l], d->so[l]);
    QUANT(&a->Wgate, d->dm, d->dff, 1, kp, d->wgu[l], d->sgu[l]);
    QUANT(&a->Wup, d->dm, d->dff, 1, kp, d->wgu[l] + (size_t)d->dff * kp, d->sgu[l] + d->dff);
    QUANT(&a->Wdown, d->dff, d->dm, 1, d->kp_ff, d->wd[l], d->sd[l]);
  }
  COPYF(d->g_final, &s->final_norm, d->dm);
  QUANT(&s->lm_head, d->dm, d->vocab, 1, kp, d->head, d->head_s);
#undef QUANT
#undef COPYF
  if (qhip_sync()) die("q_llama_quantize_from");
  qhip_free(dw);
  return m;
}

// ---------------------------------------------------------------------------
// KV cache and decode
// ---------------------------------------------------------------------------
LlamaKV q_llama_kv_create(const QLlamaModel *m) { return q_llama_kv_create_mode(m, QLLAMA_MODE_EXACT); }

LlamaKV q_llama_kv_create_mode(const QLlamaModel *m, int mode) {
  LlamaKV kv;
  memset(&kv, 0, sizeof kv);
  if (mode != QLLAMA_MODE_EXACT && mode != QLLAMA_MODE_FAST) {
    fprintf(stderr, "Error: q_llama_kv_create_mode: unknown mode %d\n", mode);
    abort();
  }
  const QDev *d = (const QDev*)m->dev;
  kv.n_layers = m->n_layers; kv.max_seq = m->max_seq; kv.kv_dim = m->n_kv * m->head_dim; kv.len = 0;
  KVDev *kd = (KVDev*)calloc(1, sizeof(KVDev));
  kv.k = (float**)malloc((size_t)m->n_layers * sizeof(float*));
  kv.v = (float**)malloc((size_t)m->n_layers * sizeof(float*));
  const size_t per = (size_t)m->max_seq * kv.kv_dim;
  if (!d || !kd || !kv.k || !kv.v) { fprintf(stderr, "Error: out of memory (kv)\n"); abort(); }
  kd->kbase = (float*)qhip_malloc((size_t)m->n_layers * per * 4);
  kd->vbase = (float*)qhip_malloc((size_t)m->n_layers * per * 4);
  if (!kd->kbase || !kd->vbase) die("q_llama_kv_create");
  for (int l = 0; l < m->n_layers; l++) { kv.k[l] = kd->kbase + (size_t)l * per; kv.v[l] = kd->vbase + (size_t)l * per; }
  kd->mode = mode;
  if (mode == QLLAMA_MODE_FAST && qhip_fattn_ok(d->H, d->KVH, d->hd, d->max_seq)) {
    const size_t fb = qhip_fattn_scratch(d->H, d->KVH, d->hd, d->max_seq);
    kd->fa_scratch = qhip_malloc(fb);
    if (!kd->fa_scratch || qhip_fill_zero(kd->fa_scratch, fb) || qhip_sync()) die("q_llama_kv_create_mode");
  }
  kv.dev = kd;
  return kv;
}

struct FDev;
static void fdev_release(struct FDev *f);

void llama_kv_free(LlamaKV *kv) {
  KVDev *kd = (KVDev*)kv->dev;
  if (kd) {
    qhip_sync();
    if (kd->graph) qhip_graph_destroy(kd->graph);
    if (kd->sgraph) qhip_graph_destroy(kd->sgraph);
    qhip_free(kd->kbase); qhip_free(kd->vbase); qhip_free(kd->fa_scratch);
    if (kd->fdev) fdev_release(kd->fdev);
    free(kd);
  } else if (kv->k && kv->v) {
    for (int l = 0; l < kv->n_layers; l++) { free(kv->k[l]); free(kv->v[l]); }
  }
  free(kv->k); free(kv->v);
  kv->k = kv->v = NULL;
  kv->dev = NULL;
}

// Enqueue one token's work (llama.c:534-594): token at d_in[pos], pos = d_state[0].
// Exact mode forms every float sum in the reference's order; fast mode
// (QLLAMA_MODE_FAST) runs the split-K attention with an online-softmax merge and
// tree-ordered rmsnorm sums, with the same integer GEMV arithmetic.
static int enqueue_step(const QDev *d, const KVDev *kd) {
  const int *dpos = &d->d_state[0];
  const size_t per = (size_t)d->max_seq * d->kvd;
  const int fast = kd->mode == QLLAMA_MODE_FAST, fa = fast && kd->fa_scratch;
  const int nbo = fa ? d->H : qhip_attention_nbm(d->H, d->hd);
  const int fuse_o = qhip_gemv_fused_ok(d->kp_qd), fuse_gu = qhip_gemv_norm_ok(d->kp_dm, d->dm);
  const int nbh = fuse_gu ? qhip_gemv_norm_blocks(d->dff) : qhip_gemv_blocks(d->dff, d->kp_dm);
  int rc = qhip_embed(d->wte, d->wte_s, d->dm, d->d_in, d->d_state, d->x);
  const int ly = !fast && d->ly_ok;
  for (int l = 0; l < d->L && !rc; l++) {
    float *kc = kd->kbase + (size_t)l * per, *vc = kd->vbase + (size_t)l * per;
    if (ly) {            // QKV GEMV, RoPE, cache append, scores, softmax and PV in one launch
      rc |= qhip_attn_layer(d->x, d->g_attn[l], d->eps, d->dm, d->wqkv[l], d->sqkv[l], d->bqkv[l], d->kp_dm, kc, vc,
                            dpos, d->H, d->KVH, d->hd, d->max_seq, d->attn_scale, d->rope_cos, d->rope_sin, d->scores,
                            d->ly_scratch, d->ly_sync, d->o, d->obm);
    } else if (fuse_gu) {       // rmsnorm inside the QKV GEMV
      rc |= qhip_gemv_plain_norm(2, fast, d->x, d->dm, d->g_attn[l], d->eps, d->wqkv[l], d->sqkv[l], d->nqkv,
                                 d->kp_dm, d->qkv, d->bqkv[l]);
    } else {
      rc |= qhip_rmsnorm_quant(d->x, 1, d->dm, d->g_attn[l], d->eps, d->qa, d->kp_dm, d->as);
      rc |= qhip_gemv_dec(0, 2, d->qa, d->as, d->wqkv[l], d->sqkv[l], d->nqkv, d->kp_dm, d->qkv, d->bqkv[l], NULL, NULL);
    }
    if (!ly && fa)
      rc |= qhip_fattn(d->qkv, kc, vc, dpos, d->H, d->KVH, d->hd, d->max_seq, d->attn_scale, d->rope_cos, d->rope_sin,
                       1, kd->fa_scratch, d->o, d->obm);
    else if (!ly)
      rc |= qhip_attention_rope(d->qkv, kc, vc, dpos, d->H, d->KVH, d->hd, d->max_seq, d->attn_scale, d->rope_cos,
                                d->rope_sin, d->scores, d->o, d->obm);
    if (fuse_o) {        // o quantized inside the Wo GEMV
      rc |= qhip_gemv_resid_q(6, d->o, d->qd, d->obm, nbo, d->wo[l], d->so[l], d->dm, d->kp_qd, d->x);
    } else {
      rc |= qhip_quant_blocks(d->o, d->qd, d->obm, nbo, d->qa, d->kp_qd, d->as);
      rc |= qhip_gemv_dec(1, 6, d->qa, d->as, d->wo[l], d->so[l], d->dm, d->kp_qd, d->x, NULL, NULL, NULL);
    }
    if (fuse_gu) {       // rmsnorm inside the gate|up GEMV
      rc |= qhip_gemv_swiglu_norm(7, fast, d->x, d->dm, d->g_ffn[l], d->eps, d->wgu[l], d->sgu[l], d->dff, d->kp_dm,
                                  d->gu, d->hbm);
    } else {
      rc |= qhip_rmsnorm_quant(d->x, 1, d->dm, d->g_ffn[l], d->eps, d->qa, d->kp_dm, d->as);
      rc |= qhip_gemv_dec(2, 7, d->qa, d->as, d->wgu[l], d->sgu[l], d->dff, d->kp_dm, d->gu, NULL, d->hbm, NULL);
    }
    // Rows of up to 8192 bytes (the 1B shape): h is quantized inside the down
    // GEMV (qhip_gemv_resid_q), one kernel boundary fewer: 1B decode +5.4% end
    // to end.  Longer rows (8B, 14336 bytes) keep the separate quantization:
    // there the fused form measured 0.4-3.6% slower in every wave layout tried
    // (the prologue's 57 KB of h per block and the fewer rows in flight cost
    // more than the boundary it saves).
    if (d->kp_ff <= 8192 && qhip_gemv_fused_ok(d->kp_ff)) {
      rc |= qhip_gemv_resid_q(9, d->gu, d->dff, d->hbm, nbh, d->wd[l], d->sd[l], d->dm, d->kp_ff, d->x);
    } else {
      rc |= qhip_quant_blocks(d->gu, d->dff, d->hbm, nbh, d->qa, d->kp_ff, d->as);
      rc |= qhip_gemv_dec(1, 9, d->qa, d->as, d->wd[l], d->sd[l], d->dm, d->kp_ff, d->x, NULL, NULL, NULL);
    }
  }
  if (!rc) rc |= qhip_rmsnorm_quant(d->x, 1, d->dm, d->g_final, d->eps, d->qa, d->kp_dm, d->as);
  if (!rc) rc |= qhip_gemv_dec(3, 10, d->qa, d->as, d->head, d->head_s, d->vocab, d->kp_dm, d->logits, NULL,
                               d->amax_v, d->amax_i);
  if (!rc) rc |= qhip_argmax_final(d->amax_v, d->amax_i, qhip_gemv_blocks(d->vocab, d->kp_dm), d->d_in, d->d_state,
                                   d->d_out, d->max_seq);
  return rc;
}

static int profiling = 0;

// After a synchronization: a k_attn_layer launch whose blocks could not all be
// resident at once has set its flag (its results are not to be used).
static int layer_check(const QDev *d, const char *who) {
  if (!d->ly_ok) return 0;
  const int e = qhip_attn_layer_failed(d->ly_sync, d->KVH);
  if (!e) return 0;
  fprintf(stderr, "Error: %s: the fused attention launch %s (QLLAMA_NO_ATTN_LAYER=1 selects the separate "
          "kernels)\n", who, e == 1 ? "timed out waiting for blocks (not resident at once, or not 32 per XCD)"
                            : e == 2 ? "ran on more than eight XCDs" : "state could not be read");
  return 1;
}

// Run `n` steps: a graph replay each, or eager launches while profiling.
static int run_steps(const QDev *d, KVDev *kd, int n) {
  // QLLAMA_NO_GRAPH=1 launches each kernel directly (same kernels, same order),
  // for tools that trace kernels but not graph nodes.
  static int no_graph = -1;
  if (no_graph < 0) no_graph = getenv("QLLAMA_NO_GRAPH") != NULL;
  if (profiling || no_graph) {
    for (int i = 0; i < n; i++) if (enqueue_step(d, kd)) return 1;
    return 0;
  }
  if (!kd->graph || kd->graph_gen != d->gen) {
    if (kd->graph) { qhip_graph_destroy(kd->graph); kd->graph = NULL; }
    if (qhip_capture_begin()) return 1;
    int rc = enqueue_step(d, kd);
    void *g = NULL;
    rc = qhip_capture_end(&g) || rc;
    if (rc) { if (g) qhip_graph_destroy(g); return 1; }
    kd->graph = g;
    kd->graph_gen = d->gen;
  }
  for (int i = 0; i < n; i++) if (qhip_graph_launch(kd->graph)) return 1;
  return 0;
}

// Stage tokens ids[0..n) at positions pos..pos+n-1 and set (pos, fill_end).
static int stage_inputs(const QDev *d, int pos, const int *ids, int n) {
  int *h = d->h_stage;
  h[0] = pos; h[1] = pos + n;
  if (qhip_h2d_async(d->d_state, h, 2 * sizeof(int))) return 1;
  memcpy(h + 2, ids, (size_t)n * sizeof(int));
  return qhip_h2d_async(d->d_in + pos, h + 2, (size_t)n * sizeof(int));
}

// Host-side guards before any device work: the positions pos .. pos+n-1 must fit
// the cache (the reference leaves this to its callers, main.c:663,804) and the
// n_ids staged token ids must be in range (main.c:568 skips bad ids).
static void check_step(const QLlamaModel *m, const LlamaKV *kv, const int *ids, int n_ids, int n_pos,
                       const char *who) {
  if (!m || !m->dev || !kv || !kv->dev) { fprintf(stderr, "Error: %s: model or cache not on the GPU\n", who); abort(); }
  // a cache serves any model of its own shape (llama.c:513-526 sizes it from the
  // model); one of another shape would be indexed past its buffers
  if (((const KVDev*)kv->dev)->fdev || kv->n_layers != m->n_layers || kv->max_seq != m->max_seq ||
      kv->kv_dim != m->n_kv * m->head_dim) {
    fprintf(stderr, "Error: %s: the cache (%d layers, max_seq %d, kv_dim %d) does not fit this model "
            "(%d layers, max_seq %d, kv_dim %d)\n", who, kv->n_layers, kv->max_seq, kv->kv_dim, m->n_layers,
            m->max_seq, m->n_kv * m->head_dim);
    abort();
  }
  if (kv->len < 0 || n_pos < 0 || (long long)kv->len + n_pos > m->max_seq) {
    fprintf(stderr, "Error: %s: position %d + %d exceeds max_seq %d\n", who, kv->len, n_pos, m->max_seq);
    abort();
  }
  for (int i = 0; i < n_ids; i++)
    if (ids[i] < 0 || ids[i] >= m->vocab) {
      fprintf(stderr, "Error: %s: token id %d out of range (vocab %d)\n", who, ids[i], m->vocab);
      abort();
    }
}

void q_llama_decode_step(const QLlamaModel *m, LlamaKV *kv, int token, Tensor *logits) {
  check_step(m, kv, &token, 1, 1, "q_llama_decode_step");
  const QDev *d = (const QDev*)m->dev;
  KVDev *kd = (KVDev*)kv->dev;
  if (stage_inputs(d, kv->len, &token, 1) || run_steps(d, kd, 1) ||
      qhip_d2h_async(d->h_logits, d->logits, (size_t)d->vocab * 4) || qhip_sync() ||
      layer_check(d, "q_llama_decode_step"))
    die("q_llama_decode_step");
  memcpy(logits->data, d->h_logits, (size_t)d->vocab * 4);
  kv->len += 1;
}

// ---------------------------------------------------------------------------
// Batched prompt ingestion: every row of the prompt through each layer at once
// (MFMA GEMMs, batched RoPE, causal attention), then the final norm, head and
// argmax of the last row with the decode kernels.  Each row is computed with
// the same operations in the same order as its decode step, so the result, the
// cache and the device position state equal those of n decode steps (only the
// argmax ids of the earlier prompt rows, which nothing reads, are not written).
// ---------------------------------------------------------------------------
#define PF_MIN_ROWS 16      // shorter prompts replay the decode graph
#define PF_CLS_GEMM 14      // profiling class of the prefill GEMMs (QK_PF_GEMM)
#define PF_MAX_ROWS 2048    // rows per pass through the layers
#define PF_WORK_BYTES ((size_t)64 << 20)   // split-K partial sums (a few planes of rows x outputs)

static int pf_supported(const QDev *d) {
  const int G = d->H / d->KVH;
  return (d->hd == 128 || d->hd == 64 || d->hd == 48) && G >= 1 && G <= 8 && G * d->hd <= 1024 &&
         d->dff <= 32768;
}

static int pf_alloc(QDev *d, int rows) {
  if (d->pf_rows >= rows) return 0;
  pf_free(d);
  const size_t R = (size_t)rows;
  d->pf_x = (float*)qhip_malloc(R * d->dm * 4);
  d->pf_qkv = (float*)qhip_malloc(R * d->nqkv * 4);
  d->pf_q = (float*)qhip_malloc(R * d->qd * 4);
  d->pf_o = (float*)qhip_malloc(R * d->qd * 4);
  d->pf_h = (float*)qhip_malloc(R * d->dff * 4);
  d->pf_as = (float*)qhip_malloc(R * 4);
  d->pf_attn = (float*)qhip_malloc(qhip_pf_attention_scratch(rows, d->H, d->max_seq) * 4);
  d->pf_qa = (int8_t*)qhip_malloc(R * d->kp_max);
  d->pf_work = (int*)qhip_malloc(PF_WORK_BYTES);
  if (!d->pf_x || !d->pf_qkv || !d->pf_q || !d->pf_o || !d->pf_h || !d->pf_as || !d->pf_attn || !d->pf_qa ||
      !d->pf_work) {
    pf_free(d);
    return 1;
  }
  d->pf_rows = rows;
  return qhip_fill_zero(d->pf_qa, R * d->kp_max);
}

static int pf_run(QDev *d, const KVDev *kd, int pos, const int *ids, int n) {
  const int rows = n < PF_MAX_ROWS ? n : PF_MAX_ROWS;
  if (pf_alloc(d, rows)) return 1;
  // the stream is idle here (every entry point ends with a sync): stage the
  // prompt ids by position and the position state the final argmax advances
  int st[2] = {pos + n - 1, pos + n};
  if (qhip_h2d(d->d_in + pos, ids, (size_t)n * sizeof(int)) || qhip_h2d(d->d_state, st, sizeof st)) return 1;
  const size_t per = (size_t)d->max_seq * d->kvd;
  const int fast_attn = kd->mode == QLLAMA_MODE_FAST && qhip_pf_attention_fast_ok(d->H, d->KVH, d->hd);
  int rc = 0;
  for (int c0 = 0; c0 < n && !rc; c0 += rows) {
    const int R = n - c0 < rows ? n - c0 : rows, p0 = pos + c0;
    rc |= qhip_pf_embed(d->wte, d->wte_s, d->dm, d->d_in + p0, R, d->pf_x);
    for (int l = 0; l < d->L && !rc; l++) {
      float *kc = kd->kbase + (size_t)l * per, *vc = kd->vbase + (size_t)l * per;
      rc |= qhip_rmsnorm_quant(d->pf_x, R, d->dm, d->g_attn[l], d->eps, d->pf_qa, d->kp_dm, d->pf_as);
      rc |= qhip_gemm_i8_ws(0, PF_CLS_GEMM, d->pf_qa, d->pf_as, d->wqkv[l], d->sqkv[l], R, d->nqkv, d->kp_dm, d->pf_qkv,
                            d->nqkv, d->bqkv[l], d->pf_work, PF_WORK_BYTES);
      rc |= qhip_pf_rope_append(d->pf_qkv, R, d->H, d->KVH, d->hd, d->rope_cos, d->rope_sin, p0, d->pf_q, kc, vc,
                                d->max_seq);
      if (fast_attn)      // fast cache: MFMA attention, a tolerance path like the fast decode
        rc |= qhip_pf_attention_fast(d->pf_q, kc, vc, R, p0, d->H, d->KVH, d->hd, d->max_seq, d->attn_scale, d->pf_o);
      else
        rc |= qhip_pf_attention(d->pf_q, kc, vc, R, p0, d->H, d->KVH, d->hd, d->max_seq, d->attn_scale, d->pf_attn,
                                d->pf_o);
      rc |= qhip_quant_rows(d->pf_o, R, d->qd, d->pf_qa, d->kp_qd, d->pf_as);
      rc |= qhip_gemm_i8_ws(1, PF_CLS_GEMM, d->pf_qa, d->pf_as, d->wo[l], d->so[l], R, d->dm, d->kp_qd, d->pf_x, d->dm,
                            NULL, d->pf_work, PF_WORK_BYTES);
      rc |= qhip_rmsnorm_quant(d->pf_x, R, d->dm, d->g_ffn[l], d->eps, d->pf_qa, d->kp_dm, d->pf_as);
      rc |= qhip_gemm_i8_ws(2, PF_CLS_GEMM, d->pf_qa, d->pf_as, d->wgu[l], d->sgu[l], R, d->dff, d->kp_dm, d->pf_h, d->dff,
                            NULL, d->pf_work, PF_WORK_BYTES);
      rc |= qhip_quant_rows(d->pf_h, R, d->dff, d->pf_qa, d->kp_ff, d->pf_as);
      rc |= qhip_gemm_i8_ws(1, PF_CLS_GEMM, d->pf_qa, d->pf_as, d->wd[l], d->sd[l], R, d->dm, d->kp_ff, d->pf_x, d->dm,
                            NULL, d->pf_work, PF_WORK_BYTES);
    }
    if (!rc && c0 + R == n) {       // last row: final norm, head, argmax (llama.c:592-593, sampler.c:36-49)
      const float *xl = d->pf_x + (size_t)(R - 1) * d->dm;
      rc |= qhip_rmsnorm_quant(xl, 1, d->dm, d->g_final, d->eps, d->qa, d->kp_dm, d->as);
      rc |= qhip_gemv_dec(3, 10, d->qa, d->as, d->head, d->head_s, d->vocab, d->kp_dm, d->logits, NULL, d->amax_v,
                          d->amax_i);
      rc |= qhip_argmax_final(d->amax_v, d->amax_i, qhip_gemv_blocks(d->vocab, d->kp_dm), d->d_in, d->d_state,
                              d->d_out, d->max_seq);
    }
  }
  return rc;
}

int q_llama_prefill(const QLlamaModel *m, LlamaKV *kv, const int *ids, int n, Tensor *logits) {
  if (n <= 0) return 0;
  check_step(m, kv, ids, n, n, "q_llama_prefill");
  QDev *d = (QDev*)m->dev;
  KVDev *kd = (KVDev*)kv->dev;
  static int no_batch = -1;     // QLLAMA_PREFILL_STEPS=1: replay decode steps instead (same results)
  if (no_batch < 0) no_batch = getenv("QLLAMA_PREFILL_STEPS") != NULL;
  if (n >= PF_MIN_ROWS && pf_supported(d) && !no_batch) {
    if (pf_run(d, kd, kv->len, ids, n)) return 1;
  } else {
    if (stage_inputs(d, kv->len, ids, n) || run_steps(d, kd, n)) return 1;
  }
  if (logits && qhip_d2h_async(d->h_logits, d->logits, (size_t)d->vocab * 4)) return 1;
  if (qhip_sync() || layer_check(d, "q_llama_prefill")) return 1;
  if (logits) memcpy(logits->data, d->h_logits, (size_t)d->vocab * 4);
  kv->len += n;
  return 0;
}

int q_llama_generate_greedy(const QLlamaModel *m, LlamaKV *kv, int token, int n_steps, int *out) {
  if (n_steps <= 0) return 0;
  check_step(m, kv, &token, 1, n_steps, "q_llama_generate_greedy");
  const QDev *d = (const QDev*)m->dev;
  KVDev *kd = (KVDev*)kv->dev;
  const int pos = kv->len;
  if (stage_inputs(d, pos, &token, 1) || run_steps(d, kd, n_steps)) return 1;
  if (out && qhip_d2h_async(d->h_stage, d->d_out + pos, (size_t)n_steps * sizeof(int))) return 1;
  if (qhip_sync() || layer_check(d, "q_llama_generate_greedy")) return 1;
  if (out) memcpy(out, d->h_stage, (size_t)n_steps * sizeof(int));
  kv->len += n_steps;
  return 0;
}

// ---------------------------------------------------------------------------
// fp32 (LLMA) decode path: llama_kv_create / llama_decode_step of llama.c:275-362
// on the GPU.  The caller keeps the reference's host LlamaModel; the first cache
// created for it uploads a device copy (looked up by the model's weight
// pointers), which lives as long as a cache of it does.  Weights are read at
// that point: host changes made afterwards are seen by caches created later.
// Device layout: every matrix keeps the reference's (K, N) row-major order (the
// GEMV reads a row's columns contiguously); Wq|Wk|Wv and Wgate|Wup are joined
// column-wise into one matrix each, so one launch serves each pair.
// ---------------------------------------------------------------------------
typedef struct FDev {
  const void *key_wte, *key_blocks;      // identity of the host model
  uint64_t gen;                          // identifies this device copy to the graphs of its caches
  int refs;
  int vocab, dm, L, H, KVH, hd, dff, max_seq, qd, kvd, nqkv;
  float eps, attn_scale;
  uint8_t *blob;
  float **wqkv, **bqkv, **wo, **wgu, **wd, **g_attn, **g_ffn;
  float *wte, *head, *g_final, *rope_cos, *rope_sin;
  float *x, *xn, *qkv, *o, *gu, *h, *logits, *scores;
  int *d_state, *d_in;
  int *h_stage;
} FDev;

#define FDEV_MAX 16
static FDev *g_fdev[FDEV_MAX];

static void fdev_free(FDev *f) {
  if (!f) return;
  qhip_free(f->blob);
  qhip_host_free(f->h_stage);
  free(f->wqkv); free(f->bqkv); free(f->wo); free(f->wgu); free(f->wd); free(f->g_attn); free(f->g_ffn);
  free(f);
}

static void fdev_release(FDev *f) {
  if (--f->refs > 0) return;
  for (int i = 0; i < FDEV_MAX; i++) if (g_fdev[i] == f) g_fdev[i] = NULL;
  qhip_sync();
  fdev_free(f);
}

static FDev *fdev_find(const LlamaModel *m) {
  for (int i = 0; i < FDEV_MAX; i++)
    if (g_fdev[i] && g_fdev[i]->key_wte == (const void*)m->wte.data && g_fdev[i]->key_blocks == (const void*)m->blocks)
      return g_fdev[i];
  return NULL;
}

static FDev *fdev_upload(const LlamaModel *m) {
  const int32_t cfg[8] = {m->vocab, m->d_model, m->n_layers, m->n_heads, m->n_kv, m->head_dim, m->d_ff, m->max_seq};
  if (!config_valid(cfg) || !config_supported(cfg) || m->d_model > qhip_gemv_f32_max_k() ||
      m->n_heads * m->head_dim > qhip_gemv_f32_max_k() || m->d_ff > qhip_gemv_f32_max_k()) {
    fprintf(stderr, "Error: llama_kv_create: config not supported by the GPU fp32 path\n");
    return NULL;
  }
  if (qhip_init() != 0) { fprintf(stderr, "Error: no usable GPU: %s\n", qhip_last_error()); return NULL; }
  int slot = -1;
  for (int i = 0; i < FDEV_MAX && slot < 0; i++) if (!g_fdev[i]) slot = i;
  if (slot < 0) { fprintf(stderr, "Error: llama_kv_create: too many fp32 models on the GPU\n"); return NULL; }
  FDev *f = (FDev*)calloc(1, sizeof(FDev));
  if (!f) return NULL;
  f->key_wte = m->wte.data; f->key_blocks = m->blocks;
  f->gen = next_generation();
  f->vocab = m->vocab; f->dm = m->d_model; f->L = m->n_layers; f->H = m->n_heads; f->KVH = m->n_kv;
  f->hd = m->head_dim; f->dff = m->d_ff; f->max_seq = m->max_seq; f->eps = m->eps;
  f->qd = f->H * f->hd; f->kvd = f->KVH * f->hd; f->nqkv = f->qd + 2 * f->kvd;
  f->attn_scale = 1.0f / sqrtf((float)f->hd);                      // llama.c:301
  const int L = f->L;
  const size_t dm = (size_t)f->dm, qd = (size_t)f->qd, kvd = (size_t)f->kvd, nqkv = (size_t)f->nqkv;
  const size_t dff = (size_t)f->dff, V = (size_t)f->vocab;
  f->wqkv = calloc(L, sizeof(float*)); f->bqkv = calloc(L, sizeof(float*)); f->wo = calloc(L, sizeof(float*));
  f->wgu = calloc(L, sizeof(float*)); f->wd = calloc(L, sizeof(float*)); f->g_attn = calloc(L, sizeof(float*));
  f->g_ffn = calloc(L, sizeof(float*));
  if (!f->wqkv || !f->bqkv || !f->wo || !f->wgu || !f->wd || !f->g_attn || !f->g_ffn) { fdev_free(f); return NULL; }
  size_t off = 0, *lo = (size_t*)calloc((size_t)L * 7, sizeof(size_t));
  if (!lo) { fdev_free(f); return NULL; }
#define FTAKE(n) (off += al256((n) * 4), off - al256((n) * 4))
#define PAN(K, N) qhip_panels_f32_size((int)(K), (int)(N))
  for (int l = 0; l < L; l++) {
    lo[l * 7 + 0] = FTAKE(PAN(dm, nqkv)); lo[l * 7 + 1] = FTAKE(nqkv); lo[l * 7 + 2] = FTAKE(PAN(qd, dm));
    lo[l * 7 + 3] = FTAKE(PAN(dm, 2 * dff)); lo[l * 7 + 4] = FTAKE(PAN(dff, dm));
    lo[l * 7 + 5] = FTAKE(dm); lo[l * 7 + 6] = FTAKE(dm);
  }
  const size_t o_wte = FTAKE(V * dm), o_head = FTAKE(PAN(dm, V)), o_gf = FTAKE(dm);
#undef PAN
  const size_t o_cos = FTAKE((size_t)f->max_seq * (f->hd / 2)), o_sin = FTAKE((size_t)f->max_seq * (f->hd / 2));
  const size_t o_x = FTAKE(dm), o_xn = FTAKE(dm), o_qkv = FTAKE(nqkv), o_o = FTAKE(qd), o_gu = FTAKE(2 * dff);
  const size_t o_h = FTAKE(dff), o_lg = FTAKE(V), o_sc = FTAKE(qhip_attention_scratch(f->H, f->max_seq));
  const size_t o_st = FTAKE(16), o_in = FTAKE((size_t)f->max_seq + 1);
#undef FTAKE
  size_t big = dm * V;                                   // row-major staging of the largest matrix
  if (dm * 2 * dff > big) big = dm * 2 * dff;
  if (dm * nqkv > big) big = dm * nqkv;
  if (qd * dm > big) big = qd * dm;
  f->blob = (uint8_t*)qhip_malloc(off);
  f->h_stage = (int*)qhip_host_alloc(64);
  float *tmp = (float*)qhip_malloc(big * 4);
  size_t big2 = dm * (qd > dff ? qd : dff);                // one part of a joined matrix
  float *tmp2 = (float*)qhip_malloc(big2 * 4);
  if (!f->blob || !f->h_stage || !tmp || !tmp2) {
    fprintf(stderr, "Error: device allocation of %zu bytes failed: %s\n", off, qhip_last_error());
    qhip_free(tmp); qhip_free(tmp2); free(lo); fdev_free(f); return NULL;
  }
  uint8_t *b = f->blob;
  for (int l = 0; l < L; l++) {
    f->wqkv[l] = (float*)(b + lo[l * 7 + 0]); f->bqkv[l] = (float*)(b + lo[l * 7 + 1]);
    f->wo[l] = (float*)(b + lo[l * 7 + 2]); f->wgu[l] = (float*)(b + lo[l * 7 + 3]);
    f->wd[l] = (float*)(b + lo[l * 7 + 4]); f->g_attn[l] = (float*)(b + lo[l * 7 + 5]);
    f->g_ffn[l] = (float*)(b + lo[l * 7 + 6]);
  }
  free(lo);
  f->wte = (float*)(b + o_wte); f->head = (float*)(b + o_head); f->g_final = (float*)(b + o_gf);
  f->rope_cos = (float*)(b + o_cos); f->rope_sin = (float*)(b + o_sin);
  f->x = (float*)(b + o_x); f->xn = (float*)(b + o_xn); f->qkv = (float*)(b + o_qkv); f->o = (float*)(b + o_o);
  f->gu = (float*)(b + o_gu); f->h = (float*)(b + o_h); f->logits = (float*)(b + o_lg);
  f->scores = (float*)(b + o_sc); f->d_state = (int*)(b + o_st); f->d_in = (int*)(b + o_in);
  int rc = qhip_upload_begin((size_t)32 << 20);
  // every matrix is staged row-major in tmp, then rewritten in the GEMV's panel
  // layout; two matrices (K, n1), (K, n2) are first joined column-wise in tmp
#define PART(src, K, ld, coloff, n) \
  (qhip_upload((float*)tmp2, (src)->data, (size_t)(K) * (n) * 4) || \
   qhip_copy2d_d2d(tmp + (coloff), (ld) * 4, tmp2, (n) * 4, (n) * 4, (K)))
  rc = rc || qhip_upload(f->wte, m->wte.data, V * dm * 4) || qhip_upload(f->g_final, m->final_norm.data, dm * 4) ||
       qhip_upload(tmp, m->lm_head.data, dm * V * 4) || qhip_to_panels_f32(tmp, (int)dm, (int)V, f->head);
  for (int l = 0; l < L && !rc; l++) {
    const LlamaBlock *a = &m->blocks[l];
    rc = PART(&a->Wq, dm, nqkv, 0, qd) || PART(&a->Wk, dm, nqkv, qd, kvd) || PART(&a->Wv, dm, nqkv, qd + kvd, kvd) ||
         qhip_to_panels_f32(tmp, (int)dm, (int)nqkv, f->wqkv[l]) ||
         PART(&a->Wgate, dm, 2 * dff, 0, dff) || PART(&a->Wup, dm, 2 * dff, dff, dff) ||
         qhip_to_panels_f32(tmp, (int)dm, (int)(2 * dff), f->wgu[l]) ||
         qhip_upload(tmp, a->Wo.data, qd * dm * 4) || qhip_to_panels_f32(tmp, (int)qd, (int)dm, f->wo[l]) ||
         qhip_upload(tmp, a->Wdown.data, dff * dm * 4) || qhip_to_panels_f32(tmp, (int)dff, (int)dm, f->wd[l]) ||
         qhip_upload(f->bqkv[l], a->b_q.data, qd * 4) || qhip_upload(f->bqkv[l] + qd, a->b_k.data, kvd * 4) ||
         qhip_upload(f->bqkv[l] + qd + kvd, a->b_v.data, kvd * 4) ||
         qhip_upload(f->g_attn[l], a->attn_norm.data, dm * 4) || qhip_upload(f->g_ffn[l], a->ffn_norm.data, dm * 4);
  }
#undef PART
  if (qhip_upload_end()) rc = 1;
  qhip_free(tmp); qhip_free(tmp2);
  if (!rc) rc = rope_upload(f->rope_cos, f->rope_sin, f->max_seq, f->hd, m->rope_base) ||
                qhip_fill_zero(f->d_in, ((size_t)f->max_seq + 1) * 4) || qhip_fill_zero(f->d_state, 64) ||
                qhip_sync();
  if (rc) {
    fprintf(stderr, "Error: upload of the fp32 model failed: %s\n", qhip_last_error());
    fdev_free(f); return NULL;
  }
  g_fdev[slot] = f;
  return f;
}

// llama.c:296-362 for the token at d_in[d_state[0]]
static int enqueue_step_f32(const FDev *f, const KVDev *kd) {
  const size_t per = (size_t)f->max_seq * f->kvd;
  int rc = qhip_embed_f32(f->wte, f->dm, f->d_in, f->d_state, f->x);
  for (int l = 0; l < f->L && !rc; l++) {
    float *kc = kd->kbase + (size_t)l * per, *vc = kd->vbase + (size_t)l * per;
    rc |= qhip_rmsnorm_f32(f->x, f->dm, f->g_attn[l], f->eps, f->xn);
    rc |= qhip_gemv_f32(0, 2, f->xn, f->dm, f->wqkv[l], f->nqkv, f->qkv, f->bqkv[l]);
    rc |= qhip_attention_rope(f->qkv, kc, vc, f->d_state, f->H, f->KVH, f->hd, f->max_seq, f->attn_scale,
                              f->rope_cos, f->rope_sin, f->scores, f->o, NULL);
    rc |= qhip_gemv_f32(1, 6, f->o, f->qd, f->wo[l], f->dm, f->x, NULL);
    rc |= qhip_rmsnorm_f32(f->x, f->dm, f->g_ffn[l], f->eps, f->xn);
    rc |= qhip_gemv_f32(0, 7, f->xn, f->dm, f->wgu[l], 2 * f->dff, f->gu, NULL);
    rc |= qhip_swiglu_f32(f->gu, f->dff, f->h);
    rc |= qhip_gemv_f32(1, 9, f->h, f->dff, f->wd[l], f->dm, f->x, NULL);
  }
  if (!rc) rc |= qhip_rmsnorm_f32(f->x, f->dm, f->g_final, f->eps, f->xn);
  if (!rc) rc |= qhip_gemv_f32(0, 10, f->xn, f->dm, f->head, f->vocab, f->logits, NULL);
  return rc;
}

// llama.c:275-288: a device cache; the model's device copy is made (or shared)
LlamaKV llama_kv_create(const LlamaModel *m) {
  LlamaKV kv;
  memset(&kv, 0, sizeof kv);
  FDev *f = fdev_find(m);
  if (!f) f = fdev_upload(m);
  if (!f) abort();
  KVDev *kd = (KVDev*)calloc(1, sizeof(KVDev));
  kv.n_layers = m->n_layers; kv.max_seq = m->max_seq; kv.kv_dim = m->n_kv * m->head_dim; kv.len = 0;
  kv.k = (float**)malloc((size_t)m->n_layers * sizeof(float*));
  kv.v = (float**)malloc((size_t)m->n_layers * sizeof(float*));
  const size_t per = (size_t)m->max_seq * kv.kv_dim;
  if (!kd || !kv.k || !kv.v) { fprintf(stderr, "Error: out of memory (kv)\n"); abort(); }
  kd->kbase = (float*)qhip_malloc((size_t)m->n_layers * per * 4);
  kd->vbase = (float*)qhip_malloc((size_t)m->n_layers * per * 4);
  if (!kd->kbase || !kd->vbase) die("llama_kv_create");
  for (int l = 0; l < m->n_layers; l++) { kv.k[l] = kd->kbase + (size_t)l * per; kv.v[l] = kd->vbase + (size_t)l * per; }
  kd->fdev = f;
  f->refs++;
  kv.dev = kd;
  return kv;
}

// llama.c:296-362 on the GPU; logits (1, vocab) in host memory.
void llama_decode_step(const LlamaModel *m, LlamaKV *kv, int token, Tensor *logits) {
  KVDev *kd = kv ? (KVDev*)kv->dev : NULL;
  FDev *f = kd ? kd->fdev : NULL;
  if (!m || !f || f != fdev_find(m)) {
    fprintf(stderr, "Error: llama_decode_step: the cache was not made by llama_kv_create for this model\n");
    abort();
  }
  if (kv->len < 0 || kv->len >= f->max_seq || token < 0 || token >= f->vocab) {
    fprintf(stderr, "Error: llama_decode_step: position %d / token %d out of range\n", kv->len, token);
    abort();
  }
  int *h = f->h_stage;
  h[0] = kv->len; h[1] = kv->len + 1; h[2] = token;
  int rc = qhip_h2d_async(f->d_state, h, 2 * sizeof(int)) || qhip_h2d_async(f->d_in + kv->len, h + 2, sizeof(int));
  if (!rc) {
    if (profiling || getenv("QLLAMA_NO_GRAPH")) {
      rc = enqueue_step_f32(f, kd);
    } else {
      if (!kd->graph || kd->graph_gen != f->gen) {
        if (kd->graph) { qhip_graph_destroy(kd->graph); kd->graph = NULL; }
        void *g = NULL;
        rc = qhip_capture_begin();
        if (!rc) {
          const int e = enqueue_step_f32(f, kd);
          rc = qhip_capture_end(&g) || e;
        }
        if (!rc) { kd->graph = g; kd->graph_gen = f->gen; }
        else if (g) qhip_graph_destroy(g);
      }
      if (!rc) rc = qhip_graph_launch(kd->graph);
    }
  }
  if (rc || qhip_d2h_async(logits->data, f->logits, (size_t)f->vocab * 4) || qhip_sync()) die("llama_decode_step");
  kv->len += 1;
}

// ---------------------------------------------------------------------------
// llama.c:167-186: logits (seq_len, vocab) for every position of ids, batched.
// Row i of the reference's forward is bit-identical to its decode step of ids[i]
// at position i after ids[0..i-1] (selftest.c:1144-1178 checks this, and so do
// the fixtures), and the device pieces keep that: the GEMMs sum each element in
// k order as the decode GEMV does, and the attention and RoPE are the int8
// prefill's, which equal the decode step's.  The forward runs layer by layer
// over all rows, a layer's rows in passes of at most FWD_ROWS; each pass appends
// its keys and values to the layer's cache (stride seq_len) before its attention
// reads them, so every row sees all earlier rows, and one cache serves every
// layer.  Head layouts the prefill attention does not take replay decode steps
// on a cache of their own (then seq_len <= max_seq).
// ---------------------------------------------------------------------------
#define FWD_ROWS 2048        // rows per pass through a layer
#define FWD_MAX_ROWS 16384   // the prefill attention's largest cache stride
#define FWD_CLS 14           // profiling class of the forward's GEMMs (QK_PF_GEMM)

static int fwd_supported(const FDev *f) {
  const int G = f->H / f->KVH;
  return (f->hd == 128 || f->hd == 64 || f->hd == 48) && G >= 1 && G <= 8 && G * f->hd <= 1024;
}

static int fwd_run(const FDev *f, float rope_base, const int *ids, int n, float *logits) {
  const int R = n < FWD_ROWS ? n : FWD_ROWS, half = f->hd / 2, own_rope = n > f->max_seq;
  const size_t dm = (size_t)f->dm, V = (size_t)f->vocab, per = (size_t)f->KVH * n * f->hd;
  size_t off = 0;
#define FTAKE(nf) (off += al256((size_t)(nf) * 4), off - al256((size_t)(nf) * 4))
  const size_t o_ids = FTAKE(n), o_x = FTAKE((size_t)n * dm), o_xn = FTAKE(R * dm), o_qkv = FTAKE((size_t)R * f->nqkv);
  const size_t o_q = FTAKE((size_t)R * f->qd), o_o = FTAKE((size_t)R * f->qd), o_gu = FTAKE((size_t)R * 2 * f->dff);
  const size_t o_h = FTAKE((size_t)R * f->dff), o_lg = FTAKE(R * V), o_kc = FTAKE(per), o_vc = FTAKE(per);
  const size_t o_ws = FTAKE(qhip_pf_attention_scratch(R, f->H, n));
  const size_t o_cos = FTAKE(own_rope ? (size_t)n * half : 1), o_sin = FTAKE(own_rope ? (size_t)n * half : 1);
#undef FTAKE
  uint8_t *b = (uint8_t*)qhip_malloc(off);
  if (!b) return 1;
  int *d_ids = (int*)(b + o_ids);
  float *X = (float*)(b + o_x), *xn = (float*)(b + o_xn), *qkv = (float*)(b + o_qkv), *q = (float*)(b + o_q);
  float *o = (float*)(b + o_o), *gu = (float*)(b + o_gu), *h = (float*)(b + o_h), *lg = (float*)(b + o_lg);
  float *kc = (float*)(b + o_kc), *vc = (float*)(b + o_vc), *ws = (float*)(b + o_ws);
  const float *cs = f->rope_cos, *sn = f->rope_sin;
  int rc = qhip_h2d(d_ids, ids, (size_t)n * sizeof(int));
  if (!rc && own_rope) {        // positions past max_seq: tables of n rows (rope.c:58-61)
    rc = rope_upload((float*)(b + o_cos), (float*)(b + o_sin), n, f->hd, rope_base);
    cs = (const float*)(b + o_cos); sn = (const float*)(b + o_sin);
  }
  if (!rc) rc = qhip_embed_f32_rows(f->wte, f->dm, d_ids, n, X);
  for (int l = 0; l < f->L && !rc; l++)
    for (int c0 = 0; c0 < n && !rc; c0 += R) {
      const int r = n - c0 < R ? n - c0 : R;
      float *Xc = X + (size_t)c0 * dm;
      rc |= qhip_rmsnorm_f32_rows(Xc, r, f->dm, f->g_attn[l], f->eps, xn);
      rc |= qhip_gemm_f32(0, FWD_CLS, xn, r, f->dm, f->wqkv[l], f->nqkv, qkv, f->bqkv[l]);
      rc |= qhip_pf_rope_append(qkv, r, f->H, f->KVH, f->hd, cs, sn, c0, q, kc, vc, n);
      rc |= qhip_pf_attention(q, kc, vc, r, c0, f->H, f->KVH, f->hd, n, f->attn_scale, ws, o);
      rc |= qhip_gemm_f32(1, FWD_CLS, o, r, f->qd, f->wo[l], f->dm, Xc, NULL);
      rc |= qhip_rmsnorm_f32_rows(Xc, r, f->dm, f->g_ffn[l], f->eps, xn);
      rc |= qhip_gemm_f32(0, FWD_CLS, xn, r, f->dm, f->wgu[l], 2 * f->dff, gu, NULL);
      rc |= qhip_swiglu_f32_rows(gu, r, f->dff, h);
      rc |= qhip_gemm_f32(1, FWD_CLS, h, r, f->dff, f->wd[l], f->dm, Xc, NULL);
    }
  for (int c0 = 0; c0 < n && !rc; c0 += R) {   // final norm and head (llama.c:182-183)
    const int r = n - c0 < R ? n - c0 : R;
    rc |= qhip_rmsnorm_f32_rows(X + (size_t)c0 * dm, r, f->dm, f->g_final, f->eps, xn);
    rc |= qhip_gemm_f32(0, FWD_CLS, xn, r, f->dm, f->head, f->vocab, lg, NULL);
    rc = rc || qhip_d2h_async(logits + (size_t)c0 * V, lg, (size_t)r * V * 4) || qhip_sync();
  }
  if (qhip_sync()) rc = 1;
  qhip_free(b);
  return rc;
}

static void fwd_steps(const LlamaModel *m, const int *ids, int seq_len, Tensor *logits) {
  LlamaKV kv = llama_kv_create(m);
  int shape[2] = {1, m->vocab};
  for (int i = 0; i < seq_len; i++) {
    Tensor row = *logits;
    row.data = logits->data + (size_t)i * m->vocab;
    row.shape = shape; row.ndim = 2; row.size = (size_t)m->vocab;
    llama_decode_step(m, &kv, ids[i], &row);
  }
  llama_kv_free(&kv);
}

void llama_model_forward(const LlamaModel *m, const int *ids, int seq_len, Tensor *logits) {
  if (!m || !ids || !logits || !logits->data || seq_len <= 0) {
    fprintf(stderr, "Error: llama_model_forward: needs seq_len >= 1, ids and a (seq_len, vocab) tensor\n");
    abort();
  }
  for (int i = 0; i < seq_len; i++)
    if (ids[i] < 0 || ids[i] >= m->vocab) {
      fprintf(stderr, "Error: llama_model_forward: token %d at %d out of range\n", ids[i], i);
      abort();
    }
  FDev *f = fdev_find(m);
  if (!f) f = fdev_upload(m);
  if (!f) abort();
  f->refs++;                          // held for the call (a cache freed meanwhile keeps it)
  // QLLAMA_FORWARD_STEPS=1: replay decode steps instead (same results)
  const int batched = fwd_supported(f) && !getenv("QLLAMA_FORWARD_STEPS");
  if (batched && seq_len <= FWD_MAX_ROWS) {
    if (fwd_run(f, m->rope_base, ids, seq_len, logits->data)) die("llama_model_forward");
  } else if (seq_len <= m->max_seq) {
    fwd_steps(m, ids, seq_len, logits);
  } else {
    fprintf(stderr, "Error: llama_model_forward: seq_len %d is above %d for this model\n", seq_len,
            batched ? FWD_MAX_ROWS : m->max_seq);
    abort();
  }
  fdev_release(f);
}

// ---------------------------------------------------------------------------
// Sampling (sampler.h).  The RNG is the reference's host xorshift64; the
// sampling arithmetic runs on the device (k_sample.hip), which also holds the
// RNG state inside q_llama_generate.
// ---------------------------------------------------------------------------
Rng rng_create(unsigned long long seed) {            // sampler.c:24-29
  Rng r;
  r.state = seed ? seed : 0x9E3779B97F4A7C15ULL;      // the all-zero state is a fixed point
  return r;
}

float rng_uniform(Rng *r) {                           // sampler.c:31-45
  unsigned long long x = r->state;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  r->state = x;
  return (float)((x >> 11) * (1.0 / 9007199254740992.0));
}

// Process-wide sampler buffers, grown to the largest vocabulary seen.
typedef struct {
  int V;
  float *row;                   // device copy of a host logits row
  void *scratch;                // qhip_sample_scratch(V)
  size_t bytes;
  unsigned long long *rng;      // device RNG state, then the token (tok)
  int *tok;
  unsigned long long *h;        // pinned: [0] RNG state, [1] token
  uint64_t gen;                 // new generation whenever the device buffers are reallocated
} SmpBuf;
static SmpBuf g_smp;

static int smp_reserve(int V) {
  if (g_smp.scratch && g_smp.V >= V) return 0;
  if (qhip_init()) return 1;
  qhip_sync();
  qhip_free(g_smp.row); qhip_free(g_smp.scratch); qhip_free(g_smp.rng);
  g_smp.row = NULL; g_smp.scratch = NULL; g_smp.rng = NULL; g_smp.tok = NULL; g_smp.V = 0;
  g_smp.bytes = qhip_sample_scratch(V);
  g_smp.row = (float*)qhip_malloc((size_t)V * 4);
  g_smp.scratch = qhip_malloc(g_smp.bytes);
  g_smp.rng = (unsigned long long*)qhip_malloc(256);
  if (!g_smp.h) g_smp.h = (unsigned long long*)qhip_host_alloc(2 * sizeof(unsigned long long));
  if (!g_smp.row || !g_smp.scratch || !g_smp.rng || !g_smp.h) return 1;
  g_smp.tok = (int*)(g_smp.rng + 1);
  g_smp.V = V;
  g_smp.gen = next_generation();
  return 0;
}

static int smp_row(const Tensor *logits, int row, int *V) {
  if (!logits || !logits->data || !logits->shape || logits->ndim < 2 || row < 0 || row >= logits->shape[0] ||
      logits->shape[1] <= 0) {
    fprintf(stderr, "Error: sample: logits must be a (rows, vocab) host tensor and row in range\n");
    abort();
  }
  *V = logits->shape[1];
  if (smp_reserve(*V)) return 1;
  return qhip_h2d(g_smp.row, logits->data + (size_t)row * *V, (size_t)*V * 4);
}

int sample_argmax(const Tensor *logits, int row) {
  int V = 0;
  if (smp_row(logits, row, &V) || qhip_argmax_row(g_smp.row, V, g_smp.tok, NULL, NULL, NULL, 0) ||
      qhip_d2h_async(&g_smp.h[1], g_smp.tok, sizeof(int)) || qhip_sync())
    die("sample_argmax");
  int t;
  memcpy(&t, &g_smp.h[1], sizeof t);
  return t;
}

int sample_token(const Tensor *logits, int row, float temperature, int top_k, float top_p, Rng *rng) {
  if (temperature <= 0.0f) return sample_argmax(logits, row);     // greedy, RNG untouched
  int V = 0;
  if (smp_row(logits, row, &V)) die("sample_token");
  g_smp.h[0] = rng->state;
  if (qhip_h2d_async(g_smp.rng, &g_smp.h[0], 8) ||
      qhip_sample(g_smp.row, V, temperature, top_k, top_p, g_smp.scratch, g_smp.bytes, g_smp.rng, g_smp.tok, NULL,
                  NULL, NULL, 0) ||
      qhip_d2h_async(&g_smp.h[0], g_smp.rng, 16) || qhip_sync())
    die("sample_token");
  rng->state = g_smp.h[0];
  int t;
  memcpy(&t, &g_smp.h[1], sizeof t);
  return t;
}

// One sampled token: the sampler writes it as the input of position d_state[0],
// then the decode step runs it.
static int enqueue_sampled(const QDev *d, const KVDev *kd, float temperature, int top_k, float top_p) {
  const int rc = temperature > 0.0f
      ? qhip_sample(d->logits, d->vocab, temperature, top_k, top_p, g_smp.scratch, g_smp.bytes, g_smp.rng,
                    g_smp.tok, d->d_in, d->d_state, d->d_out, d->max_seq)
      : qhip_argmax_row(d->logits, d->vocab, g_smp.tok, d->d_in, d->d_state, d->d_out, d->max_seq);
  return rc || enqueue_step(d, kd);
}

// n sampled tokens: one graph replay each (every launch of the step, the
// sampler's sort included, is this library's own), or eager launches while
// profiling.
static int run_sampled_steps(const QDev *d, KVDev *kd, int n, float temperature, int top_k, float top_p) {
  if (profiling || getenv("QLLAMA_NO_GRAPH")) {
    for (int i = 0; i < n; i++) if (enqueue_sampled(d, kd, temperature, top_k, top_p)) return 1;
    return 0;
  }
  if (!kd->sgraph || kd->sgraph_gen != d->gen || kd->sgraph_smp_gen != g_smp.gen ||
      kd->sg_t != temperature || kd->sg_k != top_k || kd->sg_p != top_p) {
    if (kd->sgraph) { qhip_graph_destroy(kd->sgraph); kd->sgraph = NULL; }
    if (qhip_capture_begin()) return 1;
    int rc = enqueue_sampled(d, kd, temperature, top_k, top_p);
    void *g = NULL;
    rc = qhip_capture_end(&g) || rc;
    if (rc) { if (g) qhip_graph_destroy(g); return 1; }
    kd->sgraph = g;
    kd->sgraph_gen = d->gen; kd->sgraph_smp_gen = g_smp.gen;
    kd->sg_t = temperature; kd->sg_k = top_k; kd->sg_p = top_p;
  }
  for (int i = 0; i < n; i++) if (qhip_graph_launch(kd->sgraph)) return 1;
  return 0;
}

int q_llama_generate(const QLlamaModel *m, LlamaKV *kv, int n_steps, float temperature, int top_k, float top_p,
                     Rng *rng, int *out) {
  if (n_steps <= 0) return 0;
  check_step(m, kv, NULL, 0, n_steps, "q_llama_generate");
  if (kv->len < 1 || !rng) {
    fprintf(stderr, "Error: q_llama_generate: needs a processed token (kv->len >= 1) and an Rng\n");
    return 1;
  }
  const QDev *d = (const QDev*)m->dev;
  KVDev *kd = (KVDev*)kv->dev;
  if (smp_reserve(d->vocab)) return 1;
  const int pos = kv->len;
  // position state: the next input goes to pos, and every position from pos on
  // takes the sampled token
  d->h_stage[0] = pos; d->h_stage[1] = pos;
  g_smp.h[0] = rng->state;
  if (qhip_h2d_async(d->d_state, d->h_stage, 2 * sizeof(int)) || qhip_h2d_async(g_smp.rng, &g_smp.h[0], 8)) return 1;
  if (run_sampled_steps(d, kd, n_steps, temperature, top_k, top_p)) return 1;
  if (qhip_d2h_async(g_smp.h, g_smp.rng, 8)) return 1;
  if (out && qhip_d2h_async(d->h_stage, d->d_out + pos - 1, (size_t)n_steps * sizeof(int))) return 1;
  if (qhip_sync() || layer_check(d, "q_llama_generate")) return 1;
  if (out) memcpy(out, d->h_stage, (size_t)n_steps * sizeof(int));
  rng->state = g_smp.h[0];
  kv->len += n_steps;
  return 0;
}

// ---------------------------------------------------------------------------
// quant.h API on device QTensors
// ---------------------------------------------------------------------------
QTensor qtensor_create(int rows, int cols) {
  QTensor t;
  memset(&t, 0, sizeof t);
  if (qhip_init()) die("qtensor_create");
  t.rows = rows; t.cols = cols; t.layout = QT_LAYOUT_NK; t.kpad = pad16(rows);
  t.q = (signed char*)qhip_malloc((size_t)cols * t.kpad);
  t.scale = (float*)qhip_malloc((size_t)cols * 4);
  if (!t.q || !t.scale || qhip_fill_zero(t.q, (size_t)cols * t.kpad)) die("qtensor_create");
  return t;
}

void qtensor_free(QTensor *t) {
  qhip_sync();
  qhip_free(t->q); qhip_free(t->scale);
  t->q = NULL; t->scale = NULL;
}

void qtensor_quantize(QTensor *t, const float *w) {
  const size_t n = (size_t)t->rows * t->cols;
  float *dw = (float*)qhip_malloc(n * 4);
  if (!dw || qhip_h2d(dw, w, n * 4) ||
      qhip_quantize_percol(dw, t->rows, t->cols, t->layout == QT_LAYOUT_NK, t->kpad, (int8_t*)t->q, t->scale) ||
      qhip_sync())
    die("qtensor_quantize");
  qhip_free(dw);
}

// qmatmul's device workspace (A, C, the quantized rows and their scales, and an
// NK copy of a row-major weight), grown to the largest call and kept, so calls
// after the first of a size allocate nothing.
static struct { uint8_t *p; size_t bytes; } g_qmm;

static uint8_t *qmm_workspace(size_t bytes) {
  if (g_qmm.bytes >= bytes) return g_qmm.p;
  qhip_sync();
  qhip_free(g_qmm.p);
  g_qmm.p = (uint8_t*)qhip_malloc(bytes);
  g_qmm.bytes = g_qmm.p ? bytes : 0;
  return g_qmm.p;
}

void qmatmul(const Tensor *A, const QTensor *W, Tensor *C) {
  const int M = A->shape[0], K = W->rows, N = W->cols;
  const int kp = W->layout == QT_LAYOUT_NK ? W->kpad : pad16(K);
  if (qhip_init()) die("qmatmul");
  const size_t oc = al256((size_t)M * K * 4), oq = oc + al256((size_t)M * N * 4), os = oq + al256((size_t)M * kp);
  const size_t ot = os + al256((size_t)M * 4), total = ot + (W->layout != QT_LAYOUT_NK ? al256((size_t)N * kp) : 0);
  uint8_t *b = qmm_workspace(total);
  if (!b) die("qmatmul");
  float *da = (float*)b, *dc = (float*)(b + oc), *as = (float*)(b + os);
  int8_t *qa = (int8_t*)(b + oq), *wnk = (int8_t*)W->q;
  if (W->layout != QT_LAYOUT_NK) {     // row-major device tensor: re-lay it
    wnk = (int8_t*)(b + ot);
    if (qhip_fill_zero(wnk, (size_t)N * kp) || qhip_transpose_kn_to_nk((const int8_t*)W->q, K, N, kp, wnk))
      die("qmatmul");
  }
  if (qhip_h2d(da, A->data, (size_t)M * K * 4) || qhip_quant_rows(da, M, K, qa, kp, as) ||
      qhip_qmm_product(qa, as, M, wnk, W->scale, N, kp, dc) ||
      qhip_d2h_async(C->data, dc, (size_t)M * N * 4) || qhip_sync())
    die("qmatmul");
}

void quantize_int8_percol(const float *w, int rows, int cols, signed char *q, float *scale) {
  const size_t n = (size_t)rows * cols;
  if (qhip_init()) die("quantize_int8_percol");
  float *dw = (float*)qhip_malloc(n * 4);
  int8_t *dq = (int8_t*)qhip_malloc(n);
  float *ds = (float*)qhip_malloc((size_t)cols * 4);
  if (!dw || !dq || !ds || qhip_h2d(dw, w, n * 4) ||
      qhip_quantize_percol(dw, rows, cols, 0, cols, dq, ds) ||
      qhip_d2h_async(q, dq, n) || qhip_d2h_async(scale, ds, (size_t)cols * 4) || qhip_sync())
    die("quantize_int8_percol");
  qhip_free(dw); qhip_free(dq); qhip_free(ds);
}

void dequantize_int8_percol(const signed char *q, const float *scale, int rows, int cols, float *w) {
  const size_t n = (size_t)rows * cols;
  if (qhip_init()) die("dequantize_int8_percol");
  float *dw = (float*)qhip_malloc(n * 4);
  int8_t *dq = (int8_t*)qhip_malloc(n);
  float *ds = (float*)qhip_malloc((size_t)cols * 4);
  if (!dw || !dq || !ds || qhip_h2d(dq, q, n) || qhip_h2d(ds, scale, (size_t)cols * 4) ||
      qhip_dequantize_kn(dq, ds, rows, cols, dw) || qhip_d2h_async(w, dw, n * 4) || qhip_sync())
    die("dequantize_int8_percol");
  qhip_free(dw); qhip_free(dq); qhip_free(ds);
}

void qacc_columns(const signed char *qa, const signed char *qw, int K, int N, int32_t *acc) {
  if (qhip_init()) die("qacc_columns");
  int8_t *da = (int8_t*)qhip_malloc((size_t)K);
  int8_t *dw = (int8_t*)qhip_malloc((size_t)K * N);
  int32_t *dacc = (int32_t*)qhip_malloc((size_t)N * 4);
  if (!da || !dw || !dacc || qhip_h2d(da, qa, (size_t)K) || qhip_h2d(dw, qw, (size_t)K * N) ||
      qhip_qacc_kn(da, dw, K, N, dacc) || qhip_d2h_async(acc, dacc, (size_t)N * 4) || qhip_sync())
    die("qacc_columns");
  qhip_free(da); qhip_free(dw); qhip_free(dacc);
}

int q_llama_tensor_export(const QTensor *t, signed char *q_host, float *scale_host) {
  const size_t n = (size_t)t->rows * t->cols;
  if (qhip_init()) return 1;
  if (t->layout == QT_LAYOUT_KN) {
    if (qhip_d2h(q_host, t->q, n)) return 1;
  } else {
    int8_t *tmp = (int8_t*)qhip_malloc(n);
    if (!tmp) return 1;
    int rc = qhip_nk_to_kn((const int8_t*)t->q, t->rows, t->cols, t->kpad, tmp) || qhip_d2h(q_host, tmp, n);
    qhip_free(tmp);
    if (rc) return 1;
  }
  return qhip_d2h(scale_host, t->scale, (size_t)t->cols * 4);
}

// ---------------------------------------------------------------------------
// helpers
// ---------------------------------------------------------------------------
int qllama_device_count(void) { return qhip_device_count(); }
void *qllama_dev_alloc(size_t bytes) { return qhip_init() ? NULL : qhip_malloc(bytes); }
void qllama_dev_free(void *p) { qhip_sync(); qhip_free(p); }
int qllama_h2d(void *dst, const void *src, size_t bytes) { return qhip_h2d(dst, src, bytes); }
int qllama_d2h(void *dst, const void *src, size_t bytes) { return qhip_sync() || qhip_d2h(dst, src, bytes); }
int qllama_device_sync(void) { return qhip_device_sync(); }
int qllama_sync(void) { return qhip_sync(); }

// 1 when the model's exact decode steps run the attention half of each layer in
// one launch (qhip_attn_layer), 0 when they run the separate kernels.
int qllama_attn_layer_active(const QLlamaModel *m) { return m && m->dev && ((const QDev*)m->dev)->ly_ok; }
void *qllama_stream(void) { return qhip_init() ? NULL : qhip_stream(); }
int qllama_profile(int enable) { profiling = enable ? 1 : 0; return qhip_profile_enable(enable); }

// Cold op-level timing (qllama_bench_qmatmul, qllama_gqa_decode_ex): every timed
// call is preceded by a 512 MB read, and the call's time is that of the
// (flush, call) sequence less that of the flushes alone.
static int bench_cold = 0;
int qllama_bench_cold(int on) { bench_cold = on ? 1 : 0; return 0; }

// Mean time (us) of `reps` calls of fn: back to back, or, when cold, each
// behind a cache flush with the flushes' own time taken out.
typedef int (*BenchCall)(void *ctx);
static int bench_time(BenchCall fn, void *ctx, int reps, double *us) {
  double ms = 0.0, ms_flush = 0.0;
  int rc = qhip_timer_start();
  for (int i = 0; i < reps && !rc; i++) rc = (bench_cold && qhip_flush_caches()) || fn(ctx);
  if (!rc) rc = qhip_timer_stop(&ms);
  if (!rc && bench_cold) {
    rc = qhip_timer_start();
    for (int i = 0; i < reps && !rc; i++) rc = qhip_flush_caches();
    if (!rc) rc = qhip_timer_stop(&ms_flush);
  }
  if (!rc && us) *us = 1e3 * (ms - ms_flush) / reps;
  return rc;
}
int qllama_profile_read(char *names, int names_len, double *ms, long long *count, int max) {
  return qhip_profile_read(names, names_len, ms, count, max);
}

typedef struct {
  int mode, rope, n_heads, n_kv, hd, T;
  float scale;
  float *qkv, *k, *v;
  int *pos;
  float *cos_t, *sin_t;
  void *scratch;
  float *out, *obm;
} GqaCall;

static int gqa_call(void *ctx) {
  const GqaCall *g = (const GqaCall*)ctx;
  if (g->mode == QLLAMA_MODE_FAST)
    return qhip_fattn(g->qkv, g->k, g->v, g->pos, g->n_heads, g->n_kv, g->hd, g->T, g->scale, g->cos_t, g->sin_t,
                      g->rope, g->scratch, g->out, g->obm);
  if (g->rope)
    return qhip_attention_rope(g->qkv, g->k, g->v, g->pos, g->n_heads, g->n_kv, g->hd, g->T, g->scale, g->cos_t,
                               g->sin_t, (float*)g->scratch, g->out, g->obm);
  return qhip_attention(g->qkv, g->k, g->v, g->pos, g->n_heads, g->n_kv, g->hd, g->T, g->scale, (float*)g->scratch,
                        g->out, g->obm);
}

// Op-level decode attention on device-resident data (BASELINE's GQA config):
// the cache is [n_kv][T][hd] (max_seq = T), position T-1.
int qllama_gqa_decode_ex(const float *q, const float *k, const float *v, int T, int n_heads, int n_kv, int hd,
                         float rope_base, int mode, int reps, float *o, float *k_row, double *us_per_call) {
  if (qhip_init()) return 1;
  if (T <= 0 || n_kv <= 0 || n_heads <= 0 || n_heads % n_kv || hd <= 0 || (hd & 1) ||
      (mode != QLLAMA_MODE_EXACT && mode != QLLAMA_MODE_FAST)) {
    fprintf(stderr, "Error: qllama_gqa_decode_ex: bad shape or mode\n");
    return 1;
  }
  if (mode == QLLAMA_MODE_FAST && !qhip_fattn_ok(n_heads, n_kv, hd, T)) {
    fprintf(stderr, "Error: qllama_gqa_decode_ex: shape not supported by the fast attention\n");
    return 1;
  }
  const int rope = rope_base > 0.0f, qd = n_heads * hd, kvd = n_kv * hd, half = hd / 2;
  const size_t kvn = (size_t)T * kvd;
  const size_t sc_bytes = mode == QLLAMA_MODE_FAST ? qhip_fattn_scratch(n_heads, n_kv, hd, T)
                                                   : qhip_attention_scratch(n_heads, T) * 4;
  float *dqkv = (float*)qhip_malloc((size_t)(qd + 2 * kvd) * 4), *dk = (float*)qhip_malloc(kvn * 4);
  float *dv = (float*)qhip_malloc(kvn * 4), *tmp = (float*)qhip_malloc(kvn * 4);
  float *dout = (float*)qhip_malloc((size_t)qd * 4), *dobm = (float*)qhip_malloc((size_t)qhip_attention_nbm(n_heads, hd) * 4);
  float *dcos = rope ? (float*)qhip_malloc((size_t)T * half * 4) : NULL;
  float *dsin = rope ? (float*)qhip_malloc((size_t)T * half * 4) : NULL;
  void *dsc = qhip_malloc(sc_bytes);
  int *dpos = (int*)qhip_malloc(256);
  const int pos = T - 1;
  int rc = (!dqkv || !dk || !dv || !tmp || !dout || !dobm || !dsc || !dpos || (rope && (!dcos || !dsin))) ? 1 : 0;
  if (!rc) rc = qhip_h2d(dqkv, q, (size_t)qd * 4) || qhip_h2d(dpos, &pos, 4) || qhip_fill_zero(dsc, sc_bytes);
  if (!rc && rope) rc = qhip_h2d(dqkv + qd, k + (size_t)pos * kvd, (size_t)kvd * 4) ||
                        qhip_h2d(dqkv + qd + kvd, v + (size_t)pos * kvd, (size_t)kvd * 4) ||
                        rope_upload(dcos, dsin, T, hd, rope_base);
  if (!rc) rc = qhip_h2d(tmp, k, kvn * 4) || qhip_kv_relayout(tmp, T, n_kv, hd, dk) || qhip_sync() ||
                qhip_h2d(tmp, v, kvn * 4) || qhip_kv_relayout(tmp, T, n_kv, hd, dv);
  GqaCall g = {mode, rope, n_heads, n_kv, hd, T, 1.0f / sqrtf((float)hd),      // llama.c:532
               dqkv, dk, dv, dpos, dcos, dsin, dsc, dout, dobm};
  if (!rc) rc = gqa_call(&g) || qhip_sync();
  if (!rc && reps > 0) rc = bench_time(gqa_call, &g, reps, us_per_call);
  if (!rc) rc = qhip_d2h(o, dout, (size_t)qd * 4);
  if (!rc && k_row)          // row T-1 of every KV head, in the reference's (n_kv*hd) order
    for (int h = 0; h < n_kv && !rc; h++) rc = qhip_d2h(k_row + (size_t)h * hd, dk + ((size_t)h * T + pos) * hd, (size_t)hd * 4);
  if (rc) fprintf(stderr, "Error: qllama_gqa_decode_ex: %s\n", qhip_last_error());
  qhip_free(dqkv); qhip_free(dk); qhip_free(dv); qhip_free(tmp); qhip_free(dout); qhip_free(dobm);
  qhip_free(dcos); qhip_free(dsin); qhip_free(dsc); qhip_free(dpos);
  return rc;
}

// One activation row through the decode GEMV that normalizes its own input
// (rmsnorm.c:7-21, quantization quant.c:66-78, W8A8 quant.c:79-82): mode 0
// plain (out: W->cols values), mode 2 SwiGLU over gate columns [0, N) and up
// columns [N, 2N) of W (out: N = W->cols / 2 values of h, llama.c:583-587).
// fast selects the fast decode mode's tree-ordered sum of squares.
int qllama_pf_attention_ex(const float *q, const float *k, const float *v, int R, int p0, int n_heads, int n_kv,
                           int hd, int mode, int reps, float *o, double *us_per_call) {
  if (qhip_init()) return 1;
  const int T = p0 + R;
  if (!q || !k || !v || !o || R <= 0 || p0 < 0 || n_kv <= 0 || n_heads <= 0 || n_heads % n_kv || hd <= 0 ||
      (mode != QLLAMA_MODE_EXACT && mode != QLLAMA_MODE_FAST) || T > 16384) {
    fprintf(stderr, "Error: qllama_pf_attention_ex: bad shape or mode\n");
    return 1;
  }
  const int G = n_heads / n_kv;
  if (mode == QLLAMA_MODE_FAST ? !qhip_pf_attention_fast_ok(n_heads, n_kv, hd)
                               : !((hd == 128 || hd == 64 || hd == 48) && G <= 8 && G * hd <= 1024)) {
    fprintf(stderr, "Error: qllama_pf_attention_ex: shape not supported in this mode\n");
    return 1;
  }
  const size_t qn = (size_t)R * n_heads * hd, kvn = (size_t)T * n_kv * hd;
  const size_t ws_n = mode == QLLAMA_MODE_FAST ? 1 : qhip_pf_attention_scratch(R, n_heads, T);
  float *dq = (float*)qhip_malloc(qn * 4), *dk = (float*)qhip_malloc(kvn * 4), *dv = (float*)qhip_malloc(kvn * 4);
  float *tmp = (float*)qhip_malloc(kvn * 4), *dout = (float*)qhip_malloc(qn * 4), *ws = (float*)qhip_malloc(ws_n * 4);
  int rc = (!dq || !dk || !dv || !tmp || !dout || !ws) ? 1 : 0;
  if (!rc) rc = qhip_h2d(dq, q, qn * 4) || qhip_h2d(tmp, k, kvn * 4) || qhip_kv_relayout(tmp, T, n_kv, hd, dk) ||
                qhip_sync() || qhip_h2d(tmp, v, kvn * 4) || qhip_kv_relayout(tmp, T, n_kv, hd, dv);
  const float scale = 1.0f / sqrtf((float)hd);                  // llama.c:532
#define PFA_LAUNCH()                                                                                       \
  (mode == QLLAMA_MODE_FAST ? qhip_pf_attention_fast(dq, dk, dv, R, p0, n_heads, n_kv, hd, T, scale, dout)  \
                            : qhip_pf_attention(dq, dk, dv, R, p0, n_heads, n_kv, hd, T, scale, ws, dout))
  if (!rc) rc = PFA_LAUNCH() || qhip_sync();
  if (!rc && reps > 0) {
    double ms = 0.0;
    rc = qhip_timer_start();
    for (int i = 0; i < reps && !rc; i++) rc = PFA_LAUNCH();
    if (!rc) rc = qhip_timer_stop(&ms);
    if (!rc && us_per_call) *us_per_call = 1e3 * ms / reps;
  }
#undef PFA_LAUNCH
  if (!rc) rc = qhip_d2h(o, dout, qn * 4);
  if (rc) fprintf(stderr, "Error: qllama_pf_attention_ex: %s\n", qhip_last_error());
  qhip_free(dq); qhip_free(dk); qhip_free(dv); qhip_free(tmp); qhip_free(dout); qhip_free(ws);
  return rc;
}

int qllama_norm_gemv(const float *x, const float *gamma, float eps, const QTensor *W, int mode, int fast, float *out) {
  if (qhip_init()) return 1;
  const int dm = W->rows, cols = W->cols;
  if (W->layout != QT_LAYOUT_NK || !qhip_gemv_norm_ok(W->kpad, dm) || (mode != 0 && mode != 2) ||
      (mode == 2 && (cols & 1))) {
    fprintf(stderr, "Error: qllama_norm_gemv: unsupported shape or mode\n");
    return 1;
  }
  const int N = mode == 2 ? cols / 2 : cols;
  float *dx = (float*)qhip_malloc((size_t)dm * 4), *dg = (float*)qhip_malloc((size_t)dm * 4);
  float *dout = (float*)qhip_malloc((size_t)N * 4), *dbm = (float*)qhip_malloc((size_t)qhip_gemv_norm_blocks(N) * 4);
  int rc = !dx || !dg || !dout || !dbm || qhip_h2d(dx, x, (size_t)dm * 4) || qhip_h2d(dg, gamma, (size_t)dm * 4);
  if (!rc)
    rc = mode == 2 ? qhip_gemv_swiglu_norm(QLLAMA_CLS_OTHER, fast, dx, dm, dg, eps, (const int8_t*)W->q, W->scale, N,
                                           W->kpad, dout, dbm)
                   : qhip_gemv_plain_norm(QLLAMA_CLS_OTHER, fast, dx, dm, dg, eps, (const int8_t*)W->q, W->scale, N,
                                          W->kpad, dout, NULL);
  if (!rc) rc = qhip_d2h(out, dout, (size_t)N * 4);
  if (rc) fprintf(stderr, "Error: qllama_norm_gemv: %s\n", qhip_last_error());
  qhip_free(dx); qhip_free(dg); qhip_free(dout); qhip_free(dbm);
  return rc;
}

// A device QTensor (NK layout) holding the seeded generator's N(0, sigma) (rows,
// cols) matrix of tensor id tid, quantized per column (quant.c:10-27): the
// op-level GEMV configuration's weights, built without a host copy.
QTensor qtensor_synth(int rows, int cols, uint64_t seed, uint64_t tid, double sigma) {
  QTensor t = qtensor_create(rows, cols);
  if (qhip_synth_quant_nk(seed, tid, rows, cols, t.kpad, 0, sigma, (int8_t*)t.q, t.scale) || qhip_sync())
    die("qtensor_synth");
  return t;
}

typedef struct {
  const QTensor *W;
  int M;
  float *a, *c;
  int8_t *qa;
  float *as;
} QmmCall;

static int qmm_call(void *ctx) {
  const QmmCall *q = (const QmmCall*)ctx;
  const QTensor *W = q->W;
  return qhip_quant_rows(q->a, q->M, W->rows, q->qa, W->kpad, q->as) ||
         qhip_qmm_product(q->qa, q->as, q->M, (const int8_t*)W->q, W->scale, W->cols, W->kpad, q->c);
}

// Op-level timing of qmatmul on device-resident data: M rows of N(0, 1) inputs
// (K = W->rows), reps calls after one warm-up.  *us_call: mean time of one call
// (activation quantization + product, HIP events around the whole sequence);
// *us_product / *us_quant: mean duration of the product / quantization kernels
// alone (events bound to each launch).
int qllama_bench_qmatmul(const QTensor *W, int M, int reps, double *us_call, double *us_product, double *us_quant) {
  if (qhip_init() || M < 1 || reps < 1 || W->layout != QT_LAYOUT_NK) return 1;
  const int K = W->rows, N = W->cols, kp = W->kpad;
  float *da = (float*)qhip_malloc((size_t)M * K * 4), *dc = (float*)qhip_malloc((size_t)M * N * 4);
  int8_t *qa = (int8_t*)qhip_malloc((size_t)M * kp);
  float *as = (float*)qhip_malloc((size_t)M * 4);
  int rc = !da || !dc || !qa || !as || qhip_synth_f32(4321, 77, (size_t)M * K, 1.0, da);
  QmmCall c = {W, M, da, dc, qa, as};
  if (!rc) rc = qmm_call(&c) || qhip_sync();
  if (!rc) rc = bench_time(qmm_call, &c, reps, us_call);
  // the same calls with per-launch events, each launch on a drained stream (and
  // behind a cache flush when cold): product (class "other"), quantization ("quant_rows")
  if (!rc && (us_product || us_quant)) {
    char names[1024];
    double cms[32];
    long long cnt[32];
    rc = qhip_profile_enable(1 | (bench_cold ? QHIP_PROF_COLD : QHIP_PROF_SERIAL));
    for (int i = 0; i < reps && !rc; i++) rc = qmm_call(&c);
    if (!rc) rc = qhip_sync();
    const int n = rc ? 0 : qhip_profile_read(names, sizeof names, cms, cnt, 32);
    qhip_profile_enable(0);
    char *save = NULL, *tok = strtok_r(names, ",", &save);
    for (int i = 0; i < n && tok; i++, tok = strtok_r(NULL, ",", &save)) {
      if (us_product && !strcmp(tok, "other")) *us_product = 1e3 * cms[i];
      if (us_quant && !strcmp(tok, "quant_rows")) *us_quant = 1e3 * cms[i];
    }
  }
  qhip_free(da); qhip_free(dc); qhip_free(qa); qhip_free(as);
  return rc;
}
