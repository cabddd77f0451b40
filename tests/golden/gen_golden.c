// gen_golden.c - writes the golden fixtures under tests/golden/data/ by calling
// the REFERENCE's own compiled functions (objects built from /root/reference by
// oracle/Makefile into oracle/_ref/).  This file contains no reference code: it
// only calls the reference's public API (quant.h, llama.h, rmsnorm.h, rope.h,
// gqa.h, sampler.h, tensor.h) on inputs from the seeded generator (oracle/synth.h)
// and records what comes back.  It builds only where /root/reference exists.
//
//   gen_golden <outdir> ops        quantizer, qmatmul, rmsnorm, rope, attention
//   gen_golden <outdir> gqa8192    decode attention at context 8192 (slow)
//   gen_golden <outdir> e2e <name> tiny | 1b | 8b greedy token streams
//   gen_golden <outdir> llmqhash <file>   load an LLMQ file with the reference's
//                                  q_llama_model_load and print its digest
//   gen_golden <outdir> e2e_f32 <name>   tiny | mid: greedy streams of the fp32
//                                  LLMA path (llama_decode_step, llama.c:296-362)
//   gen_golden <outdir> llmahash <file>   load an LLMA file with llama_model_load
//                                  and print its digest
//   gen_golden <outdir> sample     sample_token draws, and the `llama` command's
//                                  sampled loop (main.c:658-669) on the tiny model
//   gen_golden <outdir> gpt <name>  tiny | gpt2s | long: greedy streams of the GPT-2 KV
//                                  decode (gpt_decode_step, model.c:457-520)
//   gen_golden <outdir> gpthash <file>   load a GPTC file with gpt_load and print
//                                  its digest
//   gen_golden <outdir> qfrom      q_llama_quantize_from of two fp32 models (one at
//                                  selftest [21]'s shape, one with gains and
//                                  biases), and their decode steps
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>
#include <time.h>

#include "tensor.h"
#include "quant.h"
#include "llama.h"
#include "rmsnorm.h"
#include "rope.h"
#include "gqa.h"
#include "sampler.h"
#include "model.h"
#include "checkpoint.h"
#include "synth.h"

static const char *OUT = ".";

static double now_s(void) {
  struct timespec t; clock_gettime(CLOCK_MONOTONIC, &t);
  return (double)t.tv_sec + 1e-9 * (double)t.tv_nsec;
}

// ---- minimal .npy writer (v1.0, little-endian, C order) --------------------
static void npy_write(const char *name, const char *descr, const void *data, size_t elem,
                      int ndim, const long *shape) {
  char path[1024]; snprintf(path, sizeof path, "%s/%s.npy", OUT, name);
  char hdr[256], shp[128] = "";
  size_t n = 1;
  for (int i = 0; i < ndim; i++) {
    char t[32]; snprintf(t, sizeof t, "%ld%s", shape[i], (ndim == 1 || i < ndim - 1) ? "," : "");
    strcat(shp, t); n *= (size_t)shape[i];
  }
  int len = snprintf(hdr, sizeof hdr, "{'descr': '%s', 'fortran_order': False, 'shape': (%s), }", descr, shp);
  int total = 10 + len + 1;
  int pad = (64 - total % 64) % 64;
  FILE *f = fopen(path, "wb");
  if (!f) { fprintf(stderr, "cannot write %s\n", path); exit(1); }
  unsigned short hl = (unsigned short)(len + pad + 1);
  fwrite("\x93NUMPY\x01\x00", 1, 8, f);
  fwrite(&hl, 2, 1, f);
  fwrite(hdr, 1, (size_t)len, f);
  for (int i = 0; i < pad; i++) fputc(' ', f);
  fputc('\n', f);
  fwrite(data, elem, n, f);
  fclose(f);
}
static void npy_f32(const char *name, const float *d, int ndim, const long *s) { npy_write(name, "<f4", d, 4, ndim, s); }
static void npy_i8(const char *name, const int8_t *d, int ndim, const long *s) { npy_write(name, "|i1", d, 1, ndim, s); }
static void npy_i32(const char *name, const int32_t *d, int ndim, const long *s) { npy_write(name, "<i4", d, 4, ndim, s); }

static Tensor mat(int r, int c) { int s[2] = {r, c}; return tensor_create_nograd(s, 2); }
static Tensor vecf(int n) { int s[1] = {n}; return tensor_create_nograd(s, 1); }

// ---------------------------------------------------------------------------
// ops fixtures
// ---------------------------------------------------------------------------
static void fx_quant(FILE *js) {
  // (a) crafted 6x4: col 0 all zero (scale 1), col 1 exact half-way ties at
  // scale 1, col 2 negative extreme, col 3 tiny magnitudes.
  const int R = 6, C = 4;
  float w[24] = {
    0.0f,  127.0f, -3.0f, 1e-30f,
    0.0f,   0.5f,  1.0f, -2e-30f,
    0.0f,   1.5f, -127.5f, 3e-30f,
    0.0f,   2.5f,  64.0f, 0.0f,
    0.0f,  -0.5f,  0.25f, 5e-31f,
    0.0f,  -2.5f, -0.25f, -7e-30f};
  int8_t q[24]; float sc[4];
  quantize_int8_percol(w, R, C, (signed char*)q, sc);
  long s2[2] = {R, C}, s1[1] = {C};
  npy_f32("quant_a_w", w, 2, s2); npy_i8("quant_a_q", q, 2, s2); npy_f32("quant_a_scale", sc, 1, s1);
  // (b) random 64x48 and (c) 37x5 from the generator
  const int rb = 64, cb = 48;
  float *wb = malloc(sizeof(float) * rb * cb); int8_t *qb = malloc(rb * cb); float *sb = malloc(4 * cb);
  syn_fill(wb, (size_t)rb * cb, 7, SYN_TID_GENERIC + 1, 0.02);
  quantize_int8_percol(wb, rb, cb, (signed char*)qb, sb);
  long t2[2] = {rb, cb}, t1[1] = {cb};
  npy_f32("quant_b_w", wb, 2, t2); npy_i8("quant_b_q", qb, 2, t2); npy_f32("quant_b_scale", sb, 1, t1);
  float *deq = malloc(sizeof(float) * rb * cb);
  dequantize_int8_percol((signed char*)qb, sb, rb, cb, deq);
  npy_f32("quant_b_deq", deq, 2, t2);
  free(wb); free(qb); free(sb); free(deq);
  fprintf(js, "  \"quant\": [\"a\", \"b\"],\n");
}

static void qmm_case(const char *name, int M, int K, int N, uint64_t seed, double asig, int save_inputs,
                     FILE *js) {
  QTensor W = qtensor_create(K, N);
  float *wf = malloc(sizeof(float) * (size_t)K * N);
  syn_fill(wf, (size_t)K * N, seed, SYN_TID_GENERIC + 10, 0.02);
  qtensor_quantize(&W, wf);
  Tensor A = mat(M, K), Cc = mat(M, N);
  syn_fill(A.data, (size_t)M * K, seed, SYN_TID_GENERIC + 11, asig);
  qmatmul(&A, &W, &Cc);
  char nm[128]; long sa[2] = {M, K}, sw[2] = {K, N}, sc[1] = {N}, so[2] = {M, N};
  if (save_inputs) {
    snprintf(nm, sizeof nm, "%s_A", name); npy_f32(nm, A.data, 2, sa);
    snprintf(nm, sizeof nm, "%s_Wq", name); npy_i8(nm, (int8_t*)W.q, 2, sw);
    snprintf(nm, sizeof nm, "%s_Ws", name); npy_f32(nm, W.scale, 1, sc);
  }
  snprintf(nm, sizeof nm, "%s_C", name); npy_f32(nm, Cc.data, 2, so);
  fprintf(js, "  \"%s\": {\"M\": %d, \"K\": %d, \"N\": %d, \"seed\": %llu, \"asig\": %g},\n",
          name, M, K, N, (unsigned long long)seed, asig);
  free(wf); qtensor_free(&W); tensor_free(&A); tensor_free(&Cc);
}

// Op-level GEMV at the BASELINE shapes: W int8 [M_out, K] (reference layout (K, M_out)),
// x ~ N(0,1) rows.  Records digests of W and of the output, and the output head.
static void qmm_op(int si, int Mout, int K, FILE *js) {
  const uint64_t seed = 1234;
  QTensor W = qtensor_create(K, Mout);
  float *wf = malloc(sizeof(float) * (size_t)K * Mout);
  syn_fill(wf, (size_t)K * Mout, seed, SYN_TID_GEMV_W + (uint64_t)si, 0.02);
  qtensor_quantize(&W, wf);
  free(wf);
  uint64_t hq = syn_hash_i8((int8_t*)W.q, (size_t)K * Mout, 0);
  uint64_t hs = syn_hash_f32(W.scale, (size_t)Mout, 0);
  fprintf(js, "  \"gemv_%d\": {\"M\": %d, \"K\": %d, \"w_hash\": \"%016llx\", \"s_hash\": \"%016llx\"",
          si, Mout, K, (unsigned long long)hq, (unsigned long long)hs);
  for (int b = 1; b <= 8; b += 7) {
    Tensor X = mat(b, K), Y = mat(b, Mout);
    syn_fill(X.data, (size_t)b * K, seed, SYN_TID_GEMV_X + (uint64_t)si, 1.0);
    double t0 = now_s();
    qmatmul(&X, &W, &Y);
    double t1 = now_s();
    uint64_t hy = syn_hash_f32(Y.data, (size_t)b * Mout, 0);
    char nm[64]; long s1[1] = {256};
    snprintf(nm, sizeof nm, "gemv_%d_b%d_head", si, b);
    npy_f32(nm, Y.data, 1, s1);
    fprintf(js, ", \"b%d_hash\": \"%016llx\", \"b%d_ref_s\": %.4f", b, (unsigned long long)hy, b, t1 - t0);
    tensor_free(&X); tensor_free(&Y);
  }
  fprintf(js, "},\n");
  qtensor_free(&W);
}

static void fx_rmsnorm(FILE *js) {
  const int cols_list[3] = {288, 2048, 4096};
  for (int c = 0; c < 3; c++) {
    const int cols = cols_list[c], rows = 3;
    Tensor x = mat(rows, cols), y = mat(rows, cols), g = vecf(cols);
    syn_fill(x.data, (size_t)rows * cols, 11, SYN_TID_GENERIC + 20 + (uint64_t)c, 1.0);
    syn_fill(g.data, (size_t)cols, 11, SYN_TID_GENERIC + 30 + (uint64_t)c, 0.1);
    for (int j = 0; j < cols; j++) g.data[j] = 1.0f + g.data[j];
    x.data[5] = 1e-3f; x.data[6] = -250.0f;                  // spread the dynamic range
    rmsnorm(&x, &g, &y, 1e-5f);
    char nm[64]; long s2[2] = {rows, cols}, s1[1] = {cols};
    snprintf(nm, sizeof nm, "rms_%d_x", cols); npy_f32(nm, x.data, 2, s2);
    snprintf(nm, sizeof nm, "rms_%d_g", cols); npy_f32(nm, g.data, 1, s1);
    snprintf(nm, sizeof nm, "rms_%d_y", cols); npy_f32(nm, y.data, 2, s2);
    tensor_free(&x); tensor_free(&y); tensor_free(&g);
  }
  fprintf(js, "  \"rmsnorm\": [288, 2048, 4096],\n");
}

static void fx_rope(FILE *js) {
  const int pos_list[7] = {0, 1, 7, 511, 2047, 2559, 8191};
  for (int p = 0; p < 7; p++) {
    Tensor x = mat(1, 32 * 128);
    syn_fill(x.data, 4096, 21, SYN_TID_GENERIC + 40 + (uint64_t)p, 1.0);
    char nm[64]; long s2[2] = {1, 4096};
    snprintf(nm, sizeof nm, "rope_p%d_x", pos_list[p]); npy_f32(nm, x.data, 2, s2);
    rope_heads_pos(&x, 32, 500000.0f, pos_list[p]);
    snprintf(nm, sizeof nm, "rope_p%d_y", pos_list[p]); npy_f32(nm, x.data, 2, s2);
    tensor_free(&x);
  }
  {  // tiny-config shape, base 10000, three rows starting at position 5
    Tensor x = mat(3, 6 * 48);
    syn_fill(x.data, 3 * 288, 21, SYN_TID_GENERIC + 50, 1.0);
    long s2[2] = {3, 288};
    npy_f32("rope_tiny_x", x.data, 2, s2);
    rope_heads_pos(&x, 6, 10000.0f, 5);
    npy_f32("rope_tiny_y", x.data, 2, s2);
    tensor_free(&x);
  }
  fprintf(js, "  \"rope\": [0, 1, 7, 511, 2047, 2559, 8191],\n");
}

// Decode attention at context T = last row of gqa_forward over T positions
// (bit-identical to llama.c:554-576).  q and k rows carry RoPE at their position
// (theta 500000); the cache is N(0,1).  32 query heads, 8 KV heads, hd 128.
static void gqa_case(int ci, int T, FILE *js) {
  const int H = 32, KVH = 8, hd = 128, qd = H * hd, kd = KVH * hd;
  Tensor Q = mat(T, qd), K = mat(T, kd), V = mat(T, kd), O = mat(T, qd);
  syn_fill(Q.data, (size_t)T * qd, 31, SYN_TID_GQA_Q + (uint64_t)ci, 1.0);
  syn_fill(K.data, (size_t)T * kd, 31, SYN_TID_GQA_K + (uint64_t)ci, 1.0);
  syn_fill(V.data, (size_t)T * kd, 31, SYN_TID_GQA_V + (uint64_t)ci, 1.0);
  rope_heads_pos(&Q, H, 500000.0f, 0);
  rope_heads_pos(&K, KVH, 500000.0f, 0);
  GqaCache c = gqa_cache_create(T, H, KVH, hd);
  double t0 = now_s();
  gqa_forward(&Q, &K, &V, &c, &O);
  double t1 = now_s();
  char nm[64]; long s1[1] = {qd};
  snprintf(nm, sizeof nm, "gqa_T%d_o", T); npy_f32(nm, &O.data[(size_t)(T - 1) * qd], 1, s1);
  snprintf(nm, sizeof nm, "gqa_T%d_q", T); npy_f32(nm, &Q.data[(size_t)(T - 1) * qd], 1, s1);
  fprintf(js, "  \"gqa_T%d\": {\"case\": %d, \"T\": %d, \"k_hash\": \"%016llx\", \"v_hash\": \"%016llx\", \"ref_s\": %.3f},\n",
          T, ci, T, (unsigned long long)syn_hash_f32(K.data, (size_t)T * kd, 0),
          (unsigned long long)syn_hash_f32(V.data, (size_t)T * kd, 0), t1 - t0);
  gqa_cache_free(&c);
  tensor_free(&Q); tensor_free(&K); tensor_free(&V); tensor_free(&O);
}

// ---------------------------------------------------------------------------
// End-to-end greedy runs through q_llama_decode_step.
// ---------------------------------------------------------------------------
typedef struct { const char *name; int32_t cfg[8]; float base; int tied, prompt, gen; } E2E;
static const E2E CASES[3] = {
  {"tiny", {32000, 288, 6, 6, 2, 48, 768, 256}, 10000.0f, 0, 128, 128},
  {"1b", {128256, 2048, 16, 32, 8, 64, 8192, 768}, 500000.0f, 1, 512, 256},
  {"8b", {128256, 4096, 32, 32, 8, 128, 14336, 2560}, 500000.0f, 0, 2048, 512},
};

static void synth_q(QTensor *t, float *buf, uint64_t seed, uint64_t tid) {
  syn_fill(buf, (size_t)t->rows * t->cols, seed, tid, 0.02);
  qtensor_quantize(t, buf);
}

static uint64_t qhash(const QTensor *t, uint64_t salt) {
  return syn_hash_i8((const int8_t*)t->q, (size_t)t->rows * t->cols, salt) * 3 +
         syn_hash_f32(t->scale, (size_t)t->cols, salt ^ 0x5CA1E5ULL);
}

static void build_model(QLlamaModel *m, const E2E *e, uint64_t seed) {
  const int32_t *c = e->cfg;
  m->vocab = c[0]; m->d_model = c[1]; m->n_layers = c[2]; m->n_heads = c[3]; m->n_kv = c[4];
  m->head_dim = c[5]; m->d_ff = c[6]; m->max_seq = c[7]; m->rope_base = e->base; m->eps = 1e-5f;
  const int dm = c[1], qd = c[3] * c[5], kvd = c[4] * c[5], ff = c[6], L = c[2];
  size_t big = (size_t)c[0] * dm; if ((size_t)dm * ff > big) big = (size_t)dm * ff;
  if ((size_t)dm * qd > big) big = (size_t)dm * qd;
  float *buf = malloc(big * sizeof(float));
  m->wte = qtensor_create(c[0], dm);
  synth_q(&m->wte, buf, seed, 0);
  m->blocks = malloc(sizeof(QLlamaBlock) * (size_t)L);
  for (int l = 0; l < L; l++) {
    QLlamaBlock *b = &m->blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    b->attn_norm = vecf(dm); b->ffn_norm = vecf(dm);
    for (int j = 0; j < dm; j++) { b->attn_norm.data[j] = 1.0f; b->ffn_norm.data[j] = 1.0f; }
    b->b_q = vecf(qd); b->b_k = vecf(kvd); b->b_v = vecf(kvd);
    b->Wq = qtensor_create(dm, qd); synth_q(&b->Wq, buf, seed, t0 + 1);
    b->Wk = qtensor_create(dm, kvd); synth_q(&b->Wk, buf, seed, t0 + 2);
    b->Wv = qtensor_create(dm, kvd); synth_q(&b->Wv, buf, seed, t0 + 3);
    b->Wo = qtensor_create(qd, dm); synth_q(&b->Wo, buf, seed, t0 + 7);
    b->Wgate = qtensor_create(dm, ff); synth_q(&b->Wgate, buf, seed, t0 + 9);
    b->Wup = qtensor_create(dm, ff); synth_q(&b->Wup, buf, seed, t0 + 10);
    b->Wdown = qtensor_create(ff, dm); synth_q(&b->Wdown, buf, seed, t0 + 11);
  }
  m->final_norm = vecf(dm);
  for (int j = 0; j < dm; j++) m->final_norm.data[j] = 1.0f;
  m->lm_head = qtensor_create(dm, c[0]);
  if (e->tied) {
    float *w = malloc((size_t)c[0] * dm * sizeof(float));
    syn_fill(w, (size_t)c[0] * dm, seed, 0, 0.02);
    for (int v = 0; v < c[0]; v++)
      for (int k = 0; k < dm; k++) buf[(size_t)k * c[0] + v] = w[(size_t)v * dm + k];
    free(w);
    qtensor_quantize(&m->lm_head, buf);
  } else {
    synth_q(&m->lm_head, buf, seed, 2 + 12 * (uint64_t)L);
  }
  free(buf);
}

static uint64_t model_hash(const QLlamaModel *m) {
  uint64_t h = qhash(&m->wte, 0);
  for (int l = 0; l < m->n_layers; l++) {
    const QLlamaBlock *b = &m->blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    h = h * 31 + qhash(&b->Wq, t0 + 1);
    h = h * 31 + qhash(&b->Wk, t0 + 2);
    h = h * 31 + qhash(&b->Wv, t0 + 3);
    h = h * 31 + qhash(&b->Wo, t0 + 7);
    h = h * 31 + qhash(&b->Wgate, t0 + 9);
    h = h * 31 + qhash(&b->Wup, t0 + 10);
    h = h * 31 + qhash(&b->Wdown, t0 + 11);
  }
  return h * 31 + qhash(&m->lm_head, 2 + 12 * (uint64_t)m->n_layers);
}

static void run_e2e(const E2E *e) {
  const uint64_t seed = 1234;
  double t0 = now_s();
  QLlamaModel m;
  build_model(&m, e, seed);
  double t1 = now_s();
  fprintf(stderr, "[%s] model built in %.1f s\n", e->name, t1 - t0);
  LlamaKV kv = q_llama_kv_create(&m);
  Tensor logits = mat(1, m.vocab);
  const int P = e->prompt, G = e->gen, steps = P + G;
  int *seq = malloc(sizeof(int) * (size_t)m.max_seq);
  syn_prompt(seq, P, seed, m.vocab);
  uint64_t *lh = malloc(sizeof(uint64_t) * (size_t)steps);
  int32_t *amax = malloc(sizeof(int32_t) * (size_t)steps);
  char nm[128]; long sv[1] = {m.vocab}, sh[1] = {2048};
  kv.len = 0;
  double tp0 = now_s();
  for (int i = 0; i < P; i++) {
    q_llama_decode_step(&m, &kv, seq[i], &logits);
    lh[i] = syn_hash_f32(logits.data, (size_t)m.vocab, 0);
    amax[i] = sample_argmax(&logits, 0);
    if (i % 64 == 0) fprintf(stderr, "[%s] prompt %d/%d %.1f s\n", e->name, i, P, now_s() - tp0);
  }
  double tp1 = now_s();
  snprintf(nm, sizeof nm, "e2e_%s_logits_prompt_last", e->name);
  if (m.vocab <= 32000) npy_f32(nm, logits.data, 1, sv); else npy_f32(nm, logits.data, 1, sh);
  int n = P, s;
  for (s = 0; s < G && n < m.max_seq; s++) {
    int nxt = sample_argmax(&logits, 0);
    seq[n++] = nxt;
    q_llama_decode_step(&m, &kv, nxt, &logits);
    lh[P + s] = syn_hash_f32(logits.data, (size_t)m.vocab, 0);
    amax[P + s] = sample_argmax(&logits, 0);
    if (s % 32 == 0) fprintf(stderr, "[%s] gen %d/%d %.1f s\n", e->name, s, G, now_s() - tp1);
  }
  double tg1 = now_s();
  snprintf(nm, sizeof nm, "e2e_%s_logits_final", e->name);
  if (m.vocab <= 32000) npy_f32(nm, logits.data, 1, sv); else npy_f32(nm, logits.data, 1, sh);
  char path[1024]; snprintf(path, sizeof path, "%s/e2e_%s.json", OUT, e->name);
  FILE *js = fopen(path, "w");
  fprintf(js, "{\n  \"name\": \"%s\", \"seed\": %llu, \"cfg\": [%d,%d,%d,%d,%d,%d,%d,%d],\n",
          e->name, (unsigned long long)seed, e->cfg[0], e->cfg[1], e->cfg[2], e->cfg[3], e->cfg[4],
          e->cfg[5], e->cfg[6], e->cfg[7]);
  fprintf(js, "  \"rope_base\": %.1f, \"eps\": 1e-5, \"tied\": %d, \"prompt_len\": %d, \"gen_len\": %d,\n",
          e->base, e->tied, P, s);
  fprintf(js, "  \"model_hash\": \"%016llx\",\n", (unsigned long long)model_hash(&m));
  fprintf(js, "  \"ref_prompt_s\": %.3f, \"ref_gen_s\": %.3f, \"ref_build_s\": %.1f,\n", tp1 - tp0, tg1 - tp1, t1 - t0);
  fprintf(js, "  \"prompt\": [");
  for (int i = 0; i < P; i++) fprintf(js, "%s%d", i ? "," : "", seq[i]);
  fprintf(js, "],\n  \"gen\": [");
  for (int i = P; i < n; i++) fprintf(js, "%s%d", i > P ? "," : "", seq[i]);
  fprintf(js, "],\n  \"argmax\": [");
  for (int i = 0; i < P + s; i++) fprintf(js, "%s%d", i ? "," : "", amax[i]);
  fprintf(js, "],\n  \"logit_hashes\": [");
  for (int i = 0; i < P + s; i++) fprintf(js, "%s\"%016llx\"", i ? "," : "", (unsigned long long)lh[i]);
  fprintf(js, "]\n}\n");
  fclose(js);
  fprintf(stderr, "[%s] done: prompt %.1f s, gen %.1f s\n", e->name, tp1 - tp0, tg1 - tp1);
  free(seq); free(lh); free(amax); tensor_free(&logits); llama_kv_free(&kv); q_llama_model_free(&m);
}

// ---------------------------------------------------------------------------
// Sampling: sample_token (sampler.c:54-143) on rows regenerated by the tests
// from the seeded generator, and the `llama` command's sampled generation loop.
// ---------------------------------------------------------------------------
// Row kinds: 0 = N(0, sigma) values; 1 = the same rounded to quarters (many exact
// ties, so the order of equal probabilities matters).
static void sample_row(float *r, int V, uint64_t tid, double sigma, int kind) {
  syn_fill(r, (size_t)V, 77, tid, sigma);
  if (kind == 1)
    for (int j = 0; j < V; j++) r[j] = rintf(r[j] * 4.0f) / 4.0f;
}

typedef struct { float t; int k; float p; } SParams;

static void fx_sample(FILE *js) {
  const struct { int V; uint64_t tid; double sigma; int kind; } rows[5] = {
      {32000, 1, 1.0, 0}, {32000, 2, 1.0, 1}, {128256, 3, 1.3, 0}, {128256, 4, 4.0, 1}, {1000, 5, 0.05, 0}};
  const SParams ps[9] = {{0.8f, 40, 0.95f}, {1.0f, 0, 0.9f}, {1.0f, 0, 1.0f}, {0.5f, 5, 0.0f}, {1.5f, 1000, 0.5f},
                         {1.0f, 1, 1.0f}, {0.0f, 40, 0.95f}, {2.0f, 0, 0.99f}, {0.7f, 200000, 0.3f}};
  fprintf(js, "  \"sample_cases\": [\n");
  int first = 1;
  for (int ri = 0; ri < 5; ri++) {
    const int V = rows[ri].V;
    Tensor L = mat(1, V);
    sample_row(L.data, V, rows[ri].tid, rows[ri].sigma, rows[ri].kind);
    for (int pi = 0; pi < 9; pi++) {
      Rng rng = rng_create(1000 + 10 * ri + pi);
      int tok[8];
      for (int d = 0; d < 8; d++) tok[d] = sample_token(&L, 0, ps[pi].t, ps[pi].k, ps[pi].p, &rng);
      fprintf(js, "%s    {\"V\": %d, \"tid\": %llu, \"sigma\": %.2f, \"kind\": %d, \"t\": %.9g, \"k\": %d, "
                  "\"p\": %.9g, \"seed\": %d, \"tokens\": [",
              first ? "" : ",\n", V, (unsigned long long)rows[ri].tid, rows[ri].sigma, rows[ri].kind,
              (double)ps[pi].t, ps[pi].k, (double)ps[pi].p, 1000 + 10 * ri + pi);
      for (int d = 0; d < 8; d++) fprintf(js, "%s%d", d ? "," : "", tok[d]);
      fprintf(js, "], \"state\": \"%016llx\"}", (unsigned long long)rng.state);
      first = 0;
    }
    tensor_free(&L);
  }
  fprintf(js, "\n  ],\n");
  // edge cases: one entry, all-equal logits, -inf logits, extreme temperatures and
  // top-k / top-p settings (rows rebuilt by the tests from these recipes)
  fprintf(js, "  \"edge_cases\": [\n");
  const struct { const char *row; float t; int k; float p; } ec[15] = {
      {"V1", 0.8f, 40, 0.95f}, {"V1", 2.0f, 0, 1.0f}, {"flat", 1.0f, 0, 0.5f}, {"flat", 0.7f, 64, 0.3f},
      {"flat", 1.0f, 4096, 1.0f}, {"plain", 1e-30f, 0, 0.9f}, {"plain", 1e3f, 40, 0.95f}, {"plain", 1.0f, 5000, 0.0f},
      {"plain", 1.0f, 0, 1e-7f}, {"plain", 1.0f, 0, 0.999999f}, {"plain", 0.9f, -3, 2.0f}, {"ninf", 0.8f, 40, 0.95f},
      {"ninf", 1.0f, 0, 0.99f}, {"wide", 0.8f, 40, 0.95f}, {"wide", 1.1f, 0, 0.9f}};
  for (int ci = 0; ci < 15; ci++) {
    int V = 5000;
    if (!strcmp(ec[ci].row, "V1")) V = 1;
    else if (!strcmp(ec[ci].row, "flat")) V = 4096;
    else if (!strcmp(ec[ci].row, "wide")) V = 131072;
    Tensor L = mat(1, V);
    if (V == 1) L.data[0] = 0.25f;
    else if (V == 4096) for (int j = 0; j < V; j++) L.data[j] = 1.5f;
    else if (V == 131072) sample_row(L.data, V, 61, 3.0, 1);
    else {
      sample_row(L.data, V, 60, 1.0, 0);
      if (!strcmp(ec[ci].row, "ninf")) for (int j = 0; j < V; j += 3) L.data[j] = -INFINITY;
    }
    Rng rng = rng_create(2024);
    int tok[5];
    for (int d = 0; d < 5; d++) tok[d] = sample_token(&L, 0, ec[ci].t, ec[ci].k, ec[ci].p, &rng);
    fprintf(js, "%s    {\"row\": \"%s\", \"t\": %.9g, \"k\": %d, \"p\": %.9g, \"tokens\": [%d,%d,%d,%d,%d], "
                "\"state\": \"%016llx\"}", ci ? ",\n" : "", ec[ci].row, (double)ec[ci].t, ec[ci].k, (double)ec[ci].p,
            tok[0], tok[1], tok[2], tok[3], tok[4], (unsigned long long)rng.state);
    tensor_free(&L);
  }
  fprintf(js, "\n  ],\n");
  // rng_uniform's first values from a few seeds (seed 0 maps to the fixed constant)
  fprintf(js, "  \"uniform\": [");
  const unsigned long long seeds[3] = {0, 1, 1234};
  for (int i = 0; i < 3; i++) {
    Rng r = rng_create(seeds[i]);
    fprintf(js, "%s[%llu", i ? ", " : "", seeds[i]);
    for (int d = 0; d < 4; d++) { float u = rng_uniform(&r); uint32_t b; memcpy(&b, &u, 4); fprintf(js, ", %u", b); }
    fprintf(js, "]");
  }
  fprintf(js, "],\n");
}

// The LLMQ branch of the `llama` command (main.c:658-669) on the tiny model:
// rng_create(1234) once, then per input line: kv.len = 0, the prompt through
// q_llama_decode_step, and n_new sampled tokens (T 0.8, top-k 40, top-p 0.95).
static void fx_cli(FILE *js) {
  QLlamaModel m;
  build_model(&m, &CASES[0], 1234);
  LlamaKV kv = q_llama_kv_create(&m);
  Tensor logits = mat(1, m.vocab);
  Rng rng = rng_create(1234);
  const int lens[2] = {20, 7}, n_new = 40;
  int *seq = malloc(sizeof(int) * (size_t)m.max_seq);
  fprintf(js, "  \"cli\": {\"model\": \"tiny\", \"seed\": 1234, \"n_new\": %d, \"lines\": [\n", n_new);
  for (int li = 0; li < 2; li++) {
    int n = lens[li];
    syn_prompt(seq, n, 4321 + li, m.vocab);
    fprintf(js, "%s    {\"prompt\": [", li ? ",\n" : "");
    for (int i = 0; i < n; i++) fprintf(js, "%s%d", i ? "," : "", seq[i]);
    kv.len = 0;
    for (int i = 0; i < n; i++) q_llama_decode_step(&m, &kv, seq[i], &logits);
    fprintf(js, "], \"gen\": [");
    for (int s = 0; s < n_new && n < m.max_seq; s++) {
      int nxt = sample_token(&logits, 0, 0.8f, 40, 0.95f, &rng);
      seq[n++] = nxt;
      fprintf(js, "%s%d", s ? "," : "", nxt);
      q_llama_decode_step(&m, &kv, nxt, &logits);
    }
    fprintf(js, "]}");
  }
  fprintf(js, "\n  ]},\n");
  free(seq); tensor_free(&logits); llama_kv_free(&kv); q_llama_model_free(&m);
}

// ---------------------------------------------------------------------------
// fp32 (LLMA) path: the generator's N(0, 0.02) weights, not quantized.
// ---------------------------------------------------------------------------
typedef struct { const char *name; int32_t cfg[8]; float base; int tied, prompt, gen; } E2EF;
static const E2EF FCASES[2] = {
  {"tiny", {32000, 288, 6, 6, 2, 48, 768, 256}, 10000.0f, 0, 32, 32},
  {"mid", {32000, 1024, 4, 16, 4, 64, 2816, 256}, 500000.0f, 1, 40, 24},
};

static void build_fmodel(LlamaModel *m, const E2EF *e, uint64_t seed) {
  const int32_t *c = e->cfg;
  *m = llama_model_create(c[0], c[1], c[2], c[3], c[4], c[5], c[6], c[7], e->base, 1e-5f);
  const int dm = c[1], L = c[2];
  syn_fill(m->wte.data, (size_t)c[0] * dm, seed, 0, 0.02);
  for (int l = 0; l < L; l++) {
    LlamaBlock *b = &m->blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l;
    for (int j = 0; j < dm; j++) { b->attn_norm.data[j] = 1.0f; b->ffn_norm.data[j] = 1.0f; }
    memset(b->b_q.data, 0, b->b_q.size * 4); memset(b->b_k.data, 0, b->b_k.size * 4);
    memset(b->b_v.data, 0, b->b_v.size * 4);
    syn_fill(b->Wq.data, b->Wq.size, seed, t0 + 1, 0.02);
    syn_fill(b->Wk.data, b->Wk.size, seed, t0 + 2, 0.02);
    syn_fill(b->Wv.data, b->Wv.size, seed, t0 + 3, 0.02);
    syn_fill(b->Wo.data, b->Wo.size, seed, t0 + 7, 0.02);
    syn_fill(b->Wgate.data, b->Wgate.size, seed, t0 + 9, 0.02);
    syn_fill(b->Wup.data, b->Wup.size, seed, t0 + 10, 0.02);
    syn_fill(b->Wdown.data, b->Wdown.size, seed, t0 + 11, 0.02);
  }
  for (int j = 0; j < dm; j++) m->final_norm.data[j] = 1.0f;
  if (e->tied) {
    for (int v = 0; v < c[0]; v++)
      for (int k = 0; k < dm; k++) m->lm_head.data[(size_t)k * c[0] + v] = m->wte.data[(size_t)v * dm + k];
  } else {
    syn_fill(m->lm_head.data, m->lm_head.size, seed, 2 + 12 * (uint64_t)L, 0.02);
  }
}

// Digest of every tensor of an fp32 model in the canonical order (llama.c:198-219).
static uint64_t fmodel_hash(const LlamaModel *m) {
  uint64_t h = syn_hash_f32(m->wte.data, m->wte.size, 0);
  for (int l = 0; l < m->n_layers; l++) {
    const LlamaBlock *b = &m->blocks[l];
    const Tensor *t[12] = {&b->attn_norm, &b->Wq, &b->Wk, &b->Wv, &b->b_q, &b->b_k, &b->b_v, &b->Wo,
                           &b->ffn_norm, &b->Wgate, &b->Wup, &b->Wdown};
    for (int i = 0; i < 12; i++) h = h * 31 + syn_hash_f32(t[i]->data, t[i]->size, 0);
  }
  h = h * 31 + syn_hash_f32(m->final_norm.data, m->final_norm.size, 0);
  return h * 31 + syn_hash_f32(m->lm_head.data, m->lm_head.size, 0);
}

static void run_e2e_f32(const E2EF *e) {
  const uint64_t seed = 1234;
  LlamaModel m;
  build_fmodel(&m, e, seed);
  LlamaKV kv = llama_kv_create(&m);
  Tensor logits = mat(1, m.vocab);
  const int P = e->prompt, G = e->gen;
  int *seq = malloc(sizeof(int) * (size_t)m.max_seq);
  uint64_t *lh = malloc(sizeof(uint64_t) * (size_t)(P + G));
  syn_prompt(seq, P, seed, m.vocab);
  kv.len = 0;
  for (int i = 0; i < P; i++) {
    llama_decode_step(&m, &kv, seq[i], &logits);
    lh[i] = syn_hash_f32(logits.data, (size_t)m.vocab, 0);
  }
  // the batched forward over the same prompt (llama.c:167-186): one row per position
  uint64_t *fh = malloc(sizeof(uint64_t) * (size_t)P);
  {
    Tensor L = mat(P, m.vocab);
    llama_model_forward(&m, seq, P, &L);
    for (int i = 0; i < P; i++) fh[i] = syn_hash_f32(L.data + (size_t)i * m.vocab, (size_t)m.vocab, 0);
    tensor_free(&L);
  }
  char nm[128]; long sv[1] = {m.vocab};
  snprintf(nm, sizeof nm, "e2e_f32_%s_logits_prompt_last", e->name);
  npy_f32(nm, logits.data, 1, sv);
  int n = P;
  for (int s = 0; s < G; s++) {
    int nxt = sample_argmax(&logits, 0);
    seq[n++] = nxt;
    llama_decode_step(&m, &kv, nxt, &logits);
    lh[P + s] = syn_hash_f32(logits.data, (size_t)m.vocab, 0);
  }
  snprintf(nm, sizeof nm, "e2e_f32_%s_logits_final", e->name);
  npy_f32(nm, logits.data, 1, sv);
  char path[1024]; snprintf(path, sizeof path, "%s/e2e_f32_%s.json", OUT, e->name);
  FILE *js = fopen(path, "w");
  fprintf(js, "{\n  \"name\": \"%s\", \"seed\": %llu, \"cfg\": [%d,%d,%d,%d,%d,%d,%d,%d],\n", e->name,
          (unsigned long long)seed, e->cfg[0], e->cfg[1], e->cfg[2], e->cfg[3], e->cfg[4], e->cfg[5], e->cfg[6],
          e->cfg[7]);
  fprintf(js, "  \"rope_base\": %.1f, \"eps\": 1e-5, \"tied\": %d,\n", e->base, e->tied);
  fprintf(js, "  \"model_hash\": \"%016llx\",\n  \"prompt\": [", (unsigned long long)fmodel_hash(&m));
  for (int i = 0; i < P; i++) fprintf(js, "%s%d", i ? "," : "", seq[i]);
  fprintf(js, "],\n  \"gen\": [");
  for (int i = P; i < n; i++) fprintf(js, "%s%d", i > P ? "," : "", seq[i]);
  fprintf(js, "],\n  \"logit_hashes\": [");
  for (int i = 0; i < P + G; i++) fprintf(js, "%s\"%016llx\"", i ? "," : "", (unsigned long long)lh[i]);
  fprintf(js, "],\n  \"forward_hashes\": [");
  for (int i = 0; i < P; i++) fprintf(js, "%s\"%016llx\"", i ? "," : "", (unsigned long long)fh[i]);
  fprintf(js, "]\n}\n");
  fclose(js);
  free(seq); free(lh); free(fh); tensor_free(&logits); llama_kv_free(&kv); llama_model_free(&m);
}

// The LLMA branch of the `llama` command (main.c:686-700) on the tiny fp32 model:
// a generator of its own (rng_create(1234)), per line kv.len = 0, the prompt
// through llama_decode_step, n_new sampled tokens.
static void fx_cli_f32(FILE *js) {
  LlamaModel m;
  build_fmodel(&m, &FCASES[0], 1234);
  LlamaKV kv = llama_kv_create(&m);
  Tensor logits = mat(1, m.vocab);
  Rng rng = rng_create(1234);
  const int lens[2] = {20, 7}, n_new = 40;
  int *seq = malloc(sizeof(int) * (size_t)m.max_seq);
  fprintf(js, "  \"cli_f32\": {\"model\": \"tiny\", \"seed\": 1234, \"n_new\": %d, \"lines\": [\n", n_new);
  for (int li = 0; li < 2; li++) {
    int n = lens[li];
    syn_prompt(seq, n, 4321 + li, m.vocab);
    fprintf(js, "%s    {\"prompt\": [", li ? ",\n" : "");
    for (int i = 0; i < n; i++) fprintf(js, "%s%d", i ? "," : "", seq[i]);
    kv.len = 0;
    for (int i = 0; i < n; i++) llama_decode_step(&m, &kv, seq[i], &logits);
    fprintf(js, "], \"gen\": [");
    for (int s = 0; s < n_new && n < m.max_seq; s++) {
      int nxt = sample_token(&logits, 0, 0.8f, 40, 0.95f, &rng);
      seq[n++] = nxt;
      fprintf(js, "%s%d", s ? "," : "", nxt);
      llama_decode_step(&m, &kv, nxt, &logits);
    }
    fprintf(js, "]}");
  }
  fprintf(js, "\n  ]},\n");
  free(seq); tensor_free(&logits); llama_kv_free(&kv); llama_model_free(&m);
}

// ---------------------------------------------------------------------------
// GPT-2 (GPTC) KV decode: the reference's own model (gpt_create), every weight
// then overwritten from the generator by its position t in the GPTC order
// (checkpoint.c:17-44) as tensor id t: matrices, embeddings, biases and
// LayerNorm betas N(0, 0.02); gammas 1 + N(0, 0.1).
// ---------------------------------------------------------------------------
typedef struct { const char *name; int32_t cfg[6]; int prompt, gen; } GCase;   // vocab, dm, heads, layers, ff, seq
static const GCase GCASES[3] = {
  {"tiny", {512, 64, 4, 2, 256, 128}, 48, 48},
  {"gpt2s", {50257, 768, 12, 12, 3072, 1024}, 32, 32},
  // GPT-2-small's width, heads and context with 2 layers and a short vocabulary,
  // decoded to position 1000 of its 1024
  {"long", {2048, 768, 12, 2, 3072, 1024}, 32, 968},
};

static int gpt_list(GPT *m, Tensor **t) {
  int n = 0;
  t[n++] = &m->wte; t[n++] = &m->wpe;
  for (int l = 0; l < m->n_layers; l++) {
    BlockWeights *b = &m->blocks[l];
    Tensor *blk[16] = {&b->W_q, &b->W_k, &b->W_v, &b->W_o, &b->b_q, &b->b_k, &b->b_v, &b->b_o,
                       &b->gamma1, &b->beta1, &b->gamma2, &b->beta2, &b->ff_W1, &b->ff_b1, &b->ff_W2, &b->ff_b2};
    for (int i = 0; i < 16; i++) t[n++] = blk[i];
  }
  t[n++] = &m->ln_f_gamma; t[n++] = &m->ln_f_beta; t[n++] = &m->lm_head;
  return n;
}

static void build_gpt(GPT *m, const GCase *c, uint64_t seed) {
  *m = gpt_create(c->cfg[0], c->cfg[1], c->cfg[2], c->cfg[3], c->cfg[4], c->cfg[5]);
  Tensor **t = malloc(sizeof(Tensor*) * (size_t)(5 + 16 * m->n_layers));
  const int n = gpt_list(m, t);
  for (int i = 0; i < n; i++) {
    const int in_layer = i >= 2 && i < 2 + 16 * m->n_layers, slot = in_layer ? (i - 2) % 16 : -1;
    const int gamma = (in_layer && (slot == 8 || slot == 10)) || i == n - 3;
    syn_fill(t[i]->data, t[i]->size, seed, (uint64_t)i, gamma ? 0.1 : 0.02);
    if (gamma) for (size_t k = 0; k < t[i]->size; k++) t[i]->data[k] = 1.0f + t[i]->data[k];
  }
  free(t);
}

static uint64_t gpt_hash(GPT *m) {
  Tensor **t = malloc(sizeof(Tensor*) * (size_t)(5 + 16 * m->n_layers));
  const int n = gpt_list(m, t);
  uint64_t h = 0;
  for (int i = 0; i < n; i++) h = h * 31 + syn_hash_f32(t[i]->data, t[i]->size, 0);
  free(t);
  return h;
}

static void run_gpt(const GCase *c) {
  const uint64_t seed = 1234;
  GPT m;
  build_gpt(&m, c, seed);
  KVCache kv = gpt_kvcache_create(&m);
  Tensor logits = mat(1, m.vocab_size);
  const int P = c->prompt, G = c->gen, V = m.vocab_size;
  int *seq = malloc(sizeof(int) * (size_t)(P + G + 1));
  uint64_t *lh = malloc(sizeof(uint64_t) * (size_t)(P + G));
  syn_prompt(seq, P, seed, V);
  const double t0 = now_s();
  for (int i = 0; i < P; i++) {
    gpt_decode_step(&m, &kv, seq[i], &logits);
    lh[i] = syn_hash_f32(logits.data, (size_t)V, 0);
  }
  char nm[128]; long sh[1] = {V < 2048 ? V : 2048};
  snprintf(nm, sizeof nm, "gpt_%s_logits_prompt_last", c->name);
  npy_f32(nm, logits.data, 1, sh);
  int n = P;
  for (int s = 0; s < G; s++) {
    const int nxt = sample_argmax(&logits, 0);
    seq[n++] = nxt;
    gpt_decode_step(&m, &kv, nxt, &logits);
    lh[P + s] = syn_hash_f32(logits.data, (size_t)V, 0);
  }
  const double t1 = now_s();
  snprintf(nm, sizeof nm, "gpt_%s_logits_final", c->name);
  npy_f32(nm, logits.data, 1, sh);
  char path[1024]; snprintf(path, sizeof path, "%s/gpt_%s.json", OUT, c->name);
  FILE *js = fopen(path, "w");
  fprintf(js, "{\n  \"name\": \"%s\", \"seed\": %llu, \"cfg\": [%d,%d,%d,%d,%d,%d],\n", c->name,
          (unsigned long long)seed, c->cfg[0], c->cfg[1], c->cfg[2], c->cfg[3], c->cfg[4], c->cfg[5]);
  fprintf(js, "  \"model_hash\": \"%016llx\", \"ref_decode_s\": %.3f,\n  \"prompt\": [",
          (unsigned long long)gpt_hash(&m), t1 - t0);
  for (int i = 0; i < P; i++) fprintf(js, "%s%d", i ? "," : "", seq[i]);
  fprintf(js, "],\n  \"gen\": [");
  for (int i = P; i < n; i++) fprintf(js, "%s%d", i > P ? "," : "", seq[i]);
  fprintf(js, "],\n  \"logit_hashes\": [");
  for (int i = 0; i < P + G; i++) fprintf(js, "%s\"%016llx\"", i ? "," : "", (unsigned long long)lh[i]);
  fprintf(js, "]\n}\n");
  fclose(js);
  free(seq); free(lh); tensor_free(&logits); gpt_kvcache_free(&kv); gpt_free(&m);
}

// ---------------------------------------------------------------------------
// q_llama_quantize_from (llama.c:490-511): an fp32 model from the generator
// quantized by the reference, then its decode steps.  Tensor ids: the fp32
// path's (build_fmodel), plus gains 1 + N(0, g) and biases N(0, b) at ids
// 1000 + 8 l + {0 attn_norm, 1 b_q, 2 b_k, 3 b_v, 4 ffn_norm} and 999 for the
// final norm; lm_head's column 5 is zeroed (an all-zero column: scale 1).
// ---------------------------------------------------------------------------
typedef struct { const char *name; int32_t cfg[8]; float gsig, bsig; int n_ids; int ids[8]; } QFCase;
static const QFCase QFCASES[2] = {
  // selftest [21]'s model shape and token ids (selftest.c:1215-1250)
  {"selftest21", {32, 8, 2, 4, 2, 2, 16, 64}, 0.0f, 0.0f, 6, {3, 7, 1, 9, 2, 5}},
  // gains and biases away from 1 and 0, head size 16, three query heads per KV head
  {"biased", {300, 96, 2, 6, 2, 16, 160, 48}, 0.1f, 0.1f, 8, {11, 290, 7, 3, 150, 42, 99, 0}},
};

static void qf_fill(Tensor *t, uint64_t tid, double sig, float base) {
  syn_fill(t->data, t->size, 21, tid, sig > 0 ? sig : 0.0);
  for (size_t i = 0; i < t->size; i++) t->data[i] = sig > 0 ? base + t->data[i] : base;
}

static void run_qfrom(const QFCase *c) {
  const int32_t *g = c->cfg;
  LlamaModel f = llama_model_create(g[0], g[1], g[2], g[3], g[4], g[5], g[6], g[7], 10000.0f, 1e-5f);
  const int L = g[2];
  syn_fill(f.wte.data, f.wte.size, 21, 0, 1.0);
  for (int l = 0; l < L; l++) {
    LlamaBlock *b = &f.blocks[l];
    const uint64_t t0 = 1 + 12 * (uint64_t)l, u = 1000 + 8 * (uint64_t)l;
    syn_fill(b->Wq.data, b->Wq.size, 21, t0 + 1, 0.3);
    syn_fill(b->Wk.data, b->Wk.size, 21, t0 + 2, 0.3);
    syn_fill(b->Wv.data, b->Wv.size, 21, t0 + 3, 0.3);
    syn_fill(b->Wo.data, b->Wo.size, 21, t0 + 7, 0.3);
    syn_fill(b->Wgate.data, b->Wgate.size, 21, t0 + 9, 0.3);
    syn_fill(b->Wup.data, b->Wup.size, 21, t0 + 10, 0.3);
    syn_fill(b->Wdown.data, b->Wdown.size, 21, t0 + 11, 0.3);
    qf_fill(&b->attn_norm, u + 0, c->gsig, 1.0f);
    qf_fill(&b->b_q, u + 1, c->bsig, 0.0f);
    qf_fill(&b->b_k, u + 2, c->bsig, 0.0f);
    qf_fill(&b->b_v, u + 3, c->bsig, 0.0f);
    qf_fill(&b->ffn_norm, u + 4, c->gsig, 1.0f);
  }
  qf_fill(&f.final_norm, 999, c->gsig, 1.0f);
  syn_fill(f.lm_head.data, f.lm_head.size, 21, 2 + 12 * (uint64_t)L, 0.3);
  for (int k = 0; k < g[1]; k++) f.lm_head.data[(size_t)k * g[0] + 5] = 0.0f;

  QLlamaModel m = q_llama_quantize_from(&f);
  LlamaKV kv = q_llama_kv_create(&m);
  Tensor logits = mat(1, m.vocab);
  const int G = 12, S = c->n_ids + G;
  float *all = malloc(sizeof(float) * (size_t)S * m.vocab);
  int seq[32], n = 0;
  for (int i = 0; i < c->n_ids; i++) {
    seq[n] = c->ids[i];
    q_llama_decode_step(&m, &kv, seq[n], &logits);
    memcpy(all + (size_t)n++ * m.vocab, logits.data, sizeof(float) * m.vocab);
  }
  for (int s = 0; s < G; s++) {
    seq[n] = sample_argmax(&logits, 0);
    q_llama_decode_step(&m, &kv, seq[n], &logits);
    memcpy(all + (size_t)n++ * m.vocab, logits.data, sizeof(float) * m.vocab);
  }
  char nm[128]; long sv[2] = {S, m.vocab};
  snprintf(nm, sizeof nm, "qfrom_%s_logits", c->name);
  npy_f32(nm, all, 2, sv);
  char path[1024]; snprintf(path, sizeof path, "%s/qfrom_%s.json", OUT, c->name);
  FILE *js = fopen(path, "w");
  fprintf(js, "{\n  \"name\": \"%s\", \"seed\": 21, \"cfg\": [%d,%d,%d,%d,%d,%d,%d,%d],\n", c->name, g[0], g[1],
          g[2], g[3], g[4], g[5], g[6], g[7]);
  fprintf(js, "  \"rope_base\": 10000.0, \"eps\": 1e-5, \"gain_sigma\": %.2f, \"bias_sigma\": %.2f,\n", c->gsig,
          c->bsig);
  fprintf(js, "  \"fp32_hash\": \"%016llx\", \"model_hash\": \"%016llx\",\n  \"tokens\": [",
          (unsigned long long)fmodel_hash(&f), (unsigned long long)model_hash(&m));
  for (int i = 0; i < S; i++) fprintf(js, "%s%d", i ? "," : "", seq[i]);
  fprintf(js, "],\n  \"n_prompt\": %d\n}\n", c->n_ids);
  fclose(js);
  free(all); tensor_free(&logits); llama_kv_free(&kv); q_llama_model_free(&m); llama_model_free(&f);
}

int main(int argc, char **argv) {
  if (argc < 3) { fprintf(stderr, "usage: gen_golden <outdir> ops|gqa8192|sample|e2e <name>\n"); return 2; }
  OUT = argv[1];
  if (!strcmp(argv[2], "ops")) {
    char path[1024]; snprintf(path, sizeof path, "%s/ops.json", OUT);
    FILE *js = fopen(path, "w");
    fprintf(js, "{\n");
    fx_quant(js);
    qmm_case("qmm_1x64x48", 1, 64, 48, 5, 1.0, 1, js);
    qmm_case("qmm_3x300x17", 3, 300, 17, 6, 1.0, 1, js);
    qmm_case("qmm_8x256x96", 8, 256, 96, 8, 0.05, 1, js);
    qmm_case("qmm_2x1024x1024", 2, 1024, 1024, 9, 1.0, 0, js);   // threaded path (K*N >= 2^19)
    fx_rmsnorm(js);
    fx_rope(js);
    const int Ts[3] = {1, 512, 2048};
    for (int i = 0; i < 3; i++) gqa_case(i, Ts[i], js);
    const int shapes[4][2] = {{4096, 4096}, {14336, 4096}, {4096, 14336}, {128256, 4096}};
    for (int i = 0; i < 4; i++) qmm_op(i, shapes[i][0], shapes[i][1], js);
    fprintf(js, "  \"done\": true\n}\n");
    fclose(js);
    return 0;
  }
  if (!strcmp(argv[2], "gqa8192")) {
    char path[1024]; snprintf(path, sizeof path, "%s/gqa8192.json", OUT);
    FILE *js = fopen(path, "w");
    fprintf(js, "{\n");
    gqa_case(3, 8192, js);
    fprintf(js, "  \"done\": true\n}\n");
    fclose(js);
    return 0;
  }
  if (!strcmp(argv[2], "sample")) {
    char path[1024]; snprintf(path, sizeof path, "%s/sample.json", OUT);
    FILE *js = fopen(path, "w");
    fprintf(js, "{\n");
    fx_sample(js);
    fx_cli(js);
    fx_cli_f32(js);
    fprintf(js, "  \"done\": true\n}\n");
    fclose(js);
    return 0;
  }
  if (!strcmp(argv[2], "llmqhash") && argc > 3) {
    QLlamaModel m;
    if (q_llama_model_load(argv[3], &m) != 0) return 1;
    printf("%016llx\n", (unsigned long long)model_hash(&m));
    q_llama_model_free(&m);
    return 0;
  }
  if (!strcmp(argv[2], "e2e_f32") && argc > 3) {
    for (int i = 0; i < 2; i++) if (!strcmp(argv[3], FCASES[i].name)) { run_e2e_f32(&FCASES[i]); return 0; }
  }
  if (!strcmp(argv[2], "llmahash") && argc > 3) {
    LlamaModel m;
    if (llama_model_load(argv[3], &m) != 0) return 1;
    printf("%016llx\n", (unsigned long long)fmodel_hash(&m));
    llama_model_free(&m);
    return 0;
  }
  if (!strcmp(argv[2], "gpt") && argc > 3) {
    for (int i = 0; i < 3; i++) if (!strcmp(argv[3], GCASES[i].name)) { run_gpt(&GCASES[i]); return 0; }
  }
  if (!strcmp(argv[2], "gpthash") && argc > 3) {
    GPT m;
    if (gpt_load(argv[3], &m) != 0) return 1;
    printf("%016llx\n", (unsigned long long)gpt_hash(&m));
    gpt_free(&m);
    return 0;
  }
  if (!strcmp(argv[2], "qfrom")) {
    for (int i = 0; i < 2; i++) run_qfrom(&QFCASES[i]);
    return 0;
  }
  if (!strcmp(argv[2], "e2e") && argc > 3) {
    for (int i = 0; i < 3; i++) if (!strcmp(argv[3], CASES[i].name)) { run_e2e(&CASES[i]); return 0; }
  }
  fprintf(stderr, "unknown request\n");
  return 2;
}
