// oracle.h - CPU restatement of the reference's int8 LLaMA decode path.
//
// TEST INFRASTRUCTURE ONLY.  This is the checker: tests/, the smoke check and
// bench.py's cpu_baseline leg may build against it, nothing else.  The GPU
// library never links, loads or calls it, and has no CPU fallback to it.
//
// Every function restates one piece of /root/reference (file:line given at each
// definition) in plain C11 with the reference's evaluation order, so that when
// it is compiled like the reference (ISO C11: no floating-point contraction, no
// reassociation) it reproduces the reference's results bit for bit.  That claim
// is pinned by tests/test_oracle_golden.py against fixtures written by the
// compiled reference itself (tests/golden/gen_golden.c).
//
// Weight layout is the reference's: a (rows = in, cols = out) matrix is int8
// row-major with one fp32 scale per column (quant.h:22-27).
#ifndef QL_ORACLE_H
#define QL_ORACLE_H

#include <stdint.h>
#include <stddef.h>

typedef struct { int rows, cols; int8_t *q; float *scale; } OrQT;

typedef struct {
  float *attn_norm, *ffn_norm, *b_q, *b_k, *b_v;
  OrQT Wq, Wk, Wv, Wo, Wgate, Wup, Wdown;
} OrBlock;

typedef struct {
  int vocab, d_model, n_layers, n_heads, n_kv, head_dim, d_ff, max_seq;
  float rope_base, eps;
  OrQT wte;
  OrBlock *blocks;
  float *final_norm;
  OrQT lm_head;
} OrModel;

// k, v: [n_layers][max_seq][kv_dim] fp32, as llama.c:513-526 (one block per layer).
typedef struct { int n_layers, max_seq, kv_dim, len; float *k, *v; } OrKV;

void or_set_threads(int n);          // 0 = all online CPUs (TF_THREADS semantics)
int  or_get_threads(void);

void or_quantize_int8_percol(const float *w, int rows, int cols, int8_t *q, float *scale);
void or_dequantize_int8_percol(const int8_t *q, const float *scale, int rows, int cols, float *w);
void or_qacc_columns(const int8_t *qa, const int8_t *qw, int K, int N, int32_t *acc);
void or_qmatmul(const float *A, int M, const OrQT *W, float *C);
// qmatmul with its intermediates exposed: qa[M*K], as[M], acc[M*N].
void or_qmatmul_ex(const float *A, int M, const OrQT *W, float *C,
                   int8_t *qa_out, float *as_out, int32_t *acc_out);
void or_rmsnorm(const float *x, int rows, int cols, const float *gamma, float eps, float *y);
void or_rope_heads_pos(float *x, int rows, int cols, int n_heads, float base, int pos0);
void or_gqa_forward(const float *Q, const float *K, const float *V, int n, int H, int KVH,
                    int hd, float *att, float *O);
void or_attn_decode(const float *q, const float *kc, const float *vc, int kvd, int pos,
                    int n_heads, int n_kv, int hd, float *sc, float *o);
int  or_argmax(const float *r, int n);
// sampler.c:24-45 (state in, state out) and sampler.c:54-143
uint64_t or_rng_create(uint64_t seed);
float or_rng_uniform(uint64_t *state);
int  or_sample_token(const float *l, int V, float temperature, int top_k, float top_p, uint64_t *state);

// Model from the seeded generator (synth.h), quantized as llama.c:490-511 does.
int  or_model_synth(OrModel *m, const int32_t cfg[8], float rope_base, float eps,
                    uint64_t seed, int tied);
// Model whose weights are copied in from caller buffers laid out like the
// reference (used to take weights back from the GPU for the CPU baseline).
int  or_model_alloc(OrModel *m, const int32_t cfg[8], float rope_base, float eps);
void or_model_free(OrModel *m);
uint64_t or_model_hash(const OrModel *m);

int  or_kv_create(OrKV *kv, const OrModel *m);
void or_kv_free(OrKV *kv);
void or_decode_step(const OrModel *m, OrKV *kv, int token, float *logits);

// fp32 (LLMA) model, reference layout: every matrix (rows = in, cols = out) f32
// row-major (llama.h:19-37, 58-66).
typedef struct {
  float *attn_norm, *ffn_norm, *b_q, *b_k, *b_v;
  float *Wq, *Wk, *Wv, *Wo, *Wgate, *Wup, *Wdown;
} OrFBlock;

typedef struct {
  int vocab, d_model, n_layers, n_heads, n_kv, head_dim, d_ff, max_seq;
  float rope_base, eps;
  float *wte;
  OrFBlock *blocks;
  float *final_norm;
  float *lm_head;
} OrFModel;

void or_matmul_row(const float *a, const float *W, int K, int N, float *c);
// Weights N(0, 0.02) from the generator with the int8 model's tensor ids, not quantized.
int  or_fmodel_synth(OrFModel *m, const int32_t cfg[8], float rope_base, float eps, uint64_t seed, int tied);
void or_fmodel_free(OrFModel *m);
int  or_fkv_create(OrKV *kv, const OrFModel *m);
void or_f32_decode_step(const OrFModel *m, OrKV *kv, int token, float *logits);
// llama.c:490-511: the int8 model of an fp32 model (allocates m).
int  or_model_quantize_from(OrModel *m, const OrFModel *f);

// Bitwise mismatches of got[i] against the host libm expf at bit pattern start+i.
long long or_expf_mismatches(uint32_t start, uint32_t count, const float *got);

// GPT-2 (GPTC) fp32 model, reference layout (model.h:8-31): matrices (rows = in,
// cols = out) f32 row-major; wpe (max_seq, d_model); lm_head (d_model, vocab).
typedef struct {
  float *Wq, *Wk, *Wv, *Wo, *bq, *bk, *bv, *bo, *g1, *be1, *g2, *be2, *W1, *bf1, *W2, *bf2;
} OrGBlock;

typedef struct {
  int vocab, d_model, n_heads, n_layers, d_ff, max_seq;   // the GPTC config order (checkpoint.c:75-77)
  float *wte, *wpe;
  OrGBlock *blocks;
  float *lnf_g, *lnf_b, *lm_head;
} OrGPT;

void or_layernorm(const float *x, int rows, int cols, const float *gamma, const float *beta, float eps, float *y);
void or_gelu(const float *x, size_t n, float *y);
int  or_gpt_alloc(OrGPT *m, const int32_t cfg[6]);
int  or_gpt_synth(OrGPT *m, const int32_t cfg[6], uint64_t seed);
void or_gpt_free(OrGPT *m);
int  or_gpt_tensors(const OrGPT *m, float **list, size_t *sizes);    // GPTC order (checkpoint.c:17-44)
uint64_t or_gpt_hash(const OrGPT *m);
int  or_gkv_create(OrKV *kv, const OrGPT *m);                       // kv_dim = d_model
void or_gpt_decode_step(const OrGPT *m, OrKV *kv, int token, float *logits);
long long or_tanhf_mismatches(uint32_t start, uint32_t count, const float *got);

#endif
