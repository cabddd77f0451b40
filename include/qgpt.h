// qgpt.h - C ABI of the MI355X library for the reference's GPT-2 (GPTC) KV-cache
// decode (model.c:437-520) and its checkpoint format (checkpoint.c:17-174).
//
// Same names, argument meaning and error behaviour as model.h / checkpoint.h:
//   * GPT is the reference's host model (fp32 tensors in host memory, as gpt_load
//     fills them); the library never changes it.
//   * a KVCache takes a device copy of the model's weights when it is created,
//     and again when gpt_decode_step is given another model of the same shape;
//     host edits of the same tensors made after that are not seen.  Its K[l] /
//     V[l] are device views laid out [n_heads][max_seq_len][head_dim]; callers
//     only read and reset len, as in the reference (main.c:139-150).
//   * logits of gpt_decode_step are host memory (1, vocab), bit-identical to the
//     reference's: every float operation is the reference's, in its order.
//   * Errors: loaders print "Error: ..." and return nonzero; the void calls
//     print and abort (a bad token or position, a device error).
//
// Standalone this header defines every type it needs.  Inside the reference's
// build it takes the place of model.h's cache section (model.h:120-137), where
// model.h has already defined GPT and tensor.h Tensor.
#ifndef QGPT_H
#define QGPT_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// tensor.h:10-16
#if !defined(TENSOR_H) && !defined(QL_TENSOR_DEFINED)
#define QL_TENSOR_DEFINED
typedef struct {
  float *data;
  float *grad;
  int *shape;
  int ndim;
  size_t size;
} Tensor;
#endif

#ifndef MODEL_H
// model.h:8-31 (fp32, host)
typedef struct {
  Tensor W_q, W_k, W_v, W_o;      // (d_model, d_model)
  Tensor b_q, b_k, b_v, b_o;      // (d_model)
  Tensor gamma1, beta1;           // LayerNorm 1 (d_model)
  Tensor gamma2, beta2;           // LayerNorm 2 (d_model)
  Tensor ff_W1, ff_b1;            // (d_model, d_ff), (d_ff)
  Tensor ff_W2, ff_b2;            // (d_ff, d_model), (d_model)
} BlockWeights;

typedef struct {
  int vocab_size, d_model, n_heads, n_layers, d_ff, max_seq_len;
  Tensor wte, wpe;                // (vocab, d_model), (max_seq_len, d_model)
  BlockWeights *blocks;
  Tensor ln_f_gamma, ln_f_beta;
  Tensor lm_head;                 // (d_model, vocab)
} GPT;
#endif

// model.h:124-129 plus the device-side state
typedef struct {
  int n_layers, d_model, n_heads, max_seq_len;
  int len;            // positions cached; callers may reset it to 0 to restart
  Tensor *K;          // n_layers device views
  Tensor *V;
  void *dev;          // library-private
} KVCache;

// checkpoint.c:129-174  Read a 'GPTC' v2 checkpoint into a host GPT.
int gpt_load(const char *path, GPT *out);
// checkpoint.c:62-112  Write one (same byte order), through path.tmp renamed
// over path only once complete: a failed save leaves an existing file intact.
int gpt_save(const char *path, const GPT *m);
// model.c:95-122 (gpt_free): the host model's memory
void gpt_free(GPT *m);
// model.c:437-448  A device cache of max_seq_len positions per layer.
KVCache gpt_kvcache_create(const GPT *m);
// model.c:450-455
void gpt_kvcache_free(KVCache *kv);
// (no counterpart: the reference's step reads the host tensors every time)
// The device copy of the weights is made when the cache is created and again
// when gpt_decode_step is given a different model; weights changed in place
// (the same buffers) are seen only after this call.  0 on success.
int gpt_kvcache_refresh(KVCache *kv, const GPT *m);
// model.c:457-520  One token at position kv->len; logits (1, vocab) in host memory.
void gpt_decode_step(const GPT *m, KVCache *kv, int token, Tensor *logits);

#ifdef __cplusplus
}
#endif

#endif
