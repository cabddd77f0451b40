// qllama.h - C ABI of the MI355X library for the reference's int8 LLaMA decode path.
//
// Drop-in for the quantized section of the reference's llama.h (llama.h:114-140),
// for quant.h (quant.h:15-33), for qacc_columns (matrix.h:55), for sampler.h
// (sampler.h:12-31) and for the fp32 cache / decode step / forward of llama.h
// (llama.h:80, 101-106).  Same names, argument meaning and error behaviour; the
// difference is where the data lives:
//
//   * QTensor.q / QTensor.scale point to DEVICE memory (MI355X HBM).  q is stored
//     output-channel major: element (row k, col j) of the reference's (rows, cols)
//     matrix sits at q[j * kpad + k], kpad = rows rounded up to 16 (zero padded),
//     so each output channel's K inputs are contiguous (layout QT_LAYOUT_NK).  The
//     token embedding keeps the reference's row-major order (QT_LAYOUT_KN) because
//     it is read one row per token.  Callers of the reference never read q or
//     scale (main.c:649-671, selftest.c:1231-1249); they are opaque here.
//   * Tensor members of QLlamaBlock / QLlamaModel hold device pointers as well.
//   * LlamaKV.k / .v hold one device pointer per layer; callers only read and
//     reset LlamaKV.len (main.c:661), which this library honours.
//   * Tensor arguments of qmatmul and the logits of q_llama_decode_step are host
//     memory, exactly as in the reference.
//   * The fp32 LlamaModel stays the reference's host structure; the library keeps
//     a private device copy of its weights for llama_kv_create's caches, and the
//     logits of llama_decode_step / llama_model_forward and the logits that
//     sample_token reads are host memory.
//
// Errors follow the reference: loaders return nonzero and print "Error: ..." to
// stderr; void functions print and abort on a device error.  Entry points that
// are additive (no reference counterpart) return 0 on success.
//
// Used standalone this header defines every type it needs.  Inside the
// reference's build it takes the place of quant.h and of the KV / quantized
// section of llama.h (llama.h:94-140): Tensor then comes from tensor.h and the
// fp32 LlamaBlock / LlamaModel from llama.h, which must be included first.
#ifndef QLLAMA_H
#define QLLAMA_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#ifdef QUANT_H
#error "qllama.h replaces quant.h: its QTensor holds device memory and a layout tag"
#endif
#define QUANT_H   // everything quant.h declares is declared here

// tensor.h:10-16 (host tensors; inside a QLlamaModel the data pointer is device memory)
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

#define QT_LAYOUT_NK 0   // device, output-channel major, K contiguous, rows padded to 16
#define QT_LAYOUT_KN 1   // device, reference row-major (rows, cols)

// quant.h:22-27 plus a layout tag and the padded row length.
typedef struct {
  int rows, cols;
  signed char *q;     // device
  float *scale;       // device, cols entries
  int layout;         // QT_LAYOUT_*
  int kpad;           // padded K for QT_LAYOUT_NK (multiple of 16), else cols
} QTensor;

#ifndef LLAMA_H
// llama.h:19-37 (fp32, host) - input of q_llama_quantize_from.
typedef struct {
  int d_model, n_heads, n_kv, head_dim, d_ff;
  float rope_base, eps;
  Tensor attn_norm, Wq, Wk, Wv, b_q, b_k, b_v, Wo, ffn_norm, Wgate, Wup, Wdown;
} LlamaBlock;

// llama.h:58-66 (fp32, host)
typedef struct {
  int vocab, d_model, n_layers, n_heads, n_kv, head_dim, d_ff, max_seq;
  float rope_base, eps;
  Tensor wte;
  LlamaBlock *blocks;
  Tensor final_norm;
  Tensor lm_head;
} LlamaModel;
#endif

// llama.h:94-99 plus the device-side state.
typedef struct {
  int n_layers, max_seq, kv_dim;
  int len;            // positions cached; callers may reset it to 0 to restart
  float **k;          // host array of n_layers device pointers, [n_kv][max_seq][head_dim]
  float **v;
  void *dev;          // library-private
} LlamaKV;

// llama.h:117-121
typedef struct {
  Tensor attn_norm, ffn_norm;                  // device f32
  Tensor b_q, b_k, b_v;                        // device f32
  QTensor Wq, Wk, Wv, Wo, Wgate, Wup, Wdown;   // device int8
} QLlamaBlock;

// llama.h:123-130 plus the device-side state.
typedef struct {
  int vocab, d_model, n_layers, n_heads, n_kv, head_dim, d_ff, max_seq;
  float rope_base, eps;
  QTensor wte;
  QLlamaBlock *blocks;
  Tensor final_norm;
  QTensor lm_head;
  void *dev;          // library-private
} QLlamaModel;

// ---------------------------------------------------------------------------
// Drop-in entry points (reference file:line each one replaces)
// ---------------------------------------------------------------------------

// llama.c:610-657  Load an 'LLMQ' v2 checkpoint straight into device memory.
int q_llama_model_load(const char *path, QLlamaModel *out);
// llama.c:483-488
void q_llama_model_free(QLlamaModel *m);
// llama.c:490-511  Quantize a host fp32 model (per output channel) on the GPU.
QLlamaModel q_llama_quantize_from(const LlamaModel *src);
// llama.c:513-526  Device KV cache of max_seq positions per layer (exact mode).
LlamaKV q_llama_kv_create(const QLlamaModel *m);
// llama.c:290-294
void llama_kv_free(LlamaKV *kv);
// llama.c:528-600  One token at position kv->len; logits (1, vocab) in host memory.
void q_llama_decode_step(const QLlamaModel *m, LlamaKV *kv, int token, Tensor *logits);

// quant.c:35-41 / 43-46 / 48-50  (device QTensor, QT_LAYOUT_NK)
QTensor qtensor_create(int rows, int cols);
void qtensor_free(QTensor *t);
void qtensor_quantize(QTensor *t, const float *w);            // w: host (rows, cols) f32
// quant.c:60-85  C[m,j] = (as[m] * scale[j]) * sum_k qa[m,k] q[k,j]; A, C host.
void qmatmul(const Tensor *A, const QTensor *W, Tensor *C);
// quant.c:10-27 / 29-33  (host arrays in, host arrays out; computed on the GPU)
void quantize_int8_percol(const float *w, int rows, int cols, signed char *q, float *scale);
void dequantize_int8_percol(const signed char *q, const float *scale, int rows, int cols, float *w);
// matrix.c:370-374  acc[j] = sum_k qa[k] * qw[k*N + j]  (host arrays, computed on the GPU)
void qacc_columns(const signed char *qa, const signed char *qw, int K, int N, int32_t *acc);

// llama.c:275-288 / 296-362  The fp32 (LLMA) decode step on the GPU, for the
// reference's host LlamaModel (llama.h:58-66).  The first cache made for a model
// uploads a device copy of its weights (found again by the model's weight
// pointers); the copy is freed with the last of its caches (llama_kv_free).
// The copy is taken when the first live cache of the model is created: host
// weight changes made while a cache of it lives are not seen until every cache
// has been freed and a new one is made.
// logits: host (1, vocab).  Every output sums in the reference's order, so the
// logits are the reference's bit for bit.
LlamaKV llama_kv_create(const LlamaModel *m);
void llama_decode_step(const LlamaModel *m, LlamaKV *kv, int token, Tensor *logits);
// llama.c:167-186  Logits (seq_len, vocab) of every position of ids (host tensor),
// on the GPU.  Row i equals the reference's batched forward bit for bit (which
// equals its decode step at position i).  Batched over all rows for head_dim 48,
// 64 or 128 with at most 8 query heads per KV head, seq_len <= 16384 (max_seq
// does not bound it); other head layouts replay decode steps, seq_len <= max_seq.
// Uses the model's device copy if a cache holds one, else uploads one for the
// call.  Ids outside [0, vocab) abort with a message.
void llama_model_forward(const LlamaModel *m, const int *ids, int seq_len, Tensor *logits);

// sampler.h:12-31.  Inside the reference's build this takes the place of
// sampler.h (which, included first, supplies Rng itself).
#ifndef SAMPLER_H
#define SAMPLER_H
typedef struct {
  unsigned long long state;
} Rng;
#endif
// sampler.c:24-29 / 40-45 (host: xorshift64, top 53 bits to a float in [0, 1))
Rng rng_create(unsigned long long seed);
float rng_uniform(Rng *r);
// sampler.c:8-21  First index of the largest logit of row `row` (host Tensor of
// shape (rows, vocab)); evaluated on the GPU.
int sample_argmax(const Tensor *logits, int row);
// sampler.c:54-143  Temperature + top-k + top-p sampling of row `row` (host
// Tensor), evaluated on the GPU with the reference's arithmetic: the same token
// and the same advance of *rng (none when temperature <= 0, which is greedy).
int sample_token(const Tensor *logits, int row, float temperature, int top_k, float top_p, Rng *rng);

// ---------------------------------------------------------------------------
// Additive entry points
// ---------------------------------------------------------------------------

// Sampled generation kept on the device (the loop of main.c:663-667): n_steps
// times, sample a token from the logits of the last token this model processed
// (sample_token's arithmetic, rng state advanced on the device), record it in
// out[i] and feed it at position kv->len.  Needs kv->len >= 1 (a prompt or a
// decode step before it) and kv->len + n_steps <= max_seq.  *rng is advanced as
// n_steps calls of sample_token would.  Returns 0 on success.
int q_llama_generate(const QLlamaModel *m, LlamaKV *kv, int n_steps, float temperature, int top_k, float top_p,
                     Rng *rng, int *out);

// Decode modes of a KV cache, chosen when it is created.
#define QLLAMA_MODE_EXACT 0  // every float sum in the reference's order: logits bit-identical to llama.c:528-600
#define QLLAMA_MODE_FAST  1  // split-K attention with an online-softmax merge and tree-ordered rmsnorm sums;
                             // the integer GEMV arithmetic is unchanged.  NOT the reference's arithmetic:
                             // a reordered sum moves an activation by an ulp, which can flip an int8 code
                             // of the per-row quantizer, and from there the greedy stream departs (measured
                             // on the 1B and 8B fixtures: 194 of 256 and 289 of 512 tokens equal, logits
                             // outside max-abs 1e-3 / relative 1e-4 from the first step)
// q_llama_kv_create (llama.c:513-526) with a decode mode; every entry point that
// takes the cache then decodes in that mode.  Prompt ingestion on a fast cache
// runs the batched prefill with fp32 MFMA prompt attention (an online softmax,
// not the reference's order) at head_dim 64 and 128; its GEMMs stay exact.
LlamaKV q_llama_kv_create_mode(const QLlamaModel *m, int mode);

// Prompt ingestion: n tokens at positions kv->len .. kv->len+n-1.  Same result
// as n calls of q_llama_decode_step (main.c:662); logits are those of the last
// token.  logits may be NULL.  Returns 0 on success.
int q_llama_prefill(const QLlamaModel *m, LlamaKV *kv, const int *ids, int n, Tensor *logits);

// Greedy generation kept on the device: feeds `token` at kv->len, then each
// argmax (first index of the maximum, sampler.c:8-21) back in, n_steps times;
// out[i] receives the i-th generated id.  Equals the reference loop
// main.c:663-668 with temperature 0.  Returns 0 on success.
int q_llama_generate_greedy(const QLlamaModel *m, LlamaKV *kv, int token, int n_steps, int *out);

// Model from the seeded synthetic generator (fp32 N(0, 0.02) weights quantized
// per output channel, gains 1, biases 0), built on the device.  cfg = {vocab,
// d_model, n_layers, n_heads, n_kv, head_dim, d_ff, max_seq}.  Returns 0 on success.
int q_llama_model_synth(QLlamaModel *out, const int32_t cfg[8], float rope_base, float eps,
                        uint64_t seed, int tied);
// Order-independent digest of every int8 tensor and scale vector, in the
// reference's (rows, cols) indexing; equal to the generator's CPU digest.
uint64_t q_llama_model_hash(const QLlamaModel *m);

// Write the model as an 'LLMQ' v2 checkpoint that q_llama_model_load (and the
// reference's loader, llama.c:603-657) reads back: the int8 byte order of the
// reference's writer (tools/convert_llama.py:73-97).  Returns 0 on success.
int q_llama_model_save(const QLlamaModel *m, const char *path);

// Copy a device QTensor back to host memory in the reference's layout (quant.h:22-27):
// q (rows, cols) row-major int8 and scale (cols).  Counterpart of the loader's
// read order (llama.c:603-608).  Returns 0 on success.
int q_llama_tensor_export(const QTensor *t, signed char *q_host, float *scale_host);

// No counterpart in the reference: an allocation-free qmatmul (quant.c:60-85) for
// callers that cannot allocate -- code under HIP graph capture, tight serving
// loops, harnesses that forbid hipMalloc.  A (M, K = W->rows) and C (M, W->cols)
// are f32 row-major DEVICE buffers; W is a device QTensor in QT_LAYOUT_NK.  The
// quantized activation rows live in a static device array of
// QLLAMA_NOALLOC_SCRATCH_BYTES per GPU (held until the process ends), so M *
// W->kpad + 4 * M + 256 must fit in it (else the call fails with a message),
// and K <= 16384.  Results equal qmatmul's bit for bit.  The work is enqueued on
// qllama_stream() and the call returns without waiting (qllama_sync() waits);
// it calls no hipMalloc, hipFree or allocating library routine after its first
// call on a device (which looks up the array's address).  Every call on a GPU
// shares that GPU's array: calls that overlap on one GPU (concurrent graph
// replays, other streams) race.  Returns 0 on success.
#define QLLAMA_NOALLOC_SCRATCH_BYTES ((size_t)16 << 20)
int qmatmul_device_noalloc(const float *A, int M, const QTensor *W, float *C);

// Device-side helpers for tests and benchmarks.
int  qllama_device_count(void);
// A device QTensor (QT_LAYOUT_NK) of the seeded generator's N(0, sigma) (rows,
// cols) matrix (tensor id tid), quantized per column (quant.c:10-27) on the device.
QTensor qtensor_synth(int rows, int cols, uint64_t seed, uint64_t tid, double sigma);
// qmatmul on device-resident data (M rows of N(0, 1) inputs): mean microseconds
// per call (quantization + product, events around reps back-to-back calls) and
// of the product and quantization kernels alone (events on each launch, each
// launched on a drained stream).  Returns 0 on success.
int  qllama_bench_qmatmul(const QTensor *W, int M, int reps, double *us_call, double *us_product, double *us_quant);
// Cold op-level timing for qllama_bench_qmatmul and qllama_gqa_decode_ex while
// on: each timed call is preceded by a 512 MB read (twice the memory-side
// cache), the per-call time is that of the (read, call) sequence less that of
// the reads alone, and the per-launch times are taken behind a read each.
int  qllama_bench_cold(int on);
// Device buffers for callers that bring their own (qmatmul_device_noalloc's A
// and C): allocate, free (after the stream drains), and synchronous copies in
// stream order.
void *qllama_dev_alloc(size_t bytes);
void qllama_dev_free(void *p);
int  qllama_h2d(void *dst, const void *src, size_t bytes);
int  qllama_d2h(void *dst, const void *src, size_t bytes);
int  qllama_device_sync(void);
int  qllama_sync(void);
void *qllama_stream(void);               // the hipStream_t every launch goes to
// 1 when the model's exact decode steps run the attention half of each layer
// (QKV GEMV, RoPE, cache append, scores, softmax, PV) as one launch, 0 when
// they run it as separate kernels (shapes the one launch does not serve, or
// QLLAMA_NO_ATTN_LAYER=1 in the environment when the model was made).
int  qllama_attn_layer_active(const QLlamaModel *m);
// Average duration (ms) of each kernel class over the decode steps run while
// profiling was on; returns the number of classes written.  enable: 0 off,
// 1 on; 3 serialized (each timed launch waits for the stream to drain, so the
// events of back-to-back launches do not overlap); 5 cold (serialized, behind
// a 512 MB read each).
int  qllama_profile(int enable);
int  qllama_profile_read(char *names, int names_len, double *ms, long long *count, int max);
// The device tanhf (the one GPT-2's GELU uses) on the float bit patterns start,
// start+1, ..., start+count-1, written to host memory.  For parity tests.
int  qllama_test_tanhf(uint32_t start, uint32_t count, float *out);
// The device expf (the one attention and SwiGLU use) on the float bit patterns
// start, start+1, ..., start+count-1, written to host memory.  For parity tests.
int  qllama_test_expf(uint32_t start, uint32_t count, float *out);
// Decode attention (llama.c:554-576) of one query row at position T-1 against
// T cached rows, on the device: q (n_heads*hd), k and v (T, n_kv*hd) in the
// reference's cache layout, o (n_heads*hd); all host memory.  For op-level parity.
int  qllama_gqa_decode(const float *q, const float *k, const float *v, int T, int n_heads, int n_kv,
                       int hd, float *o);
// The same with a decode mode (QLLAMA_MODE_*) and, for rope_base > 0, the RoPE
// of the decode step on the device: q and rows T-1 of k and v arrive
// unrotated; the device rotates q and k (host-libm tables, rope.c:48-68),
// appends row T-1 to the cache and attends; k_row (n_kv*hd, may be NULL)
// receives the rotated row as cached.  reps > 0 times that many launches after
// one warm-up (HIP events on the library stream, cold under qllama_bench_cold);
// *us_per_call receives the mean.
int  qllama_gqa_decode_ex(const float *q, const float *k, const float *v, int T, int n_heads, int n_kv, int hd,
                          float rope_base, int mode, int reps, float *o, float *k_row, double *us_per_call);
// Causal prompt attention (llama.c:554-576 for rows p0 .. p0+R-1) on the device:
// q (R, n_heads*hd) already rotated, k and v (p0+R, n_kv*hd) in the reference's
// cache layout, o (R, n_heads*hd); all host memory.  mode QLLAMA_MODE_EXACT is
// q_llama_prefill's exact path (every row equal to its decode step);
// QLLAMA_MODE_FAST is the fast mode's fp32 MFMA attention (head_dim 64 or 128).
// reps > 0 times that many launches after one warm-up; *us_per_call receives the
// mean.  For op-level parity and the bench.
int  qllama_pf_attention_ex(const float *q, const float *k, const float *v, int R, int p0, int n_heads, int n_kv,
                            int hd, int mode, int reps, float *o, double *us_per_call);
// One activation row through the decode GEMV that normalizes its own input:
// rmsnorm (rmsnorm.c:7-21) + activation quantization (quant.c:66-78) formed in
// every block, then the W8A8 product (quant.c:79-82).  mode 0: out = W->cols
// values; mode 2: SwiGLU (llama.c:583-587) over gate columns [0, N) and up
// columns [N, 2N), out = N values of h.  fast = 1 uses the fast decode mode's
// tree-ordered sum of squares.  W: device QTensor (rows = d_model, NK layout,
// kpad 2048, 4096 or 8192); x, gamma, out: host.  For parity tests.
int  qllama_norm_gemv(const float *x, const float *gamma, float eps, const QTensor *W, int mode, int fast, float *out);
// The device's exact evaluation of the sequential float sum ((0 + a_0) + a_1) + ...
// of n <= 16384 non-negative terms (the form of rmsnorm.c:15 and llama.c:567):
// *out = the sum, info[0] = number of serially evaluated steps, info[1] = 1 when
// the block fell back to the plain loop.  For parity tests.
int  qllama_test_seqsum(const float *a, int n, float *out, int *info);
// One plain device-to-device copy of `bytes` (a multiple of 16) between two
// fresh buffers, on the library's stream: the known-size reference that
// scales the HBM traffic counters of a profiler run.
int  qllama_test_copy(size_t bytes);
// One int8 GEMM of the prompt path (mode 0 plain + bias, 1 residual add, 2
// SwiGLU over W's 2N rows; quant.c:60-85 over M rows) from host operands, run
// whole and with K split over extra blocks; both results (out_plain, out_split:
// residual inputs on entry) and the split count used.  For parity tests.
int  qllama_test_gemm_split(int mode, const int8_t *A, const float *as, const int8_t *W, const float *ws, int M,
                            int N, int kpad, const float *bias, float *out_plain, float *out_split, int *splits);
// Prompt attention (the batched prefill's, llama.c:554-576 over P rows) on the
// VALU-only kernels (on = 1: every product a v_mul_f32) or on the default
// outer-product kernels (on = 0: products from K = 1 fp32 MFMAs); both give the
// same bits.  Holds for the rest of the process.  For parity tests.
int  qllama_test_pf_valu(int on);

#ifdef __cplusplus
}
#endif

#endif
