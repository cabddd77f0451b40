// qhip.h - the thin extern "C" HIP layer under the C11 decode loop.
//
// Every launcher enqueues on the library's single HIP stream and returns 0, or
// a nonzero code after recording a message for qhip_last_error().  Pointers are
// device pointers unless a name says "host".  Shapes are plain ints.
#ifndef QHIP_H
#define QHIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

// ---- runtime ----------------------------------------------------------------
int         qhip_init(void);
int         qhip_device_count(void);
const char *qhip_last_error(void);
void       *qhip_malloc(size_t bytes);                   // NULL on failure
void        qhip_free(void *p);
void       *qhip_host_alloc(size_t bytes);               // pinned
void        qhip_host_free(void *p);
int         qhip_h2d(void *dst, const void *host_src, size_t n);        // synchronous
int         qhip_d2h(void *host_dst, const void *src, size_t n);        // synchronous
int         qhip_h2d_async(void *dst, const void *host_src, size_t n);  // pinned src
int         qhip_d2h_async(void *host_dst, const void *src, size_t n);
int         qhip_d2d_async(void *dst, const void *src, size_t n);
int         qhip_copy2d_d2d(void *dst, size_t dpitch, const void *src, size_t spitch, size_t width, size_t height);
int         qhip_fill_zero(void *p, size_t n);           // kernel, capture-safe
int         qhip_flush_caches(void);                     // reads 512 MB: the next kernel starts cold
// Staged upload from any host memory (a mapped file, say) through two pinned
// buffers of `chunk` bytes: qhip_upload returns once src may be reused, the copy
// itself completes in stream order; qhip_upload_end waits for all of it.
int         qhip_upload_begin(size_t chunk);
int         qhip_upload(void *dst, const void *host_src, size_t n);
int         qhip_upload_end(void);
int         qhip_sync(void);
void       *qhip_stream(void);

// graphs: capture the launches issued between begin and end on the stream
int  qhip_capture_begin(void);
int  qhip_capture_end(void **exec);
int  qhip_graph_launch(void *exec);
void qhip_graph_destroy(void *exec);

// elapsed time (ms) of the work enqueued between start and stop (HIP events on the stream)
int  qhip_timer_start(void);
int  qhip_timer_stop(double *ms);

// per-kernel-class timing with HIP events on the library stream.  on: 0 off,
// 1 on; | QHIP_PROF_SERIAL: each timed launch first waits for the stream to
// drain (events of back-to-back launches otherwise overlap); | QHIP_PROF_COLD:
// and reads 512 MB first, so the kernel finds its operands in neither L2 nor
// the memory-side cache.
#define QHIP_PROF_SERIAL 2
#define QHIP_PROF_COLD 4
int  qhip_profile_enable(int on);
int  qhip_profile_read(char *names, int names_len, double *ms, long long *count, int max);
int  qhip_profiling(void);

// ---- generator / weights ------------------------------------------------------
// Seeded N(0, sigma) matrix of the reference's (rows, cols) shape, quantized per
// column and stored output-channel major: q[j*kpad + k], scale[j].  tid_src and
// transpose_src select the generator tensor and index order (tied heads read the
// embedding generator at (col, row)).
int qhip_synth_quant_nk(uint64_t seed, uint64_t tid, int rows, int cols, int kpad, int transpose_src,
                        double sigma, int8_t *q, float *scale);
// Same, stored row-major (rows, cols) (embedding).
int qhip_synth_quant_kn(uint64_t seed, uint64_t tid, int rows, int cols, double sigma,
                        int8_t *q, float *scale);
// Seeded f32 values (same generator) into a device buffer.
int qhip_synth_f32(uint64_t seed, uint64_t tid, size_t n, double sigma, float *out);
int qhip_fill_f32(float *p, size_t n, float v);
// Quantize a device f32 (rows, cols) matrix per column (quant.c:10-27) into
// NK layout or into row-major KN layout.
int qhip_quantize_percol(const float *w, int rows, int cols, int layout_nk, int kpad,
                         int8_t *q, float *scale);
int qhip_dequantize_kn(const int8_t *q, const float *scale, int rows, int cols, float *w);
// Row-major (rows, cols) int8 -> NK layout.
int qhip_transpose_kn_to_nk(const int8_t *src, int rows, int cols, int kpad, int8_t *dst);
// NK layout (q[j*kpad + i]) -> row-major (rows, cols).
int qhip_nk_to_kn(const int8_t *src, int rows, int cols, int kpad, int8_t *dst);
int qhip_device_sync(void);
// Order-independent digests in the reference's (rows, cols) index space.
int qhip_hash_i8(const int8_t *q, int rows, int cols, int layout_nk, int kpad, uint64_t salt,
                 uint64_t *out);
int qhip_hash_f32(const float *x, size_t n, uint64_t salt, uint64_t *out);

// ---- decode kernels ------------------------------------------------------------
// x[j] = (float)wte[token*dm + j] * s[j]   (llama.c:534-536), token = d_in[d_state[0]]
int qhip_embed(const int8_t *wte, const float *wte_s, int dm, const int *d_in, const int *d_state,
               float *x);
// rows of x (rows, dm): y = rmsnorm(x) (rmsnorm.c:7-21), then per-row int8
// quantization (quant.c:66-78): qa (rows, kpad), as (rows)
int qhip_rmsnorm_quant(const float *x, int rows, int dm, const float *gamma, float eps,
                       int8_t *qa, int kpad, float *as);
// per-row int8 quantization only
int qhip_quant_rows(const float *v, int rows, int n, int8_t *qa, int kpad, float *as);
// h = SiLU(g) * u over gu = [g | u] (llama.c:583-587), then quantize h
int qhip_swiglu_quant(const float *gu, int rows, int dff, int8_t *qa, int kpad, float *as);
// out[m, j] = (as[m] * ws[j]) * acc[m, j] (+ bias[j]) or out[m, j] += that (residual);
// cls names the call site for event timing (QK_* in qhip_internal.h, 12 = other)
int qhip_gemv(const int8_t *qa, const float *as, int rows, const int8_t *W, const float *ws,
              int N, int kpad, float *out, const float *bias, int residual, int cls);
// decode attention over cache rows 0..*d_pos (llama.c:554-576); scores must hold
// qhip_attention_scratch(n_heads, max_seq) floats
size_t qhip_attention_scratch(int n_heads, int max_seq);
// obm (optional) receives qhip_attention_nbm(n_heads, hd) maxima of |o| by block.
int qhip_attention(const float *q, const float *kc, const float *vc, const int *d_pos,
                   int n_heads, int n_kv, int hd, int max_seq, float scale, float *scores,
                   float *o, float *obm);
// qhip_attention with RoPE and the cache append folded in: q, k, v of position
// pos = *d_pos arrive unrotated in qkv (n_heads + 2 n_kv heads); k (rotated)
// and v are appended to the per-layer cache [n_kv][max_seq][hd] at pos; RoPE uses
// the host-built tables (rope.c:48-68).
int qhip_attention_rope(const float *qkv, float *kc, float *vc, const int *d_pos, int n_heads, int n_kv, int hd,
                        int max_seq, float scale, const float *cos_t, const float *sin_t, float *scores, float *o,
                        float *obm);
int qhip_attention_nbm(int n_heads, int hd);
// The attention half of a decode layer in one launch (exact mode): the QKV GEMV
// with its rmsnorm prologue (as qhip_gemv_plain_norm), RoPE, the cache append,
// the scores, the softmax and PV (as qhip_attention_rope), one KV head per XCD.
// qhip_attn_layer_ok tells whether a shape (and the device) is served;
// scratch holds qhip_attn_layer_scratch floats, sync qhip_attn_layer_sync_words
// words that are zero before the first launch and then left to the kernel.
// obm receives qhip_attention_nbm maxima.  qhip_attn_layer_failed reports a
// launch whose blocks could not all meet (it synchronizes the stream).
int    qhip_attn_layer_probe(void);
int    qhip_attn_layer_ok(int n_heads, int n_kv, int hd, int kpad, int max_seq);
size_t qhip_attn_layer_scratch(int n_heads, int n_kv, int hd);
size_t qhip_attn_layer_sync_words(int n_kv);
int    qhip_attn_layer(const float *x, const float *gain, float eps, int dm, const int8_t *W, const float *ws,
                       const float *bias, int kpad, float *kc, float *vc, const int *d_pos, int n_heads, int n_kv,
                       int hd, int max_seq, float scale, const float *cos_t, const float *sin_t, float *scores,
                       float *scratch, unsigned *sync, float *o, float *obm);
int    qhip_attn_layer_failed(const unsigned *sync, int n_kv);
// The fast decode mode's attention (k_fattn.hip): split-K over positions with an
// online-softmax merge, same inputs and outputs as qhip_attention_rope (rope = 1)
// or qhip_attention (rope = 0, q pre-rotated and row pos already cached); obm
// receives n_heads maxima of |o| (one per query head).  scratch:
// qhip_fattn_scratch bytes (the chunks' partial results).
int qhip_fattn_ok(int n_heads, int n_kv, int hd, int max_seq);
size_t qhip_fattn_scratch(int n_heads, int n_kv, int hd, int max_seq);
int qhip_fattn(const float *qkv, float *kc, float *vc, const int *d_pos, int n_heads, int n_kv, int hd, int max_seq,
               float scale, const float *cos_t, const float *sin_t, int rope, void *scratch, float *o, float *obm);
// Decode GEMV with one activation row (k_gemv.hip): mode 0 plain (+bias), 1
// residual add, 2 SwiGLU over gate rows [0,N) and up rows [N,2N) writing h and
// per-block max |h| into bm (qhip_gemv_blocks(N, kpad) entries).
// Mode 3 is plain without bias plus, per block, the first index of its maximum
// output in bi[] with the value in bm[] (for qhip_argmax_final).
int qhip_gemv_dec(int mode, int cls, const int8_t *qa, const float *as, const int8_t *W, const float *ws,
                  int N, int kpad, float *out, const float *bias, float *bm, int *bi);
int qhip_argmax_final(const float *bv, const int *bidx, int nb, int *d_in, int *d_state, int *d_out, int max_seq);
// Residual GEMV (mode 1) quantizing its activation v (n values) in each block
// from the producer's per-block maxima vbm (nvbm of them); kpad in
// {2048, 4096, 8192, 14336} (qhip_gemv_fused_ok).
int qhip_gemv_resid_q(int cls, const float *v, int n, const float *vbm, int nvbm, const int8_t *W, const float *ws,
                      int N, int kpad, float *out);
int qhip_gemv_fused_ok(int kpad);
int qhip_gemv_blocks(int N, int kpad);
// SwiGLU GEMV (mode 2) whose activation is rmsnorm(x; gamma, eps) quantized,
// formed in each block from the dm values of x; kpad in {2048, 4096, 8192}
// (qhip_gemv_norm_ok).  It writes qhip_gemv_norm_blocks(N) per-block maxima.
// fast = 1: the sum of squares in a fixed tree order (the fast decode mode).
int qhip_gemv_swiglu_norm(int cls, int fast, const float *x, int dm, const float *gamma, float eps, const int8_t *W,
                          const float *ws, int N, int kpad, float *out, float *bm);
int qhip_gemv_norm_ok(int kpad, int dm);
// Plain GEMV (mode 0, QKV) whose activation is rmsnorm(x; gamma, eps) quantized,
// formed in each block like qhip_gemv_swiglu_norm's; same shapes.
int qhip_gemv_plain_norm(int cls, int fast, const float *x, int dm, const float *gamma, float eps, const int8_t *W,
                         const float *ws, int N, int kpad, float *out, const float *bias);
int qhip_gemv_norm_blocks(int N);
// Quantize v (n values) into qa (kpad, zero padded) and *as from nbm per-block maxima.
int qhip_quant_blocks(const float *v, int n, const float *bm, int nbm, int8_t *qa, int kpad, float *as);

// 1..16 activation rows against W [N][kpad] on MFMA (k_gemv.hip):
// out[m * ldo + j] = (as[m] * ws[j]) * (float)acc[m][j]  (quant.c:81-82).
// Persistent skinny W8A8 product for 2..16 rows (k_gemv_skinny);
// qhip_gemv_skinny_ok says which (M, N, kpad) it serves.
int qhip_gemv_skinny_ok(int M, int N, int kpad);
// k_gemv_rows: 2..8 rows, kpad = 1024 * (1..8), whole 1 KiB weight-row loads;
// qhip_gemv_rows_ok says which (M, N, kpad) it serves.
int qhip_gemv_rows_ok(int M, int N, int kpad);
int qhip_gemv_rows(int cls, const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws, int N,
                   int kpad, float *out, int ldo);
int qhip_gemv_skinny(int cls, const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws, int N,
                     int kpad, float *out, int ldo);
int qhip_gemv_mfma(int cls, const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws, int N,
                   int kpad, float *out, int ldo);

// qmatmul's product for M quantized rows (qa [M][kpad], as [M]) into C [M][N]:
// k_gemv_dec for one row, k_gemv_mfma up to 16, k_gemm_i8 beyond.
int qhip_qmm_product(const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws, int N, int kpad,
                     float *C);

// Many-row int8 GEMM on MFMA (k_gemm.hip): out[i][j] for i < M, j < N from
// activation rows A [M][kpad] and weight rows W [N][kpad] (SwiGLU: [2N][kpad]),
// with the decode GEMV's epilogues (mode 0 plain + bias, 1 residual, 2 SwiGLU).
int qhip_gemm_i8(int mode, int cls, const int8_t *A, const float *as, const int8_t *W, const float *ws, int M, int N,
                 int kpad, float *out, int ldo, const float *bias);
// As qhip_gemm_i8, splitting K over more blocks when the tiles leave CUs idle and
// work (work_bytes of device memory, int32 partial sums) is lent; the results
// are the same bits (the int32 sums are exact in any order).
int qhip_gemm_i8_ws(int mode, int cls, const int8_t *A, const float *as, const int8_t *W, const float *ws, int M,
                    int N, int kpad, float *out, int ldo, const float *bias, int *work, size_t work_bytes);

// Prompt ingestion over R rows at positions p0 .. p0+R-1 (k_decode.hip, k_attn.hip).
int qhip_pf_embed(const int8_t *wte, const float *wte_s, int dm, const int *ids, int R, float *x);
int qhip_pf_rope_append(const float *qkv, int R, int n_heads, int n_kv, int hd, const float *cos_t,
                        const float *sin_t, int p0, float *q_out, float *kc, float *vc, int max_seq);
// Causal attention of the R query rows q [R][n_heads*hd] against cache rows
// 0 .. p0+R-1; o [R][n_heads*hd].  ws is scratch of qhip_pf_attention_scratch floats.
int qhip_pf_attention(const float *q, const float *kc, const float *vc, int R, int p0, int n_heads, int n_kv,
                      int hd, int max_seq, float scale, float *ws, float *o);
size_t qhip_pf_attention_scratch(int R, int n_heads, int max_seq);
// The fast mode's prompt attention (k_pfa.hip): the same causal attention with
// fp32 MFMA and an online softmax (not bit-exact); head_dim 64 or 128, G <= 8.
int qhip_pf_attention_fast_ok(int n_heads, int n_kv, int hd);
int qhip_pf_attention_fast(const float *q, const float *kc, const float *vc, int R, int p0, int n_heads, int n_kv,
                           int hd, int max_seq, float scale, float *o);

// Token sampling on the device (k_sample.hip).  qhip_sample: temperature > 0,
// top-k, top-p over one row of V logits (sampler.c:54-143) with the xorshift64
// state *rng advanced on the device; scratch holds qhip_sample_scratch(V) bytes.
// qhip_argmax_row: first index of the maximum (sampler.c:8-21).  Both write the
// token to *tok; with d_state (decode state [pos, fill_end]) they also record it
// as the output of position d_state[0]-1 and the input of position d_state[0].
size_t qhip_sample_scratch(int V);
int qhip_sample_topk_path(int V, int top_k);     // 1: the top-k path (top_k <= 64), 0: the full radix sort
int qhip_sample(const float *logits, int V, float temperature, int top_k, float top_p, void *scratch,
                size_t scratch_bytes, unsigned long long *rng, int *tok, int *d_in, const int *d_state, int *d_out,
                int max_seq);
int qhip_argmax_row(const float *logits, int V, int *tok, int *d_in, const int *d_state, int *d_out, int max_seq);

// fp32 (LLMA) decode path (k_gemv_f32.hip).  qhip_gemv_f32: out[j] = c[j] (+bias[j])
// or out[j] += c[j] with c = x (K) times W (K, N), every c[j] summed in k order
// (matrix.c:178-190); W in the panel layout qhip_to_panels_f32 writes (from the
// reference's row-major (K, N); qhip_panels_f32_size floats); K <= qhip_gemv_f32_max_k().
size_t qhip_panels_f32_size(int K, int N);
int qhip_to_panels_f32(const float *src, int K, int N, float *dst);
// mode 0: out = c (+ bias); 1: out += c; 2: out = out + (c + bias); 3: out = gelu(c + bias).
int qhip_gemv_f32(int mode, int cls, const float *x, int K, const float *W, int N, float *out, const float *bias);
int qhip_gemv_f32_max_k(void);
int qhip_embed_f32(const float *wte, int dm, const int *d_in, const int *d_state, float *x);
int qhip_rmsnorm_f32(const float *x, int dm, const float *gamma, float eps, float *y);
int qhip_swiglu_f32(const float *gu, int dff, float *h);
// The batched fp32 forward (llama.c:167-186) over R rows: x [R][dm] = wte[ids];
// rmsnorm of each row; h [R][dff] from gu [R][2 dff]; and out (M, N) = c (+ bias)
// (mode 0) or out += c (mode 1) with c = A (M, K) times W (K, N) in the panel
// layout, every c[i][j] summed in k order as the GEMV does.
int qhip_embed_f32_rows(const float *wte, int dm, const int *ids, int R, float *x);
int qhip_rmsnorm_f32_rows(const float *x, int R, int dm, const float *gamma, float eps, float *y);
int qhip_swiglu_f32_rows(const float *gu, int R, int dff, float *h);
int qhip_gemm_f32(int mode, int cls, const float *A, int M, int K, const float *W, int N, float *out,
                  const float *bias);

// cache rows (T, n_kv*hd) in the reference's layout -> [n_kv][T][hd]
int qhip_kv_relayout(const float *src, int T, int n_kv, int hd, float *dst);

// GPT-2 (GPTC) decode pieces (k_gpt.hip, k_attn.hip): x = wte[token] + wpe[pos];
// LayerNorm in the reference's order (layernorm.c:8-38); the new k, v rows of
// qkv = [q | k | v] into caches [head][max_seq][head_dim]; decode attention with
// weights e_j / sum (model.c:485-504).
int qhip_gpt_embed(const float *wte, const float *wpe, int dm, const int *d_in, const int *d_state, float *x);
int qhip_layernorm_f32(const float *x, int dm, const float *gamma, const float *beta, float eps, float *y);
int qhip_gpt_kv_append(const float *qkv, int dm, int hd, int max_seq, const int *d_state, float *kc, float *vc);
int qhip_attention_div(const float *q, const float *kc, const float *vc, const int *d_pos, int n_heads, int n_kv,
                       int hd, int max_seq, float scale, float *scores, float *o);

// reference-layout column accumulate (matrix.c:354-374) for qacc_columns
int qhip_qacc_kn(const int8_t *qa, const int8_t *qw, int K, int N, int32_t *acc);

#ifdef __cplusplus
}
#endif

#endif
