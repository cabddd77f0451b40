// qllama_cli.c - the reference's `transformer llama` command for LLMQ (int8) and
// LLMA (f32) checkpoints (main.c:624-702), running on the MI355X library.
//
//   qllama-cli llama <checkpoint.bin> [n_new=40]
//
// Same protocol as the reference: one line of space-separated token ids per
// stdin line (a UTF-8 BOM is skipped, out-of-range ids are reported on stderr
// and skipped, at most max_seq ids are kept); for each line the cache restarts,
// the prompt is ingested, and up to n_new tokens are sampled with temperature
// 0.8, top-k 40 and top-p 0.95 from one generator seeded 1234 for the whole
// run.  Each token is printed as "t <id>" as soon as it exists, and the line
// ends with "gen: <prompt and generated ids>".  The prompt goes through
// q_llama_prefill (equal to the reference's per-token q_llama_decode_step
// calls) and each token through q_llama_generate (sampling and the next decode
// step on the device).  'LLMA' (f32) checkpoints take the command's f32 branch
// (main.c:686-700): the file is read into a host LlamaModel, and
// llama_kv_create / llama_decode_step / sample_token run on the GPU.  The
// tokenizer text mode is not part of this build: it is reported and refused.
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qllama.h"

// One stdin line into token ids, with the protocol of main.c:561-572: a
// leading UTF-8 byte order mark is ignored; fields are separated by spaces,
// tabs, CR and LF and each is read as atoi reads it; an id outside [0, vocab)
// is reported on stderr and dropped; once max_seq ids are kept, the rest of the
// line is not looked at.
static int read_prompt(char *line, int *ids, int vocab, int max_seq) {
  static const char sep[] = " \t\r\n";
  char *cur = line;
  if ((unsigned char)cur[0] == 0xEF && (unsigned char)cur[1] == 0xBB && (unsigned char)cur[2] == 0xBF) cur += 3;
  int kept = 0;
  while (kept < max_seq) {
    cur += strspn(cur, sep);
    if (!*cur) break;
    const size_t len = strcspn(cur, sep);
    const char end = cur[len];
    cur[len] = '\0';
    const int id = atoi(cur);
    cur[len] = end;
    cur += len;
    if (id >= 0 && id < vocab) ids[kept++] = id;
    else fprintf(stderr, "skip out-of-range id %d (vocab %d)\n", id, vocab);
  }
  return kept;
}

// The line that ends each prompt's output (main.c:574-579): "gen:" and every id
// of the sequence, each after one space.
static void emit_gen(const int *ids, int count) {
  fputs("gen:", stdout);
  for (int i = 0; i < count; i++) printf(" %d", ids[i]);
  putchar('\n');
  fflush(stdout);
}

// ---- the f32 branch -------------------------------------------------------------
static Tensor host_tensor(int r, int c) {   // (r, c), or (r) when c == 0; zero-filled
  Tensor t;
  const size_t n = (size_t)r * (c ? c : 1);
  t.data = (float*)calloc(n, sizeof(float));
  t.grad = NULL;
  t.ndim = c ? 2 : 1;
  t.shape = (int*)malloc(2 * sizeof(int));
  if (!t.data || !t.shape) { fprintf(stderr, "Error: out of memory\n"); exit(EXIT_FAILURE); }
  t.shape[0] = r; t.shape[1] = c;
  t.size = n;
  return t;
}

static void free_tensor(Tensor *t) { free(t->data); free(t->shape); t->data = NULL; t->shape = NULL; }

static void free_model(LlamaModel *m) {
  free_tensor(&m->wte); free_tensor(&m->final_norm); free_tensor(&m->lm_head);
  for (int l = 0; l < m->n_layers && m->blocks; l++) {
    LlamaBlock *b = &m->blocks[l];
    Tensor *t[12] = {&b->attn_norm, &b->Wq, &b->Wk, &b->Wv, &b->b_q, &b->b_k, &b->b_v, &b->Wo,
                     &b->ffn_norm, &b->Wgate, &b->Wup, &b->Wdown};
    for (int i = 0; i < 12; i++) free_tensor(t[i]);
  }
  free(m->blocks); m->blocks = NULL;
}

// An 'LLMA' v2 file into a host LlamaModel: header, config, then every tensor's
// f32 values in the canonical order (llama.c:198-219, 388-437).
static int load_llma(const char *path, LlamaModel *m) {
  FILE *f = fopen(path, "rb");
  if (!f) { fprintf(stderr, "Error: cannot open '%s' for reading\n", path); return 1; }
  uint32_t header[2];
  int32_t c[8];
  float fc[2];
  if (fread(header, 4, 2, f) != 2 || fread(c, 4, 8, f) != 8 || fread(fc, 4, 2, f) != 2) {
    fprintf(stderr, "Error: '%s' is truncated (bad header)\n", path);
    fclose(f); return 1;
  }
  if (header[0] != 0x414D4C4Cu || header[1] != 2u) {
    fprintf(stderr, "Error: '%s' is not a v2 LLMA checkpoint\n", path);
    fclose(f); return 1;
  }
  for (int i = 0; i < 8; i++)
    if (c[i] <= 0 || c[i] > 1000000 || (i == 4 && c[3] % c[4])) {
      fprintf(stderr, "Error: '%s' has an invalid/unsupported config\n", path);
      fclose(f); return 1;
    }
  memset(m, 0, sizeof *m);
  m->vocab = c[0]; m->d_model = c[1]; m->n_layers = c[2]; m->n_heads = c[3]; m->n_kv = c[4];
  m->head_dim = c[5]; m->d_ff = c[6]; m->max_seq = c[7]; m->rope_base = fc[0]; m->eps = fc[1];
  const int dm = c[1], qd = c[3] * c[5], kvd = c[4] * c[5], ff = c[6];
  m->wte = host_tensor(c[0], dm);
  m->blocks = (LlamaBlock*)calloc((size_t)c[2], sizeof(LlamaBlock));
  if (!m->blocks) { fclose(f); return 1; }
  int ok = fread(m->wte.data, 4, m->wte.size, f) == m->wte.size;
  for (int l = 0; l < c[2]; l++) {
    LlamaBlock *b = &m->blocks[l];
    b->d_model = dm; b->n_heads = c[3]; b->n_kv = c[4]; b->head_dim = c[5]; b->d_ff = ff;
    b->rope_base = fc[0]; b->eps = fc[1];
    b->attn_norm = host_tensor(dm, 0); b->Wq = host_tensor(dm, qd); b->Wk = host_tensor(dm, kvd);
    b->Wv = host_tensor(dm, kvd); b->b_q = host_tensor(qd, 0); b->b_k = host_tensor(kvd, 0);
    b->b_v = host_tensor(kvd, 0); b->Wo = host_tensor(qd, dm); b->ffn_norm = host_tensor(dm, 0);
    b->Wgate = host_tensor(dm, ff); b->Wup = host_tensor(dm, ff); b->Wdown = host_tensor(ff, dm);
    Tensor *t[12] = {&b->attn_norm, &b->Wq, &b->Wk, &b->Wv, &b->b_q, &b->b_k, &b->b_v, &b->Wo,
                     &b->ffn_norm, &b->Wgate, &b->Wup, &b->Wdown};
    for (int i = 0; i < 12 && ok; i++) ok = fread(t[i]->data, 4, t[i]->size, f) == t[i]->size;
  }
  m->final_norm = host_tensor(dm, 0);
  m->lm_head = host_tensor(dm, c[0]);
  if (ok) ok = fread(m->final_norm.data, 4, m->final_norm.size, f) == m->final_norm.size &&
               fread(m->lm_head.data, 4, m->lm_head.size, f) == m->lm_head.size;
  fclose(f);
  if (!ok) {
    fprintf(stderr, "Error: '%s' is truncated (bad weights)\n", path);
    free_model(m);
    return 1;
  }
  return 0;
}

static int run_llama_f32(const char *path, int n_new) {
  const float temperature = 0.8f;   // main.c:641-644
  const int top_k = 40;
  const float top_p = 0.95f;
  Rng rng = rng_create(1234);
  char line[8192];
  LlamaModel m;
  if (load_llma(path, &m) != 0) return 1;
  fprintf(stderr, "loaded LLMA (f32, MI355X): vocab %d d_model %d layers %d heads %d kv %d head_dim %d d_ff %d\n",
          m.vocab, m.d_model, m.n_layers, m.n_heads, m.n_kv, m.head_dim, m.d_ff);
  LlamaKV kv = llama_kv_create(&m);
  Tensor logits = host_tensor(1, m.vocab);
  int *seq = (int*)malloc((size_t)m.max_seq * sizeof(int));
  if (!seq) { fprintf(stderr, "Error: out of memory\n"); return 1; }
  while (fgets(line, sizeof(line), stdin)) {
    int n = read_prompt(line, seq, m.vocab, m.max_seq);
    if (n == 0) continue;
    kv.len = 0;
    for (int i = 0; i < n; i++) llama_decode_step(&m, &kv, seq[i], &logits);
    for (int s = 0; s < n_new && n < m.max_seq; s++) {
      int nxt = sample_token(&logits, 0, temperature, top_k, top_p, &rng);
      seq[n++] = nxt;
      printf("t %d\n", nxt);
      fflush(stdout);
      llama_decode_step(&m, &kv, nxt, &logits);
    }
    emit_gen(seq, n);
  }
  free(seq);
  free_tensor(&logits);
  llama_kv_free(&kv);
  free_model(&m);
  return 0;
}

static int run_llama(int argc, char **argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: qllama-cli llama <checkpoint.bin> [n_new=40]\n"
                    "  LLMQ (int8) or LLMA (f32) checkpoint, run on the GPU;\n"
                    "  reads space-separated token IDs per stdin line; prints 't <id>' per token and 'gen: <ids>'\n");
    return 2;
  }
  const int n_new = (argc > 3) ? atoi(argv[3]) : 40;
  if (argc > 4) {
    fprintf(stderr, "Error: the tokenizer text mode is not part of this build (token ids only)\n");
    return 2;
  }
  FILE *pf = fopen(argv[2], "rb");
  if (!pf) { fprintf(stderr, "Error: cannot open '%s'\n", argv[2]); return 1; }
  unsigned int magic = 0;
  if (fread(&magic, sizeof(unsigned int), 1, pf) != 1) {
    fclose(pf);
    fprintf(stderr, "Error: '%s' too small\n", argv[2]);
    return 1;
  }
  fclose(pf);
  if (magic == 0x414D4C4Cu) return run_llama_f32(argv[2], n_new);   // 'LLMA'
  if (magic != 0x514D4C4Cu) {   // 'LLMQ'
    fprintf(stderr, "Error: '%s' is not an LLMA or LLMQ checkpoint\n", argv[2]);
    return 1;
  }

  const float temperature = 0.8f;   // main.c:641-644
  const int top_k = 40;
  const float top_p = 0.95f;
  Rng rng = rng_create(1234);
  char line[8192];

  QLlamaModel m;
  if (q_llama_model_load(argv[2], &m) != 0) return 1;
  fprintf(stderr, "loaded LLMQ (int8, MI355X): vocab %d d_model %d layers %d heads %d kv %d head_dim %d d_ff %d\n",
          m.vocab, m.d_model, m.n_layers, m.n_heads, m.n_kv, m.head_dim, m.d_ff);
  LlamaKV kv = q_llama_kv_create(&m);
  int *seq = (int*)malloc((size_t)m.max_seq * sizeof(int));
  if (!seq) { fprintf(stderr, "Error: out of memory\n"); return 1; }
  int rc = 0;
  while (!rc && fgets(line, sizeof(line), stdin)) {
    int n = read_prompt(line, seq, m.vocab, m.max_seq);
    if (n == 0) continue;
    kv.len = 0;
    if (q_llama_prefill(&m, &kv, seq, n, NULL) != 0) { rc = 1; break; }
    for (int s = 0; s < n_new && n < m.max_seq; s++) {
      int nxt;
      if (q_llama_generate(&m, &kv, 1, temperature, top_k, top_p, &rng, &nxt) != 0) { rc = 1; break; }
      seq[n++] = nxt;
      printf("t %d\n", nxt);
      fflush(stdout);
    }
    if (!rc) emit_gen(seq, n);
  }
  if (rc) fprintf(stderr, "Error: generation failed on the GPU\n");
  free(seq);
  llama_kv_free(&kv);
  q_llama_model_free(&m);
  return rc;
}

int main(int argc, char **argv) {
  if (argc >= 2 && !strcmp(argv[1], "llama")) return run_llama(argc, argv);
  fprintf(stderr, "usage: qllama-cli llama <checkpoint.bin> [n_new=40]\n");
  return 2;
}
