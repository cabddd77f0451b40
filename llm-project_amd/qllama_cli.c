// qllama_cli.c - the reference's `transformer llama` command for int8 LLMQ
// checkpoints (main.c:624-671), running on the MI355X library.
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
// step on the device).  'LLMA' f32 checkpoints and the tokenizer text mode are
// not part of this build: they are reported and refused.
#define _POSIX_C_SOURCE 200809L
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#include "qllama.h"

// main.c:561-572
static int parse_ids(char *line, int *seq, int vocab, int max_seq) {
  char *p = line;
  if ((unsigned char)p[0] == 0xEF && (unsigned char)p[1] == 0xBB && (unsigned char)p[2] == 0xBF) p += 3;
  int n = 0;
  for (char *t = strtok(p, " \t\r\n"); t && n < max_seq; t = strtok(NULL, " \t\r\n")) {
    int id = atoi(t);
    if (id < 0 || id >= vocab) { fprintf(stderr, "skip out-of-range id %d (vocab %d)\n", id, vocab); continue; }
    seq[n++] = id;
  }
  return n;
}

// main.c:574-579
static void print_gen(const int *seq, int n) {
  printf("gen:");
  for (int i = 0; i < n; i++) printf(" %d", seq[i]);
  printf("\n");
  fflush(stdout);
}

static int run_llama(int argc, char **argv) {
  if (argc < 3) {
    fprintf(stderr, "usage: qllama-cli llama <checkpoint.bin> [n_new=40]\n"
                    "  LLMQ (int8) checkpoint, run on the GPU;\n"
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
  if (magic != 0x514D4C4Cu) {   // 'LLMQ'
    fprintf(stderr, "Error: '%s' is not an LLMQ (int8) checkpoint; f32 LLMA checkpoints are not supported\n",
            argv[2]);
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
    int n = parse_ids(line, seq, m.vocab, m.max_seq);
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
    if (!rc) print_gen(seq, n);
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
