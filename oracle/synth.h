// synth.h - CPU side of the seeded synthetic-input generator (TEST INFRASTRUCTURE).
//
// This file belongs to the oracle: only tests/, the smoke check and bench.py's
// cpu_baseline leg may build against it.  The GPU library carries its own,
// independently written device implementation of the same specification; the
// per-tensor hash fixtures under tests/golden/ prove the two agree bit for bit.
//
// Specification (the contract both sides implement):
//   mix(z)      = splitmix64 finaliser: z ^= z>>30; z *= 0xBF58476D1CE4E5B9;
//                 z ^= z>>27; z *= 0x94D049BB133111EB; z ^= z>>31
//   key(s, t)   = mix(mix(s + G) ^ (t * 0xD1B54A32D192ED03)),  G = 0x9E3779B97F4A7C15
//   element i of tensor t, pair p = i >> 1:
//     h1 = mix(key + (p + 1) * G),  h2 = mix(h1 ^ 0x6A09E667F3BCC909)
//     u1 = ((h1 >> 11) + 1) * 2^-53  in (0, 1]
//     u2 =  (h2 >> 11)      * 2^-53  in [0, 1)
//     z  = sqrt(-2 ln u1) * (i even ? cos(2 pi u2) : sin(2 pi u2))
//   ln, sqrt, cos, sin are evaluated with +, -, * on doubles only, in the fixed
//   order written in synth.c (no division, no fused multiply-add), so every
//   IEEE-754 machine gets the same bits.
//   value(i) = (float)(z * sigma)                        (sigma = 0.02 for weights)
//   token id i of a prompt = ((mix(key + (i + 1) * G) >> 32) * vocab) >> 32
//
// Tensor ids follow the LLMQ canonical order (llama.c:199-220, 635-648):
//   0 = wte; layer l uses 1 + 12*l + {0 attn_norm, 1 Wq, 2 Wk, 3 Wv, 4 b_q, 5 b_k,
//   6 b_v, 7 Wo, 8 ffn_norm, 9 Wgate, 10 Wup, 11 Wdown}; then final_norm, lm_head.
//   Element i is the reference's row-major index (row * cols + col) of the
//   (rows = in_features, cols = out_features) matrix.  Norm gains are 1.0 and
//   biases 0.0.  A tied lm_head takes lm_head[k][v] = wte value at (v, k) and is
//   then quantized on its own (per vocab column).
#ifndef QL_SYNTH_H
#define QL_SYNTH_H

#include <stdint.h>
#include <stddef.h>

#define SYN_TID_GEMV_W   1000   // + shape index
#define SYN_TID_GEMV_X   2000   // + shape index
#define SYN_TID_GQA_Q    3000   // + case index
#define SYN_TID_GQA_K    3100
#define SYN_TID_GQA_V    3200
#define SYN_TID_PROMPT   4000
#define SYN_TID_GENERIC  5000

uint64_t syn_mix(uint64_t z);
uint64_t syn_key(uint64_t seed, uint64_t tid);
double   syn_normal(uint64_t key, uint64_t i);
float    syn_value(uint64_t key, uint64_t i, double sigma);
void     syn_fill(float *dst, size_t n, uint64_t seed, uint64_t tid, double sigma);
int      syn_token(uint64_t key, uint64_t i, int vocab);
void     syn_prompt(int *ids, int n, uint64_t seed, int vocab);

// Deterministic double-precision helpers (exported for their own tests).
double syn_ln(double u);
double syn_sqrt(double y);
void   syn_cos_sin_2pi(double v, double *c, double *s);

// Order-independent 64-bit digest of an int8 tensor and of a float vector,
// computed the same way by the GPU library: sum over elements of
// mix((i << 8) ^ byte ^ salt) and of mix((i << 32) ^ bits ^ salt), mod 2^64.
uint64_t syn_hash_i8(const int8_t *q, size_t n, uint64_t salt);
uint64_t syn_hash_f32(const float *x, size_t n, uint64_t salt);

#endif
