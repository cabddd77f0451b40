// synth.c - CPU implementation of the seeded synthetic-input generator.
// TEST INFRASTRUCTURE: see synth.h for the specification and who may use it.
#include "synth.h"

#include <pthread.h>
#include <string.h>

#define SYN_G 0x9E3779B97F4A7C15ULL

static inline uint64_t bits_of(double d) { uint64_t u; memcpy(&u, &d, 8); return u; }
static inline double dbl_of(uint64_t u) { double d; memcpy(&d, &u, 8); return d; }

uint64_t syn_mix(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

uint64_t syn_key(uint64_t seed, uint64_t tid) {
  return syn_mix(syn_mix(seed + SYN_G) ^ (tid * 0xD1B54A32D192ED03ULL));
}

// ln(u) for u in [2^-53, 1]: u = m * 2^e with m in (0.707, 1.415], then
// ln m = 2 atanh(t), t = (m - 1) / (m + 1), the reciprocal by Newton steps.
double syn_ln(double u) {
  uint64_t b = bits_of(u);
  int e = (int)((b >> 52) & 0x7ff) - 1023;
  double m = dbl_of((b & 0x000FFFFFFFFFFFFFULL) | 0x3FF0000000000000ULL);
  if (m > 1.4142135623730951) { m = m * 0.5; e = e + 1; }
  double d = m + 1.0;
  double r = 0.5;
  for (int k = 0; k < 6; k++) r = r * (2.0 - d * r);
  double t = (m - 1.0) * r;
  double t2 = t * t;
  double p = 1.0 / 23.0;
  p = p * t2 + 1.0 / 21.0;
  p = p * t2 + 1.0 / 19.0;
  p = p * t2 + 1.0 / 17.0;
  p = p * t2 + 1.0 / 15.0;
  p = p * t2 + 1.0 / 13.0;
  p = p * t2 + 1.0 / 11.0;
  p = p * t2 + 1.0 / 9.0;
  p = p * t2 + 1.0 / 7.0;
  p = p * t2 + 1.0 / 5.0;
  p = p * t2 + 1.0 / 3.0;
  p = p * t2 + 1.0;
  return (double)e * 0.6931471805599453 + (2.0 * t) * p;
}

// sqrt(y) for y >= 0 via Newton steps on 1/sqrt(y) from a bit-level estimate.
double syn_sqrt(double y) {
  if (!(y > 0.0)) return 0.0;
  double g = dbl_of(0x5FE6EB50C7B537A9ULL - (bits_of(y) >> 1));
  double hy = 0.5 * y;
  for (int k = 0; k < 6; k++) g = g * (1.5 - (hy * g) * g);
  return y * g;
}

// cos and sin of 2*pi*v, v in [0, 1): octant reduction, Taylor series on [0, pi/4].
void syn_cos_sin_2pi(double v, double *c, double *s) {
  double v8 = v * 8.0;
  int q = (int)v8;
  double f = v8 - (double)q;
  int odd = q & 1;
  if (odd) f = 1.0 - f;
  double a = f * 0.78539816339744830962;
  double a2 = a * a;
  double sp = -1.0 / 355687428096000.0;
  sp = sp * a2 + 1.0 / 1307674368000.0;
  sp = sp * a2 - 1.0 / 6227020800.0;
  sp = sp * a2 + 1.0 / 39916800.0;
  sp = sp * a2 - 1.0 / 362880.0;
  sp = sp * a2 + 1.0 / 5040.0;
  sp = sp * a2 - 1.0 / 120.0;
  sp = sp * a2 + 1.0 / 6.0;
  double sa = a - (a * a2) * sp;
  double cp = 1.0 / 6402373705728000.0;
  cp = cp * a2 - 1.0 / 20922789888000.0;
  cp = cp * a2 + 1.0 / 87178291200.0;
  cp = cp * a2 - 1.0 / 479001600.0;
  cp = cp * a2 + 1.0 / 3628800.0;
  cp = cp * a2 - 1.0 / 40320.0;
  cp = cp * a2 + 1.0 / 720.0;
  cp = cp * a2 - 1.0 / 24.0;
  cp = cp * a2 + 0.5;
  double ca = 1.0 - a2 * cp;
  double cb = odd ? sa : ca, sb = odd ? ca : sa;
  switch (q >> 1) {
    case 0:  *c = cb;  *s = sb;  break;
    case 1:  *c = -sb; *s = cb;  break;
    case 2:  *c = -cb; *s = -sb; break;
    default: *c = sb;  *s = -cb; break;
  }
}

double syn_normal(uint64_t key, uint64_t i) {
  uint64_t p = i >> 1;
  uint64_t h1 = syn_mix(key + (p + 1) * SYN_G);
  uint64_t h2 = syn_mix(h1 ^ 0x6A09E667F3BCC909ULL);
  double u1 = (double)((h1 >> 11) + 1) * 0x1p-53;
  double u2 = (double)(h2 >> 11) * 0x1p-53;
  double rad = syn_sqrt(-2.0 * syn_ln(u1));
  double c, s;
  syn_cos_sin_2pi(u2, &c, &s);
  return rad * ((i & 1) ? s : c);
}

float syn_value(uint64_t key, uint64_t i, double sigma) {
  return (float)(syn_normal(key, i) * sigma);
}

typedef struct { float *dst; size_t lo, hi; uint64_t key; double sigma; } FillJob;

static void *fill_worker(void *arg) {
  FillJob *j = (FillJob*)arg;
  for (size_t i = j->lo; i < j->hi; i++) j->dst[i] = syn_value(j->key, i, j->sigma);
  return NULL;
}

void syn_fill(float *dst, size_t n, uint64_t seed, uint64_t tid, double sigma) {
  const uint64_t key = syn_key(seed, tid);
  enum { NT = 16 };
  if (n < ((size_t)1 << 16)) {
    for (size_t i = 0; i < n; i++) dst[i] = syn_value(key, i, sigma);
    return;
  }
  pthread_t th[NT];
  FillJob jobs[NT];
  size_t per = (n + NT - 1) / NT;
  for (int t = 0; t < NT; t++) {
    size_t lo = (size_t)t * per, hi = lo + per;
    if (lo > n) lo = n;
    if (hi > n) hi = n;
    jobs[t] = (FillJob){dst, lo, hi, key, sigma};
    pthread_create(&th[t], NULL, fill_worker, &jobs[t]);
  }
  for (int t = 0; t < NT; t++) pthread_join(th[t], NULL);
}

int syn_token(uint64_t key, uint64_t i, int vocab) {
  uint64_t h = syn_mix(key + (i + 1) * SYN_G);
  return (int)(((h >> 32) * (uint64_t)vocab) >> 32);
}

void syn_prompt(int *ids, int n, uint64_t seed, int vocab) {
  const uint64_t key = syn_key(seed, SYN_TID_PROMPT);
  for (int i = 0; i < n; i++) ids[i] = syn_token(key, (uint64_t)i, vocab);
}

uint64_t syn_hash_i8(const int8_t *q, size_t n, uint64_t salt) {
  uint64_t h = 0;
  for (size_t i = 0; i < n; i++) h += syn_mix(((uint64_t)i << 8) ^ (uint64_t)(uint8_t)q[i] ^ salt);
  return h;
}

uint64_t syn_hash_f32(const float *x, size_t n, uint64_t salt) {
  uint64_t h = 0;
  for (size_t i = 0; i < n; i++) {
    uint32_t b; memcpy(&b, &x[i], 4);
    h += syn_mix(((uint64_t)i << 32) ^ (uint64_t)b ^ salt);
  }
  return h;
}
