// qdev_seqsum.h - exact, parallel evaluation of a sequential float32 sum of
// non-negative terms:  s = ((0 + a_0) + a_1) + ... + a_{n-1}, every + rounded to
// nearest-even in float32, exactly as a C loop `s += a[i]` computes it.  The
// reference forms two such sums per use: rmsnorm's sum of squares (rmsnorm.c:15)
// and the softmax denominator (llama.c:567).
//
// Why it can be parallel: with a_i >= 0 the partial sums never decrease.  While a
// partial sum s stays inside one binade [2^e, 2^(e+1)) every float there is a
// multiple of u = 2^(e-23), so s + a_i rounds to s + u * rne(a_i / u): the step
// adds an integer number of u that depends on a_i alone (unless a_i / u ends in
// exactly .5, where the tie goes to the even neighbour and depends on s).  Sums
// of integers do not depend on their order.
//
// Method (one block, scratch in LDS):
//   1. P_i = a_0 + ... + a_{i-1} (a float block scan) predicts the binade of
//      each partial sum s_i.  Steps whose prediction is ambiguous (P_i or P_{i+1}
//      near a power of two), that change binade, or that are exact ties are hard.
//   2. Every other (easy) step i contributes k_i = rne(a_i / u_i); a block scan
//      of the k_i gives the integer total of each run of easy steps between two
//      hard steps, and that total times the run's u is an exact float.
//   3. One lane walks the hard steps only: s += run total; s = s + a_hard (a real
//      float add, so ties and binade changes round exactly as the loop does).
//   4. Every run is checked afterwards: its exact start must lie in the binade
//      predicted for it and its exact end must not pass the top of that binade
//      (reaching it exactly is consistent).  Partial sums are monotone, so then
//      every step of the run was on that grid.  If any check fails, or there are
//      more hard steps than the scratch holds, the block falls back to the plain
//      sequential loop.  The result is the sequential sum in every case; the
//      prediction margin only decides how often the fast path applies.
#ifndef QDEV_SEQSUM_H
#define QDEV_SEQSUM_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qd {

constexpr int kSeqMaxN = 16384;            // longest sum supported
constexpr int kSeqMaxHard = 480;           // hard steps held in LDS
constexpr int kSeqMaxWaves = 16;           // blocks of up to 1024 threads

struct SeqSumScratch {
  float pscan[kSeqMaxWaves + 1];
  unsigned kscan[kSeqMaxWaves + 1];
  int hscan[kSeqMaxWaves + 1];
  int hidx[kSeqMaxHard];
  unsigned hk[kSeqMaxHard];
  float ha[kSeqMaxHard];
  int hafter[kSeqMaxHard];
  float sa[kSeqMaxHard];
  float segu[kSeqMaxHard + 1];
  float sb[kSeqMaxHard + 1];
  unsigned ktot;
  int nhard;
  int fail;
  float result;
};

// Binade of a partial sum predicted as P >= 0: e for P in [2^e, 2^(e+1)), -127
// for [0, 2^-126) (one grid, 2^-149, covers 0 and the subnormals).  amb = 1
// when P is within relative margin rho of an edge.
__device__ __forceinline__ int seq_binade(float P, float rho, int &amb) {
  const uint32_t b = __float_as_uint(P);
  const int ex = (int)((b >> 23) & 0xff);
  if (ex == 0) {
    amb = P > 0x1p-126f * (1.0f - rho);
    return -127;
  }
  const float m = __uint_as_float((b & 0x007FFFFFu) | 0x3F800000u);   // P / 2^e in [1, 2)
  amb = (m < 1.0f + rho) || (m > 2.0f - 2.0f * rho);
  return ex - 127;
}

// binade of an exact float partial sum s >= 0
__device__ __forceinline__ int seq_binade_f(float s) {
  const int ex = (int)((__float_as_uint(s) >> 23) & 0xff);
  return ex == 0 ? -127 : ex - 127;
}

__device__ __forceinline__ float seq_unit(int e) {        // grid spacing of binade e (>= 2^-149)
  return e == -127 ? 0x1p-149f : ldexpf(1.0f, e - 23);
}

__device__ __forceinline__ float seq_top(int e) {         // 2^(e+1), the binade's upper edge
  return __uint_as_float((uint32_t)(e + 1 + 127) << 23);
}

// a scaled to units of the grid of binade e; exact where it is used (a < 2^(e+1))
__device__ __forceinline__ float seq_scaled(float a, int e) {
  return e == -127 ? ldexpf(a, 149) : ldexpf(a, 23 - e);
}

// Step i takes s_i (predicted by P) to s_i + a.  Returns true when the step is
// easy, with k its exact increment in units of the grid; eafter is the binade
// predicted for s_{i+1}.  rho is the relative prediction margin.
__device__ __forceinline__ bool seq_classify(float P, float a, float rho, int &k, int &eafter) {
  int amb0, amb1;
  const int e0 = seq_binade(P, rho, amb0);
  const int e1 = seq_binade(P + a, rho, amb1);
  eafter = e1;
  k = 0;
  if (amb0 || amb1 || e0 != e1) return false;
  const float t = seq_scaled(a, e0);
  if (t - floorf(t) == 0.5f) return false;           // exact tie: the parity of s decides
  k = (int)__builtin_rintf(t);
  return true;
}

// Prediction margin for the steps up to index i, relative to the partial sum:
// 16 standard deviations of the rounding error a sequential sum of i terms
// accumulates (each below half a unit in the last place), plus the error of the
// float prefix scan that forms the prediction (a few dozen roundings).
__device__ __forceinline__ float seq_margin(int i) {
  return 0x1p-20f * sqrtf((float)(i + 2)) + 0x1p-17f;
}

// Wave inclusive scan by DPP row shifts and row broadcasts (32-bit lanes).

__device__ __forceinline__ unsigned seq_dpp_u(unsigned x, int sel) {
  int v = (int)x, r = 0;
  switch (sel) {
    case 0: r = __builtin_amdgcn_update_dpp(0, v, 0x111, 0xf, 0xf, false); break;   // row_shr:1
    case 1: r = __builtin_amdgcn_update_dpp(0, v, 0x112, 0xf, 0xf, false); break;   // row_shr:2
    case 2: r = __builtin_amdgcn_update_dpp(0, v, 0x114, 0xf, 0xf, false); break;   // row_shr:4
    case 3: r = __builtin_amdgcn_update_dpp(0, v, 0x118, 0xf, 0xf, false); break;   // row_shr:8
    case 4: r = __builtin_amdgcn_update_dpp(0, v, 0x142, 0xa, 0xf, false); break;   // row_bcast:15
    default: r = __builtin_amdgcn_update_dpp(0, v, 0x143, 0xc, 0xf, false); break;  // row_bcast:31
  }
  return (unsigned)r;
}

__device__ __forceinline__ float seq_wave_scan(float x) {
#pragma unroll
  for (int k = 0; k < 6; k++) x += __uint_as_float(seq_dpp_u(__float_as_uint(x), k));
  return x;
}

__device__ __forceinline__ unsigned seq_wave_scan(unsigned x) {
#pragma unroll
  for (int k = 0; k < 6; k++) x += seq_dpp_u(x, k);
  return x;
}

__device__ __forceinline__ int seq_wave_scan(int x) {
#pragma unroll
  for (int k = 0; k < 6; k++) x += (int)seq_dpp_u((unsigned)x, k);
  return x;
}

// Exclusive block scans of up to two 32-bit quantities at once: wave scans by
// DPP, then wave 0 scans the wave totals.
template <int NT, typename A, typename B>
__device__ __forceinline__ void seq_block_scan2(A va, B vb, A *ta, B *tb, A &ea, B &eb, A &tota, B &totb) {
  constexpr int NW = NT / 64;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const A xa = seq_wave_scan(va);
  const B xb = seq_wave_scan(vb);
  if (lane == 63) { ta[wave] = xa; tb[wave] = xb; }
  __syncthreads();
  if (wave == 0) {
    const A a0 = lane < NW ? ta[lane] : (A)0;
    const B b0 = lane < NW ? tb[lane] : (B)0;
    const A wa = seq_wave_scan(a0);
    const B wb = seq_wave_scan(b0);
    if (lane < NW) { ta[lane] = wa - a0; tb[lane] = wb - b0; }
    if (lane == NW - 1) { ta[NW] = wa; tb[NW] = wb; }
  }
  __syncthreads();
  ea = ta[wave] + xa - va;
  eb = tb[wave] + xb - vb;
  tota = ta[NW];
  totb = tb[NW];
  __syncthreads();
}

// The plain loop, for the fallback and as the definition of the result.
__device__ __forceinline__ float seq_serial(const float *a, int n) {
  float s = 0.0f;
  int i = 0;
  const float4 *a4 = reinterpret_cast<const float4 *>(a);
  for (; i + 4 <= n; i += 4) {
    const float4 v = a4[i >> 2];
    s += v.x;
    s += v.y;
    s += v.z;
    s += v.w;
  }
  for (; i < n; i++) s += a[i];
  return s;
}

// The sequential float32 sum of a[0..n), a in LDS (16-byte aligned), every a_i
// finite and >= 0.  All NT threads of the block (NT = blockDim.x, a multiple of
// 64, at most 1024) must call it; all get the result.  n <= kSeqMaxN.
template <int NT>
__device__ float seq_sum_nonneg(const float *a, int n, SeqSumScratch &S) {
  static_assert(NT % 64 == 0 && NT / 64 <= kSeqMaxWaves, "block size");
  const int tid = threadIdx.x;
  const int per = (n + NT - 1) / NT;
  const int i0 = min(n, tid * per), i1 = min(n, i0 + per);

  // 1. predicted partial sums (float prefix; its own error is inside the margin)
  float ls = 0.0f;
  for (int i = i0; i < i1; i++) ls += a[i];
  float P, ptot;
  int idummy, idtot;
  seq_block_scan2<NT, float, int>(ls, 0, S.pscan, S.hscan, P, idummy, ptot, idtot);

  // 2. classify each step; count the hard ones and total the k of the easy ones
  // (k totals are kept modulo 2^32: only differences within one run are used,
  // and a run stays inside one binade, so its total is below 2^23)
  const float Pstart = P;
  const float rho = seq_margin(i1);                  // covers every step of this thread
  unsigned ksum = 0;
  int nh = 0;
  for (int i = i0; i < i1; i++) {
    int k, eafter;
    const float ai = a[i];
    if (seq_classify(P, ai, rho, k, eafter)) ksum += (unsigned)k;
    else nh++;
    P += ai;
  }
  unsigned kbase, ktot;
  int hbase, htot;
  seq_block_scan2<NT, unsigned, int>(ksum, nh, S.kscan, S.hscan, kbase, hbase, ktot, htot);
  if (htot > kSeqMaxHard) {
    if (tid == 0) S.result = seq_serial(a, n);
    __syncthreads();
    return S.result;
  }

  // 3a. hard steps in order (the same classification replayed): index, exclusive
  // k-prefix, term, and the binade predicted for the run after it
  {
    unsigned kex = kbase;
    int m = hbase;
    P = Pstart;
    for (int i = i0; i < i1; i++) {
      int k, eafter;
      const float ai = a[i];
      if (seq_classify(P, ai, rho, k, eafter)) {
        kex += (unsigned)k;
      } else {
        S.hidx[m] = i;
        S.hk[m] = kex;
        S.ha[m] = ai;
        S.hafter[m] = eafter;
        m++;
      }
      P += ai;
    }
  }
  if (tid == 0) { S.nhard = htot; S.ktot = ktot; S.fail = 0; }
  __syncthreads();
  const int H = S.nhard;
  // 3b. run m precedes hard step m (run H is the tail); its total in exact float
  for (int m = tid; m <= H; m += NT) {
    const unsigned k0 = m == 0 ? 0u : S.hk[m - 1];
    const unsigned k1 = m == H ? S.ktot : S.hk[m];
    const int e = m == 0 ? -127 : S.hafter[m - 1];
    S.segu[m] = (float)(k1 - k0) * seq_unit(e);       // difference taken modulo 2^32
  }
  __syncthreads();
  // 3c. the walk over hard steps
  if (tid == 0) {
    float s = 0.0f;
    for (int m = 0; m < H; m++) {
      s = s + S.segu[m];
      S.sb[m] = s;
      s = s + S.ha[m];
      S.sa[m] = s;
    }
    s = s + S.segu[H];
    S.sb[H] = s;
    S.result = s;
  }
  __syncthreads();
  // 4. check every non-empty run against its predicted binade
  for (int m = tid; m <= H; m += NT) {
    const int first = m == 0 ? 0 : S.hidx[m - 1] + 1;
    const int end = m == H ? n : S.hidx[m];
    if (end > first) {
      const int e = m == 0 ? -127 : S.hafter[m - 1];
      const float st = m == 0 ? 0.0f : S.sa[m - 1];
      const float en = S.sb[m];
      const bool ok = seq_binade_f(st) == e && (seq_binade_f(en) == e || en == seq_top(e));
      if (!ok) S.fail = 1;
    }
  }
  __syncthreads();
  if (S.fail) {
    if (tid == 0) S.result = seq_serial(a, n);
    __syncthreads();
  }
  const float res = S.result;
  __syncthreads();
  return res;
}

}  // namespace qd

#endif
