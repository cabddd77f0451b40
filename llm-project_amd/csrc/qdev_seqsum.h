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
// of integers do not depend on their order.  Grids are named by g = E, the
// biased exponent field; the unit of grid g >= 1 is 2^(g-150).  Grid 0 (zero and
// the subnormals) takes the unit 2^-150, half their spacing: every float there
// is a multiple of it and sums that stay below 2^-126 are exact, so its steps
// add exact integer multiples as well.
//
// Method (one block; thread t holds terms [t*CM, t*CM + CM) in registers):
//   1. P, a float block scan of the chunk totals, predicts every partial sum.
//      A float sum of non-negative terms is never below the largest term it has
//      added, so L_i = max(a_0..a_{i-1}) bounds s_i from below for certain.
//      Step i is easy when max(P_i*(1-rho), L_i) and P_{i+1}*(1+rho) lie on one
//      grid g and a_i / u_g is not a tie; it then adds k_i = rne(a_i / u_g).
//      Other steps are hard.  (L keeps the common softmax case, a sum that
//      sits just above the 1.0 of its largest term, off the binade edge.)  Consecutive easy steps of one thread share their grid
//      (P is monotone), and a thread-boundary check makes every run of easy
//      steps between two hard steps share one grid.
//   2. A block scan of the k_i gives each run's integer total K_m.
//   3. One lane walks the hard steps: s += K_m * u (exact when the run is on its
//      grid), then s = s + a_hard, a real float add.  On the way it proves every
//      run that has steps, K_m = 0 included: the run starts inside its grid's
//      binade and K_m * u fits below the binade's top.  Partial sums are monotone, so every step of the run was
//      on that grid; ending exactly at the top is consistent with both grids.
//   4. If a proof fails, or there are more hard steps than the scratch holds,
//      thread 0 runs the plain loop.  The result is the sequential sum in every
//      case; the prediction margin rho only decides how often the fast path
//      applies.
#ifndef QDEV_SEQSUM_H
#define QDEV_SEQSUM_H

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "qdev_math.h"

namespace qd {

constexpr int kSeqMaxHard = 512;           // hard steps held in LDS (kSeqMaxHard / waves per wave)
constexpr int kSeqMaxWaves = 16;           // blocks of up to 1024 threads

struct SeqScratch {
  float wf[kSeqMaxWaves];        // per wave: predicted total of its terms
  unsigned wm[kSeqMaxWaves];     //           bits of the largest term
  unsigned wk[kSeqMaxWaves];     //           total of its k (mod 2^32)
  int wh[kSeqMaxWaves];          //           hard steps
  int wg[kSeqMaxWaves];          //           grid of the run continuing past its last step
  int wgi[kSeqMaxWaves];         //           grid of its first step if that step is easy, else -1
  int4 hs[kSeqMaxHard];          // hard steps by wave: k prefix within the wave, index, term bits, grid after it
  float2 walk[72];               // one batch of the walk: run total, hard term (+8 read ahead)
  float wst[64];                 //                         partial sum the run starts from
  int bad;
  float result;
};

// Lane i receives lane i-1's value, lane 0 receives 0 (DPP wave_shr:1).
__device__ __forceinline__ unsigned seq_shr1(unsigned x) {
  return (unsigned)__builtin_amdgcn_update_dpp(0, (int)x, 0x138, 0xf, 0xf, true);
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

// Inclusive scan of the maximum, on the bits of floats >= 0 (ordered as the values).
__device__ __forceinline__ unsigned seq_wave_scan_umax(unsigned x) {
#pragma unroll
  for (int k = 0; k < 6; k++) x = max(x, seq_dpp_u(x, k));
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

// Inclusive scan within the first row of 16 lanes (row_shr only).
__device__ __forceinline__ unsigned seq_row_scan(unsigned x) {
#pragma unroll
  for (int k = 0; k < 4; k++) x += seq_dpp_u(x, k);
  return x;
}

// grid of a float p >= 0 (see above), and of the larger of p and the float
// whose bits are lb (both >= 0: their bits are ordered as their values)
__device__ __forceinline__ int seq_grid(float p) { return (int)(__float_as_uint(p) >> 23); }
__device__ __forceinline__ int seq_grid_max(float p, unsigned lb) { return (int)(max(__float_as_uint(p), lb) >> 23); }

// The plain loop over term(0..n), for the fallback and as the definition.
template <typename Term>
__device__ float seq_serial(int n, Term term) {
  float s = 0.0f;
  for (int i = 0; i < n; i++) s += term(i);
  return s;
}

// The sequential float32 sum of n terms, every one finite and >= 0.  Thread t
// of the NT participating threads (threads 0 .. NT-1 of the block, NT a multiple
// of 64, at most 1024) holds terms t*CM .. t*CM+CM-1 in a[], zero past n;
// n <= NT*CM.  term(i) returns term i again, for the rare fallback.  All NT
// threads must call it; all get the result.  Three meetings, through sync: the
// block barrier by default (then NT = blockDim.x), or GroupSync over the first
// NT/64 waves, which leaves the block's other waves running (LDS only: global
// loads in flight stay in flight).  S may be used again by the next call
// without another.
// info (optional, written by one thread): number of hard steps, 1 if the
// fallback ran.
template <int NT, int CM, typename Term, typename Sync = BlockSync>
__device__ float seq_sum_nonneg(const float (&a)[CM], int n, SeqScratch &S, Term term, int *info = nullptr,
                                const Sync &sync = Sync()) {
  static_assert(NT % 64 == 0 && NT / 64 <= kSeqMaxWaves, "block size");
  static_assert(CM >= 1 && CM <= 32, "terms per thread");
  constexpr int NW = NT / 64;
  constexpr int HCAP = kSeqMaxHard / NW;           // hard steps recorded per wave
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;

  // 1. predicted partial sum at the start of this thread's chunk (any order will
  // do) and the largest term before it
  // (largest terms are kept as bits: for floats >= 0 the integer maximum is the
  // float maximum)
  float loc;
  unsigned cmx = 0u;
  {
    float q[4] = {0.0f, 0.0f, 0.0f, 0.0f};
#pragma unroll
    for (int c = 0; c < CM; c++) {
      q[c & 3] += a[c];
      cmx = max(cmx, __float_as_uint(a[c]));
    }
    loc = (q[0] + q[1]) + (q[2] + q[3]);
  }
  const float xin = seq_wave_scan(loc);
  const unsigned mex = seq_wave_scan_umax(seq_shr1(cmx));   // exclusive
  if (lane == 63) { S.wf[wave] = xin; S.wm[wave] = max(mex, cmx); }
  if (tid == 0) S.bad = 0;
  sync();
  float P0 = xin - loc;
  unsigned M0 = mex;
#pragma unroll
  for (int w = 0; w < NW - 1; w++)
    if (w < wave) { P0 += S.wf[w]; M0 = max(M0, S.wm[w]); }

  // 2. classify; rho: 16 standard deviations of the rounding error a sequential sum
  // of i terms accumulates (each below half a unit in the last place), plus the
  // error of the float scan that forms the prediction.  kp[c] is the k total of
  // this thread's steps before step c.
  const float rho = 0x1p-20f * __builtin_amdgcn_sqrtf((float)((tid + 1) * CM + 2)) + 0x1p-17f;
  const float lo = 1.0f - rho, hi = 1.0f + rho;
  unsigned ks = 0, hardmask = 0;
  int nh = 0, gin = -1, gout = 0;
  unsigned kp[CM];
  int gh[CM];
  const int gA = seq_grid_max(P0 * lo, M0), gB = seq_grid((P0 + loc) * hi);
  if (wave * 64 * CM >= n) {
    // a wave wholly past n holds only +0 terms, and s + 0 is s on any grid: no
    // step to classify, no hard step, and no boundary to check (gin = -1)
#pragma unroll
    for (int c = 0; c < CM; c++) {
      kp[c] = 0u;
      gh[c] = 0;
    }
  } else if (__all(gA == gB)) {
    // every chunk of the wave is predicted on one grid: only exact ties are hard
    // (a term of the chunk is below the grid's binade top, so t < 2^24)
#pragma unroll
    for (int c = 0; c < CM; c++) {
      const float t = ldexpf(a[c], 150 - gA);
      const bool tie = __builtin_amdgcn_fractf(t) == 0.5f;
      kp[c] = ks;
      ks += tie ? 0u : (unsigned)__builtin_rintf(t);
      nh += tie ? 1 : 0;
      hardmask |= tie ? (1u << c) : 0u;
      gh[c] = gA;
    }
    gin = (hardmask & 1u) ? -1 : gA;
    gout = gA;
  } else {
    // (an easy step's term is below its grid's binade top, so t < 2^24; a hard
    // step's t, possibly huge, is not used)
    float P = P0;
    unsigned L = M0;
    int g0 = seq_grid_max(P * lo, L);
#pragma unroll
    for (int c = 0; c < CM; c++) {
      const float Pn = P + a[c];
      L = max(L, __float_as_uint(a[c]));
      const int g1 = seq_grid(Pn * hi);
      const float t = ldexpf(a[c], 150 - g0);
      const bool easy = (g0 == g1) && (__builtin_amdgcn_fractf(t) != 0.5f);
      kp[c] = ks;
      ks += easy ? (unsigned)__builtin_rintf(t) : 0u;
      nh += easy ? 0 : 1;
      hardmask |= easy ? 0u : (1u << c);
      if (c == 0) gin = easy ? g0 : -1;
      const int gn = seq_grid_max(Pn * lo, L);           // the next step's grid: the grid after a hard step
      gh[c] = gn;
      gout = easy ? g0 : gn;                             // grid of the run continuing past this step
      g0 = gn;
      P = Pn;
    }
  }

  // 3. wave scans of the k totals and hard counts, the boundary check between
  // lanes, and the hard steps recorded in the wave's region in order (k totals
  // are kept modulo 2^32: only differences within one run are used, and a run
  // on grid g adds at most 2^23 units)
  const unsigned kin = seq_wave_scan(ks);
  const int hin = seq_wave_scan(nh);
  const int gprev = (int)seq_shr1((unsigned)gout);
  if (lane > 0 && gin >= 0 && gin != gprev) S.bad = 1;
  if (nh && hin <= HCAP) {
    const unsigned kb = kin - ks;
    int m = wave * HCAP + hin - nh;
#pragma unroll
    for (int c = 0; c < CM; c++) {
      const bool h = (hardmask >> c) & 1u;
      if (h) S.hs[m] = make_int4((int)(kb + kp[c]), tid * CM + c, __float_as_int(a[c]), gh[c]);
      m += h ? 1 : 0;
    }
  }
  if (lane == 63) { S.wk[wave] = kin; S.wh[wave] = hin; S.wg[wave] = gout; }
  if (lane == 0) S.wgi[wave] = gin;
  sync();

  // 4. wave 0: the waves' offsets, the boundary checks between waves, and the
  // walk with the proof of every run.  The hard steps are taken 64 at a time:
  // lane i prepares run m = base + i (the run before hard step m; run htot is
  // the tail) and its exact total, the serial part adds only run totals and
  // hard terms, and the runs are then proven in parallel.
  if (wave == 0) {
    const unsigned wk_l = lane < NW ? S.wk[lane] : 0u;
    const int wh_l = lane < NW ? S.wh[lane] : 0;
    const int wg_prev = lane >= 1 && lane < NW ? S.wg[lane - 1] : 0;
    const int wgi_l = lane < NW ? S.wgi[lane] : -1;
    const unsigned koff_l = seq_row_scan(wk_l) - wk_l;            // lanes 0..NW-1
    const int hend_l = (int)seq_row_scan((unsigned)wh_l);        // end of the wave's hard steps
    const int hoff_l = hend_l - wh_l;
    const unsigned ktot = (unsigned)__builtin_amdgcn_readlane((int)(koff_l + wk_l), NW - 1);
    const int htot = __builtin_amdgcn_readlane(hend_l, NW - 1);
    bool ok = S.bad == 0 && !__any(lane < NW && (wh_l > HCAP || (wgi_l >= 0 && wgi_l != wg_prev)));
    int hend_s[NW];
#pragma unroll
    for (int v = 0; v < NW; v++) hend_s[v] = __builtin_amdgcn_readlane(hend_l, v);
    float s = 0.0f;
    int cx = 0, cy = -1, cw = 0;    // the record before the batch's first run: k prefix, index, grid after
    for (int base = 0; ok && base <= htot; base += 64) {
      const int m = base + lane;
      // the wave holding hard step m is the number of waves whose hard steps end
      // at or before m (NW for the tail); its offsets come from its lane
      int v = 0;
#pragma unroll
      for (int u = 0; u < NW; u++) v += hend_s[u] <= m ? 1 : 0;
      const int src = 4 * min(v, NW - 1);
      const int hoff_v = __builtin_amdgcn_ds_bpermute(src, hoff_l);
      const unsigned koff_v = (unsigned)__builtin_amdgcn_ds_bpermute(src, (int)koff_l);
      int4 cur = make_int4((int)ktot, NT * CM, 0, 0);                // the tail
      if (m < htot) {
        cur = S.hs[v * HCAP + m - hoff_v];
        cur.x = (int)((unsigned)cur.x + koff_v);
      }
      // the record before run m is lane m-1's (lane 0: the carry, DPP wave_shr:1)
      const int px = __builtin_amdgcn_update_dpp(cx, cur.x, 0x138, 0xf, 0xf, false);
      const int py = __builtin_amdgcn_update_dpp(cy, cur.y, 0x138, 0xf, 0xf, false);
      const int gp = __builtin_amdgcn_update_dpp(cw, cur.w, 0x138, 0xf, 0xf, false);
      cx = __builtin_amdgcn_readlane(cur.x, 63);
      cy = __builtin_amdgcn_readlane(cur.y, 63);
      cw = __builtin_amdgcn_readlane(cur.w, 63);
      const unsigned K = (unsigned)cur.x - (unsigned)px;
      const bool live = m <= htot && cur.y > py + 1;     // run m has steps
      const float T = live ? ldexpf((float)K, gp - 150) : 0.0f;   // 0 past the tail: adds nothing
      const float ah = __int_as_float(cur.z);                     // 0 from the tail on
      // The serial part: lane 0 alone (exec holds one lane, so its LDS reads,
      // adds and writes cost the least) adds the pairs in order, 8 at a time
      // with the next 8 in flight, and records the partial sum each run starts
      // from.  Pairs past the tail are (+0, +0) and leave s unchanged; the reads
      // ahead past them stay inside walk[] and are not used.  A wave's LDS
      // operations complete in order, so lane 0 reads what the wave has just
      // written, and the wave reads back what lane 0 has written.
      S.walk[lane] = make_float2(T, ah);
      asm volatile("" ::: "memory");                      // keep the reads below the writes
      if (lane == 0) {
        const int cnt = min(64, htot + 1 - base);
        const float4 *wp = reinterpret_cast<const float4 *>(S.walk);
        float4 q0 = wp[0], q1 = wp[1], q2 = wp[2], q3 = wp[3];
        for (int c = 0; c < cnt; c += 8) {
          const float4 n0 = wp[(c >> 1) + 4], n1 = wp[(c >> 1) + 5], n2 = wp[(c >> 1) + 6], n3 = wp[(c >> 1) + 7];
          float4 r0, r1;
          r0.x = s; s = s + q0.x; s = s + q0.y;
          r0.y = s; s = s + q0.z; s = s + q0.w;
          r0.z = s; s = s + q1.x; s = s + q1.y;
          r0.w = s; s = s + q1.z; s = s + q1.w;
          r1.x = s; s = s + q2.x; s = s + q2.y;
          r1.y = s; s = s + q2.z; s = s + q2.w;
          r1.z = s; s = s + q3.x; s = s + q3.y;
          r1.w = s; s = s + q3.z; s = s + q3.w;
          *reinterpret_cast<float4 *>(&S.wst[c]) = r0;
          *reinterpret_cast<float4 *>(&S.wst[c + 4]) = r1;
          q0 = n0; q1 = n1; q2 = n2; q3 = n3;
        }
      }
      asm volatile("" ::: "memory");
      const float st = S.wst[lane];                       // read only where live
      const float top = __uint_as_float((unsigned)(gp + 1) << 23);
      const bool bad = live && !(K <= (1u << 23) && seq_grid(st) == gp && T <= top - st);
      ok = ok && !__any(bad);
    }
    if (!ok && lane == 0) s = seq_serial(n, term);
    if (lane == 0) {
      S.result = s;
      if (info) { info[0] = htot; info[1] = !ok; }
    }
  }
  sync();
  return S.result;
}

}  // namespace qd

#endif
