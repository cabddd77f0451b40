// qdev_math.h - device arithmetic that must agree bit for bit with the host.
//
// Compiled with -ffp-contract=off: every product and sum below is rounded where
// it is written, exactly as ISO C evaluates the same expressions on the host.
#ifndef QDEV_MATH_H
#define QDEV_MATH_H

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qd {

// ---------------------------------------------------------------------------
// expf with the results of glibc 2.35's x86-64 FMA variant, which is what the
// reference's `expf` resolves to on its hosts (llama.c:567,585).  Published
// method (glibc sysdeps/ieee754/flt-32/e_expf.c, from Arm's optimized-routines):
// x*32/ln2 = k + r, 2^(k/32) from a 32-entry table, 2^(r/32) from a cubic, all
// in double; the reduction and the polynomial steps are fused multiply-adds.
// The table holds the double nearest to 2^(i/32), minus i << 47 in its bits, so
// adding k << 47 applies the exponent.  Verified against the host libm on every
// float input (tests/test_gpu_parity.py).
// ---------------------------------------------------------------------------
__device__ __constant__ static const uint64_t kExp2Tab[32] = {
    0x3ff0000000000000ULL, 0x3fefd9b0d3158574ULL, 0x3fefb5586cf9890fULL, 0x3fef9301d0125b51ULL,
    0x3fef72b83c7d517bULL, 0x3fef54873168b9aaULL, 0x3fef387a6e756238ULL, 0x3fef1e9df51fdee1ULL,
    0x3fef06fe0a31b715ULL, 0x3feef1a7373aa9cbULL, 0x3feedea64c123422ULL, 0x3feece086061892dULL,
    0x3feebfdad5362a27ULL, 0x3feeb42b569d4f82ULL, 0x3feeab07dd485429ULL, 0x3feea47eb03a5585ULL,
    0x3feea09e667f3bcdULL, 0x3fee9f75e8ec5f74ULL, 0x3feea11473eb0187ULL, 0x3feea589994cce13ULL,
    0x3feeace5422aa0dbULL, 0x3feeb737b0cdc5e5ULL, 0x3feec49182a3f090ULL, 0x3feed503b23e255dULL,
    0x3feee89f995ad3adULL, 0x3feeff76f2fb5e47ULL, 0x3fef199bdd85529cULL, 0x3fef3720dcef9069ULL,
    0x3fef5818dcfba487ULL, 0x3fef7c97337b9b5fULL, 0x3fefa4afa2a490daULL, 0x3fefd0765b6e4540ULL};

// tab: the table above, or a copy of it (an LDS copy saves a memory round trip
// per value when many values are formed); the result does not depend on it.
//
// The special cases of |x| >= 88 (glibc's abstop >= 0x42b branch) are applied
// by selects after the main path, which every lane evaluates (its table index
// is masked, so any input is safe there): -inf and x < -0x1.9fe368p6 give +0,
// x > 0x1.62e42ep6 gives +inf, NaN and +inf give x + x; every other input,
// those with 88 <= |x| in between included, takes the main path's value, as in
// glibc.  No branch, so that many values in a wave cost no divergence.
__device__ __forceinline__ float expf_glibc(float x, const uint64_t *tab = kExp2Tab) {
  const uint32_t ux = __float_as_uint(x);
  const uint32_t abstop = (ux >> 20) & 0x7ffu;
  const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double Shift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
  const double xd = (double)x;
  double kd = __builtin_fma(InvLn2N, xd, Shift);
  const uint64_t ki = (uint64_t)__double_as_longlong(kd);
  kd -= Shift;
  const double r = __builtin_fma(InvLn2N, xd, -kd);
  const uint64_t t = tab[ki & 31] + (ki << 47);
  const double s = __longlong_as_double((long long)t);
  const double z = __builtin_fma(C0, r, C1);
  const double r2 = r * r;
  double y = __builtin_fma(C2, r, 1.0);
  y = __builtin_fma(z, r2, y);
  y = y * s;
  float res = (float)y;
  res = x < -0x1.9fe368p6f ? 0.0f : res;                            // underflow, -inf
  res = x > 0x1.62e42ep6f ? __uint_as_float(0x7f800000u) : res;     // overflow, +inf
  res = abstop >= 0x7f8u && ux != 0xff800000u ? x + x : res;        // nan, +inf
  return res;
}

// expf_glibc of N values in place, the same operations stage by stage within
// batches of up to 8 values: the batch's reductions, then its table reads, then
// its polynomials, so that the values' dependent chains and table reads overlap
// (eight at a time: a whole row of 32 would hold 32 doubles of each stage in
// registers).  The empty asm marks the main path's result as needed on every
// lane, so the compiler cannot turn the special-case selects into branches
// around it (which serialises the values).
template <int N>
__device__ __forceinline__ void expf_glibc_n(float (&v)[N], const uint64_t *tab) {
  constexpr int B = N < 8 ? N : 8;
  static_assert(N % B == 0, "batches of 8");
  const double InvLn2N = 0x1.71547652b82fep+0 * 32.0;
  const double Shift = 0x1.8p+52;
  const double C0 = 0x1.c6af84b912394p-5 / 32.0 / 32.0 / 32.0;
  const double C1 = 0x1.ebfce50fac4f3p-3 / 32.0 / 32.0;
  const double C2 = 0x1.62e42ff0c52d6p-1 / 32.0;
#pragma unroll
  for (int b = 0; b < N; b += B) {
    double r[B];
    uint64_t ki[B], t[B];
#pragma unroll
    for (int c = 0; c < B; c++) {
      const double xd = (double)v[b + c];
      double kd = __builtin_fma(InvLn2N, xd, Shift);
      ki[c] = (uint64_t)__double_as_longlong(kd);
      kd -= Shift;
      r[c] = __builtin_fma(InvLn2N, xd, -kd);
    }
#pragma unroll
    for (int c = 0; c < B; c++) t[c] = tab[ki[c] & 31];
#pragma unroll
    for (int c = 0; c < B; c++) {
      const double s = __longlong_as_double((long long)(t[c] + (ki[c] << 47)));
      const double z = __builtin_fma(C0, r[c], C1);
      const double r2 = r[c] * r[c];
      double y = __builtin_fma(C2, r[c], 1.0);
      y = __builtin_fma(z, r2, y);
      y = y * s;
      float res = (float)y;
      asm volatile("" : "+v"(res));
      const float x = v[b + c];
      const uint32_t ux = __float_as_uint(x);
      res = x < -0x1.9fe368p6f ? 0.0f : res;
      res = x > 0x1.62e42ep6f ? __uint_as_float(0x7f800000u) : res;
      res = ((ux >> 20) & 0x7ffu) >= 0x7f8u && ux != 0xff800000u ? x + x : res;
      v[b + c] = res;
    }
  }
}

// ---------------------------------------------------------------------------
// tanhf with the results of glibc 2.35's, which the reference's GELU calls
// (activation.c:43-50).  Published method (glibc sysdeps/ieee754/flt-32/
// s_tanhf.c and s_expm1f.c, from Sun's fdlibm): tanh(x) = 1 - 2 / (expm1(2|x|)
// + 2) for |x| >= 1, -t / (t + 2) with t = expm1(-2|x|) below, and expm1 by an
// argument reduction x = k ln2 + r (ln2 split in two floats) and a rational
// correction of degree 5 in r^2, all in float (glibc's generic float build has
// no fused multiply-adds).  Checked against the host libm on every float input
// (tests/test_gpu_gpt.py).
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ float expm1f_glibc(float x) {
  const float one = 1.0f, huge = 1.0e+30f, tiny = 1.0e-30f;
  const float o_threshold = 8.8721679688e+01f, ln2_hi = 6.9313812256e-01f, ln2_lo = 9.0580006145e-06f;
  const float invln2 = 1.4426950216e+00f;
  const float Q1 = -3.3333335072e-02f, Q2 = 1.5873016091e-03f, Q3 = -7.9365076090e-05f, Q4 = 4.0082177293e-06f,
              Q5 = -2.0109921195e-07f;
  float y, hi, lo, c = 0.0f, t, e, hxs, hfx, r1;
  int k;
  uint32_t hx = __builtin_bit_cast(uint32_t, x);
  const uint32_t xsb = hx & 0x80000000u;
  hx &= 0x7fffffffu;
  if (hx >= 0x4195b844u) {                       // |x| >= 27 ln2
    if (hx >= 0x42b17218u) {
      if (hx > 0x7f800000u) return x + x;        // NaN
      if (hx == 0x7f800000u) return xsb == 0 ? x : -1.0f;
      if (x > o_threshold) return huge * huge;
    }
    if (xsb != 0) return tiny - one;
  }
  if (hx > 0x3eb17218u) {                        // |x| > ln2 / 2: reduce
    if (hx < 0x3F851592u) {
      if (xsb == 0) { hi = x - ln2_hi; lo = ln2_lo; k = 1; }
      else { hi = x + ln2_hi; lo = -ln2_lo; k = -1; }
    } else {
      k = (int)(invln2 * x + (xsb == 0 ? 0.5f : -0.5f));
      t = (float)k;
      hi = x - t * ln2_hi;
      lo = t * ln2_lo;
    }
    x = hi - lo;
    c = (hi - x) - lo;
  } else if (hx < 0x33000000u) {                 // |x| < 2^-25
    t = huge + x;
    return x - (t - (huge + x));
  } else {
    k = 0;
  }
  hfx = 0.5f * x;
  hxs = x * hfx;
  r1 = one + hxs * (Q1 + hxs * (Q2 + hxs * (Q3 + hxs * (Q4 + hxs * Q5))));
  t = 3.0f - r1 * hfx;
  e = hxs * ((r1 - t) / (6.0f - x * t));
  if (k == 0) return x - (x * e - hxs);
  e = (x * (e - c) - c);
  e -= hxs;
  if (k == -1) return 0.5f * (x - e) - 0.5f;
  if (k == 1) {
    if (x < -0.25f) return -2.0f * (e - (x + 0.5f));
    return one + 2.0f * (x - e);
  }
  if (k <= -2 || k > 56) {
    y = one - (e - x);
    y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
    return y - one;
  }
  if (k < 23) {
    t = __builtin_bit_cast(float, 0x3f800000u - (0x1000000u >> k));     // 1 - 2^-k
    y = t - (e - x);
    y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
  } else {
    t = __builtin_bit_cast(float, (uint32_t)(0x7f - k) << 23);          // 2^-k
    y = x - (e + t);
    y += one;
    y = __builtin_bit_cast(float, __builtin_bit_cast(uint32_t, y) + ((uint32_t)k << 23));
  }
  return y;
}

__host__ __device__ __forceinline__ float tanhf_glibc(float x) {
  const float one = 1.0f, two = 2.0f, tiny = 1.0e-30f;
  float t, z;
  const uint32_t jx = __builtin_bit_cast(uint32_t, x), ix = jx & 0x7fffffffu;
  if (ix >= 0x7f800000u) return (int)jx >= 0 ? one / x + one : one / x - one;   // +-inf, NaN
  if (ix < 0x41b00000u) {                        // |x| < 22
    if (ix == 0) return x;
    if (ix < 0x24000000u) return x * (one + x);  // |x| < 2^-55
    if (ix >= 0x3f800000u) {
      t = expm1f_glibc(two * fabsf(x));
      z = one - two / (t + two);
    } else {
      t = expm1f_glibc(-two * fabsf(x));
      z = -t / (t + two);
    }
  } else {
    z = one - tiny;
  }
  return (int)jx >= 0 ? z : -z;
}

// GELU, tanh form (activation.c:43-50): 0.5 x (1 + tanh(k (x + 0.044715 x^3))),
// with C's left-to-right evaluation of the products.
__device__ __forceinline__ float gelu_tanh(float x) {
  const float k = 0.7978845608028654f;
  const float inner = k * (x + 0.044715f * x * x * x);
  return 0.5f * x * (1.0f + tanhf_glibc(inner));
}

// Block barrier for LDS hand-offs: waits for this wave's LDS operations and then
// for the other waves, leaving global loads in flight (__syncthreads() waits for
// every outstanding global load too, which would stall any prefetch across it).
// The memory clobber keeps the compiler from moving memory accesses across it.
__device__ __forceinline__ void lds_sync() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

// The meeting points of a block-wide routine (the exact sums, rmsnorm): every
// wave of the block at s_barrier ...
struct BlockSync {
  __device__ __forceinline__ void operator()() const { lds_sync(); }
};

// ... or only the first `waves` waves, at an LDS counter, so that the block's
// other waves (loading weights, say) are not waited for.  ctr is zeroed and
// published (one block barrier) before its first use; epoch is the calling
// wave's running target.  Every wave of the group calls it the same number of
// times.  A wave's LDS writes have landed before its increment, and LDS
// requests are served in order, so once a wave sees the count reach the target
// it sees every group member's earlier writes.  The wait polls the counter
// without sleeping between reads (sleeping added latency to every meeting).
struct GroupSync {
  unsigned *ctr;
  unsigned waves;
  unsigned *epoch;
  __device__ __forceinline__ void operator()() const {
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    const unsigned target = (*epoch += waves);
    if ((threadIdx.x & 63) == 0) __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    while (__hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < target) {
    }
    asm volatile("" ::: "memory");
  }
};

// Copies the table into LDS (dst: 32 entries); the caller synchronizes.
__device__ __forceinline__ void exp_table_to_lds(uint64_t *dst) {
  if (threadIdx.x < 32) dst[threadIdx.x] = kExp2Tab[threadIdx.x];
}

// ---------------------------------------------------------------------------
// Seeded generator: the device side of the specification in oracle/synth.h
// (splitmix64 finaliser keyed by (seed, tensor id), Box-Muller with ln, sqrt,
// cos and sin evaluated by +, -, * only).  Written independently of the CPU
// checker; equality is proven by the per-tensor digests.
// ---------------------------------------------------------------------------
__host__ __device__ __forceinline__ uint64_t mix64(uint64_t z) {
  z = (z ^ (z >> 30)) * 0xBF58476D1CE4E5B9ULL;
  z = (z ^ (z >> 27)) * 0x94D049BB133111EBULL;
  return z ^ (z >> 31);
}

__host__ __device__ __forceinline__ uint64_t gen_key(uint64_t seed, uint64_t tid) {
  return mix64(mix64(seed + 0x9E3779B97F4A7C15ULL) ^ (tid * 0xD1B54A32D192ED03ULL));
}

__device__ __forceinline__ double gen_ln(double u) {
  const uint64_t b = (uint64_t)__double_as_longlong(u);
  int e = (int)((b >> 52) & 0x7ff) - 1023;
  double m = __longlong_as_double((long long)((b & 0x000FFFFFFFFFFFFFULL) | 0x3FF0000000000000ULL));
  if (m > 1.4142135623730951) { m = m * 0.5; e = e + 1; }
  const double d = m + 1.0;
  double r = 0.5;
#pragma unroll
  for (int k = 0; k < 6; k++) r = r * (2.0 - d * r);
  const double t = (m - 1.0) * r;
  const double t2 = t * t;
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

__device__ __forceinline__ double gen_sqrt(double y) {
  if (!(y > 0.0)) return 0.0;
  double g = __longlong_as_double((long long)(0x5FE6EB50C7B537A9ULL - ((uint64_t)__double_as_longlong(y) >> 1)));
  const double hy = 0.5 * y;
#pragma unroll
  for (int k = 0; k < 6; k++) g = g * (1.5 - (hy * g) * g);
  return y * g;
}

__device__ __forceinline__ void gen_cos_sin_2pi(double v, double &c, double &s) {
  const double v8 = v * 8.0;
  const int q = (int)v8;
  double f = v8 - (double)q;
  const int odd = q & 1;
  if (odd) f = 1.0 - f;
  const double a = f * 0.78539816339744830962;
  const double a2 = a * a;
  double sp = -1.0 / 355687428096000.0;
  sp = sp * a2 + 1.0 / 1307674368000.0;
  sp = sp * a2 - 1.0 / 6227020800.0;
  sp = sp * a2 + 1.0 / 39916800.0;
  sp = sp * a2 - 1.0 / 362880.0;
  sp = sp * a2 + 1.0 / 5040.0;
  sp = sp * a2 - 1.0 / 120.0;
  sp = sp * a2 + 1.0 / 6.0;
  const double sa = a - (a * a2) * sp;
  double cp = 1.0 / 6402373705728000.0;
  cp = cp * a2 - 1.0 / 20922789888000.0;
  cp = cp * a2 + 1.0 / 87178291200.0;
  cp = cp * a2 - 1.0 / 479001600.0;
  cp = cp * a2 + 1.0 / 3628800.0;
  cp = cp * a2 - 1.0 / 40320.0;
  cp = cp * a2 + 1.0 / 720.0;
  cp = cp * a2 - 1.0 / 24.0;
  cp = cp * a2 + 0.5;
  const double ca = 1.0 - a2 * cp;
  const double cb = odd ? sa : ca, sb = odd ? ca : sa;
  switch (q >> 1) {
    case 0: c = cb; s = sb; break;
    case 1: c = -sb; s = cb; break;
    case 2: c = -cb; s = -sb; break;
    default: c = sb; s = -cb; break;
  }
}

__device__ __forceinline__ double gen_normal(uint64_t key, uint64_t i) {
  const uint64_t p = i >> 1;
  const uint64_t h1 = mix64(key + (p + 1) * 0x9E3779B97F4A7C15ULL);
  const uint64_t h2 = mix64(h1 ^ 0x6A09E667F3BCC909ULL);
  const double u1 = (double)((h1 >> 11) + 1) * 0x1p-53;
  const double u2 = (double)(h2 >> 11) * 0x1p-53;
  const double rad = gen_sqrt(-2.0 * gen_ln(u1));
  double c, s;
  gen_cos_sin_2pi(u2, c, s);
  return rad * ((i & 1) ? s : c);
}

__device__ __forceinline__ float gen_value(uint64_t key, uint64_t i, double sigma) {
  return (float)(gen_normal(key, i) * sigma);
}

// int8 quantization of one value with the reference's rounding (quant.c:74-77):
// lrintf is round-half-even in the default mode, then clamp to +-127; NaN gives 0
// ((int)lrintf(NaN) is the low half of LONG_MIN on x86-64).  v_cvt_i32_f32 turns
// NaN into 0 and saturates values out of the int range, so clamping the integer
// after it is clamping the float before it.
__device__ __forceinline__ int quant_i8(float v, float inv) {
  int q;
  asm("v_cvt_i32_f32 %0, %1" : "=v"(q) : "v"(__builtin_rintf(v * inv)));
  return min(max(q, -127), 127);
}

// The low bytes of four quantized values, little-endian in one word (v_perm_b32:
// selector bytes 0-3 pick the second operand's bytes, 4-7 the first's, 12 gives 0).
__device__ __forceinline__ uint32_t pack_i8x4(int q0, int q1, int q2, int q3) {
  const uint32_t lo = __builtin_amdgcn_perm((uint32_t)q1, (uint32_t)q0, 0x0c0c0400u);
  const uint32_t hi = __builtin_amdgcn_perm((uint32_t)q3, (uint32_t)q2, 0x0c0c0400u);
  return __builtin_amdgcn_perm(hi, lo, 0x05040100u);
}

__device__ __forceinline__ uint32_t quant_i8x4(float a, float b, float c, float d, float inv) {
  return pack_i8x4(quant_i8(a, inv), quant_i8(b, inv), quant_i8(c, inv), quant_i8(d, inv));
}

// ---------------------------------------------------------------------------
// wave64 reductions through DPP lane moves (no LDS round trips): within each
// row of 16 lanes by swaps at distance 1 and 2 (quad_perm) and the half-row and
// row mirrors, then across the four rows by reading lanes 0, 16, 32 and 48.
// Every lane receives the result.
// ---------------------------------------------------------------------------
template <int CTRL>
__device__ __forceinline__ int dpp_mov(int v) {
  return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xf, 0xf, false);
}

__device__ __forceinline__ int wave_sum_i32(int v) {
  v += dpp_mov<0xB1>(v);      // quad_perm [1,0,3,2]
  v += dpp_mov<0x4E>(v);      // quad_perm [2,3,0,1]
  v += dpp_mov<0x141>(v);     // row_half_mirror
  v += dpp_mov<0x140>(v);     // row_mirror
  return __builtin_amdgcn_readlane(v, 0) + __builtin_amdgcn_readlane(v, 16) + __builtin_amdgcn_readlane(v, 32) +
         __builtin_amdgcn_readlane(v, 48);
}

// Sum over the wave in a fixed order; every lane receives the same bits.
__device__ __forceinline__ float wave_sum_f32(float v) {
  v += __int_as_float(dpp_mov<0xB1>(__float_as_int(v)));
  v += __int_as_float(dpp_mov<0x4E>(__float_as_int(v)));
  v += __int_as_float(dpp_mov<0x141>(__float_as_int(v)));
  v += __int_as_float(dpp_mov<0x140>(__float_as_int(v)));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return (r0 + r1) + (r2 + r3);
}

__device__ __forceinline__ float wave_max_f32(float v) {
  v = fmaxf(v, __int_as_float(dpp_mov<0xB1>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<0x4E>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<0x141>(__float_as_int(v))));
  v = fmaxf(v, __int_as_float(dpp_mov<0x140>(__float_as_int(v))));
  const float r0 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 0));
  const float r1 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 16));
  const float r2 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 32));
  const float r3 = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), 48));
  return fmaxf(fmaxf(r0, r1), fmaxf(r2, r3));
}

}  // namespace qd

#endif
