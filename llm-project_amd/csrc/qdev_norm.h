// qdev_norm.h - rmsnorm of one activation row by one block (rmsnorm.c:7-21),
// shared by the standalone norm kernel and the GEMVs that normalize their own
// input.
//
//   ms = (sum_i x_i^2, in order) * (1 / n);  r = 1 / sqrtf(ms + eps);  y_i = (x_i * r) * g_i
//
// The sum of squares is the reference's sequential loop, evaluated exactly by
// seq_sum_nonneg; every other step is the reference's operation on each
// element.  The returned scale is the activation quantizer's (quant.c:66-70):
// max|y| / 127, or 1 for an all-zero row.
#ifndef QDEV_NORM_H
#define QDEV_NORM_H

#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qdev_seqsum.h"

namespace qd {

// Thread t of the NT-thread block owns elements [t*CM, t*CM + CM) of the row xr
// (n values, NT*CM >= n).  rmsnorm_load issues the loads of its x values into
// y[] and of the gains into gm[] (0 past n), so that a caller can put other
// loads in flight before the values are needed.
template <int CM>
__device__ __forceinline__ void rmsnorm_load(const float *xr, int n, const float *gamma, float (&y)[CM],
                                             float (&gm)[CM]) {
  static_assert(CM % 4 == 0, "chunk of whole 16-byte words");
  const int j0 = threadIdx.x * CM;
  if (j0 + CM <= n && (n & 3) == 0) {
#pragma unroll
    for (int c = 0; c < CM; c += 4) {
      const float4 t = *reinterpret_cast<const float4 *>(xr + j0 + c);
      const float4 u = *reinterpret_cast<const float4 *>(gamma + j0 + c);
      y[c] = t.x; y[c + 1] = t.y; y[c + 2] = t.z; y[c + 3] = t.w;
      gm[c] = u.x; gm[c + 1] = u.y; gm[c + 2] = u.z; gm[c + 3] = u.w;
    }
  } else {
#pragma unroll
    for (int c = 0; c < CM; c++) {
      y[c] = j0 + c < n ? xr[j0 + c] : 0.0f;
      gm[c] = j0 + c < n ? gamma[j0 + c] : 0.0f;
    }
  }
}

// Normalizes the loaded y[] in place (0 past n) and returns the quantization
// scale of the whole row.  red holds NT/64 floats.  All NT threads must call it;
// sync as for seq_sum_nonneg.
template <int NT, int CM, typename Sync = BlockSync>
__device__ __forceinline__ float rmsnorm_apply(const float *xr, int n, float eps, float (&y)[CM],
                                               const float (&gm)[CM], float *red, SeqScratch &seq,
                                               const Sync &sync = Sync()) {
  const int j0 = threadIdx.x * CM;
  float sq[CM];
#pragma unroll
  for (int c = 0; c < CM; c++) sq[c] = y[c] * y[c];
  float ms = seq_sum_nonneg<NT, CM>(sq, n, seq, [&](int i) { return xr[i] * xr[i]; }, nullptr, sync);   // rmsnorm.c:15
  ms *= 1.0f / (float)n;
  const float r = 1.0f / sqrtf(ms + eps);
  float mx = 0.0f;
#pragma unroll
  for (int c = 0; c < CM; c++) {
    y[c] = j0 + c < n ? y[c] * r * gm[c] : 0.0f;
    mx = fmaxf(mx, fabsf(y[c]));
  }
  mx = wave_max_f32(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  sync();
  mx = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; w++) mx = fmaxf(mx, red[w]);
  return (mx > 0.0f) ? mx / 127.0f : 1.0f;
}

// The fast decode mode's form of rmsnorm_apply: the sum of squares is a fixed-
// shape tree (per-thread partial sums, then the wave, then the waves in order),
// so it is deterministic but not the reference's sequential order; everything
// after it is the same.  red holds 2 * NT/64 floats; sync as for rmsnorm_apply.
template <int NT, int CM, typename Sync = BlockSync>
__device__ __forceinline__ float rmsnorm_apply_fast(int n, float eps, float (&y)[CM], const float (&gm)[CM],
                                                    float *red, const Sync &sync = Sync()) {
  const int j0 = threadIdx.x * CM;
  float ss = 0.0f;
#pragma unroll
  for (int c = 0; c < CM; c++) ss = __builtin_fmaf(y[c], y[c], ss);      // y is 0 past n
  ss = wave_sum_f32(ss);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = ss;
  sync();
  ss = red[0];
#pragma unroll
  for (int w = 1; w < NT / 64; w++) ss += red[w];
  const float ms = ss * (1.0f / (float)n);
  const float r = 1.0f / sqrtf(ms + eps);
  float mx = 0.0f;
#pragma unroll
  for (int c = 0; c < CM; c++) {
    y[c] = j0 + c < n ? y[c] * r * gm[c] : 0.0f;
    mx = fmaxf(mx, fabsf(y[c]));
  }
  mx = wave_max_f32(mx);
  if ((threadIdx.x & 63) == 0) red[NT / 64 + (threadIdx.x >> 6)] = mx;
  sync();
  mx = red[NT / 64];
#pragma unroll
  for (int w = 1; w < NT / 64; w++) mx = fmaxf(mx, red[NT / 64 + w]);
  return (mx > 0.0f) ? mx / 127.0f : 1.0f;
}

// Both steps: y[] receives this thread's normalized values.
template <int NT, int CM>
__device__ __forceinline__ float rmsnorm_row(const float *xr, int n, const float *gamma, float eps, float (&y)[CM],
                                             float *red, SeqScratch &seq) {
  float gm[CM];
  rmsnorm_load<CM>(xr, n, gamma, y, gm);
  return rmsnorm_apply<NT, CM>(xr, n, eps, y, gm, red, seq);
}

// The quantized bytes of y[c .. c+3] (quant.c:71-78), packed little-endian.
template <int CM>
__device__ __forceinline__ uint32_t quant_word(const float (&y)[CM], int c, float inv) {
  return quant_i8x4(y[c], y[c + 1], y[c + 2], y[c + 3], inv);
}

}  // namespace qd

#endif
