// k_sample.hip - token sampling on the device: greedy (sampler.c:8-21) and
// temperature + top-k + top-p (sampler.c:54-143), with the reference's results
// bit for bit.
//
// Order of work for one logits row of V values (temperature > 0):
//   k_smp_probs   one block: max, e_j = expf((l_j - max) / T), the sequential
//                 float sum of the e_j evaluated exactly (qdev_seqsum.h, in
//                 chunks whose first term carries the previous partial sum),
//                 then p_j = e_j / sum (a true division, as sampler.c:79).
//   radix sort    (p, index) pairs by p descending.  The sort is stable, so equal
//                 probabilities keep ascending index order: the order the
//                 reference's qsort (glibc's merge sort, stable) leaves them in.
//   k_smp_pick    one wave: keep = top-k, then the top-p cut over the running
//                 sum, the kept mass z, u = uniform * z from the xorshift64
//                 state held in device memory, and the first kept entry whose
//                 running sum reaches u.  Every running sum is the reference's
//                 left-to-right float sum.
#include <hip/hip_runtime.h>
#include <hipcub/hipcub.hpp>

#include <climits>

#include "qdev_math.h"
#include "qdev_seqsum.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

constexpr int kNT = 1024;      // threads of the one-block kernels
constexpr int kCM = 32;        // terms per thread in one exact-sum chunk

__device__ float block_max(float v, float *red) {
  v = qd::wave_max_f32(v);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = v;
  __syncthreads();
  float m = red[0];
  for (int w = 1; w < (int)(blockDim.x >> 6); w++) m = fmaxf(m, red[w]);
  return m;
}

// p[j] = expf((l[j] - max_l) / temperature) / sum  (sampler.c:68-79)
__global__ __launch_bounds__(kNT) void k_smp_probs(const float *l, int V, float temperature, float *p) {
  __shared__ qd::SeqScratch S;
  __shared__ float red[kNT / 64];
  const int tid = threadIdx.x;
  float mx = -INFINITY;
  for (int j = tid; j < V; j += kNT) mx = fmaxf(mx, l[j]);
  mx = block_max(mx, red);
  for (int j = tid; j < V; j += kNT) p[j] = qd::expf_glibc((l[j] - mx) / temperature);
  __syncthreads();
  // sum = ((0 + e_0) + e_1) + ... in chunks of kNT*kCM terms; after the first
  // chunk, term 0 of a chunk is the partial sum so far ((0 + s) = s exactly).
  float s = 0.0f;
  for (int base = 0, off = 0; base < V; off = 1) {
    const int nnew = min(V - base, kNT * kCM - off), n = nnew + off;
    const float s0 = s;
    const int b0 = base, o0 = off;
    float a[kCM];
#pragma unroll
    for (int c = 0; c < kCM; c++) {
      const int q = tid * kCM + c;
      a[c] = q < n ? (q < o0 ? s0 : p[b0 + q - o0]) : 0.0f;
    }
    s = qd::seq_sum_nonneg<kNT, kCM>(a, n, S, [=](int i) { return i < o0 ? s0 : p[b0 + i - o0]; });
    base += nnew;
  }
  for (int j = tid; j < V; j += kNT) p[j] = p[j] / s;
}

// First index of the maximum (sampler.c:8-21).  Optional decode-state update as
// k_smp_pick's.
__global__ __launch_bounds__(kNT) void k_smp_argmax(const float *l, int V, int *tok, int *d_in, const int *d_state,
                                                     int *d_out, int max_seq) {
  __shared__ float sv[kNT / 64];
  __shared__ int si[kNT / 64];
  float best = -INFINITY;
  int idx = INT_MAX;
  for (int j = threadIdx.x; j < V; j += kNT) {
    const float v = l[j];
    if (idx == INT_MAX || v > best) { best = v; idx = j; }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (oi != INT_MAX && (idx == INT_MAX || ob > best || (ob == best && oi < idx))) { best = ob; idx = oi; }
  }
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int i0 = si[0];
    for (int w = 1; w < kNT / 64; w++)
      if (si[w] != INT_MAX && (i0 == INT_MAX || sv[w] > b || (sv[w] == b && si[w] < i0))) { b = sv[w]; i0 = si[w]; }
    tok[0] = i0;
    if (d_state) {
      const int P = d_state[0];
      if (P >= 1 && P - 1 < max_seq) d_out[P - 1] = i0;
      if (P >= d_state[1] && P <= max_seq) d_in[P] = i0;
    }
  }
}

__global__ void k_smp_iota(int *idx, int V) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j < V) idx[j] = j;
}

// Left-to-right float sum s = ((0 + ps[0]) + ps[1]) + ... over i < n, stopping at
// the first i where stop(s) holds; returns that i, or -1.  The wave loads 64
// terms at a time and every lane forms the same serial sum.
template <typename Stop>
__device__ int wave_sum_until(const float *ps, int n, float &s, Stop stop) {
  const int lane = threadIdx.x & 63;
  s = 0.0f;
  for (int b = 0; b < n; b += 64) {
    const float v = b + lane < n ? ps[b + lane] : 0.0f;
    const int cnt = min(64, n - b);
    for (int i = 0; i < cnt; i++) {
      s = s + __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), i));
      if (stop(s)) return b + i;
    }
  }
  return -1;
}

// sampler.c:81-139 over the sorted (ps, is) pairs; the xorshift64 step and
// uniform of sampler.c:31-45 on the device state *rng.  When d_state is given
// (decode loop) the token also becomes the next input: position P = d_state[0]
// (already advanced past the row's position) gets d_in[P] = token when P is past
// the prompt, and d_out[P - 1] records it, as k_argmax_final does for greedy.
__global__ __launch_bounds__(64) void k_smp_pick(const float *ps, const int *is, int V, int top_k, float top_p,
                                                  unsigned long long *rng, int *tok, int *d_in, const int *d_state,
                                                  int *d_out, int max_seq) {
  int keep = V;
  if (top_k > 0 && top_k < keep) keep = top_k;
  float s;
  if (top_p > 0.0f && top_p < 1.0f) {
    const int i = wave_sum_until(ps, keep, s, [=](float c) { return c >= top_p; });
    if (i >= 0) keep = i + 1;
  }
  if (keep < 1) keep = 1;
  float z;
  wave_sum_until(ps, keep, z, [](float) { return false; });
  unsigned long long x = *rng;
  x ^= x << 13;
  x ^= x >> 7;
  x ^= x << 17;
  const float r = (float)((double)(x >> 11) * (1.0 / 9007199254740992.0));
  const float u = r * z;
  const int i = wave_sum_until(ps, keep, s, [=](float acc) { return u <= acc; });
  const int t = is[i >= 0 ? i : keep - 1];
  if (threadIdx.x == 0) {
    *rng = x;
    tok[0] = t;
    if (d_state) {
      const int P = d_state[0];
      if (P >= 1 && P - 1 < max_seq) d_out[P - 1] = t;
      if (P >= d_state[1] && P <= max_seq) d_in[P] = t;
    }
  }
}

size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

size_t sort_temp_bytes(int V) {
  size_t bytes = 0;
  const hipError_t e = hipcub::DeviceRadixSort::SortPairsDescending(
      nullptr, bytes, (const float *)nullptr, (float *)nullptr, (const int *)nullptr, (int *)nullptr, V, 0, 32,
      qh::stream());
  return e == hipSuccess ? bytes : 0;
}

}  // namespace

// Scratch of qhip_sample for rows of V logits: p, sorted p, indices, sorted
// indices and the radix sort's temporary storage.
extern "C" size_t qhip_sample_scratch(int V) {
  if (V <= 0) return 0;
  return 4 * al256((size_t)V * 4) + al256(sort_temp_bytes(V));
}

extern "C" int qhip_sample(const float *logits, int V, float temperature, int top_k, float top_p, void *scratch,
                           size_t scratch_bytes, unsigned long long *rng, int *tok, int *d_in, const int *d_state,
                           int *d_out, int max_seq) {
  if (V <= 0 || !(temperature > 0.0f)) return qh::fail_msg("sample: needs V > 0 and temperature > 0");
  if (scratch_bytes < qhip_sample_scratch(V)) return qh::fail_msg("sample: scratch too small");
  uint8_t *b = static_cast<uint8_t *>(scratch);
  const size_t slot = al256((size_t)V * 4);
  float *p = reinterpret_cast<float *>(b), *ps = reinterpret_cast<float *>(b + slot);
  int *idx = reinterpret_cast<int *>(b + 2 * slot), *is = reinterpret_cast<int *>(b + 3 * slot);
  void *temp = b + 4 * slot;
  size_t temp_bytes = scratch_bytes - 4 * slot;
  QH_LAUNCH(QK_OTHER, k_smp_probs, dim3(1), dim3(kNT), 0, logits, V, temperature, p);
  QH_LAUNCH(QK_OTHER, k_smp_iota, dim3((V + 255) / 256), dim3(256), 0, idx, V);
  hipError_t e = hipcub::DeviceRadixSort::SortPairsDescending(temp, temp_bytes, p, ps, idx, is, V, 0, 32, qh::stream());
  if (e != hipSuccess) return qh::fail("sample: radix sort", e);
  QH_LAUNCH(QK_OTHER, k_smp_pick, dim3(1), dim3(64), 0, ps, is, V, top_k, top_p, rng, tok, d_in, d_state, d_out,
            max_seq);
  return 0;
}

extern "C" int qhip_argmax_row(const float *logits, int V, int *tok, int *d_in, const int *d_state, int *d_out,
                               int max_seq) {
  if (V <= 0) return qh::fail_msg("argmax: needs V > 0");
  QH_LAUNCH(QK_OTHER, k_smp_argmax, dim3(1), dim3(kNT), 0, logits, V, tok, d_in, d_state, d_out, max_seq);
  return 0;
}
