// k_sample.hip - token sampling on the device: greedy (sampler.c:8-21) and
// temperature + top-k + top-p (sampler.c:54-143), with the reference's results
// bit for bit.
//
// Order of work for one logits row of V values (temperature > 0):
//   k_smp_bmax, k_smp_exp   blockwise: max, e_j = expf((l_j - max) / T)
//   k_smp_sum     one block: the sequential float sum of the e_j evaluated
//                 exactly (qdev_seqsum.h, in chunks whose first term carries the
//                 previous partial sum); p_j = e_j / sum (a true division,
//                 sampler.c:79) is formed where it is used.
//   top-k <= 64   each block selects the 64 largest (p, index) keys of its 1024
//                 by a bitwise search for the 64th largest; one block selects
//                 the 64 largest of those (the global top-k is among the blocks'
//                 top-k) and one wave sorts them.
//   otherwise     a stable radix sort of all (p, index) pairs by p descending
//                 (k_rs_*: four passes of 8 bits over the bits of p).  Both
//                 orders are p descending, then index ascending: the order the
//                 reference's qsort (glibc's merge sort, stable) leaves them in.
//   k_smp_pick    one wave: keep = top-k, then the top-p cut over the running
//                 sum, the kept mass z, u = uniform * z from the xorshift64
//                 state held in device memory, and the first kept entry whose
//                 running sum reaches u.  Every running sum is the reference's
//                 left-to-right float sum.
#include <hip/hip_runtime.h>

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

constexpr int kSlice = 1024;   // logits per block in the blockwise kernels (256 threads x 4)
constexpr int kTopC = 64;      // candidates each block passes to the top-k merge
constexpr int kMergeCap = 8192;

// Per-block maximum of the logits.
__global__ __launch_bounds__(256) void k_smp_bmax(const float *l, int V, float *bm) {
  __shared__ float red[4];
  const int j0 = blockIdx.x * kSlice + threadIdx.x;
  float mx = -INFINITY;
#pragma unroll
  for (int r = 0; r < 4; r++)
    if (j0 + 256 * r < V) mx = fmaxf(mx, l[j0 + 256 * r]);
  mx = block_max(mx, red);
  if (threadIdx.x == 0) bm[blockIdx.x] = mx;
}

// e[j] = expf((l[j] - max_l) / temperature)  (sampler.c:68-76); max_l from the
// per-block maxima (a maximum does not depend on the order it is taken in).
__global__ __launch_bounds__(256) void k_smp_exp(const float *l, int V, float temperature, const float *bm, int nb,
                                                 float *e) {
  __shared__ float red[4];
  float mx = -INFINITY;
  for (int i = threadIdx.x; i < nb; i += 256) mx = fmaxf(mx, bm[i]);
  mx = block_max(mx, red);
  const int j0 = blockIdx.x * kSlice + threadIdx.x;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int j = j0 + 256 * r;
    if (j < V) e[j] = qd::expf_glibc((l[j] - mx) / temperature);
  }
}

// *S = ((0 + e_0) + e_1) + ... + e_{V-1} in float (sampler.c:76), evaluated exactly
// in chunks of kSumNT*kCM terms; after the first chunk, term 0 of a chunk is the
// partial sum so far ((0 + s) = s exactly).  Eight waves: each wave may record
// up to 64 hard steps (the first chunk's partial sums cross many binades early
// on) before the exact-sum walk has to fall back to the loop; sixteen waves
// (32 each) fell back on real logits.
constexpr int kSumNT = 512;
__global__ __launch_bounds__(kSumNT) void k_smp_sum(const float *e, int V, float *S_out) {
  __shared__ qd::SeqScratch S;
  const int tid = threadIdx.x;
  float s = 0.0f;
  for (int base = 0, off = 0; base < V; off = 1) {
    const int nnew = min(V - base, kSumNT * kCM - off), n = nnew + off;
    const float s0 = s;
    const int b0 = base, o0 = off;
    float a[kCM];
#pragma unroll
    for (int c = 0; c < kCM; c++) {
      const int q = tid * kCM + c;
      a[c] = q < n ? (q < o0 ? s0 : e[b0 + q - o0]) : 0.0f;
    }
    s = qd::seq_sum_nonneg<kSumNT, kCM>(a, n, S, [=](int i) { return i < o0 ? s0 : e[b0 + i - o0]; });
    base += nnew;
  }
  if (tid == 0) S_out[0] = s;
}

// p[j] = e[j] / S  (sampler.c:79)
__global__ __launch_bounds__(256) void k_smp_div(const float *e, int V, const float *S, float *p) {
  const float s = S[0];
  const int j0 = blockIdx.x * kSlice + threadIdx.x;
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int j = j0 + 256 * r;
    if (j < V) p[j] = e[j] / s;
  }
}

// Sort key of (p, j): probability descending, then index ascending (the order
// of a stable sort by probability, sampler.c:82).  p >= 0, so its bits order
// like its values; 0 never is a real key (j < 2^31).
__device__ __forceinline__ unsigned long long prob_key(float p, int j) {
  return ((unsigned long long)__float_as_uint(p) << 32) | (unsigned)(0xffffffffu - (unsigned)j);
}

// Sum of one int per thread over the block; red holds 2 * (NT / 64) ints and
// alternates halves between calls (parity), so one barrier per call suffices.
template <int NT>
__device__ __forceinline__ int block_count(int n, int *red, int parity) {
  n = qd::wave_sum_i32(n);
  int *r = red + parity * (NT / 64);
  if ((threadIdx.x & 63) == 0) r[threadIdx.x >> 6] = n;
  __syncthreads();
  int t = 0;
#pragma unroll
  for (int w = 0; w < NT / 64; w++) t += r[w];
  return t;
}

// The K largest of the block's keys (NK per thread; nonzero keys are distinct, 0
// is an empty slot), written unordered to out[0 .. K-1] with K = min(want, number
// of nonzero keys): the K-th largest key is found bit by bit from the top (the
// largest T with at least K keys >= T), then the keys >= T are gathered.
template <int NT, int NK>
__device__ int block_top(const unsigned long long (&k)[NK], int want, unsigned long long *out, int *red, int *cnt) {
  int nz = 0;
#pragma unroll
  for (int i = 0; i < NK; i++) nz += k[i] != 0ull;
  const int K = min(want, block_count<NT>(nz, red, 0));
  unsigned long long T = 0;
  if (K > 0) {
    for (int b = 63; b >= 0; b--) {
      const unsigned long long c = T | (1ull << b);
      int n = 0;
#pragma unroll
      for (int i = 0; i < NK; i++) n += k[i] >= c;
      if (block_count<NT>(n, red, b & 1) >= K) T = c;
    }
  }
  if (threadIdx.x == 0) *cnt = 0;
  __syncthreads();
  if (K > 0) {
#pragma unroll
    for (int i = 0; i < NK; i++)
      if (k[i] >= T) out[atomicAdd(cnt, 1)] = k[i];
  }
  __syncthreads();
  return K;
}

// Per block: p = e / S over its slice and the slice's kTopC largest keys
// (unordered; empty slots 0).
__global__ __launch_bounds__(256) void k_smp_topk_block(const float *e, int V, const float *S,
                                                        unsigned long long *cand) {
  __shared__ unsigned long long top[kTopC];
  __shared__ int red[8], cnt;
  const float sum = S[0];
  const int j0 = blockIdx.x * kSlice + threadIdx.x;
  unsigned long long k[4];
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int j = j0 + 256 * r;
    k[r] = j < V ? prob_key(e[j] / sum, j) : 0ull;
  }
  const int K = block_top<256, 4>(k, kTopC, top, red, &cnt);
  if (threadIdx.x < kTopC) cand[(size_t)blockIdx.x * kTopC + threadIdx.x] = (int)threadIdx.x < K ? top[threadIdx.x] : 0ull;
}

// The kTopC largest of n candidate keys, as sorted (p, index) pairs: selected by
// block_top, then ordered by one wave's bitonic network (descending).
__global__ __launch_bounds__(kNT) void k_smp_topk_merge(const unsigned long long *cand, int n, float *ps, int *is) {
  constexpr int NK = kMergeCap / kNT;
  __shared__ unsigned long long top[kTopC];
  __shared__ int red[2 * (kNT / 64)], cnt;
  unsigned long long k[NK];
#pragma unroll
  for (int i = 0; i < NK; i++) {
    const int c = (int)threadIdx.x + kNT * i;
    k[i] = c < n ? cand[c] : 0ull;
  }
  const int K = block_top<kNT, NK>(k, kTopC, top, red, &cnt);
  if (threadIdx.x < 64) {
    const int lane = threadIdx.x;
    unsigned long long x = lane < K ? top[lane] : 0ull;
    for (int kk = 2; kk <= 64; kk <<= 1) {
      for (int j = kk >> 1; j > 0; j >>= 1) {
        const unsigned long long y = __shfl_xor(x, j, 64);
        const bool desc = (lane & kk) == 0, lower = (lane & j) == 0;
        x = (desc == lower) ? (x > y ? x : y) : (x < y ? x : y);
      }
    }
    if (lane < K) {
      ps[lane] = __uint_as_float((unsigned)(x >> 32));
      is[lane] = (int)(0xffffffffu - (unsigned)x);
    }
  }
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

// ---- stable LSD radix sort of (p, index) by p descending ----
// p >= 0, so the bits of p order like its values; a pass sorts by one byte of
// them, digit = 255 - byte (ascending digits = descending p), keeping the order
// of equal digits, so four passes from the low byte leave p descending with
// equal p in their input (index) order.  A block owns a tile of kRsTile items
// taken in kRsRounds rounds of 256 (item = tile start + 256 * round + thread),
// which is their input order.
constexpr int kRsNT = 256, kRsRounds = 16, kRsTile = kRsNT * kRsRounds;

int rs_blocks(int V) { return (V + kRsTile - 1) / kRsTile; }

__device__ __forceinline__ int rs_digit(float p, int shift) {
  return 255 - (int)((__float_as_uint(p) >> shift) & 255u);
}

// counts[d * nbs + b]: items of tile b with digit d
__global__ __launch_bounds__(kRsNT) void k_rs_hist(const float *keys, int V, int shift, int *counts, int nbs) {
  __shared__ int h[256];
  const int tid = threadIdx.x;
  h[tid] = 0;
  __syncthreads();
  const int j0 = blockIdx.x * kRsTile + tid;
  for (int r = 0; r < kRsRounds; r++) {
    const int j = j0 + kRsNT * r;
    if (j < V) atomicAdd(&h[rs_digit(keys[j], shift)], 1);
  }
  __syncthreads();
  counts[tid * nbs + blockIdx.x] = h[tid];
}

// In place: counts[d * nbs + b] becomes the output position of the first item of
// tile b with digit d (an exclusive scan in (digit, tile) order).  One block.
__global__ __launch_bounds__(kRsNT) void k_rs_scan(int *counts, int nbs) {
  __shared__ int tot[256];
  const int d = threadIdx.x;
  int t = 0;
  for (int b = 0; b < nbs; b++) t += counts[d * nbs + b];
  tot[d] = t;
  __syncthreads();
  int base = 0;                                   // exclusive prefix over the digits below d
  for (int e = 0; e < d; e++) base += tot[e];
  for (int b = 0; b < nbs; b++) {
    const int c = counts[d * nbs + b];
    counts[d * nbs + b] = base;
    base += c;
  }
}

// Each item to offs[digit, tile] + the number of earlier items of its tile with
// the same digit: in a round, the lanes of a wave with the same digit are found
// by ballots over the digit's bits, and the waves' counts per digit are added in
// wave order.
__global__ __launch_bounds__(kRsNT) void k_rs_scatter(const float *kin, const int *vin, float *kout, int *vout, int V,
                                                      int shift, const int *offs, int nbs) {
  constexpr int NW = kRsNT / 64;
  __shared__ int base[256];
  __shared__ int wc[NW][256];
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  base[tid] = offs[tid * nbs + blockIdx.x];
  const unsigned long long lt = (1ull << lane) - 1ull;
  const int j0 = blockIdx.x * kRsTile + tid;
  for (int r = 0; r < kRsRounds; r++) {
#pragma unroll
    for (int w = 0; w < NW; w++) wc[w][tid] = 0;
    __syncthreads();
    const int j = j0 + kRsNT * r;
    const bool ok = j < V;
    const float key = ok ? kin[j] : 0.0f;
    const int val = ok ? vin[j] : 0;
    const int d = ok ? rs_digit(key, shift) : 256;    // 256: no item (9 bits tell it apart)
    unsigned long long peers = __ballot(1);
#pragma unroll
    for (int bit = 0; bit < 9; bit++) {
      const bool set = (d >> bit) & 1;
      const unsigned long long m = __ballot(set);
      peers &= set ? m : ~m;
    }
    const int rank = __popcll(peers & lt);
    if (ok && rank == 0) wc[wave][d] = __popcll(peers);
    __syncthreads();
    {                                             // thread tid = digit tid: offsets of the waves
      int acc = base[tid];
#pragma unroll
      for (int w = 0; w < NW; w++) {
        const int c = wc[w][tid];
        wc[w][tid] = acc;
        acc += c;
      }
      base[tid] = acc;
    }
    __syncthreads();
    if (ok) {
      const int pos = wc[wave][d] + rank;
      kout[pos] = key;
      vout[pos] = val;
    }
    __syncthreads();
  }
}

int nblocks(int V) { return (V + kSlice - 1) / kSlice; }

// Scratch layout: e, p, sorted p, indices, sorted indices (V each), block maxima,
// the sum, top-k candidates, then the radix sort's digit counts per tile.
struct Layout {
  float *e, *p, *ps, *bm, *S;
  int *idx, *is, *counts;
  unsigned long long *cand;
  size_t total;
};

Layout layout(void *base, int V) {
  Layout L{};
  uint8_t *b = static_cast<uint8_t *>(base);
  const size_t slot = al256((size_t)V * 4), nb = (size_t)nblocks(V);
  size_t o = 0;
  L.e = reinterpret_cast<float *>(b + o); o += slot;
  L.p = reinterpret_cast<float *>(b + o); o += slot;
  L.ps = reinterpret_cast<float *>(b + o); o += slot;
  L.idx = reinterpret_cast<int *>(b + o); o += slot;
  L.is = reinterpret_cast<int *>(b + o); o += slot;
  L.bm = reinterpret_cast<float *>(b + o); o += al256(nb * 4);
  L.S = reinterpret_cast<float *>(b + o); o += 256;
  L.cand = reinterpret_cast<unsigned long long *>(b + o); o += al256(nb * kTopC * 8);
  L.counts = reinterpret_cast<int *>(b + o); o += al256((size_t)256 * rs_blocks(V) * 4);
  L.total = o;
  return L;
}

}  // namespace

// Scratch of qhip_sample for rows of V logits.
extern "C" size_t qhip_sample_scratch(int V) {
  if (V <= 0) return 0;
  return layout(nullptr, V).total;
}

// Whether qhip_sample takes the top-k path (top_k <= 64) for these arguments
// rather than the full radix sort.
extern "C" int qhip_sample_topk_path(int V, int top_k) {
  return top_k >= 1 && top_k <= kTopC && V > 0 && (size_t)nblocks(V) * kTopC <= (size_t)kMergeCap;
}

extern "C" int qhip_sample(const float *logits, int V, float temperature, int top_k, float top_p, void *scratch,
                           size_t scratch_bytes, unsigned long long *rng, int *tok, int *d_in, const int *d_state,
                           int *d_out, int max_seq) {
  if (V <= 0 || !(temperature > 0.0f)) return qh::fail_msg("sample: needs V > 0 and temperature > 0");
  if (scratch_bytes < qhip_sample_scratch(V)) return qh::fail_msg("sample: scratch too small");
  const Layout L = layout(scratch, V);
  const int nb = nblocks(V);
  QH_LAUNCH(QK_OTHER, k_smp_bmax, dim3(nb), dim3(256), 0, logits, V, L.bm);
  QH_LAUNCH(QK_OTHER, k_smp_exp, dim3(nb), dim3(256), 0, logits, V, temperature, L.bm, nb, L.e);
  QH_LAUNCH(QK_OTHER, k_smp_sum, dim3(1), dim3(kSumNT), 0, L.e, V, L.S);
  if (qhip_sample_topk_path(V, top_k)) {
    // the top_k <= kTopC largest of all V are among the kTopC largest of each block
    QH_LAUNCH(QK_OTHER, k_smp_topk_block, dim3(nb), dim3(256), 0, L.e, V, L.S, L.cand);
    QH_LAUNCH(QK_OTHER, k_smp_topk_merge, dim3(1), dim3(kNT), 0, L.cand, nb * kTopC, L.ps, L.is);
  } else {
    // p and the indices start in (ps, is); four passes, ping-ponging through
    // (p, idx), leave them sorted in (ps, is)
    QH_LAUNCH(QK_OTHER, k_smp_div, dim3(nb), dim3(256), 0, L.e, V, L.S, L.ps);
    QH_LAUNCH(QK_OTHER, k_smp_iota, dim3((V + 255) / 256), dim3(256), 0, L.is, V);
    const int nbs = rs_blocks(V);
    for (int pass = 0; pass < 4; pass++) {
      const int shift = 8 * pass;
      const float *ki = pass & 1 ? L.p : L.ps;
      const int *vi = pass & 1 ? L.idx : L.is;
      float *ko = pass & 1 ? L.ps : L.p;
      int *vo = pass & 1 ? L.is : L.idx;
      QH_LAUNCH(QK_OTHER, k_rs_hist, dim3(nbs), dim3(kRsNT), 0, ki, V, shift, L.counts, nbs);
      QH_LAUNCH(QK_OTHER, k_rs_scan, dim3(1), dim3(kRsNT), 0, L.counts, nbs);
      QH_LAUNCH(QK_OTHER, k_rs_scatter, dim3(nbs), dim3(kRsNT), 0, ki, vi, ko, vo, V, shift, L.counts, nbs);
    }
  }
  QH_LAUNCH(QK_OTHER, k_smp_pick, dim3(1), dim3(64), 0, L.ps, L.is, V, top_k, top_p, rng, tok, d_in, d_state,
            d_out, max_seq);
  return 0;
}

extern "C" int qhip_argmax_row(const float *logits, int V, int *tok, int *d_in, const int *d_state, int *d_out,
                               int max_seq) {
  if (V <= 0) return qh::fail_msg("argmax: needs V > 0");
  QH_LAUNCH(QK_OTHER, k_smp_argmax, dim3(1), dim3(kNT), 0, logits, V, tok, d_in, d_state, d_out, max_seq);
  return 0;
}
