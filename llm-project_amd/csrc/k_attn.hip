// k_attn.hip - decode attention over the device KV cache (llama.c:554-576).
//
// Exactness: the reference forms, per query head h,
//   dot_j = sum_d q_d * K_jd      (d = 0..hd-1, in order)
//   s_j   = dot_j * scale,  m = max_j s_j,  e_j = expf(s_j - m)
//   S     = sum_j e_j             (j = 0..T-1, in order)
//   w_j   = e_j * (1 / S),  o_d = sum_j w_j * V_jd   (j in order, from 0)
// Every one of those sums is formed here in the same order, by one lane each;
// the parallelism is across positions (scores), across (head, d) chains, and
// between the lanes that form the products w_j * V_jd and the lanes that add them.
//
// Kernel 1 (k_attn_scores): grid (H, ceil(max_seq/256)); one thread per (head,
//   position) computes dot_j and s_j; each block writes its maximum.
// Kernel 2 (k_attn_pv): grid (H, ceil(hd/64)), 512 threads.  Softmax weights for
//   the head in LDS, then wave 0 owns 64 output chains o_d while waves 1-7 stream
//   V tiles of 128 positions, form the products w_j * V_jd into a double-buffered
//   LDS tile and keep the V values of the next four tiles in flight in registers.
#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qdev_seqsum.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

constexpr int kScoreBlock = 256;
constexpr int kTile = 128;      // positions per PV tile
constexpr int kChains = 64;     // output dims per PV block (wave 0's lanes)
constexpr int kPvThreads = 512;
constexpr int kProducers = kPvThreads - 64;
constexpr int kSlots = (kTile * kChains + kProducers - 1) / kProducers;   // 19

// Barrier for LDS hand-offs only: waits for this wave's LDS operations
// (lgkmcnt(0)) and then for the other waves, but leaves global loads in flight.
// __syncthreads() would also drain every outstanding global load (its fence
// covers global memory), which would cancel the producers' V prefetch.
__device__ __forceinline__ void lds_barrier() {
  __builtin_amdgcn_s_waitcnt(0xC07F);        // vmcnt(63) expcnt(7) lgkmcnt(0)
  __builtin_amdgcn_s_barrier();
}

__device__ __forceinline__ float block_max(float m, float *red) {
  m = qd::wave_max_f32(m);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  __syncthreads();
  if (lane == 0) red[w] = m;
  __syncthreads();
  float r = red[0];
  for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = fmaxf(r, red[i]);
  return r;
}

template <bool VEC4>
__global__ __launch_bounds__(kScoreBlock) void k_attn_scores(const float *q, const float *kc, const int *d_pos, int H,
                                                              int KVH, int hd, int max_seq, float scale,
                                                              float *scores, float *bmax, int nch) {
  extern __shared__ float qs[];
  __shared__ float red[kScoreBlock / 64];
  const int h = blockIdx.x, c = blockIdx.y;
  const int T = *d_pos + 1;
  if (c * kScoreBlock >= T) return;                      // uniform for the block
  const int kvh = h / (H / KVH);
  for (int d = threadIdx.x; d < hd; d += kScoreBlock) qs[d] = q[(size_t)h * hd + d];
  __syncthreads();
  const int j = c * kScoreBlock + threadIdx.x;
  float s = -INFINITY;
  if (j < T) {
    const float *kr = kc + ((size_t)kvh * max_seq + j) * hd;
    float dot = 0.0f;
    if (VEC4) {
      const float4 *k4 = reinterpret_cast<const float4 *>(kr);
      const float4 *q4 = reinterpret_cast<const float4 *>(qs);
      for (int i = 0; i < (hd >> 2); i++) {
        const float4 kv = k4[i], qv = q4[i];
        dot += qv.x * kv.x;
        dot += qv.y * kv.y;
        dot += qv.z * kv.z;
        dot += qv.w * kv.w;
      }
    } else {
      for (int d = 0; d < hd; d++) dot += qs[d] * kr[d];
    }
    s = dot * scale;
    scores[(size_t)h * max_seq + j] = s;
  }
  s = block_max(s, red);
  if (threadIdx.x == 0) bmax[(size_t)h * nch + c] = s;
}

// Producer slot k of thread pid covers tile row jj = pid / 64 + kRowsPass * k and
// column dd = pid % 64 (the producers cover kRowsPass rows of 64 per pass).
constexpr int kRowsPass = kProducers / kChains;
static_assert(kProducers == kRowsPass * kChains, "producers must fill whole tile rows");

// Products for tile t: P[jj][dd] = w_j * V_j,d0+dd from prefetched V values.
// Branch-free (a select per slot) so the compiler can keep counting the V loads
// that are still in flight instead of waiting for all of them.
__device__ __forceinline__ void pv_produce(float *P, const float *W, const float (&v)[kSlots], int t, int T, int pid) {
  const int jj0 = pid >> 6, dd = pid & 63;
#pragma unroll
  for (int k = 0; k < kSlots; k++) {
    const int jj = jj0 + kRowsPass * k;
    if (kRowsPass * k + kRowsPass - 1 < kTile || jj < kTile) {   // compile-time true except the last slot
      const int j = t * kTile + jj;
      const float w = W[min(j, T - 1)];
      const float p = w * v[k];
      P[min(jj, kTile - 1) * kChains + dd] = (j < T && jj < kTile) ? p : 0.0f;
    }
  }
}

// V values of tile t for this thread's slots; out-of-range slots read an
// in-bounds element and are zeroed by the producer's select.
__device__ __forceinline__ void pv_load(float (&v)[kSlots], const float *Vh, int t, int T, int hd, int d0, int pid) {
  const int jj0 = pid >> 6;
  const int col = min(d0 + (pid & 63), hd - 1);
#pragma unroll
  for (int k = 0; k < kSlots; k++) {
    const int j = min(t * kTile + jj0 + kRowsPass * k, T - 1);
    v[k] = __builtin_nontemporal_load(&Vh[(size_t)j * hd + col]);
  }
}

__global__ __launch_bounds__(kPvThreads) void k_attn_pv(const float *scores, const float *bmax, const float *vc,
                                                        const int *d_pos, int H, int KVH, int hd, int max_seq,
                                                        int nch, float *o, float *obm) {
  extern __shared__ float lds[];
  __shared__ float red[kPvThreads / 64];
  __shared__ float s_inv;
  __shared__ qd::SeqSumScratch seq;
  const int h = blockIdx.x, d0 = blockIdx.y * kChains;
  const int T = *d_pos + 1;
  const int kvh = h / (H / KVH);
  const int wcap = (max_seq + 3) & ~3;
  float *W = lds;
  float *P = lds + wcap;                                 // 2 x kTile x kChains
  const int tid = threadIdx.x;

  // softmax weights of head h (llama.c:557-572)
  const int nc = (T + kScoreBlock - 1) / kScoreBlock;
  float m = -INFINITY;
  for (int c = tid; c < nc; c += kPvThreads) m = fmaxf(m, bmax[(size_t)h * nch + c]);
  m = block_max(m, red);
  const float *sh = scores + (size_t)h * max_seq;
  for (int j = tid; j < T; j += kPvThreads) W[j] = qd::expf_glibc(sh[j] - m);
  __syncthreads();
  {
    const float sum = qd::seq_sum_nonneg<kPvThreads>(W, T, seq);   // llama.c:567, exactly
    if (tid == 0) s_inv = 1.0f / sum;
  }
  __syncthreads();
  const float inv = s_inv;
  for (int j = tid; j < T; j += kPvThreads) W[j] = W[j] * inv;
  __syncthreads();

  // o_d = sum_j w_j * V_jd, j in order (llama.c:570-575)
  const int ntile = (T + kTile - 1) / kTile;
  const float *Vh = vc + (size_t)kvh * max_seq * hd;
  if (tid < 64) {
    const int d = d0 + tid;
    float acc = 0.0f;
    for (int t = 0; t < ntile; t++) {
      lds_barrier();
      const float *Pt = P + (t & 1) * kTile * kChains + tid;
      const int nj = min(kTile, T - t * kTile);
      if (nj == kTile) {
        // straight-line over the whole tile: the reads run ahead of the add chain
#pragma unroll
        for (int jj = 0; jj < kTile; jj++) acc += Pt[jj * kChains];
      } else {
        for (int jj = 0; jj < nj; jj++) acc += Pt[jj * kChains];
      }
    }
    if (d < hd) o[(size_t)h * hd + d] = acc;
    if (obm) {                 // max |o| of this block, for the activation quantizer
      const float mo = qd::wave_max_f32(d < hd ? fabsf(acc) : 0.0f);
      if (tid == 0) obm[(size_t)h * gridDim.y + blockIdx.y] = mo;
    }
  } else {
    // Producers: tile k is formed from register set k % 4 into LDS buffer k % 2;
    // its V values are requested four tiles ahead of use.
    const int pid = tid - 64;
    float r0[kSlots], r1[kSlots], r2[kSlots], r3[kSlots];
    float *B0 = P, *B1 = P + kTile * kChains;
    pv_load(r0, Vh, 0, T, hd, d0, pid);
    if (ntile > 1) pv_load(r1, Vh, 1, T, hd, d0, pid);
    if (ntile > 2) pv_load(r2, Vh, 2, T, hd, d0, pid);
    if (ntile > 3) pv_load(r3, Vh, 3, T, hd, d0, pid);
    pv_produce(B0, W, r0, 0, T, pid);
    if (ntile > 4) pv_load(r0, Vh, 4, T, hd, d0, pid);
    for (int t = 0; t < ntile; t += 4) {
      lds_barrier();                                   // consumer takes tile t
      if (t + 1 < ntile) {
        pv_produce(B1, W, r1, t + 1, T, pid);
        if (t + 5 < ntile) pv_load(r1, Vh, t + 5, T, hd, d0, pid);
        lds_barrier();                                 // consumer takes tile t+1
        if (t + 2 < ntile) {
          pv_produce(B0, W, r2, t + 2, T, pid);
          if (t + 6 < ntile) pv_load(r2, Vh, t + 6, T, hd, d0, pid);
          lds_barrier();                               // tile t+2
          if (t + 3 < ntile) {
            pv_produce(B1, W, r3, t + 3, T, pid);
            if (t + 7 < ntile) pv_load(r3, Vh, t + 7, T, hd, d0, pid);
            lds_barrier();                             // tile t+3
            if (t + 4 < ntile) {
              pv_produce(B0, W, r0, t + 4, T, pid);
              if (t + 8 < ntile) pv_load(r0, Vh, t + 8, T, hd, d0, pid);
            }
          }
        }
      }
    }
  }
}

size_t g_pv_attr_bytes = 0;   // dynamic LDS the PV kernel is currently allowed

}  // namespace

extern "C" int qhip_attention(const float *q, const float *kc, const float *vc, const int *d_pos, int n_heads,
                              int n_kv, int hd, int max_seq, float scale, float *scores, float *o, float *obm) {
  const int nch = (max_seq + kScoreBlock - 1) / kScoreBlock;
  float *bmax = scores + (size_t)n_heads * max_seq;
  const size_t pv_lds = ((size_t)((max_seq + 3) & ~3) + 2 * kTile * kChains) * 4;
  if (pv_lds + sizeof(qd::SeqSumScratch) + 1024 > 160 * 1024)
    return qh::fail_msg("attention: max_seq too large for the LDS-resident weights");
  if (pv_lds > 64 * 1024 && pv_lds > g_pv_attr_bytes) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_pv),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)pv_lds);
    if (e != hipSuccess) return qh::fail("hipFuncSetAttribute(k_attn_pv)", e);
    g_pv_attr_bytes = pv_lds;
  }
  if ((hd & 3) == 0) {
    QH_LAUNCH(QK_ATTN, k_attn_scores<true>, dim3(n_heads, nch), dim3(kScoreBlock), (size_t)hd * 4, q, kc, d_pos,
              n_heads, n_kv, hd, max_seq, scale, scores, bmax, nch);
  } else {
    QH_LAUNCH(QK_ATTN, k_attn_scores<false>, dim3(n_heads, nch), dim3(kScoreBlock), (size_t)hd * 4, q, kc, d_pos,
              n_heads, n_kv, hd, max_seq, scale, scores, bmax, nch);
  }
  QH_LAUNCH(QK_ATTN, k_attn_pv, dim3(n_heads, (hd + kChains - 1) / kChains), dim3(kPvThreads), pv_lds, scores, bmax,
            vc, d_pos, n_heads, n_kv, hd, max_seq, nch, o, obm);
  return 0;
}

// Number of per-block maxima qhip_attention writes to obm.
extern "C" int qhip_attention_nbm(int n_heads, int hd) { return n_heads * ((hd + kChains - 1) / kChains); }

// Size (floats) of the scores scratch qhip_attention needs.
extern "C" size_t qhip_attention_scratch(int n_heads, int max_seq) {
  return (size_t)n_heads * max_seq + (size_t)n_heads * ((max_seq + kScoreBlock - 1) / kScoreBlock);
}
