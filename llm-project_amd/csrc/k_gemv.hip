// k_gemv.hip - the decode W8A8 GEMV (quant.c:60-85 with one activation row).
//
// Weights are output-channel major ([N][kpad] int8, K contiguous).  One wave owns
// R consecutive output channels; its 64 lanes split K in 16-byte chunks, so every
// load is a coalesced 1 KiB wave access.  The quantized activation row (kpad
// bytes) is loaded once per wave into registers and reused for all R channels.
// Products accumulate exactly in int32 (v_dot4_i32_i8; |acc| <= 127^2 * K < 2^31)
// and are summed across the wave, so the result is independent of the split.
// The next channel's weights are in flight while the current one is reduced.
//
// Epilogues (the reference's order of rounding, quant.c:81-82):
//   PLAIN  out[j] = (as * ws[j]) * (float)acc (+ bias[j], llama.c:546-548)
//   RESID  out[j] = out[j] + (as * ws[j]) * (float)acc       (llama.c:578, 589)
//   SWIGLU rows j and N+j are gate and up; out[j] = (g * (1 / (1 + expf(-g)))) * u
//          (llama.c:583-587) and each block records max |out| for the quantizer.
#include <hip/hip_runtime.h>

#include <type_traits>

#include "qdev_math.h"
#include "qdev_norm.h"
#include "qhip.h"
#include "qhip_internal.h"
#include "qdev_tl.h"

QTL_DEFINE(gemv)

namespace {

enum { MODE_PLAIN = 0, MODE_RESID = 1, MODE_SWIGLU = 2, MODE_HEAD = 3 };

typedef int v4i __attribute__((ext_vector_type(4)));
typedef const __attribute__((address_space(4))) float cfloat_t;   // loads through the scalar cache

template <int KCH>
__device__ __forceinline__ void load_row(v4i (&w)[KCH], const int8_t *row, int lane) {
  const v4i *r = reinterpret_cast<const v4i *>(row);
#pragma unroll
  for (int i = 0; i < KCH; i++) w[i] = __builtin_nontemporal_load(&r[lane + 64 * i]);
}

template <int KCH>
__device__ __forceinline__ int dot_row(const v4i (&w)[KCH], const v4i (&a)[KCH]) {
  int t = 0;
#pragma unroll
  for (int i = 0; i < KCH; i++) {
    t = __builtin_amdgcn_sdot4(a[i].x, w[i].x, t, false);
    t = __builtin_amdgcn_sdot4(a[i].y, w[i].y, t, false);
    t = __builtin_amdgcn_sdot4(a[i].z, w[i].z, t, false);
    t = __builtin_amdgcn_sdot4(a[i].w, w[i].w, t, false);
  }
  return t;
}

// PRO = 1 inputs of this thread (one of NTP): the maximum of its share of the
// block maxima vbm (nvbm values) and its NQ chunks of 16 activation values
// (chunk c = threadIdx.x + NTP * i holds v[16c .. 16c+15], 0 past n).
template <int KCH, int NQ, int NTP = 256>
__device__ __forceinline__ void pro1_load(const float *v, int n, const float *vbm, int nvbm, float (&qx)[NQ][16],
                                          float &qm) {
  float mx = 0.0f;
  for (int i = threadIdx.x; i < nvbm; i += NTP) mx = fmaxf(mx, vbm[i]);
  qm = mx;
#pragma unroll
  for (int ci = 0; ci < NQ; ci++) {
    const int k0 = 16 * (threadIdx.x + NTP * ci);
    if (k0 + 16 <= n) {
#pragma unroll
      for (int e = 0; e < 16; e += 4) {
        const float4 t = *reinterpret_cast<const float4 *>(v + k0 + e);
        qx[ci][e] = t.x; qx[ci][e + 1] = t.y; qx[ci][e + 2] = t.z; qx[ci][e + 3] = t.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 16; e++) qx[ci][e] = k0 + e < n ? v[k0 + e] : 0.0f;
    }
  }
}

// KCH = kpad / 1024 chunks of 16 bytes per lane (kpad a multiple of 1024).
// PRO = 1: the activation arrives unquantized (v, n values, with per-block
// maxima of |v| in vbm); every block quantizes it itself (quant.c:66-78, the
// operations of k_quant_blocks) into LDS while its first weights are in flight.
// PRO = 2: the activation is the residual stream v (n values) before its
// rmsnorm (gain vbm, epsilon eps); every block normalizes and quantizes it
// itself (the operations of k_rmsnorm_quant) while its first weights are in
// flight.  PRO = 3: the same with the fast mode's tree-ordered sum of squares.
// The prologue's inputs are requested before the weights: a wave's loads
// return in the order they were issued, so waiting for inputs requested after
// the weights would wait for the weights too, and the prologue would follow the
// weight stream instead of overlapping it.
// NS: weight rows (pairs, for SWIGLU) held in registers; rows r+1 .. r+NS-1 are
// in flight while row r is reduced.
template <int MODE, int KCH, int R, int PRO, int NS>
__global__ __launch_bounds__(256) void k_gemv_dec(const int8_t *qa, const float *as_p, const int8_t *W,
                                                  const float *ws, int N, int kpad, float *out, const float *bias,
                                                  float *bm, int *bi, const float *v, int n, const float *vbm,
                                                  int nvbm, float eps) {
  __shared__ float red[8];
  __shared__ int redi[4];
  __shared__ __attribute__((aligned(16))) int8_t qsh[PRO ? KCH * 1024 : 16];
  __shared__ typename std::conditional<PRO == 2, qd::SeqScratch, int>::type seq;
  float best = -INFINITY;
  int besti = 0x7fffffff;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  if (wave == 0) QTL_MARK(3 + MODE, 0);
  QTL_ID(3 + MODE);
  const int j0 = (blockIdx.x * 4 + wave) * R;
  float hmax = 0.0f;
  // the prologue's inputs, then the weights
  constexpr int CM = PRO >= 2 ? 4 * KCH : 1;         // 256 threads x CM values = kpad
  float y[CM], gm[CM];
  if constexpr (PRO >= 2) qd::rmsnorm_load<CM>(v, n, vbm, y, gm);
  constexpr int NQ = PRO == 1 ? (KCH * 64 + 255) / 256 : 1;   // 16-value chunks per thread
  float qx[NQ][16], qm = 0.0f;
  if constexpr (PRO == 1) pro1_load<KCH, NQ>(v, n, vbm, nvbm, qx, qm);
  __builtin_amdgcn_sched_barrier(0);
  v4i w[NS][KCH], u[NS][KCH];
#pragma unroll
  for (int r = 0; r < NS; r++) {                     // in flight during the prologue
    if (r < R && j0 + r < N) {
      load_row(w[r], W + (size_t)(j0 + r) * kpad, lane);
      if (MODE == MODE_SWIGLU) load_row(u[r], W + (size_t)(N + j0 + r) * kpad, lane);
    }
  }
  __builtin_amdgcn_sched_barrier(0);
  v4i a[KCH];
  float as;
  if constexpr (PRO == 2 || PRO == 3) {
    if constexpr (PRO == 2) as = qd::rmsnorm_apply<256, CM>(v, n, eps, y, gm, red, seq);
    else as = qd::rmsnorm_apply_fast<256, CM>(n, eps, y, gm, red);
    const float inv = 1.0f / as;
#pragma unroll
    for (int c = 0; c < CM; c += 4)
      *reinterpret_cast<uint32_t *>(qsh + threadIdx.x * CM + c) = qd::quant_word(y, c, inv);
    qd::lds_sync();                                  // the first weights stay in flight
#pragma unroll
    for (int i = 0; i < KCH; i++) a[i] = *reinterpret_cast<const v4i *>(qsh + 16 * (lane + 64 * i));
  } else if (PRO == 1) {
    float mx = qd::wave_max_f32(qm);
    if (lane == 0) red[wave] = mx;
    qd::lds_sync();
    mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    as = (mx > 0.0f) ? mx / 127.0f : 1.0f;
    const float inv = 1.0f / as;
#pragma unroll
    for (int ci = 0; ci < NQ; ci++) {                // 16 values per chunk
      const int c = threadIdx.x + 256 * ci;
      if (c >= KCH * 64) break;
      const int k0 = 16 * c;
      const float *x = qx[ci];
      v4i pk;                                          // values past n were loaded as 0 and give 0
#pragma unroll
      for (int wd = 0; wd < 4; wd++)
        pk[wd] = (int)qd::quant_i8x4(x[4 * wd], x[4 * wd + 1], x[4 * wd + 2], x[4 * wd + 3], inv);
      *reinterpret_cast<v4i *>(qsh + k0) = pk;
    }
    qd::lds_sync();
#pragma unroll
    for (int i = 0; i < KCH; i++) a[i] = *reinterpret_cast<const v4i *>(qsh + 16 * (lane + 64 * i));
  } else {
    const v4i *q4 = reinterpret_cast<const v4i *>(qa);
#pragma unroll
    for (int i = 0; i < KCH; i++) a[i] = q4[lane + 64 * i];
    as = *as_p;
  }
#pragma unroll
  for (int r = 0; r < R; r++) {
    const int j = j0 + r;
    if (j >= N) break;
    const int accw = dot_row(w[r % NS], a);
    int accu = 0;
    if (MODE == MODE_SWIGLU) accu = dot_row(u[r % NS], a);
    if (r + NS < R && j + NS < N) {                  // the slot takes row r + NS
      load_row(w[r % NS], W + (size_t)(j + NS) * kpad, lane);
      if (MODE == MODE_SWIGLU) load_row(u[r % NS], W + (size_t)(N + j + NS) * kpad, lane);
    }
    const int sw = qd::wave_sum_i32(accw);
    if (MODE == MODE_SWIGLU) {
      const int su = qd::wave_sum_i32(accu);
      const float g = (as * ws[j]) * (float)sw;
      const float up = (as * ws[N + j]) * (float)su;
      const float s = 1.0f / (1.0f + qd::expf_glibc(-g));
      const float h = (g * s) * up;
      hmax = fmaxf(hmax, fabsf(h));
      if (lane == 0) out[j] = h;
    } else {
      const float c = (as * ws[j]) * (float)sw;
      if (MODE == MODE_HEAD && (besti == 0x7fffffff || c > best)) { best = c; besti = j; }
      if (lane == 0) {
        if (MODE == MODE_RESID) out[j] = out[j] + c;
        else out[j] = bias ? c + bias[j] : c;
      }
    }
  }
  if (MODE == MODE_SWIGLU) {
    if (lane == 0) red[wave] = hmax;
    __syncthreads();
    if (threadIdx.x == 0) bm[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
  if (MODE == MODE_HEAD) {         // first index of this block's maximum (sampler.c:8-21)
    if (lane == 0) { red[wave] = best; redi[wave] = besti; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float b = red[0];
      int i0 = redi[0];
      for (int w = 1; w < 4; w++)
        if (redi[w] != 0x7fffffff && (i0 == 0x7fffffff || red[w] > b || (red[w] == b && redi[w] < i0))) {
          b = red[w];
          i0 = redi[w];
        }
      bm[blockIdx.x] = b;
      bi[blockIdx.x] = i0;
    }
  }
  QTL_MAX(3 + MODE, 4);
}

// Warp-specialized decode GEMV for the GEMVs with a prologue (PRO 1, 2, 3; the
// operations of k_gemv_dec's prologues and epilogues, in the same order).  512
// threads: the first PW waves form the quantized activation and meet at an LDS
// counter (qd::GroupSync) instead of the block barrier; the RWV waves after them own
// the output rows, RW consecutive rows (row pairs for SWIGLU) each, request
// their first NS rows at kernel start and wait on an LDS flag for the
// activation.  A wave issues its
// instructions in order and stalls while the memory system holds all it can
// take, so in k_gemv_dec a wave reaches its prologue only once most of its
// weight loads are accepted, and every block barrier of the prologue waits for
// the slowest wave; here the prologue waves issue no weight loads and never
// wait for a row wave, and the weight stream runs under the whole prologue.
// The block's one s_barrier, before any wave works, publishes the zeroed
// counters.  grid: ceil(N / (RWV RW)) blocks; SWIGLU writes one max|h| per block.
#ifndef QLLAMA_GEMV_WS
#define QLLAMA_GEMV_WS 1
#endif
constexpr bool kUseWs = QLLAMA_GEMV_WS != 0;     // the prologue GEMVs run k_gemv_ws (else k_gemv_dec)

// Prologue waves, row waves and weight slots (rows, or row pairs, in registers
// per row wave) per mode, measured end to end at the 8B shape (same-box A/B of
// the decode bench): QKV 8 + 8 waves holding all 3 rows of a row wave; gate|up
// 4 + 8 waves with 3 row pairs in flight; Wo 4 + 8 waves with 2 rows.  Four
// waves per SIMD (1024 threads) made the prologue spill; one row wave per SIMD
// left the stream short of requests.
#ifndef QLLAMA_WS_PW_PLAIN
#define QLLAMA_WS_PW_PLAIN 8
#endif
#ifndef QLLAMA_WS_RWV_PLAIN
#define QLLAMA_WS_RWV_PLAIN 8
#endif
#ifndef QLLAMA_WS_SLOTS_PLAIN
#define QLLAMA_WS_SLOTS_PLAIN 12
#endif
#ifndef QLLAMA_WS_PW_SWIGLU
#define QLLAMA_WS_PW_SWIGLU 4
#endif
#ifndef QLLAMA_WS_RWV_SWIGLU
#define QLLAMA_WS_RWV_SWIGLU 8
#endif
#ifndef QLLAMA_WS_SLOTS_SWIGLU
#define QLLAMA_WS_SLOTS_SWIGLU 12
#endif
#ifndef QLLAMA_WS_PW_RESID
#define QLLAMA_WS_PW_RESID 4
#endif
#ifndef QLLAMA_WS_RWV_RESID
#define QLLAMA_WS_RWV_RESID 8
#endif
#ifndef QLLAMA_WS_SLOTS_RESID
#define QLLAMA_WS_SLOTS_RESID 8
#endif
#ifndef QLLAMA_WS_RWV_LONG
#define QLLAMA_WS_RWV_LONG 6
#endif
#ifndef QLLAMA_WS_PW_LONG
#define QLLAMA_WS_PW_LONG 2
#endif
constexpr int ws_pro_waves(int mode, int kch) {
  return mode == MODE_PLAIN ? QLLAMA_WS_PW_PLAIN
         : mode == MODE_SWIGLU ? QLLAMA_WS_PW_SWIGLU
         : kch > 8 ? QLLAMA_WS_PW_LONG : QLLAMA_WS_PW_RESID;
}
constexpr int ws_row_waves(int mode, int kch) {
  // long rows (the down projection's 14336 bytes): 2 prologue and 6 row waves
  // holding two rows each (eight waves: 256 registers a wave)
  return mode == MODE_PLAIN ? QLLAMA_WS_RWV_PLAIN
         : mode == MODE_SWIGLU ? QLLAMA_WS_RWV_SWIGLU
         : kch > 8 ? QLLAMA_WS_RWV_LONG : QLLAMA_WS_RWV_RESID;
}
// slots x KCH (16-byte chunks per lane and row) is the register budget
constexpr int ws_slots(int mode, int kch) {
  const int budget = mode == MODE_PLAIN ? QLLAMA_WS_SLOTS_PLAIN
                     : mode == MODE_SWIGLU ? QLLAMA_WS_SLOTS_SWIGLU : kch > 8 ? 2 * kch : QLLAMA_WS_SLOTS_RESID;
  return budget / kch > 0 ? budget / kch : 1;
}

template <int MODE, int KCH, int PRO, int NS, int PW, int RWV>
__global__ __launch_bounds__(64 * (PW + RWV)) void k_gemv_ws(const int8_t *W, const float *ws, int N, int kpad, int RW,
                                                 float *out, const float *bias, float *bm, const float *v, int n,
                                                 const float *vbm, int nvbm, float eps) {
  static_assert(PRO >= 1 && PRO <= 3, "prologue GEMVs only");
  constexpr int NTP = 64 * PW;                         // prologue threads
  constexpr int CM = PRO >= 2 ? 1024 * KCH / NTP : 4;  // NTP prologue threads x CM values = kpad
  static_assert(PRO == 1 || (CM % 4 == 0 && CM >= 4), "whole 16-byte words per prologue thread");
  __shared__ float red[2 * PW];
  __shared__ float hred[RWV];
  __shared__ unsigned gctr, ready, done, issued;
  __shared__ float as_sh;
  __shared__ __attribute__((aligned(16))) int8_t qsh[KCH * 1024];
  __shared__ typename std::conditional<PRO == 2, qd::SeqScratch, int>::type seq;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  // timeline id: the down projection (rows of 8 KiB and more) apart from Wo
  [[maybe_unused]] constexpr int TK = MODE == MODE_RESID && KCH >= 8 ? 5 : MODE;
  if (wave == 0) QTL_MARK(TK, 0);
  QTL_ID(TK);
  if (threadIdx.x == 0) { gctr = 0u; ready = 0u; done = 0u; issued = 0u; }
  __syncthreads();
  if (wave < PW) {
    // ---- the prologue waves ----
    unsigned epoch = 0u;
    const qd::GroupSync gs{&gctr, (unsigned)PW, &epoch};
    float as;
    if constexpr (PRO >= 2) {
      float y[CM], gm[CM];
      qd::rmsnorm_load<CM>(v, n, vbm, y, gm);
      if constexpr (PRO == 2) {                          // inputs requested: the row waves may start
        __builtin_amdgcn_sched_barrier(0);
        if (lane == 0) __hip_atomic_fetch_add(&issued, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      if constexpr (PRO == 2) as = qd::rmsnorm_apply<NTP, CM>(v, n, eps, y, gm, red, seq, gs);
      else as = qd::rmsnorm_apply_fast<NTP, CM>(n, eps, y, gm, red, gs);
      const float inv = 1.0f / as;
#pragma unroll
      for (int c = 0; c < CM; c += 4)
        *reinterpret_cast<uint32_t *>(qsh + threadIdx.x * CM + c) = qd::quant_word(y, c, inv);
    } else {
      constexpr int NQ = (KCH * 64 + NTP - 1) / NTP;   // 16-value chunks per thread
      float qx[NQ][16], qm = 0.0f;
      pro1_load<KCH, NQ, NTP>(v, n, vbm, nvbm, qx, qm);
      if constexpr (KCH > 8) {                           // inputs requested: the row waves may start
        __builtin_amdgcn_sched_barrier(0);
        if (lane == 0) __hip_atomic_fetch_add(&issued, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
      }
      float mx = qd::wave_max_f32(qm);
      if (lane == 0) red[wave] = mx;
      gs();
      mx = red[0];
#pragma unroll
      for (int i = 1; i < PW; i++) mx = fmaxf(mx, red[i]);
      as = (mx > 0.0f) ? mx / 127.0f : 1.0f;
      const float inv = 1.0f / as;
#pragma unroll
      for (int ci = 0; ci < NQ; ci++) {
        const int c = threadIdx.x + NTP * ci;
        if (c >= KCH * 64) break;
        const int k0 = 16 * c;
        v4i pk;                                        // values past n were loaded as 0 and give 0
#pragma unroll
        for (int wd = 0; wd < 4; wd++)
          pk[wd] = (int)qd::quant_i8x4(qx[ci][4 * wd], qx[ci][4 * wd + 1], qx[ci][4 * wd + 2], qx[ci][4 * wd + 3], inv);
        *reinterpret_cast<v4i *>(qsh + k0) = pk;
      }
    }
    if (threadIdx.x == 0) as_sh = as;
    if (wave == 0) QTL_MARK(TK, 1);
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");  // this wave's bytes (and as) have landed
    if (lane == 0) __hip_atomic_fetch_add(&ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    return;
  }
  // ---- the row waves ----
  const int rw = wave - PW;
  const int j0 = (blockIdx.x * RWV + rw) * RW;
#ifndef QLLAMA_WS_LONG_WAIT
#define QLLAMA_WS_LONG_WAIT 1
#endif
  if constexpr (PRO == 2 || (KCH > 8 && QLLAMA_WS_LONG_WAIT)) {
    // the prologue's inputs are requested before any weight, so that they do
    // not queue behind the weight stream: for the exact rmsnorm (its long
    // prologue is the kernel's critical path) and for long rows (57 KB of
    // activations per block); the short quantization prologues gain nothing
    while (__hip_atomic_load(&issued, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (unsigned)PW) {
    }
  }
  v4i w[NS][KCH], u[NS][KCH];
#pragma unroll
  for (int sl = 0; sl < NS; sl++) {
    if (sl < RW && j0 + sl < N) {
      load_row(w[sl], W + (size_t)(j0 + sl) * kpad, lane);
      if (MODE == MODE_SWIGLU) load_row(u[sl], W + (size_t)(N + j0 + sl) * kpad, lane);
    }
  }
  while (__hip_atomic_load(&ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (unsigned)PW) {
  }
  asm volatile("" ::: "memory");
  if (rw == 0) QTL_MARK(TK, 2);
  // the activation in registers, or (long rows) read from LDS at each row
  constexpr bool A_LDS = KCH > 8;
  v4i a[A_LDS ? 1 : KCH];
  if constexpr (!A_LDS) {
#pragma unroll
    for (int i = 0; i < KCH; i++) a[i] = *reinterpret_cast<const v4i *>(qsh + 16 * (lane + 64 * i));
  }
  auto dot = [&](const v4i (&wr)[KCH]) {
    if constexpr (A_LDS) {
      int t = 0;
#pragma unroll
      for (int i = 0; i < KCH; i++) {
        const v4i al = *reinterpret_cast<const v4i *>(qsh + 16 * (lane + 64 * i));
        t = __builtin_amdgcn_sdot4(al.x, wr[i].x, t, false);
        t = __builtin_amdgcn_sdot4(al.y, wr[i].y, t, false);
        t = __builtin_amdgcn_sdot4(al.z, wr[i].z, t, false);
        t = __builtin_amdgcn_sdot4(al.w, wr[i].w, t, false);
      }
      return t;
    } else {
      return dot_row(wr, reinterpret_cast<const v4i (&)[KCH]>(a));
    }
  };
  const float as = as_sh;
  float hmax = 0.0f;
  for (int r0 = 0; r0 < RW; r0 += NS) {
#pragma unroll
    for (int sl = 0; sl < NS; sl++) {
      const int r = r0 + sl, j = j0 + r;
      if (r < RW && j < N) {
        const int accw = dot(w[sl]);
        int accu = 0;
        if (MODE == MODE_SWIGLU) accu = dot(u[sl]);
        if (r + NS < RW && j + NS < N) {             // the slot takes row r + NS
          load_row(w[sl], W + (size_t)(j + NS) * kpad, lane);
          if (MODE == MODE_SWIGLU) load_row(u[sl], W + (size_t)(N + j + NS) * kpad, lane);
        }
        const int sw = qd::wave_sum_i32(accw);
        if (MODE == MODE_SWIGLU) {
          const int su = qd::wave_sum_i32(accu);
          const float g = (as * ws[j]) * (float)sw;
          const float up = (as * ws[N + j]) * (float)su;
          const float sg = 1.0f / (1.0f + qd::expf_glibc(-g));
          const float h = (g * sg) * up;
          hmax = fmaxf(hmax, fabsf(h));
          if (lane == 0) out[j] = h;
        } else {
          const float c = (as * ws[j]) * (float)sw;
          if (lane == 0) {
            if (MODE == MODE_RESID) out[j] = out[j] + c;
            else out[j] = bias ? c + bias[j] : c;
          }
        }
        if (rw == 0 && r == 0) QTL_MARK(TK, 3);
      }
    }
  }
  QTL_MAX(TK, 4);
  if (MODE == MODE_SWIGLU) {       // the block's max |h|: the last row wave to finish writes it
    if (lane == 0) hred[rw] = hmax;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    unsigned old = 0u;
    if (lane == 0) old = __hip_atomic_fetch_add(&done, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    old = (unsigned)__builtin_amdgcn_readfirstlane((int)old);
    if (old == RWV - 1u && lane == 0) {
      float mb = hred[0];
#pragma unroll
      for (int i = 1; i < RWV; i++) mb = fmaxf(mb, hred[i]);
      bm[blockIdx.x] = mb;
    }
  }
}

// Generic K: lanes loop over the 16-byte chunks.
template <int MODE>
__global__ __launch_bounds__(256) void k_gemv_dec_any(const int8_t *qa, const float *as_p, const int8_t *W,
                                                      const float *ws, int N, int kpad, float *out,
                                                      const float *bias, float *bm, int *bi) {
  __shared__ float red[4];
  __shared__ int redi[4];
  float best = -INFINITY;
  int besti = 0x7fffffff;
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int j = blockIdx.x * 4 + wave;
  const int nchunk = kpad >> 4;
  float hmax = 0.0f;
  if (j < N) {
    const int4 *q4 = reinterpret_cast<const int4 *>(qa);
    const int4 *wr = reinterpret_cast<const int4 *>(W + (size_t)j * kpad);
    const int4 *ur = reinterpret_cast<const int4 *>(W + (size_t)(N + j) * kpad);
    int tw = 0, tu = 0;
    for (int c = lane; c < nchunk; c += 64) {
      const int4 av = q4[c], wv = wr[c];
      tw = __builtin_amdgcn_sdot4(av.x, wv.x, tw, false);
      tw = __builtin_amdgcn_sdot4(av.y, wv.y, tw, false);
      tw = __builtin_amdgcn_sdot4(av.z, wv.z, tw, false);
      tw = __builtin_amdgcn_sdot4(av.w, wv.w, tw, false);
      if (MODE == MODE_SWIGLU) {
        const int4 uv = ur[c];
        tu = __builtin_amdgcn_sdot4(av.x, uv.x, tu, false);
        tu = __builtin_amdgcn_sdot4(av.y, uv.y, tu, false);
        tu = __builtin_amdgcn_sdot4(av.z, uv.z, tu, false);
        tu = __builtin_amdgcn_sdot4(av.w, uv.w, tu, false);
      }
    }
    const float as = *as_p;
    const int sw = qd::wave_sum_i32(tw);
    if (MODE == MODE_SWIGLU) {
      const int su = qd::wave_sum_i32(tu);
      const float g = (as * ws[j]) * (float)sw;
      const float up = (as * ws[N + j]) * (float)su;
      const float s = 1.0f / (1.0f + qd::expf_glibc(-g));
      const float h = (g * s) * up;
      hmax = fabsf(h);
      if (lane == 0) out[j] = h;
    } else {
      const float c = (as * ws[j]) * (float)sw;
      if (MODE == MODE_HEAD) { best = c; besti = j; }
      if (lane == 0) {
        if (MODE == MODE_RESID) out[j] = out[j] + c;
        else out[j] = bias ? c + bias[j] : c;
      }
    }
  }
  if (MODE == MODE_SWIGLU) {
    if (lane == 0) red[wave] = hmax;
    __syncthreads();
    if (threadIdx.x == 0) bm[blockIdx.x] = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  }
  if (MODE == MODE_HEAD) {
    if (lane == 0) { red[wave] = best; redi[wave] = besti; }
    __syncthreads();
    if (threadIdx.x == 0) {
      float b = red[0];
      int i0 = redi[0];
      for (int w = 1; w < 4; w++)
        if (redi[w] != 0x7fffffff && (i0 == 0x7fffffff || red[w] > b || (red[w] == b && redi[w] < i0))) {
          b = red[w];
          i0 = redi[w];
        }
      bm[blockIdx.x] = b;
      bi[blockIdx.x] = i0;
    }
  }
}

// Reduce the per-block (max, first index) candidates of the head GEMV to the
// greedy token; then record it and advance the position (see qhip.h).
__global__ __launch_bounds__(1024) void k_argmax_final(const float *bv, const int *bidx, int nb, int *d_in,
                                                       int *d_state, int *d_out, int max_seq) {
  __shared__ float sv[16];
  __shared__ int si[16];
  float best = -INFINITY;
  int idx = 0x7fffffff;
  // 16 candidates per thread per pass, all requested before any is compared
  // (one memory round trip per pass instead of one per candidate)
  constexpr int U = 16;
  for (int i0 = 0; i0 < nb; i0 += U * (int)blockDim.x) {
    float v[U];
    int k[U];
#pragma unroll
    for (int u = 0; u < U; u++) {
      const int i = i0 + u * (int)blockDim.x + (int)threadIdx.x;
      v[u] = i < nb ? bv[i] : -INFINITY;
      k[u] = i < nb ? bidx[i] : 0x7fffffff;
    }
#pragma unroll
    for (int u = 0; u < U; u++)
      if (k[u] != 0x7fffffff && (idx == 0x7fffffff || v[u] > best || (v[u] == best && k[u] < idx))) {
        best = v[u];
        idx = k[u];
      }
  }
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) {
    const float ob = __shfl_xor(best, o, 64);
    const int oi = __shfl_xor(idx, o, 64);
    if (oi != 0x7fffffff && (idx == 0x7fffffff || ob > best || (ob == best && oi < idx))) { best = ob; idx = oi; }
  }
  if ((threadIdx.x & 63) == 0) { sv[threadIdx.x >> 6] = best; si[threadIdx.x >> 6] = idx; }
  __syncthreads();
  if (threadIdx.x == 0) {
    float b = sv[0];
    int i0 = si[0];
    for (int w = 1; w < (int)(blockDim.x >> 6); w++)
      if (si[w] != 0x7fffffff && (i0 == 0x7fffffff || sv[w] > b || (sv[w] == b && si[w] < i0))) { b = sv[w]; i0 = si[w]; }
    const int pos = d_state[0];
    if (pos < max_seq) d_out[pos] = i0;
    if (pos + 1 >= d_state[1] && pos + 1 <= max_seq) d_in[pos + 1] = i0;
    d_state[0] = pos + 1;
  }
}

// Quantize v (n values, quant.c:66-78) given per-block maxima of |v|; grid
// ceil(kpad/1024) blocks of 256 threads x 4 values; block 0 writes the scale.
// The values are requested together with the maxima (one memory round trip).
__global__ __launch_bounds__(256) void k_quant_blocks(const float *v, int n, const float *bm, int nbm, int8_t *qa,
                                                      int kpad, float *as_out) {
  __shared__ float red[4];
  if (threadIdx.x < 64) QTL_MARK(7, 0);
  QTL_ID(7);
  const int k0 = blockIdx.x * 1024 + threadIdx.x * 4;
  float x[4];
#pragma unroll
  for (int r = 0; r < 4; r++) x[r] = k0 + r < n ? v[k0 + r] : 0.0f;
  float mx = 0.0f;
  for (int i = threadIdx.x; i < nbm; i += 256) mx = fmaxf(mx, bm[i]);
  mx = qd::wave_max_f32(mx);
  if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = mx;
  __syncthreads();
  mx = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
  const float as = (mx > 0.0f) ? mx / 127.0f : 1.0f;
  const float inv = 1.0f / as;
  if (k0 < kpad)                                       // values past n were loaded as 0 and give 0
    *reinterpret_cast<uint32_t *>(qa + k0) = qd::quant_i8x4(x[0], x[1], x[2], x[3], inv);
  if (blockIdx.x == 0 && threadIdx.x == 0) *as_out = as;
  QTL_MAX(7, 4);
}

// Output channels per wave.  The GEMVs that normalize their own input take
// several, so that at the 8B shape their blocks are resident together and each
// block's prologue runs once: 6 (gate, up) pairs for SwiGLU, 4 rows for QKV.
constexpr int rows_per_wave(int mode, int pro) { return pro >= 2 ? (mode == MODE_SWIGLU ? 6 : 4) : 2; }

// Weight rows in registers (measured at the 8B shape): all of the wave's rows
// for the GEMVs with a prologue that stay resident with them (QKV: 4, Wo: 2),
// so that the whole weight stream overlaps the prologue; two for the
// 14336-wide down projection; else one (the SwiGLU GEMV's 6 row pairs would
// not stay resident).
constexpr int weight_slots(int mode, int pro, int kch) {
  return (pro >= 2 && mode != MODE_SWIGLU) || pro == 1 ? rows_per_wave(mode, pro) : (pro == 0 && kch == 14) ? 2 : 1;
}

template <int MODE, int PRO>
int launch(int cls, const int8_t *qa, const float *as, const int8_t *W, const float *ws, int N, int kpad, float *out,
           const float *bias, float *bm, int *bi, const float *v, int n, const float *vbm, int nvbm, float eps) {
  constexpr int R = rows_per_wave(MODE, PRO);
  const dim3 grid((N + 4 * R - 1) / (4 * R));
#define QG(KCH)                                                                                                    \
  QH_LAUNCH(cls, (k_gemv_dec<MODE, KCH, R, PRO, weight_slots(MODE, PRO, KCH)>), grid, dim3(256), 0, qa, as, W, ws, N, \
            kpad, out, bias, bm, bi, v, n, vbm, nvbm, eps)
  if constexpr (PRO >= 2) {                          // 256 threads x 4*KCH values of the row
    switch (kpad) {
      case 2048: QG(2); return 0;
      case 4096: QG(4); return 0;
      case 8192: QG(8); return 0;
      default: return qh::fail_msg("gemv: fused rmsnorm needs kpad 2048/4096/8192");
    }
  } else {
    switch (kpad) {
      case 2048: QG(2); return 0;
      case 4096: QG(4); return 0;
      case 8192: QG(8); return 0;
      case 14336: QG(14); return 0;
      default:
        if (PRO) return qh::fail_msg("gemv: fused quantization needs kpad 2048/4096/8192/14336");
        QH_LAUNCH(cls, k_gemv_dec_any<MODE>, dim3((N + 3) / 4), dim3(256), 0, qa, as, W, ws, N, kpad, out, bias, bm,
                  bi);
        return 0;
    }
  }
#undef QG
}

// Rows per row wave and blocks of k_gemv_ws with RWV row waves: one block per
// CU where the rows allow (N rows, or row pairs for SWIGLU).
static inline void ws_shape(int N, int rwv, int &rw, int &blocks) {
  const int cus = qh::num_cus() > 0 ? qh::num_cus() : 256;
  int nb = (N + rwv - 1) / rwv;
  if (nb > cus) nb = cus;
  rw = (N + rwv * nb - 1) / (rwv * nb);
  blocks = (N + rwv * rw - 1) / (rwv * rw);
}

template <int MODE, int PRO>
int launch_ws(int cls, const int8_t *W, const float *ws, int N, int kpad, float *out, const float *bias, float *bm,
              const float *v, int n, const float *vbm, int nvbm, float eps) {
  int rw, blocks;
#define QW(KCH)                                                                                                     \
  ws_shape(N, ws_row_waves(MODE, KCH), rw, blocks);                                                                  \
  QH_LAUNCH(cls, (k_gemv_ws<MODE, KCH, PRO, ws_slots(MODE, KCH), ws_pro_waves(MODE, KCH), ws_row_waves(MODE, KCH)>), \
            dim3(blocks), dim3(64 * (ws_pro_waves(MODE, KCH) + ws_row_waves(MODE, KCH))), 0, W, ws, N, kpad, rw, out,   \
            bias, bm, v, n, vbm, nvbm, eps)
  switch (kpad) {
    case 2048: QW(2); return 0;
    case 4096: QW(4); return 0;
    case 8192: QW(8); return 0;
    case 14336:
      if constexpr (PRO == 1) { QW(14); return 0; }
      return qh::fail_msg("gemv: fused rmsnorm needs kpad 2048/4096/8192");
    default: return qh::fail_msg("gemv: fused prologue needs kpad 2048/4096/8192/14336");
  }
#undef QW
}

// Skinny W8A8 product for 2..16 activation rows (qmatmul with a few rows; the
// batch-8 GEMV of the op-level configuration).  One block of 8 waves per 16
// output channels; wave w takes the 64-byte K steps w, w + 8, w + 16, ... and
// forms each with one v_mfma_i32_16x16x64_i8: activation rows as A (rows past M
// are zero), the 16 weight rows as B.  Fragment layout (as in k_gemm.hip): lane
// l holds row l % 16 and bytes 16 * (l / 16) .. +15 of the step; result element
// e of lane l is C[4 * (l / 16) + e][l % 16].  The next batch of steps is in
// flight while the current one is multiplied.  The waves' int32 tiles are summed
// in LDS (exact in any order), then out[m][j] = (as[m] * ws[j]) * (float)acc
// (quant.c:81-82).
constexpr int kSkWaves = 8, kSkBatch = 4;

__global__ __launch_bounds__(64 * kSkWaves) void k_gemv_mfma(const int8_t *qa, const float *as, int M,
                                                             const int8_t *W, const float *ws, int N, int kpad,
                                                             float *out, int ldo) {
  __shared__ v4i red[kSkWaves][64];
  const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
  const int n0 = blockIdx.x * 16;
  const int fr = lane & 15, kq = lane >> 4;
  const bool a_ok = fr < M;
  const int8_t *ap = qa + (size_t)(a_ok ? fr : 0) * kpad + 16 * kq;
  const int8_t *bp = W + (size_t)min(n0 + fr, N - 1) * kpad + 16 * kq;
  const int nk = (kpad + 63) / 64;
  const int ns = wave < nk ? (nk - wave + kSkWaves - 1) / kSkWaves : 0;   // steps of this wave
  const v4i z = {0, 0, 0, 0};
  auto load = [&](int i, v4i &a, v4i &b) {
    const int off = 64 * (wave + kSkWaves * i);
    const bool in = i < ns && off + 16 * kq < kpad;
    a = in && a_ok ? *reinterpret_cast<const v4i *>(ap + off) : z;
    b = in ? __builtin_nontemporal_load(reinterpret_cast<const v4i *>(bp + off)) : z;
  };
  v4i acc = z;
  v4i a0[kSkBatch], b0[kSkBatch], a1[kSkBatch], b1[kSkBatch];
#pragma unroll
  for (int u = 0; u < kSkBatch; u++) load(u, a0[u], b0[u]);
  for (int i0 = 0; i0 < ns; i0 += 2 * kSkBatch) {
#pragma unroll
    for (int u = 0; u < kSkBatch; u++) load(i0 + kSkBatch + u, a1[u], b1[u]);
#pragma unroll
    for (int u = 0; u < kSkBatch; u++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a0[u], b0[u], acc, 0, 0, 0);
    if (i0 + kSkBatch >= ns) break;
#pragma unroll
    for (int u = 0; u < kSkBatch; u++) load(i0 + 2 * kSkBatch + u, a0[u], b0[u]);
#pragma unroll
    for (int u = 0; u < kSkBatch; u++) acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a1[u], b1[u], acc, 0, 0, 0);
  }
  red[wave][lane] = acc;
  __syncthreads();
  if (threadIdx.x < 256) {
    const int m = threadIdx.x >> 4, n = threadIdx.x & 15;
    const int l = 16 * (m >> 2) + n, e = m & 3;
    int t = 0;
#pragma unroll
    for (int w = 0; w < kSkWaves; w++) t += red[w][l][e];
    if (m < M && n0 + n < N) out[(size_t)m * ldo + n0 + n] = (as[m] * ws[n0 + n]) * (float)t;
  }
}

// Skinny W8A8 product for 2..16 activation rows, persistent (the op-level
// batch-8 GEMV at the vocabulary-sized shape; qmatmul with a few rows).  The M
// activation rows sit in LDS (row stride kpad + 16: the 16 rows of an MFMA
// fragment fall on different banks).  A task is (group of 16 output channels, K
// split): S waves of a block share a group, each taking a contiguous 1/S of its
// 64-byte K steps, and form one v_mfma_i32_16x16x64_i8 per step (fragment
// layout as k_gemv_mfma's: activation rows as A, rows past M zero without a
// read; 16 weight rows as B, lane l holding row l % 16, bytes 16 * (l / 16) ..
// +15 of the step).  The block takes 16 / S groups a round; a wave walks its
// steps of all its rounds with the weight fragments of the next FD steps in
// flight (a ring of registers), so its loads do not wait for a round to end.
// With S > 1 the S int32 partial tiles of a group are added in LDS after the
// round (exact in any order); then out[m][n] = (as[m] * ws[n]) * (float)acc
// (quant.c:81-82), the 16 channel scales through scalar loads.
constexpr int kSkRing = 8;                                       // K steps in flight per wave
constexpr int kSkBlockWaves = 16;

template <int S>
__global__ __launch_bounds__(64 * kSkBlockWaves) void k_gemv_skinny(const int8_t *qa, const float *as, int M,
                                                                    const int8_t *W, const float *ws, int N,
                                                                    int kpad, float *out, int ldo) {
  extern __shared__ __attribute__((aligned(16))) int8_t xs[];    // M rows, stride kpad + 16
  __shared__ v4i part[S > 1 ? kSkBlockWaves : 1][64];            // partial tiles of the splits
  constexpr int GPB = kSkBlockWaves / S;                         // groups per block and round
  constexpr int FD = kSkRing;
  const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int gsub = wave / S, split = wave % S;
  const int nk = kpad / 64, ng = (N + 15) / 16;
  const int k0 = split * nk / S, kn = (split + 1) * nk / S - k0;  // this wave's steps of a group (>= 1)
  const int nround = (ng + GPB - 1) / GPB;                       // block rounds over all groups
  const int myrounds = (int)blockIdx.x < nround ? (nround - (int)blockIdx.x + (int)gridDim.x - 1) / (int)gridDim.x : 0;
  const int nunit = myrounds * kn;
  if (nunit == 0) return;                                        // the same for every wave of the block
  const int fr = lane & 15, kq = lane >> 4;
  const int xstride = kpad + 16;
  const v4i z = {0, 0, 0, 0};
  float asl[4];                                                  // the scales of this lane's result rows
#pragma unroll
  for (int e = 0; e < 4; e++) asl[e] = as[min(4 * kq + e, M - 1)];
  // The wave's units in order: round r (the block's groups r * gridDim.x +
  // blockIdx.x), step k0 + t of the group, t < kn.  The loads run FD units
  // ahead of the MFMAs; (lr, lt) is the unit being requested.  A group's rows
  // past N repeat row N - 1, and requests past the last unit repeat the last.
  int lr = 0, lt = 0;
  auto load_next = [&](v4i &b) {
    const int r = min(lr, myrounds - 1), t = lr < myrounds ? lt : kn - 1;
    const int g = min(((int)blockIdx.x + r * (int)gridDim.x) * GPB + gsub, ng - 1), n = min(16 * g + fr, N - 1);
    b = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(W + (size_t)n * kpad + 64 * (k0 + t) + 16 * kq));
    if (++lt == kn) { lt = 0; lr++; }
  };
  v4i rb[FD];
#pragma unroll
  for (int u = 0; u < FD; u++) load_next(rb[u]);
  for (int c = threadIdx.x; c < M * (kpad / 16); c += 64 * kSkBlockWaves) {
    const int m = c / (kpad / 16), k = c - m * (kpad / 16);
    *reinterpret_cast<v4i *>(xs + (size_t)m * xstride + 16 * k) = reinterpret_cast<const v4i *>(qa + (size_t)m * kpad)[k];
  }
  __syncthreads();
  const int8_t *xrow = xs + (size_t)fr * xstride + 16 * kq;
  v4i acc = z;
  int cr = 0, ct = 0;                                            // the unit being added
  for (int q0 = 0; q0 < nunit; q0 += FD) {
#pragma unroll
    for (int u = 0; u < FD; u++) {
      if (q0 + u >= nunit) break;                                // uniform for the block
      const v4i a = fr < M ? *reinterpret_cast<const v4i *>(xrow + 64 * (k0 + ct)) : z;
      acc = __builtin_amdgcn_mfma_i32_16x16x64_i8(a, rb[u], acc, 0, 0, 0);
      load_next(rb[u]);
      if (++ct == kn) {                                          // the group's last step: add the splits, store
        ct = 0;
        const int g = ((int)blockIdx.x + cr * (int)gridDim.x) * GPB + gsub;
        cr++;
        if constexpr (S > 1) {
          // an LDS-only meeting (a __syncthreads would also wait for the ring)
          part[wave][lane] = acc;
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();
          if (split == 0) {
#pragma unroll
            for (int t = 1; t < S; t++) acc += part[wave + t][lane];
          }
          asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
          __builtin_amdgcn_s_barrier();                          // the partials are read before they are rewritten
        }
        if (split == 0 && g < ng) {
          // the group's 16 channel scales through scalar loads (their own counter:
          // a vector load here would make the next step wait for the whole ring)
          float wsn = 0.0f;
#pragma unroll
          for (int j = 0; j < 16; j++) {
            const float v = ((cfloat_t *)ws)[min(16 * g + j, N - 1)];
            wsn = fr == j ? v : wsn;
          }
          const int n = 16 * g + fr;
#pragma unroll
          for (int e = 0; e < 4; e++) {
            const int m = 4 * kq + e;
            if (m < M && n < N) out[(size_t)m * ldo + n] = (asl[e] * wsn) * (float)acc[e];
          }
        }
        acc = z;
      }
    }
  }
}

// Few-row W8A8 product with whole-row weight loads (qmatmul with 2..8 rows,
// kpad a multiple of 1024 up to 8192: the batch-8 GEMV of the op-level
// configuration at K = 4096).  A block has kpad / 1024 waves; wave w owns the K
// bytes 1024 w .. +1023, lane l the 16 bytes 1024 w + 16 l .. +15, and keeps
// those bytes of every activation row in registers.  The block walks groups of
// 8 output channels (g = blockIdx.x, += gridDim.x); a wave requests the 8
// channels' 1 KiB slices of a group (one coalesced 1 KiB wave load each, as in
// k_gemv_dec) two groups ahead and forms 4 v_dot4_i32_i8 per row and channel.
// The (channel, row) int32 sums of a lane are folded across the wave by a
// transpose reduction: at each of the six lane bits a lane keeps half of its
// values and adds its partner's copy of the same half, so after the folds lane e
// holds the wave's whole sum for entry e (row e % MR, channel e / MR; the index
// bits in fold order).  The waves' sums meet in LDS (exact in any order; an
// LDS-only meeting, the ring stays in flight) and wave 0 stores out[m][n] =
// (as[m] * ws[n]) * (float)acc (quant.c:81-82), the row and channel scales
// through scalar loads.  (Scalars only: a private array read across the
// group's lambdas was placed in LDS, a copy per thread, and cost 11 us a call.)
constexpr int kRowsGroup = 8;                                    // output channels per group

template <int CTRL>
__device__ __forceinline__ int rows_dpp(int v) { return __builtin_amdgcn_mov_dpp(v, CTRL, 0xf, 0xf, true); }

// partner copy across fold level L: row_mirror (bit 3), row_half_mirror (bit 2),
// quad_perm xor 2 (bit 1), xor 1 (bit 0), swizzle xor 16 (bit 4), bpermute xor 32 (bit 5)
template <int L>
__device__ __forceinline__ int rows_partner(int v) {
  if constexpr (L == 0) return rows_dpp<0x140>(v);
  else if constexpr (L == 1) return rows_dpp<0x141>(v);
  else if constexpr (L == 2) return rows_dpp<0x4E>(v);
  else if constexpr (L == 3) return rows_dpp<0xB1>(v);
  else if constexpr (L == 4) return __builtin_amdgcn_ds_swizzle(v, 0x401F);
  else return __shfl_xor(v, 32, 64);
}
constexpr int kRowsLaneBit[6] = {3, 2, 1, 0, 4, 5};

// one fold of NV values at level L: NV / 2 values remain (NV >= 2), or with one
// value a plain add of the partner's
template <int L, int NV>
__device__ __forceinline__ void rows_fold(int (&v)[16], int lane) {
  if constexpr (NV == 1) {
    v[0] += rows_partner<L>(v[0]);
  } else {
    const bool hi = (lane >> kRowsLaneBit[L]) & 1;
#pragma unroll
    for (int j = 0; j < NV / 2; j++) {
      const int keep = hi ? v[2 * j + 1] : v[2 * j], send = hi ? v[2 * j] : v[2 * j + 1];
      v[j] = keep + rows_partner<L>(send);
    }
  }
}

template <int MR>
__global__ __launch_bounds__(1024) void k_gemv_rows(const int8_t *qa, const float *as, int M, const int8_t *W,
                                                    const float *ws, int N, int kpad, float *out, int ldo) {
  __shared__ int part[8][64];
  constexpr int G = kRowsGroup;
  static_assert(MR == 2 || MR == 4 || MR == 8, "rows per pass");
  constexpr int NF = MR == 2 ? 4 : MR == 4 ? 5 : 6;             // folds that halve (8 * MR entries)
  const int lane = threadIdx.x & 63, w = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int nw = (int)(blockDim.x >> 6);
  const int ng = (N + G - 1) / G;
  const int ni = ((ng - 1 - (int)blockIdx.x) / (int)gridDim.x) + 1;  // groups of this block (grid <= ng)
  const unsigned kb = 1024u * w + 16u * lane;                    // lane offset (uniform row + 32-bit offset)
  const v4i z = {0, 0, 0, 0};
  // The wave's units in order: channel c of group i (the block's groups i *
  // gridDim.x + blockIdx.x), unit 8 i + c.  The loads run 2 groups ahead of the
  // dots through a ring of registers; requests past the last unit repeat it.
  const int nunit = G * ni;
  int lu = 0;                                                    // the unit being requested
  auto load_next = [&](v4i &b) {
    const int u = min(lu, nunit - 1), g = (int)blockIdx.x + (u / G) * (int)gridDim.x;
    const int8_t *row = W + (size_t)min(G * g + u % G, N - 1) * kpad;   // uniform
    b = __builtin_nontemporal_load(reinterpret_cast<const v4i *>(row + kb));
    lu++;
  };
  v4i x[MR];
#pragma unroll
  for (int m = 0; m < MR; m++) x[m] = m < M ? *reinterpret_cast<const v4i *>(qa + (size_t)m * kpad + kb) : z;
  float asl[MR];                                                 // scalar loads: their own counter
#pragma unroll
  for (int m = 0; m < MR; m++) asl[m] = ((cfloat_t *)as)[min(m, M - 1)];
  // this lane's entry after the folds: the index bits in fold order
  int e = 0;
#pragma unroll
  for (int L = 0; L < NF; L++) e |= ((lane >> kRowsLaneBit[L]) & 1) << L;
  bool writer = true;                                            // lanes past the folds hold copies
#pragma unroll
  for (int L = NF; L < 6; L++) writer = writer && !((lane >> kRowsLaneBit[L]) & 1);
  const int em = e % MR, ec = e / MR;
  float ase = asl[0];
#pragma unroll
  for (int m = 1; m < MR; m++) ase = em == m ? asl[m] : ase;

  // the wave's sums of group i meet in LDS; wave 0 stores the group's outputs
  auto finish = [&](int i, int vsum) {
    part[w][lane] = vsum;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();                                // an LDS-only meeting (a __syncthreads
    if (w == 0) {                                                // would also wait for the ring)
      int t = 0;
#pragma unroll
      for (int u = 0; u < 8; u++)
        if (u < nw) t += part[u][lane];                           // uniform
      const int g = (int)blockIdx.x + i * (int)gridDim.x;
      float wsn = 0.0f;                                          // the 8 channel scales: scalar loads
#pragma unroll
      for (int c = 0; c < G; c++) {
        const float sv = ((cfloat_t *)ws)[min(G * g + c, N - 1)];
        wsn = ec == c ? sv : wsn;
      }
      const int n = G * g + ec;
      if (writer && em < M && n < N) out[(size_t)em * ldo + n] = (ase * wsn) * (float)t;
    }
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");
    __builtin_amdgcn_s_barrier();                                // the sums are read before they are rewritten
  };

  constexpr int FD = 2 * G;
  v4i rb[FD];
#pragma unroll
  for (int u = 0; u < FD; u++) load_next(rb[u]);
  int v[16];
  // unit q0 + u from ring slot u (then that slot requests the unit FD ahead)
  auto unit = [&](int q0, int u, bool more) {
    int a[16];
#pragma unroll
    for (int m = 0; m < MR; m++) {
      int t = __builtin_amdgcn_sdot4(x[m].x, rb[u].x, 0, false);
      t = __builtin_amdgcn_sdot4(x[m].y, rb[u].y, t, false);
      t = __builtin_amdgcn_sdot4(x[m].z, rb[u].z, t, false);
      a[m] = __builtin_amdgcn_sdot4(x[m].w, rb[u].w, t, false);
    }
    if (more) load_next(rb[u]);
    // the channel's MR row sums folded over the first log2(MR) lane bits
    if constexpr (MR >= 2) rows_fold<0, MR>(a, lane);
    if constexpr (MR >= 4) rows_fold<1, MR / 2>(a, lane);
    if constexpr (MR >= 8) rows_fold<2, MR / 4>(a, lane);
    v[u % G] = a[0];
    if (u % G == G - 1) {                                        // the group's last channel
      constexpr int L0 = MR == 2 ? 1 : MR == 4 ? 2 : 3;          // next fold level
      rows_fold<L0, 8>(v, lane);
      rows_fold<L0 + 1, 4>(v, lane);
      rows_fold<L0 + 2, 2>(v, lane);
      if constexpr (L0 + 3 < 6) rows_fold<L0 + 3, 1>(v, lane);
      if constexpr (L0 + 4 < 6) rows_fold<L0 + 4, 1>(v, lane);
      if constexpr (L0 + 5 < 6) rows_fold<L0 + 5, 1>(v, lane);
      finish((q0 + u) / G, v[0]);
    }
  };
  // whole turns of the ring with no exit inside (so the wait before each unit
  // is for that unit's load alone), then the one group that may remain (the
  // unit count is a multiple of G)
  int q0 = 0;
  for (; q0 + FD <= nunit; q0 += FD) {
#pragma unroll
    for (int u = 0; u < FD; u++) unit(q0, u, true);
  }
  if (q0 < nunit) {
#pragma unroll
    for (int u = 0; u < G; u++) unit(q0, u, false);
  }
}

}  // namespace

extern "C" int qhip_gemv_mfma(int cls, const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws,
                              int N, int kpad, float *out, int ldo) {
  if (M < 1 || M > 16 || kpad % 16 || N < 1) return qh::fail_msg("gemv_mfma: needs 1..16 rows and kpad % 16 == 0");
  QH_LAUNCH(cls, k_gemv_mfma, dim3((N + 15) / 16), dim3(64 * kSkWaves), 0, qa, as, M, W, ws, N, kpad, out, ldo);
  return 0;
}

// 2..8 activation rows, kpad a multiple of 1024 up to 8192 (k_gemv_rows; at
// kpad = 14336 its 14-wave blocks, one a CU, ran 5 % behind k_gemv_mfma: 20.0
// against 19.0 us at N = 4096, so longer rows stay there).
extern "C" int qhip_gemv_rows_ok(int M, int N, int kpad) {
  return M >= 2 && M <= 8 && N >= 1 && kpad % 1024 == 0 && kpad >= 1024 && kpad <= 8192;
}

extern "C" int qhip_gemv_rows(int cls, const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws,
                              int N, int kpad, float *out, int ldo) {
  if (!qhip_gemv_rows_ok(M, N, kpad)) return qh::fail_msg("gemv_rows: needs 2..8 rows and kpad = 1024 * (1..8)");
  const int nw = kpad / 1024, ng = (N + kRowsGroup - 1) / kRowsGroup;
  const int cus = qh::num_cus() > 0 ? qh::num_cus() : 256;
  const int grid = min(ng, cus * max(1, 16 / nw));               // about 16 waves a CU, all resident
  const dim3 block(64 * nw);
  if (M <= 2) QH_LAUNCH(cls, k_gemv_rows<2>, dim3(grid), block, 0, qa, as, M, W, ws, N, kpad, out, ldo);
  else if (M <= 4) QH_LAUNCH(cls, k_gemv_rows<4>, dim3(grid), block, 0, qa, as, M, W, ws, N, kpad, out, ldo);
  else QH_LAUNCH(cls, k_gemv_rows<8>, dim3(grid), block, 0, qa, as, M, W, ws, N, kpad, out, ldo);
  return 0;
}

namespace {
template <int S>
int launch_skinny(int cls, const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws, int N,
                  int kpad, float *out, int ldo) {
  static size_t attr = 0;
  const size_t lds = (size_t)M * (kpad + 16);
  if (lds > 64 * 1024 && lds > attr) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k_gemv_skinny<S>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return qh::fail("hipFuncSetAttribute(k_gemv_skinny)", e);
    attr = lds;
  }
  const int cus = qh::num_cus() > 0 ? qh::num_cus() : 256;
  const int nround = ((N + 15) / 16 + kSkBlockWaves / S - 1) / (kSkBlockWaves / S);
  // one block of 16 waves per CU: every block resident at once
  QH_LAUNCH(cls, k_gemv_skinny<S>, dim3(min(nround, cus)), dim3(64 * kSkBlockWaves), lds, qa, as, M, W, ws, N, kpad,
            out, ldo);
  return 0;
}
}  // namespace

// 2..16 activation rows within 128 KiB of LDS, kpad a multiple of 64, and at least 2 * 4096 groups of
// 16 channels per 2 K splits (N >= 65536 at 256 CUs: the vocabulary-sized
// products).  Narrower products need more K splits, whose meetings per group
// made this kernel slower than k_gemv_mfma (measured at N = 4096 and 14336).
extern "C" int qhip_gemv_skinny_ok(int M, int N, int kpad) {
  const int cus = qh::num_cus() > 0 ? qh::num_cus() : 256;
  return M >= 2 && M <= 16 && kpad % 64 == 0 && kpad >= 128 && (size_t)M * (kpad + 16) <= 128 * 1024 &&
         (long)((N + 15) / 16) * 2 >= 2L * cus * kSkBlockWaves;
}

// K is split over two waves where the 16-channel groups alone would leave waves
// idle (about 2 * 4096 tasks fill 256 CUs x 16 waves); every wave of a block has
// steps (kpad >= 128), as the block's meetings need.
extern "C" int qhip_gemv_skinny(int cls, const int8_t *qa, const float *as, int M, const int8_t *W,
                                const float *ws, int N, int kpad, float *out, int ldo) {
  if (!qhip_gemv_skinny_ok(M, N, kpad)) return qh::fail_msg("gemv_skinny: needs 2..16 rows, kpad % 64 == 0, N >= 65536");
  const int ng = (N + 15) / 16, nk = kpad / 64, cus = qh::num_cus() > 0 ? qh::num_cus() : 256;
  const long want = 2L * cus * kSkBlockWaves;
  const int S = ng >= want || nk < 2 ? 1 : 2;                      // qhip_gemv_skinny_ok: ng >= want / 2
  if (S == 1) return launch_skinny<1>(cls, qa, as, M, W, ws, N, kpad, out, ldo);
  return launch_skinny<2>(cls, qa, as, M, W, ws, N, kpad, out, ldo);
}

// The W8A8 product of qmatmul for M quantized rows: the decode GEMV for one row;
// for 2..8 rows with kpad = 1024 * (1..8) the whole-row kernel k_gemv_rows; for
// the other few-row shapes the persistent skinny kernel on vocabulary-sized
// products and the per-block skinny kernel otherwise; the MFMA GEMM beyond.
extern "C" int qhip_qmm_product(const int8_t *qa, const float *as, int M, const int8_t *W, const float *ws, int N,
                                int kpad, float *C) {
  if (M == 1) return qhip_gemv_dec(MODE_PLAIN, QK_OTHER, qa, as, W, ws, N, kpad, C, NULL, NULL, NULL);
#ifndef QLLAMA_NO_GEMV_ROWS
  if (qhip_gemv_rows_ok(M, N, kpad)) return qhip_gemv_rows(QK_OTHER, qa, as, M, W, ws, N, kpad, C, N);
#endif
  if (qhip_gemv_skinny_ok(M, N, kpad)) return qhip_gemv_skinny(QK_OTHER, qa, as, M, W, ws, N, kpad, C, N);
  if (M <= 16) return qhip_gemv_mfma(QK_OTHER, qa, as, M, W, ws, N, kpad, C, N);
  return qhip_gemm_i8(0, QK_OTHER, qa, as, W, ws, M, N, kpad, C, N, NULL);
}

extern "C" int qhip_gemv_blocks(int N, int kpad) {
  switch (kpad) {
    case 2048: case 4096: case 8192: case 14336: return (N + 7) / 8;
    default: return (N + 3) / 4;
  }
}

extern "C" int qhip_gemv_dec(int mode, int cls, const int8_t *qa, const float *as, const int8_t *W, const float *ws,
                             int N, int kpad, float *out, const float *bias, float *bm, int *bi) {
  if (kpad % 16) return qh::fail_msg("gemv: kpad must be a multiple of 16");
  switch (mode) {
    case MODE_PLAIN: return launch<MODE_PLAIN, 0>(cls, qa, as, W, ws, N, kpad, out, bias, bm, bi, NULL, 0, NULL, 0, 0.0f);
    case MODE_RESID: return launch<MODE_RESID, 0>(cls, qa, as, W, ws, N, kpad, out, bias, bm, bi, NULL, 0, NULL, 0, 0.0f);
    case MODE_SWIGLU: return launch<MODE_SWIGLU, 0>(cls, qa, as, W, ws, N, kpad, out, bias, bm, bi, NULL, 0, NULL, 0, 0.0f);
    case MODE_HEAD: return launch<MODE_HEAD, 0>(cls, qa, as, W, ws, N, kpad, out, bias, bm, bi, NULL, 0, NULL, 0, 0.0f);
    default: return qh::fail_msg("gemv: bad mode");
  }
}

// Residual GEMV whose activation v (n values) is quantized inside the kernel from
// the per-block maxima vbm of its producer (replaces qhip_quant_blocks + mode 1).
extern "C" int qhip_gemv_resid_q(int cls, const float *v, int n, const float *vbm, int nvbm, const int8_t *W,
                                 const float *ws, int N, int kpad, float *out) {
  if (kpad % 16 || n > kpad) return qh::fail_msg("gemv_resid_q: bad shape");
  if (kUseWs) return launch_ws<MODE_RESID, 1>(cls, W, ws, N, kpad, out, NULL, NULL, v, n, vbm, nvbm, 0.0f);
  return launch<MODE_RESID, 1>(cls, NULL, NULL, W, ws, N, kpad, out, NULL, NULL, NULL, v, n, vbm, nvbm, 0.0f);
}

// SwiGLU GEMV whose activation is rmsnorm(x) quantized, formed inside every
// block (replaces qhip_rmsnorm_quant + mode 2).
extern "C" int qhip_gemv_swiglu_norm(int cls, int fast, const float *x, int dm, const float *gamma, float eps,
                                     const int8_t *W, const float *ws, int N, int kpad, float *out, float *bm) {
  if (!qhip_gemv_norm_ok(kpad, dm)) return qh::fail_msg("gemv_swiglu_norm: unsupported shape");
  if (kUseWs) {
    if (fast) return launch_ws<MODE_SWIGLU, 3>(cls, W, ws, N, kpad, out, NULL, bm, x, dm, gamma, 0, eps);
    return launch_ws<MODE_SWIGLU, 2>(cls, W, ws, N, kpad, out, NULL, bm, x, dm, gamma, 0, eps);
  }
  if (fast) return launch<MODE_SWIGLU, 3>(cls, NULL, NULL, W, ws, N, kpad, out, NULL, bm, NULL, x, dm, gamma, 0, eps);
  return launch<MODE_SWIGLU, 2>(cls, NULL, NULL, W, ws, N, kpad, out, NULL, bm, NULL, x, dm, gamma, 0, eps);
}

// Shapes qhip_gemv_swiglu_norm supports.
extern "C" int qhip_gemv_norm_ok(int kpad, int dm) {
  return (kpad == 2048 || kpad == 4096 || kpad == 8192) && dm > 0 && dm <= kpad;
}

// Number of per-block maxima qhip_gemv_swiglu_norm writes.
extern "C" int qhip_gemv_norm_blocks(int N) {
  if (kUseWs) {
    int rw, blocks;
    ws_shape(N, ws_row_waves(MODE_SWIGLU, 4), rw, blocks);
    return blocks;
  }
  constexpr int per_block = 4 * rows_per_wave(MODE_SWIGLU, 2);
  return (N + per_block - 1) / per_block;
}

// Plain (QKV) GEMV whose activation is rmsnorm(x) quantized, formed inside
// every block (replaces qhip_rmsnorm_quant + mode 0).
extern "C" int qhip_gemv_plain_norm(int cls, int fast, const float *x, int dm, const float *gamma, float eps,
                                    const int8_t *W, const float *ws, int N, int kpad, float *out, const float *bias) {
  if (!qhip_gemv_norm_ok(kpad, dm)) return qh::fail_msg("gemv_plain_norm: unsupported shape");
  if (kUseWs) {
    if (fast) return launch_ws<MODE_PLAIN, 3>(cls, W, ws, N, kpad, out, bias, NULL, x, dm, gamma, 0, eps);
    return launch_ws<MODE_PLAIN, 2>(cls, W, ws, N, kpad, out, bias, NULL, x, dm, gamma, 0, eps);
  }
  if (fast) return launch<MODE_PLAIN, 3>(cls, NULL, NULL, W, ws, N, kpad, out, bias, NULL, NULL, x, dm, gamma, 0, eps);
  return launch<MODE_PLAIN, 2>(cls, NULL, NULL, W, ws, N, kpad, out, bias, NULL, NULL, x, dm, gamma, 0, eps);
}

// Shapes qhip_gemv_resid_q supports.
extern "C" int qhip_gemv_fused_ok(int kpad) { return kpad == 2048 || kpad == 4096 || kpad == 8192 || kpad == 14336; }

extern "C" int qhip_quant_blocks(const float *v, int n, const float *bm, int nbm, int8_t *qa, int kpad, float *as) {
  QH_LAUNCH(QK_QUANT, k_quant_blocks, dim3((kpad + 1023) / 1024), dim3(256), 0, v, n, bm, nbm, qa, kpad, as);
  return 0;
}

extern "C" int qhip_argmax_final(const float *bv, const int *bidx, int nb, int *d_in, int *d_state, int *d_out,
                                 int max_seq) {
  QH_LAUNCH(QK_ARGMAX, k_argmax_final, dim3(1), dim3(1024), 0, bv, bidx, nb, d_in, d_state, d_out, max_seq);
  return 0;
}
