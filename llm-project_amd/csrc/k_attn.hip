// k_attn.hip - decode attention over the device KV cache (llama.c:554-576).
//
// Exactness: the reference forms, per query head h,
//   dot_j = sum_d q_d * K_jd      (d = 0..hd-1, in order)
//   s_j   = dot_j * scale,  m = max_j s_j,  e_j = expf(s_j - m)
//   S     = sum_j e_j             (j = 0..T-1, in order)
//   w_j   = e_j * (1 / S),  o_d = sum_j w_j * V_jd   (j in order, from 0)
// The dot products and the weighted sums of V are formed here in the same order
// by one lane each; S is evaluated exactly in parallel (qdev_seqsum.h); maxima
// do not depend on order.  The parallelism is across positions (scores), across
// (head, d) chains, and between the lanes that form the products w_j * V_jd and
// the lane that adds them.
//
// Kernel 1 (k_attn_scores): grid (n_kv, ceil(max_seq/128)); one thread per
//   (head, position) computes dot_j and s_j; the block's K rows are copied into
//   LDS with direct global-to-LDS loads; each block writes its maximum.
// Kernel 2 (k_attn_pv): grid (H, ceil(hd/16)), 512 threads.  All threads form
//   the head's softmax weights in LDS (each thread a run of consecutive
//   positions, in registers).  Then lanes 0-15 of wave 0 own 16 output chains
//   o_d while waves 1-7 stream V tiles of 128 positions, five tiles ahead, and
//   store the products w_j * V_jd as [d][j] tiles (three buffers in LDS, the
//   producers two tiles ahead of the chains), so that the chain lane reads four
//   consecutive positions with one 16-byte LDS read and issues the reads of the
//   next tile before the barrier that ends the current one.  A chain is one
//   dependent add per position (about 5 clocks with the wave's lanes all
//   active, which is why lanes 16-63 repeat chain 15); sixteen chains per block
//   spread a head's V stream over hd/16 CUs.
#include <hip/hip_runtime.h>

#include "qdev_chain.h"
#include "qdev_math.h"
#include "qdev_norm.h"
#include "qdev_seqsum.h"
#include "qhip.h"
#include "qhip_internal.h"
#include "qdev_tl.h"

QTL_DEFINE(attn)

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v2i __attribute__((ext_vector_type(2)));

constexpr int kScoreBlock = 128;        // positions per scores block (two waves per query head)
constexpr int kTile = 128;                  // positions per PV tile
constexpr int kTS = kTile + 4;              // LDS row stride of a product tile (conflict-free 16-byte reads)
constexpr int kPBuf = 3;                    // product tiles in LDS
constexpr int kChains = 16;                 // output dims per PV block (lanes 0-15 of wave 0)
constexpr int kPvThreads = 512;
constexpr int kProducers = kPvThreads - 64;
constexpr int kPWaves = kProducers / 64;    // 7
constexpr int kUnits = kPWaves * (64 / kChains);             // 28 producer units of kChains lanes
constexpr int kGroups = kTile / 4;          // groups of 4 positions per tile
constexpr int kGSlots = (kGroups + kUnits - 1) / kUnits;     // 2 groups per producer lane

__device__ __forceinline__ void lds_barrier() { qd::lds_sync(); }

template <int NT>
__device__ __forceinline__ float block_max(float m, float *red) {
  m = qd::wave_max_f32(m);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  qd::lds_sync();
  if (lane == 0) red[w] = m;
  qd::lds_sync();
  float r = red[0];
#pragma unroll
  for (int i = 1; i < NT / 64; i++) r = fmaxf(r, red[i]);
  return r;
}

// runtime head_dim: rows loaded 8 floats ahead of the chain
__device__ __forceinline__ float score_dot_any(const float *qs, const float *kr, int hd) {
  float dot = 0.0f;
  int d = 0;
  for (; d + 8 <= hd; d += 8) {
    float k[8];
#pragma unroll
    for (int i = 0; i < 8; i++) k[i] = kr[d + i];
#pragma unroll
    for (int i = 0; i < 8; i++) dot += qs[d + i] * k[i];
  }
  for (; d < hd; d++) dot += qs[d] * kr[d];
  return dot;
}

// The block's K rows are copied straight from global memory into LDS
// (global_load_lds, 16 bytes per lane, no registers), every copy in flight at
// once; each wave instruction moves two whole 512-byte rows, so the reads are
// coalesced.  Row r keeps its 16-byte chunk c at slot (c + r mod 8) mod CPR of
// the row: lane t then reads chunk i of its own row from slot (i + t mod 8) mod
// CPR, and the eight lanes served per LDS cycle hit eight different bank
// groups.  A lane's column repeats every four copies, so a copy costs one
// pointer add.  Blocks that end past T (only the last one) clamp rows to T-1.
typedef __attribute__((address_space(3))) void *lds_void_ptr;

template <int HD>
__device__ __forceinline__ void score_copy_rows(const float *Kh, int j0, int T, float *ks, bool full, int nwaves) {
  static_assert(HD == 128, "two rows per wave instruction");
  constexpr int CPR = HD / 4;                                // 16-byte chunks per row (32)
  constexpr int NCOPY = kScoreBlock * CPR / 64;              // wave instructions for the tile (64)
  const int per = (NCOPY + nwaves - 1) / nwaves;             // copies per wave
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  const int half = lane >> 5, pos = lane & 31;
  const int k0 = wv * per, k1 = min(NCOPY, k0 + per);
  if (full) {
    // copy kk moves rows 2kk and 2kk+1; lane (half, pos) takes chunk
    // c = (pos - (2kk + half) mod 8) mod CPR of row 2kk + half
    const char *rb = reinterpret_cast<const char *>(Kh + (size_t)(j0 + half) * HD);
    for (int kk = k0; kk < k1; kk++) {
      const int c = (pos - ((2 * kk + half) & 7)) & (CPR - 1);
      __builtin_amdgcn_global_load_lds((const void *)(rb + (size_t)kk * 2 * HD * 4 + 16 * c),
                                       (lds_void_ptr)(ks + kk * 64 * 4), 16, 0, 0);
    }
  } else {
    for (int kk = k0; kk < k1; kk++) {
      const int r = 2 * kk + half;
      const int c = (pos - (r & 7)) & (CPR - 1);
      const int j = min(j0 + r, T - 1);
      __builtin_amdgcn_global_load_lds((const void *)(Kh + (size_t)j * HD + 4 * c), (lds_void_ptr)(ks + kk * 64 * 4),
                                       16, 0, 0);
    }
  }
}

// dot_j for the lane's own row in LDS: eight 16-byte row reads are issued per
// batch, then the batch's 32 steps of the sequential chain; q is wave-uniform
// and comes through the scalar cache.
template <int HD>
__device__ __forceinline__ float score_row_dot(const float *qh, const float *ks, int t) {
  constexpr int CPR = HD / 4;
  const float4 *row = reinterpret_cast<const float4 *>(ks) + t * CPR;
  const float4 *q4 = reinterpret_cast<const float4 *>(qh);
  const int sk = t & 7;
  float dot = 0.0f;
#pragma unroll
  for (int b = 0; b < CPR; b += 8) {
    float4 kv[8];
#pragma unroll
    for (int i = 0; i < 8; i++) kv[i] = row[(b + i + sk) & (CPR - 1)];
#pragma unroll
    for (int i = 0; i < 8; i++) {
      const float4 qv = q4[b + i];
      dot += qv.x * kv[i].x;
      dot += qv.y * kv[i].y;
      dot += qv.z * kv[i].z;
      dot += qv.w * kv[i].w;
    }
  }
  return dot;
}

// One block per (KV head, 128 positions) serves the G = H / n_kv query heads of
// that group: G x 128 threads, thread (g, t) computes head kvh*G + g at position
// j0 + t, and the K tile is copied into LDS once for all of them.  (64-position
// blocks, twice as many, measured no faster end to end.)  With n_kv a
// multiple of 8, consecutive KV heads also fall on different XCDs.
// ROPE: q, k and v of the current position arrive unrotated in qkv (the QKV
// GEMV's output, H + 2 n_kv heads of hd); every block rotates its G query heads
// into LDS (rope.c:48-68, the table holding cos and sin of position * inv_freq),
// and the block holding position pos rotates k, uses it for its own row and
// appends k and v to the cache (llama.c:551-552), which the later kernels read.
template <int HD, bool ROPE>
__global__ __launch_bounds__(1024) void k_attn_scores(const float *q, float *kc, float *vc, const int *d_pos, int H,
                                                       int KVH, int hd, int max_seq, float scale, float *scores,
                                                       float *bmax, int nch, const float *cos_t,
                                                       const float *sin_t) {
  __shared__ __attribute__((aligned(16))) float qs[8 * (HD ? HD : 512)];
  __shared__ __attribute__((aligned(16))) float ks[HD ? kScoreBlock * HD : 4];
  __shared__ __attribute__((aligned(16))) float kcur[HD ? HD : 512];
  __shared__ float red[16];
  const int kvh = blockIdx.x, c = blockIdx.y;
  const int G = H / KVH;
  const int pos = *d_pos, T = pos + 1;
  if (c * kScoreBlock >= T) return;                      // uniform for the block
  if (threadIdx.x < 64) QTL_MARK(0, 0);
  QTL_ID(0);
  const int g = __builtin_amdgcn_readfirstlane(threadIdx.x / kScoreBlock), t = threadIdx.x % kScoreBlock;
  const int h = kvh * G + g;
  const int j0 = c * kScoreBlock, j = j0 + t;
  const bool last = j0 + kScoreBlock >= T;               // this block holds position pos
  float *Kh = kc + (size_t)kvh * max_seq * hd;
  const int half = hd >> 1;
  if (HD) score_copy_rows<HD ? HD : 128>(Kh, j0, T, ks, j0 + kScoreBlock <= T, (int)(blockDim.x >> 6));
  // the group's query heads into LDS (rotated when ROPE)
  if (ROPE) {
    const float *ct = cos_t + (size_t)pos * half, *st = sin_t + (size_t)pos * half;
    for (int i = threadIdx.x; i < G * half; i += blockDim.x) {
      const int gg = i / half, k = i % half;
      const float *xh = q + (size_t)(kvh * G + gg) * hd;
      const float cs = ct[k], sn = st[k];
      const float x1 = xh[k], x2 = xh[k + half];
      qs[gg * hd + k] = x1 * cs - x2 * sn;
      qs[gg * hd + k + half] = x2 * cs + x1 * sn;
    }
    if (last) {
      const float *kh = q + (size_t)(H + kvh) * hd, *vh = q + (size_t)(H + KVH + kvh) * hd;
      float *kdst = Kh + (size_t)pos * hd, *vdst = vc + ((size_t)kvh * max_seq + pos) * hd;
      for (int k = threadIdx.x; k < half; k += blockDim.x) {
        const float cs = ct[k], sn = st[k];
        const float x1 = kh[k], x2 = kh[k + half];
        const float y1 = x1 * cs - x2 * sn, y2 = x2 * cs + x1 * sn;
        kcur[k] = y1;
        kcur[k + half] = y2;
        kdst[k] = y1;
        kdst[k + half] = y2;
      }
      for (int d = threadIdx.x; d < hd; d += blockDim.x) vdst[d] = vh[d];
    }
  } else {
    for (int d = threadIdx.x; d < G * hd; d += blockDim.x) qs[d] = q[(size_t)kvh * G * hd + d];
  }
  __syncthreads();                                       // q, the current k row, the K tile copies (vmcnt)
  if (threadIdx.x < 64) QTL_MARK(0, 1);
  if (HD && ROPE && last) {                              // the current row into its (skewed) place in the tile
    constexpr int CPR = (HD ? HD : 128) / 4;
    const int rr = pos - j0;
    for (int d = threadIdx.x; d < hd; d += blockDim.x)
      ks[rr * hd + 4 * (((d >> 2) + (rr & 7)) & (CPR - 1)) + (d & 3)] = kcur[d];
    __syncthreads();
  }
  float dot;
  if (HD) {
    dot = score_row_dot<HD ? HD : 128>(qs + g * hd, ks, t);
  } else {
    const float *kr = (ROPE && j == pos) ? kcur : Kh + (size_t)min(j, pos) * hd;
    dot = j < T ? score_dot_any(qs + g * hd, kr, hd) : 0.0f;
  }
  float s = -INFINITY;
  if (j < T) {
    s = dot * scale;
    scores[(size_t)h * max_seq + j] = s;
  }
  // per-head block maximum: the head's waves
  constexpr int WPH = kScoreBlock / 64;                  // waves per query head
  s = qd::wave_max_f32(s);
  if (WPH == 1) {
    if (t == 0) bmax[(size_t)h * nch + c] = s;
  } else {
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = s;
    __syncthreads();
    if (t == 0) {
      float mb = red[WPH * g];
      for (int i = 1; i < WPH; i++) mb = fmaxf(mb, red[WPH * g + i]);
      bmax[(size_t)h * nch + c] = mb;
    }
  }
  QTL_MAX(0, 4);
}

// Head of PV block x: the query heads of one KV head are given block indices
// congruent modulo n_kv.  Workgroups are dealt to the XCDs round-robin by
// index, so with n_kv a multiple of 8 a group's blocks share one XCD and its
// L2, and each KV head's V rows are fetched from HBM once per XCD.
__device__ __forceinline__ int head_of_block(int x, int H, int KVH) { return (x % KVH) * (H / KVH) + x / KVH; }

// V values of tile t for this producer lane (unit u = pid / kChains, column
// dd = pid % kChains): slot g covers positions t*kTile + 4*(u + kUnits*g) + 0..3
// at column d0 + dd.  The loads go
// through a buffer resource over this KV head's rows [0, max_seq): the lane's
// offset of each slot is fixed (vo) and the tile adds one scalar, so a load
// costs one add of address arithmetic; the whole offset is in the range-checked
// vector operand, so tiles past the last one (the prefetch runs ahead), rows
// past max_seq and unused slots read as 0 without touching memory.  Wave 0 (the
// chains) issues none.  Rows in [T, max_seq) and columns >= hd are zeroed by the
// producer.
__device__ __forceinline__ void pv_load(float (&v)[kGSlots][4], __amdgpu_buffer_rsrc_t rs, const int (&vo)[kGSlots],
                                        int t, int ntile, int hd) {
  if (threadIdx.x < 64) return;                                   // wave 0: no slots
  const int tb = t < ntile ? t * kTile * hd * 4 : 0x40000000;   // tiles past the last: no memory traffic
#pragma unroll
  for (int g = 0; g < kGSlots; g++)
#pragma unroll
    for (int i = 0; i < 4; i++)
      v[g][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, vo[g] + tb + i * hd * 4, 0, 0));
}

// Products of tile t into the [d][j] tile B: B[dd*kTS + jj] = w_j * V_j,d0+dd,
// +0 for positions >= T or dims >= hd (adding +0 leaves a chain unchanged).
// Only a partial tile or a partial column block needs the masks; they are
// applied bitwise, so that no branch delays the LDS reads or splits the quad.
// The weights of all slots are read before any product is stored.
__device__ __forceinline__ float pv_mask(float p, bool keep) {
  return __uint_as_float(__float_as_uint(p) & (keep ? 0xffffffffu : 0u));
}

// vpos >= 0: the value of V at position vpos is vpatch (for this lane's column)
// instead of what the load returned (the row the same launch has just appended).
__device__ __forceinline__ void pv_produce(float *B, const float *W, const float (&v)[kGSlots][4], int t, int T,
                                           bool cols_full, bool col_ok, int pid, int vpos = -1,
                                           float vpatch = 0.0f) {
  const int u = pid / kChains, dd = pid % kChains;
  const bool full = cols_full && (t + 1) * kTile <= T;
  float4 w[kGSlots];
#pragma unroll
  for (int g = 0; g < kGSlots; g++) {
    const int grp = u + kUnits * g;
    if (kUnits * (g + 1) <= kGroups || grp < kGroups)          // compile-time true except the last slot
      w[g] = *reinterpret_cast<const float4 *>(W + t * kTile + 4 * grp);
  }
#pragma unroll
  for (int g = 0; g < kGSlots; g++) {
    const int grp = u + kUnits * g;
    if (kUnits * (g + 1) <= kGroups || grp < kGroups) {
      const int jb = t * kTile + 4 * grp;
      float v0 = v[g][0], v1 = v[g][1], v2 = v[g][2], v3 = v[g][3];
      if (vpos >= jb && vpos < jb + 4) {
        v0 = vpos == jb ? vpatch : v0;
        v1 = vpos == jb + 1 ? vpatch : v1;
        v2 = vpos == jb + 2 ? vpatch : v2;
        v3 = vpos == jb + 3 ? vpatch : v3;
      }
      float4 p;
      p.x = w[g].x * v0;
      p.y = w[g].y * v1;
      p.z = w[g].z * v2;
      p.w = w[g].w * v3;
      if (!full) {
        p.x = pv_mask(p.x, col_ok && jb + 0 < T);
        p.y = pv_mask(p.y, col_ok && jb + 1 < T);
        p.z = pv_mask(p.z, col_ok && jb + 2 < T);
        p.w = pv_mask(p.w, col_ok && jb + 3 < T);
      }
      *reinterpret_cast<float4 *>(B + dd * kTS + 4 * grp) = p;
    }
  }
}


// The V stream of one PV block's producer lanes (waves 1-7): the buffer
// resource over its KV head's rows, each lane's slot offsets, and the first
// three tiles, requested by pv_v_start.  A caller that starts it early
// (k_attn_layer) hands it to pv_block, which otherwise starts it itself.
struct PvV {
  __amdgpu_buffer_rsrc_t rs;
  int vo[kGSlots];
  float r0[kGSlots][4], r1[kGSlots][4], r2[kGSlots][4];
};

__device__ __forceinline__ void pv_v_start(PvV &v, const float *vc, int kvh, int hd, int max_seq, int d0, int ntile) {
  const int tid = threadIdx.x, pid = tid - 64;
  const float *Vh = vc + (size_t)kvh * max_seq * hd;
  v.rs = __builtin_amdgcn_make_buffer_rsrc((void *)Vh, (short)0, max_seq * hd * 4, 0x00020000);
#pragma unroll
  for (int g = 0; g < kGSlots; g++) {
    const int grp = pid / kChains + kUnits * g;
    v.vo[g] = tid >= 64 && grp < kGroups ? (4 * grp * hd + d0 + pid % kChains) * 4 : 0x40000000;   // else: no traffic
  }
  pv_load(v.r0, v.rs, v.vo, 0, ntile, hd);
  pv_load(v.r1, v.rs, v.vo, 1, ntile, hd);
  pv_load(v.r2, v.rs, v.vo, 2, ntile, hd);
}

// One PV block with CM softmax terms per thread (512 * CM >= T).
//  1. Requests the head's block maxima, this thread's CM scores, and the
//     producers' first three V tiles, in that order, so that each wait leaves
//     the later requests in flight.
//  2. Softmax weights (llama.c:557-572): m = max of the block maxima,
//     e_j = expf(s_j - m) in registers (all CM terms formed side by side on
//     every lane, then positions >= T cleared), their sequential sum S exactly
//     (qdev_seqsum.h), then w_j = e_j * (1 / S) into LDS.
//  3. o_d = sum_j w_j * V_jd, j in order (llama.c:570-575): wave 0 owns the
//     chains; waves 1-7 form the product tiles.  Barrier k (k = 0 .. ntile-1,
//     executed by every wave) certifies that tiles <= k+1 are in LDS and that
//     the chains are done with tile k-1: tile k sits in buffer k % 3, and the
//     producers refill buffer (k+2) % 3 = (k-1) % 3 after barrier k.
// XCH: the scores and block maxima were written by other blocks of the same
// launch on this XCD (k_attn_layer): they are read past the L1, the maxima
// are at bmax[h * nch + i] for i < nbm, and V's row T-1 (appended by the same
// launch) comes from vrow instead of the cache.
// PRE: the caller has started the V stream (pre, from pv_v_start).
template <int CM, bool DIVW, bool XCH = false, bool PRE = false>
__device__ __forceinline__ void pv_block(const float *scores, const float *bmax, const float *vc, int T, int h,
                                         int kvh, int hd, int max_seq, int nch, float *o, float *obm, float *lds,
                                         float *red, qd::SeqScratch &seq, const uint64_t *tab, int slice,
                                         int nslice, int nbm = 0, const float *vrow = nullptr, PvV *pre = nullptr) {
  const int d0 = slice * kChains, tid = threadIdx.x;
  const int wcap = (max_seq + kTile - 1) / kTile * kTile;
  float *W = lds;
  float *P = lds + wcap;                                 // kPBuf tiles of kChains x kTS
  const int ntile = (T + kTile - 1) / kTile;
  const float *sh = scores + (size_t)h * max_seq;

  // 1. requests (block maxima: at most 128 <= 512 per head)
  const int nc = XCH ? nbm : (T + kScoreBlock - 1) / kScoreBlock;
  float m = -INFINITY;
  if (tid < nc)
    m = XCH ? __hip_atomic_load(bmax + (size_t)h * nch + tid, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
            : bmax[(size_t)h * nch + tid];
  const __amdgpu_buffer_rsrc_t srs = __builtin_amdgcn_make_buffer_rsrc((void *)sh, (short)0, max_seq * 4, 0x00020000);
  const int j0 = tid * CM;
  float e[CM];
  if constexpr (CM % 4 == 0) {
#pragma unroll
    for (int c = 0; c < CM; c += 4) {     // positions past max_seq read as 0; past T they are masked below
      const v4i q = __builtin_bit_cast(v4i, __builtin_amdgcn_raw_buffer_load_b128(srs, (j0 + c) * 4, 0, XCH ? 16 : 0));
      e[c] = __int_as_float(q.x); e[c + 1] = __int_as_float(q.y);
      e[c + 2] = __int_as_float(q.z); e[c + 3] = __int_as_float(q.w);
    }
  } else if constexpr (CM % 2 == 0) {    // 8-byte pieces (the chunks are 8-byte aligned)
#pragma unroll
    for (int c = 0; c < CM; c += 2) {
      const v2i q = __builtin_bit_cast(v2i, __builtin_amdgcn_raw_buffer_load_b64(srs, (j0 + c) * 4, 0, XCH ? 16 : 0));
      e[c] = __int_as_float(q.x); e[c + 1] = __int_as_float(q.y);
    }
  } else {
#pragma unroll
    for (int c = 0; c < CM; c++)
      e[c] = __int_as_float(__builtin_amdgcn_raw_buffer_load_b32(srs, (j0 + c) * 4, 0, XCH ? 16 : 0));
  }
  const int pid = tid - 64;
  PvV own;
  PvV &V = PRE ? *pre : own;
  if constexpr (!PRE) pv_v_start(own, vc, kvh, hd, max_seq, d0, ntile);
  const bool cols_full = d0 + kChains <= hd, col_ok = d0 + pid % kChains < hd;
  const int vpos = XCH ? T - 1 : -1;
  const float vpatch = XCH && tid >= 64 && col_ok
                           ? __hip_atomic_load(vrow + d0 + pid % kChains, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
                           : 0.0f;

  // 2. softmax weights
  m = block_max<kPvThreads>(m, red);
  if (tid < 64) QTL_MARK(1, 1);
  if (__builtin_amdgcn_readfirstlane(j0) < T) {          // waves wholly past T hold zeros only
#pragma unroll
    for (int c = 0; c < CM; c++) e[c] = e[c] - m;
    qd::expf_glibc_n<CM>(e, tab);
#pragma unroll
    for (int c = 0; c < CM; c++) e[c] = pv_mask(e[c], j0 + c < T);
  } else {
#pragma unroll
    for (int c = 0; c < CM; c++) e[c] = 0.0f;
  }
  const float sum = qd::seq_sum_nonneg<kPvThreads, CM>(e, T, seq, [&](int i) {
    const float si = XCH ? __hip_atomic_load(sh + i, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) : sh[i];
    return qd::expf_glibc(si - m, tab);
  });
  const float inv = 1.0f / sum;
  if (tid < 64) QTL_MARK(1, 2);
  if constexpr (CM % 4 == 0) {
#pragma unroll
    for (int c = 0; c < CM; c += 4)
      if (j0 + c < wcap) {
        if (DIVW)   // model.c:501: (e_j / sum) * V
          *reinterpret_cast<float4 *>(W + j0 + c) = make_float4(e[c] / sum, e[c + 1] / sum, e[c + 2] / sum, e[c + 3] / sum);
        else        // llama.c:568-571: e_j * (1 / sum)
          *reinterpret_cast<float4 *>(W + j0 + c) = make_float4(e[c] * inv, e[c + 1] * inv, e[c + 2] * inv, e[c + 3] * inv);
      }
  } else if constexpr (CM % 2 == 0) {
#pragma unroll
    for (int c = 0; c < CM; c += 2)
      if (j0 + c < wcap) {
        if (DIVW) *reinterpret_cast<float2 *>(W + j0 + c) = make_float2(e[c] / sum, e[c + 1] / sum);
        else *reinterpret_cast<float2 *>(W + j0 + c) = make_float2(e[c] * inv, e[c + 1] * inv);
      }
  } else {
#pragma unroll
    for (int c = 0; c < CM; c++)
      if (j0 + c < wcap) W[j0 + c] = DIVW ? e[c] / sum : e[c] * inv;
  }
  qd::lds_sync();
  if (tid < 64) QTL_MARK(1, 3);

  // 3. the chains
  if (tid < 64) {                 // lanes past kChains run garbage chains and store nothing
    const int d = d0 + tid;
    const int crow = tid < kChains ? tid : kChains - 1;
    const unsigned base = (unsigned)(uintptr_t)(P + crow * kTS);   // LDS byte address of the lane's row
    static_assert(kChains * kTS * 4 == qd::kChainBufBytes && kPBuf == 3 && kTile == 128, "chain_tiles_asm's layout");
    float acc = 0.0f;
    lds_barrier();                                         // barrier 0: tiles 0 and 1
    QTL_CYC(2, 0);
    int n = ntile;
    qd::chain_tiles_asm(acc, base, n);
    QTL_CYC(2, 1);
    QTL_MARK(1, 5);
    const bool own = tid < kChains && d < hd;
    if (own) o[(size_t)h * hd + d] = acc;
    if (obm) {                 // max |o| of this block, for the activation quantizer
      const float mo = qd::wave_max_f32(own ? fabsf(acc) : 0.0f);
      if (tid == 0) obm[(size_t)h * nslice + slice] = mo;
    }
  } else {
    // tile k is formed from register set k % 3 into LDS buffer k % 3; its V
    // values are requested five tiles ahead of use (three ahead of forming)
    float *B0 = P, *B1 = P + kChains * kTS, *B2 = P + 2 * kChains * kTS;
    pv_produce(B0, W, V.r0, 0, T, cols_full, col_ok, pid, vpos, vpatch);
    pv_load(V.r0, V.rs, V.vo, 3, ntile, hd);
    pv_produce(B1, W, V.r1, 1, T, cols_full, col_ok, pid, vpos, vpatch);   // past the last tile: zeros, never read
    pv_load(V.r1, V.rs, V.vo, 4, ntile, hd);
    lds_barrier();                                         // barrier 0
    for (int k = 0;; k += 3) {
      if (k + 1 >= ntile) break;
      pv_produce(B2, W, V.r2, k + 2, T, cols_full, col_ok, pid, vpos, vpatch);
      pv_load(V.r2, V.rs, V.vo, k + 5, ntile, hd);
      lds_barrier();                                       // barrier k+1
      if (k + 2 >= ntile) break;
      pv_produce(B0, W, V.r0, k + 3, T, cols_full, col_ok, pid, vpos, vpatch);
      pv_load(V.r0, V.rs, V.vo, k + 6, ntile, hd);
      lds_barrier();                                       // barrier k+2
      if (k + 3 >= ntile) break;
      pv_produce(B1, W, V.r1, k + 4, T, cols_full, col_ok, pid, vpos, vpatch);
      pv_load(V.r1, V.rs, V.vo, k + 7, ntile, hd);
      lds_barrier();                                       // barrier k+3
    }
  }
  QTL_MAX(1, 4);
}

template <bool DIVW>
__global__ __launch_bounds__(kPvThreads) void k_attn_pv(const float *scores, const float *bmax, const float *vc,
                                                        const int *d_pos, int H, int KVH, int hd, int max_seq,
                                                        int nch, float *o, float *obm) {
  extern __shared__ __attribute__((aligned(16))) float lds_raw[];
  float *lds = lds_raw + ((16u - ((unsigned)(uintptr_t)lds_raw & 15u)) & 15u) / 4u;   // 16-byte reads; an LDS pointer
  __shared__ float red[kPvThreads / 64];
  __shared__ qd::SeqScratch seq;
  __shared__ uint64_t tab[32];
  if (threadIdx.x < 64) QTL_MARK(1, 0);
  QTL_ID(1);
  qd::exp_table_to_lds(tab);                             // published by the block max's barrier
  const int h = head_of_block(blockIdx.x, H, KVH);
  const int T = *d_pos + 1;
  const int kvh = h / (H / KVH);
  // the fewest terms a thread that cover T: the exact sum's per-wave work shrinks with them
#define PV_BAND(CM_)                                                                                              \
  if (T <= kPvThreads * CM_) {                                                                                     \
    pv_block<CM_, DIVW>(scores, bmax, vc, T, h, kvh, hd, max_seq, nch, o, obm, lds, red, seq, tab, blockIdx.y,       \
                        gridDim.y);                                                                                \
    return;                                                                                                        \
  }
  PV_BAND(1) PV_BAND(2) PV_BAND(3) PV_BAND(4) PV_BAND(5) PV_BAND(6) PV_BAND(8) PV_BAND(16)
#undef PV_BAND
  pv_block<32, DIVW>(scores, bmax, vc, T, h, kvh, hd, max_seq, nch, o, obm, lds, red, seq, tab, blockIdx.y, gridDim.y);
}

// ---------------------------------------------------------------------------
// The attention half of a decode layer in one launch (exact mode):
//   Q  the QKV GEMV with its exact rmsnorm prologue (rmsnorm.c:7-21,
//      quant.c:60-85, llama.c:541-548), for the rows of one KV head's query,
//      key and value heads;
//   S  RoPE (rope.c:48-68), the cache append (llama.c:551-552) and the scores
//      s_j = (q . K_j) * scale of 1/32 of the positions (llama.c:557-563);
//   P  the softmax and o = sum_j w_j V_j (llama.c:564-575), as k_attn_pv.
// Grid: 32 blocks per KV head, n_kv = 8.  Workgroups are dealt to the eight
// XCDs round-robin, continuing from where the previous launches left off:
// block b runs on XCD (s + b) % 8 for a start s that changes from launch to
// launch.  A block therefore serves the KV head of the XCD it runs on (read
// from the hardware), with rank b / 8 among that XCD's 32 blocks, so a KV
// head's blocks share one XCD and its L2 whatever s is (the host probes once
// that a launch covers every XCD 32 times).  Between the phases the head's 32 blocks meet at a
// counter (ly_meet) instead of a kernel boundary, and what one block hands to
// another (the QKV outputs, the scores, the block maxima) goes through that
// shared L2: plain stores, which the write-through L1 passes on to the L2 before
// the store counter drains, and device-scope loads, which skip the L1 (whose
// lines could predate the store).  Every block must be resident at once: the host launches the
// kernel only where there are 32 * n_kv CUs for its one block per CU.  A
// meeting that waits too long (a block not resident, or an XCD given other
// than 32 blocks), sets an error flag, which the host reports as an error; the
// block goes on, so the kernel always ends.
// ---------------------------------------------------------------------------
#ifndef QLLAMA_LY_L2_COUNTER
#define QLLAMA_LY_L2_COUNTER 1
#endif
constexpr int kLyNB = 32;                   // blocks per KV head
constexpr int kLyThreads = 512;
constexpr int kLyWaves = kLyThreads / 64;
constexpr int kLyPW = 4;                    // phase Q: prologue waves (rmsnorm, quantization of x) ...
constexpr int kLyRW = kLyWaves - kLyPW;     // ... and row waves
// QKV rows of a row wave: (G + 2) * hd / (32 * 4) at most, G <= 4
constexpr int ly_rows_per_wave(int hd) { return 6 * hd / (32 * 4); }
constexpr int kLyKRows = 128;               // K rows of a block in LDS: at most 32 * 128 positions
constexpr unsigned kLySpin = 1u << 18;      // polls before a meeting gives up (~0.1 s; a meeting takes ~1 us)
static_assert(kLyThreads == kPvThreads, "phase P is the PV block");

__device__ __forceinline__ float ly_ld(const float *p) {
  return __hip_atomic_load(p, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// The blocks of one KV head meet: every wave's stores have completed, one
// thread counts the block in (the counter only grows, by kLyNB per launch) and
// waits until all of this launch's blocks have arrived.
__device__ __forceinline__ void ly_meet(unsigned *ctr, unsigned *err, int tk = -1) {
  asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
  __syncthreads();
  if (threadIdx.x == 0) {
    if (tk >= 0) QTL_MARK(tk, 5);
#if QLLAMA_LY_L2_COUNTER
    // every block of the meeting runs on this XCD: its L2 performs the add
    const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#else
    const unsigned old = __hip_atomic_fetch_add(ctr, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
#endif
    const unsigned target = old - old % kLyNB + kLyNB;
    for (unsigned n = 0;; n++) {
      const unsigned c = __hip_atomic_load(ctr, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
      if ((int)(c - target) >= 0) break;
      if (n == kLySpin) {
        __hip_atomic_store(err, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
        break;
      }
      __builtin_amdgcn_s_sleep(1);
    }
  }
  __syncthreads();
}

// Row of the QKV matrix ([q heads | k heads | v heads] x head_dim rows) that is
// local row l of KV head kvh's rows [q of its G heads | k | v].
__device__ __forceinline__ int ly_row(int kvh, int l, int G, int H, int KVH, int hd) {
  if (l < G * hd) return kvh * G * hd + l;
  l -= G * hd;
  if (l < hd) return H * hd + kvh * hd + l;
  return H * hd + KVH * hd + kvh * hd + (l - hd);
}

template <int KCH>
__device__ __forceinline__ void ly_load_row(v4i (&w)[KCH], const int8_t *row, int lane) {
  const v4i *p = reinterpret_cast<const v4i *>(row);
#pragma unroll
  for (int i = 0; i < KCH; i++) w[i] = __builtin_nontemporal_load(&p[lane + 64 * i]);
}

template <int KCH>
__device__ __forceinline__ int ly_dot_row(const v4i (&w)[KCH], const v4i (&a)[KCH]) {
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

// K rows j0 .. j0+nr-1 (nr <= kLyKRows) into LDS, laid out as score_copy_rows
// lays them out (row rr's 16-byte chunk c at slot (c + rr mod 8) mod CPR), so
// score_row_dot reads them; rows past nr repeat the last one (the same lines:
// no extra HBM traffic).
template <int HD>
__device__ __forceinline__ void ly_copy_k(const float *Kh, int j0, int nr, float *ks) {
  constexpr int CPR = HD / 4;                 // 16-byte chunks per row
  constexpr int RPI = 64 / CPR;               // rows per wave instruction
  constexpr int NI = kLyKRows / RPI / kLyRW;  // copies per row wave: a fixed count, so that the compiler
                                              // can wait for earlier loads without waiting for these
  const int lane = threadIdx.x & 63;
  const int wv = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6) - kLyPW;
  const int sub = lane / CPR, slot = lane % CPR;
  const int last = nr > 0 ? j0 + nr - 1 : 0;      // a block without positions copies row 0 (never read)
#pragma unroll
  for (int i = 0; i < NI; i++) {
    const int kk = wv + kLyRW * i;
    const int rr = kk * RPI + sub;
    const int c = (slot - (rr & 7)) & (CPR - 1);
    const int j = min(j0 + rr, last);
    // nontemporal: each K row is read by one block once, and a nontemporal
    // line does not push other lines (the kernels' code among them) out of L2
    // (decode +1.7 % end to end)
    __builtin_amdgcn_global_load_lds((const void *)(Kh + (size_t)j * HD + 4 * c), (lds_void_ptr)(ks + kk * 64 * 4),
                                     16, 0, 2);
  }
}

template <int HD, int KCH>
__global__ __launch_bounds__(kLyThreads) void k_attn_layer(const float *x, const float *gain, float eps, int dm,
                                                           const int8_t *W, const float *ws, const float *bias,
                                                           int kpad, float *kc, float *vc, const int *d_pos, int H,
                                                           int KVH, int max_seq, float scale, const float *cos_t,
                                                           const float *sin_t, float *scores, float *bmax,
                                                           float *qx, unsigned *sync, float *o, float *obm) {
  // the K rows, then the PV weights and tiles: 16-byte reads, so the array
  // starts at the first 16-byte boundary past the static variables (the
  // launch requests 16 bytes more than it uses)
  extern __shared__ __attribute__((aligned(16))) float lds_raw[];
  float *lds = lds_raw + ((16u - ((unsigned)(uintptr_t)lds_raw & 15u)) & 15u) / 4u;   // still an LDS pointer
  __shared__ __attribute__((aligned(16))) float qs[4 * HD];
  __shared__ __attribute__((aligned(16))) float kcur[HD];
  __shared__ __attribute__((aligned(16))) int8_t qsh[KCH * 1024];
  __shared__ float red[2 * (kLyThreads / 64)];
  __shared__ qd::SeqScratch seq;
  __shared__ uint64_t tab[32];
  __shared__ unsigned ly_gctr, ly_issued, ly_ready;
  __shared__ float ly_as;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  unsigned xcc;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(xcc));
  const int kvh = (int)(xcc & 7u), r = blockIdx.x / 8;        // the KV head of this XCD; rank on it
  const int G = H / KVH;
  const int nrow = (G + 2) * HD, RB = nrow / kLyNB;           // the KV head's QKV rows; per block
  const int T = *d_pos + 1, pos = T - 1;
  const int PB = (T + kLyNB - 1) / kLyNB;                     // score positions per block
  const int j0 = r * PB, j1 = min(T, j0 + PB), nr = max(0, j1 - j0);
  float *Kh = kc + (size_t)kvh * max_seq * HD;
  float *xq = qx + (size_t)kvh * nrow;                         // this launch's q (G heads), k, v of the KV head
  unsigned *err = sync + 2 * 64 * KVH;
  if (wave == 0) QTL_MARK(3, 0);
  QTL_ID(3);
  const uint64_t tabv = tid < 32 ? qd::kExp2Tab[tid] : 0;      // to LDS after the prologue: a store
                                                              // now would wait for the load at once
  if (tid == 0) {
    ly_gctr = 0u; ly_issued = 0u; ly_ready = 0u;
    if (xcc > 7u) __hip_atomic_store(err, 2u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_SYSTEM);
  }
  __syncthreads();                                             // the counters

  // ---- Q: the KV head's QKV rows (k_gemv_ws PRO = 2's operations and order) ----
  // Waves 0-3 normalize and quantize x into LDS, meeting at an LDS counter;
  // waves 4-7 request their weight rows and this block's K rows of phase S as
  // soon as the prologue's inputs are requested, then wait on an LDS flag.  At
  // the end the producer waves (1-7) request phase P's first V tiles, which the
  // meeting after this phase lets land.
  const int NS = (HD + kChains - 1) / kChains;
  const bool pv = r < G * NS;                                   // this block has a phase P
  const int ph = kvh * G + r / NS, pslice = r % NS;
  PvV vpre;
  if (wave < kLyPW) {
    constexpr int NTP = 64 * kLyPW, CMQ = KCH * 1024 / NTP;    // kpad = NTP * CMQ
    unsigned epoch = 0u;
    const qd::GroupSync gs{&ly_gctr, (unsigned)kLyPW, &epoch};
    float y[CMQ], gm[CMQ];
    qd::rmsnorm_load<CMQ>(x, dm, gain, y, gm);
    __builtin_amdgcn_sched_barrier(0);
    if (lane == 0) __hip_atomic_fetch_add(&ly_issued, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
#if QLLAMA_TIMELINE
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");            // (stamped builds only) x has arrived
    if (wave == 0) { QTL_MARK(3, 6); QTL_MARK(4, 0); QTL_CYC(4, 3); }
#endif
    const float as = qd::rmsnorm_apply<NTP, CMQ>(x, dm, eps, y, gm, red, seq, gs);
    if (wave == 0) { QTL_MARK(4, 1); QTL_CYC(4, 5); }
    const float inv = 1.0f / as;
#pragma unroll
    for (int c = 0; c < CMQ; c += 4) *reinterpret_cast<uint32_t *>(qsh + tid * CMQ + c) = qd::quant_word(y, c, inv);
    if (wave == 0) { QTL_MARK(4, 2); QTL_MARK(4, 4); }
    if (tid == 0) ly_as = as;
    asm volatile("s_waitcnt lgkmcnt(0)" ::: "memory");        // this wave's bytes (and as) have landed
    if (lane == 0) __hip_atomic_fetch_add(&ly_ready, 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
    if (wave == 0) QTL_MARK(3, 1);
  } else {
    const int rw = wave - kLyPW;
    while (__hip_atomic_load(&ly_issued, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (unsigned)kLyPW) {
    }
    constexpr int RPW = ly_rows_per_wave(HD);
    v4i w[RPW][KCH];
    float wsc[RPW], wb[RPW];
#pragma unroll
    for (int s = 0; s < RPW; s++) {
      const int l = min(rw + kLyRW * s, RB - 1);                // rows past RB repeat the last (not used)
      const int j = ly_row(kvh, r * RB + l, G, H, KVH, HD);
      ly_load_row<KCH>(w[s], W + (size_t)j * kpad, lane);
      wsc[s] = ws[j];
      wb[s] = bias ? bias[j] : 0.0f;
    }
    __builtin_amdgcn_sched_barrier(0);                          // the K copies after every weight and scale
    ly_copy_k<HD>(Kh, j0, nr, lds);                             // phase S's K rows, straight into LDS
    __builtin_amdgcn_sched_barrier(0);
    while (__hip_atomic_load(&ly_ready, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP) < (unsigned)kLyPW) {
    }
    asm volatile("" ::: "memory");
    const float as = ly_as;
    v4i a[KCH];
#pragma unroll
    for (int i = 0; i < KCH; i++) a[i] = *reinterpret_cast<const v4i *>(qsh + 16 * (lane + 64 * i));
#pragma unroll
    for (int s = 0; s < RPW; s++) {
      const int l = rw + kLyRW * s;
      const int acc = qd::wave_sum_i32(ly_dot_row<KCH>(w[s], a));
      if (rw == 0 && s == 0) QTL_MARK(3, 2);
      if (l < RB) {
        const float c = (as * wsc[s]) * (float)acc;
        if (lane == 0) xq[r * RB + l] = bias ? c + wb[s] : c;
      }
    }
    if (rw == 0) QTL_MARK(3, 3);
  }
  if (pv) pv_v_start(vpre, vc, kvh, HD, max_seq, pslice * kChains, (T + kTile - 1) / kTile);
  if (tid < 32) tab[tid] = tabv;                               // published by the meeting
  ly_meet(sync + (0 * KVH + kvh) * 64, err, 3);                  // also: this block's K rows are in LDS
  if (wave == 0) QTL_MARK(3, 4);

  // ---- S: RoPE, the cache append, the scores of positions j0 .. j1-1 ----
  if (wave == 0) QTL_MARK(0, 0);
  constexpr int half = HD / 2;
  const bool holds = j0 <= pos && pos < j1;
  {
    const float *ct = cos_t + (size_t)pos * half, *st = sin_t + (size_t)pos * half;
    for (int i = tid; i < G * half; i += kLyThreads) {
      const int gg = i / half, k = i % half;
      const float cs = ct[k], sn = st[k];
      const float x1 = ly_ld(xq + gg * HD + k), x2 = ly_ld(xq + gg * HD + k + half);
      qs[gg * HD + k] = x1 * cs - x2 * sn;
      qs[gg * HD + k + half] = x2 * cs + x1 * sn;
    }
    if (holds) {
      float *kdst = Kh + (size_t)pos * HD, *vdst = vc + ((size_t)kvh * max_seq + pos) * HD;
      for (int k = tid; k < half; k += kLyThreads) {
        const float cs = ct[k], sn = st[k];
        const float x1 = ly_ld(xq + G * HD + k), x2 = ly_ld(xq + G * HD + k + half);
        const float y1 = x1 * cs - x2 * sn, y2 = x2 * cs + x1 * sn;
        kcur[k] = y1;
        kcur[k + half] = y2;
        kdst[k] = y1;
        kdst[k + half] = y2;
      }
      for (int d = tid; d < HD; d += kLyThreads) vdst[d] = ly_ld(xq + (G + 1) * HD + d);
    }
  }
  __syncthreads();
  if (holds) {                                                 // the current row into its place in the tile
    constexpr int CPR = HD / 4;
    const int rr = pos - j0;
    for (int d = tid; d < HD; d += kLyThreads) lds[rr * HD + 4 * (((d >> 2) + (rr & 7)) & (CPR - 1)) + (d & 3)] = kcur[d];
    __syncthreads();
  }
  if (wave == 0) QTL_MARK(0, 1);
  {
    const int g = __builtin_amdgcn_readfirstlane(tid / kScoreBlock), t = tid % kScoreBlock;
    float s = -INFINITY;
    if (g < G && t < nr) {
      s = score_row_dot<HD>(qs + g * HD, lds, t) * scale;
      scores[(size_t)(kvh * G + g) * max_seq + j0 + t] = s;
    }
    s = qd::wave_max_f32(s);                                   // two waves per query head
    if (lane == 0) red[wave] = s;
    __syncthreads();
    if (tid < G) bmax[(size_t)(kvh * G + tid) * kLyNB + r] = fmaxf(red[2 * tid], red[2 * tid + 1]);
  }
  QTL_MAX(0, 4);
  ly_meet(sync + (1 * KVH + kvh) * 64, err);

  // ---- P: softmax weights and the chains of 16 output dims of one query head ----
  if (pv) {
    if (wave == 0) QTL_MARK(1, 0);
    QTL_ID(1);
    const int nbm = (T + PB - 1) / PB;                         // blocks that had positions
    const float *vrow = xq + (G + 1) * HD;
    // the fewest terms a thread that cover T (T <= 4096 here): the exact sum's
    // per-wave work shrinks with them
#define LY_PV_BAND(CM_)                                                                                          \
  if (T <= kPvThreads * CM_) {                                                                                    \
    pv_block<CM_, false, true, true>(scores, bmax, vc, T, ph, kvh, HD, max_seq, kLyNB, o, obm, lds, red, seq, tab, \
                                     pslice, NS, nbm, vrow, &vpre);                                                \
    return;                                                                                                       \
  }
    LY_PV_BAND(1) LY_PV_BAND(2) LY_PV_BAND(3) LY_PV_BAND(4) LY_PV_BAND(5) LY_PV_BAND(6)
#undef LY_PV_BAND
    pv_block<8, false, true, true>(scores, bmax, vc, T, ph, kvh, HD, max_seq, kLyNB, o, obm, lds, red, seq, tab,
                                   pslice, NS, nbm, vrow, &vpre);
  }
}

// The XCC (XCD) each of n blocks ran on.
__global__ void k_xcc_probe(unsigned *out) {
  if (threadIdx.x == 0) {
    unsigned v;
    asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(v));
    out[blockIdx.x] = v & 0xfu;
  }
}

// ---------------------------------------------------------------------------
// Prompt ingestion: causal attention of R query rows at positions p0 .. p0+R-1
// against cache rows 0 .. p0+R-1, each row exactly as its decode step forms it
// (the same sums in the same order).  Scratch w[h][r][Tp] holds the scores and
// then, in place, the softmax weights.
// ---------------------------------------------------------------------------
constexpr int kPvRows = 8;            // query rows per PV block (half for short prompts)
#ifndef QLLAMA_PF_SMALL_ROWS
#define QLLAMA_PF_SMALL_ROWS 1024     // prompts of at most this many rows per pass take the half blocks
#endif
constexpr size_t kPfScratchBytes = (size_t)1 << 30;   // score scratch per attention pass (bounds the rows of a pass)

// Softmax weights of one (head, row) (llama.c:557-572): NT threads, thread t
// holds the scores j in [t*CM, t*CM + CM) in registers (one read of the row),
// the block takes their maximum, forms e_j, evaluates their sequential sum
// exactly, and writes w_j = e_j * (1 / S) in place.
template <int NT, int CM>
__device__ __forceinline__ void pf_softmax_row(float *row, int T, qd::SeqScratch &seq, float *red,
                                               const uint64_t *tab) {
  static_assert(CM % 4 == 0, "whole float4 words");
  const int j0 = threadIdx.x * CM;
  float e[CM];
#pragma unroll
  for (int c = 0; c < CM; c += 4) {                  // rows are 16-byte aligned (Tp % 4 == 0)
    float4 t = make_float4(-INFINITY, -INFINITY, -INFINITY, -INFINITY);
    if (j0 + c + 4 <= T) t = *reinterpret_cast<const float4 *>(row + j0 + c);
    else if (j0 + c < T) {
      t.x = row[j0 + c];
      if (j0 + c + 1 < T) t.y = row[j0 + c + 1];
      if (j0 + c + 2 < T) t.z = row[j0 + c + 2];
    }
    e[c] = t.x; e[c + 1] = t.y; e[c + 2] = t.z; e[c + 3] = t.w;
  }
  float m = e[0];
#pragma unroll
  for (int c = 1; c < CM; c++) m = fmaxf(m, e[c]);
  m = qd::wave_max_f32(m);
  if constexpr (NT > 64) {
    if ((threadIdx.x & 63) == 0) red[threadIdx.x >> 6] = m;
    __syncthreads();
    m = red[0];
#pragma unroll
    for (int i = 1; i < NT / 64; i++) m = fmaxf(m, red[i]);
  }
#pragma unroll
  for (int c = 0; c < CM; c++) e[c] = e[c] - m;                         // -inf past T: expf gives +0
  qd::expf_glibc_n<CM>(e, tab);
  const float sum = qd::seq_sum_nonneg<NT, CM>(e, T, seq, [&](int i) { return qd::expf_glibc(row[i] - m, tab); });
  const float inv = 1.0f / sum;
#pragma unroll
  for (int c = 0; c < CM; c += 4) {
    if (j0 + c + 4 <= T) {
      *reinterpret_cast<float4 *>(row + j0 + c) = make_float4(e[c] * inv, e[c + 1] * inv, e[c + 2] * inv, e[c + 3] * inv);
    } else {
#pragma unroll
      for (int u = 0; u < 4; u++)
        if (j0 + c + u < T) row[j0 + c + u] = e[c + u] * inv;
    }
  }
}

// Rows r_lo .. r_hi-1 of every head (T = p0 + r + 1 <= NT * CM), the longest
// first.  One instantiation per row length band: a block's registers and its
// terms per thread follow its own rows, not the longest row of the pass.  The
// one-wave bands of 24 and 32 terms are held to 4 and 3 waves per SIMD (128 and
// 168 registers, no spills): the 32-term band ran 10 % faster so.
template <int NT, int CM>
__global__ __launch_bounds__(NT, NT == 64 && CM == 32 ? 3 : NT == 64 && CM == 24 ? 4 : 1) void k_pf_softmax(float *w, int R, int p0, int Tp, int r_hi) {
  __shared__ qd::SeqScratch seq;
  __shared__ float red[NT / 64];
  __shared__ uint64_t tab[32];
  qd::exp_table_to_lds(tab);
  __syncthreads();                                   // publishes the exp table
  const int h = blockIdx.x, r = r_hi - 1 - blockIdx.y;
  const int T = p0 + r + 1;
  float *row = w + ((size_t)h * R + r) * Tp;
  pf_softmax_row<NT, CM>(row, T, seq, red, tab);
}

// The bands: (threads, terms per thread); a row of T positions takes the first
// band with NT * CM >= T.  One wave per row up to 2048 positions (more waves
// per row measured slower: each adds its share of the sum's fixed steps), in
// bands of 512 positions past 1024.
struct PfBand { int nt, cm; };
constexpr PfBand kPfBands[] = {{64, 4}, {64, 8}, {64, 16}, {64, 24}, {64, 32}, {128, 24}, {128, 32},
                               {256, 32}, {512, 32}};
constexpr int kPfBandCount = sizeof(kPfBands) / sizeof(kPfBands[0]);

int pf_softmax_band(int band, float *w, int R, int p0, int Tp, int r_lo, int r_hi, int H) {
  const dim3 grid(H, r_hi - r_lo), block(kPfBands[band].nt);
#define PF_SM(NT_, CM_) QH_LAUNCH(QK_PF_ATTN, (k_pf_softmax<NT_, CM_>), grid, block, 0, w, R, p0, Tp, r_hi)
  switch (band) {
    case 0: PF_SM(64, 4); break;
    case 1: PF_SM(64, 8); break;
    case 2: PF_SM(64, 16); break;
    case 3: PF_SM(64, 24); break;
    case 4: PF_SM(64, 32); break;
    case 5: PF_SM(128, 24); break;
    case 6: PF_SM(128, 32); break;
    case 7: PF_SM(256, 32); break;
    default: PF_SM(512, 32); break;
  }
#undef PF_SM
  return 0;
}

// Softmax of rows 0 .. R-1 (T = p0 + r + 1), band by band from the longest rows.
int pf_softmax_rows(float *w, int R, int p0, int Tp, int H) {
  for (int b = kPfBandCount - 1; b >= 0; b--) {
    const int cap = kPfBands[b].nt * kPfBands[b].cm, lo_cap = b ? kPfBands[b - 1].nt * kPfBands[b - 1].cm : 0;
    const int r_lo = max(0, lo_cap - p0), r_hi = min(R, cap - p0);       // lo_cap < T <= cap
    if (r_hi > r_lo && pf_softmax_band(b, w, R, p0, Tp, r_lo, r_hi, H)) return 1;
  }
  return 0;
}

// Block (KV head, 8 query rows), one wave per query head of the group: lane l
// owns dims 2l, 2l+1 (HD = 128) or dim l (HD <= 64) and, for each, the chains of
// the block's 8 rows over their visible keys, in key order.  The weights of a
// group of 4 keys are the same for every lane, so they come through scalar
// loads (the weight scratch is read-only here); V rows stream through per-lane
// loads, two groups ahead.  No LDS and no barriers.  Keys a row does not see
// contribute +0 (bitwise masks on the groups at the causal diagonal).
typedef float f8v __attribute__((ext_vector_type(8)));
typedef const __attribute__((address_space(4))) float cfloat_t;
typedef const __attribute__((address_space(4))) f8v cf8v_t;

constexpr int kPvKeys = 8;                                           // keys per group (one 32-byte scalar load per row)

// V values of keys k0 .. k0+7 for this lane (keys clamped to kend - 1).
template <int DPL>
__device__ __forceinline__ void pf_pv_vload(const float *Vh, int HD, int k0, int kend, float (&v)[kPvKeys][DPL]) {
#pragma unroll
  for (int u = 0; u < kPvKeys; u++) {
    const float *row = Vh + (size_t)min(k0 + u, kend - 1) * HD;
    if constexpr (DPL == 2) {
      const float2 t = *reinterpret_cast<const float2 *>(row);
      v[u][0] = t.x;
      v[u][1] = t.y;
    } else {
      v[u][0] = *row;
    }
  }
}

// The adds of one group: every key seen by every row (MASK false) or masked
// per (row, key) at the causal diagonal.
template <bool MASK, int DPL, int PR>
__device__ __forceinline__ void pf_pv_group(float (&acc)[PR][DPL], const float (&v)[kPvKeys][DPL],
                                          const f8v (&wv)[PR], int k0, int rlast0) {
#pragma unroll
  for (int u = 0; u < kPvKeys; u++) {
#pragma unroll
    for (int c = 0; c < PR; c++) {
      const float wk = wv[c][u];
#pragma unroll
      for (int e = 0; e < DPL; e++) {
        const float p = wk * v[u][e];
        acc[c][e] += MASK ? pv_mask(p, k0 + u <= rlast0 + c) : p;
      }
    }
  }
}

template <int HD, int PR>
__global__ __launch_bounds__(512) void k_pf_pv(const float *w, const float *vc, int R, int p0, int H, int KVH,
                                               int max_seq, int Tp, float *o) {
  static_assert(HD == 128 || HD <= 64, "two dims per lane at 128, one below");
  constexpr int DPL = HD == 128 ? 2 : 1;
  const int G = H / KVH;
  const int kvh = blockIdx.x, r0 = (gridDim.y - 1 - blockIdx.y) * PR;   // longest blocks first
  const int g = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6)), lane = threadIdx.x & 63;
  const int h = kvh * G + g;
  const int rend = min(R, r0 + PR);
  const int kend = p0 + rend;                                        // keys 0 .. kend-1 are used
  const int rlast0 = p0 + r0;                                        // last key row r0 sees
  const int dfirst = DPL * lane;
  const bool lane_ok = dfirst < HD;
  const float *Vh = vc + (size_t)kvh * max_seq * HD + (lane_ok ? dfirst : 0);
  cfloat_t *wr[PR];
#pragma unroll
  for (int c = 0; c < PR; c++) wr[c] = (cfloat_t *)(w + ((size_t)h * R + min(r0 + c, R - 1)) * Tp);
  const int klast = (kend - 1) / kPvKeys * kPvKeys;                  // group starts are clamped to it

  float acc[PR][DPL];
#pragma unroll
  for (int c = 0; c < PR; c++)
#pragma unroll
    for (int e = 0; e < DPL; e++) acc[c][e] = 0.0f;
  // three V register sets in rotation: group k in set k % 3, requested two
  // groups before it is added
  float v0[kPvKeys][DPL], v1[kPvKeys][DPL], v2[kPvKeys][DPL];
  f8v wv[PR];
  pf_pv_vload<DPL>(Vh, HD, 0, kend, v0);
  pf_pv_vload<DPL>(Vh, HD, min(kPvKeys, klast), kend, v1);
  auto run = [&](int k, const float (&v)[kPvKeys][DPL]) {
#pragma unroll
    for (int c = 0; c < PR; c++) wv[c] = *(cf8v_t *)(wr[c] + k);
    if (k + kPvKeys <= rlast0 + 1) pf_pv_group<false, DPL, PR>(acc, v, wv, k, rlast0);
    else pf_pv_group<true, DPL, PR>(acc, v, wv, k, rlast0);
  };
  for (int k0 = 0; k0 < kend; k0 += 3 * kPvKeys) {
    pf_pv_vload<DPL>(Vh, HD, min(k0 + 2 * kPvKeys, klast), kend, v2);
    run(k0, v0);
    if (k0 + kPvKeys >= kend) break;
    pf_pv_vload<DPL>(Vh, HD, min(k0 + 3 * kPvKeys, klast), kend, v0);
    run(k0 + kPvKeys, v1);
    if (k0 + 2 * kPvKeys >= kend) break;
    pf_pv_vload<DPL>(Vh, HD, min(k0 + 4 * kPvKeys, klast), kend, v1);
    run(k0 + 2 * kPvKeys, v2);
  }
  if (lane_ok) {
#pragma unroll
    for (int c = 0; c < PR; c++)
      if (r0 + c < R) {
        float *orow = o + (size_t)(r0 + c) * H * HD + (size_t)h * HD + dfirst;
        if constexpr (DPL == 2) *reinterpret_cast<float2 *>(orow) = make_float2(acc[c][0], acc[c][1]);
        else *orow = acc[c][0];
      }
  }
}

// Scores with the K row in registers: block (KV head, 16 query rows, 256 keys);
// lane t of wave v owns key j0 + 64v + t and holds its whole K row.  For every
// (head, row) pair of the block the dot over d is formed in order; 4 pairs go
// together (4 independent chains per lane), their q values wave-uniform in
// scalar registers, 8 dims per scalar load.  Waves whose keys are all past the
// block's last visible key stop at once; no LDS, no barriers.
constexpr int kPsKeys = 256, kPsRows = 16, kPsPairs = 4, kPsDims = 8;

// q of 8 dims of the 4 pairs into scalar registers, issued where it stands (asm,
// immediate offset D floats); scalar loads may return out of order, so the
// wait for a chunk is a full one.
template <int D>
__device__ __forceinline__ void ps_sload(f8v (&qq)[kPsPairs], cfloat_t *const (&qp)[kPsPairs]) {
#pragma unroll
  for (int u = 0; u < kPsPairs; u++) asm volatile("s_load_dwordx8 %0, %1, %2" : "=s"(qq[u]) : "s"(qp[u]), "i"(4 * D));
}

// The accumulators pass through the wait, so that the adds before it stay
// before it (and their q registers are free again).
__device__ __forceinline__ void ps_swait(f8v (&qq)[kPsPairs], float (&acc)[kPsPairs]) {
  asm volatile("s_waitcnt lgkmcnt(0)"
               : "+s"(qq[0]), "+s"(qq[1]), "+s"(qq[2]), "+s"(qq[3]), "+v"(acc[0]), "+v"(acc[1]), "+v"(acc[2]),
                 "+v"(acc[3]));
}

// Chunk D of the 4 chains (q already waited for in cur); the next chunk is
// requested before these adds and waited for after them.
template <int HD, int D>
__device__ __forceinline__ void ps_chunk(cfloat_t *const (&qp)[kPsPairs], const float (&k)[HD], float (&acc)[kPsPairs],
                                         f8v (&cur)[kPsPairs], f8v (&nxt)[kPsPairs]) {
  if constexpr (D + kPsDims < HD) ps_sload<D + kPsDims>(nxt, qp);
#pragma unroll
  for (int e = 0; e < kPsDims; e++)
#pragma unroll
    for (int u = 0; u < kPsPairs; u++) acc[u] += cur[u][e] * k[D + e];
  if constexpr (D + kPsDims < HD) {
    ps_swait(nxt, acc);
    ps_chunk<HD, D + kPsDims>(qp, k, acc, nxt, cur);
  }
}

template <int HD, int D>
__device__ __forceinline__ void ps_chunks(cfloat_t *const (&qp)[kPsPairs], const float (&k)[HD], float (&acc)[kPsPairs]) {
  f8v qa[kPsPairs], qb[kPsPairs];
  ps_sload<0>(qa, qp);
  ps_swait(qa, acc);
  ps_chunk<HD, 0>(qp, k, acc, qa, qb);
}

template <int HD, int RB>
__global__ __launch_bounds__(kPsKeys) void k_pf_scores(const float *q, const float *kc, int R, int p0, int H,
                                                         int KVH, int max_seq, float scale, float *w, int Tp) {
  static_assert(HD % kPsDims == 0, "whole scalar loads of q");
  const int kvh = blockIdx.x, r0 = blockIdx.y * RB, j0 = blockIdx.z * kPsKeys;
  const int G = H / KVH;
  const int rend = min(R, r0 + RB);
  const int jvis = p0 + rend - 1;                                    // last key any row here sees
  const int jw = j0 + 64 * __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  if (jw > jvis) return;                                             // uniform for the wave
  const int j = jw + (threadIdx.x & 63);
  float k[HD];
  {
    const float4 *kr = reinterpret_cast<const float4 *>(kc + ((size_t)kvh * max_seq + min(j, jvis)) * HD);
#pragma unroll
    for (int i = 0; i < HD / 4; i++) {
      const float4 t = kr[i];
      k[4 * i] = t.x; k[4 * i + 1] = t.y; k[4 * i + 2] = t.z; k[4 * i + 3] = t.w;
    }
  }
  const int npair = G * RB;
#pragma unroll 1
  for (int c0 = 0; c0 < npair; c0 += kPsPairs) {
    cfloat_t *qp[kPsPairs];
#pragma unroll
    for (int u = 0; u < kPsPairs; u++) {
      const int pair = c0 + u, g = pair / RB, r = min(r0 + pair % RB, R - 1);
      qp[u] = (cfloat_t *)(q + (size_t)r * H * HD + (size_t)(kvh * G + g) * HD);
    }
    float acc[kPsPairs];
#pragma unroll
    for (int u = 0; u < kPsPairs; u++) acc[u] = 0.0f;
    ps_chunks<HD, 0>(qp, k, acc);
#pragma unroll
    for (int u = 0; u < kPsPairs; u++) {
      const int pair = c0 + u, g = pair / RB, r = r0 + pair % RB;
      if (r < R && j <= p0 + r) w[((size_t)(kvh * G + g) * R + r) * Tp + j] = acc[u] * scale;
    }
  }
}

// Prompt attention with the products on the matrix cores.  A K = 1 fp32 MFMA
// with a zero accumulator, v_mfma_f32_32x32x1_2b_f32, forms two 32 x 32 outer
// products of 64-lane operands (lanes 32b .. 32b+31 give block b's rows and
// columns), each element a * b rounded once to nearest even: the bits of
// v_mul_f32, denormal and special results included, except that an exact -0
// product comes out +0 (+0 + -0 rounds to +0).  Sums that start at +0.0f never
// hold -0, so s + (+0) and s + (-0) are the same s and the sign cannot show.
// The reference's sums stay in order on the VALU: one v_add_f32 per product
// instead of a v_mul_f32 and a v_add_f32.
// Element r of lane l of the result: block b = r / 16, row i = 8 * (r % 16 / 4)
// + 4 * (l / 32) + r % 4, column l % 32.
// A block's 32 (query head, row) pairs: pair p is head g = p / rbq of the KV
// head's group and row r0 + p % rbq, rbq = 32 / G (pairs past G * rbq idle).
typedef float v32f __attribute__((ext_vector_type(32)));

__device__ __forceinline__ v32f mx_outer(float a, float b) {
  const v32f z = {};
  return __builtin_amdgcn_mfma_f32_32x32x1f32(a, b, z, 0, 0, 0);
}
__device__ __forceinline__ int mx_pair(int r, int lane) { return 8 * ((r & 15) >> 2) + 4 * (lane >> 5) + (r & 3); }

// Pair p < 32 to (head, row): p / rbq as (p * mg) >> 16 with mg = ceil(2^16 /
// rbq), exact for p < 32 and rbq <= 32 (the error p * (mg - 2^16 / rbq) / 2^16
// stays below 1 / rbq).
struct MxPairs {
  int rbq, mg;
  __device__ explicit MxPairs(int G) : rbq(32 / G), mg((65536 + 32 / G - 1) / (32 / G)) {}
  __device__ int head(int p) const { return (p * mg) >> 16; }
  __device__ int row(int p) const { return p - head(p) * rbq; }
};

// The two outer-product shapes, as a 64-lane wave sees them.  NP = 32:
// v_mfma_f32_32x32x1_2b_f32, lanes 32b + i give block b's row i and column i,
// result element r of lane l is block r / 16, row 8 * (r % 16 / 4) + 4 * (l /
// 32) + r % 4, column l % 32.  NP = 16: v_mfma_f32_16x16x1_4b_f32, lanes 16b + i
// give block b's row i and column i, element r of lane l is block r / 4, row
// 4 * (l / 16) + r % 4, column l % 16.  Every lane group supplies the same NP
// rows, so a tile is NP rows x 64 columns (column c from lane c).
template <int NP> struct MxShape;
template <> struct MxShape<32> {
  typedef v32f tile;
  __device__ static tile outer(float a, float b) { return mx_outer(a, b); }
  __device__ static int row(int r, int l) { return mx_pair(r, l); }
  __device__ static int col(int r, int l) { return 32 * (r >> 4) + (l & 31); }
};
typedef float v16f __attribute__((ext_vector_type(16)));
template <> struct MxShape<16> {
  typedef v16f tile;
  __device__ static tile outer(float a, float b) {
    const v16f z = {};
    return __builtin_amdgcn_mfma_f32_16x16x1f32(a, b, z, 0, 0, 0);
  }
  __device__ static int row(int r, int l) { return 4 * (l >> 4) + (r & 3); }
  __device__ static int col(int r, int l) { return 16 * (r >> 2) + (l & 15); }
};

// Scores: block (KV head, rbq rows, i.e. 32 pairs, 8 * NP keys) of four waves;
// wave v takes pairs NP * (v % (32 / NP)) .. +NP-1 and keys j0 + 64 * (v / (32 /
// NP)) .. +63 (lane l supplies key j0 + l, lane l % NP the pair) and forms the
// dots over d in order for its NP x 64 (pair, key) elements at once.  Each lane
// reads its q and K rows a whole 128-byte line at a time (32 dims), so a line
// is fetched once while it is in the L1.
// Held to 4 waves per SIMD (128 registers; 134 unbounded, i.e. 3 waves): the
// issue rate of a SIMD's MFMAs and adds rises with its waves (365 against 378
// us per layer at the 8B shape, 2048 rows).
template <int HD, int NP>
__global__ __launch_bounds__(256) __attribute__((amdgpu_waves_per_eu(4))) void k_pf_scores_mx(const float *q, const float *kc, int R, int p0, int H,
                                                      int KVH, int max_seq, float scale, float *w, int Tp) {
  typedef MxShape<NP> S;
  typedef typename S::tile tile;
  constexpr int CH = HD % 32 == 0 ? 32 : 16, NQ = CH / 4;           // dims per step, float4 loads per row
  static_assert(HD % CH == 0, "whole steps");
  const int kvh = blockIdx.x, G = H / KVH;
  const MxPairs P(G);
  const int r0 = blockIdx.y * P.rbq, rend = min(R, r0 + P.rbq);
  const int jvis = p0 + rend - 1;                                    // last key any row here sees
  const int lane = threadIdx.x & 63, wv_ = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int pb = NP * (wv_ % (32 / NP));
  const int jw = blockIdx.z * 8 * NP + 64 * (wv_ / (32 / NP));
  if (jw > jvis) return;                                             // uniform for the wave
  const int pa = pb + (lane & (NP - 1)), ga = min(P.head(pa), G - 1), ra = min(r0 + P.row(pa), R - 1);
  const float4 *qr = reinterpret_cast<const float4 *>(q + ((size_t)ra * H + kvh * G + ga) * HD);
  const float4 *kr = reinterpret_cast<const float4 *>(kc + ((size_t)kvh * max_seq + min(jw + lane, jvis)) * HD);
  tile s = {};
  auto add = [&](float a, float b) {
    s += S::outer(a, b);
    __builtin_amdgcn_sched_barrier(0);                               // one product tile live at a time
  };
#pragma unroll 1
  for (int c = 0; c < HD / 4; c += NQ) {
    float4 qa[NQ], kb[NQ];
#pragma unroll
    for (int i = 0; i < NQ; i++) {
      qa[i] = qr[c + i];
      kb[i] = kr[c + i];
    }
#pragma unroll
    for (int i = 0; i < NQ; i++) {
      add(qa[i].x, kb[i].x);
      add(qa[i].y, kb[i].y);
      add(qa[i].z, kb[i].z);
      add(qa[i].w, kb[i].w);
    }
  }
#pragma unroll
  for (int r = 0; r < NP; r++) {
    const int p = pb + S::row(r, lane), g = P.head(p), row = r0 + p - g * P.rbq, j = jw + S::col(r, lane);
    if (g < G && row < R && j <= p0 + row) w[((size_t)(kvh * G + g) * R + row) * Tp + j] = s[r] * scale;
  }
}

// PV: block (KV head, rbq rows, i.e. 32 pairs); wave v takes pairs NP * (v % (32
// / NP)) .. +NP-1 and dims 64 * (v / (32 / NP)) .. +63 (lane l supplies dim
// d0 + l, lane l % NP the pair); for every key t in order the products
// w[pair][t] * V[t][d] of the wave's NP x 64 elements are added at once (NP
// adds a lane per key: with NP = 16 the longest rows' waves, which bound the
// kernel, carry half the adds of NP = 32).  Keys up to the block's first row's
// last are seen by every pair: they go 8 a chunk, one chunk in flight while the
// other is added.  Past them (at most rbq - 1 + 7 keys) a pair whose row ends
// before t supplies a zero weight, so its products are +-0 and its sums do not
// move; should such a key's V value not be finite (0 * inf is NaN), that key
// masks the products element by element instead.
template <int HD, int NP>
__global__ __launch_bounds__(64 * (32 / NP) * ((HD + 63) / 64)) __attribute__((amdgpu_waves_per_eu(4))) void k_pf_pv_mx(
    const float *w, const float *vc, int R, int p0, int H, int KVH, int max_seq, int Tp, float *o) {
  typedef MxShape<NP> S;
  typedef typename S::tile tile;
  constexpr int NE = NP;                                             // tile elements per lane
  const int kvh = blockIdx.x, G = H / KVH;
  const MxPairs P(G);
  const int r0 = (gridDim.y - 1 - blockIdx.y) * P.rbq;              // longest blocks first
  const int rend = min(R, r0 + P.rbq);
  const int lane = threadIdx.x & 63, wv_ = __builtin_amdgcn_readfirstlane((int)(threadIdx.x >> 6));
  const int pb = NP * (wv_ % (32 / NP)), d0 = 64 * (wv_ / (32 / NP));
  const int kall = p0 + r0 + 1, kend = p0 + rend;                   // keys every row sees / any row sees
  const int k8 = kall & ~7;
  const int pa = pb + (lane & (NP - 1)), ga = min(P.head(pa), G - 1), prow = P.row(pa), ra = min(r0 + prow, R - 1);
  const float *wr = w + ((size_t)(kvh * G + ga) * R + ra) * Tp;
  const float *vr = vc + (size_t)kvh * max_seq * HD + min(d0 + lane, HD - 1);
  tile s = {};
  auto add = [&](float a, float b) {
    s += S::outer(a, b);
    __builtin_amdgcn_sched_barrier(0);                               // one product tile live at a time
  };
  if (k8 > 0) {
    float4 xa0 = *reinterpret_cast<const float4 *>(wr), xa1 = *reinterpret_cast<const float4 *>(wr + 4);
    float xb[8], yb[8];
    float4 ya0, ya1;
#pragma unroll
    for (int u = 0; u < 8; u++) xb[u] = vr[u * HD];
    for (int t = 0; t < k8; t += 16) {
      const int ty = min(t + 8, k8 - 8);
      ya0 = *reinterpret_cast<const float4 *>(wr + ty);
      ya1 = *reinterpret_cast<const float4 *>(wr + ty + 4);
#pragma unroll
      for (int u = 0; u < 8; u++) yb[u] = vr[(size_t)(ty + u) * HD];
      __builtin_amdgcn_sched_barrier(0);                             // the requests go out before the adds
      add(xa0.x, xb[0]); add(xa0.y, xb[1]); add(xa0.z, xb[2]); add(xa0.w, xb[3]);
      add(xa1.x, xb[4]); add(xa1.y, xb[5]); add(xa1.z, xb[6]); add(xa1.w, xb[7]);
      if (t + 8 >= k8) break;
      const int tx = min(t + 16, k8 - 8);
      xa0 = *reinterpret_cast<const float4 *>(wr + tx);
      xa1 = *reinterpret_cast<const float4 *>(wr + tx + 4);
#pragma unroll
      for (int u = 0; u < 8; u++) xb[u] = vr[(size_t)(tx + u) * HD];
      __builtin_amdgcn_sched_barrier(0);
      add(ya0.x, yb[0]); add(ya0.y, yb[1]); add(ya0.z, yb[2]); add(ya0.w, yb[3]);
      add(ya1.x, yb[4]); add(ya1.y, yb[5]); add(ya1.z, yb[6]); add(ya1.w, yb[7]);
    }
  }
  // the rest (past the first row's last key the keys are masked per pair), 8
  // keys a batch: a pair whose row ends before a key supplies a zero weight, and
  // past the last key the V value is zero too; a batch with a masked key whose
  // V value is not finite goes key by key instead, each product masked
#pragma unroll 1
  for (int t0 = k8; t0 < kend; t0 += 8) {
    float wv[8], vv[8];
    bool bad = false;
#pragma unroll
    for (int u = 0; u < 8; u++) {
      const int t = min(t0 + u, kend - 1), dt = t0 + u - (p0 + r0);
      const bool seen = t0 + u < kend;
      wv[u] = seen && dt <= prow ? wr[t] : 0.0f;
      vv[u] = seen ? vr[(size_t)t * HD] : 0.0f;
      bad |= seen && dt > 0 && !__builtin_isfinite(vv[u]);
    }
    if (!__any(bad)) {
#pragma unroll
      for (int u = 0; u < 8; u++) add(wv[u], vv[u]);
    } else {
#pragma unroll 1
      for (int t = t0; t < min(t0 + 8, kend); t++) {
        const int dt = t - (p0 + r0);
        const tile pr = S::outer(wr[t], vr[(size_t)t * HD]);
#pragma unroll
        for (int r = 0; r < NE; r++) {
          s[r] += dt <= 0 || P.row(pb + S::row(r, lane)) >= dt ? pr[r] : 0.0f;
          __builtin_amdgcn_sched_barrier(0);                         // each row test next to its add
        }
      }
    }
  }
#pragma unroll
  for (int r = 0; r < NE; r++) {
    const int p = pb + S::row(r, lane), g = P.head(p), row = r0 + p - g * P.rbq, d = d0 + S::col(r, lane);
    if (g < G && row < R && d < HD) o[((size_t)row * H + kvh * G + g) * HD + d] = s[r];
  }
}

// 1: prompt attention on the VALU-only kernels (k_pf_scores / k_pf_pv), the
// products as v_mul_f32; 0: the outer-product kernels (the same bits).  Read from
// QLLAMA_PF_VALU at the first call; qllama_test_pf_valu sets it.
int g_pf_valu = -1;

bool pf_use_valu() {
  if (g_pf_valu < 0) g_pf_valu = getenv("QLLAMA_PF_VALU") != NULL;
  return g_pf_valu != 0;
}

template <int HD>
int pf_attention(const float *q, const float *kc, const float *vc, int R, int p0, int H, int KVH, int max_seq,
                 float scale, float *w, float *o) {
  if (!pf_use_valu()) {
    const int G = H / KVH, Tp = (max_seq + 7) & ~7, rbq = 32 / G;         // rows of a pair block
    const int nrb = (R + rbq - 1) / rbq;
    const dim3 sgrid(KVH, nrb, (p0 + R + 255) / 256);
    QH_LAUNCH(QK_PF_ATTN, (k_pf_scores_mx<HD, 32>), sgrid, dim3(256), 0, q, kc, R, p0, H, KVH, max_seq, scale, w, Tp);
    if (pf_softmax_rows(w, R, p0, Tp, H)) return 1;
    QH_LAUNCH(QK_PF_ATTN, (k_pf_pv_mx<HD, 16>), dim3(KVH, nrb), dim3(128 * ((HD + 63) / 64)), 0, w, vc, R, p0, H,
              KVH, max_seq, Tp, o);
    return 0;
  }
  const int G = H / KVH, Tp = (max_seq + 7) & ~7;          // rows of whole 32-byte words
  const int Tmax = p0 + R;
  // short prompts: half the rows per block, twice the waves (the per-row sums
  // do not depend on how rows are grouped into blocks)
  const bool small = R <= QLLAMA_PF_SMALL_ROWS;
  const int rbs = small ? kPsRows / 2 : kPsRows, rbp = small ? kPvRows / 2 : kPvRows;
  const dim3 sgrid(KVH, (R + rbs - 1) / rbs, (Tmax + kPsKeys - 1) / kPsKeys);
  if (small) QH_LAUNCH(QK_PF_ATTN, (k_pf_scores<HD, kPsRows / 2>), sgrid, dim3(kPsKeys), 0, q, kc, R, p0, H, KVH, max_seq, scale, w, Tp);
  else QH_LAUNCH(QK_PF_ATTN, (k_pf_scores<HD, kPsRows>), sgrid, dim3(kPsKeys), 0, q, kc, R, p0, H, KVH, max_seq, scale, w, Tp);
  if (pf_softmax_rows(w, R, p0, Tp, H)) return 1;
  const dim3 pgrid(KVH, (R + rbp - 1) / rbp);
  if (small) QH_LAUNCH(QK_PF_ATTN, (k_pf_pv<HD, kPvRows / 2>), pgrid, dim3(64 * G), 0, w, vc, R, p0, H, KVH, max_seq, Tp, o);
  else QH_LAUNCH(QK_PF_ATTN, (k_pf_pv<HD, kPvRows>), pgrid, dim3(64 * G), 0, w, vc, R, p0, H, KVH, max_seq, Tp, o);
  return 0;
}

size_t g_pv_attr_bytes[2] = {0, 0};   // dynamic LDS the PV kernels are currently allowed

// (16 bytes more than the weights and tiles take: the array starts on the first
// 16-byte boundary past the static variables)
size_t pv_lds_bytes(int max_seq) {
  return ((size_t)(max_seq + kTile - 1) / kTile * kTile + kPBuf * kChains * kTS) * 4 + 16;
}

}  // namespace

namespace {
template <bool ROPE, bool DIVW = false>
int attention(const float *q, float *kc, float *vc, const int *d_pos, int n_heads, int n_kv, int hd, int max_seq,
              float scale, const float *cos_t, const float *sin_t, float *scores, float *o, float *obm) {
  const int nch = (max_seq + kScoreBlock - 1) / kScoreBlock;
  float *bmax = scores + (size_t)n_heads * max_seq;
  const size_t pv_lds = pv_lds_bytes(max_seq);
  if (max_seq > kPvThreads * 32 || pv_lds + sizeof(qd::SeqScratch) + 1024 > 160 * 1024)
    return qh::fail_msg("attention: max_seq too large for the LDS-resident weights");
  if ((long long)max_seq * hd >= (1LL << 27))      // V byte offsets (plus prefetch) stay below 2^30
    return qh::fail_msg("attention: KV head region too large");
  if (pv_lds > 64 * 1024 && pv_lds > g_pv_attr_bytes[DIVW]) {
    hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void *>(k_attn_pv<DIVW>),
                                       hipFuncAttributeMaxDynamicSharedMemorySize, (int)pv_lds);
    if (e != hipSuccess) return qh::fail("hipFuncSetAttribute(k_attn_pv)", e);
    g_pv_attr_bytes[DIVW] = pv_lds;
  }
  const int G = n_heads / n_kv;
  if (G > 8 || G * kScoreBlock > 1024 || G * hd > 512 * 8)      // qs holds 8 query heads
    return qh::fail_msg("attention: more than 8 query heads per KV head");
  if (hd > 512 || (hd & 1)) return qh::fail_msg("attention: head_dim must be even and at most 512");
  const dim3 sgrid(n_kv, nch);
  const dim3 sblock(G * kScoreBlock);
  switch (hd) {
    case 128:
      QH_LAUNCH(QK_ATTN, (k_attn_scores<128, ROPE>), sgrid, sblock, 0, q, kc, vc, d_pos, n_heads, n_kv, hd, max_seq,
                scale, scores, bmax, nch, cos_t, sin_t);
      break;
    default:
      QH_LAUNCH(QK_ATTN, (k_attn_scores<0, ROPE>), sgrid, sblock, 0, q, kc, vc, d_pos, n_heads, n_kv, hd, max_seq,
                scale, scores, bmax, nch, cos_t, sin_t);
      break;
  }
  QH_LAUNCH(QK_ATTN_PV, k_attn_pv<DIVW>, dim3(n_heads, (hd + kChains - 1) / kChains), dim3(kPvThreads), pv_lds, scores,
            bmax, vc, d_pos, n_heads, n_kv, hd, max_seq, nch, o, obm);
  return 0;
}
}  // namespace

extern "C" int qhip_attention(const float *q, const float *kc, const float *vc, const int *d_pos, int n_heads,
                              int n_kv, int hd, int max_seq, float scale, float *scores, float *o, float *obm) {
  return attention<false>(q, const_cast<float *>(kc), const_cast<float *>(vc), d_pos, n_heads, n_kv, hd, max_seq,
                          scale, nullptr, nullptr, scores, o, obm);
}

extern "C" int qhip_attention_rope(const float *qkv, float *kc, float *vc, const int *d_pos, int n_heads, int n_kv,
                                   int hd, int max_seq, float scale, const float *cos_t, const float *sin_t,
                                   float *scores, float *o, float *obm) {
  return attention<true>(qkv, kc, vc, d_pos, n_heads, n_kv, hd, max_seq, scale, cos_t, sin_t, scores, o, obm);
}

// ---- the attention half of a decode layer in one launch (k_attn_layer) ----
namespace {
int g_ly_probe = -1;          // -1: not probed yet; 1: 32 * 8 blocks land on XCD (block % 8)
size_t g_ly_attr[4] = {0, 0, 0, 0};   // dynamic LDS allowed per instantiation (hd 64/128 x kpad 2048/4096)
constexpr size_t kLyLds = 96 * 1024;   // dynamic LDS: the K rows (64 KB) or the PV weights and tiles; with
                                       // the static arrays more than half of a CU's LDS: one block per CU
constexpr size_t kLyLdsLaunch = kLyLds + 16;   // room to start the array on a 16-byte boundary
}  // namespace

// Whether a launch of 32 * 8 blocks puts block b on XCD (s + b) % 8 for one
// start s, so that every XCD runs 32 blocks with distinct ranks b / 8 (what
// k_attn_layer assumes).  Probed once, with one small launch; call outside
// graph capture.
extern "C" int qhip_attn_layer_probe(void) {
  if (g_ly_probe >= 0) return g_ly_probe;
  g_ly_probe = 0;
  constexpr int n = kLyNB * 8;
  if (qh::num_cus() < n) return 0;
  unsigned *d = nullptr, h[n];
  if (hipMalloc(&d, n * sizeof(unsigned)) != hipSuccess) { (void)hipGetLastError(); return 0; }
  hipLaunchKernelGGL(k_xcc_probe, dim3(n), dim3(64), 0, qh::stream(), d);
  bool ok = hipGetLastError() == hipSuccess &&
            hipMemcpyAsync(h, d, sizeof h, hipMemcpyDeviceToHost, qh::stream()) == hipSuccess &&
            hipStreamSynchronize(qh::stream()) == hipSuccess;
  (void)hipFree(d);
  for (int b = 0; ok && b < n; b++) ok = h[b] < 8u && (h[b] + 8u - (unsigned)(b % 8)) % 8u == (h[0] + 8u) % 8u;
  g_ly_probe = ok ? 1 : 0;
  return g_ly_probe;
}

// Shapes k_attn_layer serves: 8 KV heads (one per XCD), at most 4 query heads
// per KV head, head_dim 128 or 64, kpad 2048 or 4096, max_seq <= 4096, and a device
// with the 256 CUs its blocks need at once.
extern "C" int qhip_attn_layer_ok(int n_heads, int n_kv, int hd, int kpad, int max_seq) {
  if (n_kv != 8 || n_heads % n_kv || (hd != 128 && hd != 64) || (kpad != 2048 && kpad != 4096)) return 0;
  const int G = n_heads / n_kv;
  if (G < 1 || G > 4 || (G + 2) * hd % kLyNB || (G + 2) * hd / kLyNB > kLyRW * ly_rows_per_wave(hd)) return 0;
  if (G * ((hd + kChains - 1) / kChains) > kLyNB || max_seq > kLyNB * kLyKRows) return 0;
  if (pv_lds_bytes(max_seq) > kLyLds || (size_t)kLyKRows * hd * 4 > kLyLds) return 0;
  return qh::num_cus() >= kLyNB * n_kv && qhip_attn_layer_probe() == 1;
}

// Scratch of k_attn_layer: floats (the exchanged QKV outputs and block maxima),
// and 32-bit words of meeting counters and error flag, zero before first use.
extern "C" size_t qhip_attn_layer_scratch(int n_heads, int n_kv, int hd) {
  return (size_t)n_kv * (n_heads / n_kv + 2) * hd + (size_t)n_heads * kLyNB;
}
extern "C" size_t qhip_attn_layer_sync_words(int n_kv) { return (size_t)2 * 64 * n_kv + 64; }

extern "C" int qhip_attn_layer(const float *x, const float *gain, float eps, int dm, const int8_t *W,
                               const float *ws, const float *bias, int kpad, float *kc, float *vc, const int *d_pos,
                               int n_heads, int n_kv, int hd, int max_seq, float scale, const float *cos_t,
                               const float *sin_t, float *scores, float *scratch, unsigned *sync, float *o,
                               float *obm) {
  if (!qhip_attn_layer_ok(n_heads, n_kv, hd, kpad, max_seq) || dm > kpad || dm + 15 < kpad)
    return qh::fail_msg("attn_layer: unsupported shape");
  const int G = n_heads / n_kv;
  float *qx = scratch, *bmax = scratch + (size_t)n_kv * (G + 2) * hd;
  const int kch = kpad / 1024, v = (hd == 128 ? 2 : 0) + (kch == 4 ? 1 : 0);
  const void *fns[4] = {reinterpret_cast<const void *>(k_attn_layer<64, 2>),
                        reinterpret_cast<const void *>(k_attn_layer<64, 4>),
                        reinterpret_cast<const void *>(k_attn_layer<128, 2>),
                        reinterpret_cast<const void *>(k_attn_layer<128, 4>)};
  if (g_ly_attr[v] < kLyLdsLaunch) {
    hipError_t e = hipFuncSetAttribute(fns[v], hipFuncAttributeMaxDynamicSharedMemorySize, (int)kLyLdsLaunch);
    if (e != hipSuccess) return qh::fail("hipFuncSetAttribute(k_attn_layer)", e);
    g_ly_attr[v] = kLyLdsLaunch;
  }
#define LY_LAUNCH(HD_, KCH_)                                                                                      \
  QH_LAUNCH(QK_ATTN_LAYER, (k_attn_layer<HD_, KCH_>), dim3(kLyNB * n_kv), dim3(kLyThreads), kLyLdsLaunch, x, gain, \
            eps, dm, W, ws, bias, kpad, kc, vc, d_pos, n_heads, n_kv, max_seq, scale, cos_t, sin_t, scores, bmax, qx,  \
            sync, o, obm)
  switch (v) {
    case 0: LY_LAUNCH(64, 2); break;
    case 1: LY_LAUNCH(64, 4); break;
    case 2: LY_LAUNCH(128, 2); break;
    default: LY_LAUNCH(128, 4); break;
  }
#undef LY_LAUNCH
  return 0;
}

// The k_attn_layer error flag since the sync words were zeroed: 0 none, 1 a
// meeting timed out (blocks not resident at once, or an XCD given other than
// 32 blocks), 2 an XCC id past 7, -1 the flag could not be read (synchronizes
// the stream).
extern "C" int qhip_attn_layer_failed(const unsigned *sync, int n_kv) {
  unsigned e = 0;
  if (hipMemcpyAsync(&e, sync + 2 * 64 * n_kv, sizeof e, hipMemcpyDeviceToHost, qh::stream()) != hipSuccess ||
      hipStreamSynchronize(qh::stream()) != hipSuccess)
    return -1;
  return (int)e;
}

// GPT-2's decode attention (model.c:485-504): as qhip_attention (q given, row
// *d_pos already cached) with the weights formed as e_j / sum.
extern "C" int qhip_attention_div(const float *q, const float *kc, const float *vc, const int *d_pos, int n_heads,
                                  int n_kv, int hd, int max_seq, float scale, float *scores, float *o) {
  return attention<false, true>(q, const_cast<float *>(kc), const_cast<float *>(vc), d_pos, n_heads, n_kv, hd, max_seq,
                                scale, nullptr, nullptr, scores, o, nullptr);
}

// Number of per-block maxima qhip_attention writes to obm.
extern "C" int qhip_attention_nbm(int n_heads, int hd) { return n_heads * ((hd + kChains - 1) / kChains); }

// Size (floats) of the scores scratch qhip_attention needs.
extern "C" size_t qhip_attention_scratch(int n_heads, int max_seq) {
  return (size_t)n_heads * max_seq + (size_t)n_heads * ((max_seq + kScoreBlock - 1) / kScoreBlock);
}

// Rows per attention pass: as many as the scratch budget holds (whole prompts of
// the model shapes here: 2048 rows at the 8B shape take 671 MB), so that every
// kernel of the pass has work for the whole chip.
static int pf_pass_rows(int R, int n_heads, int max_seq) {
  const size_t row_bytes = (size_t)n_heads * (size_t)((max_seq + 7) & ~7) * 4;
  size_t cap = kPfScratchBytes / row_bytes;
  if (cap < 64) cap = 64;
  cap -= cap % 16;
  return R < (int)cap ? R : (int)cap;
}

// Causal attention of R prompt rows (R may exceed one pass: rows are taken
// pf_pass_rows at a time, each pass seeing every earlier position).
extern "C" int qhip_pf_attention(const float *q, const float *kc, const float *vc, int R, int p0, int n_heads,
                                 int n_kv, int hd, int max_seq, float scale, float *ws, float *o) {
  const int G = n_heads / n_kv;
  if (G < 1 || G > 8 || G * hd > 1024) return qh::fail_msg("pf_attention: unsupported head grouping");
  if (p0 + R > max_seq || max_seq > 16384) return qh::fail_msg("pf_attention: positions out of range");
  const int pass = pf_pass_rows(R, n_heads, max_seq);
  for (int c0 = 0; c0 < R; c0 += pass) {
    const int rr = min(pass, R - c0);
    const float *qc = q + (size_t)c0 * n_heads * hd;
    float *oc = o + (size_t)c0 * n_heads * hd;
    int rc;
    switch (hd) {
      case 128: rc = pf_attention<128>(qc, kc, vc, rr, p0 + c0, n_heads, n_kv, max_seq, scale, ws, oc); break;
      case 64: rc = pf_attention<64>(qc, kc, vc, rr, p0 + c0, n_heads, n_kv, max_seq, scale, ws, oc); break;
      case 48: rc = pf_attention<48>(qc, kc, vc, rr, p0 + c0, n_heads, n_kv, max_seq, scale, ws, oc); break;
      default: return qh::fail_msg("pf_attention: head_dim not supported");
    }
    if (rc) return rc;
  }
  return 0;
}

// Test hook: 1 puts prompt attention on the VALU-only kernels, 0 on the
// outer-product kernels, for the rest of the process (both give the same bits).
extern "C" int qllama_test_pf_valu(int on) {
  g_pf_valu = on ? 1 : 0;
  return 0;
}

// Floats of scratch qhip_pf_attention needs.
extern "C" size_t qhip_pf_attention_scratch(int R, int n_heads, int max_seq) {
  return (size_t)n_heads * (size_t)pf_pass_rows(R, n_heads, max_seq) * (size_t)((max_seq + 7) & ~7);
}
