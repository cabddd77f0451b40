// k_fattn.hip - split-K decode attention with an online-softmax merge: the
// attention of the fast decode mode (llama.c:554-576, gqa.c:16-50 semantics;
// only the order of the floating-point sums differs from the reference).
//
// The exact path (k_attn.hip) forms every sum in the reference's order, which
// serialises the softmax denominator and the sum of w_j * V_j over positions.
// Here positions are split into chunks of C rows that run in parallel:
//
//   * grid: one block per (KV head, chunk) -- KVH x ceil(max_seq / C) blocks;
//     blocks whose chunk starts past the current position exit at once.  Block
//     x serves KV head x % KVH, so consecutive KV heads land on different XCDs
//     and a head's chunks share one.  A block serves the G query heads of its KV
//     head, so every K and V row is read from HBM once per token.
//   * a row of hd floats is spread over hd/4 lanes (16-byte loads, two rows per
//     wave instruction at hd 128, four at hd 64 and 48), so every load is
//     coalesced; the V rows of the first batch are requested together with the
//     K rows, so both streams are in flight at once.
//   * per chunk and head: s_j = (q . K_j) * scale (a lane-group reduction per
//     row), m = max_j s_j, e_j = expf(s_j - m), l = sum_j e_j and the
//     unnormalised o = sum_j e_j V_j go to the chunk's scratch slot.
//   * a second launch merges the chunks, one block per query head:
//     M = max_c m_c, w_c = expf(m_c - M), o = (sum_c w_c o_c) * (1 / sum_c w_c l_c),
//     and records max |o| per head, which the Wo GEMV's activation quantizer
//     reads.  (Merging inside the first launch, by the last block of a KV head
//     to finish, needs a device-scope release per block: an L2 write-back,
//     which cost more than the second launch.)
//
// With ROPE, q, k and v of the current position arrive unrotated (the QKV
// GEMV's output); every block rotates its G query heads with the host-built
// table (rope.c:48-68), and the block holding the current position rotates k,
// appends k and v to the cache (llama.c:551-552) and uses them from LDS.
//
// Every reduction has a fixed shape, so a result does not vary from run to run.
#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

constexpr int kFaThreads = 256;
constexpr int kFaWaves = kFaThreads / 64;
constexpr int kFaMaxChunk = 256;       // positions per block at most
constexpr int kFaMaxSplits = 256;      // chunks per KV head at most
constexpr int kFaBatch = 8;            // row loads in flight per lane and stream

template <int HD>
struct FaGeo {
  static constexpr int LPR = HD > 64 ? 32 : 16;    // lanes per row
  static constexpr int NV = HD / 4;                // lanes of a row that hold data (float4 each)
  static constexpr int RPW = 64 / LPR;             // rows per wave instruction
  static constexpr int RPR = RPW * kFaWaves;       // rows per block round
  static_assert(HD % 4 == 0 && NV <= LPR, "row must fit one lane group");
};

template <int CTRL>
__device__ __forceinline__ float dpp_f(float v) {
  return __int_as_float(__builtin_amdgcn_update_dpp(0, __float_as_int(v), CTRL, 0xf, 0xf, false));
}

// Sum over each group of LPR lanes (16 or 32); every lane of the group gets the
// same bits (each step adds a value to its partner's, and float addition is
// commutative).
template <int LPR>
__device__ __forceinline__ float group_sum(float v) {
  v += dpp_f<0xB1>(v);      // quad_perm [1,0,3,2]
  v += dpp_f<0x4E>(v);      // quad_perm [2,3,0,1]
  v += dpp_f<0x141>(v);     // row_half_mirror
  v += dpp_f<0x140>(v);     // row_mirror
  if (LPR == 32) v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));   // lane ^ 16
  return v;
}

typedef float v4f __attribute__((ext_vector_type(4)));

__device__ __forceinline__ float4 f4_zero() { return make_float4(0.0f, 0.0f, 0.0f, 0.0f); }

__device__ __forceinline__ float4 fma4(float e, const float4 &v, const float4 &a) {
  return make_float4(__builtin_fmaf(e, v.x, a.x), __builtin_fmaf(e, v.y, a.y), __builtin_fmaf(e, v.z, a.z),
                     __builtin_fmaf(e, v.w, a.w));
}

__device__ __forceinline__ float dot4(const float4 &a, const float4 &b) {
  return __builtin_fmaf(a.w, b.w, __builtin_fmaf(a.z, b.z, __builtin_fmaf(a.y, b.y, a.x * b.x)));
}

// Heads of a group padded to whole 16-byte words, so that one row's weights
// for every head come with one or two LDS reads.
template <int G>
constexpr int fa_gp() { return (G + 3) / 4 * 4; }

template <int G, int HD>
struct FaLds {
  float qs[G * HD];                    // the group's (rotated) queries
  float kcur[HD], vcur[HD];            // the current position's k (rotated) and v
  float sc[(kFaMaxChunk + 32) * fa_gp<G>()];   // scores, then e_j, [row][head] (0 past the chunk)
  float ro[kFaWaves * G * HD];         // per-wave partial o
  float sm[G], sl[G];                  // chunk max and sum by head
};

// part layout (floats): m [KVH][nsmax][G], l [KVH][nsmax][G], o [KVH][nsmax][G][HD]
template <int HD, int G, bool ROPE>
__global__ __launch_bounds__(kFaThreads) void k_fattn(const float *qkv, float *kc, float *vc, const int *d_pos, int H,
                                                      int KVH, int max_seq, int chunk, int nsmax, float scale,
                                                      const float *cos_t, const float *sin_t, float *part) {
  using Geo = FaGeo<HD>;
  constexpr int LPR = Geo::LPR, NV = Geo::NV, RPW = Geo::RPW, RPR = Geo::RPR;
  __shared__ __attribute__((aligned(16))) FaLds<G, HD> S;
  const int kvh = blockIdx.x % KVH, split = blockIdx.x / KVH;
  const int pos = *d_pos, T = pos + 1;
  const int s0 = split * chunk;
  if (s0 >= T) return;                                   // uniform for the block
  const int n = min(chunk, T - s0);
  const bool holds_pos = s0 + n == T;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int c = lane % LPR, rsub = lane / LPR;
  const bool cok = c < NV;
  const int half = HD / 2;
  // Loads of K and V rows go through buffer resources over this KV head's rows
  // [0, max_seq): a row outside the chunk (or the current row, which comes from
  // LDS) gets an offset past the end and reads as 0 without memory traffic, so
  // every lane issues the same loads and the compiler can count them.
  const __amdgpu_buffer_rsrc_t krs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(kc + (size_t)kvh * max_seq * HD), (short)0, max_seq * HD * 4, 0x00020000);
  const __amdgpu_buffer_rsrc_t vrs = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(vc + (size_t)kvh * max_seq * HD), (short)0, max_seq * HD * 4, 0x00020000);
  // rows of this lane: round b covers row b*RPR + wave*RPW + rsub of the chunk
  const int nround = (n + RPR - 1) / RPR;
  const int rlane = wave * RPW + rsub;
  auto row_pos = [&](int b) { return s0 + b * RPR + rlane; };
  auto row_off = [&](int b) {
    const int j = row_pos(b);
    const bool ok = cok && b * RPR + rlane < n && !(ROPE && j == pos);
    return ok ? (j * HD + 4 * c) * 4 : 0x7ffffff0;
  };
  auto load4 = [&](__amdgpu_buffer_rsrc_t rs, int off) {
    const v4f t = __builtin_bit_cast(v4f, __builtin_amdgcn_raw_buffer_load_b128(rs, off, 0, 0));
    return make_float4(t.x, t.y, t.z, t.w);
  };

  // A. requests in order of need: the group's q (and the current k, v), then
  // the first batch of K rows, then of V rows
  constexpr int QP = (G * HD / 2 + kFaThreads - 1) / kFaThreads;    // q pairs per thread
  float qx1[QP], qx2[QP], qc[QP], qsn[QP];
  float kx1 = 0.0f, kx2 = 0.0f, kcs = 0.0f, ksn = 0.0f, vx = 0.0f;
  const float *ct = ROPE ? cos_t + (size_t)pos * half : nullptr, *st = ROPE ? sin_t + (size_t)pos * half : nullptr;
  if (ROPE) {
#pragma unroll
    for (int u = 0; u < QP; u++) {
      const int i = tid + u * kFaThreads;
      if (i < G * half) {
        const int g = i / half, k = i % half;
        const float *xh = qkv + (size_t)(kvh * G + g) * HD;
        qx1[u] = xh[k]; qx2[u] = xh[k + half]; qc[u] = ct[k]; qsn[u] = st[k];
      }
    }
    if (holds_pos) {
      const float *kh = qkv + (size_t)(H + kvh) * HD, *vh = qkv + (size_t)(H + KVH + kvh) * HD;
      if (tid < half) { kx1 = kh[tid]; kx2 = kh[tid + half]; kcs = ct[tid]; ksn = st[tid]; }
      if (tid < HD) vx = vh[tid];
    }
  }
  float4 kr[kFaBatch], vr[kFaBatch];
#pragma unroll
  for (int b = 0; b < kFaBatch; b++) kr[b] = load4(krs, b < nround ? row_off(b) : 0x7ffffff0);
#pragma unroll
  for (int b = 0; b < kFaBatch; b++) vr[b] = load4(vrs, b < nround ? row_off(b) : 0x7ffffff0);

  // the group's query heads into LDS (rotated when ROPE); the current k, v
  if (ROPE) {
#pragma unroll
    for (int u = 0; u < QP; u++) {
      const int i = tid + u * kFaThreads;
      if (i < G * half) {
        const int g = i / half, k = i % half;
        S.qs[g * HD + k] = qx1[u] * qc[u] - qx2[u] * qsn[u];
        S.qs[g * HD + k + half] = qx2[u] * qc[u] + qx1[u] * qsn[u];
      }
    }
    if (holds_pos) {
      float *kdst = kc + ((size_t)kvh * max_seq + pos) * HD, *vdst = vc + ((size_t)kvh * max_seq + pos) * HD;
      if (tid < half) {
        const float y1 = kx1 * kcs - kx2 * ksn, y2 = kx2 * kcs + kx1 * ksn;
        S.kcur[tid] = y1;
        S.kcur[tid + half] = y2;
        kdst[tid] = y1;
        kdst[tid + half] = y2;
      }
      if (tid < HD) {
        S.vcur[tid] = vx;
        vdst[tid] = vx;
      }
    }
  } else {
    for (int i = tid; i < G * HD; i += kFaThreads) S.qs[i] = qkv[(size_t)kvh * G * HD + i];
  }
  qd::lds_sync();                                        // the K and V rows stay in flight
  float4 qf[G];
#pragma unroll
  for (int g = 0; g < G; g++) qf[g] = cok ? *reinterpret_cast<const float4 *>(&S.qs[g * HD + 4 * c]) : f4_zero();

  // 1. scores (the current row, which reads as 0 from the cache, is formed
  // after the loop from LDS by every lane group and stored by its owner)
  constexpr int GP = fa_gp<G>();
  auto store_scores = [&](const float4 &k, int r) {
    float d[GP];
#pragma unroll
    for (int g = 0; g < GP; g++) d[g] = g < G ? group_sum<LPR>(dot4(qf[g], k)) * scale : 0.0f;
    if (c == 0 && r < n) {
#pragma unroll
      for (int g = 0; g < GP; g += 4)
        *reinterpret_cast<float4 *>(&S.sc[r * GP + g]) = make_float4(d[g], d[g + 1], d[g + 2], d[g + 3]);
    }
  };
  for (int b0 = 0; b0 < nround; b0 += kFaBatch) {
    if (b0) {
#pragma unroll
      for (int b = 0; b < kFaBatch; b++) kr[b] = load4(krs, b0 + b < nround ? row_off(b0 + b) : 0x7ffffff0);
    }
#pragma unroll
    for (int b = 0; b < kFaBatch; b++) {
      if (b0 + b >= nround) break;
      store_scores(kr[b], (b0 + b) * RPR + rlane);
    }
  }
  // row n-1 is the last row of its lane group (rows go round-robin over the groups)
  const bool owns_pos = ROPE && holds_pos && rlane == (n - 1) % RPR;
  if (ROPE && holds_pos)
    store_scores(cok ? *reinterpret_cast<const float4 *>(&S.kcur[4 * c]) : f4_zero(), owns_pos ? n - 1 : n);
  qd::lds_sync();

  // 2. chunk softmax by head: m, e_j (in place), l; rows n .. nround*RPR-1,
  // which the PV loop reads, are set to 0
  const int nz = nround * RPR;
  for (int g = wave; g < G; g += kFaWaves) {
    float m = -INFINITY;
    for (int r = lane; r < n; r += 64) m = fmaxf(m, S.sc[r * GP + g]);
    m = qd::wave_max_f32(m);
    float l = 0.0f;
    for (int r = lane; r < nz; r += 64) {
      const float e = r < n ? qd::expf_glibc(S.sc[r * GP + g] - m) : 0.0f;
      S.sc[r * GP + g] = e;
      l += e;
    }
    l = qd::wave_sum_f32(l);
    if (lane == 0) { S.sm[g] = m; S.sl[g] = l; }
  }
  qd::lds_sync();

  // 3. o = sum_j e_j V_j over the chunk
  float4 acc[G];
#pragma unroll
  for (int g = 0; g < G; g++) acc[g] = f4_zero();
  for (int b0 = 0; b0 < nround; b0 += kFaBatch) {
    if (b0) {
#pragma unroll
      for (int b = 0; b < kFaBatch; b++) vr[b] = load4(vrs, b0 + b < nround ? row_off(b0 + b) : 0x7ffffff0);
    }
#pragma unroll
    for (int b = 0; b < kFaBatch; b++) {
      if (b0 + b >= nround) break;
      const int r = (b0 + b) * RPR + rlane;             // rows past n have e = 0 and v = 0
      float w[GP];
#pragma unroll
      for (int g = 0; g < GP; g += 4) {
        const float4 t = *reinterpret_cast<const float4 *>(&S.sc[r * GP + g]);
        w[g] = t.x; w[g + 1] = t.y; w[g + 2] = t.z; w[g + 3] = t.w;
      }
#pragma unroll
      for (int g = 0; g < G; g++) acc[g] = fma4(w[g], vr[b], acc[g]);
    }
  }
  if (owns_pos) {       // the current row (read as 0 above) is its lane group's last row
    const float4 v = cok ? *reinterpret_cast<const float4 *>(&S.vcur[4 * c]) : f4_zero();
#pragma unroll
    for (int g = 0; g < G; g++) acc[g] = fma4(S.sc[(n - 1) * GP + g], v, acc[g]);
  }
  // rows of one wave instruction, then the waves (fixed order)
#pragma unroll
  for (int g = 0; g < G; g++) {
    float4 a = acc[g];
    if (RPW == 4) {
      a.x += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(a.x), 0x401F));
      a.y += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(a.y), 0x401F));
      a.z += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(a.z), 0x401F));
      a.w += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(a.w), 0x401F));
    }
    a.x += __shfl_xor(a.x, 32, 64);
    a.y += __shfl_xor(a.y, 32, 64);
    a.z += __shfl_xor(a.z, 32, 64);
    a.w += __shfl_xor(a.w, 32, 64);
    if (rsub == 0 && cok) *reinterpret_cast<float4 *>(&S.ro[(wave * G + g) * HD + 4 * c]) = a;
  }
  qd::lds_sync();
  const size_t slot = (size_t)kvh * nsmax + split;
  float *pm = part, *pl = part + (size_t)KVH * nsmax * G, *po = part + (size_t)2 * KVH * nsmax * G;
  for (int i = tid; i < G * HD; i += kFaThreads) {
    float s = S.ro[i];
#pragma unroll
    for (int w = 1; w < kFaWaves; w++) s += S.ro[w * G * HD + i];
    po[slot * G * HD + i] = s;
  }
  if (tid < G) { pm[slot * G + tid] = S.sm[tid]; pl[slot * G + tid] = S.sl[tid]; }

}

// Merge of the chunks of one query head (one thread per dim, in whole waves):
// M = max_c m_c, w_c = expf(m_c - M), o = (sum_c w_c o_c) * (1 / sum_c w_c l_c),
// c in order; obm[h] = max_d |o_d| (the Wo GEMV's activation quantizer reads
// these).  Block b serves KV head b % KVH, like the chunk blocks (x % KVH), so
// with KVH a multiple of 8 it runs on the XCD whose L2 holds that head's
// partials.
template <int HD>
constexpr int merge_threads() { return (HD + 63) / 64 * 64; }

template <int HD>
__global__ __launch_bounds__(merge_threads<HD>()) void k_fattn_merge(const float *part, const int *d_pos, int KVH,
                                                                     int G, int chunk, int nsmax, float *o,
                                                                     float *obm) {
  constexpr int NT = merge_threads<HD>(), NW = NT / 64;
  constexpr int SPT = (kFaMaxSplits + NT - 1) / NT;     // chunk slots a thread may hold
  __shared__ float wm[kFaMaxSplits];
  __shared__ float red[3][NW];
  const int kvh = blockIdx.x % KVH, g = blockIdx.x / KVH, h = kvh * G + g;
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const bool dim_ok = tid < HD;
  const int T = *d_pos + 1, nact = (T + chunk - 1) / chunk;
  const float *pm = part, *pl = part + (size_t)KVH * nsmax * G, *po = part + (size_t)2 * KVH * nsmax * G;
  const size_t base = (size_t)kvh * nsmax;
  // every request first: the o of up to 64 chunks for this thread's dim, and the
  // m and l of the thread's chunks s = tid, tid + NT, ...
  constexpr int U = 64;
  // (through a buffer resource over the head's nact chunk slots: an offset past
  // them reads 0 without memory traffic, so no load needs a branch)
  float ov[U];
  const __amdgpu_buffer_rsrc_t ors = __builtin_amdgcn_make_buffer_rsrc(
      (void *)(po + base * G * HD + (size_t)g * HD), (short)0, nact * G * HD * 4, 0x00020000);
  const int vo = (dim_ok ? tid : 0) * 4, ostep = G * HD * 4;
  auto oload = [&](int c) { return __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(ors, vo + c * ostep, 0, 0)); };
#pragma unroll
  for (int u = 0; u < U; u++) ov[u] = oload(u);
  float mv[SPT], lv[SPT];
#pragma unroll
  for (int u = 0; u < SPT; u++) {
    const int s = tid + u * NT;
    mv[u] = s < nact ? pm[(base + s) * G + g] : -INFINITY;
    lv[u] = s < nact ? pl[(base + s) * G + g] : 0.0f;
  }
  float M = -INFINITY;
#pragma unroll
  for (int u = 0; u < SPT; u++) M = fmaxf(M, mv[u]);
  M = qd::wave_max_f32(M);
  if (lane == 0) red[0][wave] = M;
  __syncthreads();
  M = red[0][0];
#pragma unroll
  for (int w = 1; w < NW; w++) M = fmaxf(M, red[0][w]);
  float L = 0.0f;
#pragma unroll
  for (int u = 0; u < SPT; u++) {
    const int s = tid + u * NT;
    if (s < nact) {
      const float w = qd::expf_glibc(mv[u] - M);
      wm[s] = w;
      L = __builtin_fmaf(w, lv[u], L);
    }
  }
  L = qd::wave_sum_f32(L);
  if (lane == 0) red[1][wave] = L;
  __syncthreads();                                       // wm and the partial sums
  L = red[1][0];
#pragma unroll
  for (int w = 1; w < NW; w++) L += red[1][w];
  float a = 0.0f;
#pragma unroll
  for (int u = 0; u < U; u++) if (u < nact) a = __builtin_fmaf(wm[u], ov[u], a);
  for (int s0 = U; s0 < nact; s0 += U) {
#pragma unroll
    for (int u = 0; u < U; u++) ov[u] = oload(s0 + u);
#pragma unroll
    for (int u = 0; u < U; u++) if (s0 + u < nact) a = __builtin_fmaf(wm[s0 + u], ov[u], a);
  }
  const float r = a * (1.0f / L);
  if (dim_ok) o[(size_t)h * HD + tid] = r;
  float mo = qd::wave_max_f32(dim_ok ? fabsf(r) : 0.0f);
  if (lane == 0) red[2][wave] = mo;
  __syncthreads();
  mo = red[2][0];
#pragma unroll
  for (int w = 1; w < NW; w++) mo = fmaxf(mo, red[2][w]);
  if (tid == 0 && obm) obm[h] = mo;
}

template <int HD, bool ROPE>
int launch_g(int G, dim3 grid, const float *qkv, float *kc, float *vc, const int *d_pos, int H, int KVH, int max_seq,
             int chunk, int nsmax, float scale, const float *cos_t, const float *sin_t, float *part) {
#define FA(GG)                                                                                                  \
  QH_LAUNCH(QK_ATTN_FAST, (k_fattn<HD, GG, ROPE>), grid, dim3(kFaThreads), 0, qkv, kc, vc, d_pos, H, KVH,      \
            max_seq, chunk, nsmax, scale, cos_t, sin_t, part);                                                  \
  return 0
  switch (G) {
    case 1: FA(1);
    case 2: FA(2);
    case 3: FA(3);
    case 4: FA(4);
    case 5: FA(5);
    case 6: FA(6);
    case 7: FA(7);
    case 8: FA(8);
    default: return qh::fail_msg("fast attention: more than 8 query heads per KV head");
  }
#undef FA
}

// Positions per block: 64, or more where max_seq would need more than
// kFaMaxSplits chunks.
int fa_chunk(int max_seq) {
  int c = 64;
  while ((max_seq + c - 1) / c > kFaMaxSplits) c += 64;
  return c;
}

}  // namespace

extern "C" int qhip_fattn_ok(int n_heads, int n_kv, int hd, int max_seq) {
  if (n_kv <= 0 || n_heads % n_kv) return 0;
  const int G = n_heads / n_kv;
  return (hd == 128 || hd == 64 || hd == 48) && G >= 1 && G <= 8 && max_seq >= 1 &&
         fa_chunk(max_seq) <= kFaMaxChunk;
}

extern "C" size_t qhip_fattn_scratch(int n_heads, int n_kv, int hd, int max_seq) {
  const int nsmax = (max_seq + fa_chunk(max_seq) - 1) / fa_chunk(max_seq);
  return (size_t)n_kv * nsmax * (size_t)(n_heads / n_kv) * (hd + 2) * 4 + 256;
}

// Two launches: the chunks (k_fattn), then one merge block per query head.
extern "C" int qhip_fattn(const float *qkv, float *kc, float *vc, const int *d_pos, int n_heads, int n_kv, int hd,
                          int max_seq, float scale, const float *cos_t, const float *sin_t, int rope, void *scratch,
                          float *o, float *obm) {
  if (!qhip_fattn_ok(n_heads, n_kv, hd, max_seq)) return qh::fail_msg("fast attention: unsupported shape");
  if ((long long)max_seq * hd * 4 >= (1LL << 31) - 16) return qh::fail_msg("fast attention: KV head region too large");
  const int G = n_heads / n_kv, chunk = fa_chunk(max_seq), nsmax = (max_seq + chunk - 1) / chunk;
  float *part = static_cast<float *>(scratch);
  const dim3 grid(n_kv * nsmax);
  int rc;
#define FAH(HD)                                                                                                   \
  rc = rope ? launch_g<HD, true>(G, grid, qkv, kc, vc, d_pos, n_heads, n_kv, max_seq, chunk, nsmax, scale, cos_t,   \
                                 sin_t, part)                                                                       \
            : launch_g<HD, false>(G, grid, qkv, kc, vc, d_pos, n_heads, n_kv, max_seq, chunk, nsmax, scale, cos_t,  \
                                  sin_t, part);                                                                     \
  if (rc) return rc;                                                                                                \
  QH_LAUNCH(QK_ATTN_FAST, k_fattn_merge<HD>, dim3(n_heads), dim3(merge_threads<HD>()), 0, part, d_pos, n_kv, G, chunk, nsmax, o, obm); \
  return 0
  switch (hd) {
    case 128: FAH(128);
    case 64: FAH(64);
    case 48: FAH(48);
    default: return qh::fail_msg("fast attention: head_dim not supported");
  }
#undef FAH
}
