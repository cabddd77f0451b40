// k_gemm.hip - int8 MFMA GEMM for prompt ingestion: quant.c:60-85 over many
// activation rows at once (qmatmul with M = the prompt length).
//
// C[i][j] = (as[i] * ws[j]) * (float)acc[i][j],  acc = sum_k qa[i][k] * W[j][k]
//
// acc is an exact int32 sum (|acc| <= 127^2 * K < 2^31), so the MFMA order of
// accumulation changes nothing: every row equals the decode GEMV's result, and
// the epilogues below are the decode GEMV's, operation for operation:
//   PLAIN  out = c (+ bias)                              (llama.c:546-548)
//   RESID  out = out + c                                 (llama.c:578, 589)
//   SWIGLU gate j and up j -> h = (g * (1 / (1 + expf(-g)))) * u  (llama.c:583-587)
//
// Operands are K-contiguous (activation rows [M][kpad], weight rows [N][kpad]).
// Two kernels, both in K steps of 64 bytes through LDS:
//  - k_gemm_i8_pipe (kpad % 64 == 0): block tiles of 128 x 128 or 256 x 128 (SWIGLU:
//    half the columns are gate rows, half the matching up rows), 8 waves of
//    v_mfma_i32_32x32x32_i8 (the 16x16x64 form runs at half its rate on gfx950).
//    Both operand tiles are copied straight from global memory into LDS
//    (global_load_lds, no staging registers), three or four K steps ahead.
//  - k_gemm_i8 (other K): 128 x 128 tiles staged through registers into
//    double-buffered LDS, 4 waves of 4 x 4 v_mfma_i32_16x16x64_i8; chunks past
//    kpad are zero.
// Fragment layouts (checked on gfx950): 16x16x64: lane l holds row l % 16 and
// bytes 16 * (l / 16) .. +15 of the 64 K values, result element r of lane l is
// C[4 * (l / 16) + r][l % 16]; 32x32x32: lane l holds row l % 32 and bytes
// 16 * (l / 32) .. +15 of 32 K values, result element e of lane l is
// C[8 * (e / 4) + 4 * (l / 32) + e % 4][l % 32].
#include <hip/hip_runtime.h>

#include <type_traits>

#include "qdev_math.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));
typedef int v16i __attribute__((ext_vector_type(16)));

enum { GM_PLAIN = 0, GM_RESID = 1, GM_SWIGLU = 2 };

constexpr int BM = 128, BN = 128, BK = 64;

// Byte offset of 16-byte chunk c of staged row r: rows are 64 bytes, and the
// chunk index is XORed with bits 1-2 of the row, so that the 16-byte accesses of
// 16 consecutive rows (a fragment read) and of 4 consecutive rows x 4 chunks
// (a staging write) fall in distinct bank groups.
__device__ __forceinline__ int stage_off(int r, int c) { return r * BK + ((c ^ ((r >> 1) & 3)) << 4); }

// Block b -> (M tile, N tile): the row tiles of one weight tile run on one XCD
// (workgroups are dealt to the 8 XCDs round-robin by index), so a weight tile
// is fetched from HBM once and then served from that XCD's L2.
__device__ __forceinline__ void gemm_tile(int b, int mt_count, int &mt, int &nt) {
  const int x8 = b & 7, q = b >> 3;
  mt = q % mt_count;
  nt = 8 * (q / mt_count) + x8;
}

template <int MODE>
__global__ __launch_bounds__(256) void k_gemm_i8(const int8_t *A, const float *as, const int8_t *W, const float *ws,
                                                 int M, int N, int kpad, float *out, int ldo, const float *bias,
                                                 int mt_count, int nt_count) {
  __shared__ __attribute__((aligned(16))) int8_t sA[2][BM * BK];
  __shared__ __attribute__((aligned(16))) int8_t sB[2][BN * BK];
  int mtile, ntile;
  gemm_tile(blockIdx.x, mt_count, mtile, ntile);
  if (ntile >= nt_count) return;                                   // uniform for the block
  const int tid = threadIdx.x, lane = tid & 63, wave = tid >> 6;
  const int wm = wave >> 1, wn = wave & 1;
  const int m0 = mtile * BM;
  constexpr int NOUT = MODE == GM_SWIGLU ? BN / 2 : BN;
  const int n0 = ntile * NOUT;

  // global -> LDS: each operand tile is 512 chunks of 16 bytes; thread tid moves
  // chunks tid and tid + 256 (row = chunk / 4, part = chunk % 4)
  const int8_t *ga[2], *gb[2];
  int soff[2], part[2];
#pragma unroll
  for (int i = 0; i < 2; i++) {
    const int c = tid + 256 * i, row = c >> 2;
    part[i] = c & 3;
    soff[i] = stage_off(row, part[i]);
    ga[i] = A + (size_t)min(m0 + row, M - 1) * kpad + part[i] * 16;
    int wrow;
    if (MODE == GM_SWIGLU) wrow = row < 64 ? min(n0 + row, N - 1) : N + min(n0 + row - 64, N - 1);
    else wrow = min(n0 + row, N - 1);
    gb[i] = W + (size_t)wrow * kpad + part[i] * 16;
  }
  const int nk = (kpad + BK - 1) / BK;
  v4i ra[2], rb[2];
  auto gload = [&](int kt) {
    const int k0 = kt * BK;
#pragma unroll
    for (int i = 0; i < 2; i++) {
      const bool in = k0 + part[i] * 16 < kpad;
      const v4i z = {0, 0, 0, 0};
      ra[i] = in ? *reinterpret_cast<const v4i *>(ga[i] + k0) : z;
      rb[i] = in ? *reinterpret_cast<const v4i *>(gb[i] + k0) : z;
    }
  };
  auto sstore = [&](int buf) {
#pragma unroll
    for (int i = 0; i < 2; i++) {
      *reinterpret_cast<v4i *>(&sA[buf][soff[i]]) = ra[i];
      *reinterpret_cast<v4i *>(&sB[buf][soff[i]]) = rb[i];
    }
  };

  // this lane's fragment rows inside the staged tiles
  int arow[4], brow[4];
#pragma unroll
  for (int t = 0; t < 4; t++) {
    arow[t] = stage_off(wm * 64 + t * 16 + (lane & 15), lane >> 4);
    const int bl = MODE == GM_SWIGLU ? (t < 2 ? wn * 32 + t * 16 : 64 + wn * 32 + (t - 2) * 16) : wn * 64 + t * 16;
    brow[t] = stage_off(bl + (lane & 15), lane >> 4);
  }

  v4i acc[4][4];
#pragma unroll
  for (int a = 0; a < 4; a++)
#pragma unroll
    for (int b = 0; b < 4; b++) acc[a][b] = (v4i){0, 0, 0, 0};

  gload(0);
  sstore(0);
  __syncthreads();
  for (int kt = 0; kt < nk; kt++) {
    const int buf = kt & 1;
    if (kt + 1 < nk) gload(kt + 1);
    v4i fa[4], fb[4];
#pragma unroll
    for (int t = 0; t < 4; t++) {
      fa[t] = *reinterpret_cast<const v4i *>(&sA[buf][arow[t]]);
      fb[t] = *reinterpret_cast<const v4i *>(&sB[buf][brow[t]]);
    }
#pragma unroll
    for (int a = 0; a < 4; a++)
#pragma unroll
      for (int b = 0; b < 4; b++) acc[a][b] = __builtin_amdgcn_mfma_i32_16x16x64_i8(fa[a], fb[b], acc[a][b], 0, 0, 0);
    if (kt + 1 < nk) sstore(buf ^ 1);
    __syncthreads();
  }

  // epilogue (the decode GEMV's operations and order)
#pragma unroll
  for (int a = 0; a < 4; a++) {
#pragma unroll
    for (int r = 0; r < 4; r++) {
      const int i = m0 + wm * 64 + a * 16 + 4 * (lane >> 4) + r;
      if (i >= M) continue;
      const float asi = as[i];
      if (MODE == GM_SWIGLU) {
#pragma unroll
        for (int b = 0; b < 2; b++) {
          const int j = n0 + wn * 32 + b * 16 + (lane & 15);
          if (j < N) {
            const float g = (asi * ws[j]) * (float)acc[a][b][r];
            const float up = (asi * ws[N + j]) * (float)acc[a][b + 2][r];
            const float s = 1.0f / (1.0f + qd::expf_glibc(-g));
            out[(size_t)i * ldo + j] = (g * s) * up;
          }
        }
      } else {
#pragma unroll
        for (int b = 0; b < 4; b++) {
          const int j = n0 + wn * 64 + b * 16 + (lane & 15);
          if (j < N) {
            const float c = (asi * ws[j]) * (float)acc[a][b][r];
            float *o = out + (size_t)i * ldo + j;
            if (MODE == GM_RESID) *o = *o + c;
            else *o = bias ? c + bias[j] : c;
          }
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// Pipelined variant for kpad % 64 == 0: the same tiles, fragments and epilogues,
// but both operand tiles go straight from global memory into LDS
// (global_load_lds, 16 bytes per lane, no staging registers), NSTAGE K steps
// deep.  Wave instruction i of a tile fills LDS slots 64i .. 64i+63 of 16 bytes;
// slot s holds chunk (s % 4) ^ ((r >> 1) % 4) of row r = s / 4, i.e. the lane
// fetches the global chunk that the swizzled layout puts there.  The waits
// before each step's barrier name only the step's own loads (vmcnt of the
// later stages stay in flight); the barrier itself is s_barrier without a
// fence, which would drain every outstanding load.
// ---------------------------------------------------------------------------
typedef __attribute__((address_space(3))) void *lds_ptr_t;

// Staged layout of the pipelined kernel: 64-byte rows, 16-byte chunk c of row r
// at slot c ^ swz32(r).  The fragment reads of v_mfma_i32_32x32x32_i8 take one
// chunk of 32 consecutive rows per half-wave.  XOR with row bits 2-3 makes those
// 16-byte reads conflict-free on gfx950 (measured with SQ_LDS_BANK_CONFLICT on
// this access pattern: bits 2-3 or 3-4, or 80-byte rows, 0 conflict cycles;
// bits 1-2, or bits 1^3 and 2^4, half of the LDS cycles; bits 0-1 or none,
// three quarters).  The staging writes fill whole 1 KiB runs and never conflict.
__device__ __forceinline__ int swz32(int r) { return (r >> 2) & 3; }
__device__ __forceinline__ int stage_off32(int r, int c) { return r * BK + ((c ^ swz32(r)) << 4); }

template <int N>
__device__ __forceinline__ void wait_vmcnt() {
  static_assert(N >= 0 && N < 64, "vmcnt range");
  __builtin_amdgcn_s_waitcnt((N & 15) | (7 << 4) | (15 << 8) | ((N >> 4) << 14));
}

__device__ __forceinline__ void block_sync_lds() {
  asm volatile("" ::: "memory");
  __builtin_amdgcn_s_barrier();
  asm volatile("" ::: "memory");
}

// Block tile TM x TN, waves WM x WN, each wave (TM/WM) x (TN/WN) from 32 x 32
// v_mfma_i32_32x32x32_i8 blocks: RB row blocks x 2 column blocks (SWIGLU: the
// wave's 32 gate columns and the matching 32 up columns).
//
// Split K (PART): block b of the grid takes tile b % bps and the K steps
// [split * nks, split * nks + nks) of split b / bps, and stores its int32 partial
// sums to part[split][M][N] (SWIGLU: [split][M][2N], up columns at N + j) for
// k_gemm_split_epi.
template <int MODE, int TM, int TN, int WM, int WN, int NSTAGE, bool PART = false>
__global__ __launch_bounds__(64 * WM * WN) void k_gemm_i8_pipe(const int8_t *A, const float *as, const int8_t *W,
                                                              const float *ws, int M, int N, int kpad, float *out,
                                                              int ldo, const float *bias, int mt_count, int nt_count,
                                                              int bps, int nks, int *part) {
  static_assert(NSTAGE == 3 || NSTAGE == 4, "pipeline depth");
  constexpr int NWAVE = WM * WN, RB = TM / WM / 32;
  static_assert(TN == 64 * WN, "two 32-column blocks per wave");
  static_assert(TM % (16 * NWAVE) == 0 && TN % (16 * NWAVE) == 0, "whole wave instructions per tile");
  constexpr int LA = TM / 16 / NWAVE, LB = TN / 16 / NWAVE;        // 1 KiB copies per wave and stage
  constexpr int LPS = LA + LB;                                       // vmcnt per stage
  // one LDS buffer per stage and operand, as distinct variables: the compiler
  // then knows which copies in flight write which buffer
  __shared__ __attribute__((aligned(16))) int8_t sA0[TM * BK], sA1[TM * BK], sA2[TM * BK], sA3[NSTAGE > 3 ? TM * BK : 16];
  __shared__ __attribute__((aligned(16))) int8_t sB0[TN * BK], sB1[TN * BK], sB2[TN * BK], sB3[NSTAGE > 3 ? TN * BK : 16];
  int mtile, ntile;
  const int split = PART ? (int)blockIdx.x / bps : 0;
  gemm_tile(PART ? (int)blockIdx.x % bps : (int)blockIdx.x, mt_count, mtile, ntile);
  if (ntile >= nt_count) return;                                   // uniform for the block
  const int kt0 = split * nks;                                     // first K step of this block
  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave / WN, wn = wave % WN;
  const int m0 = mtile * TM;
  constexpr int NOUT = MODE == GM_SWIGLU ? TN / 2 : TN;
  const int n0 = ntile * NOUT;

  // this lane's global chunks: wave instructions wave*LA + i of the A tile and
  // wave*LB + i of the B tile
  const int8_t *ga[LA], *gb[LB];
#pragma unroll
  for (int i = 0; i < LA; i++) {
    const int slot = (wave * LA + i) * 64 + lane, row = slot >> 2;
    const int c = (slot & 3) ^ swz32(row);
    ga[i] = A + (size_t)min(m0 + row, M - 1) * kpad + c * 16 + (size_t)kt0 * BK;
  }
#pragma unroll
  for (int i = 0; i < LB; i++) {
    const int slot = (wave * LB + i) * 64 + lane, row = slot >> 2;
    const int c = (slot & 3) ^ swz32(row);
    int wrow;
    if (MODE == GM_SWIGLU) wrow = row < TN / 2 ? min(n0 + row, N - 1) : N + min(n0 + row - TN / 2, N - 1);
    else wrow = min(n0 + row, N - 1);
    gb[i] = W + (size_t)wrow * kpad + c * 16 + (size_t)kt0 * BK;
  }
  const int nk = PART ? min(nks, kpad / BK - kt0) : kpad / BK;
  auto bufA = [&](auto st) -> int8_t * {
    if constexpr (decltype(st)::value == 0) return sA0;
    else if constexpr (decltype(st)::value == 1) return sA1;
    else if constexpr (decltype(st)::value == 2) return sA2;
    else return sA3;
  };
  auto bufB = [&](auto st) -> int8_t * {
    if constexpr (decltype(st)::value == 0) return sB0;
    else if constexpr (decltype(st)::value == 1) return sB1;
    else if constexpr (decltype(st)::value == 2) return sB2;
    else return sB3;
  };
  auto issue = [&](auto st, int kt) {
    const int k0 = kt * BK;
    int8_t *da = bufA(st), *db = bufB(st);
#pragma unroll
    for (int i = 0; i < LA; i++)
      __builtin_amdgcn_global_load_lds((const void *)(ga[i] + k0), (lds_ptr_t)(da + (wave * LA + i) * 1024), 16, 0, 0);
#pragma unroll
    for (int i = 0; i < LB; i++)
      __builtin_amdgcn_global_load_lds((const void *)(gb[i] + k0), (lds_ptr_t)(db + (wave * LB + i) * 1024), 16, 0, 0);
  };

  // fragments of v_mfma_i32_32x32x32_i8: lane l supplies row l % 32 and bytes
  // 16 * (l / 32) .. +15 of a 32-byte K half, i.e. chunk 2 * kh + l / 32 of the
  // 64-byte staged row; result element e of lane l is
  // C[8 * (e / 4) + 4 * (l / 32) + e % 4][l % 32] (checked on gfx950)
  int arow[RB][2], brow[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; kh++) {
#pragma unroll
    for (int t = 0; t < RB; t++) arow[t][kh] = stage_off32(wm * (TM / WM) + t * 32 + (lane & 31), 2 * kh + (lane >> 5));
#pragma unroll
    for (int t = 0; t < 2; t++) {
      const int bl = MODE == GM_SWIGLU ? t * (TN / 2) + wn * 32 : wn * 64 + t * 32;
      brow[t][kh] = stage_off32(bl + (lane & 31), 2 * kh + (lane >> 5));
    }
  }

  v16i acc[RB][2];
#pragma unroll
  for (int a = 0; a < RB; a++)
#pragma unroll
    for (int b = 0; b < 2; b++) acc[a][b] = (v16i){};

  // step kt from stage ST: wait for its copies, barrier, refill stage ST-1 with
  // step kt + NSTAGE - 1, multiply
  auto step = [&](auto st, int kt) {
    constexpr int ST = decltype(st)::value;
    const int later = min(NSTAGE - 2, nk - 1 - kt);      // steps issued after kt
    if (later >= NSTAGE - 2) wait_vmcnt<LPS * (NSTAGE - 2)>();
    else if (NSTAGE > 3 && later == 1) wait_vmcnt<LPS>();
    else wait_vmcnt<0>();
    block_sync_lds();                   // every wave's copies of step kt have landed; step kt-1 is consumed
    if (kt + NSTAGE - 1 < nk) issue(std::integral_constant<int, (ST + NSTAGE - 1) % NSTAGE>(), kt + NSTAGE - 1);
    // fragment reads in asm, with their own waits: the compiler would otherwise
    // wait for every copy in flight before reading an LDS buffer it cannot
    // tell apart from the ones being filled
    const unsigned la = (unsigned)(uintptr_t)bufA(st), lb = (unsigned)(uintptr_t)bufB(st);
    v4i fa[RB][2], fb[2][2];
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
#pragma unroll
      for (int t = 0; t < 2; t++) asm volatile("ds_read_b128 %0, %1" : "=v"(fb[t][kh]) : "v"(lb + brow[t][kh]));
#pragma unroll
      for (int t = 0; t < RB; t++) asm volatile("ds_read_b128 %0, %1" : "=v"(fa[t][kh]) : "v"(la + arow[t][kh]));
    }
#pragma unroll
    for (int kh = 0; kh < 2; kh++) {
      // the kh = 0 fragments are the first 2 + RB reads issued
      if (kh == 0) __builtin_amdgcn_s_waitcnt(0xC07F | ((2 + RB) << 8));
      else __builtin_amdgcn_s_waitcnt(0xC07F);
#pragma unroll
      for (int t = 0; t < 2; t++) asm volatile("" : "+v"(fb[t][kh]));
#pragma unroll
      for (int t = 0; t < RB; t++) asm volatile("" : "+v"(fa[t][kh]));
#pragma unroll
      for (int a = 0; a < RB; a++)
#pragma unroll
        for (int b = 0; b < 2; b++)
          acc[a][b] = __builtin_amdgcn_mfma_i32_32x32x32_i8(fa[a][kh], fb[b][kh], acc[a][b], 0, 0, 0);
      __builtin_amdgcn_sched_barrier(0);   // the kh = 0 products go before the wait for the kh = 1 reads
    }
  };

  issue(std::integral_constant<int, 0>(), 0);
  if (1 < nk) issue(std::integral_constant<int, 1>(), 1);
  if (NSTAGE > 3 && 2 < nk) issue(std::integral_constant<int, (NSTAGE > 3 ? 2 : 0)>(), 2);
  for (int kt = 0; kt < nk; kt += NSTAGE) {
    step(std::integral_constant<int, 0>(), kt);
    if (kt + 1 < nk) step(std::integral_constant<int, 1>(), kt + 1);
    if (kt + 2 < nk) step(std::integral_constant<int, 2>(), kt + 2);
    if (NSTAGE > 3 && kt + 3 < nk) step(std::integral_constant<int, (NSTAGE > 3 ? 3 : 0)>(), kt + 3);
  }

  if constexpr (PART) {                // int32 partial sums of this split
    const int ldp = MODE == GM_SWIGLU ? 2 * N : N;
    int *pp = part + (size_t)split * M * ldp;
#pragma unroll
    for (int a = 0; a < RB; a++) {
#pragma unroll
      for (int e = 0; e < 16; e++) {
        const int i = m0 + wm * (TM / WM) + a * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
        if (i >= M) continue;
        if (MODE == GM_SWIGLU) {
          const int j = n0 + wn * 32 + (lane & 31);
          if (j < N) {
            pp[(size_t)i * ldp + j] = acc[a][0][e];
            pp[(size_t)i * ldp + N + j] = acc[a][1][e];
          }
        } else {
#pragma unroll
          for (int b = 0; b < 2; b++) {
            const int j = n0 + wn * 64 + b * 32 + (lane & 31);
            if (j < N) pp[(size_t)i * ldp + j] = acc[a][b][e];
          }
        }
      }
    }
    return;
  }

  // epilogue (the decode GEMV's operations and order)
#pragma unroll
  for (int a = 0; a < RB; a++) {
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int i = m0 + wm * (TM / WM) + a * 32 + 8 * (e >> 2) + 4 * (lane >> 5) + (e & 3);
      if (i >= M) continue;
      const float asi = as[i];
      if (MODE == GM_SWIGLU) {
        const int j = n0 + wn * 32 + (lane & 31);
        if (j < N) {
          const float g = (asi * ws[j]) * (float)acc[a][0][e];
          const float up = (asi * ws[N + j]) * (float)acc[a][1][e];
          const float s = 1.0f / (1.0f + qd::expf_glibc(-g));
          out[(size_t)i * ldo + j] = (g * s) * up;
        }
      } else {
#pragma unroll
        for (int b = 0; b < 2; b++) {
          const int j = n0 + wn * 64 + b * 32 + (lane & 31);
          if (j < N) {
            const float c = (asi * ws[j]) * (float)acc[a][b][e];
            float *o = out + (size_t)i * ldo + j;
            if (MODE == GM_RESID) *o = *o + c;
            else *o = bias ? c + bias[j] : c;
          }
        }
      }
    }
  }
}

constexpr int kMaxSplits = 16;         // K splits of one GEMM at most

// Split-K epilogue: acc = the sum of the S int32 partials (exact in any order:
// every partial sum of the products is bounded like the whole, |acc| <= 127^2 K),
// then the fused epilogue's operations on it.  Grid (ceil(N / 256), M).
template <int MODE>
__global__ __launch_bounds__(256) void k_gemm_split_epi(const int *part, int S, const float *as, const float *ws,
                                                        int M, int N, float *out, int ldo, const float *bias) {
  const int j = blockIdx.x * 256 + threadIdx.x, i = blockIdx.y;
  if (j >= N) return;
  const int ldp = MODE == GM_SWIGLU ? 2 * N : N;
  const size_t plane = (size_t)M * ldp;
  const int *pp = part + (size_t)i * ldp + j;
  // every partial requested before the first add (S <= kMaxSplits)
  int pv[kMaxSplits], pu[kMaxSplits];
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++) {
    pv[s] = s < S ? pp[s * plane] : 0;
    pu[s] = MODE == GM_SWIGLU && s < S ? pp[s * plane + N] : 0;
  }
  int acc = 0, accu = 0;
#pragma unroll
  for (int s = 0; s < kMaxSplits; s++) {
    acc += pv[s];
    accu += pu[s];
  }
  const float asi = as[i];
  if (MODE == GM_SWIGLU) {
    const float g = (asi * ws[j]) * (float)acc;
    const float up = (asi * ws[N + j]) * (float)accu;
    const float sg = 1.0f / (1.0f + qd::expf_glibc(-g));
    out[(size_t)i * ldo + j] = (g * sg) * up;
  } else {
    const float c = (asi * ws[j]) * (float)acc;
    float *o = out + (size_t)i * ldo + j;
    if (MODE == GM_RESID) *o = *o + c;
    else *o = bias ? c + bias[j] : c;
  }
}

// Tiles that leave CUs idle (a short prompt, a narrow output) split K when the
// caller lends a workspace: S splits of at least 8 K steps, so that tiles x S
// reach one block per CU, with S partial planes of M x N int32 in the workspace.
int g_last_splits = 1;                 // K splits of the last pipelined launch (for the split test)

template <int MODE, int TM, int TN, int WM, int WN, int NS>
int launch_pipe(const int8_t *A, const float *as, const int8_t *W, const float *ws, int M, int N, int kpad, float *out,
                int ldo, const float *bias, int cls, int *work, size_t work_bytes) {
  const int nout = MODE == GM_SWIGLU ? TN / 2 : TN;
  const int mt = (M + TM - 1) / TM, nt = (N + nout - 1) / nout;
  const int blocks = 8 * mt * ((nt + 7) / 8);
  const int nkt = kpad / BK;
  int S = 1;
  if (work) {
    const int cus = qh::num_cus() > 0 ? qh::num_cus() : 256, active = mt * nt;
    if (active < cus) {
      S = min(min((cus + active - 1) / active, nkt / 8), kMaxSplits);
      const size_t plane = (size_t)M * (MODE == GM_SWIGLU ? 2 * N : N) * 4;
      while (S > 1 && (size_t)S * plane > work_bytes) S--;
    }
  }
  g_last_splits = S < 2 ? 1 : S;
  if (S < 2) {
    QH_LAUNCH(cls, (k_gemm_i8_pipe<MODE, TM, TN, WM, WN, NS>), dim3(blocks), dim3(64 * WM * WN), 0, A, as, W, ws, M,
              N, kpad, out, ldo, bias, mt, nt, blocks, nkt, static_cast<int *>(nullptr));
    return 0;
  }
  const int nks = (nkt + S - 1) / S;
  S = (nkt + nks - 1) / nks;                                       // every split has steps
  g_last_splits = S;
  QH_LAUNCH(cls, (k_gemm_i8_pipe<MODE, TM, TN, WM, WN, NS, true>), dim3(blocks * S), dim3(64 * WM * WN), 0, A, as, W,
            ws, M, N, kpad, out, ldo, bias, mt, nt, blocks, nks, work);
  QH_LAUNCH(cls, k_gemm_split_epi<MODE>, dim3((N + 255) / 256, M), dim3(256), 0, work, S, as, ws, M, N, out, ldo,
            bias);
  return 0;
}

// Tile choice (measured at the 8B prefill shapes, M = 2048): 256 x 128 blocks for
// the wide gate|up GEMM and for long K; 128 x 128 blocks of 8 waves otherwise.
// K not a multiple of 64 takes the register-staged kernel.
template <int MODE>
int launch(const int8_t *A, const float *as, const int8_t *W, const float *ws, int M, int N, int kpad, float *out,
           int ldo, const float *bias, int cls, int *work, size_t work_bytes) {
  if (kpad % BK == 0) {
    if (MODE == GM_SWIGLU || (MODE == GM_RESID && kpad >= 8192))
      return launch_pipe<MODE, 256, 128, 4, 2, 3>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls, work, work_bytes);
    if (MODE == GM_RESID)
      return launch_pipe<MODE, 128, 128, 4, 2, 3>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls, work, work_bytes);
    return launch_pipe<MODE, 128, 128, 4, 2, 4>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls, work, work_bytes);
  }
  const int nout = MODE == GM_SWIGLU ? BN / 2 : BN;
  const int mt = (M + BM - 1) / BM, nt = (N + nout - 1) / nout;
  const int blocks = 8 * mt * ((nt + 7) / 8);
  QH_LAUNCH(cls, k_gemm_i8<MODE>, dim3(blocks), dim3(256), 0, A, as, W, ws, M, N, kpad, out, ldo, bias, mt, nt);
  return 0;
}

}  // namespace

extern "C" int qhip_gemm_i8_ws(int mode, int cls, const int8_t *A, const float *as, const int8_t *W, const float *ws,
                               int M, int N, int kpad, float *out, int ldo, const float *bias, int *work,
                               size_t work_bytes) {
  if (M <= 0 || N <= 0 || kpad <= 0 || kpad % 16) return qh::fail_msg("gemm_i8: bad shape");
  switch (mode) {
    case GM_PLAIN: return launch<GM_PLAIN>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls, work, work_bytes);
    case GM_RESID: return launch<GM_RESID>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls, work, work_bytes);
    case GM_SWIGLU: return launch<GM_SWIGLU>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls, work, work_bytes);
    default: return qh::fail_msg("gemm_i8: bad mode");
  }
}

extern "C" int qhip_gemm_i8(int mode, int cls, const int8_t *A, const float *as, const int8_t *W, const float *ws,
                            int M, int N, int kpad, float *out, int ldo, const float *bias) {
  return qhip_gemm_i8_ws(mode, cls, A, as, W, ws, M, N, kpad, out, ldo, bias, nullptr, 0);
}

// Test entry: one GEMM (mode 0 plain + bias, 1 residual, 2 SwiGLU) from host
// operands, run whole and with a 64 MB split-K workspace; out_plain and
// out_split hold the residual's initial values on entry (mode 1) and the two
// results on return; *splits = the K splits the second run used.
extern "C" int qllama_test_gemm_split(int mode, const int8_t *A, const float *as, const int8_t *W, const float *ws,
                                      int M, int N, int kpad, const float *bias, float *out_plain, float *out_split,
                                      int *splits) {
  if (qhip_init()) return 1;
  if (mode < 0 || mode > 2 || M <= 0 || N <= 0 || kpad <= 0 || kpad % 16) return qh::fail_msg("test_gemm_split: bad shape");
  const size_t wrows = mode == GM_SWIGLU ? 2 * (size_t)N : (size_t)N, nout = (size_t)M * N;
  const size_t work_bytes = (size_t)64 << 20;
  int8_t *dA = (int8_t *)qhip_malloc((size_t)M * kpad), *dW = (int8_t *)qhip_malloc(wrows * kpad);
  float *das = (float *)qhip_malloc((size_t)M * 4), *dws = (float *)qhip_malloc(wrows * 4);
  float *db = bias ? (float *)qhip_malloc((size_t)N * 4) : nullptr;
  float *o1 = (float *)qhip_malloc(nout * 4), *o2 = (float *)qhip_malloc(nout * 4);
  int *work = (int *)qhip_malloc(work_bytes);
  int rc = (!dA || !dW || !das || !dws || (bias && !db) || !o1 || !o2 || !work) ? 1 : 0;
  if (!rc)
    rc = qhip_h2d(dA, A, (size_t)M * kpad) || qhip_h2d(dW, W, wrows * kpad) || qhip_h2d(das, as, (size_t)M * 4) ||
         qhip_h2d(dws, ws, wrows * 4) || (bias && qhip_h2d(db, bias, (size_t)N * 4)) ||
         qhip_h2d(o1, out_plain, nout * 4) || qhip_h2d(o2, out_split, nout * 4);
  if (!rc) rc = qhip_gemm_i8(mode, QK_OTHER, dA, das, dW, dws, M, N, kpad, o1, N, db);
  if (!rc) rc = qhip_gemm_i8_ws(mode, QK_OTHER, dA, das, dW, dws, M, N, kpad, o2, N, db, work, work_bytes);
  if (!rc) *splits = g_last_splits;
  if (!rc) rc = qhip_device_sync() || qhip_d2h(out_plain, o1, nout * 4) || qhip_d2h(out_split, o2, nout * 4);
  qhip_free(dA); qhip_free(dW); qhip_free(das); qhip_free(dws); qhip_free(db); qhip_free(o1); qhip_free(o2);
  qhip_free(work);
  return rc;
}
