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
// A 256-thread block computes a 128 x 128 tile of C (SWIGLU: 64 outputs from 64
// gate and the 64 matching up rows) in K steps of 64 bytes: both tiles are
// staged through double-buffered LDS in a swizzled layout (conflict-free 16-byte
// fragment reads and writes), and each wave computes 64 x 64 with 4 x 4
// v_mfma_i32_16x16x64_i8.  Fragment layout (checked on gfx950): lane l holds
// row l % 16 and bytes 16 * (l / 16) .. +15 of the 64 K values; result element
// r of lane l is C[4 * (l / 16) + r][l % 16].
#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

typedef int v4i __attribute__((ext_vector_type(4)));

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

template <int MODE>
int launch(const int8_t *A, const float *as, const int8_t *W, const float *ws, int M, int N, int kpad, float *out,
           int ldo, const float *bias, int cls) {
  const int nout = MODE == GM_SWIGLU ? BN / 2 : BN;
  const int mt = (M + BM - 1) / BM, nt = (N + nout - 1) / nout;
  const int blocks = 8 * mt * ((nt + 7) / 8);
  QH_LAUNCH(cls, k_gemm_i8<MODE>, dim3(blocks), dim3(256), 0, A, as, W, ws, M, N, kpad, out, ldo, bias, mt, nt);
  return 0;
}

}  // namespace

extern "C" int qhip_gemm_i8(int mode, int cls, const int8_t *A, const float *as, const int8_t *W, const float *ws,
                            int M, int N, int kpad, float *out, int ldo, const float *bias) {
  if (M <= 0 || N <= 0 || kpad <= 0 || kpad % 16) return qh::fail_msg("gemm_i8: bad shape");
  switch (mode) {
    case GM_PLAIN: return launch<GM_PLAIN>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls);
    case GM_RESID: return launch<GM_RESID>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls);
    case GM_SWIGLU: return launch<GM_SWIGLU>(A, as, W, ws, M, N, kpad, out, ldo, bias, cls);
    default: return qh::fail_msg("gemm_i8: bad mode");
  }
}
