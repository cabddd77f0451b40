// k_gemv_f32.hip - the fp32 (LLMA) decode path's kernels: the f32 matmul of one
// row (matrix.c:178-190) with the reference's summation order, and the small
// elementwise pieces of llama.c:296-362.
//
// Order: the reference forms c[j] = ((0 + a_0*W_0j) + a_1*W_1j) + ... in k order
// (the k loop is outer, j inner), every product rounded before its add.  Here
// each output column is one serial chain: lane dd of wave 0 owns column
// j0 + dd of its block and adds the products of its column in k order.  The
// products themselves do not depend on the running sum, so waves 1-7 form them
// ahead: each tile of kFT rows is loaded, multiplied by x[k] from LDS and stored
// as a [column][k] tile in LDS, double buffered, with the W values of three
// later tiles in flight.  The chain lanes are the critical path: K dependent
// adds per column.
//
// Device layout of W ("panels of 16"): the reference's (K, N) row-major matrix
// is stored as ceil(N/16) panels, panel p holding columns 16p .. 16p+15 of every
// row, row after row (element (k, j) at [(j/16)*K + k]*16 + j%16; columns past N
// are 0).  A block streams one contiguous panel, so no 128-byte line is shared
// with a block that may run on another XCD.
#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qdev_norm.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

constexpr int kFT = 128;                       // rows (k) per tile
constexpr int kFS = kFT + 4;                   // LDS stride of a product tile row
constexpr int kFC = 16;                        // columns (chains) per block
constexpr int kFThreads = 512;
constexpr int kFUnits = (kFThreads - 64) / kFC;            // 28 producer units of kFC lanes
constexpr int kFGroups = kFT / 4;                          // groups of 4 rows per tile
constexpr int kFSlots = (kFGroups + kFUnits - 1) / kFUnits;   // groups per producer lane and tile
constexpr int kFD = 6;                                     // tiles whose W values are in flight

enum { FMODE_PLAIN = 0, FMODE_RESID = 1, FMODE_RESID_BIAS = 2, FMODE_GELU_BIAS = 3 };

// W values of tile t for this producer lane: slot g covers rows
// t*kFT + 4*(u + kFUnits*g) + 0..3 of its column.  The loads go through a buffer
// resource over the block's panel: the lane's offset of each slot is fixed
// (vo), the rows are immediate offsets and the tile is one scalar, so a load
// costs no vector arithmetic (the producers share SIMDs with the chains, whose
// adds would otherwise wait behind address math).  Rows past K and unused slots
// read as 0 without touching memory, and a zero product leaves a chain that
// starts at +0 unchanged.
__device__ __forceinline__ void f_load(float (&v)[kFSlots][4], __amdgpu_buffer_rsrc_t rs, const int (&vo)[kFSlots],
                                       int t, int ntile) {
  if (threadIdx.x < 64 || t >= ntile) return;          // tiles past the last are never formed
  const int so = t * kFT * kFC * 4;
#pragma unroll
  for (int g = 0; g < kFSlots; g++)
#pragma unroll
    for (int i = 0; i < 4; i++)
      v[g][i] = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rs, vo[g] + i * kFC * 4, so, 0));
}

// Products of tile t: B[dd*kFS + kk] = x[k] * W[k][col]
__device__ __forceinline__ void f_produce(float *B, const float *xs, const float (&v)[kFSlots][4], int t, int u,
                                          int dd) {
#pragma unroll
  for (int g = 0; g < kFSlots; g++) {
    const int grp = u + kFUnits * g;
    if (grp >= kFGroups) continue;
    const float4 xv = *reinterpret_cast<const float4 *>(xs + t * kFT + 4 * grp);
    float4 p;
    p.x = xv.x * v[g][0];
    p.y = xv.y * v[g][1];
    p.z = xv.z * v[g][2];
    p.w = xv.w * v[g][3];
    *reinterpret_cast<float4 *>(B + dd * kFS + 4 * grp) = p;
  }
}

// out[j] = c[j] (+ bias[j]) or out[j] = out[j] + c[j] (llama.c:319-321, 347, 352);
// GPT-2 (model.c:505-514, feedforward.c:23-37): out[j] = out[j] + (c[j] + bias[j])
// and out[j] = gelu(c[j] + bias[j]) (activation.c:43-50)
template <int MODE>
__global__ __launch_bounds__(kFThreads) void k_gemv_f32(const float *x, int K, const float *W, int N, float *out,
                                                       const float *bias) {
  extern __shared__ float lds[];
  const int j0 = blockIdx.x * kFC, tid = threadIdx.x;
  const int ntile = (K + kFT - 1) / kFT;
  const int xcap = ntile * kFT;
  float *xs = lds;                                   // x, zero past K
  float *P = lds + xcap;                             // two product tiles of kFC x kFS
  const int pid = tid - 64, u = pid / kFC, dd = pid % kFC;
  const float *Wp = W + (size_t)blockIdx.x * K * kFC;   // this block's panel
  const __amdgpu_buffer_rsrc_t rs = __builtin_amdgcn_make_buffer_rsrc((void *)Wp, (short)0, K * kFC * 4, 0x00020000);
  int vo[kFSlots];
#pragma unroll
  for (int g = 0; g < kFSlots; g++) {
    const int grp = u + kFUnits * g;
    vo[g] = tid >= 64 && grp < kFGroups ? (4 * grp * kFC + dd) * 4 : 0x40000000;   // else: no traffic
  }
  float r[kFD][kFSlots][4];
#pragma unroll
  for (int d = 0; d < kFD; d++) f_load(r[d], rs, vo, d, ntile);   // W first: in flight during the x copy
  for (int i = tid; i < xcap; i += kFThreads) xs[i] = i < K ? x[i] : 0.0f;
  qd::lds_sync();                                    // x in LDS; the W loads stay in flight

  if (tid < 64) {
    const int crow = tid < kFC ? tid : kFC - 1;
    float acc = 0.0f;
    for (int t = 0; t < ntile; t++) {
      qd::lds_sync();                                // tile t is complete
      const float4 *Pt = reinterpret_cast<const float4 *>(P + (t & 1) * kFC * kFS + crow * kFS);
      constexpr int GR = 8, NG = kFT / 4 / GR;
      float4 buf[2][GR];
#pragma unroll
      for (int i = 0; i < GR; i++) buf[0][i] = Pt[i];
#pragma unroll
      for (int g = 0; g < NG; g++) {
        if (g + 1 < NG) {
#pragma unroll
          for (int i = 0; i < GR; i++) buf[(g + 1) & 1][i] = Pt[(g + 1) * GR + i];
        }
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int i = 0; i < GR; i++) {
          acc += buf[g & 1][i].x;
          acc += buf[g & 1][i].y;
          acc += buf[g & 1][i].z;
          acc += buf[g & 1][i].w;
        }
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    const int j = j0 + tid;
    if (tid < kFC && j < N) {
      if (MODE == FMODE_RESID) out[j] = out[j] + acc;
      else if (MODE == FMODE_RESID_BIAS) out[j] = out[j] + (acc + bias[j]);
      else if (MODE == FMODE_GELU_BIAS) out[j] = qd::gelu_tanh(acc + bias[j]);
      else out[j] = bias ? acc + bias[j] : acc;
    }
  } else {
    // tile tt is formed from register set tt % kFD into LDS buffer tt % 2, then
    // that set takes tile tt + kFD; one barrier per tile hands it to the chains
    for (int t0 = 0; t0 < ntile; t0 += kFD) {
#pragma unroll
      for (int d = 0; d < kFD; d++) {
        const int tt = t0 + d;
        if (tt < ntile) {
          f_produce(P + (tt & 1) * kFC * kFS, xs, r[d], tt, u, dd);
          f_load(r[d], rs, vo, tt + kFD, ntile);
          qd::lds_sync();
        }
      }
    }
  }
}

// (K, N) row-major -> panels of 16 columns (see the top of this file)
__global__ void k_to_panels(const float *src, int K, int N, float *dst) {
  const size_t i = (size_t)blockIdx.x * 256 + threadIdx.x;
  const int np = (N + kFC - 1) / kFC;
  if (i >= (size_t)K * np * kFC) return;
  const int dd = (int)(i % kFC);
  const size_t r = i / kFC;
  const int k = (int)(r % K), p = (int)(r / K);
  const int j = p * kFC + dd;
  dst[i] = j < N ? src[(size_t)k * N + j] : 0.0f;
}

// x = wte[token] (llama.c:304), token = d_in[d_state[0]]
__global__ void k_embed_f32(const float *wte, int dm, const int *d_in, const int *d_state, float *x) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= dm) return;
  x[j] = wte[(size_t)d_in[d_state[0]] * dm + j];
}

// Row r of x = wte[ids[r]] (llama.c:172-174)
__global__ void k_embed_f32_rows(const float *wte, int dm, const int *ids, float *x) {
  const int j = blockIdx.x * 256 + threadIdx.x, r = blockIdx.y;
  if (j >= dm) return;
  x[(size_t)r * dm + j] = wte[(size_t)ids[r] * dm + j];
}

// y = rmsnorm(x) (rmsnorm.c:7-21), one block per row of dm floats
template <int NT, int CM>
__global__ __launch_bounds__(NT) void k_rmsnorm_f32(const float *x, int dm, const float *gamma, float eps, float *y) {
  __shared__ float red[NT / 64];
  __shared__ qd::SeqScratch seq;
  x += (size_t)blockIdx.x * dm;
  y += (size_t)blockIdx.x * dm;
  float v[CM];
  (void)qd::rmsnorm_row<NT, CM>(x, dm, gamma, eps, v, red, seq);
  const int j0 = threadIdx.x * CM;
#pragma unroll
  for (int c = 0; c < CM; c++)
    if (j0 + c < dm) y[j0 + c] = v[c];
}

// h = SiLU(g) * u = (g * (1 / (1 + expf(-g)))) * u over gu = [g | u] (swiglu.c:7-10, 36-39),
// row blockIdx.y of gu [rows][2 dff] into h [rows][dff]
__global__ void k_swiglu_f32(const float *gu, int dff, float *h) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= dff) return;
  gu += (size_t)blockIdx.y * 2 * dff;
  h += (size_t)blockIdx.y * dff;
  const float z = gu[j];
  const float s = 1.0f / (1.0f + qd::expf_glibc(-z));
  h[j] = (z * s) * gu[dff + j];
}

// ---------------------------------------------------------------------------
// Many-row f32 matmul (matrix.c:178-190 over M rows): the GEMMs of the batched
// forward.  Every output element is one serial chain in k order, the
// reference's, with each product rounded before its add.  A 64 x 64 block tile
// gives each of 256 threads 4 rows x 4 columns, 16 independent chains; K is
// staged kKT rows at a time through LDS (A transposed to [k][row], W from the
// block's four panels as [k][column]), and the next stage's global loads are in
// flight while the current one is summed.  A chain takes exactly K terms: a
// padded 0 * w term would turn a -0 sum into +0.
// ---------------------------------------------------------------------------
constexpr int kMT = 64;           // rows per block tile
constexpr int kNT = 4 * kFC;      // columns per block tile: four panels
constexpr int kKT = 32;           // k rows per LDS stage
constexpr int kAS = kMT + 4;      // LDS stride of a k row of A
constexpr int kWS = kNT + 4;      // LDS stride of a k row of W

template <int MODE>
__global__ __launch_bounds__(256) void k_gemm_f32(const float *A, int M, int K, const float *W, int N, float *out,
                                                  const float *bias) {
  __shared__ __align__(16) float As[kKT * kAS];
  __shared__ __align__(16) float Ws[kKT * kWS];
  const int tid = threadIdx.x;
  const int i0 = blockIdx.y * kMT, j0 = blockIdx.x * kNT;
  const int np = (N + kFC - 1) / kFC;
  const bool vec = (K & 3) == 0 && (reinterpret_cast<uintptr_t>(A) & 15) == 0;   // whole aligned float4s
  // staging of A: thread -> row ar, k offsets ak .. ak+7 of the stage
  const int ar = tid >> 2, ak = (tid & 3) * 8;
  const bool arow = i0 + ar < M;
  const float *Ar = A + (size_t)(arow ? i0 + ar : 0) * K;
  // staging of W: float4 f = tid + 256 g is panel f / 128, k row (f % 128) / 4, column quad f % 4
  float av[8];
  float4 wv[2];
  auto gload = [&](int k0) {
    if (vec) {
#pragma unroll
      for (int h = 0; h < 2; h++) {
        const int k = k0 + ak + 4 * h;
        const float4 v = arow && k < K ? *reinterpret_cast<const float4 *>(Ar + k) : make_float4(0.f, 0.f, 0.f, 0.f);
        av[4 * h] = v.x; av[4 * h + 1] = v.y; av[4 * h + 2] = v.z; av[4 * h + 3] = v.w;
      }
    } else {
#pragma unroll
      for (int e = 0; e < 8; e++) av[e] = arow && k0 + ak + e < K ? Ar[k0 + ak + e] : 0.0f;
    }
#pragma unroll
    for (int g = 0; g < 2; g++) {
      const int f = tid + 256 * g, p = blockIdx.x * 4 + (f >> 7), k = k0 + ((f & 127) >> 2);
      wv[g] = p < np && k < K ? *reinterpret_cast<const float4 *>(W + ((size_t)p * K + k) * kFC + (f & 3) * 4)
                              : make_float4(0.f, 0.f, 0.f, 0.f);
    }
  };
  const int ty = tid >> 4, tx = tid & 15;
  float acc[4][4];
#pragma unroll
  for (int r = 0; r < 4; r++)
#pragma unroll
    for (int c = 0; c < 4; c++) acc[r][c] = 0.0f;
  gload(0);
  for (int k0 = 0; k0 < K; k0 += kKT) {
    __syncthreads();                              // the previous stage is summed
#pragma unroll
    for (int e = 0; e < 8; e++) As[(ak + e) * kAS + ar] = av[e];
#pragma unroll
    for (int g = 0; g < 2; g++) {
      const int f = tid + 256 * g;
      *reinterpret_cast<float4 *>(&Ws[((f & 127) >> 2) * kWS + (f >> 7) * kFC + (f & 3) * 4]) = wv[g];
    }
    __syncthreads();
    if (k0 + kKT < K) gload(k0 + kKT);
    const int kn = min(kKT, K - k0);
    auto step = [&](int kk) {
      const float4 a = *reinterpret_cast<const float4 *>(&As[kk * kAS + ty * 4]);
      const float4 w = *reinterpret_cast<const float4 *>(&Ws[kk * kWS + tx * 4]);
      const float ar4[4] = {a.x, a.y, a.z, a.w}, wr4[4] = {w.x, w.y, w.z, w.w};
#pragma unroll
      for (int r = 0; r < 4; r++)
#pragma unroll
        for (int c = 0; c < 4; c++) acc[r][c] = acc[r][c] + ar4[r] * wr4[c];
    };
    if (kn == kKT) {
#pragma unroll 8
      for (int kk = 0; kk < kKT; kk++) step(kk);
    } else {
      for (int kk = 0; kk < kn; kk++) step(kk);
    }
  }
#pragma unroll
  for (int r = 0; r < 4; r++) {
    const int i = i0 + ty * 4 + r;
    if (i >= M) continue;
#pragma unroll
    for (int c = 0; c < 4; c++) {
      const int j = j0 + tx * 4 + c;
      if (j >= N) continue;
      float *o = out + (size_t)i * N + j;
      if (MODE == FMODE_RESID) *o = *o + acc[r][c];
      else *o = bias ? acc[r][c] + bias[j] : acc[r][c];
    }
  }
}

size_t gemv_lds(int K) { return ((size_t)(K + kFT - 1) / kFT * kFT + 2 * kFC * kFS) * 4; }
size_t g_lds_attr[4] = {0, 0, 0, 0};

}  // namespace

// Largest K the fp32 GEMV takes (x and two product tiles in LDS).
extern "C" int qhip_gemv_f32_max_k(void) { return 32768; }

extern "C" int qhip_gemv_f32(int mode, int cls, const float *x, int K, const float *W, int N, float *out,
                             const float *bias) {
  if (K <= 0 || N <= 0 || K > qhip_gemv_f32_max_k()) return qh::fail_msg("gemv_f32: bad shape");
  if (mode < 0 || mode > 3 || (mode >= 2 && !bias)) return qh::fail_msg("gemv_f32: bad mode");
  const size_t lds = gemv_lds(K);
  const void *fns[4] = {reinterpret_cast<const void *>(k_gemv_f32<FMODE_PLAIN>),
                        reinterpret_cast<const void *>(k_gemv_f32<FMODE_RESID>),
                        reinterpret_cast<const void *>(k_gemv_f32<FMODE_RESID_BIAS>),
                        reinterpret_cast<const void *>(k_gemv_f32<FMODE_GELU_BIAS>)};
  if (lds > 64 * 1024 && lds > g_lds_attr[mode]) {
    hipError_t e = hipFuncSetAttribute(fns[mode], hipFuncAttributeMaxDynamicSharedMemorySize, (int)lds);
    if (e != hipSuccess) return qh::fail("hipFuncSetAttribute(k_gemv_f32)", e);
    g_lds_attr[mode] = lds;
  }
  const dim3 grid((N + kFC - 1) / kFC);
  switch (mode) {
    case 0: QH_LAUNCH(cls, k_gemv_f32<FMODE_PLAIN>, grid, dim3(kFThreads), lds, x, K, W, N, out, bias); break;
    case 1: QH_LAUNCH(cls, k_gemv_f32<FMODE_RESID>, grid, dim3(kFThreads), lds, x, K, W, N, out, bias); break;
    case 2: QH_LAUNCH(cls, k_gemv_f32<FMODE_RESID_BIAS>, grid, dim3(kFThreads), lds, x, K, W, N, out, bias); break;
    default: QH_LAUNCH(cls, k_gemv_f32<FMODE_GELU_BIAS>, grid, dim3(kFThreads), lds, x, K, W, N, out, bias); break;
  }
  return 0;
}

// Floats of a (K, N) matrix in the panel layout.
extern "C" size_t qhip_panels_f32_size(int K, int N) { return (size_t)K * ((N + kFC - 1) / kFC) * kFC; }

extern "C" int qhip_to_panels_f32(const float *src, int K, int N, float *dst) {
  const size_t n = qhip_panels_f32_size(K, N);
  QH_LAUNCH(QK_OTHER, k_to_panels, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, src, K, N, dst);
  return 0;
}

extern "C" int qhip_embed_f32(const float *wte, int dm, const int *d_in, const int *d_state, float *x) {
  QH_LAUNCH(QK_EMBED, k_embed_f32, dim3((dm + 255) / 256), dim3(256), 0, wte, dm, d_in, d_state, x);
  return 0;
}

extern "C" int qhip_rmsnorm_f32_rows(const float *x, int R, int dm, const float *gamma, float eps, float *y) {
  const dim3 g(R);
  if (R <= 0) return qh::fail_msg("rmsnorm_f32: no rows");
  if (dm <= 256 * 4) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 4>), g, dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 256 * 8) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 8>), g, dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 256 * 16) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 16>), g, dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 256 * 32) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 32>), g, dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 1024 * 16) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<1024, 16>), g, dim3(1024), 0, x, dm, gamma, eps, y);
  else return qh::fail_msg("rmsnorm_f32: d_model above 16384");
  return 0;
}

extern "C" int qhip_rmsnorm_f32(const float *x, int dm, const float *gamma, float eps, float *y) {
  return qhip_rmsnorm_f32_rows(x, 1, dm, gamma, eps, y);
}

extern "C" int qhip_swiglu_f32_rows(const float *gu, int R, int dff, float *h) {
  QH_LAUNCH(QK_SWIGLU, k_swiglu_f32, dim3((dff + 255) / 256, R), dim3(256), 0, gu, dff, h);
  return 0;
}

extern "C" int qhip_swiglu_f32(const float *gu, int dff, float *h) { return qhip_swiglu_f32_rows(gu, 1, dff, h); }

extern "C" int qhip_embed_f32_rows(const float *wte, int dm, const int *ids, int R, float *x) {
  QH_LAUNCH(QK_EMBED, k_embed_f32_rows, dim3((dm + 255) / 256, R), dim3(256), 0, wte, dm, ids, x);
  return 0;
}

extern "C" int qhip_gemm_f32(int mode, int cls, const float *A, int M, int K, const float *W, int N, float *out,
                             const float *bias) {
  if (M <= 0 || K <= 0 || N <= 0 || M > 65535 * kMT) return qh::fail_msg("gemm_f32: bad shape");
  const dim3 grid((N + kNT - 1) / kNT, (M + kMT - 1) / kMT);
  if (mode == 0) QH_LAUNCH(cls, k_gemm_f32<FMODE_PLAIN>, grid, dim3(256), 0, A, M, K, W, N, out, bias);
  else if (mode == 1) QH_LAUNCH(cls, k_gemm_f32<FMODE_RESID>, grid, dim3(256), 0, A, M, K, W, N, out, bias);
  else return qh::fail_msg("gemm_f32: bad mode");
  return 0;
}
