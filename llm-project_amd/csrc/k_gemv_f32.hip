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

// y = rmsnorm(x) (rmsnorm.c:7-21), one block
template <int NT, int CM>
__global__ __launch_bounds__(NT) void k_rmsnorm_f32(const float *x, int dm, const float *gamma, float eps, float *y) {
  __shared__ float red[NT / 64];
  __shared__ qd::SeqScratch seq;
  float v[CM];
  (void)qd::rmsnorm_row<NT, CM>(x, dm, gamma, eps, v, red, seq);
  const int j0 = threadIdx.x * CM;
#pragma unroll
  for (int c = 0; c < CM; c++)
    if (j0 + c < dm) y[j0 + c] = v[c];
}

// h = SiLU(g) * u = (g * (1 / (1 + expf(-g)))) * u over gu = [g | u] (swiglu.c:7-10, 36-39)
__global__ void k_swiglu_f32(const float *gu, int dff, float *h) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= dff) return;
  const float z = gu[j];
  const float s = 1.0f / (1.0f + qd::expf_glibc(-z));
  h[j] = (z * s) * gu[dff + j];
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

extern "C" int qhip_rmsnorm_f32(const float *x, int dm, const float *gamma, float eps, float *y) {
  if (dm <= 256 * 4) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 4>), dim3(1), dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 256 * 8) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 8>), dim3(1), dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 256 * 16) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 16>), dim3(1), dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 256 * 32) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<256, 32>), dim3(1), dim3(256), 0, x, dm, gamma, eps, y);
  else if (dm <= 1024 * 16) QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_f32<1024, 16>), dim3(1), dim3(1024), 0, x, dm, gamma, eps, y);
  else return qh::fail_msg("rmsnorm_f32: d_model above 16384");
  return 0;
}

extern "C" int qhip_swiglu_f32(const float *gu, int dff, float *h) {
  QH_LAUNCH(QK_SWIGLU, k_swiglu_f32, dim3((dff + 255) / 256), dim3(256), 0, gu, dff, h);
  return 0;
}
