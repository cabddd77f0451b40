// k_decode.hip - the per-token kernels of the int8 decode step.
//
// Bit-exactness with the reference CPU path rests on three rules kept in every
// kernel here: integer dot products are exact in any order; every floating
// point sum the reference forms sequentially (rmsnorm's sum of squares, the
// attention dot products, the softmax denominator and the weighted sum of V) is
// formed here in the same sequential order; and no product is fused into an add
// (the library is compiled with -ffp-contract=off, as ISO C11 compiles the
// reference).  Maxima are order independent.
#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qdev_norm.h"
#include "qdev_seqsum.h"
#include "qhip.h"
#include "qhip_internal.h"
#include "qllama.h"

namespace {

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

// Write row `row` of qa (int8, kpad wide, zero padded) from values v[0..n) held
// in LDS, given the row's max |v| (quant.c:66-78).
// Four codes per thread and store (kpad is a multiple of 16).
__device__ __forceinline__ void quantize_row_lds(const float *v, int n, int kpad, float mx, int8_t *qa_row,
                                                 float *as_out) {
  const float as = (mx > 0.0f) ? mx / 127.0f : 1.0f;
  const float inv = 1.0f / as;
  for (int k = 4 * threadIdx.x; k < kpad; k += 4 * blockDim.x) {
    const float a = k < n ? v[k] : 0.0f, b = k + 1 < n ? v[k + 1] : 0.0f;
    const float c = k + 2 < n ? v[k + 2] : 0.0f, d = k + 3 < n ? v[k + 3] : 0.0f;
    *reinterpret_cast<uint32_t *>(qa_row + k) = qd::quant_i8x4(a, b, c, d, inv);
  }
  if (threadIdx.x == 0) *as_out = as;
}

// x[j] = (float)wte[token*dm + j] * scale[j]   (llama.c:534-536)
__global__ void k_embed(const int8_t *wte, const float *s, int dm, const int *d_in, const int *d_state, float *x) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= dm) return;
  const int tok = d_in[d_state[0]];
  x[j] = (float)wte[(size_t)tok * dm + j] * s[j];
}

// One block per row: rmsnorm.c:7-21 then the activation quantization of qmatmul.
// Thread t holds elements [t*CM, t*CM + CM) (NT*CM >= kpad).
template <int NT, int CM>
__global__ __launch_bounds__(NT) void k_rmsnorm_quant(const float *x, int dm, const float *gamma, float eps,
                                                       int8_t *qa, int kpad, float *as) {
  __shared__ float red[NT / 64];
  __shared__ qd::SeqScratch seq;
  const int row = blockIdx.x;
  const int j0 = threadIdx.x * CM;
  float y[CM];
  const float a_s = qd::rmsnorm_row<NT, CM>(x + (size_t)row * dm, dm, gamma, eps, y, red, seq);
  const float inv = 1.0f / a_s;
  int8_t *qr = qa + (size_t)row * kpad;
#pragma unroll
  for (int c = 0; c < CM; c += 4)
    if (j0 + c < kpad) *reinterpret_cast<uint32_t *>(qr + j0 + c) = qd::quant_word(y, c, inv);
  if (threadIdx.x == 0) as[row] = a_s;
}

// One block per row: quantize v (rows, n) -> qa (rows, kpad), as (rows).
__global__ __launch_bounds__(1024) void k_quant_rows(const float *vin, int n, int8_t *qa, int kpad, float *as) {
  extern __shared__ float lds[];
  __shared__ float red[16];
  const int row = blockIdx.x;
  const float *vr = vin + (size_t)row * n;
  float mx = 0.0f;
  if ((n & 3) == 0 && (reinterpret_cast<uintptr_t>(vr) & 15) == 0) {   // whole aligned 16-byte words
    const float4 *v4 = reinterpret_cast<const float4 *>(vr);
    float4 *l4 = reinterpret_cast<float4 *>(lds);
    for (int j = threadIdx.x; j < n / 4; j += blockDim.x) {
      const float4 a = v4[j];
      l4[j] = a;
      mx = fmaxf(fmaxf(mx, fmaxf(fabsf(a.x), fabsf(a.y))), fmaxf(fabsf(a.z), fabsf(a.w)));
    }
  } else {
    for (int j = threadIdx.x; j < n; j += blockDim.x) {
      const float a = vr[j];
      lds[j] = a;
      mx = fmaxf(mx, fabsf(a));
    }
  }
  mx = block_max(mx, red);
  __syncthreads();
  quantize_row_lds(lds, n, kpad, mx, qa + (size_t)row * kpad, as + row);
}

// h_j = (z * (1 / (1 + expf(-z)))) * u_j over gu = [g | u]  (llama.c:583-587), then quantize h.
__global__ __launch_bounds__(1024) void k_swiglu_quant(const float *gu, int dff, int8_t *qa, int kpad, float *as) {
  extern __shared__ float lds[];
  __shared__ float red[16];
  const int row = blockIdx.x;
  const float *g = gu + (size_t)row * 2 * dff, *u = g + dff;
  float mx = 0.0f;
  for (int j = threadIdx.x; j < dff; j += blockDim.x) {
    const float z = g[j];
    const float s = 1.0f / (1.0f + qd::expf_glibc(-z));
    const float h = (z * s) * u[j];
    lds[j] = h;
    mx = fmaxf(mx, fabsf(h));
  }
  mx = block_max(mx, red);
  __syncthreads();
  quantize_row_lds(lds, dff, kpad, mx, qa + (size_t)row * kpad, as + row);
}

// W8A8 GEMV: one wave per output channel j; lanes stride K in 16-byte chunks and
// accumulate exact int32 dot products (v_dot4), reduced across the wave.
// Epilogue: c = (as * ws[j]) * (float)acc  (quant.c:81-82), then + bias or
// residual (llama.c:546-548, 578, 589).  W is [N][kpad], qa is [rows][kpad].
constexpr int kMaxRows = 8;
__global__ __launch_bounds__(256) void k_gemv(const int8_t *qa, const float *as, int rows, const int8_t *W,
                                              const float *ws, int N, int kpad, float *out, const float *bias,
                                              int residual) {
  const int lane = threadIdx.x & 63;
  const int j = blockIdx.x * 4 + (threadIdx.x >> 6);
  if (j >= N) return;
  const int nchunk = kpad >> 4;
  const int4 *wrow = reinterpret_cast<const int4 *>(W + (size_t)j * kpad);
  int acc[kMaxRows];
#pragma unroll
  for (int m = 0; m < kMaxRows; m++) acc[m] = 0;
  for (int c = lane; c < nchunk; c += 64) {
    const int4 w = wrow[c];
#pragma unroll
    for (int m = 0; m < kMaxRows; m++) {
      if (m < rows) {
        const int4 a = reinterpret_cast<const int4 *>(qa + (size_t)m * kpad)[c];
        int t = acc[m];
        t = __builtin_amdgcn_sdot4(a.x, w.x, t, false);
        t = __builtin_amdgcn_sdot4(a.y, w.y, t, false);
        t = __builtin_amdgcn_sdot4(a.z, w.z, t, false);
        t = __builtin_amdgcn_sdot4(a.w, w.w, t, false);
        acc[m] = t;
      }
    }
  }
  const float wsj = ws[j];
#pragma unroll
  for (int m = 0; m < kMaxRows; m++) {
    if (m < rows) {
      const int a = qd::wave_sum_i32(acc[m]);
      if (lane == 0) {
        const float c = (as[m] * wsj) * (float)a;
        float *o = out + (size_t)m * N + j;
        if (residual) *o = *o + c;
        else *o = bias ? c + bias[j] : c;
      }
    }
  }
}

// Prompt rows: x[r][j] = (float)wte[ids[r]*dm + j] * scale[j]  (llama.c:534-536)
__global__ void k_pf_embed(const int8_t *wte, const float *s, int dm, const int *ids, float *x) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x, r = blockIdx.y;
  if (j >= dm) return;
  x[(size_t)r * dm + j] = (float)wte[(size_t)ids[r] * dm + j] * s[j];
}

// Prompt rows: RoPE at position p0 + r (rope.c:48-68) with cos/sin from the host
// tables; query heads rotate into q_out row r, key heads into the cache at
// p0 + r, and value heads are copied there.  One block per row: the threads
// take the (k, k + hd/2) pairs of the H + KVH rotated heads, then the value
// elements.
__global__ __launch_bounds__(256) void k_pf_rope_append(const float *qkv, int H, int KVH, int hd,
                                                        const float *cos_t, const float *sin_t, int p0, float *q_out,
                                                        float *kc, float *vc, int max_seq) {
  const int r = blockIdx.x, pos = p0 + r;
  const int half = hd >> 1;
  const int nqkv = (H + 2 * KVH) * hd;
  const float *row = qkv + (size_t)r * nqkv;
  const float *ct = cos_t + (size_t)pos * half, *st = sin_t + (size_t)pos * half;
  const int nrot = (H + KVH) * half;
  for (int i = threadIdx.x; i < nrot; i += blockDim.x) {
    const int b = i / half, k = i % half;
    const float *xh = row + (size_t)b * hd;
    float *dst = b < H ? q_out + (size_t)r * H * hd + (size_t)b * hd : kc + ((size_t)(b - H) * max_seq + pos) * hd;
    const float c = ct[k], s = st[k];
    const float x1 = xh[k], x2 = xh[k + half];
    dst[k] = x1 * c - x2 * s;
    dst[k + half] = x2 * c + x1 * s;
  }
  const float *vrow = row + (size_t)(H + KVH) * hd;
  for (int i = threadIdx.x; i < KVH * hd; i += blockDim.x) {
    const int h = i / hd, d = i % hd;
    vc[((size_t)h * max_seq + pos) * hd + d] = vrow[i];
  }
}

// matrix.c:354-374 on the reference's row-major (K, N) layout: one thread per column.
__global__ void k_qacc_kn(const int8_t *qa, const int8_t *qw, int K, int N, int32_t *acc) {
  const int j = blockIdx.x * blockDim.x + threadIdx.x;
  if (j >= N) return;
  int a = 0;
  for (int k = 0; k < K; k++) a += (int)qa[k] * (int)qw[(size_t)k * N + j];
  acc[j] = a;
}


}  // namespace

extern "C" {

int qhip_embed(const int8_t *wte, const float *wte_s, int dm, const int *d_in, const int *d_state, float *x) {
  QH_LAUNCH(QK_EMBED, k_embed, dim3((dm + 255) / 256), dim3(256), 0, wte, wte_s, dm, d_in, d_state, x);
  return 0;
}

int qhip_rmsnorm_quant(const float *x, int rows, int dm, const float *gamma, float eps, int8_t *qa, int kpad,
                       float *as) {
  if (kpad % 4 || kpad < dm) return qh::fail_msg("rmsnorm_quant: bad row padding");
  if (kpad <= 1024)
    QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_quant<64, 16>), dim3(rows), dim3(64), 0, x, dm, gamma, eps, qa, kpad, as);
  else if (kpad <= 4096)
    QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_quant<256, 16>), dim3(rows), dim3(256), 0, x, dm, gamma, eps, qa, kpad, as);
  else if (kpad <= 8192)
    QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_quant<256, 32>), dim3(rows), dim3(256), 0, x, dm, gamma, eps, qa, kpad, as);
  else if (kpad <= 16384)
    QH_LAUNCH(QK_RMSNORM, (k_rmsnorm_quant<512, 32>), dim3(rows), dim3(512), 0, x, dm, gamma, eps, qa, kpad, as);
  else
    return qh::fail_msg("rmsnorm_quant: d_model above 16384");
  return 0;
}

int qhip_quant_rows(const float *v, int rows, int n, int8_t *qa, int kpad, float *as) {
  if (n > 32768) return qh::fail_msg("quant_rows: row above 32768");
  if (kpad % 16 || kpad < n) return qh::fail_msg("quant_rows: bad row padding");
  QH_LAUNCH(QK_QUANT, k_quant_rows, dim3(rows), dim3(1024), (size_t)n * 4, v, n, qa, kpad, as);
  return 0;
}

int qhip_swiglu_quant(const float *gu, int rows, int dff, int8_t *qa, int kpad, float *as) {
  if (dff > 32768) return qh::fail_msg("swiglu_quant: d_ff above 32768");
  if (kpad % 16 || kpad < dff) return qh::fail_msg("swiglu_quant: bad row padding");
  QH_LAUNCH(QK_SWIGLU, k_swiglu_quant, dim3(rows), dim3(1024), (size_t)dff * 4, gu, dff, qa, kpad, as);
  return 0;
}

int qhip_gemv(const int8_t *qa, const float *as, int rows, const int8_t *W, const float *ws, int N, int kpad,
              float *out, const float *bias, int residual, int cls) {
  if (kpad % 16) return qh::fail_msg("gemv: kpad must be a multiple of 16");
  for (int m0 = 0; m0 < rows; m0 += kMaxRows) {
    const int r = rows - m0 < kMaxRows ? rows - m0 : kMaxRows;
    QH_LAUNCH(cls, k_gemv, dim3((N + 3) / 4), dim3(256), 0, qa + (size_t)m0 * kpad, as + m0,
              r, W, ws, N, kpad, out + (size_t)m0 * N, bias, residual);
  }
  return 0;
}

int qhip_pf_embed(const int8_t *wte, const float *wte_s, int dm, const int *ids, int R, float *x) {
  QH_LAUNCH(QK_PF_OTHER, k_pf_embed, dim3((dm + 255) / 256, R), dim3(256), 0, wte, wte_s, dm, ids, x);
  return 0;
}

int qhip_pf_rope_append(const float *qkv, int R, int n_heads, int n_kv, int hd, const float *cos_t,
                        const float *sin_t, int p0, float *q_out, float *kc, float *vc, int max_seq) {
  QH_LAUNCH(QK_PF_OTHER, k_pf_rope_append, dim3(R), dim3(256), 0, qkv, n_heads, n_kv, hd, cos_t, sin_t, p0, q_out,
            kc, vc, max_seq);
  return 0;
}

int qhip_qacc_kn(const int8_t *qa, const int8_t *qw, int K, int N, int32_t *acc) {
  QH_LAUNCH(QK_OTHER, k_qacc_kn, dim3((N + 255) / 256), dim3(256), 0, qa, qw, K, N, acc);
  return 0;
}

}  // extern "C"

// ---------------------------------------------------------------------------
// test entry points
// ---------------------------------------------------------------------------
namespace {
// expf_glibc of inputs start .. start+count-1, eight consecutive inputs per lane
// also through expf_glibc_n: where the two differ, the lowest bit of the output
// is flipped, so that the host comparison fails for either form.
__global__ void k_expf_range(uint32_t start, uint32_t count, float *out) {
  const uint32_t stride = gridDim.x * blockDim.x * 8u;
  for (uint32_t i0 = (blockIdx.x * blockDim.x + threadIdx.x) * 8u; i0 < count; i0 += stride) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; u++) v[u] = __uint_as_float(start + i0 + u);
    float a[8];
#pragma unroll
    for (int u = 0; u < 8; u++) a[u] = v[u];
    qd::expf_glibc_n<8>(a, qd::kExp2Tab);
#pragma unroll
    for (int u = 0; u < 8; u++)
      if (i0 + u < count) {
        const uint32_t sc = __float_as_uint(qd::expf_glibc(v[u]));
        out[i0 + u] = __uint_as_float(sc == __float_as_uint(a[u]) ? sc : sc ^ 1u);
      }
  }
}

// reference cache rows (T, n_kv*hd) -> [n_kv][T][hd]
__global__ void k_kv_relayout(const float *src, int T, int n_kv, int hd, float *dst) {
  const size_t n = (size_t)T * n_kv * hd;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) {
    const int d = (int)(i % hd);
    const int h = (int)((i / hd) % n_kv);
    const size_t t = i / ((size_t)hd * n_kv);
    dst[((size_t)h * T + t) * hd + d] = src[i];
  }
}
}  // namespace

extern "C" int qhip_kv_relayout(const float *src, int T, int n_kv, int hd, float *dst) {
  QH_LAUNCH(QK_OTHER, k_kv_relayout, dim3(4096), dim3(256), 0, src, T, n_kv, hd, dst);
  return 0;
}

extern "C" int qllama_test_expf(uint32_t start, uint32_t count, float *out) {
  if (qhip_init()) return 1;
  float *d = (float *)qhip_malloc((size_t)count * 4);
  if (!d) return 1;
  hipLaunchKernelGGL(k_expf_range, dim3(8192), dim3(256), 0, qh::stream(), start, count, d);
  int rc = qh::check_launch("k_expf_range");
  if (!rc) rc = qhip_d2h(out, d, (size_t)count * 4);
  qhip_free(d);
  return rc;
}

extern "C" int qllama_gqa_decode(const float *q, const float *k, const float *v, int T, int n_heads, int n_kv,
                                 int hd, float *o) {
  if (qhip_init()) return 1;
  if (T <= 0 || n_kv <= 0 || n_heads % n_kv || hd <= 0) return qh::fail_msg("gqa_decode: bad shape");
  const size_t kvn = (size_t)T * n_kv * hd;
  float *dq = (float *)qhip_malloc((size_t)n_heads * hd * 4), *dk = (float *)qhip_malloc(kvn * 4);
  float *dv = (float *)qhip_malloc(kvn * 4), *tmp = (float *)qhip_malloc(kvn * 4);
  float *dsc = (float *)qhip_malloc(qhip_attention_scratch(n_heads, T) * 4), *dout = (float *)qhip_malloc((size_t)n_heads * hd * 4);
  int *dpos = (int *)qhip_malloc(4);
  const int pos = T - 1;
  int rc = (!dq || !dk || !dv || !tmp || !dsc || !dout || !dpos) ? 1 : 0;
  if (!rc) rc = qhip_h2d(dq, q, (size_t)n_heads * hd * 4) || qhip_h2d(dpos, &pos, 4) ||
                qhip_h2d(tmp, k, kvn * 4);
  if (!rc) {
    hipLaunchKernelGGL(k_kv_relayout, dim3(4096), dim3(256), 0, qh::stream(), tmp, T, n_kv, hd, dk);
    rc = qh::check_launch("k_kv_relayout") || qhip_h2d(tmp, v, kvn * 4);
  }
  if (!rc) {
    hipLaunchKernelGGL(k_kv_relayout, dim3(4096), dim3(256), 0, qh::stream(), tmp, T, n_kv, hd, dv);
    rc = qh::check_launch("k_kv_relayout");
  }
  const float scale = 1.0f / sqrtf((float)hd);
  if (!rc) rc = qhip_attention(dq, dk, dv, dpos, n_heads, n_kv, hd, T, scale, dsc, dout, NULL);
  if (!rc) rc = qhip_d2h(o, dout, (size_t)n_heads * hd * 4);
  qhip_free(dq); qhip_free(dk); qhip_free(dv); qhip_free(tmp); qhip_free(dsc); qhip_free(dout); qhip_free(dpos);
  return rc;
}

namespace {
__global__ __launch_bounds__(1024) void k_seqsum_test(const float *a, int n, float *out, int *info) {
  constexpr int CM = 16;
  float t[CM];
  const int i0 = threadIdx.x * CM;
#pragma unroll
  for (int c = 0; c < CM; c++) t[c] = i0 + c < n ? a[i0 + c] : 0.0f;
  __shared__ qd::SeqScratch S;
  const float s = qd::seq_sum_nonneg<1024, CM>(t, n, S, [&](int i) { return a[i]; }, info);
  if (threadIdx.x == 0) out[0] = s;
}
}  // namespace

extern "C" int qllama_test_seqsum(const float *a, int n, float *out, int *info) {
  if (qhip_init()) return 1;
  if (n < 0 || n > 16384) return qh::fail_msg("seqsum: n out of range");
  float *da = (float *)qhip_malloc((size_t)(n + 4) * 4), *dout = (float *)qhip_malloc(16);
  int *dinfo = (int *)qhip_malloc(16);
  int rc = (!da || !dout || !dinfo) ? 1 : 0;
  if (!rc) rc = qhip_h2d(da, a, (size_t)n * 4);
  if (!rc) {
    hipLaunchKernelGGL(k_seqsum_test, dim3(1), dim3(1024), 0, qh::stream(), da, n, dout, dinfo);
    rc = qh::check_launch("k_seqsum_test");
  }
  if (!rc) rc = qhip_d2h(out, dout, 4) || qhip_d2h(info, dinfo, 8);
  qhip_free(da); qhip_free(dout); qhip_free(dinfo);
  return rc;
}

namespace {
typedef int v4i __attribute__((ext_vector_type(4)));
__global__ __launch_bounds__(256) void k_copy_v4(const v4i *src, v4i *dst, size_t n16) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    dst[i] = __builtin_nontemporal_load(&src[i]);
}
}  // namespace

// Reads every 16-byte word of a buffer twice the size of the memory-side cache,
// so that the next kernel finds neither its operands in L2 nor in that cache
// (cold timing of the op-level benchmarks).
__global__ __launch_bounds__(256) void k_flush_read(const v4i *src, size_t n16, int *sink) {
  int s = 0;
  for (size_t i = (size_t)blockIdx.x * blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x) {
    const v4i v = __builtin_nontemporal_load(src + i);
    s ^= v.x ^ v.y ^ v.z ^ v.w;
  }
  if (s == 0x5eed5eed) sink[0] = s;                // keeps the loads
}

namespace {
void *g_flush_buf = nullptr;
constexpr size_t kFlushBytes = (size_t)512 << 20;
}  // namespace

extern "C" int qhip_flush_caches(void) {
  if (!g_flush_buf) {
    if (hipMalloc(&g_flush_buf, kFlushBytes + 256) != hipSuccess) {
      g_flush_buf = nullptr;
      return qh::fail_msg("flush: allocation failed");
    }
    if (hipMemsetAsync(g_flush_buf, 1, kFlushBytes + 256, qh::stream()) != hipSuccess) return qh::fail_msg("flush");
  }
  QH_LAUNCH(QK_FLUSH, k_flush_read, dim3(4096), dim3(256), 0, (const v4i *)g_flush_buf, kFlushBytes / 16,
            (int *)((char *)g_flush_buf + kFlushBytes));
  return 0;
}

extern "C" int qllama_test_copy(size_t bytes) {
  if (qhip_init()) return 1;
  if (bytes == 0 || bytes % 16) return qh::fail_msg("test_copy: size must be a positive multiple of 16");
  void *a = qhip_malloc(bytes), *b = qhip_malloc(bytes);
  int rc = (!a || !b) ? 1 : 0;
  if (!rc) {
    hipLaunchKernelGGL(k_copy_v4, dim3(4096), dim3(256), 0, qh::stream(), (const v4i *)a, (v4i *)b, bytes / 16);
    rc = qh::check_launch("k_copy_v4");
  }
  if (!rc) rc = qhip_device_sync();
  qhip_free(a); qhip_free(b);
  return rc;
}
