// k_gpt.hip - the GPT-2 (GPTC) decode step's small kernels (model.c:457-520):
// the token + position embedding, LayerNorm with the reference's evaluation
// order, and the cache append.  The projections are the fp32 GEMV
// (k_gemv_f32.hip) and the attention is the exact decode attention (k_attn.hip)
// with the weights formed as e_j / sum.
#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qdev_seqsum.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

// x = wte[token] + wpe[pos] (model.c:467-469); token = d_in[pos], pos = d_state[0]
__global__ void k_gpt_embed(const float *wte, const float *wpe, int dm, const int *d_in, const int *d_state,
                            float *x) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= dm) return;
  const int pos = d_state[0];
  x[j] = wte[(size_t)d_in[pos] * dm + j] + wpe[(size_t)pos * dm + j];
}

// layernorm.c:8-38 for one row, one block of NT threads (thread t holds
// elements [t*CM, t*CM + CM)):
//   mean = (sum_j x_j, in order) / cols       -- a serial chain (signed terms), one lane
//   var  = (sum_j (x_j - mean)^2, in order) / cols   -- exact parallel sum (qdev_seqsum.h)
//   y_j  = ((x_j - mean) * (1 / sqrtf(var + eps))) * gamma_j + beta_j
template <int NT, int CM>
__global__ __launch_bounds__(NT) void k_layernorm_f32(const float *x, int dm, const float *gamma, const float *beta,
                                                      float eps, float *y) {
  __shared__ __attribute__((aligned(16))) float xs[NT * CM];
  __shared__ qd::SeqScratch seq;
  __shared__ float mean_s;
  const int j0 = threadIdx.x * CM;
  float v[CM], ga[CM], be[CM];
#pragma unroll
  for (int c = 0; c < CM; c++) {
    v[c] = j0 + c < dm ? x[j0 + c] : 0.0f;
    ga[c] = j0 + c < dm ? gamma[j0 + c] : 0.0f;       // requested now, used at the end
    be[c] = j0 + c < dm ? beta[j0 + c] : 0.0f;
  }
#pragma unroll
  for (int c = 0; c < CM; c++) xs[j0 + c] = v[c];
  qd::lds_sync();
  if (threadIdx.x == 0) {
    // the chain over exactly dm terms, 16 at a time from LDS with the next 16
    // requested before the current ones are added (the reads land while the
    // adds run); a tail of dm % 16 terms one by one
    const float4 *x4 = reinterpret_cast<const float4 *>(xs);
    const int n16 = dm / 16;
    float s = 0.0f;
    float4 a[4], b[4];
#pragma unroll
    for (int u = 0; u < 4; u++) a[u] = n16 > 0 ? x4[u] : make_float4(0.f, 0.f, 0.f, 0.f);
    for (int i = 0; i < n16; i++) {
      const int nx = i + 1 < n16 ? i + 1 : i;
#pragma unroll
      for (int u = 0; u < 4; u++) b[u] = x4[4 * nx + u];
#pragma unroll
      for (int u = 0; u < 4; u++) {
        s += a[u].x;
        s += a[u].y;
        s += a[u].z;
        s += a[u].w;
      }
#pragma unroll
      for (int u = 0; u < 4; u++) a[u] = b[u];
    }
    for (int j = 16 * n16; j < dm; j++) s += xs[j];
    mean_s = s / (float)dm;
  }
  qd::lds_sync();
  const float mean = mean_s;
  float sq[CM];
#pragma unroll
  for (int c = 0; c < CM; c++) {
    const float d = v[c] - mean;
    sq[c] = j0 + c < dm ? d * d : 0.0f;
  }
  float var = qd::seq_sum_nonneg<NT, CM>(sq, dm, seq, [&](int i) {
    const float d = x[i] - mean;
    return d * d;
  });
  var = var / (float)dm;
  const float inv_std = 1.0f / sqrtf(var + eps);
#pragma unroll
  for (int c = 0; c < CM; c++) {
    if (j0 + c < dm) {
      const float t = (v[c] - mean) * inv_std;
      y[j0 + c] = t * ga[c] + be[c];
    }
  }
}

// The new position's k and v rows (model.c:481-482) into the per-layer caches
// laid out [head][max_seq][head_dim]; qkv holds [q | k | v] of d_model each.
__global__ void k_gpt_kv_append(const float *qkv, int dm, int hd, int max_seq, const int *d_state, float *kc,
                                float *vc) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i >= dm) return;
  const int pos = d_state[0], h = i / hd, d = i % hd;
  const size_t at = ((size_t)h * max_seq + pos) * hd + d;
  kc[at] = qkv[dm + i];
  vc[at] = qkv[2 * dm + i];
}

__global__ void k_tanhf_test(uint32_t start, uint32_t count, float *out) {
  const uint32_t i = blockIdx.x * 256u + threadIdx.x;
  if (i < count) out[i] = qd::tanhf_glibc(__uint_as_float(start + i));
}

}  // namespace

// The device tanhf (the one GELU uses) on the float bit patterns start .. start +
// count - 1, written to host memory; for the exhaustive parity test.
extern "C" int qllama_test_tanhf(uint32_t start, uint32_t count, float *out) {
  if (qhip_init()) return 1;
  float *d = (float *)qhip_malloc((size_t)count * 4);
  if (!d) return 1;
  hipLaunchKernelGGL(k_tanhf_test, dim3((count + 255) / 256), dim3(256), 0, qh::stream(), start, count, d);
  int rc = qh::check_launch("k_tanhf_test") || qhip_d2h(out, d, (size_t)count * 4);
  qhip_free(d);
  return rc;
}

extern "C" int qhip_gpt_embed(const float *wte, const float *wpe, int dm, const int *d_in, const int *d_state,
                              float *x) {
  QH_LAUNCH(QK_EMBED, k_gpt_embed, dim3((dm + 255) / 256), dim3(256), 0, wte, wpe, dm, d_in, d_state, x);
  return 0;
}

extern "C" int qhip_layernorm_f32(const float *x, int dm, const float *gamma, const float *beta, float eps, float *y) {
  if (dm <= 256 * 4)
    QH_LAUNCH(QK_RMSNORM, (k_layernorm_f32<256, 4>), dim3(1), dim3(256), 0, x, dm, gamma, beta, eps, y);
  else if (dm <= 256 * 8)
    QH_LAUNCH(QK_RMSNORM, (k_layernorm_f32<256, 8>), dim3(1), dim3(256), 0, x, dm, gamma, beta, eps, y);
  else if (dm <= 256 * 16)
    QH_LAUNCH(QK_RMSNORM, (k_layernorm_f32<256, 16>), dim3(1), dim3(256), 0, x, dm, gamma, beta, eps, y);
  else if (dm <= 256 * 32)
    QH_LAUNCH(QK_RMSNORM, (k_layernorm_f32<256, 32>), dim3(1), dim3(256), 0, x, dm, gamma, beta, eps, y);
  else
    return qh::fail_msg("layernorm_f32: d_model above 8192");
  return 0;
}

extern "C" int qhip_gpt_kv_append(const float *qkv, int dm, int hd, int max_seq, const int *d_state, float *kc,
                                  float *vc) {
  QH_LAUNCH(QK_ROPE, k_gpt_kv_append, dim3((dm + 255) / 256), dim3(256), 0, qkv, dm, hd, max_seq, d_state, kc, vc);
  return 0;
}
