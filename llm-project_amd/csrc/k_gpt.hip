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
//   mean = (sum_j x_j, in order) / cols       -- a serial chain (signed terms)
//   var  = (sum_j (x_j - mean)^2, in order) / cols   -- exact parallel sum (qdev_seqsum.h)
//   y_j  = ((x_j - mean) * (1 / sqrtf(var + eps))) * gamma_j + beta_j
template <int NT, int CM>
__global__ __launch_bounds__(NT) void k_layernorm_f32(const float *x, int dm, const float *gamma, const float *beta,
                                                      float eps, float *y) {
  __shared__ float xs[NT * CM];
  __shared__ qd::SeqScratch seq;
  __shared__ float mean_s;
  const int j0 = threadIdx.x * CM;
  float v[CM];
#pragma unroll
  for (int c = 0; c < CM; c++) {
    v[c] = j0 + c < dm ? x[j0 + c] : 0.0f;
    xs[j0 + c] = v[c];                                  // +0 past dm: adds nothing to the chain
  }
  qd::lds_sync();
  if (threadIdx.x == 0) {
    float s = 0.0f;
    for (int j = 0; j < dm; j += 8) {                   // eight loads in flight ahead of the adds
      float t[8];
#pragma unroll
      for (int u = 0; u < 8; u++) t[u] = j + u < dm ? xs[j + u] : 0.0f;
#pragma unroll
      for (int u = 0; u < 8; u++) s += t[u];
    }
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
      y[j0 + c] = t * gamma[j0 + c] + beta[j0 + c];
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
