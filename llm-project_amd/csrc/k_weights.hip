// k_weights.hip - building and checking int8 weights on the device: the seeded
// generator, per-column quantization (quant.c:10-27), layout transposes and
// order-independent digests.  None of this is on the per-token path.
#include <hip/hip_runtime.h>

#include "qdev_math.h"
#include "qhip.h"
#include "qhip_internal.h"

namespace {

constexpr int kRowsPerBlock = 1024;   // NK kernels: 256 threads x 4 consecutive rows

__device__ __forceinline__ float block_max_256(float m, float *red) {
  m = qd::wave_max_f32(m);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = m;
  __syncthreads();
  if (threadIdx.x == 0) {
    float r = red[0];
    for (int i = 1; i < (int)(blockDim.x >> 6); i++) r = fmaxf(r, red[i]);
    red[0] = r;
  }
  __syncthreads();
  const float r = red[0];
  __syncthreads();
  return r;
}

// Logical reference index of (row i, col j); tied heads read the embedding
// generator transposed.
__device__ __forceinline__ uint64_t src_index(int i, int j, int rows, int cols, int transpose_src) {
  return transpose_src ? (uint64_t)j * (uint64_t)rows + (uint64_t)i : (uint64_t)i * (uint64_t)cols + (uint64_t)j;
}

// Per-column max|w| of a generated (rows, cols) matrix; grid (cols, ceil(rows/1024)).
__global__ __launch_bounds__(256) void k_synth_colmax_nk(uint64_t key, int rows, int cols, int transpose_src,
                                                         double sigma, unsigned *colmax) {
  __shared__ float red[4];
  const int j = blockIdx.x;
  const int i0 = blockIdx.y * kRowsPerBlock + threadIdx.x * 4;
  float m = 0.0f;
  for (int r = 0; r < 4; r++) {
    const int i = i0 + r;
    if (i < rows) m = fmaxf(m, fabsf(qd::gen_value(key, src_index(i, j, rows, cols, transpose_src), sigma)));
  }
  m = block_max_256(m, red);
  if (threadIdx.x == 0) atomicMax(&colmax[j], __float_as_uint(m));
}

// Quantize the generated column j into q[j*kpad + i]; rows..kpad-1 get 0.
__global__ __launch_bounds__(256) void k_synth_quant_nk(uint64_t key, int rows, int cols, int kpad, int transpose_src,
                                                        double sigma, const unsigned *colmax, int8_t *q,
                                                        float *scale) {
  const int j = blockIdx.x;
  const int i0 = blockIdx.y * kRowsPerBlock + threadIdx.x * 4;
  if (i0 >= kpad) return;
  const float mx = __uint_as_float(colmax[j]);
  const float s = (mx > 0.0f) ? mx / 127.0f : 1.0f;
  const float inv = 1.0f / s;
  if (blockIdx.y == 0 && threadIdx.x == 0) scale[j] = s;
  uint32_t packed = 0;
  for (int r = 0; r < 4; r++) {
    const int i = i0 + r;
    int v = 0;
    if (i < rows) v = qd::quant_i8(qd::gen_value(key, src_index(i, j, rows, cols, transpose_src), sigma), inv);
    packed |= (uint32_t)(uint8_t)(int8_t)v << (8 * r);
  }
  *reinterpret_cast<uint32_t *>(q + (size_t)j * kpad + i0) = packed;
}

// Row-major (KN) variants: a thread owns one column over a tile of 256 rows.
__global__ __launch_bounds__(256) void k_synth_colmax_kn(uint64_t key, int rows, int cols, double sigma,
                                                         unsigned *colmax) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= cols) return;
  const int r0 = blockIdx.y * 256, r1 = min(rows, r0 + 256);
  float m = 0.0f;
  for (int i = r0; i < r1; i++) m = fmaxf(m, fabsf(qd::gen_value(key, (uint64_t)i * cols + j, sigma)));
  atomicMax(&colmax[j], __float_as_uint(m));
}

__global__ __launch_bounds__(256) void k_synth_quant_kn(uint64_t key, int rows, int cols, double sigma,
                                                        const unsigned *colmax, int8_t *q, float *scale) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= cols) return;
  const float mx = __uint_as_float(colmax[j]);
  const float s = (mx > 0.0f) ? mx / 127.0f : 1.0f;
  const float inv = 1.0f / s;
  if (blockIdx.y == 0) scale[j] = s;
  const int r0 = blockIdx.y * 256, r1 = min(rows, r0 + 256);
  for (int i = r0; i < r1; i++)
    q[(size_t)i * cols + j] = (int8_t)qd::quant_i8(qd::gen_value(key, (uint64_t)i * cols + j, sigma), inv);
}

__global__ void k_synth_f32(uint64_t key, size_t n, double sigma, float *out) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    out[i] = qd::gen_value(key, i, sigma);
}

__global__ void k_fill_f32(float *p, size_t n, float v) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = v;
}

__global__ void k_fill_zero_u8(uint8_t *p, size_t n) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x) p[i] = 0;
}

__global__ void k_fill_zero_u128(uint4 *p, size_t n16) {
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n16; i += (size_t)gridDim.x * blockDim.x)
    p[i] = make_uint4(0, 0, 0, 0);
}

// Per-column max of a device f32 (rows, cols) matrix.
__global__ __launch_bounds__(256) void k_colmax_f32(const float *w, int rows, int cols, unsigned *colmax) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= cols) return;
  const int r0 = blockIdx.y * 256, r1 = min(rows, r0 + 256);
  float m = 0.0f;
  for (int i = r0; i < r1; i++) {
    const float a = fabsf(w[(size_t)i * cols + j]);
    if (a > m) m = a;
  }
  atomicMax(&colmax[j], __float_as_uint(m));
}

__global__ __launch_bounds__(256) void k_quant_f32_kn(const float *w, int rows, int cols, const unsigned *colmax,
                                                      int8_t *q, float *scale) {
  const int j = blockIdx.x * 256 + threadIdx.x;
  if (j >= cols) return;
  const float mx = __uint_as_float(colmax[j]);
  const float s = (mx > 0.0f) ? mx / 127.0f : 1.0f;
  const float inv = 1.0f / s;
  if (blockIdx.y == 0) scale[j] = s;
  const int r0 = blockIdx.y * 256, r1 = min(rows, r0 + 256);
  for (int i = r0; i < r1; i++) q[(size_t)i * cols + j] = (int8_t)qd::quant_i8(w[(size_t)i * cols + j], inv);
}

__global__ void k_dequant_kn(const int8_t *q, const float *scale, int rows, int cols, float *w) {
  const size_t n = (size_t)rows * cols;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    w[i] = (float)q[i] * scale[i % (size_t)cols];
}

// (rows, cols) row-major int8 -> dst[j*kpad + i], 64x64 tiles through LDS; rows..kpad-1 -> 0.
__global__ __launch_bounds__(256) void k_transpose_kn_nk(const int8_t *src, int rows, int cols, int kpad,
                                                         int8_t *dst) {
  __shared__ int tile[64][65];
  const int i0 = blockIdx.x * 64, j0 = blockIdx.y * 64;
  const int t = threadIdx.x;
  for (int r = 0; r < 16; r++) {
    const int ii = r * 4 + (t >> 6), jj = t & 63;
    const int i = i0 + ii, j = j0 + jj;
    tile[ii][jj] = (i < rows && j < cols) ? (int)src[(size_t)i * cols + j] : 0;
  }
  __syncthreads();
  for (int r = 0; r < 16; r++) {
    const int jj = r * 4 + (t >> 6), ii = t & 63;
    const int i = i0 + ii, j = j0 + jj;
    if (j < cols && i < kpad) dst[(size_t)j * kpad + i] = (int8_t)tile[ii][jj];
  }
}

// q[j*kpad + i] -> dst[i*cols + j]; grid (cols, ceil(rows/256))
__global__ __launch_bounds__(256) void k_nk_to_kn(const int8_t *src, int rows, int cols, int kpad, int8_t *dst) {
  const int j = blockIdx.x, i = blockIdx.y * 256 + threadIdx.x;
  if (i < rows) dst[(size_t)i * cols + j] = src[(size_t)j * kpad + i];
}

__device__ __forceinline__ unsigned long long block_sum_u64(unsigned long long v, unsigned long long *red) {
#pragma unroll
  for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, 64);
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  if (lane == 0) red[w] = v;
  __syncthreads();
  unsigned long long r = 0;
  if (threadIdx.x == 0)
    for (int i = 0; i < (int)(blockDim.x >> 6); i++) r += red[i];
  return r;
}

// digest of an NK tensor: grid (cols, ceil(rows/1024))
__global__ __launch_bounds__(256) void k_hash_nk(const int8_t *q, int rows, int cols, int kpad, uint64_t salt,
                                                 unsigned long long *out) {
  __shared__ unsigned long long red[4];
  const int j = blockIdx.x;
  const int i0 = blockIdx.y * kRowsPerBlock + threadIdx.x * 4;
  unsigned long long h = 0;
  for (int r = 0; r < 4; r++) {
    const int i = i0 + r;
    if (i < rows) {
      const uint64_t idx = (uint64_t)i * cols + j;
      h += qd::mix64((idx << 8) ^ (uint64_t)(uint8_t)q[(size_t)j * kpad + i] ^ salt);
    }
  }
  h = block_sum_u64(h, red);
  if (threadIdx.x == 0) atomicAdd(out, h);
}

__global__ __launch_bounds__(256) void k_hash_kn(const int8_t *q, size_t n, uint64_t salt, unsigned long long *out) {
  __shared__ unsigned long long red[4];
  unsigned long long h = 0;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    h += qd::mix64(((uint64_t)i << 8) ^ (uint64_t)(uint8_t)q[i] ^ salt);
  h = block_sum_u64(h, red);
  if (threadIdx.x == 0) atomicAdd(out, h);
}

__global__ __launch_bounds__(256) void k_hash_f32(const float *x, size_t n, uint64_t salt, unsigned long long *out) {
  __shared__ unsigned long long red[4];
  unsigned long long h = 0;
  for (size_t i = blockIdx.x * (size_t)blockDim.x + threadIdx.x; i < n; i += (size_t)gridDim.x * blockDim.x)
    h += qd::mix64(((uint64_t)i << 32) ^ (uint64_t)__float_as_uint(x[i]) ^ salt);
  h = block_sum_u64(h, red);
  if (threadIdx.x == 0) atomicAdd(out, h);
}

unsigned grid_for(size_t n, unsigned cap = 65536) {
  size_t g = (n + 255) / 256;
  if (g < 1) g = 1;
  return (unsigned)(g > cap ? cap : g);
}

}  // namespace

extern "C" {

int qhip_fill_zero(void *p, size_t n) {
  if (!n) return 0;
  if (((uintptr_t)p & 15) == 0 && (n & 15) == 0) {
    QH_LAUNCH(QK_OTHER, k_fill_zero_u128, dim3(grid_for(n / 16)), dim3(256), 0, (uint4 *)p, n / 16);
  } else {
    QH_LAUNCH(QK_OTHER, k_fill_zero_u8, dim3(grid_for(n)), dim3(256), 0, (uint8_t *)p, n);
  }
  return 0;
}

int qhip_fill_f32(float *p, size_t n, float v) {
  if (!n) return 0;
  QH_LAUNCH(QK_OTHER, k_fill_f32, dim3(grid_for(n)), dim3(256), 0, p, n, v);
  return 0;
}

int qhip_synth_f32(uint64_t seed, uint64_t tid, size_t n, double sigma, float *out) {
  if (!n) return 0;
  QH_LAUNCH(QK_OTHER, k_synth_f32, dim3(grid_for(n)), dim3(256), 0, qd::gen_key(seed, tid), n, sigma, out);
  return 0;
}

int qhip_synth_quant_nk(uint64_t seed, uint64_t tid, int rows, int cols, int kpad, int transpose_src,
                        double sigma, int8_t *q, float *scale) {
  if (kpad % 16 || kpad < rows || rows <= 0 || cols <= 0 || kpad > 65535 * kRowsPerBlock)
    return qh::fail_msg("synth_quant_nk: bad shape");
  unsigned *colmax = (unsigned *)qhip_malloc((size_t)cols * 4);
  if (!colmax) return 1;
  const uint64_t key = qd::gen_key(seed, tid);
  int rc = qhip_fill_zero(colmax, (size_t)cols * 4);
  if (!rc)
    QH_LAUNCH(QK_OTHER, k_synth_colmax_nk, dim3(cols, (rows + kRowsPerBlock - 1) / kRowsPerBlock), dim3(256), 0,
              key, rows, cols, transpose_src, sigma, colmax);
  if (!rc)
    QH_LAUNCH(QK_OTHER, k_synth_quant_nk, dim3(cols, (kpad + kRowsPerBlock - 1) / kRowsPerBlock), dim3(256), 0,
              key, rows, cols, kpad, transpose_src, sigma, colmax, q, scale);
  if (!rc) rc = qhip_sync();
  qhip_free(colmax);
  return rc;
}

int qhip_synth_quant_kn(uint64_t seed, uint64_t tid, int rows, int cols, double sigma, int8_t *q, float *scale) {
  unsigned *colmax = (unsigned *)qhip_malloc((size_t)cols * 4);
  if (!colmax) return 1;
  const uint64_t key = qd::gen_key(seed, tid);
  int rc = qhip_fill_zero(colmax, (size_t)cols * 4);
  const dim3 grid((cols + 255) / 256, (rows + 255) / 256);
  if (!rc) QH_LAUNCH(QK_OTHER, k_synth_colmax_kn, grid, dim3(256), 0, key, rows, cols, sigma, colmax);
  if (!rc) QH_LAUNCH(QK_OTHER, k_synth_quant_kn, grid, dim3(256), 0, key, rows, cols, sigma, colmax, q, scale);
  if (!rc) rc = qhip_sync();
  qhip_free(colmax);
  return rc;
}

int qhip_quantize_percol(const float *w, int rows, int cols, int layout_nk, int kpad, int8_t *q, float *scale) {
  unsigned *colmax = (unsigned *)qhip_malloc((size_t)cols * 4);
  int8_t *tmp = layout_nk ? (int8_t *)qhip_malloc((size_t)rows * cols) : q;
  if (!colmax || !tmp) { qhip_free(colmax); if (layout_nk) qhip_free(tmp); return 1; }
  int rc = qhip_fill_zero(colmax, (size_t)cols * 4);
  const dim3 grid((cols + 255) / 256, (rows + 255) / 256);
  if (!rc) QH_LAUNCH(QK_OTHER, k_colmax_f32, grid, dim3(256), 0, w, rows, cols, colmax);
  if (!rc) QH_LAUNCH(QK_OTHER, k_quant_f32_kn, grid, dim3(256), 0, w, rows, cols, colmax, tmp, scale);
  if (!rc && layout_nk) rc = qhip_transpose_kn_to_nk(tmp, rows, cols, kpad, q);
  if (!rc) rc = qhip_sync();
  qhip_free(colmax);
  if (layout_nk) qhip_free(tmp);
  return rc;
}

int qhip_dequantize_kn(const int8_t *q, const float *scale, int rows, int cols, float *w) {
  const size_t n = (size_t)rows * cols;
  QH_LAUNCH(QK_OTHER, k_dequant_kn, dim3(grid_for(n)), dim3(256), 0, q, scale, rows, cols, w);
  return 0;
}

int qhip_transpose_kn_to_nk(const int8_t *src, int rows, int cols, int kpad, int8_t *dst) {
  if (kpad < rows || (cols + 63) / 64 > 65535) return qh::fail_msg("transpose: bad shape");
  QH_LAUNCH(QK_OTHER, k_transpose_kn_nk, dim3((kpad + 63) / 64, (cols + 63) / 64), dim3(256), 0,
            src, rows, cols, kpad, dst);
  return 0;
}

int qhip_nk_to_kn(const int8_t *src, int rows, int cols, int kpad, int8_t *dst) {
  QH_LAUNCH(QK_OTHER, k_nk_to_kn, dim3(cols, (rows + 255) / 256), dim3(256), 0, src, rows, cols, kpad, dst);
  return 0;
}

int qhip_hash_i8(const int8_t *q, int rows, int cols, int layout_nk, int kpad, uint64_t salt, uint64_t *out) {
  unsigned long long *d = (unsigned long long *)qhip_malloc(8);
  if (!d) return 1;
  int rc = qhip_fill_zero(d, 8);
  if (!rc) {
    if (layout_nk) {
      QH_LAUNCH(QK_OTHER, k_hash_nk, dim3(cols, (rows + kRowsPerBlock - 1) / kRowsPerBlock), dim3(256), 0,
                q, rows, cols, kpad, salt, d);
    } else {
      const size_t n = (size_t)rows * cols;
      QH_LAUNCH(QK_OTHER, k_hash_kn, dim3(grid_for(n, 8192)), dim3(256), 0, q, n, salt, d);
    }
  }
  if (!rc) rc = qhip_d2h(out, d, 8);
  qhip_free(d);
  return rc;
}

int qhip_hash_f32(const float *x, size_t n, uint64_t salt, uint64_t *out) {
  unsigned long long *d = (unsigned long long *)qhip_malloc(8);
  if (!d) return 1;
  int rc = qhip_fill_zero(d, 8);
  if (!rc) QH_LAUNCH(QK_OTHER, k_hash_f32, dim3(grid_for(n, 8192)), dim3(256), 0, x, n, salt, d);
  if (!rc) rc = qhip_d2h(out, d, 8);
  qhip_free(d);
  return rc;
}

}  // extern "C"
