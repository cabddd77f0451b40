// k_pfa.hip - causal prompt attention of the fast mode on fp32 MFMA
// (llama.c:554-576 for every prompt row; the order of the floating-point sums
// differs from the reference, so this is a tolerance path like the fast
// decode attention, not a bit-exact one).
//
// A block serves one KV head and 32 consecutive query rows; wave g is query
// head kvh*G + g.  Keys stream through LDS in tiles of 32 (K as [key][dim], V
// transposed to [dim][key]), shared by the G waves.  Per tile and wave:
//   S^T = K . q^T  (32 keys x 32 rows, v_mfma_f32_32x32x2_f32 over hd/2 steps);
//   lane l then holds row l % 32 for 16 of the tile's keys and lane l ^ 32 the
//   other 16, so the online softmax (running max m, running sum l, rescale of
//   the output by exp(m_old - m_new)) needs one cross-lane exchange per tile;
//   O^T += V^T . P^T  (hd x 32 rows), whose B operand is each lane's own
//   probabilities: the MFMA's K slots are matched to the keys a lane holds.
// q is pre-scaled by scale * log2(e), so p = exp2(s - m) (v_exp_f32).  At the
// end o = O / l.
//
// Later rows see more keys.  With pairing (G <= 4), block i serves row blocks i
// and nrb-1-i with 2G waves (the second set on the SIMDs of the first), so
// every block and every SIMD does nrb+1 tiles of MFMA work; the staged tiles
// serve both sets, the first set idling at the barriers once its rows have
// seen all their keys.  Without pairing (G > 4: 2G waves would not hold their
// registers) blocks of later rows are dispatched first.
#include <hip/hip_runtime.h>

#include "qhip.h"
#include "qhip_internal.h"

namespace {

typedef float v16f __attribute__((ext_vector_type(16)));

constexpr int kRows = 32;    // query rows per block (the MFMA's columns)
constexpr int kKeys = 32;    // keys per tile (the MFMA's rows of S^T)

template <int HD>
__global__ __launch_bounds__(512) void k_pf_fa(const float *q, const float *kc, const float *vc, int R, int p0, int H,
                                               int KVH, int max_seq, float qscale, float *o, int pair) {
  constexpr int QK = HD / 8;       // groups of 8 dims: lane half hf holds dims 8m + 4hf .. +3 of its row
  constexpr int NB = HD / 32;      // 32-dim blocks of the output
  constexpr int KS = HD + 4;       // LDS row stride of the K tile (conflict-free 16-byte reads)
  constexpr int VS = kKeys + 4;    // LDS row stride of the transposed V tile
  __shared__ __attribute__((aligned(16))) float Ks[kKeys * KS];
  __shared__ __attribute__((aligned(16))) float Vt[HD * VS];
  const int G = H / KVH, nrb = (R + kRows - 1) / kRows;
  const int tid = threadIdx.x, wave = tid >> 6, lane = tid & 63, hf = lane >> 5, lr = lane & 31;
  const int kvh = blockIdx.x;
  int rb, rb_last;                                 // this wave's row block, the block's longest
  bool active = true;
  if (pair) {
    const int i = blockIdx.y, j = nrb - 1 - i, second = wave >= G;
    rb = second ? j : i;
    rb_last = j;
    active = !second || j != i;                    // an odd middle block has one set
  } else {
    rb = rb_last = gridDim.y - 1 - blockIdx.y;
  }
  const int r0 = rb * kRows;
  const int h = kvh * G + wave % G;
  const int rl = min(r0 + lr, R - 1);              // this lane's query row (rows past R are not stored)
  const int pos = p0 + rl;
  const int kmine = p0 + min(r0 + kRows, R);       // keys 0 .. kmine-1 are seen by some row of the set
  const int kend = p0 + min(rb_last * kRows + kRows, R);   // ... and kend-1 by some row of the block
  const int nmine = (kmine + kKeys - 1) / kKeys;

  float qf[QK][4];
  {
    const float *qr = q + (size_t)rl * H * HD + (size_t)h * HD + 4 * hf;
#pragma unroll
    for (int m = 0; m < QK; m++) {
      const float4 v = *reinterpret_cast<const float4 *>(qr + 8 * m);
      qf[m][0] = v.x * qscale; qf[m][1] = v.y * qscale; qf[m][2] = v.z * qscale; qf[m][3] = v.w * qscale;
    }
  }
  v16f acc[NB];
#pragma unroll
  for (int b = 0; b < NB; b++) acc[b] = (v16f){};
  float mrun = -INFINITY, lrun = 0.0f;

  const float *Kh = kc + (size_t)kvh * max_seq * HD, *Vh = vc + (size_t)kvh * max_seq * HD;
  const int ntile = (kend + kKeys - 1) / kKeys, nthr = blockDim.x;
  for (int t = 0; t < ntile; t++) {
    const int k0 = t * kKeys;
    // stage the tile; keys past kend-1 repeat key kend-1 (masked below, finite)
    for (int i = tid; i < kKeys * HD / 4; i += nthr) {
      const int key = i / (HD / 4), d4 = (i % (HD / 4)) * 4;
      const size_t src = (size_t)min(k0 + key, kend - 1) * HD + d4;
      const float4 kv = *reinterpret_cast<const float4 *>(Kh + src);
      const float4 vv = *reinterpret_cast<const float4 *>(Vh + src);
      *reinterpret_cast<float4 *>(Ks + key * KS + d4) = kv;
      Vt[(d4 + 0) * VS + key] = vv.x;
      Vt[(d4 + 1) * VS + key] = vv.y;
      Vt[(d4 + 2) * VS + key] = vv.z;
      Vt[(d4 + 3) * VS + key] = vv.w;
    }
    __syncthreads();
    if (!active || t >= nmine) {                   // this set's rows have seen all their keys
      __syncthreads();
      continue;
    }

    // S^T[key][row]: A = K (lane: key lr, K slot hf), B = q (lane: row lr, K slot hf);
    // instruction (m, c) takes dim 8m + 4hf + c in both operands
    v16f s = (v16f){};
#pragma unroll
    for (int m = 0; m < QK; m++) {
      const float4 kf = *reinterpret_cast<const float4 *>(Ks + lr * KS + 8 * m + 4 * hf);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.x, qf[m][0], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.y, qf[m][1], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.z, qf[m][2], s, 0, 0, 0);
      s = __builtin_amdgcn_mfma_f32_32x32x2f32(kf.w, qf[m][3], s, 0, 0, 0);
    }
    // element e of the result is key k0 + 8(e/4) + 4hf + e%4 for this lane's row
    float mt = -INFINITY;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      const int key = k0 + 8 * (e >> 2) + 4 * hf + (e & 3);
      if (key > pos) s[e] = -INFINITY;
      mt = fmaxf(mt, s[e]);
    }
    mt = fmaxf(mt, __shfl_xor(mt, 32));
    const float mnew = fmaxf(mrun, mt);                  // finite: key 0 is seen by every row
    const float alpha = __builtin_amdgcn_exp2f(mrun - mnew);
    float p[16], ps = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; e++) {
      p[e] = __builtin_amdgcn_exp2f(s[e] - mnew);
      ps += p[e];
    }
    lrun = lrun * alpha + ps;
    mrun = mnew;
#pragma unroll
    for (int b = 0; b < NB; b++) acc[b] *= alpha;

    // O^T[dim][row] += V^T . P^T: instruction (j, c) takes key 8j + 4hf + c, i.e.
    // the lane's own p[4j + c]; A = V^T (lane: dim 32b + lr)
#pragma unroll
    for (int b = 0; b < NB; b++) {
#pragma unroll
      for (int j = 0; j < 4; j++) {
        const float4 vf = *reinterpret_cast<const float4 *>(Vt + (32 * b + lr) * VS + 8 * j + 4 * hf);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.x, p[4 * j + 0], acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.y, p[4 * j + 1], acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.z, p[4 * j + 2], acc[b], 0, 0, 0);
        acc[b] = __builtin_amdgcn_mfma_f32_32x32x2f32(vf.w, p[4 * j + 3], acc[b], 0, 0, 0);
      }
    }
    __syncthreads();                                     // the tile is consumed
  }

  const float inv = 1.0f / (lrun + __shfl_xor(lrun, 32));
  if (active && r0 + lr < R) {
    // element e of block b is dim 32b + 8(e/4) + 4hf + e%4 of this lane's row
    float *orow = o + (size_t)(r0 + lr) * H * HD + (size_t)h * HD + 4 * hf;
#pragma unroll
    for (int b = 0; b < NB; b++)
#pragma unroll
      for (int g = 0; g < 4; g++)
        *reinterpret_cast<float4 *>(orow + 32 * b + 8 * g) =
            make_float4(acc[b][4 * g] * inv, acc[b][4 * g + 1] * inv, acc[b][4 * g + 2] * inv, acc[b][4 * g + 3] * inv);
  }
}

}  // namespace

// Shapes the fast prompt attention serves: head_dim 64 or 128, 1-8 query heads per KV head.
extern "C" int qhip_pf_attention_fast_ok(int n_heads, int n_kv, int hd) {
  if (n_kv <= 0 || n_heads % n_kv) return 0;
  const int G = n_heads / n_kv;
  return (hd == 128 || hd == 64) && G >= 1 && G <= 8;
}

extern "C" int qhip_pf_attention_fast(const float *q, const float *kc, const float *vc, int R, int p0, int n_heads,
                                      int n_kv, int hd, int max_seq, float scale, float *o) {
  if (!qhip_pf_attention_fast_ok(n_heads, n_kv, hd)) return qh::fail_msg("pf_attention_fast: unsupported shape");
  if (R <= 0 || p0 < 0 || p0 + R > max_seq) return qh::fail_msg("pf_attention_fast: positions out of range");
  const int G = n_heads / n_kv, nrb = (R + kRows - 1) / kRows, pair = G <= 4 && nrb > 1;
  const dim3 grid(n_kv, pair ? (nrb + 1) / 2 : nrb), block(64 * G * (pair ? 2 : 1));
  const float qscale = scale * 1.4426950408889634f;     // log2(e): p = exp2(s * log2(e) - m)
  if (hd == 128)
    QH_LAUNCH(QK_PF_ATTN, k_pf_fa<128>, grid, block, 0, q, kc, vc, R, p0, n_heads, n_kv, max_seq, qscale, o, pair);
  else
    QH_LAUNCH(QK_PF_ATTN, k_pf_fa<64>, grid, block, 0, q, kc, vc, R, p0, n_heads, n_kv, max_seq, qscale, o, pair);
  return 0;
}
