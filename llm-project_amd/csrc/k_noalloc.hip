// k_noalloc.hip - qmatmul (quant.c:60-85) on device buffers without any
// allocation, for callers that cannot allocate: code under HIP graph capture,
// tight serving loops, harnesses that forbid hipMalloc.  It has no counterpart
// in the reference.
//
// The only memory beyond the caller's inputs and outputs -- the quantized
// activation rows and their scales -- lives in the file-scope device array
// `scratch` below (QLLAMA_NOALLOC_SCRATCH_BYTES per GPU, held until the process
// ends).  Host code never hands the array's name to a kernel: the name is a
// host-side stand-in, not a device address.  The device address is taken once
// per device with hipGetSymbolAddress on the first call made on that device
// (the set-up), kept per device, and only that address is passed on.
//
// Every call shares its GPU's array and leaves the last call's contents there;
// each call overwrites every scratch byte it reads (the quantizer writes whole
// padded rows and the scales), so nothing needs clearing.  Calls are enqueued
// on the library stream in order, so consecutive calls do not overlap; calls
// that do overlap on one GPU (graphs replayed concurrently, other streams)
// race on the array.
#include <hip/hip_runtime.h>

#include <cstdio>

#include "qhip.h"
#include "qhip_internal.h"
#include "qllama.h"

namespace {

constexpr size_t kScratchBytes = QLLAMA_NOALLOC_SCRATCH_BYTES;
__device__ __align__(256) uint8_t scratch[kScratchBytes];

constexpr int kMaxDevices = 64;
void *g_scratch_ptr[kMaxDevices];            // per device: the address of `scratch`

size_t al256(size_t n) { return (n + 255) & ~(size_t)255; }

// Set-up: the device address of this device's copy of the array.
void *device_scratch() {
  int dev = 0;
  hipError_t e = hipGetDevice(&dev);
  if (e != hipSuccess) { qh::fail("hipGetDevice", e); return nullptr; }
  if (dev < 0 || dev >= kMaxDevices) { qh::fail_msg("qmatmul_device_noalloc: device index out of range"); return nullptr; }
  if (!g_scratch_ptr[dev]) {
    void *p = nullptr;
    e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p) { qh::fail("hipGetSymbolAddress(scratch)", e); return nullptr; }
    g_scratch_ptr[dev] = p;
  }
  return g_scratch_ptr[dev];
}

int refuse(const char *why) {
  fprintf(stderr, "Error: qmatmul_device_noalloc: %s\n", why);
  return 1;
}

}  // namespace

extern "C" int qmatmul_device_noalloc(const float *A, int M, const QTensor *W, float *C) {
  if (qhip_init()) return refuse(qhip_last_error());
  if (!A || !W || !C || !W->q || !W->scale || M < 1) return refuse("null argument or M < 1");
  if (W->layout != QT_LAYOUT_NK) return refuse("W must be an output-channel-major (QT_LAYOUT_NK) QTensor");
  const int K = W->rows, N = W->cols, kpad = W->kpad;
  if (K < 1 || N < 1 || kpad < K || kpad % 16) return refuse("bad QTensor shape");
  if (K > 16384) return refuse("K above 16384 (one row of activations is quantized in one block)");
  const size_t need = al256((size_t)M * kpad) + (size_t)M * sizeof(float);
  if (need > kScratchBytes) {
    fprintf(stderr, "Error: qmatmul_device_noalloc: M * kpad = %zu bytes of quantized rows exceed the %zu-byte "
            "scratch (at most %zu rows of K = %d)\n", (size_t)M * kpad, kScratchBytes,
            (kScratchBytes - 4096) / ((size_t)kpad + 4), K);
    return 1;
  }
  uint8_t *base = static_cast<uint8_t *>(device_scratch());
  if (!base) return refuse(qhip_last_error());
  int8_t *qa = reinterpret_cast<int8_t *>(base);
  float *as = reinterpret_cast<float *>(base + al256((size_t)M * kpad));
  qh::prof_suspend(1);                        // no timing events: they are created on first use
  const int rc = qhip_quant_rows(A, M, K, qa, kpad, as) ||
                 qhip_qmm_product(qa, as, M, reinterpret_cast<const int8_t *>(W->q), W->scale, N, kpad, C);
  qh::prof_suspend(0);
  return rc ? refuse(qhip_last_error()) : 0;
}
