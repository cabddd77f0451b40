// qdev_tl.h - optional per-block timeline of the decode kernels (measurement
// only).  Built with -DQLLAMA_TIMELINE=1 (`make timeline` writes
// libqllama_tl.so); in the library's normal build every QTL_* macro expands to
// nothing and no code or storage is added.
//
// Each translation unit that records holds one array of
// kTlKernels x kTlBlocks x kTlEvents 64-bit stamps of the device's constant-rate
// clock (wall_clock64, 100 MHz on gfx950, one counter for the whole chip, so
// stamps of different kernels and blocks line up).  A kernel records under its
// own kernel id; a later launch of the same kernel overwrites the stamps, so
// after a decode step the arrays hold the last layer's launches.  Event 7 of a
// block holds (XCC id << 16) | HW_ID.  llm-project_amd/timeline.py reads the
// arrays through qllama_tl_read_<unit>.
#ifndef QDEV_TL_H
#define QDEV_TL_H

#include <hip/hip_runtime.h>

#ifndef QLLAMA_TIMELINE
#define QLLAMA_TIMELINE 0
#endif

#if QLLAMA_TIMELINE
namespace qtl {
constexpr int kTlKernels = 8, kTlBlocks = 1024, kTlEvents = 8;
constexpr int kTlWords = kTlKernels * kTlBlocks * kTlEvents;
__device__ __forceinline__ unsigned long long now() { return (unsigned long long)wall_clock64(); }
__device__ __forceinline__ unsigned hwid() {
  unsigned x, h;
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_XCC_ID)" : "=s"(x));
  asm volatile("s_getreg_b32 %0, hwreg(HW_REG_HW_ID)" : "=s"(h));
  return ((x & 0xfu) << 16) | (h & 0xffffu);
}
__device__ __forceinline__ int slot(int kid, int ev) {
  const int b = blockIdx.x + gridDim.x * blockIdx.y;
  return b < kTlBlocks ? (kid * kTlBlocks + b) * kTlEvents + ev : -1;
}
}  // namespace qtl

// The unit's array and its reader: copies the whole array to `host`
// (kTlWords words) and, when clear is nonzero, zeroes it.
#define QTL_DEFINE(unit)                                                                                 \
  static __device__ unsigned long long qtl_buf[qtl::kTlWords];                                           \
  extern "C" int qllama_tl_read_##unit(unsigned long long *host, int clear) {                             \
    if (hipDeviceSynchronize() != hipSuccess) return 1;                                                  \
    if (host && hipMemcpyFromSymbol(host, HIP_SYMBOL(qtl_buf), sizeof(qtl_buf)) != hipSuccess) return 1; \
    if (clear) {                                                                                         \
      static unsigned long long zero[qtl::kTlWords];                                                     \
      if (hipMemcpyToSymbol(HIP_SYMBOL(qtl_buf), zero, sizeof(zero)) != hipSuccess) return 1;            \
    }                                                                                                    \
    return 0;                                                                                            \
  }
// Lane 0 of the executing wave stamps event ev of this block.
#define QTL_MARK(kid, ev)                                                  \
  do {                                                                     \
    if ((threadIdx.x & 63) == 0) {                                         \
      const int s_ = qtl::slot((kid), (ev));                               \
      if (s_ >= 0) qtl_buf[s_] = qtl::now();                               \
    }                                                                      \
  } while (0)
// The latest stamp over the waves that reach it (an end event).
#define QTL_MAX(kid, ev)                                                   \
  do {                                                                     \
    if ((threadIdx.x & 63) == 0) {                                         \
      const int s_ = qtl::slot((kid), (ev));                               \
      if (s_ >= 0) atomicMax(&qtl_buf[s_], qtl::now());                    \
    }                                                                      \
  } while (0)
#define QTL_ID(kid)                                                        \
  do {                                                                     \
    if (threadIdx.x == 0) {                                                \
      const int s_ = qtl::slot((kid), 7);                                  \
      if (s_ >= 0) qtl_buf[s_] = qtl::hwid();                              \
    }                                                                      \
  } while (0)
// The shader clock (s_memtime, cycles) instead of the constant-rate clock.
#define QTL_CYC(kid, ev)                                                   \
  do {                                                                     \
    if ((threadIdx.x & 63) == 0) {                                         \
      const int s_ = qtl::slot((kid), (ev));                               \
      if (s_ >= 0) qtl_buf[s_] = (unsigned long long)clock64();           \
    }                                                                      \
  } while (0)
#else
#define QTL_DEFINE(unit)
#define QTL_MARK(kid, ev) \
  do {                    \
  } while (0)
#define QTL_MAX(kid, ev) \
  do {                   \
  } while (0)
#define QTL_ID(kid) \
  do {              \
  } while (0)
#define QTL_CYC(kid, ev) \
  do {                   \
  } while (0)
#endif

#endif
