// qhip_internal.h - shared by the HIP translation units of the library.
#ifndef QHIP_INTERNAL_H
#define QHIP_INTERNAL_H

#include <hip/hip_runtime.h>
#include <hip/hip_ext.h>

// Kernel classes for event timing (names in qhip_runtime.hip).
enum {
  QK_EMBED = 0, QK_RMSNORM, QK_GEMV_QKV, QK_ROPE, QK_ATTN, QK_QUANT, QK_GEMV_O, QK_GEMV_GU,
  QK_SWIGLU, QK_GEMV_DOWN, QK_GEMV_HEAD, QK_ARGMAX, QK_OTHER, QK_ATTN_PV, QK_PF_GEMM, QK_PF_ATTN, QK_PF_OTHER,
  QK_ATTN_FAST, QK_ATTN_LAYER, QK_FLUSH, QK_NUM_CLASSES
};

namespace qh {
hipStream_t stream();
int num_cus();            // compute units of the device (set by qhip_init)
int fail(const char *what, hipError_t e);
int fail_msg(const char *msg);
int check_launch(const char *what);
// When profiling is on: a (start, stop) event pair for one launch of class cls.
bool prof_events(int cls, hipEvent_t *start, hipEvent_t *stop);
// While suspended, launches take no timing events (an event is created on first
// use): the allocation-free entry point suspends it around its launches.
void prof_suspend(int on);
}  // namespace qh

// Launch on the library stream and turn a launch error into the function's
// nonzero return.  When profiling, the events are bound to the kernel's own
// dispatch (hipExtLaunchKernelGGL), so their interval is the kernel's
// execution alone, without the queue gaps around it.
#define QH_LAUNCH(cls, kernel, grid, block, shmem, ...)                                             \
  do {                                                                                             \
    hipEvent_t qh_a_ = nullptr, qh_b_ = nullptr;                                                   \
    if (qh::prof_events(cls, &qh_a_, &qh_b_))                                                      \
      hipExtLaunchKernelGGL(kernel, grid, block, shmem, qh::stream(), qh_a_, qh_b_, 0, __VA_ARGS__); \
    else                                                                                           \
      hipLaunchKernelGGL(kernel, grid, block, shmem, qh::stream(), __VA_ARGS__);                   \
    if (qh::check_launch(#kernel)) return 1;                                                       \
  } while (0)

#endif
