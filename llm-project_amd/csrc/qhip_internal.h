// qhip_internal.h - shared by the HIP translation units of the library.
#ifndef QHIP_INTERNAL_H
#define QHIP_INTERNAL_H

#include <hip/hip_runtime.h>

// Kernel classes for event timing (names in qhip_runtime.hip).
enum {
  QK_EMBED = 0, QK_RMSNORM, QK_GEMV_QKV, QK_ROPE, QK_ATTN, QK_QUANT, QK_GEMV_O, QK_GEMV_GU,
  QK_SWIGLU, QK_GEMV_DOWN, QK_GEMV_HEAD, QK_ARGMAX, QK_OTHER, QK_NUM_CLASSES
};

namespace qh {
hipStream_t stream();
int fail(const char *what, hipError_t e);
int fail_msg(const char *msg);
int check_launch(const char *what);
void *prof_begin(int cls);
void prof_end(void *tok);
}  // namespace qh

// Launch on the library stream, time it when profiling, and turn a launch
// error into the function's nonzero return.
#define QH_LAUNCH(cls, kernel, grid, block, shmem, ...)                         \
  do {                                                                         \
    void *qh_tok_ = qh::prof_begin(cls);                                       \
    hipLaunchKernelGGL(kernel, grid, block, shmem, qh::stream(), __VA_ARGS__); \
    qh::prof_end(qh_tok_);                                                     \
    if (qh::check_launch(#kernel)) return 1;                                   \
  } while (0)

#endif
