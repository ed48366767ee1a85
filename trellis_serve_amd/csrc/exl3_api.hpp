// Host-side helpers shared by the C-ABI translation units: status codes, the thread-local last-error string,
// HIP error checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdint.h>
#include <stdio.h>

#include "../../include/exl3_mi355x.h"

namespace exl3 {

int set_error(int code, const char* fmt, ...) __attribute__((format(printf, 2, 3)));

inline hipStream_t as_stream(void* s) { return reinterpret_cast<hipStream_t>(s); }

#define EXL3_CHECK_ARG(cond, ...)                                \
  do {                                                           \
    if (!(cond)) return ::exl3::set_error(EXL3_ERR_INVALID, __VA_ARGS__); \
  } while (0)

#define EXL3_CHECK_HIP(expr)                                                                      \
  do {                                                                                            \
    hipError_t e_ = (expr);                                                                       \
    if (e_ != hipSuccess)                                                                         \
      return ::exl3::set_error(EXL3_ERR_HIP, "%s: %s (%s:%d)", #expr, hipGetErrorString(e_), __FILE__, __LINE__); \
  } while (0)

#define EXL3_CHECK_LAUNCH() EXL3_CHECK_HIP(hipGetLastError())

// split counters at the start of a linear / MoE workspace (fixed place and size, zero between calls)
constexpr size_t kCounterBytes = EXL3_WORKSPACE_COUNTER_BYTES;
constexpr int kMaxCounters = (int)(kCounterBytes / sizeof(int));

// Rows from which a linear's rows go to the prefill decode-GEMM instead of the decode-GEMV (the dispatch of the
// torch-facing op, measured crossover on the 27B shapes); exl3_gemm_rotated switches at the same count.
constexpr int kPrefillRows = 65;

// The rotation-free prefill decode-GEMM of exl3_gemm_rotated (out = xh @ W_inner, fp16 xh), defined with the prefill
// kernels: its workspace bytes, and the call.
size_t prefill_plain_workspace_bytes(int rows, int k, int n);
int prefill_plain_gemm(const void* xh, int rows, int k, const void* trellis, int n, int K, int codebook, void* out,
                       void* workspace, size_t workspace_bytes, hipStream_t st);

// exl3_init_device's probe of the workgroup -> XCD assignment (exl3_linear.hip): enables split-K chains that stay
// in one XCD's L2
int xcd_probe(int device);
// whether a probe has passed (and EXL3_GEMV_XCD_LOCAL is not 0): workgroups whose ids agree mod 8 share an XCD
bool xcd_groups_ok();

inline bool valid_bits(int K) { return K == 2 || K == 3 || K == 4 || K == 5 || K == 6 || K == 8; }
inline bool valid_cb(int cb) { return cb >= 0 && cb <= 2; }

}  // namespace exl3
