// Host-side helpers shared by the launchers: status codes, the per-thread error message, argument checks.
#pragma once
#include <hip/hip_runtime.h>
#include <stdarg.h>
#include <stdio.h>

#include "../../include/inferd_qmm.h"

namespace ifd {

// Message of the last failure on this thread (returned by ifd_last_error()).
inline char* last_error_buf() {
  static thread_local char buf[512] = "";
  return buf;
}
inline int fail(int code, const char* fmt, ...) {
  va_list ap;
  va_start(ap, fmt);
  vsnprintf(last_error_buf(), 512, fmt, ap);
  va_end(ap);
  return code;
}
// After a kernel launch: turn a HIP launch error into IFD_ERR_LAUNCH.
inline int check_launch(const char* what) {
  hipError_t e = hipGetLastError();
  if (e != hipSuccess) return fail(IFD_ERR_LAUNCH, "%s: %s", what, hipGetErrorString(e));
  return IFD_OK;
}
inline bool aligned(const void* p, size_t a) { return ((uintptr_t)p % a) == 0; }
inline size_t align_up(size_t v, size_t a) { return (v + a - 1) / a * a; }
// compute units of the current device (256 on MI355X), read once
inline int cu_count() {
  static int n = 0;
  if (!n) {
    int dev = 0;
    (void)hipGetDevice(&dev);
    if (hipDeviceGetAttribute(&n, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || n <= 0) n = 256;
  }
  return n;
}

#define IFD_CHECK(cond, ...)                      \
  do {                                            \
    if (!(cond)) return ::ifd::fail(IFD_ERR_ARG, __VA_ARGS__); \
  } while (0)
#define IFD_TRY(expr)                \
  do {                               \
    int _rc = (expr);                \
    if (_rc != IFD_OK) return _rc;   \
  } while (0)

// Validates the common arguments of a dense 4- or 8-bit GEMM (the flip mask xr: 0x88888888 or 0x80808080).
inline int check_w4_args(const void* A, int lda, const void* wq, const void* s, const void* b, int N, int K, int ldk,
                         uint32_t xr, const void* C, int ldc, int M, int mode, int a_elem_bytes, int bits = 4) {
  IFD_CHECK(M >= 0 && N > 0 && K > 0, "bad shape M=%d N=%d K=%d", M, N, K);
  IFD_CHECK(K % 64 == 0, "K=%d is not a multiple of the group size 64", K);
  IFD_CHECK(ldk == 0 || (ldk >= K && ldk % 64 == 0), "ldk=%d must be 0 or a multiple of 64 >= K", ldk);
  const uint32_t flip = bits == 8 ? 0x80808080u : 0x88888888u;
  IFD_CHECK(xr == 0u || xr == flip, "xr=0x%x must be 0 or 0x%x", xr, flip);
  IFD_CHECK(mode >= 0 && mode <= 2, "mode=%d must be 0, 1 or 2", mode);
  IFD_CHECK(lda >= K && lda % 8 == 0, "lda=%d must be >= K and a multiple of 8", lda);
  IFD_CHECK(ldc >= N, "ldc=%d must be >= N=%d", ldc, N);
  if (M == 0) return IFD_OK;
  IFD_CHECK(A && wq && s && b && C, "null pointer");
  IFD_CHECK(aligned(A, 16) && aligned(wq, 16) && aligned(s, 4) && aligned(b, 4),
            "A and wq must be 16-byte aligned, s and b 4-byte aligned");
  (void)a_elem_bytes;
  return IFD_OK;
}

}  // namespace ifd
