// The allocation-free form of ifd_gemm_t64, for callers that cannot allocate device memory: code under HIP graph
// capture, tight serving loops, harnesses that forbid hipMalloc.
//
// Its workspace is a file-scope device array of kNoAllocScratch bytes (a copy per GPU, held until the process ends)
// instead of a caller's buffer. Host code never passes the array's name to a kernel: in host code that name is a
// stand-in, not a device address. The first call on each device looks up that device's address of the array with
// hipGetSymbolAddress and keeps it; every later use goes through that address. Each call first clears the counter
// header (its first 4096 bytes) with a fill kernel, since the previous call's contents remain, and then runs the same
// kernels as ifd_gemm_t64 with the array as the workspace. Calls that overlap on one GPU share the array and race.
#include <mutex>

#include "host.h"
#include "kernels.h"

// The largest workspace ifd_gemm_t64 asks for at decode sizes (stream-K partial slots at 65..128 rows: 64 MiB plus
// the 4 KiB header) and at BASELINE's prefill shape; larger requests are rejected.
constexpr size_t kNoAllocScratch = IFD_NOALLOC_SCRATCH_BYTES;

static __device__ __align__(256) unsigned char scratch[kNoAllocScratch];

namespace {

constexpr int kMaxDevices = 64;
std::mutex g_mu;
void* g_scratch[kMaxDevices];

// This device's address of `scratch`, looked up once per device with that device current.
int scratch_ptr(void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
    return ifd::fail(IFD_ERR_LAUNCH, "gemm_t64_noalloc: no current device (or device %d past %d)", dev, kMaxDevices);
  std::lock_guard<std::mutex> lock(g_mu);
  if (!g_scratch[dev]) {
    void* p = nullptr;
    const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
    if (e != hipSuccess || !p)
      return ifd::fail(IFD_ERR_LAUNCH, "gemm_t64_noalloc: hipGetSymbolAddress of the scratch array failed: %s",
                       hipGetErrorString(e));
    g_scratch[dev] = p;
  }
  *out = g_scratch[dev];
  return IFD_OK;
}

}  // namespace

extern "C" {

int ifd_gemm_t64_noalloc(const void* A, int lda, const void* wt, int N, int K, void* C, int ldc, int M, int mode,
                         void* stream) {
  const size_t need = ifd_gemm_t64_workspace(M, N, K);
  if (need > kNoAllocScratch)
    return ifd::fail(IFD_ERR_WORKSPACE,
                     "gemm_t64_noalloc: M=%d N=%d K=%d needs %zu bytes of workspace; the static scratch holds %zu", M,
                     N, K, need, kNoAllocScratch);
  if (need == 0) return ifd_gemm_t64(A, lda, wt, N, K, C, ldc, M, mode, nullptr, 0, stream);
  void* p = nullptr;
  IFD_TRY(scratch_ptr(&p));
  IFD_TRY(ifd::launch_zero_header(p, (hipStream_t)stream));
  return ifd_gemm_t64(A, lda, wt, N, K, C, ldc, M, mode, p, kNoAllocScratch, stream);
}

}  // extern "C"
