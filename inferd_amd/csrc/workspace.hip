// Workspace counter header: a fill kernel that zeroes it, and the host-side check of it.
//
// Every public workspace starts with kWsHeader bytes of uint32 completion counters (the in-kernel split-K fixups of
// the decode GEMV and the decode MoE's combine count arriving blocks there). Each call leaves them at zero. A call
// that fails after a partial launch, or a kernel that does not finish, can leave a counter non-zero; a later call
// would then see the wrong block as the last one of a tile and store a sum before all of its partials were written.
// ifd_workspace_check finds that state, ifd_workspace_reset clears it. The reset is a kernel, not a memset node, so
// that a caller may put it into a captured HIP graph.
#include <vector>

#include "common.h"
#include "host.h"
#include "kernels.h"

namespace ifd {

__global__ __launch_bounds__(256) void k_zero_u32(uint32_t* __restrict__ p, int n) {
  const int i = blockIdx.x * 256 + threadIdx.x;
  if (i < n) p[i] = 0u;
}

int launch_zero_header(void* ws, hipStream_t st) {
  hipLaunchKernelGGL(k_zero_u32, dim3((kWsCounters + 255) / 256), dim3(256), 0, st, (uint32_t*)ws, kWsCounters);
  return check_launch("workspace reset");
}

}  // namespace ifd

using namespace ifd;

extern "C" {

int ifd_workspace_check(const void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(workspace && ws_bytes >= kWsHeader, "a workspace with a counter header holds at least %zu bytes", kWsHeader);
  hipStream_t st = (hipStream_t)stream;
  if (hipStreamSynchronize(st) != hipSuccess) return fail(IFD_ERR_LAUNCH, "workspace check: stream synchronise failed");
  std::vector<uint32_t> h(kWsCounters);
  if (hipMemcpy(h.data(), workspace, kWsHeader, hipMemcpyDeviceToHost) != hipSuccess)
    return fail(IFD_ERR_LAUNCH, "workspace check: copy of the counter header failed");
  for (int i = 0; i < kWsCounters; i++)
    if (h[i] != 0u)
      return fail(IFD_ERR_WORKSPACE, "workspace counter %d is %u, not 0: reset the header (ifd_workspace_reset)", i,
                  h[i]);
  return IFD_OK;
}

int ifd_workspace_reset(void* workspace, size_t ws_bytes, void* stream) {
  IFD_CHECK(workspace && ws_bytes >= kWsHeader && aligned(workspace, 4),
            "a workspace with a counter header holds at least %zu bytes, 4-byte aligned", kWsHeader);
  return launch_zero_header(workspace, (hipStream_t)stream);
}

}  // extern "C"
