"""The allocation-free GEMM entry point (ifd_gemm_t64_noalloc, static device scratch) against ifd_gemm_t64 with a
caller workspace, through the C ABI: the same bits on calls in a row whose sizes shrink, and a request past the
scratch rejected before anything runs."""
import numpy as np
import pytest

from tests import gen

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _noalloc(A, T, C, mode):
    from inferd_amd._lib import lib
    M, K = A.shape
    return lib().ifd_gemm_t64_noalloc(A.data_ptr(), K, T.wt.data_ptr(), T.N, T.K, C.data_ptr(), C.shape[1], M, mode,
                                      torch.cuda.current_stream().cuda_stream)


def test_noalloc_matches_workspace_entry_on_consecutive_calls():
    """Three calls in a row on the shared scratch, each smaller than the one before: a stream-K GEMM at M = 128 (64 MiB
    of partial slots), a decode GEMV at M = 8 with the residual add (its split-K fixup counts blocks in the scratch's
    counter header, which the previous call's contents must not disturb) and M = 1 with fp32 output. Each is
    bit-identical to ifd_gemm_t64 with a workspace on the same inputs."""
    from inferd_amd import ops
    from inferd_amd._lib import IFD_OK, lib
    from tests import gpu_util as g
    cases = [(128, 34816, 5120, 0), (8, 5120, 17408, 1), (1, 5120, 5120, 2)]
    for i, (M, N, K, mode) in enumerate(cases):
        print(f"noalloc case M={M} N={N} K={K} mode={mode}", flush=True)
        assert lib().ifd_gemm_t64_workspace(M, N, K) > 4096  # every case uses the scratch
        _, wq, s, b = gen.qlinear(N, K, seed=2000 + i)
        T = ops.pack_t64(g.qlinear(wq, s, b))
        A = g.dev(gen.activations(M, K, seed=2100 + i))
        C0 = gen.activations(M, N, seed=2200 + i)
        ref = ops.gemm_t64(A, T, g.dev(C0) if mode == 1 else None, mode=mode)
        out = g.dev(C0) if mode == 1 else torch.full((M, N), 7.0, device="cuda",
                                                      dtype=torch.float32 if mode == 2 else torch.bfloat16)
        assert _noalloc(A, T, out, mode) == IFD_OK, lib().ifd_last_error()
        torch.cuda.synchronize()
        assert np.array_equal(g.host(out), g.host(ref)), (M, N, K, mode)


def test_noalloc_rejects_requests_past_the_scratch():
    """M = 512, N = 20480, K = 5120 needs 80 MiB of workspace: IFD_ERR_WORKSPACE, the output untouched."""
    from inferd_amd import ops
    from inferd_amd._lib import IFD_ERR_WORKSPACE, lib
    M, N, K = 512, 20480, 5120
    assert lib().ifd_gemm_t64_workspace(M, N, K) > (68 << 20)
    T = ops.T64Linear(torch.zeros(lib().ifd_t64_bytes(N, K, 1), dtype=torch.uint8, device="cuda"), N, K)
    A = torch.zeros((M, K), dtype=torch.bfloat16, device="cuda")
    C = torch.full((M, N), 3.0, dtype=torch.bfloat16, device="cuda")
    assert _noalloc(A, T, C, 0) == IFD_ERR_WORKSPACE
    assert b"static scratch" in lib().ifd_last_error()
    torch.cuda.synchronize()
    assert bool((C == 3.0).all())
