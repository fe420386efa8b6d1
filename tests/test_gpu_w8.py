"""GPU parity of the 8-bit weight paths (MLX affine 8-bit, group 64) against the CPU oracle, through the C ABI:
ifd_gemm_w8 (the qmv8 arithmetic, core.metal:175-248, for M <= 32; MLX's 8-bit qmm dequant above) and ifd_qmm_w8a8
(w4a8_gemm with BITS = 8, w4a8.metal:43-98). Tolerances as for 4 bits: 1e-2 RMS (bf16 paths), 2e-2 RMS (W8A8)."""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import gen

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")
FLIP8 = 0x80808080


def _gu():
    from tests import gpu_util
    return gpu_util


def _ops():
    from inferd_amd import ops
    return ops


def _check(M, N, K, mode, seed, flipped=False, bias="minus128"):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear8(N, K, seed=seed, bias=bias)
    A = gen.activations(M, K, seed=seed + 1)
    W = g.qlinear(wq ^ np.uint32(FLIP8) if flipped else wq, s, b, flipped, bits=8)
    C0 = gen.activations(M, N, seed=seed + 2) if mode == 1 else None
    out = ops.gemm(g.dev(A), W, g.dev(C0) if mode == 1 else None, mode=mode)
    torch.cuda.synchronize()
    Y = orc.qmv(A, wq, s, b, bits=8) if M <= 32 else orc.qmm(A, wq, s, b, bits=8)
    got = g.host(out)
    ref = Y + gen.bf16_to_f32(C0) if mode == 1 else Y
    st = gen.check_out(got, ref, 1e-2, (M, N, K, mode, flipped), fp32=mode == 2)
    return st if mode == 2 else st["net"]


@pytest.mark.parametrize("M", [1, 2, 5, 8, 9, 16, 17, 32, 33, 64, 65, 128, 129, 300])
def test_gemm_w8_rows(M):
    """Every routing boundary: the GEMV variants (8 / 16 / 32 rows, then 2 and 4 dequant tiles) and the prefill
    GEMM; N = 200 leaves a partial 32-column band and a partial 128-column tile."""
    _check(M, 200, 512, 0, seed=100 + M, bias="free")


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("M", [1, 48, 200])
def test_gemm_w8_modes_and_flip(M, mode):
    _check(M, 384, 1024, mode, seed=200 + M, flipped=(mode != 0))


def test_gemm_w8_config0_shape():
    """BASELINE config 0's shape with 8-bit weights: M = 1, K = N = 5120 (the K-split path)."""
    _check(1, 5120, 5120, 0, seed=300)


def test_gemm_w8_k_slice_view():
    """Columns [k0, k0 + kn) of a wider 8-bit matrix (ldk = full K): one byte per code."""
    from inferd_amd._lib import check, lib
    g = _gu()
    N, Kf, k0, kn = 128, 1024, 256, 512
    codes, wq, s, b = gen.qlinear8(N, Kf, seed=310, bias="free")
    wq_d, s_d, b_d = g.dev(wq), g.dev(s), g.dev(b)
    sub = lambda a, lo, hi: np.ascontiguousarray(a[:, lo:hi])
    for M in (4, 200):
        A = gen.activations(M, kn, seed=311 + M)
        C = torch.empty((M, N), dtype=torch.bfloat16, device="cuda")
        ws = torch.zeros(max(lib().ifd_gemm_w8_workspace(M, N, kn), 256), dtype=torch.uint8, device="cuda")
        check(lib().ifd_gemm_w8(g.dev(A).data_ptr(), kn, wq_d.data_ptr() + k0, s_d.data_ptr() + k0 // 64 * 2,
                                b_d.data_ptr() + k0 // 64 * 2, N, kn, Kf, 0, C.data_ptr(), N, M, 0, ws.data_ptr(),
                                ws.numel(), torch.cuda.current_stream().cuda_stream))
        ref = orc.qmv if M <= 32 else orc.qmm
        Y = ref(A, sub(wq, k0 // 4, (k0 + kn) // 4), sub(s, k0 // 64, (k0 + kn) // 64), sub(b, k0 // 64, (k0 + kn) // 64),
                bits=8)
        gen.check_bf16(g.host(C), Y, 1e-2, M)


@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("M,N,K", [(37, 200, 512), (128, 384, 1024), (300, 256, 5120)])
def test_w8a8(M, N, K, per_token):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear8(N, K, seed=M + 30, bias="free")
    A = gen.activations(M, K, seed=M + 31)
    U, XS = orc.a8_quant(A, per_token)
    Y = orc.w4a8(U, XS, wq, s, b, bits=8)
    for flipped, mode in ((False, 0), (True, 2), (True, 0)):
        W = g.qlinear(wq ^ np.uint32(FLIP8) if flipped else wq, s, b, flipped, bits=8)
        out = g.host(ops.qmm_w4a8(g.dev(U), g.dev(XS), per_token, W, mode=mode))
        gen.check_out(out, Y, 1e-4 if mode == 2 else 1e-2, (M, N, K, per_token, flipped, mode), fp32=mode == 2)


def test_flip_8bit_in_place():
    """ops.flip on an 8-bit layer XORs every byte with 0x80 (reference w_flip with the 8-bit mask); a GEMM on the
    flipped layer gives the unflipped result."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear8(64, 256, seed=400)
    W = g.qlinear(wq, s, b, bits=8)
    ops.flip(W)
    assert W.flipped and np.array_equal(g.host(W.wq).view(np.uint32), wq ^ np.uint32(FLIP8))
    A = gen.activations(3, 256, seed=401)
    gen.check_bf16(g.host(ops.gemm(g.dev(A), W)), orc.qmv(A, wq, s, b, bits=8), 1e-2, "flipped")
