"""GPU parity of the T64x8 path (8-bit weights repacked into MFMA fragment order, inferd_amd/csrc/t64.h) through
the C ABI: ifd_pack_t64x8 bit-exact against the numpy restatement of the layout, and ifd_gemm_t64x8_w8a8 against the
oracle's w4a8_gemm with BITS = 8 (engine/kernels/w4a8.metal:43-98, the offset 128 at :57) on the same int8
inputs: 1e-2 RMS net on bf16 outputs, 1e-4 on fp32 outputs (the product is exact integers plus fp32 rounding; the
2e-2 of BASELINE's W4A8 tolerance covers the activation quantization, which both sides share here). The shapes cover one cut tile, tiles cut into many pieces, runs of one unit, empty runs (fewer units than
CUs), ragged N and whole-tile work beside the stream-K share (the BASELINE config 3 shape, sampled rows)."""
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


@pytest.mark.parametrize("N,K", [(200, 512), (64, 64), (1024, 2048)])
@pytest.mark.parametrize("flipped", [False, True])
def test_pack_t64x8_bit_exact(N, K, flipped):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear8(N, K, seed=N + K, bias="free")
    W = g.qlinear(wq ^ np.uint32(FLIP8) if flipped else wq, s, b, flipped, bits=8)
    T = ops.pack_t64x8(W)
    torch.cuda.synchronize()
    assert T.wt.numel() == gen.pack_t64x8(codes, s, b).size
    assert np.array_equal(g.host(T.wt), gen.pack_t64x8(codes, s, b))


@pytest.mark.parametrize("M,N,K", [(37, 200, 512), (128, 384, 1024), (300, 256, 5120), (1, 32, 64),
                                   (200, 640, 17408), (129, 1000, 256), (300, 22016, 256)])
def test_gemm_t64x8_w8a8(M, N, K):
    """All store modes, independent biases (b' = b + 128 s far from 0). 37 x 200 x 512: one tile cut over 8 blocks;
    300 x 256 x 5120: 3 tiles, 240 units on 240 blocks (runs of one unit); 1 x 32 x 64: one unit on one block;
    200 x 640 x 17408: 6 tiles of 272 groups, each cut into about 43 pieces; 129 x 1000 x 256: a ragged last band
    and a second M tile of one row; 300 x 22016 x 256: 258 tiles on 256 CUs, one whole tile per block and 2 tiles of
    4 groups split over 8 blocks (the other runs empty)."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear8(N, K, seed=M + 40, bias="free")
    A = gen.activations(M, K, seed=M + 41)
    U, XS = orc.a8_quant(A, True)
    T = ops.pack_t64x8(g.qlinear(wq, s, b, bits=8))
    Y = orc.w4a8(U, XS, wq, s, b, bits=8)
    C0 = gen.activations(M, N, seed=M + 42)
    for mode in (0, 1, 2):
        C = g.dev(C0) if mode == 1 else None
        out = g.host(ops.gemm_t64x8_w8a8(g.dev(U), g.dev(XS), T, C, mode=mode))
        # the same int8 inputs on both sides: the bars are the output rounding's (bf16 1e-2 net, fp32 1e-4)
        gen.check_out(out, Y + gen.bf16_to_f32(C0) if mode == 1 else Y, 1e-4 if mode == 2 else 1e-2,
                      (M, N, K, mode), fp32=mode == 2)


def test_gemm_t64x8_w8a8_bias_low_half():
    """The bias b' = b + 128 s enters as bf16 b'_hi = bf16(b') plus b'_lo = bf16(b' - b'_hi). Here b'_lo is non-zero
    in every (column, group) and the activations have mean 1, so sum xq is large and the bias term dominates: the
    fp32 output (mode 2) is held to 1e-4 RMS, and the oracle with b'_lo dropped is shown to miss that bar by over
    10x, so a kernel that lost the low half fails."""
    g, ops = _gu(), _ops()
    M, N, K = 64, 256, 1024
    codes, wq, s, b = gen.qlinear8(N, K, seed=91, bias="free")

    def low_half(b):
        bp = gen.bf16_to_f32(b).astype(np.float64) + 128.0 * gen.bf16_to_f32(s).astype(np.float64)
        hi = gen.bf16_to_f32(gen.f32_to_bf16(bp.astype(np.float32))).astype(np.float64)
        return gen.bf16_to_f32(gen.f32_to_bf16((bp - hi).astype(np.float32))).astype(np.float64)

    b = b & np.uint16(0x7FFF)  # positive biases: b' = b + 128 s has no cancellation, so it is never finer than b
    for _ in range(32):  # where b' is exactly a bf16, move b one bf16 step
        z = low_half(b) == 0.0
        if not z.any():
            break
        b[z] = (b[z].astype(np.uint32) + 1).astype(np.uint16)
    lo = low_half(b)
    assert np.all(lo != 0.0), "every (column, group) needs a non-zero low half"
    rng = np.random.default_rng(92)
    A = gen.f32_to_bf16((1.0 + 0.5 * rng.standard_normal((M, K))).astype(np.float32))
    U, XS = orc.a8_quant(A, True)
    Y = orc.w4a8(U, XS, wq, s, b, bits=8)
    out = g.host(ops.gemm_t64x8_w8a8(g.dev(U), g.dev(XS), ops.pack_t64x8(g.qlinear(wq, s, b, bits=8)), mode=2))
    gen.check_out(out, Y, 1e-4, (M, N, K, "b' low half"), fp32=True)
    # the planted mistake, on the CPU: without b'_lo the product moves by sum_g b'_lo X_g sx
    drop = XS[:, :, 1].astype(np.float64) @ lo.T
    assert np.max(np.abs(drop)) / np.sqrt(np.mean(Y.astype(np.float64) ** 2)) > 1e-3


def test_gemm_t64x8_w8a8_flipped_minus128():
    """A flipped source layer (the reference's load-time w_flip with the 8-bit mask) packs to the same tiles, and
    b = -128 s (b' = 0) gives the same product as the MLX-layout W8A8 GEMM."""
    g, ops = _gu(), _ops()
    M, N, K = 96, 512, 2048
    codes, wq, s, b = gen.qlinear8(N, K, seed=77)
    A = gen.activations(M, K, seed=78)
    U, XS = orc.a8_quant(A, True)
    Y = orc.w4a8(U, XS, wq, s, b, bits=8)
    Wf = g.qlinear(wq ^ np.uint32(FLIP8), s, b, True, bits=8)
    out = g.host(ops.gemm_t64x8_w8a8(g.dev(U), g.dev(XS), ops.pack_t64x8(Wf)))
    gen.check_out(out, Y, 2e-2, (M, N, K, "flipped"))
    mlx = g.host(ops.qmm_w4a8(g.dev(U), g.dev(XS), True, Wf))
    gen.check_out(out, gen.bf16_to_f32(mlx), 2e-2, (M, N, K, "vs MLX-layout W8A8"))


def test_gemm_t64x8_w8a8_config3_sampled():
    """The BASELINE config 3 shape in 8 bits (M=2048, K=N=5120, per-token int8): 320 tiles on 256 CUs, so one whole
    tile per block plus 64 tiles split stream-K. The oracle on 16 sampled rows; a row-sum property on all rows."""
    g, ops = _gu(), _ops()
    M, N, K = 2048, 5120, 5120
    codes, wq, s, b = gen.qlinear8(N, K, seed=80, bias="free")
    A = gen.activations(M, K, seed=81)
    U, XS = ops.a8_quant(g.dev(A), True)
    out = g.host(ops.gemm_t64x8_w8a8(U, XS, ops.pack_t64x8(g.qlinear(wq, s, b, bits=8)), mode=2))
    rows = np.linspace(0, M - 1, 16).astype(int)
    Uh, XSh = g.host(U), g.host(XS)
    Y = orc.w4a8(Uh[rows], XSh[rows], wq, s, b, bits=8)
    gen.check_out(out[rows], Y, 1e-4, ("config3 rows",), fp32=True)
    # every row: sum over n of y[m][n] = sx sum_g (P_g . sum_n s + X_g . sum_n b') is linear in the weights, so the
    # product with the column sums of the dequantized weights (fp64 on the host) must match the row sums
    G = K // 64
    q = codes.astype(np.float64).reshape(N, G, 64)
    Wd = q * gen.bf16_to_f32(s).astype(np.float64)[..., None] + gen.bf16_to_f32(b).astype(np.float64)[..., None]
    wsum = Wd.reshape(N, K).sum(0)
    xq = Uh.astype(np.float64) * np.repeat(XSh[:, :, 0].astype(np.float64), 64, axis=1)
    ref = xq @ wsum
    got = out.astype(np.float64).sum(1)
    err = np.sqrt(np.mean((got - ref) ** 2)) / np.sqrt(np.mean(ref ** 2))
    assert err < 1e-3, err



@pytest.mark.parametrize("M,N,K", [(17, 200, 512), (32, 1024, 2048), (33, 384, 1024), (64, 640, 17408),
                                   (100, 256, 5120), (128, 5120, 1024), (300, 1000, 256), (1, 64, 64)])
def test_gemm_t64x8_bf16(M, N, K):
    """The stream-K bf16 GEMM on T64x8 weights against MLX's 8-bit qmm semantics (bf16(s q + b) dequant, fp32 sums),
    1e-2 RMS, all store modes: 32-, 64- and 128-row tiles, tiles cut into many pieces (K = 17408), ragged N and M."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear8(N, K, seed=M + 50, bias="free")
    A = gen.activations(M, K, seed=M + 51)
    T = ops.pack_t64x8(g.qlinear(wq, s, b, bits=8))
    Y = orc.qmm(A, wq, s, b, bits=8)
    C0 = gen.activations(M, N, seed=M + 52)
    for mode in (0, 1, 2):
        C = g.dev(C0) if mode == 1 else None
        out = g.host(ops.gemm_t64x8(g.dev(A), T, C, mode=mode))
        gen.check_out(out, Y + gen.bf16_to_f32(C0) if mode == 1 else Y, 1e-2, (M, N, K, mode), fp32=mode == 2)


def test_gemm_t64x8_bf16_matches_mlx_layout():
    """At M = 128 on the decode MLP's gate_up shape (N = 34816, K = 5120) the T64x8 GEMM and the MLX-layout 8-bit
    GEMM (ifd_gemm_w8, the same dequant rounding) agree; the oracle on 8 sampled rows."""
    g, ops = _gu(), _ops()
    M, N, K = 128, 34816, 5120
    codes, wq, s, b = gen.qlinear8(N, K, seed=90)
    A = gen.activations(M, K, seed=91)
    W = g.qlinear(wq, s, b, bits=8)
    out = g.host(ops.gemm_t64x8(g.dev(A), ops.pack_t64x8(W), mode=2))
    ref = g.host(ops.gemm(g.dev(A), W, mode=2))
    gen.check_out(out, ref, 1e-3, ("vs MLX layout",), fp32=True)
    rows = np.linspace(0, M - 1, 8).astype(int)
    gen.check_out(out[rows], orc.qmm(A[rows], wq, s, b, bits=8), 1e-2, ("rows",), fp32=True)


@pytest.mark.parametrize("M,N,K", [(1, 200, 512), (8, 5120, 5120), (16, 384, 17408), (5, 1000, 2048),
                                   (1, 34816, 5120)])
def test_gemm_t64x8_decode(M, N, K):
    """M <= 16 (K % 128 == 0) runs the T64 decode GEMV on T64x8 tiles: the reference's qmv8 arithmetic (per group
    s * sum q x + b * sum x, fp32), 1e-2 RMS against the oracle's qmv, all store modes; K split with the in-kernel
    fixup on the long shapes (the workspace header is checked back at zero after every GPU test)."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear8(N, K, seed=M + 60, bias="free")
    A = gen.activations(M, K, seed=M + 61)
    T = ops.pack_t64x8(g.qlinear(wq, s, b, bits=8))
    Y = orc.qmv(A, wq, s, b, bits=8)
    C0 = gen.activations(M, N, seed=M + 62)
    for mode in (0, 1, 2):
        C = g.dev(C0) if mode == 1 else None
        out = g.host(ops.gemm_t64x8(g.dev(A), T, C, mode=mode))
        gen.check_out(out, Y + gen.bf16_to_f32(C0) if mode == 1 else Y, 1e-2, (M, N, K, mode), fp32=mode == 2)


def test_t64x8_strides_through_the_c_abi():
    """The stride arguments of the T64x8 entry points, through the C ABI: ifd_pack_t64x8 from a K-slice view of a
    wider MLX matrix (ldk = 2 K, columns [K, 2 K)) packs the same bytes as the sliced matrix, and both GEMMs store
    rows ldc > N apart without touching the gap."""
    g, ops = _gu(), _ops()
    from inferd_amd._lib import lib
    N, K = 320, 1024
    codes, wq, s, b = gen.qlinear8(N, 2 * K, seed=120, bias="free")
    W2 = g.qlinear(wq, s, b, bits=8)  # [N][2K]
    T = torch.empty((lib().ifd_t64x8_bytes(N, K),), dtype=torch.uint8, device="cuda")
    # the view's first element is column K: wq words K / 4, scales K / 64
    wq_v = W2.wq.view(-1)[K // 4:]
    s_v, b_v = W2.s.view(-1)[K // 64:], W2.b.view(-1)[K // 64:]
    assert lib().ifd_pack_t64x8(ops._p(wq_v), ops._p(s_v), ops._p(b_v), N, K, 2 * K, 0, ops._p(T), ops._stream()) == 0
    torch.cuda.synchronize()
    cs, ss, bs = codes[:, K:], s[:, K // 64:], b[:, K // 64:]
    assert np.array_equal(g.host(T), gen.pack_t64x8(np.ascontiguousarray(cs), np.ascontiguousarray(ss),
                                                     np.ascontiguousarray(bs)))
    wq_s = np.ascontiguousarray(wq[:, K // 4:])
    ldc = N + 40
    for M, w8a8 in ((5, False), (40, False), (150, False), (150, True)):
        A = gen.activations(M, K, seed=M + 121)
        C = torch.full((M, ldc), 7.0, dtype=torch.float32, device="cuda")
        if w8a8:
            U, XS = orc.a8_quant(A, True)
            Y = orc.w4a8(U, XS, wq_s, np.ascontiguousarray(ss), np.ascontiguousarray(bs), bits=8)
            need = lib().ifd_gemm_t64x8_w8a8_workspace(M, N, K)
            ws = ops.workspace(need, C.device)
            dU, dXS = g.dev(U), g.dev(XS)  # held until the kernel has run (a freed block is reused at once)
            rc = lib().ifd_gemm_t64x8_w8a8(ops._p(dU), ops._p(dXS), 1, ops._p(T), N, K, ops._p(C), ldc, M, 2,
                                           ops._p(ws), ws.numel(), ops._stream())
            torch.cuda.synchronize()
        else:
            fn = orc.qmv if M <= 16 else orc.qmm
            Y = fn(A, wq_s, np.ascontiguousarray(ss), np.ascontiguousarray(bs), bits=8)
            need = lib().ifd_gemm_t64x8_workspace(M, N, K)
            ws = ops.workspace(need, C.device) if need else None
            dA = g.dev(A)
            rc = lib().ifd_gemm_t64x8(ops._p(dA), K, ops._p(T), N, K, ops._p(C), ldc, M, 2, ops._p(ws),
                                      ws.numel() if ws is not None else 0, ops._stream())
            torch.cuda.synchronize()
        assert rc == 0, lib().ifd_last_error()
        out = g.host(C)
        gen.check_out(out[:, :N], Y, 1e-4 if w8a8 else 1e-2, (M, N, K, "ldc", w8a8), fp32=True)
        assert np.all(out[:, N:] == 7.0), "a store landed in the row gap"
