"""GPU parity of the dense paths (decode GEMV, prefill GEMM, W4A8, SwiGLU, flip) against the CPU oracle.

Every call goes through the C ABI (libinferd_amd.so via inferd_amd.ops). Tolerances are BASELINE's:
max |err| <= 1e-2 RMS(ref) for bf16 paths and <= 2e-2 RMS(ref) for W4A8; integer outputs bit-exact.
Shapes at BASELINE's full sizes that the oracle cannot finish in seconds are checked on sampled rows (each output
row of a GEMM is independent of the others).
"""
import numpy as np
import pytest

from oracle import oracle as orc
from tests import gen

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


def _gu():
    from tests import gpu_util
    return gpu_util


def _ops():
    from inferd_amd import ops
    return ops


def _check_gemm(M, N, K, mode, path, seed, flipped=False, row_scale=False):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=seed)
    A = gen.activations(M, K, seed=seed + 1, row_scale=row_scale)
    W = g.qlinear(wq ^ np.uint32(0x88888888) if flipped else wq, s, b, flipped)
    C0 = gen.activations(M, N, seed=seed + 2) if mode == 1 else None
    Cd = g.dev(C0) if mode == 1 else None
    out = ops.gemm(g.dev(A), W, Cd, mode=mode, path=path)
    torch.cuda.synchronize()
    # semantics: the decode path's affine variant (M <= 32) is qmv4's, everything else MLX qmm's
    affine = (path == "qmv" or (path == "auto" and M <= 128)) and M <= 32
    Y = orc.qmv(A, wq, s, b) if affine else orc.qmm(A, wq, s, b)
    got = g.host(out)
    # against the fp32 value the bf16 store rounds (mode 1 adds the bf16 residual first)
    ref = Y + gen.bf16_to_f32(C0) if mode == 1 else Y
    st = gen.check_out(got, ref, 1e-2, (M, N, K, mode, path), fp32=mode == 2)
    return st if mode == 2 else st["net"]


@pytest.mark.parametrize("M", [1, 2, 3, 5, 8, 9, 16, 17, 32, 33, 64, 65, 100, 128])
def test_qmv_rows(M):
    _check_gemm(M, 200, 512, 0, "qmv", seed=M)


@pytest.mark.parametrize("mode", [0, 1, 2])
@pytest.mark.parametrize("M", [1, 8, 48])
def test_qmv_modes_and_flip(M, mode):
    _check_gemm(M, 384, 1024, mode, "qmv", seed=10 + M, flipped=(mode == 1))


def test_qmv_config0_full_size():
    """M=1, K=N=5120 (split-K path)."""
    err = _check_gemm(1, 5120, 5120, 0, "auto", seed=0)
    assert err < 1e-2


@pytest.mark.parametrize("M", [1, 8, 32, 128])
def test_decode_mlp_shapes_sampled(M):
    """BASELINE config 1 shapes: gate_up 5120 -> 34816 and down 17408 -> 5120 (oracle on 8 sampled rows)."""
    g, ops = _gu(), _ops()
    for (N, K, seed) in [(34816, 5120, 21), (5120, 17408, 22)]:
        codes, wq, s, b = gen.qlinear(N, K, seed=seed)
        A = gen.activations(M, K, seed=seed + M)
        out = g.host(ops.gemm(g.dev(A), g.qlinear(wq, s, b)))
        rows = np.unique(np.linspace(0, M - 1, min(M, 8)).astype(int))
        Y = orc.qmv(A[rows], wq, s, b) if M <= 32 else orc.qmm(A[rows], wq, s, b)
        gen.check_bf16(out[rows], Y, 1e-2, (M, N, K))


@pytest.mark.parametrize("M,N,K", [(129, 200, 512), (256, 256, 1024), (300, 520, 640), (1000, 1024, 2048)])
@pytest.mark.parametrize("mode", [0, 1, 2])
def test_qmm(M, N, K, mode):
    _check_gemm(M, N, K, mode, "qmm", seed=M + N + mode, flipped=(mode == 2))


def test_qmm_small_m_and_odd_n():
    for M in (1, 7, 33):
        _check_gemm(M, 72, 192, 0, "qmm", seed=M)


def test_qmm_config2_full_size_sampled():
    """M=4096, K=5120, N=17408, rows scaled by U(0.5, 2); oracle on 16 sampled rows."""
    g, ops = _gu(), _ops()
    M, N, K = 4096, 17408, 5120
    codes, wq, s, b = gen.qlinear(N, K, seed=31)
    A = gen.activations(M, K, seed=32, row_scale=True)
    out = g.host(ops.gemm(g.dev(A), g.qlinear(wq, s, b)))
    rows = np.linspace(0, M - 1, 16).astype(int)
    Y = orc.qmm(A[rows], wq, s, b)
    gen.check_bf16(out[rows], Y, 1e-2, "config 2")
    assert np.all(np.isfinite(gen.bf16_to_f32(out)))


def test_k_slice_view():
    """A K-slice view (reference kslice_of, weights.h:259-268): columns [k0, k0+kn) of a wider matrix, ldk = full K."""
    from inferd_amd._lib import check, lib
    g = _gu()
    N, Kf, k0, kn, M = 128, 1024, 256, 512, 4
    codes, wq, s, b = gen.qlinear(N, Kf, seed=40)
    A = gen.activations(M, kn, seed=41)
    wq_d, s_d, b_d = g.dev(wq), g.dev(s), g.dev(b)
    for M_ in (M, 200):
        A_ = gen.activations(M_, kn, seed=42 + M_)
        Ad = g.dev(A_)
        C = torch.empty((M_, N), dtype=torch.bfloat16, device="cuda")
        ws = torch.empty(max(lib().ifd_gemm_w4_workspace(M_, N, kn), 256), dtype=torch.uint8, device="cuda")
        check(lib().ifd_gemm_w4(Ad.data_ptr(), kn, wq_d.data_ptr() + k0 // 2, s_d.data_ptr() + k0 // 64 * 2,
                                b_d.data_ptr() + k0 // 64 * 2, N, kn, Kf, 0, C.data_ptr(), N, M_, 0, ws.data_ptr(),
                                ws.numel(), torch.cuda.current_stream().cuda_stream))
        sub = lambda a, lo, hi: np.ascontiguousarray(a[:, lo:hi])
        Y = (orc.qmv if M_ <= 32 else orc.qmm)(A_, sub(wq, k0 // 8, (k0 + kn) // 8), sub(s, k0 // 64, (k0 + kn) // 64),
                                               sub(b, k0 // 64, (k0 + kn) // 64))
        gen.check_bf16(g.host(C), Y, 1e-2, M_)


@pytest.mark.parametrize("per_token", [False, True])
def test_a8_quant_bit_exact(per_token):
    g, ops = _gu(), _ops()
    A = gen.activations(37, 1024, seed=50, row_scale=True)
    A[3, :] = 0  # all-zero row: sx = 1
    U, XS = ops.a8_quant(g.dev(A), per_token)
    Ur, XSr = orc.a8_quant(A, per_token)
    assert np.array_equal(g.host(U), Ur)
    assert np.array_equal(g.host(XS), XSr)


@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("M,N,K", [(37, 200, 512), (128, 384, 1024), (300, 256, 5120)])
def test_w4a8(M, N, K, per_token):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=M + 3)
    A = gen.activations(M, K, seed=M + 4)
    U, XS = orc.a8_quant(A, per_token)
    for flipped, mode in ((False, 0), (True, 2)):
        W = g.qlinear(wq ^ np.uint32(0x88888888) if flipped else wq, s, b, flipped)
        out = g.host(ops.qmm_w4a8(g.dev(U), g.dev(XS), per_token, W, mode=mode))
        Y = orc.w4a8(U, XS, wq, s, b)
        gen.check_out(out, Y, 1e-4 if mode == 2 else 1e-2, (M, N, K, per_token, flipped), fp32=mode == 2)


def test_w4a8_config3_sampled():
    """M=2048, K=N=5120, per-token int8 activations; oracle on 16 sampled rows."""
    g, ops = _gu(), _ops()
    M, N, K = 2048, 5120, 5120
    codes, wq, s, b = gen.qlinear(N, K, seed=60)
    A = gen.activations(M, K, seed=61)
    U, XS = ops.a8_quant(g.dev(A), True)
    out = g.host(ops.qmm_w4a8(U, XS, True, g.qlinear(wq, s, b)))
    rows = np.linspace(0, M - 1, 16).astype(int)
    Ur, XSr = orc.a8_quant(A[rows], True)
    assert np.array_equal(g.host(U)[rows], Ur)
    gen.check_bf16(out[rows], orc.w4a8(Ur, XSr, wq, s, b), 2e-2, "config 3")


def test_silu_mul_and_flip():
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(70)
    gu = gen.f32_to_bf16((rng.standard_normal((33, 2 * 512)) * 3).astype(np.float32))
    h = gen.bf16_to_f32(g.host(ops.silu_mul(g.dev(gu))))
    hr = gen.bf16_to_f32(orc.silu_mul(gu))
    # expf may differ in the last ulp between the GPU and libm: at most one bf16 step apart
    assert np.all(np.abs(h - hr) <= 2 ** -7 * np.abs(hr) + 1e-30)
    assert np.mean(h == hr) > 0.99
    codes, wq, s, b = gen.qlinear(64, 256, seed=71)
    W = g.qlinear(wq, s, b)
    ops.flip(W)
    assert W.flipped and np.array_equal(g.host(W.wq).view(np.uint32), wq ^ np.uint32(0x88888888))


@pytest.mark.parametrize("per_token", [False, True])
@pytest.mark.parametrize("R,D", [(1, 2048), (16, 5120), (37, 320)])
def test_rmsnorm_a8(R, D, per_token):
    """The fused rmsnorm_a8 gives the bits of ifd_rmsnorm then ifd_a8_quant; its quantization is the oracle's a8_quant
    of the normalised rows, bit for bit, and the rows are the oracle's rmsnorm within one bf16 step."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(90 + R)
    x = gen.f32_to_bf16((rng.standard_normal((R, D)) * rng.uniform(0.1, 10, (R, 1))).astype(np.float32))
    x[0, : D // 2] = 0  # a zero half: groups with amax 0 (sx = 1)
    w = gen.f32_to_bf16(rng.uniform(0.5, 2.0, D).astype(np.float32))
    xd, wd = g.dev(x), g.dev(w)
    y, U, XS = ops.rmsnorm_a8(xd, wd, 1e-6, per_token)
    y0 = ops.rmsnorm(xd, wd, 1e-6)
    U0, XS0 = ops.a8_quant(y0, per_token)
    y, U, XS, y0 = g.host(y), g.host(U), g.host(XS), g.host(y0)
    assert np.array_equal(y, y0) and np.array_equal(U, g.host(U0)) and np.array_equal(XS, g.host(XS0))
    Ur, XSr = orc.a8_quant(y, per_token)
    assert np.array_equal(U, Ur) and np.array_equal(XS, XSr)
    assert np.all(gen.bf16_steps(y, orc.rmsnorm(x, w, 1e-6)) <= 1)


@pytest.mark.parametrize("I", [17408, 1088])
@pytest.mark.parametrize("per_token", [False, True])
def test_silu_mul_a8(per_token, I):
    """silu_mul_a8 gives the bits of ifd_silu_mul then ifd_a8_quant, and the oracle's a8_quant of that product. Per
    group a row spreads over 2048-column blocks: I = 17408 ends in a half block, I = 1088 is less than one."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(95)
    gu = gen.f32_to_bf16((rng.standard_normal((9, 2 * I)) * 3).astype(np.float32))
    gu[2, I:] = 0  # up = 0: a zero row
    gd = g.dev(gu)
    U, XS = ops.silu_mul_a8(gd, per_token)
    h = ops.silu_mul(gd)
    U0, XS0 = ops.a8_quant(h, per_token)
    assert np.array_equal(g.host(U), g.host(U0)) and np.array_equal(g.host(XS), g.host(XS0))
    Ur, XSr = orc.a8_quant(g.host(h), per_token)
    assert np.array_equal(g.host(U), Ur) and np.array_equal(g.host(XS), XSr)


@pytest.mark.parametrize("a8", [None, False, True])
@pytest.mark.parametrize("S,R,D", [(1, 3, 256), (12, 32, 5120), (4, 128, 2048), (3, 5, 2112)])
def test_splitk_res_norm(S, R, D, a8):
    """splitk_res_norm: the updated residual rows are the oracle's split-order fp32 sum plus x, bit for bit; the
    normalised rows are ifd_rmsnorm of them and the quantization ifd_a8_quant of those, bit for bit."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(100 + S + R)
    part = (rng.standard_normal((S, R, D)) * 0.3).astype(np.float32)
    x = gen.f32_to_bf16(rng.standard_normal((R, D)).astype(np.float32))
    w = gen.f32_to_bf16(rng.uniform(0.5, 2.0, D).astype(np.float32))
    xd, wd = g.dev(x), g.dev(w)
    res = ops.splitk_res_norm(torch.from_numpy(part).cuda(), xd, wd, 1e-6, a8)
    y = res if a8 is None else res[0]
    xn = g.host(xd)
    assert np.array_equal(xn, orc.splitk_res(part, x))
    y0 = ops.rmsnorm(g.dev(xn), wd, 1e-6)
    assert np.array_equal(g.host(y), g.host(y0))
    if a8 is not None:
        U0, XS0 = ops.a8_quant(y0, a8)
        assert np.array_equal(g.host(res[1]), g.host(U0)) and np.array_equal(g.host(res[2]), g.host(XS0))


@pytest.mark.parametrize("R,D,eps", [(1, 2048, 1e-6), (16, 5120, 1e-6), (37, 333, 0.0), (5, 64, 7.0), (3, 6221, 1e-5)])
def test_rmsnorm(R, D, eps):
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(80 + R)
    x = gen.f32_to_bf16((rng.standard_normal((R, D)) * rng.uniform(0.1, 10, (R, 1))).astype(np.float32))
    w = gen.f32_to_bf16(rng.uniform(0.5, 2.0, D).astype(np.float32))
    y = g.host(ops.rmsnorm(g.dev(x), g.dev(w), eps))
    yr = orc.rmsnorm(x, w, eps)
    # the fp32 sum of squares runs in another order than the oracle's: within one bf16 step of its output
    assert np.all(gen.bf16_steps(y, yr) <= 1)
    assert np.mean(y == yr) > 0.98


def test_qa8_quant_bit_exact_and_gemm():
    """The int8 prefill path (reference qa8_quant + qa8_gemm, qa8.metal:30-210): the qa8 quantizer form is bit-exact,
    and with the per-group W4A8 GEMM on unflipped and flipped weights it matches the oracle's identity."""
    g, ops = _gu(), _ops()
    M, N, K = 300, 256, 1024
    A = gen.activations(M, K, seed=70, row_scale=True)
    A[5, 64:128] = 0  # an all-zero group: sx = 0
    U, XS = ops.a8_quant(g.dev(A), 2)
    Ur, XSr = orc.a8_quant(A, 2)
    assert np.array_equal(g.host(U), Ur)
    assert np.array_equal(g.host(XS), XSr)
    codes, wq, s, b = gen.qlinear(N, K, seed=71, bias="free")
    Y = orc.w4a8(Ur, XSr, wq, s, b)
    for flipped in (False, True):
        W = g.qlinear(wq ^ np.uint32(0x88888888) if flipped else wq, s, b, flipped)
        out = g.host(ops.qmm_w4a8(U, XS, False, W))
        gen.check_bf16(out, Y, 2e-2, flipped)
