"""Pins the CPU oracle (oracle/qmm_oracle.cpp) before anything is checked against it.

Each check is independent of the oracle's own code: exhaustive nibble known answers, exact-rational golden vectors
(tests/golden/known_answers.json), float64 textbook GEMMs in numpy, closed-form special cases (one-hot probes, the
all-8 zero weight), brute-force routing by lexsort and numpy's stable argsort for dispatch.
"""
import json
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests import gen

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")


# ---- format ---------------------------------------------------------------------------------------------------------
def test_unpack_known_words():
    wq = np.array([[0x76543210, 0xFEDCBA98]], np.uint32)
    assert orc.unpack_w4(wq, 16).tolist() == [list(range(16))]
    # flipped storage: q ^ 8 in every nibble, undone by xr
    assert orc.unpack_w4(wq ^ np.uint32(0x88888888), 16, 0x88888888).tolist() == [list(range(16))]


def test_unpack_exhaustive_every_code_every_position():
    rows = []
    for pos in range(8):
        for code in range(16):
            rows.append(code << (4 * pos))
    wq = np.array(rows, np.uint32).reshape(-1, 1)
    codes = orc.unpack_w4(wq, 8)
    i = 0
    for pos in range(8):
        for code in range(16):
            want = [0] * 8
            want[pos] = code
            assert codes[i].tolist() == want
            i += 1


def test_pack_roundtrip_matches_numpy_layout():
    codes, wq_np, _, _ = gen.qlinear(7, 256, seed=3)
    wq = orc.pack_w4(codes)
    assert np.array_equal(wq, wq_np)
    assert np.array_equal(orc.unpack_w4(wq, 256), codes)
    fl = orc.flip(wq)
    assert np.array_equal(fl, wq ^ np.uint32(0x88888888))
    assert np.array_equal(orc.unpack_w4(fl, 256, 0x88888888), codes)


def test_bf16_rounding_matches_numpy_rne():
    rng = np.random.default_rng(0)
    x = np.concatenate([rng.standard_normal(10000).astype(np.float32),
                        np.array([1.0, 1.00390625, 1.01171875, -2.5, 0.0, 65504.0], np.float32)])
    # exact ties: 1 + 2^-8 rounds down to 1 (even), 1 + 3*2^-8 rounds up
    assert np.array_equal(orc.f32_to_bf16(x), gen.f32_to_bf16(x))
    assert gen.bf16_to_f32(orc.f32_to_bf16(np.array([1.00390625], np.float32)))[0] == 1.0


# ---- golden (exact rational) --------------------------------------------------------------------------------------
def _golden_cases():
    with open(GOLDEN) as f:
        return json.load(f)["cases"]


@pytest.mark.parametrize("ci", [0, 1])
def test_golden_qmv_qmm(ci):
    c = _golden_cases()[ci]
    codes = np.array(c["codes"], np.uint8)
    s = np.array(c["s_bf16"], np.uint16)
    b = np.array(c["b_bf16"], np.uint16)
    x = np.array(c["x_bf16"], np.uint16)
    wq = gen.pack_codes(codes)
    y = orc.qmv(x, wq, s, b)
    assert gen.rel_err(y, np.array(c["qmv"])) < 1e-5
    y = orc.qmm(x, wq, s, b)
    assert gen.rel_err(y, np.array(c["qmm"])) < 1e-5
    # the two semantics differ only by the bf16 rounding of the dequantized weights
    assert gen.rel_err(np.array(c["qmm"]), np.array(c["qmv"])) < 1e-2


@pytest.mark.parametrize("ci", [0, 1])
@pytest.mark.parametrize("per_token", [False, True])
def test_golden_a8(ci, per_token):
    c = _golden_cases()[ci]
    key = "a8_token" if per_token else "a8_group"
    x = np.array(c["x_bf16"], np.uint16)
    U, XS = orc.a8_quant(x, per_token)
    assert np.array_equal(U.astype(np.int64), np.array(c[key]["xq"], np.int64))
    assert np.array_equal(XS[:, :, 0], np.array(c[key]["sx"], np.float32))
    wq = gen.pack_codes(np.array(c["codes"], np.uint8))
    y = orc.w4a8(U, XS, wq, np.array(c["s_bf16"], np.uint16), np.array(c["b_bf16"], np.uint16))
    assert gen.rel_err(y, np.array(c[key]["y"])) < 1e-5


# ---- closed forms ---------------------------------------------------------------------------------------------------
def test_one_hot_probe_is_dequant():
    N, K = 16, 256
    codes, wq, s, b = gen.qlinear(N, K, seed=11, bias="free")
    ks = [0, 1, 7, 8, 63, 64, 130, 255]
    A = np.zeros((len(ks), K), np.uint16)
    for i, k in enumerate(ks):
        A[i, k] = 0x3F80  # bf16 1.0
    w32 = orc.dequant_f32(wq, s, b, K)
    wbf = gen.bf16_to_f32(orc.dequant_bf16(wq, s, b, K))
    yv, ym = orc.qmv(A, wq, s, b), orc.qmm(A, wq, s, b)
    for i, k in enumerate(ks):
        # qmv: s*q + b exactly (fp32); qmm: bf16(s*q + b)
        sk = gen.bf16_to_f32(s[:, k // 64]).astype(np.float64)
        bk = gen.bf16_to_f32(b[:, k // 64]).astype(np.float64)
        exact = sk * codes[:, k] + bk
        assert np.allclose(yv[i], exact, rtol=2 ** -22, atol=0)
        assert np.array_equal(yv[i], w32[:, k])
        assert np.array_equal(ym[i], wbf[:, k])


def test_all_eights_is_exactly_zero():
    N, K = 8, 512
    _, _, s, b = gen.qlinear(N, K, seed=5)  # b = -8 s
    wq = gen.pack_codes(np.full((N, K), 8, np.uint8))
    A = gen.activations(4, K, seed=6)
    assert np.all(orc.qmv(A, wq, s, b) == 0)
    assert np.all(orc.qmm(A, wq, s, b) == 0)
    U, XS = orc.a8_quant(A, False)
    assert np.all(np.abs(orc.w4a8(U, XS, wq, s, b)) < 1e-3)


@pytest.mark.parametrize("M,N,K", [(37, 200, 512), (1, 64, 5120), (5, 96, 1088)])
def test_gemms_match_float64_textbook(M, N, K):
    """micro/qtest.mm's odd shape 37 x 200 x 512 and two decode-like shapes."""
    codes, wq, s, b = gen.qlinear(N, K, seed=M + N)
    A = gen.activations(M, K, seed=K)
    x64 = gen.bf16_to_f32(A).astype(np.float64)
    w64 = gen.dequant_f64(codes, s, b)
    assert gen.rel_err(orc.qmv(A, wq, s, b), x64 @ w64.T) < 1e-5
    wbf = gen.bf16_to_f32(gen.f32_to_bf16(w64.astype(np.float32))).astype(np.float64)
    ym = orc.qmm(A, wq, s, b)
    assert gen.rel_err(ym, x64 @ wbf.T) < 1e-5
    # the reference's own pass bar for this check (micro/qtest.mm:121)
    ref = x64 @ w64.T
    assert np.max(np.abs(ym - ref)) <= 2e-3 * np.max(np.abs(ref)) + 1e-2


@pytest.mark.parametrize("per_token", [False, True])
def test_a8_quant_properties(per_token):
    A = gen.activations(6, 320, seed=9, row_scale=True)
    U, XS = orc.a8_quant(A, per_token)
    x = gen.bf16_to_f32(A).astype(np.float64)
    sx = np.repeat(XS[:, :, 0], 64, axis=1).astype(np.float64)
    assert np.all(np.abs(U.astype(np.int32)) <= 127)
    # round to nearest of the fp32 quotient x / sx: within half a step up to the quotient's own rounding
    assert np.all(np.abs(U * sx - x) <= 0.5 * sx * (1 + 1e-5))
    if per_token:
        assert np.all(XS[:, :, 0] == XS[:, :1, 0])
        amax = np.abs(x).max(axis=1)
        assert np.all(np.abs(U).max(axis=1) == 127)
    q = U.reshape(6, 5, 64).sum(axis=2).astype(np.float32)
    assert np.allclose(XS[:, :, 1], XS[:, :, 0] * q)


@pytest.mark.parametrize("per_token", [False, True])
def test_w4a8_identity(per_token):
    """sum (s q + b)(sx xq) over a group = s sx sum q xq + b sx sum xq (w4a8.metal:8): the W4A8 result equals a
    float64 GEMM of the dequantized weights against the dequantized activations sx * xq."""
    M, N, K = 9, 48, 640
    codes, wq, s, b = gen.qlinear(N, K, seed=2, bias="free")
    A = gen.activations(M, K, seed=4)
    U, XS = orc.a8_quant(A, per_token)
    xd = U.astype(np.float64) * np.repeat(XS[:, :, 0], 64, axis=1)
    ref = xd @ gen.dequant_f64(codes, s, b).T
    assert gen.rel_err(orc.w4a8(U, XS, wq, s, b), ref) < 1e-5
    # flipped storage gives the same result
    assert gen.rel_err(orc.w4a8(U, XS, wq ^ np.uint32(0x88888888), s, b, xr=0x88888888), ref) < 1e-5


# ---- 8-bit weights (qmv8, core.metal:175-248; MLX 8-bit qmm; W8A8, w4a8.metal BITS = 8) ----------------------------
def test_unpack8_exhaustive_every_code_every_position():
    """Every code 0..255 in each of the four byte positions; flipped storage (q ^ 0x80) undone by xr."""
    rows = [code << (8 * pos) for pos in range(4) for code in range(256)]
    wq = np.array(rows, np.uint32).reshape(-1, 1)
    codes = orc.unpack_w8(wq, 4)
    i = 0
    for pos in range(4):
        for code in range(256):
            want = [0] * 4
            want[pos] = code
            assert codes[i].tolist() == want
            i += 1
    assert np.array_equal(orc.unpack_w8(wq ^ np.uint32(0x80808080), 4, 0x80808080), codes)
    c = np.arange(256, dtype=np.uint8).reshape(2, 128)
    assert np.array_equal(orc.pack_w8(c), gen.pack_codes8(c))
    assert int(orc.pack_w8(c)[0, 0]) == 0x03020100


def test_one_hot_probe_is_dequant_8bit():
    N, K = 16, 256
    codes, wq, s, b = gen.qlinear8(N, K, seed=12, bias="free")
    ks = [0, 1, 3, 4, 63, 64, 129, 255]
    A = np.zeros((len(ks), K), np.uint16)
    for i, k in enumerate(ks):
        A[i, k] = 0x3F80
    w32 = orc.dequant_f32_bits(wq, s, b, K, 8)
    yv, ym = orc.qmv(A, wq, s, b, bits=8), orc.qmm(A, wq, s, b, bits=8)
    for i, k in enumerate(ks):
        sk = gen.bf16_to_f32(s[:, k // 64]).astype(np.float64)
        bk = gen.bf16_to_f32(b[:, k // 64]).astype(np.float64)
        exact = sk * codes[:, k] + bk
        assert np.allclose(yv[i], exact, rtol=2 ** -22, atol=0)
        assert np.array_equal(yv[i], w32[:, k])
        assert np.array_equal(gen.f32_to_bf16(ym[i]), gen.f32_to_bf16((sk * codes[:, k] + bk).astype(np.float32)))


def test_all_128_is_exactly_zero_8bit():
    N, K = 8, 512
    _, _, s, b = gen.qlinear8(N, K, seed=5)  # b = -128 s (exact: 128 s is a power-of-two multiple)
    wq = gen.pack_codes8(np.full((N, K), 128, np.uint8))
    A = gen.activations(4, K, seed=6)
    assert np.all(orc.qmv(A, wq, s, b, bits=8) == 0)
    assert np.all(orc.qmm(A, wq, s, b, bits=8) == 0)
    U, XS = orc.a8_quant(A, False)
    assert np.all(np.abs(orc.w4a8(U, XS, wq, s, b, bits=8)) < 1e-3)


@pytest.mark.parametrize("M,N,K", [(37, 200, 512), (1, 64, 5120)])
def test_gemms_8bit_match_float64_textbook(M, N, K):
    codes, wq, s, b = gen.qlinear8(N, K, seed=M + N + 1, bias="free")
    A = gen.activations(M, K, seed=K + 1)
    x64 = gen.bf16_to_f32(A).astype(np.float64)
    w64 = gen.dequant_f64(codes, s, b)
    assert gen.rel_err(orc.qmv(A, wq, s, b, bits=8), x64 @ w64.T) < 1e-5
    wbf = gen.bf16_to_f32(gen.f32_to_bf16(w64.astype(np.float32))).astype(np.float64)
    assert gen.rel_err(orc.qmm(A, wq, s, b, bits=8), x64 @ wbf.T) < 1e-5
    # a 4-bit reading of the same words is a different matrix: the width is not silently ignored
    assert gen.rel_err(orc.qmv(A, wq[:, : K // 8], s, b), x64 @ w64.T) > 0.1


@pytest.mark.parametrize("per_token", [False, True])
def test_w8a8_identity(per_token):
    """The W8A8 identity (w4a8.metal:8 with offset 128): float64 GEMM of the dequantized 8-bit weights against
    sx * xq; flipped storage (q ^ 0x80) gives the same result."""
    M, N, K = 9, 48, 640
    codes, wq, s, b = gen.qlinear8(N, K, seed=3, bias="free")
    A = gen.activations(M, K, seed=5)
    U, XS = orc.a8_quant(A, per_token)
    xd = U.astype(np.float64) * np.repeat(XS[:, :, 0], 64, axis=1)
    ref = xd @ gen.dequant_f64(codes, s, b).T
    assert gen.rel_err(orc.w4a8(U, XS, wq, s, b, bits=8), ref) < 1e-5
    assert gen.rel_err(orc.w4a8(U, XS, wq ^ np.uint32(0x80808080), s, b, xr=0x80808080, bits=8), ref) < 1e-5


def test_store_modes():
    Y = np.array([[1.5, -2.25], [3.0e-3, 7.0]], np.float32)
    C = gen.f32_to_bf16(np.array([[1.0, 1.0], [1.0, -7.0]], np.float32))
    assert np.array_equal(orc.store(Y, 0), gen.f32_to_bf16(Y))
    assert np.array_equal(orc.store(Y, 1, C), gen.f32_to_bf16(Y + gen.bf16_to_f32(C)))
    assert np.array_equal(orc.store(Y, 2), Y)


def test_silu_mul_closed_form():
    rng = np.random.default_rng(1)
    gu = gen.f32_to_bf16(rng.standard_normal((5, 2 * 96)).astype(np.float32) * 3)
    h = gen.bf16_to_f32(orc.silu_mul(gu))
    g = gen.bf16_to_f32(gu[:, :96]).astype(np.float64)
    u = gen.bf16_to_f32(gu[:, 96:]).astype(np.float64)
    ref = g / (1 + np.exp(-g)) * u
    # two bf16 roundings: within 2^-7 relative
    assert np.all(np.abs(h - ref) <= 2 ** -7 * np.abs(ref) + 1e-30)


def test_rmsnorm_exact_rows():
    """Rows whose RMS norm is exact: a mistake in the mean (D vs D - 1), the root, where eps enters, or the weight
    index changes one of these outputs."""
    rng = np.random.default_rng(3)
    D = 16
    w = gen.f32_to_bf16(rng.uniform(0.5, 2.0, D).astype(np.float32))
    wf = gen.bf16_to_f32(w)
    x = np.zeros((3, D), np.float32)
    x[0, :] = 4.0                   # constant 2^k, eps = 0: r = 1/4, out = w exactly
    x[1, 5] = 2.0                   # one-hot c e_i: mean = c^2 / D, r = sqrt(D) / c = 2, out_i = 4 w_i
    x[2, :] = -0.5                  # sign kept
    out = gen.bf16_to_f32(orc.rmsnorm(gen.f32_to_bf16(x), w, 0.0))
    assert np.array_equal(out[0], wf)
    want1 = np.zeros(D, np.float32)
    want1[5] = 4.0 * wf[5]
    assert np.array_equal(out[1], want1)
    assert np.array_equal(out[2], -wf)
    # eps inside the root, added to the mean square: c = 3, eps = 7 -> r = 1 / 4, out = 0.75 w
    x3 = np.full((1, D), 3.0, np.float32)
    out3 = gen.bf16_to_f32(orc.rmsnorm(gen.f32_to_bf16(x3), w, 7.0))
    assert np.array_equal(out3[0], gen.bf16_to_f32(gen.f32_to_bf16(0.75 * wf)))


def test_rmsnorm_scale_invariance():
    rng = np.random.default_rng(4)
    x = gen.f32_to_bf16(rng.standard_normal((3, 64)).astype(np.float32))
    w = gen.f32_to_bf16(rng.uniform(0.5, 2.0, 64).astype(np.float32))
    xs = gen.f32_to_bf16(gen.bf16_to_f32(x) * 8.0)  # exact power-of-two scaling
    assert np.array_equal(orc.rmsnorm(x, w, 0.0), orc.rmsnorm(xs, w, 0.0))


def test_rmsnorm_a8_exact_rows():
    """rmsnorm_a8 composes rmsnorm and a8_quant on the bf16 output: a constant 2^k row with w = 1 normalises to 1.0
    exactly (eps = 1e-6 vanishes in the fp32 mean 64), so every group has amax 1, sx = 1/127, q = 127 and
    XS = (1/127, 64 * 127 * sx) in fp32; a row of zeros quantizes with sx = 1 and q = 0."""
    D = 128
    x = np.zeros((2, D), np.float32)
    x[0, :] = 8.0
    w = gen.f32_to_bf16(np.ones(D, np.float32))
    for per_token in (False, True):
        out, U, XS = orc.rmsnorm_a8(gen.f32_to_bf16(x), w, 1e-6, per_token)
        assert np.all(gen.bf16_to_f32(out[0]) == 1.0) and np.all(out[1] == 0)
        sx = np.float32(1.0) / np.float32(127.0)
        assert np.all(U[0] == 127) and np.all(U[1] == 0)
        assert np.all(XS[0, :, 0] == sx) and np.all(XS[0, :, 1] == sx * np.float32(64 * 127))
        assert np.all(XS[1, :, 0] == 1.0) and np.all(XS[1, :, 1] == 0.0)
        Ur, XSr = orc.a8_quant(out, per_token)
        assert np.array_equal(U, Ur) and np.array_equal(XS, XSr)


def test_silu_mul_a8_composes():
    """silu_mul_a8 is a8_quant of the bf16 silu_mul output: u = 0 rows quantize to zeros with sx = 1, and random rows
    match the explicit composition."""
    rng = np.random.default_rng(5)
    gu = gen.f32_to_bf16((rng.standard_normal((4, 256)) * 2).astype(np.float32))
    gu[1, 128:] = 0  # up = 0: h = 0
    for per_token in (False, True):
        U, XS = orc.silu_mul_a8(gu, per_token)
        assert np.all(U[1] == 0) and np.all(XS[1, :, 0] == 1.0)
        Ur, XSr = orc.a8_quant(orc.silu_mul(gu), per_token)
        assert np.array_equal(U, Ur) and np.array_equal(XS, XSr)


def test_splitk_res_exact_sums():
    """The residual split-K reduce of splitk_res_norm: on dyadic values whose fp32 sums are exact the result is
    bf16(sum + x) of the float64 sum (a dropped split, a wrong residual or a missing rounding fails); on random values
    the fp32 sum runs in split order (((p0 + p1) + p2) + x), not in another association."""
    rng = np.random.default_rng(6)
    S, R, D = 3, 2, 64
    part = (rng.integers(-64, 64, (S, R, D)) / 8.0).astype(np.float32)
    x = gen.f32_to_bf16((rng.integers(-32, 32, (R, D)) / 4.0).astype(np.float32))
    want = gen.f32_to_bf16((part.astype(np.float64).sum(0) + gen.bf16_to_f32(x)).astype(np.float32))
    assert np.array_equal(orc.splitk_res(part, x), want)
    # split order: 1 + 2^-24 + 2^-24 - 1 is 0 in order ((1 + e) + e) - 1 but 2^-23 when the e's are added first
    e = np.float32(2.0 ** -24)
    p = np.array([[[1.0]], [[e]], [[e]], [[-1.0]]], np.float32)
    assert gen.bf16_to_f32(orc.splitk_res(p, gen.f32_to_bf16(np.zeros((1, 1), np.float32))))[0, 0] == 0.0
    xn, out = orc.splitk_res_norm(part, x, gen.f32_to_bf16(np.ones(D, np.float32)), 1e-6)
    assert np.array_equal(xn, want) and np.array_equal(out, orc.rmsnorm(want, gen.f32_to_bf16(np.ones(D, np.float32)), 1e-6))


# ---- MoE ------------------------------------------------------------------------------------------------------------
def _brute_topk(l: np.ndarray, k: int):
    order = np.lexsort((np.arange(l.size), -l.astype(np.float64)))  # logit desc, then index asc
    return order[:k]


def test_router_gemm_one_hot_and_numpy():
    """Router logits (bf16 x bf16, fp32 accumulation): a one-hot row returns one weight column exactly; random rows
    match numpy's float64 matmul of the same bf16 values within fp32 accumulation error."""
    rng = np.random.default_rng(11)
    E1, H = 33, 256
    W = gen.f32_to_bf16((rng.standard_normal((E1, H)) * 0.02).astype(np.float32))
    x = np.zeros((2, H), np.float32)
    x[0, 17] = 1.0
    x[1, 200] = -2.0
    y = orc.gemm_bf16(gen.f32_to_bf16(x), W)
    Wf = gen.bf16_to_f32(W)
    assert np.array_equal(y[0], Wf[:, 17]) and np.array_equal(y[1], -2.0 * Wf[:, 200])
    A = gen.activations(9, H, seed=12)
    y = orc.gemm_bf16(A, W).astype(np.float64)
    ref = gen.bf16_to_f32(A).astype(np.float64) @ Wf.astype(np.float64).T
    assert np.max(np.abs(y - ref)) <= 1e-5 * np.sqrt(np.mean(ref ** 2))


@pytest.mark.parametrize("bf", [False, True])
def test_route_brute_force(bf):
    rng = np.random.default_rng(3)
    T, E, k = 64, 512, 10
    logits = (rng.standard_normal((T, E + 1)) * 0.9).astype(np.float32)
    if bf:
        logits = gen.f32_to_bf16(logits)
        lf = gen.bf16_to_f32(logits)
    else:
        lf = logits
    idx, wt, sg = orc.moe_route(logits, E, k)
    for t in range(T):
        assert idx[t].tolist() == _brute_topk(lf[t, :E], k).tolist()
    assert np.allclose(wt.sum(axis=1), 1.0, atol=1e-6)
    assert np.all(np.diff(wt, axis=1) <= 0)
    assert np.allclose(sg, 1 / (1 + np.exp(-lf[:, E].astype(np.float64))), rtol=1e-6)
    _, _, sg1 = orc.moe_route(logits, E, k, shared_gate=False)
    assert np.all(sg1 == 1.0)


def test_route_ties_pick_lowest_index():
    E, k = 64, 4
    l = np.zeros((1, E + 1), np.float32)
    l[0, [5, 9, 40, 41, 63]] = 2.0  # five-way tie for the top 4
    idx, wt, _ = orc.moe_route(l, E, k)
    assert idx[0].tolist() == [5, 9, 40, 41]
    assert np.allclose(wt, 0.25)


def test_dispatch_is_stable_counting_sort():
    rng = np.random.default_rng(8)
    T, k, E = 300, 10, 512
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    offsets, perm, inv = orc.moe_dispatch(idx, E)
    flat = idx.reshape(-1)
    assert np.array_equal(perm, np.argsort(flat, kind="stable"))
    assert np.array_equal(offsets[:-1], np.concatenate([[0], np.cumsum(np.bincount(flat, minlength=E))[:-1]]))
    assert offsets[-1] == flat.size
    assert np.array_equal(inv[perm], np.arange(flat.size))


def test_gather_qmm_is_per_row_qmm():
    rng = np.random.default_rng(2)
    E, N, K, T, k = 6, 64, 128, 20, 2
    stacks = [gen.qlinear(N, K, seed=100 + e) for e in range(E)]
    wq = np.stack([st[1] for st in stacks])
    s = np.stack([st[2] for st in stacks])
    b = np.stack([st[3] for st in stacks])
    x = gen.activations(T, K, seed=1)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    offsets, perm, inv = orc.moe_dispatch(idx, E)
    Y = orc.moe_gather_qmm(x, perm, k, offsets, wq, s, b, N, K)
    for r in range(T * k):
        e = idx.reshape(-1)[r]
        yr = orc.qmm(x[r // k:r // k + 1], wq[e], s[e], b[e])
        assert np.array_equal(Y[inv[r]], yr[0])


def test_combine_closed_form():
    rng = np.random.default_rng(4)
    T, H, k = 5, 64, 3
    yd = gen.f32_to_bf16(rng.standard_normal((T * k, H)).astype(np.float32))
    ys = gen.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    wt = rng.uniform(0, 1, (T, k)).astype(np.float32)
    sg = rng.uniform(0, 1, T).astype(np.float32)
    inv = rng.permutation(T * k).astype(np.int32)
    x0 = gen.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    out = orc.moe_combine(x0, yd, wt, ys, sg, inv, k, assign=True)
    ydf, ysf = gen.bf16_to_f32(yd).astype(np.float64), gen.bf16_to_f32(ys).astype(np.float64)
    ref = np.stack([sum(wt[t, j] * ydf[inv[t * k + j]] for j in range(k)) + sg[t] * ysf[t] for t in range(T)])
    assert np.all(np.abs(gen.bf16_to_f32(out) - ref) <= 2 ** -8 * np.abs(ref) + 1e-6)
    res = orc.moe_combine(x0, yd, wt, ys, sg, inv, k, assign=False)
    ref2 = gen.bf16_to_f32(x0) + gen.bf16_to_f32(out)
    assert np.all(np.abs(gen.bf16_to_f32(res) - ref2) <= 2 ** -8 * np.abs(ref2) + 1e-6)


def test_moe_experts_composition():
    """The composed FFN equals routing-weighted per-token expert MLPs (float64, bf16 rounding points aside)."""
    rng = np.random.default_rng(12)
    E, H, I, T, k = 8, 128, 64, 6, 2
    egu = [gen.qlinear(2 * I, H, seed=200 + e) for e in range(E)]
    edn = [gen.qlinear(H, I, seed=300 + e) for e in range(E)]
    sgu, sdn = gen.qlinear(2 * I, H, seed=400), gen.qlinear(H, I, seed=401)
    st = lambda L, i: np.stack([q[i] for q in L])
    xn = gen.activations(T, H, seed=13)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    wt = rng.uniform(0.1, 1, (T, k)).astype(np.float32)
    wt /= wt.sum(axis=1, keepdims=True)
    sg = rng.uniform(0, 1, T).astype(np.float32)
    out = orc.moe_experts(xn, idx, wt, sg, (st(egu, 1), st(egu, 2), st(egu, 3)), (st(edn, 1), st(edn, 2), st(edn, 3)),
                          ((sgu[1], sgu[2], sgu[3]), (sdn[1], sdn[2], sdn[3])), I)
    x = gen.bf16_to_f32(xn).astype(np.float64)

    def mlp(gu, dn, xr):
        h = xr @ gen.dequant_f64(gu[0], gu[2], gu[3]).T
        a = h[:, :I] / (1 + np.exp(-h[:, :I])) * h[:, I:]
        return a @ gen.dequant_f64(dn[0], dn[2], dn[3]).T

    ref = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            ref[t] += wt[t, j] * mlp(egu[idx[t, j]], edn[idx[t, j]], x[t:t + 1])[0]
        ref[t] += sg[t] * mlp(sgu, sdn, x[t:t + 1])[0]
    got = gen.bf16_to_f32(out).astype(np.float64)
    # five bf16 rounding points (gate/up, SwiGLU twice, down, combine) against an unrounded float64 pipeline; a wrong
    # expert, weight or row would be an O(1) error
    assert gen.rel_err(got, ref) < 5e-2
    assert np.sqrt(np.mean((got - ref) ** 2) / np.mean(ref ** 2)) < 1e-2


def test_moe_decode_composition():
    """The decode MoE (T <= 8) equals routing-weighted per-token expert MLPs in float64 up to its bf16 rounding points,
    and its residual form is bf16(x + its assign form) exactly."""
    rng = np.random.default_rng(21)
    E, H, I, T, k = 8, 128, 64, 5, 3
    egu = [gen.qlinear(2 * I, H, seed=500 + e, bias="free") for e in range(E)]
    edn = [gen.qlinear(H, I, seed=600 + e, bias="free") for e in range(E)]
    sgu, sdn = gen.qlinear(2 * I, H, seed=700, bias="free"), gen.qlinear(H, I, seed=701, bias="free")
    st = lambda L, i: np.stack([q[i] for q in L])
    xn = gen.activations(T, H, seed=22)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    idx[1] = idx[0]  # two tokens with the same experts
    wt = rng.uniform(0.1, 1, (T, k)).astype(np.float32)
    wt /= wt.sum(axis=1, keepdims=True)
    sg = rng.uniform(0, 1, T).astype(np.float32)
    args = ((st(egu, 1), st(egu, 2), st(egu, 3)), (st(edn, 1), st(edn, 2), st(edn, 3)),
            ((sgu[1], sgu[2], sgu[3]), (sdn[1], sdn[2], sdn[3])), I)
    out = orc.moe_decode(xn, idx, wt, sg, *args)
    x = gen.bf16_to_f32(xn).astype(np.float64)

    def mlp(gu, dn, xr):
        h = xr @ gen.dequant_f64(gu[0], gu[2], gu[3]).T
        a = h[:, :I] / (1 + np.exp(-h[:, :I])) * h[:, I:]
        return a @ gen.dequant_f64(dn[0], dn[2], dn[3]).T

    ref = np.zeros((T, H))
    for t in range(T):
        for j in range(k):
            ref[t] += wt[t, j] * mlp(egu[idx[t, j]], edn[idx[t, j]], x[t:t + 1])[0]
        ref[t] += sg[t] * mlp(sgu, sdn, x[t:t + 1])[0]
    got = gen.bf16_to_f32(out).astype(np.float64)
    assert np.sqrt(np.mean((got - ref) ** 2) / np.mean(ref ** 2)) < 1e-2
    assert np.array_equal(out[0], out[1]) == np.array_equal(xn[0], xn[1])
    x0 = gen.activations(T, H, seed=23)
    res = orc.moe_decode(xn, idx, wt, sg, *args, out=x0, assign=False)
    want = gen.f32_to_bf16(gen.bf16_to_f32(x0) + gen.bf16_to_f32(out))
    assert np.array_equal(res, want)
    # without the shared expert the shared term is absent
    no_sh = orc.moe_decode(xn, idx, wt, sg, args[0], args[1], None, I)
    ref2 = ref - sg[:, None] * np.stack([mlp(sgu, sdn, x[t:t + 1])[0] for t in range(T)])
    got2 = gen.bf16_to_f32(no_sh).astype(np.float64)
    assert np.sqrt(np.mean((got2 - ref2) ** 2) / np.mean(ref2 ** 2)) < 1e-2
    # an 8-bit shared expert (moe_gu2_4_8 / moe_dn2_4_8): the shared term is that expert's MLP in float64
    sgu8, sdn8 = gen.qlinear8(2 * I, H, seed=702, bias="free"), gen.qlinear8(H, I, seed=703, bias="free")

    def deq8(q):
        codes, _, sc, bi = q
        N, K = codes.shape
        return (codes.astype(np.float64).reshape(N, K // 64, 64) * gen.bf16_to_f32(sc).astype(np.float64)[..., None]
                + gen.bf16_to_f32(bi).astype(np.float64)[..., None]).reshape(N, K)

    def mlp8(xr):
        h = xr @ deq8(sgu8).T
        a = h[:, :I] / (1 + np.exp(-h[:, :I])) * h[:, I:]
        return a @ deq8(sdn8).T

    out8 = orc.moe_decode(xn, idx, wt, sg, args[0], args[1], ((sgu8[1], sgu8[2], sgu8[3]), (sdn8[1], sdn8[2], sdn8[3])),
                          I, shared_bits=8)
    ref8 = ref2 + sg[:, None] * np.stack([mlp8(x[t:t + 1])[0] for t in range(T)])
    got8 = gen.bf16_to_f32(out8).astype(np.float64)
    assert np.sqrt(np.mean((got8 - ref8) ** 2) / np.mean(ref8 ** 2)) < 1e-2
    # the 8-bit shared expert's term is not the 4-bit one read as 8-bit (a wrong width would be an O(1) error)
    assert np.sqrt(np.mean((got8 - ref) ** 2) / np.mean(ref ** 2)) > 1e-1


def test_qa8_quant_form():
    """The int8 prefill's quantizer (qa8.metal:30-49): q = clamp(rint(x * (127 / amax)), +-127), sx = amax / 127,
    0 for an all-zero group. amax = 127 makes q = rint(x) exactly (ties to even); a value is picked where multiplying
    by 127 / amax and dividing by amax / 127 round to different codes, so the two forms cannot be confused."""
    g0 = np.zeros(64, np.float32)
    g0[0], g0[1], g0[2], g0[3], g0[4] = 127, 2.5, -3.5, 0.5, -126.75
    # search a (amax, x) pair in bf16 where the two quotients round to different integers
    pick = None
    for amax in np.linspace(1.0, 3.0, 400, dtype=np.float32):
        a = gen.bf16_to_f32(gen.f32_to_bf16(np.array([amax], np.float32)))[0]
        xs = gen.bf16_to_f32(gen.f32_to_bf16(np.linspace(-a, a, 257, dtype=np.float32)))
        m = np.rint(xs * np.float32(127 / np.float32(a))) != np.rint(xs / np.float32(a / np.float32(127)))
        if m.any():
            pick = (a, xs[m][0])
            break
    assert pick is not None
    g1 = np.zeros(64, np.float32)
    g1[0], g1[1] = pick
    g2 = np.zeros(64, np.float32)
    A = gen.f32_to_bf16(np.concatenate([g0, g1, g2])[None])
    U, XS = orc.a8_quant(A, 2)
    assert U[0, :5].tolist() == [127, 2, -4, 0, -127]
    a, x = pick
    assert U[0, 65] == np.clip(np.rint(x * np.float32(127 / np.float32(a))), -127, 127)
    assert U[0, 65] != np.rint(x / np.float32(a / np.float32(127)))
    assert XS[0, 0, 0] == np.float32(127) / np.float32(127) and XS[0, 1, 0] == np.float32(a) / np.float32(127)
    assert XS[0, 2, 0] == 0 and XS[0, 2, 1] == 0 and (U[0, 128:] == 0).all()
    assert np.isclose(XS[0, 0, 1], XS[0, 0, 0] * U[0, :64].sum())


def test_moe_gather_w4a8_is_per_row_w4a8():
    """The int8 gathered expert GEMM (qa8g) equals, row by row, the W4A8 product of the row's expert on the token row
    it reads (up to fp32 rounding: W4A8 forms (q - 8) and b + 8 s, qa8g unflipped q and b), and the float64 GEMM of the
    dequantized weights against sx * xq."""
    rng = np.random.default_rng(31)
    E, N, K, T, k = 4, 48, 256, 6, 2
    parts = [gen.qlinear(N, K, seed=40 + e, bias="free") for e in range(E)]
    wq = np.stack([p[1] for p in parts]); s = np.stack([p[2] for p in parts]); b = np.stack([p[3] for p in parts])
    A = gen.activations(T, K, seed=32)
    U, XS = orc.a8_quant(A, 2)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    offsets, perm, inv = orc.moe_dispatch(idx, E)
    Y = orc.moe_gather_w4a8(U, XS, perm, k, offsets, wq, s, b, N, K)
    for q in range(T * k):
        e = int(np.searchsorted(offsets, q, side="right") - 1)
        r = perm[q] // k
        want = orc.w4a8(U[r:r + 1], XS[r:r + 1], wq[e], s[e], b[e])[0]
        assert gen.rel_err(Y[q:q + 1], want[None]) < 1e-5
        xd = U[r].astype(np.float64) * np.repeat(XS[r, :, 0], 64)
        ref = gen.dequant_f64(parts[e][0], parts[e][2], parts[e][3]) @ xd
        assert gen.rel_err(Y[q:q + 1], ref[None]) < 1e-5
