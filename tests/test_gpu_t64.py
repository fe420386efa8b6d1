"""GPU checks of the T64 weight layout: the repack is bit-exact against a numpy restatement of the layout, and
GEMMs on T64 weights match the CPU oracle (decode GEMV semantics) through the C ABI."""
import functools

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


@pytest.mark.parametrize("N,K,flipped", [(64, 256, False), (200, 512, True), (5120, 1024, False)])
def test_pack_t64_bit_exact(N, K, flipped):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=N + K, bias="free")
    W = g.qlinear(wq ^ np.uint32(0x88888888) if flipped else wq, s, b, flipped)
    T = ops.pack_t64(W)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(T.wt), gen.pack_t64(codes, s, b))


@pytest.mark.parametrize("M", [1, 2, 5, 8, 9, 16])
@pytest.mark.parametrize("N,K", [(200, 512), (5120, 5120), (384, 17408)])
def test_gemm_t64_decode(M, N, K):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=M * 7 + N)
    A = gen.activations(M, K, seed=M + K)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    out = g.host(ops.gemm_t64(g.dev(A), T))
    Y = orc.qmv(A, wq, s, b)
    gen.check_bf16(out, Y, 1e-2, (M, N, K))


@pytest.mark.parametrize("mode", [1, 2])
def test_gemm_t64_modes(mode):
    g, ops = _gu(), _ops()
    M, N, K = 4, 256, 1024
    codes, wq, s, b = gen.qlinear(N, K, seed=mode)
    A = gen.activations(M, K, seed=mode + 1)
    C0 = gen.activations(M, N, seed=mode + 2)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    out = g.host(ops.gemm_t64(g.dev(A), T, g.dev(C0) if mode == 1 else None, mode=mode))
    Y = orc.qmv(A, wq, s, b)
    gen.check_out(out, Y if mode == 2 else Y + gen.bf16_to_f32(C0), 1e-2, mode, fp32=mode == 2)


def _t64_semantics(M):
    """The T64 GEMM's arithmetic by M: the decode GEMV's exact affine form up to 16 rows (the reference's qmv/qmvt4
    rows), bf16 dequant (MLX qmm, which the reference runs above them) beyond. The K-split fallback for shapes past
    the counter header keeps the affine form up to 64 rows; the two forms agree well within the bar."""
    return orc.qmv if M <= 16 else orc.qmm


def _t64_arith(M, N, K, cus=256):
    """The oracle form of the arithmetic ifd_gemm_t64 routes an M x [N, K] product to (capi.hip, gemm_t64.hip,
    gemm_sk.hip): the decode GEMV's affine form (qmv4: s sum q x + b sum x) in the decode kernel (M <= 16) and in
    the K-split kernel's 32- and 64-row tiles; bf16(s q + b) dequant (MLX qmm) in the prefill tiles, the stream-K
    kernel and the K-split kernel's 128-row tiles."""
    if M <= 16:
        return orc.qmv
    bands = (N + 31) // 32
    if ((M + 255) // 256) * ((bands + 7) // 8) >= cus:
        return orc.qmm
    mt = 1 if M <= 32 else 2 if M <= 64 else 4
    if ((M + 32 * mt - 1) // (32 * mt)) * ((bands + 7) // 8) * 3 >= cus or 64 < M <= 128:
        return orc.qmm
    return orc.qmm if mt == 4 else orc.qmv


# ---- exactly what bench.py times: config 1's two products at its four M ----------------------------------------
BENCH_MS = [1, 8, 32, 128]
H1, I1 = 5120, 17408


@functools.lru_cache(maxsize=None)
def _config1_weights():
    """Seeded config-1 layer (gate_up [2 I, H] with gate rows first, down [H, I]), host arrays."""
    _, wg, sg_, bg = gen.qlinear(2 * I1, H1, seed=1000)
    _, wd, sd, bd = gen.qlinear(H1, I1, seed=1001)
    return (wg, sg_, bg), (wd, sd, bd)


@functools.lru_cache(maxsize=None)
def _config1_t64():
    g, ops = _gu(), _ops()
    (wg, sg_, bg), (wd, sd, bd) = _config1_weights()
    return ops.pack_t64(g.qlinear(wg, sg_, bg)), ops.pack_t64(g.qlinear(wd, sd, bd))


def _rows_of(lin, rows):
    return tuple(np.ascontiguousarray(a[rows]) for a in lin)


@pytest.mark.parametrize("M", BENCH_MS)
def test_gemm_t64_swiglu_bench_shapes(M):
    """bench.py's gate_up + SwiGLU call (N = 2 x 17408, K = 5120) at each of its M, every row, against the oracle on
    768 h columns (gate rows c and up rows I + c): h = silu_mul(bf16(A . W^T)) with the GEMM in the arithmetic of its
    route. Columns cover the first and last tiles and tile edges."""
    g, ops = _gu(), _ops()
    gu_w, _ = _config1_weights()
    GU, _ = _config1_t64()
    A = gen.activations(M, H1, seed=1100 + M)
    h = g.host(ops.gemm_t64_swiglu(g.dev(A), GU))
    rng = np.random.default_rng(M)
    cols = np.unique(np.concatenate([np.arange(0, 128), np.arange(I1 - 128, I1), rng.choice(I1, 512, replace=False)]))
    y = _t64_arith(M, 2 * I1, H1)(A, *_rows_of(gu_w, np.concatenate([cols, I1 + cols])))
    ref = orc.silu_mul(gen.f32_to_bf16(y))
    gen.check_bf16(h[:, cols], ref, 1e-2, M, ref_is_bf16=True)


@pytest.mark.parametrize("M", BENCH_MS)
def test_gemm_t64_down_bench_shapes(M):
    """bench.py's down call (N = 5120, K = 17408) at each of its M, every row, against the oracle on 640 output
    columns in the arithmetic of its route."""
    g, ops = _gu(), _ops()
    _, dn_w = _config1_weights()
    _, DN = _config1_t64()
    A = gen.activations(M, I1, seed=1200 + M)
    out = g.host(ops.gemm_t64(g.dev(A), DN))
    rng = np.random.default_rng(M + 1)
    cols = np.unique(np.concatenate([np.arange(0, 128), np.arange(H1 - 128, H1), rng.choice(H1, 384, replace=False)]))
    y = _t64_arith(M, H1, I1)(A, *_rows_of(dn_w, cols))
    gen.check_bf16(out[:, cols], y, 1e-2, M)


@pytest.mark.parametrize("M", BENCH_MS)
def test_mlp_decode_config1_matches_oracle(M):
    """The dense decode MLP block at config 1's shapes, x += down(SwiGLU(gate_up(rmsnorm(x)))), against the oracle's
    composition on 4 sampled rows (rows are independent through the block), each GEMM in its route's arithmetic."""
    g, ops = _gu(), _ops()
    gu_w, dn_w = _config1_weights()
    GU, DN = _config1_t64()
    x0 = gen.activations(M, H1, seed=1300 + M)
    nw = gen.f32_to_bf16(np.random.default_rng(M + 2).uniform(0.5, 1.5, H1).astype(np.float32))
    x = g.dev(x0)
    ops.mlp_decode(x, g.dev(nw), 1e-6, GU, DN)
    rows = np.unique(np.linspace(0, M - 1, 4).astype(int))
    xr = np.ascontiguousarray(x0[rows])
    h = orc.silu_mul(gen.f32_to_bf16(_t64_arith(M, 2 * I1, H1)(orc.rmsnorm(xr, nw, 1e-6), *gu_w)))
    y = _t64_arith(M, H1, I1)(h, *dn_w)
    gen.check_bf16(g.host(x)[rows], y + gen.bf16_to_f32(xr), 1e-2, M)


@pytest.mark.parametrize("M", [17, 32, 33, 64, 65, 128, 129, 300])
@pytest.mark.parametrize("N,K", [(200, 512), (1024, 2048)])
def test_gemm_t64_rows(M, N, K):
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=M + N + K)
    A = gen.activations(M, K, seed=M)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    out = g.host(ops.gemm_t64(g.dev(A), T))
    gen.check_bf16(out, _t64_semantics(M)(A, wq, s, b), 1e-2, (M, N, K))


@pytest.mark.parametrize("M,mode", [(40, 1), (128, 2), (260, 1)])
def test_gemm_t64_big_modes(M, mode):
    g, ops = _gu(), _ops()
    N, K = 320, 1024
    codes, wq, s, b = gen.qlinear(N, K, seed=M + mode)
    A = gen.activations(M, K, seed=M + 5)
    C0 = gen.activations(M, N, seed=M + 6)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    out = g.host(ops.gemm_t64(g.dev(A), T, g.dev(C0) if mode == 1 else None, mode=mode))
    Y = _t64_semantics(M)(A, wq, s, b)
    gen.check_out(out, Y if mode == 2 else Y + gen.bf16_to_f32(C0), 1e-2, (M, mode), fp32=mode == 2)


@pytest.mark.parametrize("M", [32, 128])
def test_gemm_t64_decode_mlp_sampled(M):
    """BASELINE config 1 shapes on T64 weights (oracle on 8 sampled rows)."""
    g, ops = _gu(), _ops()
    for (N, K, seed) in [(34816, 5120, 23), (5120, 17408, 24)]:
        codes, wq, s, b = gen.qlinear(N, K, seed=seed)
        A = gen.activations(M, K, seed=seed + M)
        out = g.host(ops.gemm_t64(g.dev(A), ops.pack_t64(g.qlinear(wq, s, b))))
        rows = np.unique(np.linspace(0, M - 1, 8).astype(int))
        gen.check_bf16(out[rows], _t64_semantics(M)(A[rows], wq, s, b), 1e-2, (M, N, K))


def test_gemm_t64_config2_sampled():
    """BASELINE config 2 (M=4096, K=5120, N=17408) on T64 weights; oracle on 16 sampled rows."""
    g, ops = _gu(), _ops()
    M, N, K = 4096, 17408, 5120
    codes, wq, s, b = gen.qlinear(N, K, seed=33)
    A = gen.activations(M, K, seed=34, row_scale=True)
    out = g.host(ops.gemm_t64(g.dev(A), ops.pack_t64(g.qlinear(wq, s, b))))
    rows = np.linspace(0, M - 1, 16).astype(int)
    gen.check_bf16(out[rows], orc.qmm(A[rows], wq, s, b), 1e-2, "config 2")


def test_split_k_is_deterministic():
    """K-split T64 GEMMs (fp32 partials, then a reduce in split order) give identical bits on repeated calls and match
    the oracle on sampled rows, at the decode MLP's split shapes."""
    from inferd_amd._lib import lib
    g, ops = _gu(), _ops()
    shapes = [(1, 5120, 17408), (8, 34816, 5120), (32, 5120, 17408), (128, 5120, 17408)]
    assert all(lib().ifd_gemm_t64_workspace(M, N, K) > 0 for M, N, K in shapes)  # all of them split K
    for M, N, K in shapes:
        codes, wq, s, b = gen.qlinear(N, K, seed=M + 3)
        T = ops.pack_t64(g.qlinear(wq, s, b))
        A = g.dev(gen.activations(M, K, seed=M + 4))
        outs = [g.host(ops.gemm_t64(A, T)) for _ in range(3)]
        torch.cuda.synchronize()
        assert all(np.array_equal(outs[0], o) for o in outs[1:]), (M, N, K)
        rows = np.arange(0, M, max(1, M // 4))
        Y = _t64_semantics(M)(np.ascontiguousarray(g.host(A)[rows]), wq, s, b)
        gen.check_bf16(outs[0][rows], Y, 1e-2, (M, N, K))


def _multi_linears(Ns, K, seed):
    g, ops = _gu(), _ops()
    ws = [gen.qlinear(N, K, seed=seed + i)[1:] for i, N in enumerate(Ns)]
    return ws, [ops.pack_t64(g.qlinear(*w)) for w in ws]


@pytest.mark.parametrize("M", [1, 8, 9, 16])
def test_gemm_t64_multi_matches_oracle(M):
    """Several linears sharing A in one decode launch (the attention projections' q/k/v/o widths, and 198- and
    97-wide ones that end inside a band and a 4-column quad, padding their blocks with dead bands): each output
    against the oracle, over a K split planned for their concatenated width (in-kernel fixup)."""
    import ctypes
    from inferd_amd._lib import lib
    g, ops = _gu(), _ops()
    Ns, K = [5120, 1024, 198, 4096, 97], 5120
    assert lib().ifd_gemm_t64_multi_workspace(M, len(Ns), (ctypes.c_int * len(Ns))(*Ns), K) > 0
    ws, Ts = _multi_linears(Ns, K, 40 + M)
    A = gen.activations(M, K, seed=M + 41)
    outs = [g.host(o) for o in ops.gemm_t64_multi(g.dev(A), Ts)]
    for (wq, s, b), out, N in zip(ws, outs, Ns):
        assert out.shape == (M, N)
        gen.check_bf16(out, orc.qmv(A, wq, s, b), 1e-2, (M, N, K))


@pytest.mark.parametrize("mode", [1, 2])
def test_gemm_t64_multi_modes(mode):
    """Residual add (mode 1) and fp32 out (mode 2) into strided views of wider buffers, eight linears (the most one
    launch takes) with no K split (K = 512) and with one (K = 8192)."""
    g, ops = _gu(), _ops()
    M = 5
    for K, Ns in [(512, [128, 256, 32, 640, 128, 96, 384, 128]), (8192, [512, 1536, 256])]:
        ws, Ts = _multi_linears(Ns, K, 60 + K)
        A = gen.activations(M, K, seed=K)
        C0 = [gen.activations(M, N, seed=N + i) for i, N in enumerate(Ns)]
        dt = torch.float32 if mode == 2 else torch.bfloat16
        wide = [torch.zeros((M, N + 40), dtype=dt, device="cuda") for N in Ns]
        if mode == 1:
            for w, c in zip(wide, C0):
                w[:, : c.shape[1]] = g.dev(c)
        ops.gemm_t64_multi(g.dev(A), Ts, outs=[w[:, :N] for w, N in zip(wide, Ns)], mode=mode)
        for (wq, s, b), w, c, N in zip(ws, wide, C0, Ns):
            got = g.host(w)
            Y = orc.qmv(A, wq, s, b)
            gen.check_out(got[:, :N], Y if mode == 2 else Y + gen.bf16_to_f32(c), 1e-2, (mode, K, N), fp32=mode == 2)
            assert not got[:, N:].any(), "stores past a linear's N"


def test_gemm_t64_multi_repeats_and_matches_single_calls():
    """The fixup's counters return to zero: repeated launches give identical bits, and each output stays within the
    bar of the single-linear call (their K splits differ, so the sums' order does too)."""
    g, ops = _gu(), _ops()
    Ns, K, M = [5120, 5120, 5120, 5120], 5120, 1
    _, Ts = _multi_linears(Ns, K, 90)
    A = g.dev(gen.activations(M, K, seed=91))
    runs = [[g.host(o) for o in ops.gemm_t64_multi(A, Ts)] for _ in range(3)]
    assert all(np.array_equal(a, b) for r in runs[1:] for a, b in zip(runs[0], r))
    for T, out in zip(Ts, runs[0]):
        gen.check_bf16(out, gen.bf16_to_f32(g.host(ops.gemm_t64(A, T))), 1e-2, "multi vs single")
    # one linear whose width is whole 128-column blocks: the same plan and sums as the single call, bit for bit
    for M in (1, 7, 16):
        Am = g.dev(gen.activations(M, K, seed=92 + M))
        one = g.host(ops.gemm_t64_multi(Am, Ts[:1])[0])
        assert np.array_equal(one, g.host(ops.gemm_t64(Am, Ts[0]))), M


@pytest.mark.parametrize("M,N,K,mode", [
    (32, 34816, 5120, 1),   # decode gate_up, 32-row tiles two blocks per CU: ~5 pieces per tile
    (64, 23040, 1024, 2),   # 90 tiles (the fewest stream-K takes), runs of ~6 groups: ~4 pieces per tile
    (128, 22048, 2048, 0),  # 689 bands: the last tile has one live band (clamped loads, no stores past N)
    (65, 34816, 512, 1),    # 65 rows in one 128-row tile (63 past M); runs of ~4 groups
    (200, 22528, 1024, 2),  # two M tiles per column tile
    (300, 34816, 512, 0),   # 3 x 136 tiles > CUs: every run is one whole tile (no pieces)
    (128, 5120, 17408, 1),  # decode down at M = 128: 20 tiles, each cut into ~13 pieces; residual add in the fixup
    (100, 2048, 8192, 2),   # 8 tiles of one 128-row M tile (~32 pieces each), fp32 out
])
def test_gemm_t64_stream_k(M, N, K, mode):
    """The stream-K kernel (16 < M below the prefill tiles, tiles for at least a third of the CUs, or any tile count at
    64 < M <= 128) against the oracle on sampled rows, in every store mode, at shapes whose runs cross tile boundaries,
    cut a tile into several or many pieces or cover whole tiles; a second call on the same workspace gives the same
    bits (the fixup sums the pieces in unit order) and leaves the counter header zero."""
    from inferd_amd._lib import lib
    g, ops = _gu(), _ops()
    assert lib().ifd_gemm_t64_workspace(M, N, K) > 0
    codes, wq, s, b = gen.qlinear(N, K, seed=M + N + mode)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    A = gen.activations(M, K, seed=M + 9)
    C0 = gen.activations(M, N, seed=M + 10)
    outs = []
    for _ in range(2):
        C = g.dev(C0) if mode == 1 else None
        outs.append(g.host(ops.gemm_t64(g.dev(A), T, C, mode=mode)))
    torch.cuda.synchronize()
    assert np.array_equal(outs[0], outs[1]), (M, N, K, mode)
    hdr = g.host(ops.workspace(4096, "cuda")[:4096])
    assert not hdr.any(), "counters left non-zero"
    rows = np.unique(np.linspace(0, M - 1, 8).astype(int))
    Y = orc.qmm(np.ascontiguousarray(A[rows]), wq, s, b)
    out = outs[0][rows]
    gen.check_out(out, Y + gen.bf16_to_f32(C0[rows]) if mode == 1 else Y, 1e-2, (M, N, K, mode), fp32=mode == 2)


@pytest.mark.parametrize("M,N,K,split", [
    (1, 1024, 2048, True),     # decode kernel, K split: SwiGLU in the split-K reduction
    (4, 1024, 256, False),     # decode kernel, no split: bf16 product in the workspace, then silu_mul
    (16, 2048, 1024, True),
    (40, 1024, 2048, True),    # stream-K kernel: SwiGLU in its fixup
    (40, 34816, 5120, True),
    (128, 1024, 2048, True),
    (128, 8192, 2048, True),
    (1024, 8192, 256, False),  # prefill kernel, then silu_mul
])
def test_gemm_t64_swiglu_matches_unfused(M, N, K, split):
    """The fused gate/up projection against gemm_t64 (mode 0) + silu_mul: the same bits from the decode and prefill
    kernels, within one bf16 step from the stream-K kernel (whose fused tiles split K elsewhere). Against the oracle,
    as a chain: the bf16 product is within the GEMM bar, and the fused h within one bf16 step of the oracle's SwiGLU
    of that product (expf may differ in its last ulp; a product of two rounded values is no place for a max-error /
    RMS bar, whose tail a single gate rounding flip can exceed)."""
    g, ops = _gu(), _ops()
    from inferd_amd._lib import lib
    codes, wq, s, b = gen.qlinear(N, K, seed=M + N)
    A = g.dev(gen.activations(M, K, seed=M + 1))
    T = ops.pack_t64(g.qlinear(wq, s, b))
    if M <= 16:
        assert (lib().ifd_gemm_t64_workspace(M, N, K) > 0) == split
    fused = g.host(ops.gemm_t64_swiglu(A, T))
    gu = g.host(ops.gemm_t64(A, T))
    unfused = g.host(ops.silu_mul(g.dev(gu)))
    if M <= 16 or M >= 1024:
        assert np.array_equal(fused, unfused), (M, N, K)
        h, hr = gen.bf16_to_f32(fused), gen.bf16_to_f32(orc.silu_mul(gu))
        assert np.all(np.abs(h - hr) <= 2 ** -7 * np.abs(hr) + 1e-30)
        assert np.mean(h == hr) > 0.99
    else:
        # stream-K: the fused tiles pair gate and up bands, so a column's K pieces (and the fp32 rounding of its sum)
        # differ from the plain GEMM's. Every fused h is the SwiGLU of the unfused product with its gate and up each
        # at most one bf16 ulp away, with one bf16 step of slack for expf's last ulp and 1e-4 RMS(h) absolute for
        # sums that cancel to far below their terms (there the fp32 summation order shows in the bf16 bits)
        hf, I = gen.bf16_to_f32(fused), N // 2
        tol = 1e-4 * np.sqrt(np.mean(gen.bf16_to_f32(unfused) ** 2))
        ok = np.zeros(hf.shape, dtype=bool)
        for dg in (-1, 0, 1):
            for du in (-1, 0, 1):
                nudged = gu.astype(np.int32)
                nudged[:, :I] += dg
                nudged[:, I:] += du
                cand = gen.bf16_to_f32(orc.silu_mul(nudged.astype(np.uint16)))
                ok |= np.abs(hf - cand) <= 2 ** -7 * np.abs(cand) + tol
        assert ok.all(), (M, N, K, np.argwhere(~ok)[:4])
        assert np.mean(fused == unfused) > 0.99
    rows = np.unique(np.linspace(0, M - 1, 8).astype(int))
    Y = _t64_semantics(M)(np.ascontiguousarray(g.host(A)[rows]), wq, s, b)
    gen.check_bf16(gu[rows], Y, 1e-2, (M, N, K))


def test_gemm_t64_swiglu_strided_output():
    """h written into a wider buffer (row stride ldh > N / 2) leaves the padding columns untouched."""
    g, ops = _gu(), _ops()
    M, N, K = 8, 512, 1024
    codes, wq, s, b = gen.qlinear(N, K, seed=5)
    A = g.dev(gen.activations(M, K, seed=6))
    T = ops.pack_t64(g.qlinear(wq, s, b))
    wide = torch.full((M, N // 2 + 8), -1.0, dtype=torch.bfloat16, device="cuda")
    ops.gemm_t64_swiglu(A, T, out=wide[:, : N // 2])
    ref = g.host(ops.silu_mul(ops.gemm_t64(A, T)))
    out = g.host(wide)
    assert np.array_equal(out[:, : N // 2], ref)
    assert np.all(gen.bf16_to_f32(out[:, N // 2:]) == -1.0)


@pytest.mark.parametrize("M,N,K", [(37, 200, 512), (128, 384, 1024), (300, 256, 5120), (64, 512, 17408),
                                   (200, 640, 17408)])
def test_gemm_t64_w4a8(M, N, K):
    """W4A8 on T64 weights (int8 MFMA, per-token activations) against the oracle's w4a8_gemm semantics, all store
    modes. M <= 64 runs the K-split kernel (K = 17408: the bias part per split, fp32 partials); M > 64 the stream-K
    kernel (200 x 640 x 17408: 2 x 3 tiles of 136 group pairs, every tile cut into about 40 pieces)."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=M + 7)
    A = gen.activations(M, K, seed=M + 8)
    U, XS = orc.a8_quant(A, True)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    Y = orc.w4a8(U, XS, wq, s, b)
    C0 = gen.activations(M, N, seed=M + 9)
    for mode in (0, 1, 2):
        C = g.dev(C0) if mode == 1 else None
        out = g.host(ops.gemm_t64_w4a8(g.dev(U), g.dev(XS), T, C, mode=mode))
        # the same int8 inputs on both sides: the bars are the output rounding's (bf16 1e-2 net, fp32 1e-4)
        gen.check_out(out, Y + gen.bf16_to_f32(C0) if mode == 1 else Y, 1e-4 if mode == 2 else 1e-2,
                      (M, N, K, mode), fp32=mode == 2)


@pytest.mark.parametrize("M", [1, 3, 8, 16, 17, 32, 33, 64, 65, 128, 255])
@pytest.mark.parametrize("N,K", [(384, 1024), (320, 17408)])
def test_gemm_t64_w4a8_per_group(M, N, K):
    """The reference's default W4A8 route (per-(row, 64-group) int8 activations, w4a8.metal:24-98) on T64 weights:
    the decode GEMV up to 16 rows, the affine K-split kernel above (xq as bf16 integers, every group scaled by its
    row's sx), against the oracle's w4a8 on the same int8 inputs in all store modes. Both sides compute the same
    exact integer products, so the bars are the output rounding's: 1e-2 net for bf16, 1e-4 for fp32."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=M + 17, bias="free")
    A = gen.activations(M, K, seed=M + 18)
    U, XS = orc.a8_quant(A, False)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    Y = orc.w4a8(U, XS, wq, s, b)
    C0 = gen.activations(M, N, seed=M + 19)
    for mode in (0, 1, 2):
        C = g.dev(C0) if mode == 1 else None
        out = g.host(ops.gemm_t64_w4a8(g.dev(U), g.dev(XS), T, C, mode=mode, per_token=False))
        ref = Y + gen.bf16_to_f32(C0) if mode == 1 else Y
        gen.check_out(out, ref, 1e-4 if mode == 2 else 1e-2, (M, N, K, mode, "per group"), fp32=mode == 2)


@pytest.mark.parametrize("M", [8, 32, 128])
@pytest.mark.parametrize("N,K", [(34816, 5120), (5120, 17408)])
def test_gemm_t64_w4a8_per_group_config1(M, N, K):
    """Per-group W4A8 on T64 at config 1's shapes (gate_up, down), the GPU's own quantization bit-exact against the
    oracle's; 768 sampled columns against the oracle's w4a8."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=M + N)
    A = gen.activations(M, K, seed=M + 3)
    U, XS = ops.a8_quant(g.dev(A), False)
    Uh, XSh = orc.a8_quant(A, False)
    assert np.array_equal(g.host(U), Uh) and np.array_equal(g.host(XS), XSh)
    out = g.host(ops.gemm_t64_w4a8(U, XS, ops.pack_t64(g.qlinear(wq, s, b)), per_token=False))
    cols = np.linspace(0, N - 1, 768).astype(int)
    Y = orc.w4a8(Uh, XSh, wq[cols], s[cols], b[cols])
    gen.check_bf16(out[:, cols], Y, 1e-2, (M, N, K, "per group, sampled columns"))


def test_gemm_t64_w4a8_config3_sampled():
    """BASELINE config 3 (M=2048, K=N=5120, per-token int8) on T64 weights; oracle on 16 sampled rows."""
    g, ops = _gu(), _ops()
    M, N, K = 2048, 5120, 5120
    codes, wq, s, b = gen.qlinear(N, K, seed=60)
    A = gen.activations(M, K, seed=61)
    U, XS = ops.a8_quant(g.dev(A), True)
    out = g.host(ops.gemm_t64_w4a8(U, XS, ops.pack_t64(g.qlinear(wq, s, b))))
    rows = np.linspace(0, M - 1, 16).astype(int)
    Ur, XSr = orc.a8_quant(A[rows], True)
    assert np.array_equal(g.host(U)[rows], Ur)
    gen.check_bf16(out[rows], orc.w4a8(Ur, XSr, wq, s, b), 2e-2, "config 3")


def test_gemm_t64_w4a8_tail_split():
    """A tile count just past a whole round (9 x 30 = 270 tiles): one whole tile per block, the last 14 tiles split
    stream-K over all blocks (16 pieces each, summed by the fixup); sampled rows against the oracle, all three store
    modes."""
    from inferd_amd._lib import lib
    g, ops = _gu(), _ops()
    M, N, K = 1152, 7680, 1024
    codes, wq, s, b = gen.qlinear(N, K, seed=70)
    A = gen.activations(M, K, seed=71)
    U, XS = ops.a8_quant(g.dev(A), True)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    rows = np.linspace(0, M - 1, 24).astype(int)
    Ur, XSr = orc.a8_quant(A[rows], True)
    Y = orc.w4a8(Ur, XSr, wq, s, b)
    C0 = gen.activations(M, N, seed=72)
    assert lib().ifd_gemm_t64_w4a8_workspace(M, N, K) > 4096 + 2 * M * 48 * 2  # tail partials present
    for mode in (0, 1, 2):
        out = g.host(ops.gemm_t64_w4a8(U, XS, T, g.dev(C0) if mode == 1 else None, mode=mode))[rows]
        ref = Y + gen.bf16_to_f32(C0[rows]) if mode == 1 else Y
        gen.check_out(out, ref, 1e-4 if mode == 2 else 1e-2, mode, fp32=mode == 2)


@pytest.mark.parametrize("M,N,K", [(2560, 6656, 512), (2048, 4096, 256), (1280, 5120, 256)])
def test_gemm_t64_w4a8_stream_k_plans(M, N, K):
    """The W4A8 stream-K plans past M = 64, sampled rows against the oracle in all three store modes:
    20 x 26 = 520 tiles (two whole tiles per block, the first stored in the middle of the run, then 8 stream-K tiles);
    16 x 16 = 256 tiles (one whole tile per block, no pieces, no fixup); 10 x 20 = 200 tiles of four groups
    (stream-K only: runs of three or four units, some of them a whole tile)."""
    g, ops = _gu(), _ops()
    codes, wq, s, b = gen.qlinear(N, K, seed=M + 90)
    A = gen.activations(M, K, seed=M + 91)
    U, XS = ops.a8_quant(g.dev(A), True)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    rows = np.unique(np.concatenate([np.linspace(0, M - 1, 24).astype(int), [127, 128, M - 1]]))
    Ur, XSr = orc.a8_quant(A[rows], True)
    Y = orc.w4a8(Ur, XSr, wq, s, b)
    C0 = gen.activations(M, N, seed=M + 92)
    for mode in (0, 1, 2):
        out = g.host(ops.gemm_t64_w4a8(U, XS, T, g.dev(C0) if mode == 1 else None, mode=mode))[rows]
        ref = Y + gen.bf16_to_f32(C0[rows]) if mode == 1 else Y
        gen.check_out(out, ref, 1e-4 if mode == 2 else 1e-2, (M, N, K, mode), fp32=mode == 2)


def test_gemm_t64_prefill_tiles_with_tail():
    """A prefill shape on the 256-row-tile kernel whose last round holds 4 tiles (5 x 52 = 260): those run K-split
    in a second launch. Sampled rows against the qmm oracle, all three store modes."""
    g, ops = _gu(), _ops()
    M, N, K = 1280, 13312, 1024
    codes, wq, s, b = gen.qlinear(N, K, seed=80)
    A = gen.activations(M, K, seed=81, row_scale=True)
    T = ops.pack_t64(g.qlinear(wq, s, b))
    rows = np.linspace(0, M - 1, 24).astype(int)
    Y = orc.qmm(np.ascontiguousarray(A[rows]), wq, s, b)
    C0 = gen.activations(M, N, seed=82)
    for mode in (0, 1, 2):
        out = g.host(ops.gemm_t64(g.dev(A), T, g.dev(C0) if mode == 1 else None, mode=mode))[rows]
        ref = Y + gen.bf16_to_f32(C0[rows]) if mode == 1 else Y
        gen.check_out(out, ref, 1e-2, mode, fp32=mode == 2)


def test_gemm_t64_swiglu_prefill_tiles():
    """The fused gate/up entry on a prefill shape (256-row tiles, 4 x 64 = 256 tiles): bit-identical to gemm_t64 +
    silu_mul."""
    g, ops = _gu(), _ops()
    M, N, K = 1024, 16384, 256
    codes, wq, s, b = gen.qlinear(N, K, seed=83)
    A = g.dev(gen.activations(M, K, seed=84))
    T = ops.pack_t64(g.qlinear(wq, s, b))
    assert np.array_equal(g.host(ops.gemm_t64_swiglu(A, T)), g.host(ops.silu_mul(ops.gemm_t64(A, T))))


# ---- the dense decode MLP block -----------------------------------------------------------------------------------
@pytest.mark.parametrize("M", [1, 8, 32, 128])
def test_mlp_decode_matches_its_sequence_at_config1(M):
    """BASELINE config 1's layer (H = 5120, I = 17408): the fused block is bit-identical to rmsnorm ->
    gemm_t64_swiglu -> gemm_t64 (mode 1) on the same inputs."""
    g, ops = _gu(), _ops()
    H, I = 5120, 17408
    _, wg, sg_, bg = gen.qlinear(2 * I, H, seed=700 + M)
    _, wd, sd, bd = gen.qlinear(H, I, seed=800 + M)
    GU, DN = ops.pack_t64(g.qlinear(wg, sg_, bg)), ops.pack_t64(g.qlinear(wd, sd, bd))
    x0 = gen.activations(M, H, seed=900 + M)
    nw = gen.f32_to_bf16(np.random.default_rng(M).uniform(0.5, 1.5, H).astype(np.float32))
    x = g.dev(x0)
    ops.mlp_decode(x, g.dev(nw), 1e-6, GU, DN)
    xs = g.dev(x0)
    h = ops.gemm_t64_swiglu(ops.rmsnorm(xs, g.dev(nw), 1e-6), GU)
    ops.gemm_t64(h, DN, xs, mode=1)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(x), g.host(xs))


@pytest.mark.parametrize("M", [1, 9, 40, 128])
def test_mlp_decode_matches_oracle(M):
    """x += down(SwiGLU(gate_up(rmsnorm(x)))) against the oracle's composition. At these shapes (too few column tiles
    for the stream-K kernel) the T64 GEMMs keep the decode GEMV's affine arithmetic up to 64 rows (32- and 64-row
    tiles) and dequantize above; two chained GEMMs would compound the difference between the two forms."""
    g, ops = _gu(), _ops()
    H, I = 1024, 2048
    _, wg, sg_, bg = gen.qlinear(2 * I, H, seed=710 + M)
    _, wd, sd, bd = gen.qlinear(H, I, seed=810 + M)
    GU, DN = ops.pack_t64(g.qlinear(wg, sg_, bg)), ops.pack_t64(g.qlinear(wd, sd, bd))
    x0 = gen.activations(M, H, seed=910 + M)
    nw = gen.f32_to_bf16(np.random.default_rng(M).uniform(0.5, 1.5, H).astype(np.float32))
    x = g.dev(x0)
    ops.mlp_decode(x, g.dev(nw), 1e-6, GU, DN)
    xn = orc.rmsnorm(x0, nw, 1e-6)
    sem = orc.qmv if M <= 64 else orc.qmm
    h = orc.silu_mul(gen.f32_to_bf16(sem(xn, wg, sg_, bg)))
    y = sem(h, wd, sd, bd)
    gen.check_bf16(g.host(x), y + gen.bf16_to_f32(x0), 1e-2, M)
