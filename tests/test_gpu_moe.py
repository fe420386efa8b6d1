"""GPU parity of the MoE path (router, routing, dispatch, gathered expert GEMM, combine, one-shot FFN) against the
CPU oracle, through the C ABI. Indices and permutations bit-exact; floats within 1e-2 RMS.

Routing is compared on the same logits (the GPU's): router logits from two different summation orders may
legitimately break a near-tie differently, so the end-to-end FFN check runs the oracle on the GPU's routing.
"""
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


def experts(E, N, K, seed):
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, size=(E, N, K), dtype=np.uint8)
    wq = gen.pack_codes(codes.reshape(E * N, K)).reshape(E, N, K // 8)
    s = gen.f32_to_bf16(rng.uniform(0.005, 0.02, size=(E, N, K // 64)).astype(np.float32))
    b = gen.f32_to_bf16(-8.0 * gen.bf16_to_f32(s))
    return wq, s, b


def router(E1, H, seed):
    rng = np.random.default_rng(seed)
    return gen.f32_to_bf16((rng.standard_normal((E1, H)) * 0.02).astype(np.float32))


@pytest.mark.parametrize("T,out_bf16", [(16, False), (128, True), (70, True), (300, False), (2048, True)])
def test_router_logits(T, out_bf16):
    g, ops = _gu(), _ops()
    H, E1 = 2048, 513
    x = gen.activations(T, H, seed=T)
    W = router(E1, H, seed=1)
    got = g.host(ops.moe_router_logits(g.dev(x), g.dev(W), out_bf16))
    ref = orc.gemm_bf16(x, W)
    gen.check_out(got, ref, 1e-2, T, fp32=not out_bf16)


@pytest.mark.parametrize("bf,shared_gate", [(False, True), (True, True), (True, False)])
def test_route_bit_exact(bf, shared_gate):
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(2)
    T, E, k = 300, 512, 10
    l = (rng.standard_normal((T, E + 1)) * 0.9).astype(np.float32)
    if bf:
        l = gen.f32_to_bf16(l)
        l[:5, :40] = l[:5, 40:80]  # duplicated logits: exact ties, lowest index must win
    idx, wt, sg = ops.moe_route(g.dev(l), E, k, shared_gate=shared_gate)
    ri, rw, rs = orc.moe_route(l, E, k, shared_gate=shared_gate)
    assert np.array_equal(g.host(idx), ri)
    assert np.allclose(g.host(wt), rw, rtol=1e-5, atol=1e-7)
    assert np.allclose(g.host(sg), rs, rtol=1e-5)


@pytest.mark.parametrize("T,E", [(16, 512), (128, 512), (2048, 512), (1, 8), (37, 64), (25, 512), (26, 512),
                                 (409, 512), (410, 512)])
def test_dispatch_bit_exact(T, E):
    """Up to 256 routed rows (T = 1, 16, 25 here) the three passes run as one block; T = 26 (260 rows) is the first
    count past it. T = 409 / 410: 16 chunks of 256 rows, the last one full and partial."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(T)
    k = min(10, E)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    offsets, perm, inv, tiles, ntiles, mt = ops.moe_dispatch(g.dev(idx), E)
    ro, rp, ri = orc.moe_dispatch(idx, E)
    assert np.array_equal(g.host(offsets), ro)
    assert np.array_equal(g.host(perm), rp)
    assert np.array_equal(g.host(inv), ri)
    # tile schedule: every 32-row tile of every non-empty segment, in expert order
    nt = int(g.host(ntiles)[0])
    want = [(e, q) for e in range(E) for q in range(ro[e], ro[e + 1], 32)]
    assert nt == len(want) <= mt
    assert [tuple(t) for t in g.host(tiles)[:nt].tolist()] == want


@pytest.mark.parametrize("T,E,silu", [(16, 64, True), (40, 16, False), (200, 32, True)])
def test_gather_qmm(T, E, silu):
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(E + T)
    H, I, k = 256, 128, 4
    x = gen.activations(T, H, seed=3)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    disp = ops.moe_dispatch(g.dev(idx), E)
    ro, rp, ri = orc.moe_dispatch(idx, E)
    if silu:
        # the product against the oracle; the fused SwiGLU bit-identical to silu_mul of that product
        wq, s, b = experts(E, 2 * I, H, seed=4)
        W = g.moew(wq, s, b)
        got = g.host(ops.moe_gather_qmm(g.dev(x), disp[1], k, disp, W, silu=True))
        prod = ops.moe_gather_qmm(g.dev(x), disp[1], k, disp, W, silu=False)
        assert np.array_equal(got, g.host(ops.silu_mul(prod)))
        got, ref = g.host(prod), orc.moe_gather_qmm(x, rp, k, ro, wq, s, b, 2 * I, H)
    else:
        wq, s, b = experts(E, H, H, seed=5)
        xs = g.host(ops.moe_gather(g.dev(x), disp[1], k))
        assert np.array_equal(xs, x[rp // k])
        got = g.host(ops.moe_gather_qmm(g.dev(xs), None, 1, disp, g.moew(wq, s, b), silu=False))
        ref = orc.moe_gather_qmm(xs, None, 1, ro, wq, s, b, H, H)
    gen.check_bf16(got, ref, 1e-2, (T, E, silu))


@pytest.mark.parametrize("silu", [False, True])
def test_gather_qmm_8bit(silu):
    """8-bit expert stacks on the gathered GEMM (the reference's gqmm at W.bits = 8, mlx_gqmm_b8): each expert's
    sorted rows against the oracle's 8-bit qmm (bf16(s q + b) dequant, fp32 sums), 1e-2 RMS; the fused SwiGLU
    bit-identical to silu_mul of that product."""
    g, ops = _gu(), _ops()
    from inferd_amd.ops import MoeW
    rng = np.random.default_rng(77)
    T, E, H, I, k = 40, 16, 512, 128, 4
    N, K = (2 * I, H) if silu else (H, H)
    layers = [gen.qlinear8(N, K, seed=300 + e, bias="free") for e in range(E)]
    wq = np.stack([q[1] for q in layers]); s = np.stack([q[2] for q in layers]); b = np.stack([q[3] for q in layers])
    W = MoeW(g.dev(wq), g.dev(s), g.dev(b), E, N, K, bits=8)
    x = gen.activations(T, K, seed=78)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    disp = ops.moe_dispatch(g.dev(idx), E)
    ro, rp, ri = orc.moe_dispatch(idx, E)
    prod = ops.moe_gather_qmm(g.dev(x), disp[1], k, disp, W, silu=False)
    if silu:
        got = g.host(ops.moe_gather_qmm(g.dev(x), disp[1], k, disp, W, silu=True))
        assert np.array_equal(got, g.host(ops.silu_mul(prod)))
    ref = np.zeros((T * k, N), np.float32)
    for e in range(E):
        q0, q1 = int(ro[e]), int(ro[e + 1])
        if q1 > q0:
            ref[q0:q1] = orc.qmm(np.ascontiguousarray(x[rp[q0:q1] // k]), wq[e], s[e], b[e], bits=8)
    gen.check_bf16(g.host(prod), ref, 1e-2, ("8-bit stacks", silu))


@pytest.mark.parametrize("k,T", [(10, 50), (1, 50), (16, 50), (20, 50), (10, 2100)])
def test_combine(k, T):
    """Up to 16 picks on at most 512 blocks a thread loads every pick's row before summing; past 16 picks (k = 20) or
    on more blocks (T = 2100 tokens of 512 columns: 525 blocks) it loops."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(6 + k)
    H = 512
    yd = gen.f32_to_bf16(rng.standard_normal((T * k, H)).astype(np.float32))
    ys = gen.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    wt = rng.uniform(0, 1, (T, k)).astype(np.float32)
    sg = rng.uniform(0, 1, T).astype(np.float32)
    inv = rng.permutation(T * k).astype(np.int32)
    x0 = gen.f32_to_bf16(rng.standard_normal((T, H)).astype(np.float32))
    for assign in (True, False):
        out = g.dev(x0)
        ops.moe_combine(out, g.dev(yd), g.dev(wt), g.dev(ys), g.dev(sg), g.dev(inv), k, assign)
        ref = orc.moe_combine(x0, yd, wt, ys, sg, inv, k, assign)
        gen.check_bf16(g.host(out), ref, 1e-2, assign, ref_is_bf16=True)


def _ffn_case(T, E, H, I, k, shared_gate, seed):
    """The one-shot FFN against the same pipeline run stage by stage through the C ABI (same bits), each stage
    against the oracle on the GPU's own inputs to it (one rounding per check, BASELINE's bar), and the whole against
    the oracle's composition (bf16 stages on both sides: one- and two-step shares bounded, every other element held
    to the bar)."""
    g, ops = _gu(), _ops()
    egu = experts(E, 2 * I, H, seed=seed)
    edn = experts(E, H, I, seed=seed + 1)
    sgu = experts(1, 2 * I, H, seed=seed + 2)
    sdn = experts(1, H, I, seed=seed + 3)
    R = router(E + (1 if shared_gate else 0), H, seed=seed + 4)
    xn = gen.activations(T, H, seed=seed + 5)
    sgu_h, sdn_h = (sgu[0][0], sgu[1][0], sgu[2][0]), (sdn[0][0], sdn[1][0], sdn[2][0])
    shared = (g.qlinear(*sgu_h), g.qlinear(*sdn_h))
    xd, Rd, EGU, EDN = g.dev(xn), g.dev(R), g.moew(*egu), g.moew(*edn)
    out, idx, wt, sg = ops.moe_ffn(xd, Rd, EGU, EDN, k, shared=shared, shared_gate=shared_gate, logits_bf16=T >= 64)
    # the stages
    logits = ops.moe_router_logits(xd, Rd, out_bf16=T >= 64)
    idx2, wt2, sg2 = ops.moe_route(logits, E, k, shared_gate=shared_gate)
    disp = ops.moe_dispatch(idx2, E)
    eact = ops.moe_gather_qmm(xd, disp[1], k, disp, EGU, silu=True)
    ydn = ops.moe_gather_qmm(eact, None, 1, disp, EDN, silu=False)
    sh_gu = ops.gemm(xd, shared[0])
    sh_act = ops.silu_mul(sh_gu)
    ys = ops.gemm(sh_act, shared[1])
    out2 = ops.moe_combine(torch.zeros_like(out), ydn, wt2, ys, sg2, disp[2], k, True)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(out), g.host(out2)), "one-shot FFN differs from its stages"
    assert np.array_equal(g.host(idx), g.host(idx2)) and np.array_equal(g.host(wt), g.host(wt2))
    # routing on the GPU's own logits: bit-exact; dispatch: bit-exact
    ri, rw, rs = orc.moe_route(g.host(logits), E, k, shared_gate=shared_gate)
    assert np.array_equal(g.host(idx), ri)
    assert np.allclose(g.host(wt), rw, rtol=1e-5, atol=1e-7)
    ro, rp, rinv = orc.moe_dispatch(ri, E)
    assert np.array_equal(g.host(disp[0]), ro) and np.array_equal(g.host(disp[1]), rp)
    # each stage on the GPU's inputs to it. The gate/up product (one rounding) against the oracle's; the fused
    # SwiGLU output bit-identical to silu_mul of that product (SwiGLU of two bf16 values can move several steps when
    # one input rounds the other way, so it is held to the GPU's own product, not to the oracle's)
    gu_full = ops.moe_gather_qmm(xd, disp[1], k, disp, EGU, silu=False)
    assert np.array_equal(g.host(eact), g.host(ops.silu_mul(gu_full))), "fused SwiGLU differs from silu_mul"
    eact_h, ydn_h, ys_h, sh_act_h = g.host(eact), g.host(ydn), g.host(ys), g.host(sh_act)
    y_gu = orc.moe_gather_qmm(xn, rp, k, ro, *egu, 2 * I, H)
    gen.check_bf16(g.host(gu_full), y_gu, 1e-2, "gate/up")
    gen.check_bf16(ydn_h, orc.moe_gather_qmm(eact_h, None, 1, ro, *edn, H, I), 1e-2, "down")
    sem = orc.qmv if T <= 32 else orc.qmm  # the dense route's arithmetic: decode GEMV up to 32 rows
    gen.check_bf16(g.host(sh_gu), sem(xn, *sgu_h), 1e-2, "shared gate/up")
    gen.check_bf16(ys_h, sem(sh_act_h, *sdn_h), 1e-2, "shared down")
    comb = orc.moe_combine(np.zeros((T, H), np.uint16), ydn_h, rw, ys_h, rs, rinv, k, True)
    gen.check_bf16(g.host(out), comb, 1e-2, "combine", ref_is_bf16=True)
    # end to end against the oracle's own composition
    ref = orc.moe_experts(xn, ri, rw, rs, egu, edn, (sgu_h, sdn_h), I, shared_qmv=T <= 32)
    got = g.host(out)
    gen.check_bf16(got, ref, 1e-2, ("end to end", T, E, H, I, k), ref_is_bf16=True, composition=True)
    rms = gen.bf16_to_f32(ref).astype(np.float64)
    rel_rms = np.sqrt(np.mean((gen.bf16_to_f32(got) - rms) ** 2) / np.mean(rms ** 2))
    assert rel_rms < 1e-2, rel_rms


@pytest.mark.parametrize("T,shared_gate", [(16, True), (128, False)])
def test_moe_ffn_baseline_geometry(T, shared_gate):
    """BASELINE config 4 geometry: H=2048, E=512, top-10, I=512, plus a shared expert."""
    _ffn_case(T, 512, 2048, 512, 10, shared_gate, seed=80 + T)


def test_moe_ffn_t2048():
    """BASELINE config 4 at T=2048: within tolerance of the CPU reference (the north star's MoE bar)."""
    _ffn_case(2048, 512, 2048, 512, 10, False, seed=90)


def test_moe_ffn_small_odd():
    _ffn_case(5, 8, 128, 64, 2, True, seed=95)


# ---- decode MoE (T <= 8): router, routing + plan, gate/up + SwiGLU, down + combine -----------------------------------
def _decode_case(T, E, H, I, k, shared, shared_gate, seed, assign=True):
    g, ops = _gu(), _ops()
    egu = experts(E, 2 * I, H, seed=seed)
    edn = experts(E, H, I, seed=seed + 1)
    sgu = experts(1, 2 * I, H, seed=seed + 2)
    sdn = experts(1, H, I, seed=seed + 3)
    R = router(E + (1 if shared_gate else 0), H, seed=seed + 4)
    xn = gen.activations(T, H, seed=seed + 5)
    x0 = gen.activations(T, H, seed=seed + 6)
    sh = (g.qlinear(sgu[0][0], sgu[1][0], sgu[2][0]), g.qlinear(sdn[0][0], sdn[1][0], sdn[2][0])) if shared else None
    outs = []
    for _ in range(2):  # a second call on the same workspace: the combine counters were left at zero
        out, idx, wt, sg, logits = ops.moe_decode(g.dev(xn), g.dev(R), g.moew(*egu), g.moew(*edn), k, shared=sh,
                                                  shared_gate=shared_gate, out=g.dev(x0), assign=assign)
        torch.cuda.synchronize()
        outs.append(g.host(out))
    assert np.array_equal(outs[0], outs[1])
    # logits within tolerance of the oracle's router GEMM; routing bit-exact on the GPU's own logits
    lg = g.host(logits)
    assert gen.rel_err(lg, orc.gemm_bf16(xn, R)) < 1e-4
    ri, rw, rs = orc.moe_route(lg, E, k, shared_gate=shared_gate)
    assert np.array_equal(g.host(idx), ri)
    assert np.allclose(g.host(wt), rw, rtol=1e-5, atol=1e-7)
    assert np.allclose(g.host(sg), rs, rtol=1e-5)
    shw = ((sgu[0][0], sgu[1][0], sgu[2][0]), (sdn[0][0], sdn[1][0], sdn[2][0])) if shared else None
    ref = orc.moe_decode(xn, ri, rw, rs, egu, edn, shw, I, out=x0, assign=assign)
    got = outs[0]
    gen.check_bf16(got, ref, 1e-2, (T, E, H, I, k), ref_is_bf16=True, composition=True)
    r64 = gen.bf16_to_f32(ref).astype(np.float64)
    rel_rms = np.sqrt(np.mean((gen.bf16_to_f32(got) - r64) ** 2) / np.mean(r64 ** 2))
    assert rel_rms < 1e-2, (T, rel_rms)
    return ri


@pytest.mark.parametrize("T", [1, 2, 5, 8, 9, 10, 11, 12, 16])
def test_moe_decode_baseline_geometry(T):
    """BASELINE config 4's layer (H=2048, E=512, top-10, I=512, shared expert with its gate) at decode batch sizes,
    and beyond 8 tokens while T k < 128 (the reference's per-row expert GEMVs, moe_qmv4, at 90..120 routed rows), up to
    the kernel's 16."""
    _decode_case(T, 512, 2048, 512, 10, True, True, seed=120 + T)


@pytest.mark.parametrize("T,k,shared", [(3, 10, True), (12, 10, True), (17, 4, True), (31, 4, True), (40, 2, False),
                                          (100, 1, True)])
def test_moe_rows(T, k, shared):
    """The per-row expert products on the caller's routing (reference moe_qmv4 + moe_silu_mul + moe_combine, the route
    below 128 routed rows where the four-launch path does not apply), with the shared expert's rows given: 16 tokens
    per launch group, so T = 17 .. 100 cross group edges. Against the oracle's per-token decode arithmetic (the
    routed products in qmv4 form) with the same shared rows, assign and residual."""
    g, ops = _gu(), _ops()
    E, H, I, seed = 64, 1024, 256, 400 + T
    egu, edn = experts(E, 2 * I, H, seed=seed), experts(E, H, I, seed=seed + 1)
    rng = np.random.default_rng(seed)
    xn = gen.activations(T, H, seed=seed + 2)
    x0 = gen.activations(T, H, seed=seed + 3)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    wt = rng.random((T, k)).astype(np.float32)
    wt /= wt.sum(axis=1, keepdims=True)
    sg = rng.random(T).astype(np.float32) if shared else np.ones(T, np.float32)
    ys = gen.activations(T, H, seed=seed + 4) if shared else None
    W1, W2 = g.moew(*egu), g.moew(*edn)
    d = np.empty((T * k, H), np.uint16)
    for t in range(T):
        for j in range(k):
            e = idx[t, j]
            gu = gen.f32_to_bf16(orc.qmv(xn[t:t + 1], egu[0][e], egu[1][e], egu[2][e]))
            a = orc.silu_mul(gu)
            d[t * k + j] = gen.f32_to_bf16(orc.qmv(a, edn[0][e], edn[1][e], edn[2][e]))[0]
    ident = np.arange(T * k, dtype=np.int32)
    ref_rows = {asg: orc.moe_combine(x0, d, wt, ys, sg, ident, k, asg) for asg in (True, False)}
    for assign in (True, False):
        out = ops.moe_rows(g.dev(xn), g.dev(idx), g.dev(wt), g.dev(sg), W1, W2, g.dev(ys) if shared else None,
                           out=g.dev(x0), assign=assign)
        again = ops.moe_rows(g.dev(xn), g.dev(idx), g.dev(wt), g.dev(sg), W1, W2, g.dev(ys) if shared else None,
                             out=g.dev(x0), assign=assign)
        torch.cuda.synchronize()
        assert np.array_equal(g.host(out), g.host(again))
        # the oracle: each routed row (t, j) in the decode arithmetic, bf16 d_j, then the weighted combine with the
        # given shared rows (moe.metal:115-128), rows in (t, j) order
        gen.check_bf16(g.host(out), ref_rows[assign], 1e-2, (T, k, shared, assign), ref_is_bf16=True,
                       composition=True)


@pytest.mark.parametrize("T,k,shared", [(3, 10, True), (12, 10, True), (17, 4, False), (8, 16, True), (40, 2, True),
                                          (5, 10, "weights"), (16, 4, "weights")])
def test_moe_rows_t64(T, k, shared):
    """ifd_moe_rows_t64: the per-row route on the routed experts' T64 stacks, 16 tokens per launch group (T = 17, 40
    cross group edges): against ifd_moe_rows on the same weights and routing (the same arithmetic, sums in another
    order: within 2^-6 of the output's scale) and against the oracle's per-token decode composition. shared =
    "weights": the shared expert's T64 copies run as one more slot of the launches, against its rows computed in the
    same (qmv4) arithmetic and passed as ys."""
    g, ops = _gu(), _ops()
    E, H, I, seed = 64, 1024, 256, 430 + T
    egu, edn = experts(E, 2 * I, H, seed=seed), experts(E, H, I, seed=seed + 1)
    rng = np.random.default_rng(seed)
    xn = gen.activations(T, H, seed=seed + 2)
    x0 = gen.activations(T, H, seed=seed + 3)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    wt = rng.random((T, k)).astype(np.float32)
    wt /= wt.sum(axis=1, keepdims=True)
    sg = rng.random(T).astype(np.float32) if shared else np.ones(T, np.float32)
    ys = gen.activations(T, H, seed=seed + 4) if shared else None
    sw = None
    if shared == "weights":  # the shared expert's rows in the decode arithmetic, and its T64 copies
        s1, s2 = experts(1, 2 * I, H, seed=seed + 5), experts(1, H, I, seed=seed + 6)
        gu = gen.f32_to_bf16(orc.qmv(xn, s1[0][0], s1[1][0], s1[2][0]))
        ys = gen.f32_to_bf16(orc.qmv(orc.silu_mul(gu), s2[0][0], s2[1][0], s2[2][0]))
        sw = (ops.pack_t64(g.qlinear(s1[0][0], s1[1][0], s1[2][0])), ops.pack_t64(g.qlinear(s2[0][0], s2[1][0], s2[2][0])))
    W1, W2 = g.moew(*egu), g.moew(*edn)
    T1, T2 = ops.pack_t64_stack(W1), ops.pack_t64_stack(W2)
    args = (g.dev(xn), g.dev(idx), g.dev(wt), g.dev(sg))
    ysd = g.dev(ys) if shared else None
    yst = None if sw else ysd  # the T64 call's rows: none when the weights are given
    d = np.empty((T * k, H), np.uint16)
    for t in range(T):
        for j in range(k):
            e = idx[t, j]
            gu = gen.f32_to_bf16(orc.qmv(xn[t:t + 1], egu[0][e], egu[1][e], egu[2][e]))
            d[t * k + j] = gen.f32_to_bf16(orc.qmv(orc.silu_mul(gu), edn[0][e], edn[1][e], edn[2][e]))[0]
    ident = np.arange(T * k, dtype=np.int32)
    for assign in (True, False):
        out = ops.moe_rows_t64(*args, T1, T2, yst, out=g.dev(x0), assign=assign, shared=sw)
        again = ops.moe_rows_t64(*args, T1, T2, yst, out=g.dev(x0), assign=assign, shared=sw)
        mlx = ops.moe_rows(*args, W1, W2, ysd, out=g.dev(x0), assign=assign)
        torch.cuda.synchronize()
        assert np.array_equal(g.host(out), g.host(again))
        got, m = gen.bf16_to_f32(g.host(out)), gen.bf16_to_f32(g.host(mlx))
        assert np.abs(got - m).max() <= 2 ** -6 * max(float(np.abs(m).max()), 1e-6)
        ref = orc.moe_combine(x0, d, wt, ys, sg, ident, k, assign)
        gen.check_bf16(g.host(out), ref, 1e-2, (T, k, shared, assign), ref_is_bf16=True, composition=True)


@pytest.mark.parametrize("T", [1, 4, 8, 12, 16])
def test_moe_decode_8bit_shared_expert(T):
    """An 8-bit shared expert beside the 4-bit routed experts (the reference's moe_gu2_4_8 / moe_dn2_4_8,
    moe.metal:465-476, 544-547): its slot runs the qmv8 arithmetic. Config 4's layer geometry; the oracle's decode MoE
    with the same width, 1e-2 RMS."""
    g, ops = _gu(), _ops()
    E, H, I, k, seed = 512, 2048, 512, 10, 210 + T
    egu, edn = experts(E, 2 * I, H, seed=seed), experts(E, H, I, seed=seed + 1)
    _, gq, gs, gb = gen.qlinear8(2 * I, H, seed=seed + 2, bias="free")
    _, dq, ds, db = gen.qlinear8(H, I, seed=seed + 3, bias="free")
    R = router(E + 1, H, seed=seed + 4)
    xn = gen.activations(T, H, seed=seed + 5)
    x0 = gen.activations(T, H, seed=seed + 6)
    sh = (g.qlinear(gq, gs, gb, bits=8), g.qlinear(dq, ds, db, bits=8))
    out, idx, wt, sg, logits = ops.moe_decode(g.dev(xn), g.dev(R), g.moew(*egu), g.moew(*edn), k, shared=sh,
                                              out=g.dev(x0), assign=False)
    torch.cuda.synchronize()
    ri, rw, rs = orc.moe_route(g.host(logits), E, k, shared_gate=True)
    assert np.array_equal(g.host(idx), ri)
    ref = orc.moe_decode(xn, ri, rw, rs, egu, edn, ((gq, gs, gb), (dq, ds, db)), I, out=x0, assign=False,
                         shared_bits=8)
    gen.check_bf16(g.host(out), ref, 1e-2, (T, "8-bit shared"), ref_is_bf16=True, composition=True)


def test_moe_decode_rows_independent_of_batch():
    """A token's result is the same bits whatever the other tokens of the call: 12 tokens (16-row accumulators) against
    each token alone (8-row accumulators), as the reference's per-row arithmetic gives."""
    g, ops = _gu(), _ops()
    E, H, I, k, seed = 64, 1024, 256, 6, 170
    egu, edn = experts(E, 2 * I, H, seed=seed), experts(E, H, I, seed=seed + 1)
    sgu, sdn = experts(1, 2 * I, H, seed=seed + 2), experts(1, H, I, seed=seed + 3)
    R = router(E + 1, H, seed=seed + 4)
    xn = gen.activations(12, H, seed=seed + 5)
    sh = (g.qlinear(sgu[0][0], sgu[1][0], sgu[2][0]), g.qlinear(sdn[0][0], sdn[1][0], sdn[2][0]))
    E_gu, E_dn = g.moew(*egu), g.moew(*edn)
    allr = g.host(ops.moe_decode(g.dev(xn), g.dev(R), E_gu, E_dn, k, shared=sh)[0])
    for t in (0, 5, 11):
        one = g.host(ops.moe_decode(g.dev(np.ascontiguousarray(xn[t:t + 1])), g.dev(R), E_gu, E_dn, k, shared=sh)[0])
        assert np.array_equal(one[0], allr[t]), t


@pytest.mark.parametrize("T", [1, 5, 12])
def test_moe_decode_router8(T):
    """The reference's 8-bit router (moe_router8: per group s sum q x + b sum x, fp32 logits, the shared gate as the
    last row) through gemm_w8 mode 2, then the decode MoE from those logits (ifd_moe_decode_logits): logits against the
    oracle's qmv8, routing bit-exact on the GPU's logits, the block against the oracle's composition."""
    g, ops = _gu(), _ops()
    E, H, I, k, seed = 128, 2048, 256, 8, 180 + T
    egu, edn = experts(E, 2 * I, H, seed=seed), experts(E, H, I, seed=seed + 1)
    sgu, sdn = experts(1, 2 * I, H, seed=seed + 2), experts(1, H, I, seed=seed + 3)
    _, rq, rs_, rb = gen.qlinear8(E + 1, H, seed=seed + 4)
    xn = gen.activations(T, H, seed=seed + 5)
    x0 = gen.activations(T, H, seed=seed + 6)
    Wr = g.qlinear(rq, rs_, rb, bits=8)
    lg_d = ops.gemm(g.dev(xn), Wr, mode=2)
    torch.cuda.synchronize()
    lg = g.host(lg_d)
    gen.check_f32(lg, orc.qmv(xn, rq, rs_, rb, bits=8), 1e-5, "router8 logits")
    sh = (g.qlinear(sgu[0][0], sgu[1][0], sgu[2][0]), g.qlinear(sdn[0][0], sdn[1][0], sdn[2][0]))
    out, idx, wt, sg, _ = ops.moe_decode(g.dev(xn), None, g.moew(*egu), g.moew(*edn), k, shared=sh, out=g.dev(x0),
                                         assign=False, logits_in=lg_d)
    torch.cuda.synchronize()
    ri, rw, rsg = orc.moe_route(lg, E, k, shared_gate=True)
    assert np.array_equal(g.host(idx), ri)
    assert np.allclose(g.host(wt), rw, rtol=1e-5, atol=1e-7)
    assert np.allclose(g.host(sg), rsg, rtol=1e-5)
    shw = ((sgu[0][0], sgu[1][0], sgu[2][0]), (sdn[0][0], sdn[1][0], sdn[2][0]))
    ref = orc.moe_decode(xn, ri, rw, rsg, egu, edn, shw, I, out=x0, assign=False)
    gen.check_bf16(g.host(out), ref, 1e-2, ("router8", T), ref_is_bf16=True, composition=True)


@pytest.mark.parametrize("assign", [True, False])
def test_moe_decode_shared_experts_across_tokens(assign):
    """8 tokens over 8 experts, top-3: most experts are picked by several tokens (each read once for all of them)."""
    ri = _decode_case(8, 8, 512, 128, 3, True, False, seed=140, assign=assign)
    assert len(np.unique(ri)) < ri.size


@pytest.mark.parametrize("T", [1, 5, 16])
def test_moe_decode_out_alignment(T):
    """The combine stores 8 columns at a time into a 16-byte aligned out, else one at a time: the same bits either
    way (residual add, shared expert)."""
    g, ops = _gu(), _ops()
    E, H, I, k = 32, 512, 128, 4
    egu, edn = g.moew(*experts(E, 2 * I, H, seed=170)), g.moew(*experts(E, H, I, seed=171))
    sgu, sdn = experts(1, 2 * I, H, seed=172), experts(1, H, I, seed=173)
    sh = (g.qlinear(sgu[0][0], sgu[1][0], sgu[2][0]), g.qlinear(sdn[0][0], sdn[1][0], sdn[2][0]))
    xn = g.dev(gen.activations(T, H, seed=174))
    Rd = g.dev(router(E + 1, H, seed=175))
    x0 = g.dev(gen.activations(T, H, seed=176))
    a16 = x0.clone()
    big = torch.empty((T * H + 8,), dtype=torch.bfloat16, device=x0.device)
    a2 = big[1:1 + T * H].view(T, H)  # 2 bytes past a 16-byte boundary
    a2.copy_(x0)
    ops.moe_decode(xn, Rd, egu, edn, k, shared=sh, out=a16, assign=False)
    ops.moe_decode(xn, Rd, egu, edn, k, shared=sh, out=a2, assign=False)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(a16), g.host(a2.contiguous()))
    assert not np.array_equal(g.host(a16), g.host(x0))


@pytest.mark.parametrize("T,E,H,I,k,shared,shared_gate,assign", [
    (1, 512, 2048, 512, 10, True, True, True),     # gate/up on 8 K splits
    (4, 512, 2048, 512, 10, True, False, False),
    (8, 512, 2048, 512, 10, True, True, True),     # 3 K splits
    (3, 32, 512, 128, 4, False, False, True),      # no shared expert; short K (2 splits of 4 groups)
    (8, 8, 1024, 256, 3, True, False, False),      # most experts picked by several tokens
    (5, 16, 512, 192, 2, True, False, True),       # I = 192: three groups per down band, a ping-pong block across bands
    (12, 512, 2048, 512, 10, True, True, False),   # 9 to 16 tokens: eight accumulator rows per lane
    (16, 64, 1024, 256, 4, False, False, True),
])
def test_moe_decode_t64(T, E, H, I, k, shared, shared_gate, assign):
    """The decode MoE on T64 stacks against the MLX-layout decode MoE on the same weights (the same router kernel:
    routing bit-exact; expert sums in another order: within two bf16 steps of a few elements) and against the
    oracle's composition; a second call gives the same bits (the split and combine counters reset themselves)."""
    g, ops = _gu(), _ops()
    seed = 180 + T + E
    egu, edn = (_config4_stacks()[:2] if (E, H, I) == (512, 2048, 512)
                else (experts(E, 2 * I, H, seed=seed), experts(E, H, I, seed=seed + 1)))
    sgu = experts(1, 2 * I, H, seed=seed + 2)
    sdn = experts(1, H, I, seed=seed + 3)
    R = g.dev(router(E + (1 if shared_gate else 0), H, seed=seed + 4))
    xn = gen.activations(T, H, seed=seed + 5)
    x0 = gen.activations(T, H, seed=seed + 6)
    EGU, EDN = g.moew(*egu), g.moew(*edn)
    sh = (g.qlinear(sgu[0][0], sgu[1][0], sgu[2][0]), g.qlinear(sdn[0][0], sdn[1][0], sdn[2][0])) if shared else None
    sh_t = (ops.pack_t64(sh[0]), ops.pack_t64(sh[1])) if shared else None
    TGU, TDN = ops.pack_t64_stack(EGU), ops.pack_t64_stack(EDN)
    m_out, m_idx, m_wt, _, _ = ops.moe_decode(g.dev(xn), R, EGU, EDN, k, shared=sh, shared_gate=shared_gate,
                                              out=g.dev(x0), assign=assign)
    outs = []
    for _ in range(2):
        out, idx, wt, sg, logits = ops.moe_decode_t64(g.dev(xn), R, TGU, TDN, k, shared=sh_t,
                                                      shared_gate=shared_gate, out=g.dev(x0), assign=assign)
        torch.cuda.synchronize()
        outs.append(g.host(out))
    assert np.array_equal(outs[0], outs[1])
    assert np.array_equal(g.host(idx), g.host(m_idx)) and np.array_equal(g.host(wt), g.host(m_wt))
    got, mlx = gen.bf16_to_f32(outs[0]), gen.bf16_to_f32(g.host(m_out))
    scale = max(float(np.abs(mlx).max()), 1e-6)
    assert np.abs(got - mlx).max() <= 2 ** -6 * scale, "T64 and MLX-layout decode beyond summation-order rounding"
    ri, rw, rs = orc.moe_route(g.host(logits), E, k, shared_gate=shared_gate)
    assert np.array_equal(g.host(idx), ri)
    shw = ((sgu[0][0], sgu[1][0], sgu[2][0]), (sdn[0][0], sdn[1][0], sdn[2][0])) if shared else None
    ref = orc.moe_decode(xn, ri, rw, rs, egu, edn, shw, I, out=x0, assign=assign)
    gen.check_bf16(outs[0], ref, 1e-2, ("t64", T, E, H, I, k), ref_is_bf16=True, composition=True)


def test_moe_decode_t64_logits_in():
    """With the caller's fp32 logits (an 8-bit router's) the T64 decode routes them as the MLX-layout decode does."""
    g, ops = _gu(), _ops()
    T, E, H, I, k = 2, 64, 512, 128, 4
    egu, edn = experts(E, 2 * I, H, seed=190), experts(E, H, I, seed=191)
    EGU, EDN = g.moew(*egu), g.moew(*edn)
    lg = g.dev((np.random.default_rng(192).standard_normal((T, E)) * 0.5).astype(np.float32))
    xn = g.dev(gen.activations(T, H, seed=193))
    m_out, m_idx, _, _, _ = ops.moe_decode(xn, None, EGU, EDN, k, shared_gate=False, logits_in=lg)
    out, idx, _, _, _ = ops.moe_decode_t64(xn, None, ops.pack_t64_stack(EGU), ops.pack_t64_stack(EDN), k,
                                           shared_gate=False, logits_in=lg)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(idx), g.host(m_idx))
    got, mlx = gen.bf16_to_f32(g.host(out)), gen.bf16_to_f32(g.host(m_out))
    assert np.abs(got - mlx).max() <= 2 ** -6 * max(float(np.abs(mlx).max()), 1e-6)


def test_moe_decode_no_shared_expert_long_k():
    """No shared expert; I = 1152 (two K chunks of 8 groups in the down kernel), H = 4608 (gate/up chunks too), k = 16."""
    _decode_case(3, 64, 4608, 1152, 16, False, False, seed=150)


@pytest.mark.parametrize("silu", [True, False])
def test_gather_qmm_a8(silu):
    """The gathered expert GEMM on int8 activations (reference qa8g_gemm): token rows quantized once (qa8 form) and
    read through perm, or sorted rows read directly."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(160)
    T, E, H, I, k = 40, 16, 512, 256, 4
    x = gen.activations(T, H, seed=161)
    idx = np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32)
    disp = ops.moe_dispatch(g.dev(idx), E)
    ro, rp, ri = orc.moe_dispatch(idx, E)
    if silu:
        wq, s, b = experts(E, 2 * I, H, seed=162)
        W = g.moew(wq, s, b)
        U, XS = ops.a8_quant(g.dev(x), 2)
        got = g.host(ops.moe_gather_qmm_a8(U, XS, disp[1], k, disp, W, silu=True))
        prod = ops.moe_gather_qmm_a8(U, XS, disp[1], k, disp, W, silu=False)
        assert np.array_equal(got, g.host(ops.silu_mul(prod)))  # the fused SwiGLU of the product, bit for bit
        Ur, XSr = orc.a8_quant(x, 2)
        y = orc.moe_gather_w4a8(Ur, XSr, rp, k, ro, wq, s, b, 2 * I, H)
        gen.check_bf16(g.host(prod), y, 2e-2, "gate/up")
    else:
        wq, s, b = experts(E, H, I, seed=163)
        a = gen.activations(T * k, I, seed=164)  # sorted rows (the SwiGLU output of the gate/up product)
        U, XS = ops.a8_quant(g.dev(a), 2)
        got = g.host(ops.moe_gather_qmm_a8(U, XS, None, 1, disp, g.moew(wq, s, b), silu=False))
        Ur, XSr = orc.a8_quant(a, 2)
        y = orc.moe_gather_w4a8(Ur, XSr, None, 1, ro, wq, s, b, H, I)
        gen.check_bf16(got, y, 2e-2, "down")


# ---- MoE on T64 expert stacks ---------------------------------------------------------------------------------------
@functools.lru_cache(maxsize=None)
def _config4_stacks():
    """BASELINE config 4's expert stacks (H = 2048, E = 512, I = 512) and a shared expert, host arrays."""
    return (experts(512, 1024, 2048, seed=300), experts(512, 2048, 512, seed=301), experts(1, 1024, 2048, seed=302),
            experts(1, 2048, 512, seed=303))


def _stacks(T, E, H, I):
    if (E, H, I) == (512, 2048, 512):
        return _config4_stacks()
    return (experts(E, 2 * I, H, seed=T + 1), experts(E, H, I, seed=T + 2), experts(1, 2 * I, H, seed=T + 3),
            experts(1, H, I, seed=T + 4))


@pytest.mark.parametrize("T,E,H,I,k,tile_rows", [
    (16, 64, 256, 256, 4, 32),
    (200, 32, 512, 256, 4, 64),    # ~25 rows per expert: 64-row tiles partly empty
    (300, 16, 256, 512, 2, 64),    # ~38 rows per expert, several experts past one tile
    (2048, 512, 2048, 512, 10, 64),
    (128, 512, 2048, 512, 10, 32),
])
def test_gather_qmm_t64_bit_identical(T, E, H, I, k, tile_rows):
    """The gathered GEMM on T64 stacks gives the bits of the MLX-layout one (the same bf16(s q + b) dequant and fp32
    summation order per row) for gate/up with its SwiGLU and for down, at either tile height; ifd_moe_dispatch_ex
    sorts the rows exactly as ifd_moe_dispatch and tiles every segment with its tile height."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(T + E)
    egu, edn, _, _ = _stacks(T, E, H, I)
    x = g.dev(gen.activations(T, H, seed=T + 5))
    idx = g.dev(np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32))
    d32 = ops.moe_dispatch(idx, E)
    dex = ops.moe_dispatch_ex(idx, E, k, tile_rows)
    torch.cuda.synchronize()
    for a, b_ in ((d32[0], dex[0][:E + 1]), (d32[1], dex[1]), (d32[2], dex[2])):
        assert np.array_equal(g.host(a), g.host(b_))
    ro = g.host(dex[0])
    nt = int(g.host(dex[4])[0])
    want = [(e, q) for e in range(E) for q in range(ro[e], ro[e + 1], tile_rows)]
    assert [tuple(t) for t in g.host(dex[3])[:nt].tolist()] == want
    EGU, EDN = g.moew(*egu), g.moew(*edn)
    TGU, TDN = ops.pack_t64_stack(EGU), ops.pack_t64_stack(EDN)
    h_mlx = ops.moe_gather_qmm(x, d32[1], k, d32, EGU, silu=True)
    h_t = ops.moe_gather_qmm_t64(x, dex[1], k, dex, TGU, silu=True)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(h_t), g.host(h_mlx)), "gate/up + SwiGLU"
    y_mlx = ops.moe_gather_qmm(h_t, None, 1, d32, EDN, silu=False)
    y_t = ops.moe_gather_qmm_t64(h_t, None, 1, dex, TDN, silu=False)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(y_t), g.host(y_mlx)), "down"


def _cut_items(nitems, G2, P, min_loss=8):
    """The items the balanced schedule cuts. It runs when whole-item runs would make the longest run at least
    min_loss (item, group pair) units longer than the even share; then block b runs units [b U / P, (b + 1) U / P) of
    the U = nitems G2, and an item is cut when its first and last units lie in different runs."""
    per = -(-nitems // P)
    if per * G2 * P - nitems * G2 < min_loss * P:
        return set()
    U = nitems * G2
    block_of = lambda u: (u * P + P - 1) // U  # noqa: E731
    return {it for it in range(nitems) if block_of(it * G2) != block_of(it * G2 + G2 - 1)}


def _check_balanced(g, Cb, Cw, disp, tile_rows, width, K, what):
    """Uncut items bit-identical to the whole-item schedule; cut items (their K ranges summed in K order) within
    fp32 summation-order rounding, i.e. a few bf16 steps at most. Returns the number of cut items."""
    offsets, tiles, nt = g.host(disp[0]), g.host(disp[3]), int(g.host(disp[4])[0])
    nct = Cw.shape[1] // width
    P = torch.cuda.get_device_properties(0).multi_processor_count
    cut = _cut_items(nt * nct, K // 128, P)
    b, w = gen.bf16_to_f32(g.host(Cb)), gen.bf16_to_f32(g.host(Cw))
    for it in range(nt * nct):
        e, q0 = tiles[it // nct]
        q1 = min(int(offsets[e + 1]), q0 + tile_rows)
        c0 = (it % nct) * width
        bb, ww = b[q0:q1, c0:c0 + width], w[q0:q1, c0:c0 + width]
        if it not in cut:
            assert np.array_equal(bb, ww), f"{what}: uncut item {it} differs"
        else:
            bound = 2.0 ** -5 * np.abs(ww) + 1e-6 * max(np.abs(w).max(), 1e-30)
            assert (np.abs(bb - ww) <= bound).all(), f"{what}: cut item {it} beyond summation-order rounding"
    return len(cut)


@pytest.mark.parametrize("T,E,H,I,k,tile_rows,shared,gu_cut", [
    (2, 16, 2048, 256, 2, 32, True, True),   # fewer units than blocks: empty runs, items cut into one-unit pieces
    (16, 64, 256, 256, 4, 32, True, False),  # 2 units per item: whole items always
    (300, 16, 256, 512, 2, 64, False, False),
    (16, 512, 2048, 512, 10, 32, True, True),    # BASELINE config 4 geometry: ~280 gate/up items on 256 blocks
    (128, 512, 2048, 512, 10, 32, True, False),  # ~950 items: whole-item runs within 5 units of the even share
    (2048, 512, 2048, 512, 10, 64, True, True),  # ~1090 items: 5 per block against 4.26
])
def test_gather_qmm_t64_balanced(T, E, H, I, k, tile_rows, shared, gu_cut):
    """The balanced schedule (a workspace: every block an equal share of the (item, group pair) units, cut items
    summed from their pieces by the last contributor) against the whole-item schedule on the same dispatch, for
    gate/up + SwiGLU and for down (the wide form on 64-row tiles): bit-identical on uncut items, within summation-order
    rounding on cut ones, and the same bits on a second call (the counters reset themselves). gu_cut: the schedule
    cuts gate/up items here (the kernel takes it only where whole-item runs lose at least 8 units)."""
    g, ops = _gu(), _ops()
    rng = np.random.default_rng(T + E + 1)
    egu, edn, sgu, sdn = _stacks(T, E, H, I)
    x = g.dev(gen.activations(T, H, seed=T + 6))
    idx = g.dev(np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32))
    disp = ops.moe_dispatch_ex(idx, E, k, tile_rows, shared_rows=T if shared else 0)
    TGU, TDN = ops.pack_t64_stack(g.moew(*egu)), ops.pack_t64_stack(g.moew(*edn))
    SGU = ops.pack_t64(g.qlinear(sgu[0][0], sgu[1][0], sgu[2][0])) if shared else None
    SDN = ops.pack_t64(g.qlinear(sdn[0][0], sdn[1][0], sdn[2][0])) if shared else None
    hw = ops.moe_gather_qmm_t64(x, disp[1], k, disp, TGU, silu=True, shared=SGU)
    hb = ops.moe_gather_qmm_t64(x, disp[1], k, disp, TGU, silu=True, shared=SGU, balanced=True)
    hb2 = ops.moe_gather_qmm_t64(x, disp[1], k, disp, TGU, silu=True, shared=SGU, balanced=True)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(hb), g.host(hb2)), "gate/up: a second call differs"
    ncut = _check_balanced(g, hb, hw, disp, tile_rows, 256, H, "gate/up + SwiGLU")
    assert (ncut > 0) == gu_cut, f"gate/up: {ncut} items cut"
    wide = H % 512 == 0 and tile_rows == 64
    yw = ops.moe_gather_qmm_t64(hw, None, 1, disp, TDN, silu=False, shared=SDN)
    yb = ops.moe_gather_qmm_t64(hw, None, 1, disp, TDN, silu=False, shared=SDN, balanced=True)
    torch.cuda.synchronize()
    _check_balanced(g, yb, yw, disp, tile_rows, 512 if wide else 256, I, "down")


@pytest.mark.parametrize("T,tile_rows", [(37, 32), (300, 64)])
def test_gather_qmm_t64_shared_segment(T, tile_rows):
    """The shared expert as the dispatch's expert-E segment (every token, in token order, after the routed rows): its
    gate/up product rows against the oracle's qmm of the tokens, the fused SwiGLU bit-identical to silu_mul of the
    product, and the routed rows unchanged by the extra segment."""
    g, ops = _gu(), _ops()
    E, H, I, k = 16, 512, 256, 2
    rng = np.random.default_rng(T)
    egu, _, sgu, _ = _stacks(T, E, H, I)
    xn = gen.activations(T, H, seed=T + 7)
    x = g.dev(xn)
    idx = g.dev(np.stack([rng.choice(E, size=k, replace=False) for _ in range(T)]).astype(np.int32))
    TGU = ops.pack_t64_stack(g.moew(*egu))
    SGU = ops.pack_t64(g.qlinear(sgu[0][0], sgu[1][0], sgu[2][0]))
    dsh = ops.moe_dispatch_ex(idx, E, k, tile_rows, shared_rows=T)
    dno = ops.moe_dispatch_ex(idx, E, k, tile_rows)
    R = T * k
    prod = g.host(ops.moe_gather_qmm_t64(x, dsh[1], k, dsh, TGU, silu=False, shared=SGU))
    h = ops.moe_gather_qmm_t64(x, dsh[1], k, dsh, TGU, silu=True, shared=SGU)
    h0 = ops.moe_gather_qmm_t64(x, dno[1], k, dno, TGU, silu=True)
    torch.cuda.synchronize()
    assert g.host(dsh[0])[E + 1] == R + T and np.array_equal(g.host(dsh[1])[R:], np.arange(T) * k)
    assert np.array_equal(g.host(h), g.host(ops.silu_mul(g.dev(prod))))
    assert np.array_equal(g.host(h)[:R], g.host(h0))
    gen.check_bf16(prod[R:], orc.qmm(xn, sgu[0][0], sgu[1][0], sgu[2][0]), 1e-2, "shared gate/up")


def _ffn_t64_case(T, E, H, I, k, shared_gate, seed):
    """The one-shot FFN on T64 stacks against its stages through the C ABI (same bits), the stages against the
    oracle on the GPU's own inputs, and the whole against the oracle's composition (shared expert in the gathered
    GEMM's bf16 dequant arithmetic at every T)."""
    g, ops = _gu(), _ops()
    egu, edn, sgu, sdn = _stacks(seed, E, H, I)
    R_ = router(E + (1 if shared_gate else 0), H, seed=seed + 4)
    xn = gen.activations(T, H, seed=seed + 5)
    sgu_h, sdn_h = (sgu[0][0], sgu[1][0], sgu[2][0]), (sdn[0][0], sdn[1][0], sdn[2][0])
    xd, Rd = g.dev(xn), g.dev(R_)
    TGU, TDN = ops.pack_t64_stack(g.moew(*egu)), ops.pack_t64_stack(g.moew(*edn))
    SGU, SDN = ops.pack_t64(g.qlinear(*sgu_h)), ops.pack_t64(g.qlinear(*sdn_h))
    out, idx, wt, sg = ops.moe_ffn_t64(xd, Rd, TGU, TDN, k, shared=(SGU, SDN), shared_gate=shared_gate,
                                       logits_bf16=T >= 64)
    # the stages
    R = T * k
    tile_rows = 64 if R >= 24 * E else 32
    logits = ops.moe_router_logits(xd, Rd, out_bf16=T >= 64)
    idx2, wt2, sg2 = ops.moe_route(logits, E, k, shared_gate=shared_gate)
    disp = ops.moe_dispatch_ex(idx2, E, k, tile_rows, shared_rows=T)
    # the one-shot call runs both products on the balanced schedule
    eact = ops.moe_gather_qmm_t64(xd, disp[1], k, disp, TGU, silu=True, shared=SGU, balanced=True)
    ydn = ops.moe_gather_qmm_t64(eact, None, 1, disp, TDN, silu=False, shared=SDN, balanced=True)
    out2 = ops.moe_combine(torch.zeros_like(out), ydn[:R], wt2, ydn[R:], sg2, disp[2], k, True)
    # the product itself and its fused SwiGLU on whole items (no cut sums: the same bits either way)
    gu_full = ops.moe_gather_qmm_t64(xd, disp[1], k, disp, TGU, silu=False, shared=SGU)
    eact_w = ops.moe_gather_qmm_t64(xd, disp[1], k, disp, TGU, silu=True, shared=SGU)
    torch.cuda.synchronize()
    assert np.array_equal(g.host(out), g.host(out2)), "one-shot FFN differs from its stages"
    assert np.array_equal(g.host(idx), g.host(idx2)) and np.array_equal(g.host(wt), g.host(wt2))
    assert np.array_equal(g.host(eact_w), g.host(ops.silu_mul(gu_full))), "fused SwiGLU differs from silu_mul"
    ri, rw, rs = orc.moe_route(g.host(logits), E, k, shared_gate=shared_gate)
    assert np.array_equal(g.host(idx), ri)
    ro, rp, rinv = orc.moe_dispatch(ri, E)
    eact_h, ydn_h = g.host(eact), g.host(ydn)
    gen.check_bf16(g.host(gu_full)[:R], orc.moe_gather_qmm(xn, rp, k, ro, *egu, 2 * I, H), 1e-2, "gate/up")
    gen.check_bf16(g.host(gu_full)[R:], orc.qmm(xn, *sgu_h), 1e-2, "shared gate/up")
    gen.check_bf16(ydn_h[:R], orc.moe_gather_qmm(eact_h[:R], None, 1, ro, *edn, H, I), 1e-2, "down")
    gen.check_bf16(ydn_h[R:], orc.qmm(eact_h[R:], *sdn_h), 1e-2, "shared down")
    comb = orc.moe_combine(np.zeros((T, H), np.uint16), ydn_h[:R], rw, ydn_h[R:], rs, rinv, k, True)
    gen.check_bf16(g.host(out), comb, 1e-2, "combine", ref_is_bf16=True)
    ref = orc.moe_experts(xn, ri, rw, rs, egu, edn, (sgu_h, sdn_h), I, shared_qmv=False)
    gen.check_bf16(g.host(out), ref, 1e-2, ("end to end", T, E, H, I, k), ref_is_bf16=True, composition=True)


@pytest.mark.parametrize("T,shared_gate", [(16, True), (128, False), (2048, False)])
def test_moe_ffn_t64_baseline_geometry(T, shared_gate):
    """BASELINE config 4 (H = 2048, E = 512, top-10, I = 512, shared expert) on T64 stacks at its three T."""
    _ffn_t64_case(T, 512, 2048, 512, 10, shared_gate, seed=T)


def test_moe_ffn_t64_small():
    _ffn_t64_case(40, 8, 256, 256, 2, True, seed=97)
