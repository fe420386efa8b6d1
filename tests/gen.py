"""Seeded synthetic inputs shared by the tests (numpy PCG64 generators; bf16 as uint16 bit patterns).

Distributions follow BASELINE config 0: codes q ~ U{0..15}; scales s ~ U(smin, smax) rounded to bf16; biases
b = bf16(-8 s) computed from the bf16 scale; activations x ~ N(0, 1) rounded to bf16 (RNE).
"""
from __future__ import annotations

import numpy as np


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even fp32 -> bf16 bit patterns (numpy, independent of the oracle library)."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32).astype(np.uint64)
    u = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return u.astype(np.uint16)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def pack_codes(codes: np.ndarray) -> np.ndarray:
    """codes uint8 [N, K] -> uint32 [N, K/8], element j at bits 4j (numpy restatement of the MLX layout)."""
    N, K = codes.shape
    c = codes.reshape(N, K // 8, 8).astype(np.uint32)
    w = np.zeros((N, K // 8), np.uint32)
    for j in range(8):
        w |= c[:, :, j] << np.uint32(4 * j)
    return w


def qlinear(N: int, K: int, seed: int, smin: float = 0.005, smax: float = 0.02, bias: str = "minus8"):
    """Returns (codes uint8 [N,K], wq uint32 [N,K/8], s bf16 [N,K/64], b bf16 [N,K/64])."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 16, size=(N, K), dtype=np.uint8)
    s = f32_to_bf16(rng.uniform(smin, smax, size=(N, K // 64)).astype(np.float32))
    if bias == "minus8":
        b = f32_to_bf16(-8.0 * bf16_to_f32(s))
    else:  # independent biases, as the reference's qa8_dbg / gemm_dbg generators (b = bf16(0.05 U(-1,1)))
        b = f32_to_bf16((0.05 * rng.uniform(-1, 1, size=(N, K // 64))).astype(np.float32))
    return codes, pack_codes(codes), s, b


def pack_codes8(codes: np.ndarray) -> np.ndarray:
    """codes uint8 [N, K] -> uint32 [N, K/4], element j in byte j (numpy restatement of MLX's 8-bit layout)."""
    N, K = codes.shape
    return np.ascontiguousarray(codes, dtype=np.uint8).reshape(N, K // 4, 4).view("<u4").reshape(N, K // 4).astype(np.uint32)


def qlinear8(N: int, K: int, seed: int, bias: str = "minus128"):
    """An 8-bit layer with the same weight range as qlinear: q ~ U{0..255}, s ~ U(0.005, 0.02) / 16 in bf16, and
    b = bf16(-128 s) (or independent biases). Returns (codes, wq uint32 [N, K/4], s, b)."""
    rng = np.random.default_rng(seed)
    codes = rng.integers(0, 256, size=(N, K), dtype=np.uint8)
    s = f32_to_bf16((rng.uniform(0.005, 0.02, size=(N, K // 64)) / 16).astype(np.float32))
    if bias == "minus128":
        b = f32_to_bf16(-128.0 * bf16_to_f32(s))
    else:
        b = f32_to_bf16((0.05 * rng.uniform(-1, 1, size=(N, K // 64))).astype(np.float32))
    return codes, pack_codes8(codes), s, b


def activations(M: int, K: int, seed: int, row_scale: bool = False) -> np.ndarray:
    rng = np.random.default_rng(seed)
    x = rng.standard_normal((M, K)).astype(np.float32)
    if row_scale:  # rows scaled by U(0.5, 2)
        x *= rng.uniform(0.5, 2.0, size=(M, 1)).astype(np.float32)
    return f32_to_bf16(x)


def dequant_f64(codes, s, b) -> np.ndarray:
    """float64 dequant w = s q + b (the math, for textbook references)."""
    N, K = codes.shape
    sf = np.repeat(bf16_to_f32(s).astype(np.float64), 64, axis=1)
    bf = np.repeat(bf16_to_f32(b).astype(np.float64), 64, axis=1)
    return sf * codes.astype(np.float64) + bf


def rel_err(got: np.ndarray, ref: np.ndarray) -> float:
    """max |got - ref| / RMS(ref), the BASELINE tolerance measure."""
    ref = np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(ref * ref))) or 1.0
    return float(np.max(np.abs(np.asarray(got, np.float64) - ref))) / rms


def bf16_ulp(v: np.ndarray) -> np.ndarray:
    """Spacing of bf16 values at |v| (8 significant bits)."""
    a = np.maximum(np.abs(np.asarray(v, np.float64)), 2.0 ** -126)
    return 2.0 ** (np.floor(np.log2(a)) - 7)


def _ord16(h: np.ndarray) -> np.ndarray:
    """bf16 bit patterns -> integers in the order of their values (adjacent bf16 values differ by 1; +0 = -0)."""
    h = np.ascontiguousarray(h, dtype=np.uint16).astype(np.int32)
    mag = h & 0x7FFF
    return np.where(h & 0x8000, -mag, mag)


def bf16_steps(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """Distance in bf16 steps between two arrays of bf16 bit patterns (0: same value, 1: adjacent values)."""
    return np.abs(_ord16(a) - _ord16(b))


def bf16_stats(got_bf16: np.ndarray, ref: np.ndarray, ref_is_bf16: bool = False) -> dict:
    """max |err| / RMS(ref) of a bf16 output, three ways.

    raw:  max |got - ref| / RMS(ref), nothing subtracted.
    Against an fp32 reference (the value the output rounds):
      net: max (|got - ref| - half a bf16 step of ref) / RMS. A correctly rounded output is within half a step of
           the fp32 value it rounds, so net is the kernel's error beyond its own output rounding. ulp1 is None.
    Against a bf16 reference (a computation whose last step rounds to bf16 in the oracle too):
      ulp1, ulp2, far: the shares of elements one, two and more than two bf16 steps from the reference (one step:
            the two fp32 values straddle a rounding boundary).
      net:  max |got - ref| / RMS over the elements more than one step away, with no slack.
    rel_rms: RMS(got - ref) / RMS(ref).
    """
    got = bf16_to_f32(got_bf16).astype(np.float64)
    r = bf16_to_f32(ref).astype(np.float64) if ref_is_bf16 else np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(r * r))) or 1.0
    d = np.abs(got - r)
    raw = float(np.max(d)) / rms if d.size else 0.0
    if not ref_is_bf16:
        net = float(np.max(np.maximum(d - 0.5 * bf16_ulp(r), 0.0))) / rms if d.size else 0.0
        return dict(raw=raw, net=net, ulp1=None, ulp2=None, far=None, rel_rms=None)
    steps = np.abs(_ord16(got_bf16) - _ord16(ref))
    ulp1 = float(np.mean(steps == 1)) if steps.size else 0.0
    ulp2 = float(np.mean(steps == 2)) if steps.size else 0.0
    far = steps > 1
    net = float(np.max(d[far])) / rms if far.any() else 0.0
    rel_rms = float(np.sqrt(np.mean((got - r) ** 2))) / rms if d.size else 0.0
    return dict(raw=raw, net=net, ulp1=ulp1, ulp2=ulp2, far=float(np.mean(steps > 2)) if steps.size else 0.0,
                rel_rms=rel_rms)


# Every parity figure the checks below compute, for the test session's summary (tests/conftest.py):
# (test id, what, raw, net, ulp1, tolerance, ulp2).
RECORDS: list = []


def _test_id() -> str:
    import os
    return os.environ.get("PYTEST_CURRENT_TEST", "").split(" ")[0]


def check_bf16(got_bf16: np.ndarray, ref: np.ndarray, tol: float, what="", ref_is_bf16: bool = False,
               ulp1_max: float = 0.02, composition: bool = False) -> dict:
    """Asserts BASELINE's bar (max |err| <= tol RMS(ref)) on a bf16 output as bf16_stats defines it: net <= tol, and
    against a bf16 reference also ulp1 <= ulp1_max. Records the figures for the session summary.

    composition=True is the end-to-end comparison of a chain of bf16 stages (the MoE FFN) with the oracle's own
    chain, whose stages are each checked at the bar on the GPU's inputs to them. A one-step difference at one stage
    can move a SwiGLU output several steps and carry on through the next product, so no per-element bar holds end
    to end. It asserts instead RMS(got - ref) <= tol RMS(ref), raw <= 5 tol and a one-step share <= 5% (a wrong
    rounding mode at any stage gives about 50%); the two-step and farther shares are recorded."""
    st = bf16_stats(got_bf16, ref, ref_is_bf16)
    if composition:
        RECORDS.append((_test_id(), f"{what} (composition: raw <= {5 * tol:.0e}, far share {st['far']:.1e}, rel RMS "
                                    f"{st['rel_rms']:.1e})", st["raw"], st["raw"], st["ulp1"], 5 * tol, st["ulp2"]))
        assert ref_is_bf16
        assert st["rel_rms"] <= tol and st["raw"] <= 5 * tol, (what, st)
        assert st["ulp1"] <= 0.05, (what, st)
        return st
    RECORDS.append((_test_id(), str(what), st["raw"], st["net"], st["ulp1"], tol, st["ulp2"]))
    assert st["net"] <= tol, (what, st)
    if ref_is_bf16:
        assert st["ulp1"] <= ulp1_max, (what, st, ulp1_max)
    return st


def check_f32(got: np.ndarray, ref: np.ndarray, tol: float, what="") -> float:
    """max |got - ref| / RMS(ref) <= tol for an fp32 output (no slack); recorded like check_bf16."""
    e = rel_err(got, ref)
    RECORDS.append((_test_id(), str(what), e, e, None, tol, None))
    assert e <= tol, (what, e)
    return e


def check_out(got: np.ndarray, ref: np.ndarray, tol: float, what="", fp32: bool = False):
    """check_f32 for an fp32 output (store mode 2), else check_bf16 against the fp32 value the output rounds."""
    return check_f32(got, ref, tol, what) if fp32 else check_bf16(got, ref, tol, what)


T64_NIB = (0, 4, 1, 5, 2, 6, 3, 7)  # nibble of code e (e = 0..7) inside a T64 word


def pack_t64(codes: np.ndarray, s: np.ndarray, b: np.ndarray) -> np.ndarray:
    """numpy restatement of the T64 layout (inferd_amd/csrc/t64.h) from unflipped codes [N, K]: uint8 bytes."""
    N, K = codes.shape
    G, nb = K // 64, (N + 31) // 32
    cp = np.zeros((nb * 32, K), np.uint8)
    cp[:N] = codes
    sp = np.zeros((nb * 32, G), np.uint16)
    bp = np.zeros((nb * 32, G), np.uint16)
    sp[:N], bp[:N] = s, b
    c = cp.reshape(nb, 32, G, 2, 4, 8).astype(np.uint32)  # band, j, g, h, t, e
    words = np.zeros(c.shape[:-1], np.uint32)
    for e in range(8):
        words |= c[..., e] << np.uint32(4 * T64_NIB[e])
    w = np.ascontiguousarray(words.transpose(2, 0, 3, 1, 4))  # g, band, h, j, t  (lane = 32 h + j)
    sb = (sp.astype(np.uint32) | (bp.astype(np.uint32) << np.uint32(16))).reshape(nb, 32, G).transpose(2, 0, 1)
    out = np.zeros((G, nb, 1152), np.uint8)
    out[:, :, :1024] = w.reshape(G, nb, 256).view(np.uint8).reshape(G, nb, 1024)
    out[:, :, 1024:] = np.ascontiguousarray(sb).view(np.uint8).reshape(G, nb, 128)
    return out.reshape(-1)


def pack_t64x8(codes: np.ndarray, s: np.ndarray, b: np.ndarray) -> np.ndarray:
    """numpy restatement of the T64x8 layout (inferd_amd/csrc/t64.h) from unflipped 8-bit codes [N, K]: uint8 bytes.
    Tile (g, band): [s2][lane = 32 h + j][16 bytes] of q ^ 0x80 for k = 64 g + 32 h + 16 s2 + 0..15, then the
    32 (s, b) dwords."""
    N, K = codes.shape
    G, nb = K // 64, (N + 31) // 32
    cp = np.full((nb * 32, K), 0x80, np.uint8)
    cp[:N] = codes
    sp = np.zeros((nb * 32, G), np.uint16)
    bp = np.zeros((nb * 32, G), np.uint16)
    sp[:N], bp[:N] = s, b
    c = (cp ^ np.uint8(0x80)).reshape(nb, 32, G, 2, 2, 16)  # band, j, g, h, s2, byte
    frag = np.ascontiguousarray(c.transpose(2, 0, 4, 3, 1, 5))  # g, band, s2, h, j, byte
    sb = (sp.astype(np.uint32) | (bp.astype(np.uint32) << np.uint32(16))).reshape(nb, 32, G).transpose(2, 0, 1)
    out = np.zeros((G, nb, 2176), np.uint8)
    out[:, :, :2048] = frag.reshape(G, nb, 2048)
    out[:, :, 2048:] = np.ascontiguousarray(sb).view(np.uint8).reshape(G, nb, 128)
    return out.reshape(-1)
