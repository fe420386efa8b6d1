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


def bf16_err(got_bf16: np.ndarray, ref: np.ndarray, ref_is_bf16: bool = False) -> float:
    """BASELINE's max |err| / RMS(ref) for a bf16 output, net of the output's own quantization: each element may sit
    half a bf16 step from an fp32 reference (one step from a reference that is itself bf16-rounded)."""
    got = bf16_to_f32(got_bf16).astype(np.float64)
    r = bf16_to_f32(ref).astype(np.float64) if ref_is_bf16 else np.asarray(ref, np.float64)
    rms = float(np.sqrt(np.mean(r * r))) or 1.0
    slack = bf16_ulp(r) * (1.0 if ref_is_bf16 else 0.5)
    return float(np.max(np.maximum(np.abs(got - r) - slack, 0.0))) / rms


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
