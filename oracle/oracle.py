"""numpy front end of the CPU oracle (liboracle.so, built from oracle/qmm_oracle.cpp).

TEST INFRASTRUCTURE ONLY: imported by tests/, ``__graft_entry__.smoke()`` and ``bench.py``'s cpu_baseline leg, as
the checker or the timed CPU comparator. The product package ``inferd_amd`` never imports it.

bf16 arrays are numpy ``uint16`` bit patterns. Each wrapper cites the reference function whose semantics the C++
restatement follows (the citations are repeated on the C++ side).
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
_LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None

_u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i8p = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_u32p = np.ctypeslib.ndpointer(dtype=np.uint32, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_vp = ctypes.c_void_p
_i = ctypes.c_int
_u = ctypes.c_uint32
_i64 = ctypes.c_int64


def build() -> None:
    """Compile liboracle.so with the committed Makefile."""
    subprocess.run(["make", "-s", "-C", _HERE, "liboracle.so"], check=True)


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(_LIB_PATH):
            build()
        L = ctypes.CDLL(_LIB_PATH)
        L.orc_f32_to_bf16.argtypes = [_f32p, _u16p, _i64]
        L.orc_bf16_to_f32.argtypes = [_u16p, _f32p, _i64]
        L.orc_pack_w4.argtypes = [_u8p, _u32p, _i, _i]
        L.orc_unpack_w4.argtypes = [_u32p, _u8p, _i, _i, _u]
        L.orc_flip.argtypes = [_u32p, _i64, _u]
        L.orc_dequant_f32.argtypes = [_u32p, _u16p, _u16p, _i, _i, _u, _f32p]
        L.orc_dequant_bf16.argtypes = [_u32p, _u16p, _u16p, _i, _i, _u, _u16p]
        for f in (L.orc_qmv, L.orc_qmm):
            f.argtypes = [_u16p, _i, _u32p, _u16p, _u16p, _i, _i, _u, _f32p, _i, _i]
        for f in (L.orc_qmv_b, L.orc_qmm_b):
            f.argtypes = [_u16p, _i, _u32p, _u16p, _u16p, _i, _i, _i, _u, _f32p, _i, _i]
        L.orc_wxa8.argtypes = [_i8p, _f32p, _u32p, _u16p, _u16p, _i, _i, _i, _u, _f32p, _i, _i]
        L.orc_pack_w8.argtypes = [_u8p, _u32p, _i, _i]
        L.orc_unpack_w8.argtypes = [_u32p, _u8p, _i, _i, _u]
        L.orc_dequant_f32_b.argtypes = [_u32p, _u16p, _u16p, _i, _i, _i, _u, _f32p]
        L.orc_moe_gather_w4a8.argtypes = [_i8p, _f32p, _vp, _i, _i32p, _u32p, _u16p, _u16p, _i, _i, _i, _f32p, _i]
        L.orc_moe_decode.argtypes = [_u16p, _i, _i, _i, _i, _i32p, _f32p, _f32p,
                                     _u32p, _u16p, _u16p, _u32p, _u16p, _u16p,
                                     _vp, _vp, _vp, _vp, _vp, _vp, _u16p, _i]
        L.orc_moe_decode_b.argtypes = [_u16p, _i, _i, _i, _i, _i32p, _f32p, _f32p,
                                       _u32p, _u16p, _u16p, _u32p, _u16p, _u16p,
                                       _vp, _vp, _vp, _vp, _vp, _vp, _i, _u16p, _i]
        L.orc_store.argtypes = [_f32p, _vp, _i, _i, _i, _i]
        L.orc_a8_quant.argtypes = [_u16p, _i, _i, _i, _i, _i8p, _f32p]
        L.orc_w4a8.argtypes = [_i8p, _f32p, _u32p, _u16p, _u16p, _i, _i, _u, _f32p, _i, _i]
        L.orc_silu_mul.argtypes = [_u16p, _u16p, _i, _i]
        L.orc_rmsnorm.argtypes = [_u16p, _i, _u16p, _u16p, _i, _i, _i, ctypes.c_float]
        L.orc_gemm_bf16.argtypes = [_u16p, _u16p, _f32p, _i, _i, _i, _i]
        L.orc_moe_route.argtypes = [_vp, _i, _i, _i, _i, _i, _i, _i, _i32p, _f32p, _f32p]
        L.orc_moe_dispatch.argtypes = [_i32p, _i, _i, _i32p, _i32p, _i32p]
        L.orc_moe_gather_qmm.argtypes = [_u16p, _vp, _i, _i32p, _u32p, _u16p, _u16p, _i, _i, _i, _f32p, _i, _i]
        L.orc_moe_combine.argtypes = [_u16p, _u16p, _f32p, _vp, _f32p, _i32p, _i, _i, _i, _i]
        L.orc_moe_experts.argtypes = [_u16p, _i, _i, _i, _i, _i, _i32p, _f32p, _f32p,
                                      _u32p, _u16p, _u16p, _u32p, _u16p, _u16p,
                                      _vp, _vp, _vp, _vp, _vp, _vp, _i, _u16p, _i, _i]
        _lib = L
    return _lib


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


# ---- bf16 ---------------------------------------------------------------------------------------------------------
def f32_to_bf16(x) -> np.ndarray:
    x = _c(x, np.float32)
    y = np.empty(x.shape, np.uint16)
    lib().orc_f32_to_bf16(x.reshape(-1), y.reshape(-1), x.size)
    return y


def bf16_to_f32(x) -> np.ndarray:
    x = _c(x, np.uint16)
    y = np.empty(x.shape, np.float32)
    lib().orc_bf16_to_f32(x.reshape(-1), y.reshape(-1), x.size)
    return y


# ---- weight format ------------------------------------------------------------------------------------------------
def pack_w4(codes) -> np.ndarray:
    codes = _c(codes, np.uint8)
    N, K = codes.shape
    wq = np.empty((N, K // 8), np.uint32)
    lib().orc_pack_w4(codes, wq, N, K)
    return wq


def unpack_w4(wq, K: int, xr: int = 0) -> np.ndarray:
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    codes = np.empty((N, K), np.uint8)
    lib().orc_unpack_w4(wq, codes, N, K, xr)
    return codes


def flip(wq, mask: int = 0x88888888) -> np.ndarray:
    out = _c(wq, np.uint32).copy()
    lib().orc_flip(out.reshape(-1), out.size, mask)
    return out


def dequant_f32(wq, s, b, K: int, xr: int = 0) -> np.ndarray:
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    w = np.empty((N, K), np.float32)
    lib().orc_dequant_f32(wq, _c(s, np.uint16), _c(b, np.uint16), N, K, xr, w)
    return w


def dequant_bf16(wq, s, b, K: int, xr: int = 0) -> np.ndarray:
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    w = np.empty((N, K), np.uint16)
    lib().orc_dequant_bf16(wq, _c(s, np.uint16), _c(b, np.uint16), N, K, xr, w)
    return w


# ---- GEMMs (fp32 results before the store) ------------------------------------------------------------------------
def qmv(A, wq, s, b, xr: int = 0, nthreads: int = 0, bits: int = 4) -> np.ndarray:
    """qmv4 / qmv8 semantics (engine/kernels/core.metal:85-171, 175-248)."""
    A = _c(A, np.uint16)
    M, K = A.shape
    N = wq.shape[0]
    Y = np.empty((M, N), np.float32)
    if bits == 4:
        lib().orc_qmv(A, K, _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16), N, K, xr, Y, M, nthreads)
    else:
        lib().orc_qmv_b(A, K, _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16), N, K, bits, xr, Y, M, nthreads)
    return Y


def qmm(A, wq, s, b, xr: int = 0, nthreads: int = 0, bits: int = 4) -> np.ndarray:
    """MLX affine_qmm_t semantics (bf16-rounded dequant; quantized.h:528-535, quantized_nax.h:938-1076)."""
    A = _c(A, np.uint16)
    M, K = A.shape
    N = wq.shape[0]
    Y = np.empty((M, N), np.float32)
    if bits == 4:
        lib().orc_qmm(A, K, _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16), N, K, xr, Y, M, nthreads)
    else:
        lib().orc_qmm_b(A, K, _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16), N, K, bits, xr, Y, M, nthreads)
    return Y


def pack_w8(codes) -> np.ndarray:
    """codes uint8 [N, K] -> uint32 [N, K/4], byte j of a word = element j (MLX affine 8-bit)."""
    codes = _c(codes, np.uint8)
    N, K = codes.shape
    wq = np.empty((N, K // 4), np.uint32)
    lib().orc_pack_w8(codes, wq, N, K)
    return wq


def unpack_w8(wq, K: int, xr: int = 0) -> np.ndarray:
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    codes = np.empty((N, K), np.uint8)
    lib().orc_unpack_w8(wq, codes, N, K, xr)
    return codes


def dequant_f32_bits(wq, s, b, K: int, bits: int, xr: int = 0) -> np.ndarray:
    wq = _c(wq, np.uint32)
    N = wq.shape[0]
    w = np.empty((N, K), np.float32)
    lib().orc_dequant_f32_b(wq, _c(s, np.uint16), _c(b, np.uint16), N, K, bits, xr, w)
    return w


def store(Y, mode: int, C=None) -> np.ndarray:
    """GEMM store modes (core.metal:14-15): 0 bf16, 1 bf16 residual add into C, 2 fp32."""
    Y = _c(Y, np.float32)
    M, N = Y.shape
    if mode == 2:
        out = np.empty((M, N), np.float32)
    elif mode == 1:
        out = _c(C, np.uint16).copy()
    else:
        out = np.empty((M, N), np.uint16)
    lib().orc_store(Y, out.ctypes.data, N, M, N, mode)
    return out


def a8_quant(A, per_token):
    """a8_quant (engine/kernels/w4a8.metal:24-41); per_token: one amax per row; per_token = 2: the int8 prefill's
    qa8_quant form (qa8.metal:30-49)."""
    A = _c(A, np.uint16)
    M, K = A.shape
    U = np.empty((M, K), np.int8)
    XS = np.empty((M, K // 64, 2), np.float32)
    lib().orc_a8_quant(A, K, M, K, 2 if per_token == 2 else (1 if per_token else 0), U, XS)
    return U, XS


def w4a8(U, XS, wq, s, b, xr: int = 0, nthreads: int = 0, bits: int = 4) -> np.ndarray:
    """w4a8_gemm semantics (engine/kernels/w4a8.metal:7-8, 78-87); bits = 8: W8A8 (offset 128, :57)."""
    U = _c(U, np.int8)
    M, K = U.shape
    N = wq.shape[0]
    Y = np.empty((M, N), np.float32)
    if bits == 4:
        lib().orc_w4a8(U, _c(XS, np.float32), _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16), N, K, xr, Y, M,
                       nthreads)
    else:
        lib().orc_wxa8(U, _c(XS, np.float32), _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16), N, K, bits, xr,
                       Y, M, nthreads)
    return Y


def silu_mul(gu) -> np.ndarray:
    gu = _c(gu, np.uint16)
    R, I2 = gu.shape
    h = np.empty((R, I2 // 2), np.uint16)
    lib().orc_silu_mul(gu, h, I2 // 2, R)
    return h


def rmsnorm(x, w, eps: float) -> np.ndarray:
    x = _c(x, np.uint16)
    R, D = x.shape
    out = np.empty((R, D), np.uint16)
    lib().orc_rmsnorm(x, D, _c(w, np.uint16), out, D, R, D, eps)
    return out


def rmsnorm_a8(x, w, eps: float, per_token: bool):
    """rmsnorm_a8 (engine/kernels/core.metal:502-537): rmsnorm, then a8_quant of its bf16 output (the reference states
    the fused kernel bit-identical to that pair)."""
    out = rmsnorm(x, w, eps)
    U, XS = a8_quant(out, per_token)
    return out, U, XS


def silu_mul_a8(gu, per_token: bool):
    """silu_mul_a8 (core.metal:789-814): a8_quant of the bf16 silu_mul output, which is not kept."""
    return a8_quant(silu_mul(gu), per_token)


def splitk_res(part, x) -> np.ndarray:
    """The residual split-K reduce of splitk_res_norm (core.metal:564-572; splitk_reduce with add,
    qmm_splitk.metal:90-107): bf16(sum_z part[z] + x), the fp32 sum taken in split order."""
    part = _c(part, np.float32)
    acc = np.zeros(part.shape[1:], np.float32)
    for z in range(part.shape[0]):
        acc = (acc + part[z]).astype(np.float32)
    return f32_to_bf16(acc + bf16_to_f32(x))


def splitk_res_norm(part, x, w, eps: float, a8=None):
    """splitk_res_norm / splitk_res_norm_a8 (core.metal:539-595): the residual reduce, then rmsnorm of the updated rows
    (and, with a8 = per_token, a8_quant of the output). Returns (x', out) or (x', out, U, XS)."""
    xn = splitk_res(part, x)
    out = rmsnorm(xn, w, eps)
    if a8 is None:
        return xn, out
    U, XS = a8_quant(out, a8)
    return xn, out, U, XS


def gemm_bf16(A, W, nthreads: int = 0) -> np.ndarray:
    A = _c(A, np.uint16)
    W = _c(W, np.uint16)
    M, K = A.shape
    N = W.shape[0]
    Y = np.empty((M, N), np.float32)
    lib().orc_gemm_bf16(A, W, Y, M, N, K, nthreads)
    return Y


# ---- MoE ----------------------------------------------------------------------------------------------------------
def moe_route(logits, E: int, k: int, norm: bool = True, shared_gate: bool = True):
    """moe_route / moe_route_bf (moe.metal:60-101, qwen4.metal:1462-1503). logits fp32 or bf16 (uint16)."""
    is_bf = logits.dtype == np.uint16
    logits = np.ascontiguousarray(logits)
    T, stride = logits.shape
    idx = np.empty((T, k), np.int32)
    wt = np.empty((T, k), np.float32)
    sg = np.empty((T,), np.float32)
    lib().orc_moe_route(logits.ctypes.data, 1 if is_bf else 0, T, E, k, stride, 1 if norm else 0,
                        1 if shared_gate else 0, idx, wt, sg)
    return idx, wt, sg


def moe_dispatch(idx, E: int):
    idx = _c(idx, np.int32).reshape(-1)
    R = idx.size
    offsets = np.empty((E + 1,), np.int32)
    perm = np.empty((R,), np.int32)
    inv = np.empty((R,), np.int32)
    lib().orc_moe_dispatch(idx, R, E, offsets, perm, inv)
    return offsets, perm, inv


def moe_gather_qmm(A, perm, div: int, offsets, wq, s, b, N: int, K: int) -> np.ndarray:
    A = _c(A, np.uint16)
    offsets = _c(offsets, np.int32)
    E = offsets.size - 1
    R = int(offsets[-1])
    Y = np.empty((R, N), np.float32)
    permc = None if perm is None else _c(perm, np.int32)
    lib().orc_moe_gather_qmm(A, None if permc is None else permc.ctypes.data, div, offsets, _c(wq, np.uint32),
                             _c(s, np.uint16), _c(b, np.uint16), E, N, K, Y, R, 0)
    return Y


def moe_combine(x, yd, wt, ys, sg, inv, k: int, assign: bool) -> np.ndarray:
    out = _c(x, np.uint16).copy()
    T, H = out.shape
    ysc = None if ys is None else _c(ys, np.uint16)
    lib().orc_moe_combine(out, _c(yd, np.uint16), _c(wt, np.float32), None if ysc is None else ysc.ctypes.data,
                          _c(sg, np.float32), _c(inv, np.int32), T, H, k, 1 if assign else 0)
    return out


def moe_experts(xn, idx, wt, sg, egu, edn, shared, I: int, out=None, assign: bool = True, nthreads: int = 0,
                shared_qmv: bool = False):
    """Sorted-path MoE FFN composition (engine/src/qwen35.h:1869-1980) for given routing.

    egu / edn / shared: tuples (wq, s, b) — routed stacks [E, 2I, H/8] and [E, H, I/8]; shared = ((gu), (dn)) or None.
    shared_qmv: the shared expert's dense GEMMs take the decode GEMV semantics (else qmm's).
    """
    xn = _c(xn, np.uint16)
    T, H = xn.shape
    idx = _c(idx, np.int32)
    k = idx.shape[1]
    E = egu[0].shape[0]
    o = np.zeros((T, H), np.uint16) if out is None else _c(out, np.uint16).copy()
    keep = []

    def p(a, dt):
        if a is None:
            return None
        a = _c(a, dt)
        keep.append(a)
        return a.ctypes.data

    if shared is not None:
        (sgw, sgs, sgb), (sdw, sds, sdb) = shared
        sh = [p(sgw, np.uint32), p(sgs, np.uint16), p(sgb, np.uint16), p(sdw, np.uint32), p(sds, np.uint16),
              p(sdb, np.uint16)]
    else:
        sh = [None] * 6
    lib().orc_moe_experts(xn, T, H, I, E, k, idx, _c(wt, np.float32), _c(sg, np.float32),
                          _c(egu[0], np.uint32), _c(egu[1], np.uint16), _c(egu[2], np.uint16),
                          _c(edn[0], np.uint32), _c(edn[1], np.uint16), _c(edn[2], np.uint16),
                          *sh, 1 if shared_qmv else 0, o, 1 if assign else 0, nthreads)
    return o


# ---- checkpoint formats (host-side restatement of the loader's arithmetic) ----------------------------------------
def expand_groups(sb, gs: int) -> np.ndarray:
    """A group of gs values becomes gs / 64 groups of 64 with its scale (or bias) repeated (load_moe, moe.h:69-83):
    [..., K / gs] -> [..., K / 64]."""
    if gs % 64:
        raise ValueError("group size must be a multiple of 64")
    return np.repeat(_c(sb, np.uint16), gs // 64, axis=-1)


def pack_affine(codes, bits: int) -> np.ndarray:
    """Codes [N, K] -> uint32 words [N, K bits / 32], element j of a word at bits bits * j, low first
    (weights.h:349-350)."""
    codes = np.asarray(codes, np.uint32)
    N, K = codes.shape
    per = 32 // bits
    c = codes.reshape(N, K // per, per)
    return np.bitwise_or.reduce(c << (bits * np.arange(per, dtype=np.uint32)), axis=-1).astype(np.uint32)


def quantize_affine(w_bf16, bits: int):
    """Load-time affine quantization, group 64 (load_qlinear_bf16_q8, weights.h:349-406): per group lo / hi the
    min / max, sc = (hi - lo) / (2^bits - 1) in fp32 (1e-8 when 0), sc and lo rounded to bf16 (nearest even), then
    q = clamp(round_half_away((w - lo_bf16) / sc_bf16), 0, 2^bits - 1) in fp32. Returns (wq, s, b, codes)."""
    w = bf16_to_f32(w_bf16)
    N, K = w.shape
    levels = np.float32((1 << bits) - 1)
    g = w.reshape(N, K // 64, 64)
    lo = g.min(axis=-1)
    hi = g.max(axis=-1)
    sc = ((hi - lo) / levels).astype(np.float32)
    sc[sc == 0] = np.float32(1e-8)
    sb = f32_to_bf16(sc)
    bb = f32_to_bf16(lo)
    v = ((g - bf16_to_f32(bb)[..., None]) / bf16_to_f32(sb)[..., None]).astype(np.float32)
    v64 = v.astype(np.float64)
    r = np.trunc(v64 + np.copysign(0.5, v64))  # std::round: half away from zero (exact in float64)
    codes = np.clip(r, 0, float(levels)).astype(np.uint32).reshape(N, K)
    return pack_affine(codes, bits), sb, bb, codes


def moe_decode(xn, idx, wt, sg, egu, edn, shared, I: int, out=None, assign: bool = True,
               shared_bits: int = 4) -> np.ndarray:
    """Decode MoE for T <= 8 tokens (engine/kernels/moe.metal:326-551): per token and pick the decode GEMV arithmetic
    for gate/up and down, SwiGLU, bf16 expert outputs, weighted combine (plus sg * the shared expert).
    egu / edn: (wq, s, b) stacks [E, 2I, H/8] and [E, H, I/8]; shared = ((gu), (dn)) or None, of shared_bits 4 or 8
    (moe_gu2_4_8 / moe_dn2_4_8, moe.metal:465-476, 544-547: the qmv8 dot)."""
    xn = _c(xn, np.uint16)
    T, H = xn.shape
    idx = _c(idx, np.int32)
    k = idx.shape[1]
    o = np.zeros((T, H), np.uint16) if out is None else _c(out, np.uint16).copy()
    keep = []

    def p(a, dt):
        a = _c(a, dt)
        keep.append(a)
        return a.ctypes.data

    if shared is not None:
        (sgw, sgs, sgb), (sdw, sds, sdb) = shared
        sh = [p(sgw, np.uint32), p(sgs, np.uint16), p(sgb, np.uint16), p(sdw, np.uint32), p(sds, np.uint16),
              p(sdb, np.uint16)]
    else:
        sh = [None] * 6
    lib().orc_moe_decode_b(xn, T, H, I, k, idx, _c(wt, np.float32), _c(sg, np.float32),
                           _c(egu[0], np.uint32), _c(egu[1], np.uint16), _c(egu[2], np.uint16),
                           _c(edn[0], np.uint32), _c(edn[1], np.uint16), _c(edn[2], np.uint16), *sh, shared_bits, o,
                           1 if assign else 0)
    return o


def moe_gather_w4a8(U, XS, perm, div: int, offsets, wq, s, b, N: int, K: int, nthreads: int = 0) -> np.ndarray:
    """qa8g_gemm semantics (engine/kernels/qa8.metal:212-397): the gathered expert GEMM on int8 activations."""
    offsets = _c(offsets, np.int32)
    E = len(offsets) - 1
    R = int(offsets[-1])
    Y = np.zeros((R, N), np.float32)
    pp = None if perm is None else _c(perm, np.int32)
    lib().orc_moe_gather_w4a8(_c(U, np.int8), _c(XS, np.float32), None if pp is None else pp.ctypes.data, div, offsets,
                              _c(wq, np.uint32), _c(s, np.uint16), _c(b, np.uint16), E, N, K, Y, nthreads)
    return Y
