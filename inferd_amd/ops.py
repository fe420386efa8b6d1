"""Python mirror of the engine-facing operators over the C ABI (include/inferd_qmm.h).

torch supplies device memory and the current HIP stream; every computation runs in libinferd_amd.so.
Names follow the reference engine: ``QLinear`` (engine/src/weights.h:226-236), ``MoeW`` (engine/src/moe.h:8-11),
``gemm`` (Qwen35::gemm, engine/src/qwen35.h:1465) and ``moe_ffn`` (Qwen35::encode_moe, qwen35.h:1869).
"""
from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

import ctypes

import torch

from ._lib import check, lib

FLIP_MASK = 0x88888888
FLIP_MASK_8 = 0x80808080


def _p(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def _stream() -> int:
    return torch.cuda.current_stream().cuda_stream


_ws_cache: dict = {}


def workspace(nbytes: int, device) -> torch.Tensor:
    """A cached uint8 device buffer of at least nbytes (grown on demand), reused across calls on one stream.
    Allocated zeroed: a workspace's leading counters must start at zero, and the library keeps them there."""
    key = str(device)
    buf = _ws_cache.get(key)
    if buf is None or buf.numel() < nbytes:
        buf = torch.zeros(max(nbytes, 256), dtype=torch.uint8, device=device)
        _ws_cache[key] = buf
    return buf


@dataclass
class QLinear:
    """MLX affine group-64 linear [N, K]: wq int32 [N, K bits/32] (uint32 bit patterns), s/b bf16 [N, K/64];
    bits 4 (nibbles) or 8 (bytes)."""
    wq: torch.Tensor
    s: torch.Tensor
    b: torch.Tensor
    N: int
    K: int
    flipped: bool = False
    bits: int = 4

    @property
    def flip_mask(self) -> int:
        return FLIP_MASK_8 if self.bits == 8 else FLIP_MASK

    @property
    def xr(self) -> int:
        return self.flip_mask if self.flipped else 0


@dataclass
class T64Linear:
    """A linear [N, K] repacked into the T64 layout (inferd_amd/csrc/t64.h): a uint8 device buffer."""
    wt: torch.Tensor
    N: int
    K: int


def pack_t64(W: "QLinear") -> T64Linear:
    """One-time repack of an MLX-layout linear into the T64 layout (undoes a flip)."""
    if W.bits != 4:
        raise ValueError("pack_t64 takes 4-bit layers; 8-bit layers go to pack_t64x8")
    nbytes = lib().ifd_t64_bytes(W.N, W.K, 1)
    wt = torch.empty((nbytes,), dtype=torch.uint8, device=W.wq.device)
    check(lib().ifd_pack_t64(_p(W.wq), _p(W.s), _p(W.b), W.N, W.K, 0, W.xr, 1, _p(wt), _stream()))
    return T64Linear(wt, W.N, W.K)


def gemm_t64(A: torch.Tensor, W: T64Linear, C: Optional[torch.Tensor] = None, mode: int = 0) -> torch.Tensor:
    """C (mode) = A . W^T for T64 weights."""
    M, K = A.shape
    assert K == W.K and A.dtype == torch.bfloat16 and A.is_contiguous()
    if C is None:
        C = torch.empty((M, W.N), dtype=torch.float32 if mode == 2 else torch.bfloat16, device=A.device)
    need = lib().ifd_gemm_t64_workspace(M, W.N, W.K)
    ws = workspace(need, A.device) if need else None
    check(lib().ifd_gemm_t64(_p(A), K, _p(W.wt), W.N, W.K, _p(C), C.shape[1], M, mode, _p(ws),
                             ws.numel() if ws is not None else 0, _stream()))
    return C


def gemm_t64_multi_call(A: torch.Tensor, Ws: list, outs: list, mode: int = 0):
    """A prepared gemm_t64_multi: the pointer arrays and the workspace are built once, and the returned function
    launches C_l (mode) = A . W_l^T with one library call (it keeps A, Ws, outs and the workspace alive)."""
    M, K = A.shape
    n = len(Ws)
    assert A.dtype == torch.bfloat16 and A.is_contiguous() and 1 <= n <= 8 and len(outs) == n
    assert all(W.K == K for W in Ws)
    Ns = (ctypes.c_int * n)(*[W.N for W in Ws])
    wts = (ctypes.c_void_p * n)(*[W.wt.data_ptr() for W in Ws])
    Cs = (ctypes.c_void_p * n)(*[C.data_ptr() for C in outs])
    ldcs = (ctypes.c_int * n)(*[C.stride(0) for C in outs])
    need = lib().ifd_gemm_t64_multi_workspace(M, n, Ns, K)
    ws = workspace(need, A.device) if need else None
    args = (_p(A), K, n, wts, Ns, K, Cs, ldcs, M, mode, _p(ws), ws.numel() if ws is not None else 0)
    keep = (A, Ws, outs, ws)

    def call() -> None:
        assert keep
        check(lib().ifd_gemm_t64_multi(*args, _stream()))

    return call


def gemm_t64_multi(A: torch.Tensor, Ws: list, outs: Optional[list] = None, mode: int = 0) -> list:
    """C_l (mode) = A . W_l^T for 1 to 8 T64 linears that share A and K (M <= 16), in one launch; mode 1 adds into
    the given outputs, mode 2 writes fp32."""
    M = A.shape[0]
    if outs is None:
        outs = [torch.empty((M, W.N), dtype=torch.float32 if mode == 2 else torch.bfloat16, device=A.device)
                for W in Ws]
    gemm_t64_multi_call(A, Ws, outs, mode)()
    return outs


def gemm_t64_swiglu(A: torch.Tensor, W: T64Linear, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """h = silu_mul(bf16(A . W^T)) for T64 weights holding [gate | up] rows: the fused gate/up projection."""
    M, K = A.shape
    assert K == W.K and A.dtype == torch.bfloat16 and A.is_contiguous() and W.N % 2 == 0
    h = torch.empty((M, W.N // 2), dtype=torch.bfloat16, device=A.device) if out is None else out
    need = lib().ifd_gemm_t64_swiglu_workspace(M, W.N, W.K)
    ws = workspace(need, A.device) if need else None
    check(lib().ifd_gemm_t64_swiglu(_p(A), K, _p(W.wt), W.N, W.K, _p(h), h.stride(0), M, _p(ws),
                                    ws.numel() if ws is not None else 0, _stream()))
    return h


def gemm_t64_w4a8(U: torch.Tensor, XS: torch.Tensor, W: T64Linear, C: Optional[torch.Tensor] = None,
                  mode: int = 0, per_token: bool = True) -> torch.Tensor:
    """C (mode) = W4A8 product of int8 activations with T64 weights: per-token (ops.a8_quant(A, True)) on the int8
    MFMA kernels, or per 64-group (ops.a8_quant(A, False), the reference's default W4A8 route) on the affine T64
    kernels."""
    M, K = U.shape
    assert K == W.K and U.dtype == torch.int8 and U.is_contiguous()
    if C is None:
        C = torch.empty((M, W.N), dtype=torch.float32 if mode == 2 else torch.bfloat16, device=U.device)
    need = lib().ifd_gemm_t64_w4a8_workspace(M, W.N, W.K)
    ws = workspace(need, U.device) if need else None
    check(lib().ifd_gemm_t64_w4a8(_p(U), _p(XS), 1 if per_token else 0, _p(W.wt), W.N, W.K, _p(C), C.shape[1], M,
                                  mode, _p(ws), ws.numel() if ws is not None else 0, _stream()))
    return C


@dataclass
class T64x8Linear:
    """An 8-bit linear [N, K] repacked into the T64x8 layout (inferd_amd/csrc/t64.h): a uint8 device buffer."""
    wt: torch.Tensor
    N: int
    K: int


def pack_t64x8(W: QLinear) -> T64x8Linear:
    """One-time repack of an MLX-layout 8-bit linear into the T64x8 layout (undoes a flip)."""
    if W.bits != 8:
        raise ValueError("pack_t64x8 takes 8-bit layers")
    nbytes = lib().ifd_t64x8_bytes(W.N, W.K)
    wt = torch.empty((nbytes,), dtype=torch.uint8, device=W.wq.device)
    check(lib().ifd_pack_t64x8(_p(W.wq), _p(W.s), _p(W.b), W.N, W.K, 0, W.xr, _p(wt), _stream()))
    return T64x8Linear(wt, W.N, W.K)


def gemm_t64x8(A: torch.Tensor, W: T64x8Linear, C: Optional[torch.Tensor] = None, mode: int = 0) -> torch.Tensor:
    """C (mode) = A . W^T for T64x8 (8-bit) weights, bf16(s q + b) dequant."""
    M, K = A.shape
    assert K == W.K and A.dtype == torch.bfloat16 and A.is_contiguous()
    if C is None:
        C = torch.empty((M, W.N), dtype=torch.float32 if mode == 2 else torch.bfloat16, device=A.device)
    need = lib().ifd_gemm_t64x8_workspace(M, W.N, W.K)
    ws = workspace(need, A.device) if need else None
    check(lib().ifd_gemm_t64x8(_p(A), K, _p(W.wt), W.N, W.K, _p(C), C.shape[1], M, mode, _p(ws),
                               ws.numel() if ws is not None else 0, _stream()))
    return C


def gemm_t64x8_w8a8(U: torch.Tensor, XS: torch.Tensor, W: T64x8Linear, C: Optional[torch.Tensor] = None,
                    mode: int = 0) -> torch.Tensor:
    """C (mode) = W8A8 product of per-token int8 activations (ops.a8_quant(A, True)) with T64x8 weights."""
    M, K = U.shape
    assert K == W.K and U.dtype == torch.int8 and U.is_contiguous()
    if C is None:
        C = torch.empty((M, W.N), dtype=torch.float32 if mode == 2 else torch.bfloat16, device=U.device)
    need = lib().ifd_gemm_t64x8_w8a8_workspace(M, W.N, W.K)
    ws = workspace(need, U.device) if need else None
    check(lib().ifd_gemm_t64x8_w8a8(_p(U), _p(XS), 1, _p(W.wt), W.N, W.K, _p(C), C.shape[1], M, mode, _p(ws),
                                    ws.numel() if ws is not None else 0, _stream()))
    return C


@dataclass
class MoeW:
    """Stacked experts [E, N, K] in the same affine layout (engine/src/moe.h:8-11), 4-bit (wq [E, N, K/8]) or 8-bit
    (wq [E, N, K/4]; moe_gather_qmm only)."""
    wq: torch.Tensor
    s: torch.Tensor
    b: torch.Tensor
    E: int
    N: int
    K: int
    bits: int = 4


# ---- dense ----------------------------------------------------------------------------------------------------------
def gemm(A: torch.Tensor, W: QLinear, C: Optional[torch.Tensor] = None, mode: int = 0, path: str = "auto") -> torch.Tensor:
    """C (mode) = A . W^T. mode 0 bf16 out, 1 bf16 residual add into C, 2 fp32 out. path: auto | qmv | qmm."""
    M, K = A.shape
    assert K == W.K and A.dtype == torch.bfloat16 and A.is_contiguous()
    if C is None:
        C = torch.empty((M, W.N), dtype=torch.float32 if mode == 2 else torch.bfloat16, device=A.device)
    if W.bits == 8:
        assert path == "auto", "8-bit weights take the routed entry point"
        fn, need = lib().ifd_gemm_w8, lib().ifd_gemm_w8_workspace(M, W.N, W.K)
    else:
        fn = {"auto": lib().ifd_gemm_w4, "qmv": lib().ifd_qmv_w4, "qmm": lib().ifd_qmm_w4}[path]
        need = lib().ifd_gemm_w4_workspace(M, W.N, W.K)
    ws = workspace(need, A.device) if need else None
    check(fn(_p(A), K, _p(W.wq), _p(W.s), _p(W.b), W.N, W.K, 0, W.xr, _p(C), C.shape[1], M, mode, _p(ws),
             ws.numel() if ws is not None else 0, _stream()))
    return C


def flip(W: QLinear) -> None:
    """In-place flip: nibbles q ^ 8 or bytes q ^ 0x80 (reference w_flip / Qwen35::flip)."""
    check(lib().ifd_flip_w4(_p(W.wq), W.wq.numel(), W.flip_mask, _stream()))
    W.flipped = not W.flipped


def silu_mul(gu: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    R, I2 = gu.shape
    h = torch.empty((R, I2 // 2), dtype=torch.bfloat16, device=gu.device) if out is None else out
    check(lib().ifd_silu_mul(_p(gu), _p(h), I2 // 2, R, _stream()))
    return h


def rmsnorm(x: torch.Tensor, w: torch.Tensor, eps: float, out: Optional[torch.Tensor] = None) -> torch.Tensor:
    """Row RMS norm of bf16 x [R, D] with bf16 weight w [D] (reference rmsnorm, core.metal:486-500)."""
    R, D = x.shape
    y = torch.empty((R, D), dtype=torch.bfloat16, device=x.device) if out is None else out
    check(lib().ifd_rmsnorm(_p(x), x.stride(0), _p(w), _p(y), y.stride(0), R, D, float(eps), _stream()))
    return y


def rmsnorm_a8(x: torch.Tensor, w: torch.Tensor, eps: float, per_token: bool):
    """rmsnorm of bf16 x [R, D] and the W4A8 quantization of its output (reference rmsnorm_a8, core.metal:502-537):
    returns (out bf16 [R, D], U int8 [R, D], XS fp32 [R, D/64, 2])."""
    R, D = x.shape
    y = torch.empty((R, D), dtype=torch.bfloat16, device=x.device)
    U = torch.empty((R, D), dtype=torch.int8, device=x.device)
    XS = torch.empty((R, D // 64, 2), dtype=torch.float32, device=x.device)
    check(lib().ifd_rmsnorm_a8(_p(x), x.stride(0), _p(w), _p(y), D, R, D, float(eps), 1 if per_token else 0, _p(U),
                               _p(XS), _stream()))
    return y, U, XS


def silu_mul_a8(gu: torch.Tensor, per_token: bool):
    """The W4A8 quantization of silu_mul(gu) without writing h (reference silu_mul_a8, core.metal:789-814)."""
    R, I2 = gu.shape
    I = I2 // 2
    U = torch.empty((R, I), dtype=torch.int8, device=gu.device)
    XS = torch.empty((R, I // 64, 2), dtype=torch.float32, device=gu.device)
    check(lib().ifd_silu_mul_a8(_p(gu), I, R, 1 if per_token else 0, _p(U), _p(XS), _stream()))
    return U, XS


def splitk_res_norm(part: torch.Tensor, x: torch.Tensor, w: torch.Tensor, eps: float, a8: Optional[bool] = None):
    """x += the split sum of part [S, R, D] (in place, bf16), then rmsnorm of x and, with a8 set (per_token), its W4A8
    quantization (reference splitk_res_norm, core.metal:539-595): returns out or (out, U, XS)."""
    S, R, D = part.shape
    y = torch.empty((R, D), dtype=torch.bfloat16, device=x.device)
    U = XS = None
    if a8 is not None:
        U = torch.empty((R, D), dtype=torch.int8, device=x.device)
        XS = torch.empty((R, D // 64, 2), dtype=torch.float32, device=x.device)
    check(lib().ifd_splitk_res_norm(_p(part), S, _p(x), x.stride(0), _p(w), _p(y), D, R, D, float(eps),
                                    1 if a8 else 0, _p(U) if U is not None else None,
                                    _p(XS) if XS is not None else None, _stream()))
    return y if a8 is None else (y, U, XS)


def a8_quant(A: torch.Tensor, per_token):
    """int8 activations: per_token False (per 64-group), True (per row) or 2 (the int8 prefill's qa8 form)."""
    M, K = A.shape
    U = torch.empty((M, K), dtype=torch.int8, device=A.device)
    XS = torch.empty((M, K // 64, 2), dtype=torch.float32, device=A.device)
    form = 2 if per_token == 2 else (1 if per_token else 0)
    check(lib().ifd_a8_quant(_p(A), K, M, K, form, _p(U), _p(XS), _stream()))
    return U, XS


def qmm_w4a8(U: torch.Tensor, XS: torch.Tensor, per_token: bool, W: QLinear, C: Optional[torch.Tensor] = None,
             mode: int = 0) -> torch.Tensor:
    M, K = U.shape
    if C is None:
        C = torch.empty((M, W.N), dtype=torch.float32 if mode == 2 else torch.bfloat16, device=U.device)
    fn = lib().ifd_qmm_w8a8 if W.bits == 8 else lib().ifd_qmm_w4a8
    check(fn(_p(U), _p(XS), 1 if per_token else 0, _p(W.wq), _p(W.s), _p(W.b), W.N, W.K, 0, W.xr,
             _p(C), C.shape[1], M, mode, None, 0, _stream()))
    return C


# ---- MoE ------------------------------------------------------------------------------------------------------------
def moe_router_logits(x: torch.Tensor, w: torch.Tensor, out_bf16: bool) -> torch.Tensor:
    T, H = x.shape
    E1 = w.shape[0]
    out = torch.empty((T, E1), dtype=torch.bfloat16 if out_bf16 else torch.float32, device=x.device)
    check(lib().ifd_moe_router_logits(_p(x), _p(w), T, H, E1, 1 if out_bf16 else 0, _p(out), _stream()))
    return out


def moe_route(logits: torch.Tensor, E: int, k: int, norm: bool = True, shared_gate: bool = True):
    T, stride = logits.shape
    idx = torch.empty((T, k), dtype=torch.int32, device=logits.device)
    wt = torch.empty((T, k), dtype=torch.float32, device=logits.device)
    sg = torch.empty((T,), dtype=torch.float32, device=logits.device)
    check(lib().ifd_moe_route(_p(logits), 1 if logits.dtype == torch.bfloat16 else 0, T, E, k, stride,
                              1 if norm else 0, 1 if shared_gate else 0, _p(idx), _p(wt), _p(sg), _stream()))
    return idx, wt, sg


def moe_dispatch(idx: torch.Tensor, E: int):
    R = idx.numel()
    dev = idx.device
    offsets = torch.empty((E + 1,), dtype=torch.int32, device=dev)
    perm = torch.empty((max(R, 1),), dtype=torch.int32, device=dev)
    inv = torch.empty((max(R, 1),), dtype=torch.int32, device=dev)
    mt = lib().ifd_moe_tiles_max(R, E)
    tiles = torch.empty((max(mt, 1), 2), dtype=torch.int32, device=dev)
    ntiles = torch.empty((1,), dtype=torch.int32, device=dev)
    need = lib().ifd_moe_dispatch_workspace(R, E)
    ws = workspace(need, dev)
    check(lib().ifd_moe_dispatch(_p(idx), R, E, _p(offsets), _p(perm), _p(inv), _p(tiles), _p(ntiles), _p(ws),
                                 ws.numel(), _stream()))
    return offsets, perm[:R], inv[:R], tiles, ntiles, mt


def moe_gather(x: torch.Tensor, perm: torch.Tensor, div: int) -> torch.Tensor:
    R = perm.numel()
    H = x.shape[1]
    xs = torch.empty((R, H), dtype=torch.bfloat16, device=x.device)
    check(lib().ifd_moe_gather(_p(x), _p(perm), div, R, H, _p(xs), _stream()))
    return xs


def moe_gather_qmm(A: torch.Tensor, perm: Optional[torch.Tensor], div: int, disp, W: MoeW, silu: bool) -> torch.Tensor:
    offsets, perm_sorted, _, tiles, ntiles, mt = disp
    R = perm_sorted.numel()
    NO = W.N // 2 if silu else W.N
    C = torch.empty((R, NO), dtype=torch.bfloat16, device=A.device)
    check(lib().ifd_moe_gather_qmm_ex(_p(A), _p(perm), div, _p(offsets), _p(tiles), _p(ntiles), mt, _p(W.wq),
                                      _p(W.s), _p(W.b), W.E, W.N, W.K, W.bits, 1 if silu else 0, _p(C), R, _stream()))
    return C


def moe_gather_qmm_a8(U: torch.Tensor, XS: torch.Tensor, perm: Optional[torch.Tensor], div: int, disp, W: MoeW,
                      silu: bool) -> torch.Tensor:
    """The gathered expert GEMM on int8 activations (U, XS from a8_quant with per-group scales)."""
    offsets, perm_sorted, _, tiles, ntiles, mt = disp
    R = perm_sorted.numel()
    NO = W.N // 2 if silu else W.N
    C = torch.empty((R, NO), dtype=torch.bfloat16, device=U.device)
    check(lib().ifd_moe_gather_qmm_a8(_p(U), _p(XS), _p(perm), div, _p(offsets), _p(tiles), _p(ntiles), mt, _p(W.wq),
                                      _p(W.s), _p(W.b), W.E, W.N, W.K, 1 if silu else 0, _p(C), R, _stream()))
    return C


def moe_combine(out: torch.Tensor, yd: torch.Tensor, wt: torch.Tensor, ys: Optional[torch.Tensor],
                sg: Optional[torch.Tensor], inv: torch.Tensor, k: int, assign: bool) -> torch.Tensor:
    T, H = out.shape
    check(lib().ifd_moe_combine(_p(out), _p(yd), _p(wt), _p(ys), _p(sg), _p(inv), T, H, k, 1 if assign else 0,
                                _stream()))
    return out


def moe_ffn(xn: torch.Tensor, router: torch.Tensor, egu: MoeW, edn: MoeW, k: int,
            shared: Optional[tuple] = None, shared_gate: bool = True, norm: bool = True,
            logits_bf16: bool = True, out: Optional[torch.Tensor] = None, assign: bool = True):
    """One-shot MoE FFN (reference encode_moe's sorted path). shared = (QLinear gate_up [2Is, H], QLinear down [H, Is]).

    Returns (out, idx, wt, sg)."""
    T, H = xn.shape
    E, I = egu.E, egu.N // 2
    dev = xn.device
    if out is None:
        out = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    wt = torch.empty((T, k), dtype=torch.float32, device=dev)
    sg = torch.empty((T,), dtype=torch.float32, device=dev)
    Is = shared[1].K if shared is not None else 0
    need = lib().ifd_moe_ffn_workspace(T, H, I, E, k, Is)
    ws = workspace(need, dev)
    sgu, sdn = shared if shared is not None else (None, None)
    check(lib().ifd_moe_ffn(
        _p(xn), T, H, _p(router), E, k, 1 if norm else 0, 1 if shared_gate else 0, 1 if logits_bf16 else 0,
        _p(egu.wq), _p(egu.s), _p(egu.b), _p(edn.wq), _p(edn.s), _p(edn.b), I,
        _p(sgu.wq) if sgu else None, _p(sgu.s) if sgu else None, _p(sgu.b) if sgu else None,
        _p(sdn.wq) if sdn else None, _p(sdn.s) if sdn else None, _p(sdn.b) if sdn else None, Is,
        _p(out), 1 if assign else 0, _p(idx), _p(wt), _p(sg), _p(ws), ws.numel(), _stream()))
    return out, idx, wt, sg


def moe_rows(xn: torch.Tensor, idx: torch.Tensor, wt: torch.Tensor, sg: Optional[torch.Tensor], egu: MoeW,
             edn: MoeW, ys: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
             assign: bool = True) -> torch.Tensor:
    """The per-row expert products on the caller's routing (ifd_moe_rows; reference moe_qmv4 + moe_silu_mul +
    moe_combine below 128 routed rows): idx int32 / wt fp32 [T, k], sg fp32 [T] and the shared expert's output rows
    ys bf16 [T, H] (or None). Any T. out = bf16(acc) (assign) or out += bf16(acc)."""
    T, H = xn.shape
    k = idx.shape[1]
    E, I = egu.E, egu.N // 2
    assert idx.dtype == torch.int32 and wt.dtype == torch.float32 and idx.is_contiguous() and wt.is_contiguous()
    assert ys is None or (ys.dtype == torch.bfloat16 and ys.shape == (T, H) and ys.is_contiguous() and sg is not None)
    if out is None:
        out = torch.zeros((T, H), dtype=torch.bfloat16, device=xn.device)
    ws = workspace(lib().ifd_moe_rows_workspace(T, H, I, E, k), xn.device)
    check(lib().ifd_moe_rows(_p(xn), T, H, E, k, _p(idx), _p(wt), _p(sg), _p(egu.wq), _p(egu.s), _p(egu.b),
                             _p(edn.wq), _p(edn.s), _p(edn.b), I, _p(ys), _p(out), 1 if assign else 0, _p(ws),
                             ws.numel(), _stream()))
    return out


def moe_rows_t64(xn: torch.Tensor, idx: torch.Tensor, wt: torch.Tensor, sg: Optional[torch.Tensor], egu: T64Stack,
                 edn: T64Stack, ys: Optional[torch.Tensor] = None, out: Optional[torch.Tensor] = None,
                 assign: bool = True, shared: Optional[tuple] = None) -> torch.Tensor:
    """moe_rows on T64 stacks (ifd_moe_rows_t64): the same arguments, 16 tokens per launch group; or the shared
    expert as shared = (T64Linear gate_up, T64Linear down) run in the same launches instead of its rows ys."""
    T, H = xn.shape
    k = idx.shape[1]
    E, I = egu.E, egu.N // 2
    assert idx.dtype == torch.int32 and wt.dtype == torch.float32 and idx.is_contiguous() and wt.is_contiguous()
    assert ys is None or (ys.dtype == torch.bfloat16 and ys.shape == (T, H) and ys.is_contiguous() and sg is not None)
    if out is None:
        out = torch.zeros((T, H), dtype=torch.bfloat16, device=xn.device)
    ws = workspace(lib().ifd_moe_rows_t64_workspace(T, H, I, E, k), xn.device)
    sgu, sdn = shared if shared is not None else (None, None)
    check(lib().ifd_moe_rows_t64(_p(xn), T, H, E, k, _p(idx), _p(wt), _p(sg), _p(egu.wt), _p(edn.wt), I,
                                 _p(sgu.wt) if sgu else None, _p(sdn.wt) if sdn else None, _p(ys), _p(out),
                                 1 if assign else 0, _p(ws), ws.numel(), _stream()))
    return out


def moe_decode(xn: torch.Tensor, router: Optional[torch.Tensor], egu: MoeW, edn: MoeW, k: int,
               shared: Optional[tuple] = None, shared_gate: bool = True, norm: bool = True,
               out: Optional[torch.Tensor] = None, assign: bool = True, logits_in: Optional[torch.Tensor] = None):
    """Decode MoE for T <= 16 tokens (reference moe_plan / moe_gu2 / moe_dn2, and its per-row expert GEMVs below 128
    routed rows): each distinct expert read once. shared = (QLinear gate_up [2I, H], QLinear down [H, I]) with the
    routed experts' I, 4- or 8-bit (ifd_moe_decode_ex with the layers' width). With logits_in (fp32 [T, E +
    shared_gate], e.g. an 8-bit router through gemm_w8 mode 2) the router is not read (ifd_moe_decode_logits_ex).

    Returns (out, idx, wt, sg, logits)."""
    T, H = xn.shape
    E, I = egu.E, egu.N // 2
    dev = xn.device
    if out is None:
        out = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    wt = torch.empty((T, k), dtype=torch.float32, device=dev)
    sg = torch.empty((T,), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E + (1 if shared_gate else 0)), dtype=torch.float32, device=dev)
    ws = workspace(lib().ifd_moe_decode_workspace(T, H, I, E, k), dev)
    sgu, sdn = shared if shared is not None else (None, None)
    sbits = sgu.bits if sgu is not None else 4
    assert sdn is None or sdn.bits == sbits
    if logits_in is not None:
        assert logits_in.dtype == torch.float32 and logits_in.is_contiguous()
        assert logits_in.shape == (T, E + (1 if shared_gate else 0))
        check(lib().ifd_moe_decode_logits_ex(
            _p(logits_in), _p(xn), T, H, E, k, 1 if norm else 0, 1 if shared_gate else 0,
            _p(egu.wq), _p(egu.s), _p(egu.b), _p(edn.wq), _p(edn.s), _p(edn.b), I,
            _p(sgu.wq) if sgu else None, _p(sgu.s) if sgu else None, _p(sgu.b) if sgu else None,
            _p(sdn.wq) if sdn else None, _p(sdn.s) if sdn else None, _p(sdn.b) if sdn else None, sbits,
            _p(out), 1 if assign else 0, _p(idx), _p(wt), _p(sg), _p(ws), ws.numel(), _stream()))
        return out, idx, wt, sg, logits_in
    check(lib().ifd_moe_decode_ex(
        _p(xn), T, H, _p(router), E, k, 1 if norm else 0, 1 if shared_gate else 0,
        _p(egu.wq), _p(egu.s), _p(egu.b), _p(edn.wq), _p(edn.s), _p(edn.b), I,
        _p(sgu.wq) if sgu else None, _p(sgu.s) if sgu else None, _p(sgu.b) if sgu else None,
        _p(sdn.wq) if sdn else None, _p(sdn.s) if sdn else None, _p(sdn.b) if sdn else None, sbits,
        _p(out), 1 if assign else 0, _p(idx), _p(wt), _p(sg), _p(logits), _p(ws), ws.numel(), _stream()))
    return out, idx, wt, sg, logits


def moe_decode_t64(xn: torch.Tensor, router: Optional[torch.Tensor], egu: T64Stack, edn: T64Stack, k: int,
                   shared: Optional[tuple] = None, shared_gate: bool = True, norm: bool = True,
                   out: Optional[torch.Tensor] = None, assign: bool = True, logits_in: Optional[torch.Tensor] = None):
    """The decode MoE on T64 stacks (T <= 16): shared = (T64Linear gate_up [2I, H], T64Linear down [H, I]), 4-bit.
    With logits_in (fp32 [T, E + shared_gate]) the router is not read. Returns (out, idx, wt, sg, logits)."""
    T, H = xn.shape
    E, I = egu.E, egu.N // 2
    dev = xn.device
    if out is None:
        out = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    wt = torch.empty((T, k), dtype=torch.float32, device=dev)
    sg = torch.empty((T,), dtype=torch.float32, device=dev)
    logits = torch.empty((T, E + (1 if shared_gate else 0)), dtype=torch.float32, device=dev)
    ws = workspace(lib().ifd_moe_decode_t64_workspace(T, H, I, E, k), dev)
    sgu, sdn = shared if shared is not None else (None, None)
    if logits_in is not None:
        assert logits_in.dtype == torch.float32 and logits_in.is_contiguous()
        assert logits_in.shape == (T, E + (1 if shared_gate else 0))
    check(lib().ifd_moe_decode_t64(
        _p(xn), T, H, _p(router) if logits_in is None else None, _p(logits_in) if logits_in is not None else None, E,
        k, 1 if norm else 0, 1 if shared_gate else 0, _p(egu.wt), _p(edn.wt), I, _p(sgu.wt) if sgu else None,
        _p(sdn.wt) if sdn else None, _p(out), 1 if assign else 0, _p(idx), _p(wt), _p(sg),
        _p(logits) if logits_in is None else None, _p(ws), ws.numel(), _stream()))
    return out, idx, wt, sg, (logits if logits_in is None else logits_in)


def mlp_decode(x: torch.Tensor, norm_w: torch.Tensor, eps: float, gu: T64Linear, dn: T64Linear) -> torch.Tensor:
    """The dense decode MLP block in place: x += down(SwiGLU(gate_up(rmsnorm(x)))) (T64 weights)."""
    M, H = x.shape
    I = dn.K
    assert gu.N == 2 * I and gu.K == H and dn.N == H and x.is_contiguous()
    ws = workspace(lib().ifd_mlp_decode_workspace(M, H, I), x.device)
    check(lib().ifd_mlp_decode(_p(x), H, _p(norm_w), eps, _p(gu.wt), _p(dn.wt), M, H, I, _p(ws), ws.numel(),
                               _stream()))
    return x


# ---- workspace header and measurement probes ----------------------------------------------------------------------
def workspace_check(ws: torch.Tensor) -> None:
    """Raises unless every counter of the workspace header (its first 4096 bytes) is zero (synchronises)."""
    check(lib().ifd_workspace_check(_p(ws), ws.numel(), _stream()))


def workspace_reset(ws: torch.Tensor) -> None:
    """Zeroes the workspace's counter header on the current stream (a fill kernel)."""
    check(lib().ifd_workspace_reset(_p(ws), ws.numel(), _stream()))


def probe_stream_read(src: torch.Tensor, sink: torch.Tensor, blocks: int = 4096) -> None:
    """One coalesced read of every byte of src (HBM read ceiling); sink: >= 4096 bytes on the device."""
    check(lib().ifd_probe_stream_read(_p(src), src.numel() * src.element_size(), _p(sink), blocks, _stream()))


def probe_mfma(int8: bool, iters: int, blocks: int, out: torch.Tensor) -> float:
    """MFMA-only loop; returns the operations it performs (FLOP for bf16, OP for int8). out: float [blocks * 256]."""
    check(lib().ifd_probe_mfma(1 if int8 else 0, iters, blocks, _p(out), _stream()))
    return float(blocks) * 4 * 8 * iters * (65536 if int8 else 32768)


# ---- MoE on T64 expert stacks -------------------------------------------------------------------------------------
@dataclass
class T64Stack:
    """E experts [E, N, K] packed expert by expert into the T64 layout (a uint8 device buffer)."""
    wt: torch.Tensor
    E: int
    N: int
    K: int


def pack_t64_stack(W: MoeW) -> T64Stack:
    """One-time repack of an MLX-layout expert stack into T64 tiles."""
    if W.bits != 4:
        raise ValueError("pack_t64_stack takes 4-bit expert stacks")
    nbytes = lib().ifd_t64_bytes(W.N, W.K, W.E)
    wt = torch.empty((nbytes,), dtype=torch.uint8, device=W.wq.device)
    check(lib().ifd_pack_t64(_p(W.wq), _p(W.s), _p(W.b), W.N, W.K, 0, 0, W.E, _p(wt), _stream()))
    return T64Stack(wt, W.E, W.N, W.K)


def moe_dispatch_ex(idx: torch.Tensor, E: int, k: int, tile_rows: int = 32, shared_rows: int = 0):
    """ifd_moe_dispatch_ex: returns (offsets [E + 2], perm, inv, tiles, ntiles, max_tiles, tile_rows)."""
    R = idx.numel()
    dev = idx.device
    Rt = R + shared_rows
    offsets = torch.empty((E + 2,), dtype=torch.int32, device=dev)
    perm = torch.empty((max(Rt, 1),), dtype=torch.int32, device=dev)
    inv = torch.empty((max(R, 1),), dtype=torch.int32, device=dev)
    mt = lib().ifd_moe_tiles_max(Rt, E + 1)
    tiles = torch.empty((max(mt, 1), 2), dtype=torch.int32, device=dev)
    ntiles = torch.empty((1,), dtype=torch.int32, device=dev)
    ws = workspace(lib().ifd_moe_dispatch_workspace(R, E), dev)
    check(lib().ifd_moe_dispatch_ex(_p(idx), R, E, k, tile_rows, shared_rows, _p(offsets), _p(perm), _p(inv),
                                    _p(tiles), _p(ntiles), _p(ws), ws.numel(), _stream()))
    return offsets, perm[:Rt], inv[:R], tiles, ntiles, mt, tile_rows


def moe_gather_qmm_t64(A: torch.Tensor, perm: Optional[torch.Tensor], div: int, disp, W: T64Stack, silu: bool,
                       shared: Optional[T64Linear] = None, balanced: bool = False) -> torch.Tensor:
    """The gathered expert GEMM on a T64 stack (disp from moe_dispatch_ex; shared: the expert-E segment's weights).
    balanced: the balanced schedule (a workspace), else whole items per block (the bits of moe_gather_qmm)."""
    offsets, perm_sorted, _, tiles, ntiles, _, tile_rows = disp
    rows = perm_sorted.numel()
    NO = W.N // 2 if silu else W.N
    C = torch.empty((rows, NO), dtype=torch.bfloat16, device=A.device)
    ws = workspace(lib().ifd_moe_gather_qmm_t64_workspace(tile_rows), A.device) if balanced else None
    check(lib().ifd_moe_gather_qmm_t64(_p(A), A.shape[1], _p(perm), div, _p(offsets), _p(tiles), _p(ntiles), tile_rows,
                                       _p(W.wt), _p(shared.wt) if shared is not None else None, W.E, W.N, W.K,
                                       1 if silu else 0, _p(C), NO, rows, _p(ws) if ws is not None else None,
                                       ws.numel() if ws is not None else 0, _stream()))
    return C


def moe_ffn_t64(xn: torch.Tensor, router: torch.Tensor, egu: T64Stack, edn: T64Stack, k: int,
                shared: Optional[tuple] = None, shared_gate: bool = True, norm: bool = True,
                logits_bf16: bool = True, out: Optional[torch.Tensor] = None, assign: bool = True):
    """One-shot MoE FFN on T64 stacks; shared = (T64Linear gate_up [2I, H], T64Linear down [H, I]) with the routed
    experts' I. Returns (out, idx, wt, sg)."""
    T, H = xn.shape
    E, I = egu.E, egu.N // 2
    dev = xn.device
    if out is None:
        out = torch.zeros((T, H), dtype=torch.bfloat16, device=dev)
    idx = torch.empty((T, k), dtype=torch.int32, device=dev)
    wt = torch.empty((T, k), dtype=torch.float32, device=dev)
    sg = torch.empty((T,), dtype=torch.float32, device=dev)
    ws = workspace(lib().ifd_moe_ffn_t64_workspace(T, H, I, E, k, 1 if shared is not None else 0), dev)
    sgu, sdn = shared if shared is not None else (None, None)
    check(lib().ifd_moe_ffn_t64(
        _p(xn), T, H, _p(router), E, k, 1 if norm else 0, 1 if shared_gate else 0, 1 if logits_bf16 else 0,
        _p(egu.wt), _p(edn.wt), I, _p(sgu.wt) if sgu is not None else None, _p(sdn.wt) if sdn is not None else None,
        _p(out), 1 if assign else 0, _p(idx), _p(wt), _p(sg), _p(ws), ws.numel(), _stream()))
    return out, idx, wt, sg
